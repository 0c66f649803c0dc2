"""ming_lin_noalloc (the projection entry point that allocates nothing: its
scratch is the device's static array) against ming_lin, through the C-ABI:
the same bits on consecutive calls that shrink, on the fast route's unsplit
and split kernels and the general route; no device memory taken by it; and
its refusals (a call beyond the array, a weight whose adapter stacks are not
built) before anything runs. The auto, general and wide routes, and a dense
weight on a few tiles (the split-K bf16 GEMM) are each held to ming_lin. It has no counterpart in the reference."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import (CFG2_RANKS, CFG2_SCALES, bf16, empty_bf16, from_dev, make_lora,
                     make_weight, randn, sync, to_dev)

pytestmark = pytest.mark.gpu


def _weight(ctx, seed, N, K, bits, ranks):
    pack, _ = make_weight(seed, N, K, bits)
    if bits == 16:
        qw = m.QWeight.dense(ctx, pack["w"])
    else:
        qw = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)
    for s, r in enumerate(ranks):
        A, B = make_lora(seed + 10 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
    return qw


def _both(ctx, qw, x, M, scales):
    """(ming_lin's y, ming_lin_noalloc's y) as host bit patterns."""
    y0 = empty_bf16(M, qw.N)
    y1 = empty_bf16(M, qw.N)
    y1.fill_(0x1234)
    sync()
    ctx.lin(qw, x, y0, M, scales)
    ctx.lin_noalloc(qw, x, y1, M, scales)
    ctx.synchronize()
    sync()
    return from_dev(y0), from_dev(y1)


def test_noalloc_matches_ming_lin_on_calls_that_shrink(ctx):
    import torch
    ctx.set_route("auto")
    cases = [  # (M, N, K, bits, ranks, scales): each smaller than the last
        (4352, 10240, 3840, 4, CFG2_RANKS, CFG2_SCALES),       # 680 tiles, 8-chunk tail
        (300, 512, 640, 8, (16, 64), (0.7, -0.4)),             # ragged, two slots
        (256, 3840, 3840, 4, CFG2_RANKS, CFG2_SCALES),         # 15 tiles: split K
        # dense, no adapter, 15 tiles: the split-K bf16 GEMM (its partials
        # carved from the array)
        (256, 3840, 2560, 16, (), ()),
    ]
    weights = [_weight(ctx, 900 + 7 * i, N, K, b, r) for i, (M, N, K, b, r, s) in enumerate(cases)]
    xs = [to_dev(bf16(randn(950 + i, (M, K)))) for i, (M, N, K, b, r, s) in enumerate(cases)]
    for route in ("auto", "general", "wide"):
        ctx.set_route(route)
        for (M, N, K, bits, ranks, sc), qw, x in zip(cases, weights, xs):
            print(f"case noalloc {route} M={M} N={N} K={K} w{bits}", flush=True)
            ctx.reset_engagement()
            y0, y1 = _both(ctx, qw, x, M, sc)
            eng = ctx.engagement()
            adapted = 2 if ranks else 0
            assert eng["lora_proj"] == adapted and eng["lora_xa"] == adapted
            if bits == 16:
                assert eng["gemm_dense"] == 2 and eng["gemm_fast"] == 0
            elif route == "auto":
                # the fast route splits K below 64 tiles into about one round of
                # the chip, at least 6 K steps a slice, when that gives 2 or more
                tiles = ((M + 255) // 256) * ((N + 255) // 256)
                split = tiles < 64 and min(256 // tiles, (K // 64) // 6) >= 2
                assert eng["gemm_fast"] == 2 and eng["gemm_split"] == (2 if split else 0)
            assert np.array_equal(y0, y1)
    ctx.set_route("auto")
    # the calls themselves take no device memory
    M, N, K, bits, ranks, sc = cases[0]
    y = empty_bf16(M, N)
    sync()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        ctx.lin_noalloc(weights[0], xs[0], y, M, sc)
    ctx.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    for w in weights:
        w.close()


def test_noalloc_refusals_launch_nothing(ctx):
    ctx.set_route("auto")
    # beyond the array: the fp16 copy of x alone is 4352 x 10240 x 2 = 89 MB
    M, N, K = 4352, 512, 10240
    qw = _weight(ctx, 960, N, K, 4, ())
    x = to_dev(bf16(randn(961, (M, K))))
    y = empty_bf16(M, N)
    y.fill_(0x2345)
    sync()
    with pytest.raises(m.MingError) as e:
        ctx.lin_noalloc(qw, x, y, M, None)
    assert e.value.code == m.ERR_SHAPE and "MING_NOALLOC_SCRATCH_BYTES" in str(e.value)
    ctx.synchronize()
    sync()
    assert np.all(from_dev(y) == 0x2345)
    qw.close()
    # a binding changed since the last ming_lin: its stacks are not built
    M, N, K = 200, 256, 512
    qw = _weight(ctx, 970, N, K, 4, (16,))
    x = to_dev(bf16(randn(971, (M, K))))
    y0, y1 = _both(ctx, qw, x, M, [0.5])
    assert np.array_equal(y0, y1)
    A, B = make_lora(975, N, K, 32)
    qw.bind_lora(1, A, B)
    y = empty_bf16(M, N)
    sync()
    with pytest.raises(m.MingError) as e:
        ctx.lin_noalloc(qw, x, y, M, [0.5, 0.25])
    assert e.value.code == m.ERR_STATE
    y0, y1 = _both(ctx, qw, x, M, [0.5, 0.25])   # ming_lin builds them; then equal
    assert np.array_equal(y0, y1)
    qw.close()
