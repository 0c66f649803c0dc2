"""ming_lin_bias: LlmOps::linear with a bias (ming-ops.h:84-90,
ming-ops.cc:119-141), whose GEMM takes the bias in its epilogue -- the bias
is added to the f32 result before the output's one bf16 rounding. Every
route a dense weight takes: the general kernel (64 tiles or more, and the
general and wide routes), the split-K dense GEMM of few tiles (its reduce,
and its one-slice direct write), and the GEMV (M <= 8)."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import bf16, empty_bf16, f32, from_dev, make_lora, make_weight, randn, sync, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dense(ctx, seed, N, K):
    pack, w = make_weight(seed, N, K, 16, std=1.0 / np.sqrt(K))
    return m.QWeight.dense(ctx, pack["w"]), w


def _run(ctx, qw, x, M, bias, scales=None, plain=False):
    y = empty_bf16(M, qw.N)
    sync()
    if plain:
        ctx.lin(qw, x, y, M, scales)
    else:
        ctx.lin_bias(qw, x, y, M, bias, scales)
    sync()
    return from_dev(y)


CASES = [
    # (M, N, K, what the auto route runs)
    (2048, 2048, 512, "general kernel (64 tiles)"),
    (300, 768, 2560, "split-K dense GEMM and its reduce"),
    (300, 768, 256, "one-slice dense GEMM, direct write"),
    (1, 1024, 640, "GEMV"),
    (8, 1024, 640, "GEMV"),
]


@pytest.mark.parametrize("route", ["auto", "general", "wide"])
@pytest.mark.parametrize("M,N,K,what", CASES)
def test_lin_bias_parity(ctx, orc, M, N, K, what, route):
    print(f"case lin_bias M={M} N={N} K={K} ({what}) route={route}", flush=True)
    qw, w = _dense(ctx, 7000 + K, N, K)
    x = bf16(randn(7100 + M, (M, K)))
    b = bf16(randn(7200 + N, (N,), 0.5))
    xd, bd = to_dev(x), to_dev(b)
    ctx.set_route(route)
    try:
        y = _run(ctx, qw, xd, M, bd)
        ref = orc.proj(x, w) + f32(b)[None, :]
        assert orc.rel_l2(f32(y), ref) <= TOL
        # a zero activation leaves the bias alone, bit for bit
        z = to_dev(np.zeros((M, K), np.uint16))
        assert np.array_equal(_run(ctx, qw, z, M, bd), np.broadcast_to(b, (M, N)))
        # a zero bias is ming_lin (but for the sign of an exact zero)
        y0 = _run(ctx, qw, xd, M, to_dev(np.zeros(N, np.uint16)))
        yp = _run(ctx, qw, xd, M, None, plain=True)
        nz = yp != 0x8000
        assert np.array_equal(y0[nz], yp[nz])
        # one rounding, not ming_lin then a rounded add: the two differ, and
        # the one-rounding output is the closer to the exact result
        two = bf16(f32(yp) + f32(b)[None, :])
        assert not np.array_equal(y, two)
        assert orc.rel_l2(f32(y), ref) <= orc.rel_l2(f32(two), ref)
    finally:
        ctx.set_route("auto")
    qw.close()


def test_lin_bias_with_a_live_adapter(ctx, orc):
    """A dense weight with a live slot: the general kernel's LoRA tail, then
    the bias, then the one rounding."""
    M, N, K = 300, 512, 640
    qw, w = _dense(ctx, 7300, N, K)
    A, B = make_lora(7301, N, K, 16)
    qw.bind_lora(2, A, B)
    sc = [0.0, 0.0, 0.8, 0.0, 0.0, 0.0, 0.0, 0.0]
    x = bf16(randn(7302, (M, K)))
    b = bf16(randn(7303, (N,), 0.5))
    y = _run(ctx, qw, to_dev(x), M, to_dev(b), sc)
    ref = orc.proj(x, w, [(A, B, 0.8)]) + f32(b)[None, :]
    assert orc.rel_l2(f32(y), ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w) + f32(b)[None, :]) > 10 * TOL
    qw.close()


def test_lin_bias_refusals(ctx):
    pack, _ = make_weight(7400, 256, 256, 4)
    q4 = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], 4)
    x = to_dev(bf16(randn(7401, (64, 256))))
    y = empty_bf16(64, 256)
    b = to_dev(bf16(randn(7402, (256,))))
    with pytest.raises(m.MingError, match="dense"):
        ctx.lin_bias(q4, x, y, 64, b)
    qd, _ = _dense(ctx, 7403, 256, 256)
    with pytest.raises(m.MingError):
        ctx.lin_bias(qd, x, y, 64, None)
    q4.close()
    qd.close()
