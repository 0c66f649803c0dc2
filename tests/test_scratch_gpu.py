"""Context scratch planes grow independently: growing one never frees
another. Regression: growing the attention V^T plane once freed the
general route's SwiGLU plane too, and the next growth freed that address
again -- by then part of a live weight, which then failed to free."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import bf16, randn, to_dev, empty_bf16, sync, make_weight

pytestmark = pytest.mark.gpu


def _qw(ctx, seed, N, K):
    pack, _ = make_weight(seed, N, K, 4)
    return m.QWeight.quantized(ctx, pack["codes"], pack["scales"],
                               pack["biases"], 4)


def test_scratch_growth_keeps_other_planes(ctx):
    M, H, F = 128, 256, 512
    ctx.set_route("general")
    try:
        w3 = _qw(ctx, 700, F, H)
        x = to_dev(bf16(randn(701, (M, H))))
        g = to_dev(bf16(randn(702, (M, F))))
        out = empty_bf16(M, F)
        sync()
        ctx.lin_swiglu(w3, x, g, out, M)          # allocates the SwiGLU plane
        ctx.synchronize()
        first = out.clone()
    finally:
        ctx.set_route("auto")
    for rows in (512, 2048, 4096):                # grows the V^T plane twice
        qkv = to_dev(bf16(randn(703, (rows, 3 * 128))))
        o = empty_bf16(rows, 128)
        sync()
        ctx.attention(qkv, 3 * 128, 0, 128, 256, o, 128, rows, 1)
        ctx.synchronize()
    # weights made and destroyed after the growth; none may fail
    for i in range(4):
        w = _qw(ctx, 710 + i, 1024, 256)
        w.close()
    ctx.set_route("general")
    try:
        out2 = empty_bf16(M, F)
        sync()
        ctx.lin_swiglu(w3, x, g, out2, M)         # the SwiGLU plane still works
        ctx.synchronize()
    finally:
        ctx.set_route("auto")
    assert np.array_equal(first.cpu().numpy(), out2.cpu().numpy())
    w3.close()
