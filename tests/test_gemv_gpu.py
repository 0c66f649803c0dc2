"""The projection at a handful of rows (route 'auto', M <= 8, no live adapter)
runs the GEMV: parity against the fp32 dequant+GEMM oracle at the shapes the
forward uses it at (the adaLN [4H, adaln_dim] at M = 1, the timestep MLP) and
ragged ones, for w4, w8 and dense bf16 weights.

Bar (north_star): rel-L2 <= 2e-3 against the fp32 reference; strength 0 is
bit-identical to no adapter (ming-dit-test.cc:1249-1273). Engagement is
asserted before accuracy (ming-dit.h:55-103)."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import (bf16, empty_bf16, from_dev, make_lora, make_weight, randn,
                     sync, to_dev)

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _qw(ctx, pack, bits):
    if bits == 16:
        return m.QWeight.dense(ctx, pack["w"])
    return m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)


def _run(ctx, qw, xd, M, scales=None, ldx=None, ldy=None):
    ldy = ldy or qw.N
    y = empty_bf16(M, ldy)
    sync()
    ctx.reset_engagement()
    ctx.lin(qw, xd, y, M, scales, ldx=ldx, ldy=ldy)
    sync()
    return from_dev(y)[:, :qw.N], ctx.engagement()


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(1, 15360, 256), (1, 3840, 1024), (3, 264, 3840),
                                   (8, 1000, 192)])
def test_gemv_parity(ctx, orc, bits, M, N, K):
    print(f"case bits={bits} M={M} N={N} K={K}", flush=True)
    x = bf16(randn(8000 + M, (M, K)))
    pack, w = make_weight(8100 + N % 89, N, K, bits)
    qw = _qw(ctx, pack, bits)
    y, eng = _run(ctx, qw, to_dev(x), M)
    key = {4: "gemm_q4", 8: "gemm_q8", 16: "gemm_dense"}[bits]
    assert eng["gemv"] == 1 and eng[key] == 1 and eng["gemm_fast"] == 0
    assert eng["gemm_flops"] == 2 * M * N * K
    ref = orc.proj(x, w)
    assert orc.rel_l2(orc.bf16_to_f32(y), ref) <= TOL
    qw.close()


def test_gemv_strided_rows(ctx, orc):
    """Row strides in and out (ldx > K, ldy > N): only the M x N block is
    written."""
    M, N, K = 5, 512, 640
    ldx, ldy = K + 64, N + 40
    x = bf16(randn(8201, (M, ldx)))
    pack, w = make_weight(8202, N, K, 4)
    qw = _qw(ctx, pack, 4)
    y = to_dev(np.full((M, ldy), 0x1234, np.uint16))
    sync()
    ctx.lin(qw, to_dev(x), y, M, ldx=ldx, ldy=ldy)
    sync()
    out = from_dev(y)
    assert (out[:, N:] == 0x1234).all()
    ref = orc.proj(np.ascontiguousarray(x[:, :K]), w)
    assert orc.rel_l2(orc.bf16_to_f32(np.ascontiguousarray(out[:, :N])), ref) <= TOL
    qw.close()


def test_gemv_agrees_with_the_general_route(ctx, orc):
    """The GEMV and the general kernel compute the same function: both within
    the bar. The GEMV dequantizes in f32 without rounding the weights, so it
    is no further from the fp32 reference than the general kernel; the two
    differ by output roundings (outputs whose f32 values straddle a bf16
    rounding boundary)."""
    M, N, K = 1, 15360, 256
    xh = bf16(randn(8301, (M, K)))
    x = to_dev(xh)
    pack, w = make_weight(8302, N, K, 8)
    qw = _qw(ctx, pack, 8)
    yg, eg = _run(ctx, qw, x, M)
    ctx.set_route("general")
    try:
        yk, ek = _run(ctx, qw, x, M)
    finally:
        ctx.set_route("auto")
    assert eg["gemv"] == 1 and ek["gemv"] == 0
    ref = orc.proj(xh, w)
    rg = orc.rel_l2(orc.bf16_to_f32(yg), ref)
    rk = orc.rel_l2(orc.bf16_to_f32(yk), ref)
    print(f"rel-L2 vs fp32: gemv {rg:.3e}, general {rk:.3e}")
    assert rg <= TOL and rk <= TOL and rg <= rk + 1e-4
    assert orc.rel_l2(orc.bf16_to_f32(yg), orc.bf16_to_f32(yk)) < TOL
    qw.close()


def test_gemv_strength_zero_and_live_adapters(ctx, orc):
    """Adapters bound at strength 0 stay on the GEMV, bit-identical to the
    unadapted weight; a live adapter takes the adapter route, to the bar."""
    M, N, K = 2, 768, 512
    x = bf16(randn(8401, (M, K)))
    xd = to_dev(x)
    pack, w = make_weight(8402, N, K, 4)
    qw, plain = _qw(ctx, pack, 4), _qw(ctx, pack, 4)
    A, B = make_lora(8403, N, K, 16)
    qw.bind_lora(1, A, B)
    y0, e0 = _run(ctx, qw, xd, M, [0.0, 0.0])
    yp, ep = _run(ctx, plain, xd, M)
    assert e0["gemv"] == 1 and ep["gemv"] == 1 and e0["lora_proj"] == 0
    assert np.array_equal(y0, yp)
    yl, el = _run(ctx, qw, xd, M, [0.0, 0.9])
    assert el["gemv"] == 0 and el["lora_proj"] == 1
    ref = orc.proj(x, w, [(A, B, 0.9)])
    assert orc.rel_l2(orc.bf16_to_f32(yl), ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w)) > 10 * TOL
    qw.close()
    plain.close()
