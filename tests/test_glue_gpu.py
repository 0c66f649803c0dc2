"""GPU parity of the block glue (SwiGLU, gated/plain residual, modulation,
bias+SiLU, the final LayerNorm) and the pack quantizer against the oracle,
plus the profiler's buckets."""
import numpy as np
import pytest
import torch

from helpers import bf16, empty_bf16, f32, from_dev, randn, sync, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ulps(a, b):
    return np.abs(a.view(np.int16).astype(np.int32) - b.view(np.int16).astype(np.int32))


def test_swiglu(ctx, orc):
    rows, n = 300, 10240
    g = bf16(randn(1, (rows, n), 2.0))
    u = bf16(randn(2, (rows, n)))
    out = empty_bf16(rows, n)
    sync()
    ctx.swiglu(to_dev(g), to_dev(u), out, rows, n)
    sync()
    got, want = from_dev(out), orc.swiglu(g, u)
    # expf on the GPU vs glibc: at most one bf16 ulp, rarely
    assert _ulps(got, want).max() <= 1 and (got != want).mean() < 1e-3


@pytest.mark.parametrize("gated", [True, False])
def test_residuals(ctx, orc, gated):
    rows, n = 257, 3840
    h = bf16(randn(3, (rows, n)))
    sub = bf16(randn(4, (rows, n)))
    gate = bf16(randn(5, (n,)))
    hd = to_dev(h)
    sync()
    if gated:
        ctx.gated_residual(hd, to_dev(gate), to_dev(sub), rows, n)
        want = orc.gated_residual(h, gate, sub)
        term = np.tanh(f32(gate).astype(np.float64)) * f32(sub)
    else:
        ctx.residual_add(hd, to_dev(sub), rows, n)
        want = bf16(f32(h) + f32(sub))
        term = f32(sub).astype(np.float64)
    sync()
    got = from_dev(hd)
    # The kernel rounds the product, then the sum, as the oracle does; tanhf
    # may still differ by an f32 ulp between the GPU and glibc, which near
    # cancellation is many ulps of the sum, so bound by the operands. Such
    # elements are rare (measured: 2e-5 of them).
    mag = np.abs(f32(h)) + np.abs(term)
    assert np.all(np.abs(f32(got) - f32(want)) <= 2.0 ** -8 * mag + 1e-30)
    assert (got != want).mean() < 1e-3


def test_modulate_is_fold_gain(ctx, orc):
    n = 3840
    w = bf16(randn(6, (n,)))
    s = bf16(randn(7, (n,), 0.3))
    y = empty_bf16(1, n)
    sync()
    ctx.modulate(to_dev(w), to_dev(s), y, 1, n)
    sync()
    assert np.array_equal(from_dev(y)[0], orc.fold_gain(w, s))


@pytest.mark.parametrize("silu", [False, True])
def test_bias_act(ctx, orc, silu):
    rows, n = 3, 15360
    y = bf16(randn(8, (rows, n)))
    b = bf16(randn(9, (n,)))
    yd = to_dev(y)
    sync()
    ctx.bias_act(yd, to_dev(b), rows, n, silu)
    sync()
    got, want = from_dev(yd), orc.bias_act(y, b, silu)
    assert _ulps(got, want).max() <= 1 and (got != want).mean() < 1e-3


def test_ln_modulate(ctx, orc):
    rows, D = 100, 3840
    x = bf16(randn(10, (rows, D), 3.0))
    s = bf16(randn(11, (D,), 0.2))
    y = empty_bf16(rows, D)
    sync()
    ctx.ln_modulate(to_dev(x), to_dev(s), y, rows, D, 1e-6)
    sync()
    got, want = from_dev(y), orc.ln_modulate(x, s, 1e-6)
    assert _ulps(got, want).max() <= 2 and (got != want).mean() < 2e-2
    assert orc.rel_l2(f32(got), f32(want)) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_pack_bit_exact(ctx, orc, bits):
    """The GPU pack writer is integer work: bit-exact with the oracle."""
    N, K = 512, 3840
    w = randn(20 + bits, (N, K), 0.02)
    w[3, :64] = 0.0                      # an all-zero group
    w[4, 64:128] = 0.5                   # a constant group
    wd = torch.from_numpy(w).cuda()
    codes = torch.empty((N, K * bits // 32), dtype=torch.int32, device="cuda")
    sc = empty_bf16(N, K // 64)
    bi = empty_bf16(N, K // 64)
    sync()
    ctx.quantize_pack(wd, N, K, bits, codes, sc, bi)
    sync()
    c_ref, s_ref, b_ref = orc.quantize(w, bits)
    assert np.array_equal(codes.cpu().numpy().view(np.uint32), c_ref)
    assert np.array_equal(from_dev(sc), s_ref)
    assert np.array_equal(from_dev(bi), b_ref)


def test_profiler_buckets(ctx, orc):
    rows, n = 64, 1024
    g = to_dev(bf16(randn(30, (rows, n))))
    out = empty_bf16(rows, n)
    ctx.profile_collect()
    ctx.set_profiling(True)
    sync()
    for _ in range(3):
        ctx.swiglu(g, g, out, rows, n)
    prof = ctx.profile_collect()
    ctx.set_profiling(False)
    assert prof["swiglu"]["launches"] == 3 and prof["swiglu"]["ms"] > 0
    assert prof["swiglu"]["bytes"] == 3 * 6.0 * rows * n
    ctx.swiglu(g, g, out, rows, n)
    assert ctx.profile_collect() == {}
