"""GPU parity of RMSNorm, the rotary tables and the fused qk-norm + RoPE
against the CPU oracle. bf16 outputs may differ from the oracle by one
bf16 ulp where the f32 sum order (a wave reduction vs a serial sum) moves
a value across a rounding boundary; the rel-L2 bar is the north_star's."""
import numpy as np
import pytest

from helpers import bf16, empty_bf16, f32, from_dev, randn, sync, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ulps(a, b):
    return np.abs(a.view(np.int16).astype(np.int32) -
                  b.view(np.int16).astype(np.int32))


@pytest.mark.parametrize("rows,D", [(300, 3840), (4352, 3840), (77, 2560),
                                    (1000, 128), (5, 64), (3, 8192)])
def test_rmsnorm_parity(ctx, orc, rows, D):
    print(f"case rmsnorm rows={rows} D={D}", flush=True)
    x = bf16(randn(rows + D, (rows, D)))
    w = bf16(1.0 + randn(7 + D, (D,), 0.2))
    xd, wd = to_dev(x), to_dev(w)
    y = empty_bf16(rows, D)
    ctx.reset_engagement()
    sync()
    ctx.rmsnorm(xd, wd, y, rows, D)
    sync()
    assert ctx.engagement()["rmsnorm"] == 1
    got = from_dev(y)
    want = orc.rmsnorm(x, w)
    u = _ulps(got, want)
    assert u.max() <= 1 and (u > 0).mean() < 0.01
    assert orc.rel_l2(f32(got), f32(want)) <= TOL


def test_rmsnorm_in_place_and_strided(ctx, orc):
    rows, D = 130, 3840
    x = bf16(randn(3, (rows, 2 * D)))
    w = bf16(1.0 + randn(4, (D,), 0.2))
    xd, wd = to_dev(x), to_dev(w)
    sync()
    ctx.rmsnorm(xd[:, D:], wd, xd[:, D:], rows, D, ldx=2 * D, ldy=2 * D)
    sync()
    got = from_dev(xd)
    assert np.array_equal(got[:, :D], x[:, :D])
    want = orc.rmsnorm(np.ascontiguousarray(x[:, D:]), w)
    assert _ulps(np.ascontiguousarray(got[:, D:]), want).max() <= 1


def test_rope_table_parity(ctx, orc):
    L = orc.build_layout(64, 64, 0, 256)
    n = L["joint_len"]
    import torch
    pt, ph, pw = (to_dev(L[k]) for k in ("pos_t", "pos_h", "pos_w"))
    c = torch.empty((n, 64), dtype=torch.float32, device="cuda")
    s = torch.empty((n, 64), dtype=torch.float32, device="cuda")
    sync()
    ctx.rope_table(pt, ph, pw, n, c, s)
    sync()
    wc, ws = orc.rope_table(L["pos_t"], L["pos_h"], L["pos_w"])
    gc, gs = from_dev(c), from_dev(s)
    # f64 angles on both sides; the f32 results agree to the last bit save
    # for rare double-rounding ties
    assert (gc != wc).mean() < 1e-4 and (gs != ws).mean() < 1e-4
    assert np.max(np.abs(gc - wc)) <= 1.2e-7 and np.max(np.abs(gs - ws)) <= 1.2e-7


@pytest.mark.parametrize("rows,n_heads,ld_extra", [(300, 30, 0), (4352, 30, 3840),
                                                   (33, 2, 0)])
def test_qk_norm_rope_parity(ctx, orc, rows, n_heads, ld_extra):
    print(f"case qk_norm_rope rows={rows} heads={n_heads}", flush=True)
    import torch
    Hd = 128
    width = 2 * n_heads * Hd + ld_extra
    x = bf16(randn(rows, (rows, width)))
    wq = bf16(1.0 + randn(5, (Hd,), 0.2))
    wk = bf16(1.0 + randn(6, (Hd,), 0.2))
    L = orc.build_layout(rows, 1, 0, 1)
    pos = {k: np.ascontiguousarray(L[k][:rows]) for k in ("pos_t", "pos_h", "pos_w")}
    c, s = orc.rope_table(pos["pos_t"], pos["pos_h"], pos["pos_w"])
    xd = to_dev(x)
    cd, sd = torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()
    ctx.reset_engagement()
    sync()
    ctx.qk_norm_rope(xd, width, 0, n_heads * Hd, rows, n_heads, to_dev(wq),
                     to_dev(wk), cd, sd)
    sync()
    assert ctx.engagement()["qk_norm_rope"] == 1
    got = from_dev(xd)
    want = orc.qk_norm_rope(x, 0, n_heads * Hd, n_heads, Hd, wq, wk, c, s)
    # A one-ulp difference in a normalized input (f32 sum order) moves a
    # rotated output by up to an ulp of the PAIR's magnitude, which near
    # cancellation (a*c ~ b*s) is many ulps of the output itself. So the
    # element bound is 2 bf16 ulps of the pair norm the rotation preserves.
    g2 = f32(got)[:, :2 * n_heads * Hd].reshape(rows, -1, 2)
    w2 = f32(want)[:, :2 * n_heads * Hd].reshape(rows, -1, 2)
    pn = np.sqrt((w2.astype(np.float64) ** 2).sum(-1, keepdims=True))
    assert np.all(np.abs(g2 - w2) <= 2.0 ** -6 * pn + 1e-30)
    assert (_ulps(got, want) > 0).mean() < 0.02
    assert orc.rel_l2(f32(got), f32(want)) <= TOL
    # untouched columns past q and k
    assert np.array_equal(got[:, 2 * n_heads * Hd:], x[:, 2 * n_heads * Hd:])
