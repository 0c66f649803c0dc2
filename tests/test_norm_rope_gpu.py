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
                                                   (33, 2, 0),
                                                   # more row pairs than the grid's y
                                                   # extent (65535): the grid-stride loop
                                                   (140000, 1, 0)])
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
    # The kernel rounds where the oracle does (each product of the rotation,
    # then the sum); only the head's sum of squares runs in another order.
    # A one-ulp difference in a normalized input moves a rotated output by
    # up to an ulp of the PAIR's magnitude, which near cancellation
    # (a*c ~ b*s) is many ulps of the output itself. So the element bound is
    # 2 bf16 ulps of the pair norm the rotation preserves, and such elements
    # are rare (measured: 3e-6 of them at 4352 rows).
    g2 = f32(got)[:, :2 * n_heads * Hd].reshape(rows, -1, 2)
    w2 = f32(want)[:, :2 * n_heads * Hd].reshape(rows, -1, 2)
    pn = np.sqrt((w2.astype(np.float64) ** 2).sum(-1, keepdims=True))
    assert np.all(np.abs(g2 - w2) <= 2.0 ** -6 * pn + 1e-30)
    assert (_ulps(got, want) > 0).mean() < 1e-3
    assert orc.rel_l2(f32(got), f32(want)) <= TOL
    # untouched columns past q and k
    assert np.array_equal(got[:, 2 * n_heads * Hd:], x[:, 2 * n_heads * Hd:])


def _llm_tables(rows, R, theta=10000.0):
    """1-D positions 0..rows-1 at R frequencies theta^(-j/R) (the encoder's
    plain rotary), f64 angles stored f32 [rows][R]."""
    inv = theta ** (-np.arange(R, dtype=np.float64) / R)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("rows,n_q,n_k,n_v,rot_half,norm", [
    (300, 16, 4, 4, 64, True),        # grouped keys, the whole head rotated
    (4352, 30, 30, 30, 64, True),     # the DiT's head count at 1024^2
    (257, 14, 2, 2, 32, True),        # partial rotary: dims 64..127 pass through
    (100, 8, 8, 0, 0, True),          # norm only
    (100, 8, 2, 2, 64, False),        # rotation only
    (140000, 1, 1, 1, 32, True),      # more row pairs than the grid's y extent (65535)
])
def test_llm_qk_norm_rope_parity(ctx, orc, rows, n_q, n_k, n_v, rot_half, norm):
    """LlmOps::qk_norm_rope (ming-ops.h:118-122; ming_llm.metal:100-178)
    through ming_llm_qk_norm_rope against the oracle: q heads then k heads
    from column 0 of the fused rows, value columns untouched, rotate-half of
    width 64 / 32 / 0, norm with both weights or none."""
    print(f"case llm_qk_norm_rope rows={rows} nq={n_q} nk={n_k} rot={rot_half} "
          f"norm={norm}", flush=True)
    import torch
    stride = (n_q + n_k + n_v) * 128 + 8
    x = bf16(randn(900 + rows, (rows, stride)))
    qw = bf16(1.0 + randn(901, (128,), 0.2)) if norm else None
    kw = bf16(0.7 + randn(902, (128,), 0.2)) if norm else None
    c = s = None
    if rot_half:
        c, s = _llm_tables(rows, rot_half)
    xd = to_dev(x)
    dev = {k: (None if v is None else (to_dev(v) if v.dtype == np.uint16 else
                                        torch.from_numpy(v).cuda()))
           for k, v in (("qw", qw), ("kw", kw), ("c", c), ("s", s))}
    ctx.reset_engagement()
    sync()
    ctx.llm_qk_norm_rope(xd, dev["qw"], dev["kw"], dev["c"], dev["s"], rows, stride,
                         n_q, n_k, rot_half, 1e-6)
    sync()
    assert ctx.engagement()["qk_norm_rope"] == 1
    got = from_dev(xd)
    want = orc.llm_qk_norm_rope(x, qw, kw, c, s, n_q, n_k, rot_half, 1e-6)
    nh = (n_q + n_k) * 128
    assert np.array_equal(got[:, nh:], x[:, nh:])           # the values and the tail
    u = _ulps(got[:, :nh], want[:, :nh])
    if not norm:
        # the rotation alone: each product rounded, then the sum, as the
        # oracle rounds -- the same bits
        assert np.array_equal(got, want)
    if rot_half == 0:
        assert u.max() <= 1 and (u > 0).mean() < 1e-3
    else:
        # a one-ulp difference in a normalized input moves a rotated output by
        # up to an ulp of its pair's magnitude: bound each element by 2 bf16
        # ulps of the pair norm the rotation preserves
        R = rot_half
        g = f32(got[:, :nh]).reshape(rows, n_q + n_k, 128).astype(np.float64)
        w = f32(want[:, :nh]).reshape(rows, n_q + n_k, 128).astype(np.float64)
        pn = np.sqrt(w[..., :R] ** 2 + w[..., R:2 * R] ** 2)
        pn = np.concatenate([pn, pn], axis=-1)
        assert np.all(np.abs(g[..., :2 * R] - w[..., :2 * R]) <= 2.0 ** -6 * pn + 1e-30)
        assert (u > 0).mean() < 1e-3
        if R == 32:
            assert _ulps(got[:, :nh].reshape(rows, -1, 128)[..., 64:],
                         want[:, :nh].reshape(rows, -1, 128)[..., 64:]).max() <= 1
    assert orc.rel_l2(f32(got[:, :nh]), f32(want[:, :nh])) <= TOL


def test_llm_qk_norm_rope_refusals(ctx):
    import ming_dit_amd as m
    x = empty_bf16(4, 3 * 128)
    c = empty_bf16(4, 128)           # 4 x 64 f32 worth of bytes
    with pytest.raises(m.MingError):  # rot_half 16 is no mode
        ctx.llm_qk_norm_rope(x, None, None, c, c, 4, 3 * 128, 1, 1, 16, 1e-6)
    with pytest.raises(m.MingError):  # heads past the row
        ctx.llm_qk_norm_rope(x, None, None, c, c, 4, 3 * 128, 2, 2, 64, 1e-6)
    with pytest.raises(m.MingError):  # a rotation without its tables
        ctx.llm_qk_norm_rope(x, None, None, None, None, 4, 3 * 128, 1, 1, 64, 1e-6)
