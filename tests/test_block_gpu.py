"""One DiT block (run_block, ming-dit.cc:2065-2263) through ming_block_forward
against the oracle's composition of the same pieces, at reduced width (H=256,
2 heads, ffn 512) where the f64 oracle runs in seconds; config 3's full size
(H 3840, 30 heads, ffn 10240, 4352 rows) by size-independent properties.

Tolerances (rel-L2 against the f64 oracle): the block output at 1e-2 and
the block's update (output - input) at 2e-2. A block chains five
projection stages (q/k/v -> attention -> o, then w1/w3 -> w2), each held
to the projection bar of 2e-3 (fp16 dequant tiles, bf16 LoRA
intermediate), plus attention's bf16 P; the errors add roughly in
quadrature to ~5e-3 on the update. On an unmodulated block the update is
as large as the residual stream (no tanh gate), so the output sees it
undiminished.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import (CFG2_RANKS, CFG2_SCALES, bf16, f32, randn, to_dev,
                     from_dev, sync, build_block, grid_positions)

pytestmark = pytest.mark.gpu

H, NH, F, ADA = 256, 2, 512, 64
SCALES = (1.0, 0.0, 0.0, -0.5, 0.0, 0.0, 0.0, 0.0)


def dims():
    import ming_dit_amd as m
    return m.BlockDims(H, NH, F, ADA, 1e-5)


def tables(rows, row0=0):
    pt, ph, pw = grid_positions(rows + row0)
    c, s = orc.rope_table(pt, ph, pw)
    return c[row0:], s[row0:]


def run_gpu(ctx, desc, d, x, rows, c, s, temb, scales):
    xd = to_dev(x)
    cd, sd = to_dev(np.ascontiguousarray(c)), to_dev(np.ascontiguousarray(s))
    td = to_dev(temb) if temb is not None else None
    sync()
    ctx.block_forward(desc, d, xd, rows, cd, sd, td, scales)
    ctx.synchronize()
    return from_dev(xd)


@pytest.mark.parametrize("modulated,rows,bits", [(True, 200, 4), (False, 96, 4),
                                                 (True, 130, 8)])
def test_block_matches_oracle(ctx, modulated, rows, bits):
    ob, gp, desc = build_block(ctx, 500 + rows, H, F, ADA, bits, modulated)
    x = bf16(randn(41, (rows, H)))
    temb = bf16(randn(43, (ADA,))) if modulated else None
    c, s = tables(rows)
    got = run_gpu(ctx, desc, dims(), x, rows, c, s, temb, SCALES)
    ref = orc.block_forward(x, ob, NH, c, s, temb, SCALES)
    err = orc.rel_l2(f32(got), f32(ref))
    upd = orc.rel_l2(f32(got) - f32(x), f32(ref) - f32(x))
    print(f"block modulated={modulated} rows={rows} w{bits}: output rel-L2 "
          f"{err:.3e}, update rel-L2 {upd:.3e}")
    assert err <= 1e-2, f"block output rel-L2 {err:.3e}"
    assert upd <= 2e-2, f"block update rel-L2 {upd:.3e}"


def test_block_rope_row_offset(ctx):
    """Context-refiner style: tables taken from row IMG of the joint table."""
    rows, row0 = 80, 64
    ob, gp, desc = build_block(ctx, 777, H, F, ADA, 4, modulated=False)
    x = bf16(randn(45, (rows, H)))
    c, s = tables(rows, row0)
    got = run_gpu(ctx, desc, dims(), x, rows, c, s, None, SCALES)
    ref = orc.block_forward(x, ob, NH, c, s, None, SCALES)
    err = orc.rel_l2(f32(got), f32(ref))
    print(f"block rope row offset: output rel-L2 {err:.3e}")
    assert err <= 1e-2


def test_block_zero_strengths_equal_unbound(ctx):
    """All eight strengths 0 == the same block with no adapter bound, bit for
    bit (ming-dit-test.cc:1249-1273)."""
    rows = 150
    _, gp_a, desc_a = build_block(ctx, 900, H, F, ADA, 4, True)
    _, gp_b, desc_b = build_block(ctx, 900, H, F, ADA, 4, True, slots=())
    x = bf16(randn(47, (rows, H)))
    temb = bf16(randn(49, (ADA,)))
    c, s = tables(rows)
    a = run_gpu(ctx, desc_a, dims(), x, rows, c, s, temb, [0.0] * 8)
    b = run_gpu(ctx, desc_b, dims(), x, rows, c, s, temb, [0.0] * 8)
    assert np.array_equal(a, b)
    live = run_gpu(ctx, desc_a, dims(), x, rows, c, s, temb, SCALES)
    assert not np.array_equal(a, live)


def test_block_rejects_bad_desc(ctx):
    import ming_dit_amd as m
    rows = 64
    ob, gp, desc = build_block(ctx, 950, H, F, ADA, 4, True)
    x = to_dev(bf16(randn(51, (rows, H))))
    c, s = tables(rows)
    cd, sd = to_dev(np.ascontiguousarray(c)), to_dev(np.ascontiguousarray(s))
    with pytest.raises(m.MingError):          # modulated block without temb
        ctx.block_forward(desc, dims(), x, rows, cd, sd, None, SCALES)
    bad = m.block_desc(**dict(gp, w2=gp["w1"]))   # w2 of the wrong shape
    with pytest.raises(m.MingError):
        ctx.block_forward(bad, dims(), x, rows, cd, sd,
                          to_dev(bf16(randn(53, (ADA,)))), SCALES)


def test_block_config3_full_size(ctx):
    """Config 3: H 3840, 30 heads, ffn 10240, 4352 rows, w4g64, the config-2
    adapter set on all seven projections. Against the fp32 reference
    (tests/torch_ref.py, pinned to the oracle at reduced width) by the
    reference's own rule for full-size checks (ming-dit-test.cc:2131): within
    twice the distance of a bf16 run from f32, floored at the reduced-width
    bars (output 1e-2, update 2e-2). Then finite, deterministic, and all
    strengths 0 equal to the unadapted block bit for bit."""
    import torch
    import ming_dit_amd as m
    import torch_ref as tr
    Hf, NHf, Ff, ADAf, rows = 3840, 30, 10240, 256, 4352
    gen = torch.Generator(device="cuda").manual_seed(3)
    packs = {}

    def qw(N, K):
        w = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        codes = torch.empty((N, K // 8), dtype=torch.int32, device="cuda")
        sc = torch.empty((N, K // 64), dtype=torch.int16, device="cuda")
        bi = torch.empty((N, K // 64), dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        ctx.quantize_pack(w, N, K, 4, codes, sc, bi)
        ctx.synchronize()
        q = m.QWeight.quantized(ctx, codes, sc, bi, 4, on_device=True)
        packs[id(q)] = {"codes": codes, "scales": sc, "biases": bi, "bits": 4}
        return q

    def vec(n, base=1.0, std=0.1):
        v = base + std * torch.randn((n,), generator=gen, device="cuda")
        return v.to(torch.bfloat16).view(torch.int16).contiguous()

    shapes = {"q": (Hf, Hf), "k": (Hf, Hf), "v": (Hf, Hf), "o": (Hf, Hf),
              "w1": (Ff, Hf), "w3": (Ff, Hf), "w2": (Hf, Ff)}
    parts = {n: qw(*sh) for n, sh in shapes.items()}
    ref_blk = {"loras": {n: [] for n in shapes}}
    for n, (N, K) in shapes.items():
        for slot, r in enumerate(CFG2_RANKS):
            A = (torch.randn((r, K), generator=gen, device="cuda") / K ** 0.5
                 ).to(torch.bfloat16).view(torch.int16)
            B = (torch.randn((N, r), generator=gen, device="cuda") * 0.01
                 ).to(torch.bfloat16).view(torch.int16)
            torch.cuda.synchronize()
            parts[n].bind_lora(slot, A, B, 1.0, on_device=True)
            ref_blk["loras"][n].append((A, B, 1.0))
    ada = qw(4 * Hf, ADAf)
    gains = dict(ada_b=vec(4 * Hf, 0.0, 0.1), an1=vec(Hf), an2=vec(Hf),
                 fn1=vec(Hf), fn2=vec(Hf), nq=vec(128), nk=vec(128))
    desc = m.block_desc(ada=ada, **parts, **gains)
    d = m.BlockDims(Hf, NHf, Ff, ADAf, 1e-5)
    x0 = (torch.randn((rows, Hf), generator=gen, device="cuda")
          ).to(torch.bfloat16).view(torch.int16)
    temb = (torch.randn((ADAf,), generator=gen, device="cuda")
            ).to(torch.bfloat16).view(torch.int16)
    # config 3's positions: the 64 x 64 patch grid at (257, h, w), then the
    # 256 text rows at (1 + i, 0, 0)
    img, cap = 4096, 256
    pt = np.concatenate([np.full(img, cap + 1), 1 + np.arange(cap)]).astype(np.int32)
    ph = np.concatenate([np.arange(img) // 64, np.zeros(cap)]).astype(np.int32)
    pw = np.concatenate([np.arange(img) % 64, np.zeros(cap)]).astype(np.int32)
    c, s = orc.rope_table(pt, ph, pw)
    cd, sd = to_dev(c), to_dev(s)
    ws = torch.empty(ctx.block_workspace_bytes(d, rows), dtype=torch.uint8,
                     device="cuda")

    def run(dsc, scales):
        x = x0.clone()
        torch.cuda.synchronize()
        ctx.block_forward(dsc, d, x, rows, cd, sd, temb, scales, ws)
        ctx.synchronize()
        return from_dev(x)

    a = run(desc, CFG2_SCALES)
    assert np.all(np.isfinite(f32(a)))
    assert not np.array_equal(a, from_dev(x0))
    # the fp32 reference, and the bf16 run that sets the bar
    ref_blk.update({n: packs[id(q)] for n, q in dict(parts, ada=ada).items()})
    ref_blk.update(gains)
    x0f = tr.bf(x0, "cuda")
    ct, st = torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()
    tt = tr.bf(temb, "cuda")
    outs = {}
    for mode in ("f32", "bf16"):
        outs[mode] = tr.Ref(mode, "cuda").block(x0f, ref_blk, NHf, ct, st, tt, CFG2_SCALES)
        torch.cuda.synchronize()
    got = torch.from_numpy(f32(a)).cuda()
    rel = tr.rel_l2(got, outs["f32"])
    upd = tr.rel_l2(got - x0f, outs["f32"] - x0f)
    bar_out = max(1e-2, 2 * tr.rel_l2(outs["bf16"], outs["f32"]))
    bar_upd = max(2e-2, 2 * tr.rel_l2(outs["bf16"] - x0f, outs["f32"] - x0f))
    print(f"configs[2] block vs fp32: output {rel:.3e} (bar {bar_out:.3e}), update "
          f"{upd:.3e} (bar {bar_upd:.3e}); vs the bf16 run: update "
          f"{tr.rel_l2(got - x0f, outs['bf16'] - x0f):.3e}", flush=True)
    assert rel <= bar_out and upd <= bar_upd
    del outs, got
    assert np.array_equal(a, run(desc, CFG2_SCALES))
    z = run(desc, [0.0] * 8)
    assert not np.array_equal(a, z)
    # strengths 0 on the adapted weights == no adapter at all: the same
    # packs with every slot unbound
    for n in shapes:
        for slot in range(8):
            parts[n].unbind_lora(slot)
    assert np.array_equal(z, run(desc, [0.0] * 8))


def public_block(ctx, gp, x, rows, c, s, temb, scales, modulated):
    """run_block's attention half and the feed-forward pre-norm composed from
    the public entry points one by one (each projection converting its own
    input, the post-norm in place, then the residual kernel): the sequence
    the block driver fuses."""
    import torch
    Hh = H
    xd = to_dev(x)
    cd, sd = to_dev(np.ascontiguousarray(c)), to_dev(np.ascontiguousarray(s))
    dev = lambda *sh: torch.empty(sh, dtype=torch.int16, device="cuda")
    nrm, qkv, ob, ffg = dev(rows, Hh), dev(rows, 3 * Hh), dev(rows, Hh), dev(rows, F)
    g1, g3 = gp["an1"], gp["fn1"]
    if modulated:
        mods, nw1, nw3 = dev(1, 4 * Hh), dev(1, Hh), dev(1, Hh)
        ctx.lin(gp["ada"], to_dev(temb), mods, 1, None)
        ctx.bias_act(mods, gp["ada_b"], 1, 4 * Hh)
        ctx.modulate(gp["an1"], mods, nw1, 1, Hh)
        ctx.modulate(gp["fn1"], mods[:, 2 * Hh:], nw3, 1, Hh)
        g1, g3 = nw1, nw3
    sync()
    ctx.rmsnorm(xd, g1, nrm, rows, Hh)
    ctx.lin(gp["q"], nrm, qkv, rows, scales, ldy=3 * Hh)
    ctx.lin(gp["k"], nrm, qkv[:, Hh:], rows, scales, ldy=3 * Hh)
    ctx.lin(gp["v"], nrm, qkv[:, 2 * Hh:], rows, scales, ldy=3 * Hh)
    ctx.qk_norm_rope(qkv, 3 * Hh, 0, Hh, rows, NH, gp["nq"], gp["nk"], cd, sd)
    ctx.attention(qkv, 3 * Hh, 0, Hh, 2 * Hh, nrm, Hh, rows, NH, 1.0 / np.sqrt(128.0))
    ctx.lin(gp["o"], nrm, ob, rows, scales)
    ctx.rmsnorm(ob, gp["an2"], ob, rows, Hh)
    if modulated:
        ctx.gated_residual(xd, mods[:, Hh:], ob, rows, Hh)
    else:
        ctx.residual_add(xd, ob, rows, Hh)
    ctx.rmsnorm(xd, g3, nrm, rows, Hh)
    return xd, nrm, qkv, ob, ffg, g3, mods if modulated else None


@pytest.mark.parametrize("route", ["auto", "general"])
@pytest.mark.parametrize("modulated", [True, False])
def test_block_forward_equals_the_public_calls(ctx, modulated, route):
    """The block driver's fusions (the norm writing the fp16 copy q, k, v and
    w1, w3 read; post-norm + residual in one pass) give the same bits as the
    public entry points called one by one, on either projection route."""
    import torch
    rows = 136
    ob, gp, desc = build_block(ctx, 900 + modulated, H, F, ADA, 4, modulated)
    x = bf16(randn(47, (rows, H)))
    temb = bf16(randn(49, (ADA,))) if modulated else None
    c, s = tables(rows)
    ctx.set_route(route)
    try:
        ctx.reset_engagement()
        got = run_gpu(ctx, desc, dims(), x, rows, c, s, temb, SCALES)
        eng = ctx.engagement()
        assert eng["qk_norm_rope"] == 1
        assert (eng["gemm_fast"] > 0) == (route == "auto")
        xd, nrm, qkv, obd, ffg, g3, mods = public_block(ctx, gp, x, rows, c, s, temb,
                                                        SCALES, modulated)
        # the feed-forward half, public calls
        y = torch.empty((rows, H), dtype=torch.int16, device="cuda")
        ctx.ffn(gp["w1"], gp["w3"], gp["w2"], nrm, y, rows, SCALES, h=ffg)
        ctx.rmsnorm(y, gp["fn2"], y, rows, H)
        if modulated:
            ctx.gated_residual(xd, mods[:, 3 * H:], y, rows, H)
        else:
            ctx.residual_add(xd, y, rows, H)
        ctx.synchronize()
    finally:
        ctx.set_route("auto")
    want = from_dev(xd)
    assert np.array_equal(got, want)
