"""BASELINE configs[3] and configs[4] at full size (16640-token joint sequences,
all 34 blocks, 238 adapted modules).

Each config's velocity is held against an fp32 reference of the whole forward
(tests/torch_ref.py on the GPU, pinned to the CPU oracle at reduced width) by
the reference's own rule for its real-size check (ming-dit-test.cc:2107-2131)
and its w8 check (ming-quant-test.cc:826-831): within twice the distance of a
bf16 run from f32, floored at kSmallTol = 0.035 -- configs[3] (w4) at one
sigma, configs[4] (w8, eight rank-64 slots) on both forwards of its CFG pair.
Both configs are also held to the size-independent properties the reference's
own tests state (ming-dit-test.cc:1249-1273, 2030-2035):
  * strengths changed between forwards and changed back give identical bits;
  * all strengths 0 is bit-identical to the same weights with no adapter bound;
  * the adapters move the output, and every projection carried them;
  * the denoise loop at 2048^2 with CFG is deterministic and finite."""
import sys

import numpy as np
import pytest

import oracle as orc
from helpers import f32, from_dev

pytestmark = pytest.mark.gpu


def _bench():
    import os
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    return bench


def _forward(model, torch, lat, capt, img, cap, pos):
    out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    assert model.forward(lat, capt, 2560, img, cap, cap, *pos, 0.5, out)
    torch.cuda.synchronize()
    return from_dev(out)


def test_config4_forward_2048_strengths_live(ctx):
    import torch
    import ming_dit_amd as m
    import torch_ref as tr
    bench = _bench()
    gen = torch.Generator(device="cuda").manual_seed(41)
    ref = {}
    model = bench.build_forward_model(ctx, m, torch, gen, ref=ref)
    model.set_caption_cache(False)
    img, cap, pos = bench.layout_2048()
    lat = torch.randn((img, 64), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    for i, s in enumerate(bench.SCALES):
        model.set_lora_scale(i, s)
    ctx.reset_engagement()
    a = _forward(model, torch, lat, capt, img, cap, pos)
    assert ctx.engagement()["lora_proj"] == 238          # 7 x 34, every one adapted
    assert np.isfinite(f32(a)).all()
    # the fp32 reference of the same forward, and the bf16 run that sets the bar
    c, s = orc.rope_table(*pos)
    tin = orc.time_proj(0.5, 1000.0, 256)
    outs = {}
    for mode in ("f32", "bf16"):
        outs[mode] = tr.Ref(mode, "cuda").forward(ref, lat, capt, img, cap, cap, c, s, 0.5,
                                                  bench.SCALES, tin)
        torch.cuda.synchronize()
        print(f"2048^2: {mode} reference forward done", flush=True)
    got = torch.from_numpy(f32(a)).cuda()
    rel = tr.rel_l2(got, outs["f32"])
    bf_floor = tr.rel_l2(outs["bf16"], outs["f32"])
    bar = max(0.035, 2 * bf_floor)
    print(f"configs[3] velocity vs fp32: {rel:.3e} (bf16 run {bf_floor:.3e}, bar {bar:.3e}); "
          f"vs the bf16 run {tr.rel_l2(got, outs['bf16']):.3e}", flush=True)
    assert rel <= bar
    del outs, got, ref
    other = (0.3, -0.5, 0.0, 1.0, 0.0, 0.7, 0.0, -0.25)
    for i, s in enumerate(other):
        model.set_lora_scale(i, s)
    b = _forward(model, torch, lat, capt, img, cap, pos)
    for i, s in enumerate(bench.SCALES):
        model.set_lora_scale(i, s)
    c = _forward(model, torch, lat, capt, img, cap, pos)
    assert np.array_equal(a, c)                           # changed and back: same bits
    for i in range(8):
        model.set_lora_scale(i, 0.0)
    ctx.reset_engagement()
    z = _forward(model, torch, lat, capt, img, cap, pos)
    assert ctx.engagement()["lora_proj"] == 0
    for q in model.projections:                          # now truly unadapted
        for slot in range(8):
            q.unbind_lora(slot)
    u = _forward(model, torch, lat, capt, img, cap, pos)
    assert np.array_equal(z, u)                           # strength 0 == no adapter
    moved_a = orc.rel_l2(f32(a), f32(z))
    moved_b = orc.rel_l2(f32(b), f32(a))
    print(f"2048^2: adapters move the velocity {moved_a:.3e}; other strengths {moved_b:.3e}")
    assert moved_a > 1e-2 and moved_b > 1e-2
    model.close()


def test_config5_cfg_denoise_2048(ctx):
    """the w8g64 model with eight rank-64 slots at strengths
    uniform in [-1, 1.5] (512 live ranks on all 238 modules: 16-chunk tails
    on the w8 paired and unsplit kernels). Its CFG pair of forwards (the
    caption, then the all-zero negative of the same shape, as the denoise
    loop wires it) at a sigma of the shift-6 schedule is held to the fp32
    reference by the reference's w8 rule, max(0.035, 2 x the bf16 run)
    (ming-quant-test.cc:826-831); then the 2-step CFG loop is deterministic,
    finite and moved by guidance."""
    import torch
    import ming_dit_amd as m
    import torch_ref as tr
    from helpers import CFG5_RANKS, CFG5_SCALES
    bench = _bench()
    gen = torch.Generator(device="cuda").manual_seed(43)
    ref = {}
    model = bench.build_forward_model(ctx, m, torch, gen, bits=8, ranks=CFG5_RANKS, ref=ref)
    for i, s in enumerate(CFG5_SCALES):
        model.set_lora_scale(i, s)
    img, cap, pos = bench.layout_2048()
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    noise = torch.randn((img, 64), generator=gen, device="cuda").float().cpu().numpy()
    sigma = float(orc.schedule_sigmas(11, 6.0)[5])
    lat = torch.from_numpy(noise).cuda().to(torch.bfloat16).view(torch.int16)
    zero = torch.zeros_like(capt)
    c, s = orc.rope_table(*pos)
    tin = orc.time_proj(sigma, 1000.0, 256)
    model.set_caption_cache(False)
    for name, cp in (("positive", capt), ("zero negative", zero)):
        ctx.reset_engagement()
        out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        assert model.forward(lat, cp, 2560, img, cap, cap, *pos, sigma, out)
        torch.cuda.synchronize()
        eng = ctx.engagement()
        assert eng["gemm_q8"] == 270 and eng["lora_proj"] == 238
        a = from_dev(out)
        assert np.isfinite(f32(a)).all()
        outs = {mode: tr.Ref(mode, "cuda").forward(ref, lat, cp, img, cap, cap, c, s, sigma,
                                                   CFG5_SCALES, tin)
                for mode in ("f32", "bf16")}
        torch.cuda.synchronize()
        got = torch.from_numpy(f32(a)).cuda()
        rel = tr.rel_l2(got, outs["f32"])
        bf_floor = tr.rel_l2(outs["bf16"], outs["f32"])
        bar = max(0.035, 2 * bf_floor)
        print(f"configs[4] w8 {name} velocity vs fp32: {rel:.3e} (bf16 run {bf_floor:.3e}, "
              f"bar {bar:.3e}); vs the bf16 run {tr.rel_l2(got, outs['bf16']):.3e}", flush=True)
        assert rel <= bar
        del outs, got
    del ref
    model.set_caption_cache(True)
    x1, x2 = noise.copy(), noise.copy()
    ctx.reset_engagement()
    assert model.denoise(x1, capt, 2560, cap, cap, pos, img, 2, 6.0, 4.0)
    eng = ctx.engagement()
    # 4 forwards x (34 x 7 projections + 32 adaLN), less the context refiner's
    # 2 x 7 in the two step-2 forwards, whose captions the cache served
    assert eng["cap_cache_hits"] == 2
    assert eng["gemm_q8"] == 4 * 270 - 2 * 14 and eng["lora_proj"] == 4 * 238 - 2 * 14
    assert model.denoise(x2, capt, 2560, cap, cap, pos, img, 2, 6.0, 4.0)
    assert np.array_equal(x1, x2) and np.isfinite(x1).all()
    # guidance moves the latent: the unguided loop lands elsewhere
    x3 = noise.copy()
    assert model.denoise(x3, capt, 2560, cap, cap, pos, img, 2, 6.0, 1.0)
    moved = np.linalg.norm(x1 - x3) / np.linalg.norm(x3 - noise)
    print(f"2048^2 CFG: guided vs unguided latent update differs by {moved:.3e} (relative)")
    assert moved > 1e-2
    model.close()
