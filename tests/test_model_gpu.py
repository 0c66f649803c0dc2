"""The model forward (MingDit::forward, ming-dit.cc:1490-2563) through
ming_model_forward against oracle.model_forward at reduced width: H=256,
2 heads, ffn 512, one context-refiner block, one noise-refiner block and two
layers, an 8x8 latent grid and a 24-row caption (8 query rows through
cap_embedder, 16 bypassing it).

The velocity is held to rel-L2 2e-2 against the oracle: it passes four
blocks (each within its own 1e-2 / 2e-2 bars) and the final layer.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import bf16, f32, randn, to_dev, from_dev, empty_bf16, sync, build_model

pytestmark = pytest.mark.gpu

GRID, CAP, QROWS, PD, CAPD, H = 8, 24, 8, 64, 128, 256
SCALES = (1.0, 0.0, 0.0, -0.5, 0.0, 0.0, 0.0, 0.0)


def inputs():
    lay = orc.build_layout(GRID, GRID, QROWS, CAP - QROWS)
    assert lay["img_tokens"] == GRID * GRID and lay["joint_len"] == GRID * GRID + CAP
    img = GRID * GRID
    lat = bf16(randn(61, (img, PD)))
    cs = max(CAPD, H)
    cap = np.zeros((CAP, cs), np.uint16)
    cap[:QROWS, :CAPD] = bf16(randn(63, (QROWS, CAPD)))
    cap[QROWS:, :H] = bf16(randn(65, (CAP - QROWS, H), 0.5))
    return lay, img, lat, cap, cs


def run(model, lay, img, lat, cap, cs, sigma):
    out = empty_bf16(img, PD)
    ld, cd = to_dev(lat), to_dev(cap)
    sync()
    model.forward(ld, cd, cs, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                  lay["pos_w"], sigma, out)
    return from_dev(out)


def test_model_forward_matches_oracle(ctx):
    mo, model = build_model(ctx, 7)
    for i, s in enumerate(SCALES):
        model.set_lora_scale(i, s)
    lay, img, lat, cap, cs = inputs()
    got = run(model, lay, img, lat, cap, cs, 0.6)
    ref = orc.model_forward(mo, lat, cap, img, CAP, QROWS, lay["pos_t"],
                            lay["pos_h"], lay["pos_w"], 0.6, SCALES)
    err = orc.rel_l2(f32(got), f32(ref))
    print(f"model forward: velocity rel-L2 {err:.3e}")
    assert err <= 2e-2
    model.close()


def test_model_strength_change_and_back_is_bit_identical(ctx):
    """Strengths are live between forwards, and a change undone gives the
    same bits (ming-dit-test.cc:1257-1264)."""
    mo, model = build_model(ctx, 8)
    lay, img, lat, cap, cs = inputs()
    for i, s in enumerate(SCALES):
        model.set_lora_scale(i, s)
    a = run(model, lay, img, lat, cap, cs, 0.3)
    model.set_lora_scale(0, 2.0)
    assert model.lora_scale(0) == 2.0
    b = run(model, lay, img, lat, cap, cs, 0.3)
    model.set_lora_scale(0, SCALES[0])
    c = run(model, lay, img, lat, cap, cs, 0.3)
    assert not np.array_equal(a, b)
    assert np.array_equal(a, c)
    model.close()


def test_model_rejects_bad_layout(ctx):
    import ming_dit_amd as m
    mo, model = build_model(ctx, 9, n_layers=1)
    lay, img, lat, cap, cs = inputs()
    out = empty_bf16(img, PD)
    ld, cd = to_dev(lat), to_dev(cap)
    bad = np.array(lay["pos_t"], np.int32)
    bad[0] = 5000                       # past axes_lens[0] = 4096
    with pytest.raises(m.MingError):
        model.forward(ld, cd, cs, img, CAP, QROWS, bad, lay["pos_h"],
                      lay["pos_w"], 0.5, out)
    with pytest.raises(m.MingError):     # more query rows than caption rows
        model.forward(ld, cd, cs, img, CAP, CAP + 1, lay["pos_t"], lay["pos_h"],
                      lay["pos_w"], 0.5, out)
    model.close()


def test_caption_cache_follows_direct_rebinding(ctx):
    """Binding or unbinding an adapter directly on a borrowed context-refiner
    weight (not through the model) is never answered from the caption cache:
    the next forward refines the caption again, with the binding in force,
    and gives the bits of an uncached forward."""
    from helpers import make_lora
    mo, model = build_model(ctx, 9)
    for i, s in enumerate(SCALES):
        model.set_lora_scale(i, s)
    lay, img, lat, cap, cs = inputs()
    ctx.reset_engagement()
    a = run(model, lay, img, lat, cap, cs, 0.6)
    assert np.array_equal(run(model, lay, img, lat, cap, cs, 0.6), a)
    assert ctx.engagement()["cap_cache_hits"] == 1
    w1 = model._keep[0]["w1"]              # the context refiner's w1, borrowed
    A, B = make_lora(901, w1.N, w1.K, 16)
    w1.bind_lora(0, A, B)                  # slot 0 is live (strength 1)
    rebound = run(model, lay, img, lat, cap, cs, 0.6)
    assert ctx.engagement()["cap_cache_hits"] == 1
    assert not np.array_equal(rebound, a)
    model.set_caption_cache(False)
    assert np.array_equal(run(model, lay, img, lat, cap, cs, 0.6), rebound)
    model.set_caption_cache(True)
    assert np.array_equal(run(model, lay, img, lat, cap, cs, 0.6), rebound)
    assert ctx.engagement()["cap_cache_hits"] == 1     # refilled, not hit
    assert np.array_equal(run(model, lay, img, lat, cap, cs, 0.6), rebound)
    assert ctx.engagement()["cap_cache_hits"] == 2     # now cached
    w1.unbind_lora(0)
    unbound = run(model, lay, img, lat, cap, cs, 0.6)
    assert ctx.engagement()["cap_cache_hits"] == 2
    model.set_caption_cache(False)
    assert np.array_equal(run(model, lay, img, lat, cap, cs, 0.6), unbound)
    model.close()
