"""MingDit::load from a transformer directory (ming_model_load), adapter
files bound at load (bind_loras_, ming-dit.cc:2918-3005, as
ming-dit-test.cc:1148-1386 tests it), and the lifecycle hooks (stop,
progress, caption cache; ming-dit.h:150-223), on a reduced-width model:
dim 384 (3 heads), ffn 1024, one refiner block of each kind, two layers.

Bars: a directory load is bit-identical to the same weights handed over in
memory (ming_model_create); against the oracle the velocity is held to
rel-L2 2e-2 as in the model test; adapters in every spelling give the same
bits as the in-memory binding with fold alpha / rank.
"""
import numpy as np
import pytest

import oracle as orc
import ming_dit_amd as m
from ckpt import (adapter_factors, config, make_checkpoint, module_list,
                  oracle_model, read_dir, write_adapter, write_st)
from helpers import f32, randn, bf16, to_dev, from_dev, empty_bf16, sync

pytestmark = pytest.mark.gpu

CFG = config()
DIM, FFN, PD = 384, 1024, 64
GRID, CAP, QROWS = 8, 24, 8
RANK, ALPHA = 8, 4.0
CAPACITY = 7 * (2 * 1 + 2)


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    root = tmp_path_factory.mktemp("load")
    dense = str(root / "dense")
    make_checkpoint(dense, seed=11, cfg=CFG)
    p4, p8 = str(root / "w4"), str(root / "w8")
    m.pack_write(dense, p4, 4)
    m.pack_write(dense, p8, 8)
    fac = adapter_factors(CFG, 21, RANK)
    ad = {}
    for sp in ("diffusers", "pipeline", "peft", "kohya"):
        ad[sp] = str(root / f"adapter_{sp}.safetensors")
        write_adapter(ad[sp], fac, sp, alpha=ALPHA)
    ad["foreign"] = str(root / "foreign.safetensors")
    write_st(ad["foreign"], [
        ("transformer_blocks.0.attn.to_q.lora_A.weight", "BF16", bf16(np.full((4, DIM), .01, np.float32))),
        ("transformer_blocks.0.attn.to_q.lora_B.weight", "BF16", bf16(np.full((DIM, 4), .01, np.float32)))])
    ad["wrong"] = str(root / "wrong.safetensors")
    write_st(ad["wrong"], [
        ("layers.0.attention.to_q.lora_A.weight", "BF16", bf16(np.full((4, DIM // 2), .01, np.float32))),
        ("layers.0.attention.to_q.lora_B.weight", "BF16", bf16(np.full((DIM // 2, 4), .01, np.float32))),
        ("layers.1.attention.to_q.lora_A.weight", "BF16", bf16(np.full((4, DIM), .01, np.float32))),
        ("layers.1.attention.to_q.lora_B.weight", "BF16", bf16(np.full((DIM, 4), .01, np.float32)))])
    return {"dense": dense, "w4": p4, "w8": p8, "ad": ad, "fac": fac}


def inputs(seed=61):
    lay = orc.build_layout(GRID, GRID, QROWS, CAP - QROWS)
    img = GRID * GRID
    lat = bf16(randn(seed, (img, PD)))
    cs = DIM
    cap = np.zeros((CAP, cs), np.uint16)
    cap[:QROWS, :128] = bf16(randn(seed + 2, (QROWS, 128)))
    cap[QROWS:, :DIM] = bf16(randn(seed + 4, (CAP - QROWS, DIM), 0.5))
    return lay, img, lat, cap, cs


def run(model, inp=None, sigma=0.6):
    lay, img, lat, cap, cs = inp or inputs()
    out = empty_bf16(img, PD)
    ld, cd = to_dev(lat), to_dev(cap)
    sync()
    ran = model.forward(ld, cd, cs, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                        lay["pos_w"], sigma, out)
    sync()
    return from_dev(out) if ran else None


def in_memory_model(ctx, tensors, loras=None):
    """The same weights through ming_model_create: packed matrices as
    QWeight.quantized, dense ones narrowed to bf16; `loras` {module: (A, B,
    fold)} bound on slot 0."""
    mo = oracle_model(CFG, tensors)
    keep = []

    def qw(w):
        if "codes" in w:
            return m.QWeight.quantized(ctx, w["codes"], w["scales"], w["biases"], w["bits"])
        return m.QWeight.dense(ctx, w["w"])

    def blk(ob, modulated):
        parts = {k: qw(ob[k]) for k in ("q", "k", "v", "o", "w1", "w3", "w2")}
        if modulated:
            parts["ada"] = qw(ob["ada"])
            parts["ada_b"] = to_dev(ob["ada_b"])
        for g in ("an1", "an2", "fn1", "fn2", "nq", "nk"):
            parts[g] = to_dev(ob[g])
        keep.append(parts)
        return parts, m.block_desc(**parts)

    cb, mb, parts_of = [], [], {}
    for i, ob in enumerate(mo["ctx_blocks"]):
        p, d = blk(ob, False)
        parts_of[("ctx_blocks", i)] = p
        cb.append(d)
    for i, ob in enumerate(mo["blocks"]):
        p, d = blk(ob, True)
        parts_of[("blocks", i)] = p
        mb.append(d)
    if loras:
        for mod, N, K, lst, bi, key in module_list(CFG):
            if mod in loras:
                A, B, fold = loras[mod]
                parts_of[(lst, bi)][key].bind_lora(0, A, B, fold)
    dev = {}
    for name in ("time_1", "time_2", "x_in", "cap_in", "final_ada", "final_lin"):
        dev[name] = qw(mo[name])
    for name in ("time_1b", "time_2b", "x_in_b", "cap_in_b", "final_ada_b",
                 "final_lin_b", "cap_norm"):
        dev[name] = to_dev(mo[name])
    d = m.ModelDesc()
    d.hidden, d.n_heads, d.ffn, d.n_layers, d.n_refiner = DIM, 3, FFN, 2, 1
    d.adaln_dim, d.time_freq, d.time_mid = 256, 256, 1024
    d.patch_dim, d.cap_dim = PD, 128
    d.eps, d.rope_theta, d.t_scale = 1e-5, 256.0, 1000.0
    d.axes[:] = [32, 48, 48]
    d.axes_lens[:] = list(CFG["axes_lens"])
    for name, obj in dev.items():
        setattr(d, name, m._h(obj))
    return m.Model(ctx, d, cb, mb, keep=keep + [dev]), mo


def bf16_factors(fac, fold):
    return {k: (bf16(A), bf16(B), fold) for k, (A, B) in fac.items()}


def test_dense_directory_equals_in_memory_weights(ctx, files):
    model = m.Model.load(ctx, files["dense"])
    ctx.reset_engagement()
    got = run(model)
    eng = ctx.engagement()
    assert eng["gemm_dense"] > 0 and eng["gemm_q4"] == 0 and eng["gemm_q8"] == 0
    ref_model, mo = in_memory_model(ctx, read_dir(files["dense"]))
    ref = run(ref_model)
    assert np.array_equal(got, ref)
    model.close()
    ref_model.close()


@pytest.mark.parametrize("bits", [4, 8])
def test_pack_directory_equals_in_memory_and_oracle(ctx, files, bits):
    model = m.Model.load(ctx, files[f"w{bits}"])
    ctx.reset_engagement()
    got = run(model)
    eng = ctx.engagement()
    # 7 projections + adaLN per modulated block, 7 per context block
    assert eng[f"gemm_q{bits}"] == 3 * 8 + 7
    tensors = read_dir(files[f"w{bits}"])
    ref_model, mo = in_memory_model(ctx, tensors)
    assert np.array_equal(got, run(ref_model))
    lay, img, lat, cap, cs = inputs()
    want = orc.model_forward(mo, lat, cap, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                             lay["pos_w"], 0.6)
    err = orc.rel_l2(f32(got), f32(want))
    print(f"w{bits} pack load: velocity rel-L2 vs oracle {err:.3e}")
    assert err <= 2e-2
    model.close()
    ref_model.close()


def test_every_spelling_binds_every_module_with_alpha_folded(ctx, files):
    msgs = []
    m.set_log_sink(lambda lvl, s: msgs.append((lvl, s)))
    try:
        base_model = m.Model.load(ctx, files["w4"])
        base = run(base_model)
        base_model.close()
        first = None
        for sp in ("diffusers", "pipeline", "peft", "kohya"):
            model = m.Model.load(ctx, files["w4"], [(files["ad"][sp], 1.0)])
            assert model.lora_modules(0) == CAPACITY and model.lora_skipped(0) == 0, sp
            assert f"bound {CAPACITY} of {CAPACITY} modules" in model.lora_report(0)
            ctx.reset_engagement()
            got = run(model)
            assert ctx.engagement()["lora_proj"] == CAPACITY, sp  # cold cache: every block ran
            if first is None:
                first = got
            else:
                assert np.array_equal(got, first), sp
            model.close()
        assert sum(lvl == m.LOG_INFO for lvl, _ in msgs) == 4
    finally:
        m.set_log_sink(None)
    # the same factors bound in memory with fold alpha / rank give the same bits
    ref_model, mo = in_memory_model(ctx, read_dir(files["w4"]),
                                    bf16_factors(files["fac"], ALPHA / RANK))
    ref_model.set_lora_scale(0, 1.0)
    assert np.array_equal(first, run(ref_model))
    ref_model.close()
    # and the adapter moves the output far past the fused-reference floor
    for mod, N, K, lst, bi, key in module_list(CFG):
        A, B = files["fac"][mod]
        mo[lst][bi]["loras"][key][0] = (bf16(A), bf16(B), ALPHA / RANK)
    lay, img, lat, cap, cs = inputs()
    want = orc.model_forward(mo, lat, cap, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                             lay["pos_w"], 0.6, (1.0,) + (0.0,) * 7)
    vs = orc.rel_l2(f32(first), f32(want))
    moved = orc.rel_l2(f32(base), f32(first))
    print(f"adapter: vs oracle {vs:.3e}, moved {moved:.3e}")
    assert vs <= 2e-2 and moved > 0.1 and moved > 10 * vs


def test_strength_zero_is_the_base_exactly_and_positional_slots(ctx, files):
    base_model = m.Model.load(ctx, files["w4"])
    base = run(base_model)
    base_model.close()
    model = m.Model.load(ctx, files["w4"], [(files["ad"]["kohya"], 1.0)])
    first = run(model)
    model.set_lora_scale(0, 0.0)
    ctx.reset_engagement()
    z = run(model)
    assert np.array_equal(z, base) and ctx.engagement()["lora_proj"] == 0
    model.set_lora_scale(0, 1.0)
    assert np.array_equal(run(model), first)
    model.close()
    # `lora2` alone: slot 0 stays empty and slot 1 carries the adapter
    m2 = m.Model.load(ctx, files["w4"], [(None, 1.0), (files["ad"]["diffusers"], 1.0)])
    assert m2.lora_modules(0) == 0 and m2.lora_modules(1) == CAPACITY
    assert np.array_equal(run(m2), first)
    m2.set_lora_scale(0, 0.7)       # an empty slot: no effect
    assert np.array_equal(run(m2), first)
    m2.set_lora_scale(1, 0.0)
    assert np.array_equal(run(m2), base)
    m2.close()
    # `lora8` alone
    m8 = m.Model.load(ctx, files["w4"], [(None, 1.0)] * 7 + [(files["ad"]["peft"], 1.0)])
    assert all(m8.lora_modules(i) == 0 for i in range(7)) and m8.lora_modules(7) == CAPACITY
    assert np.array_equal(run(m8), first)
    m8.close()
    # the same adapter in two slots at 0.5 each is the adapter at 1, up to
    # rounding: the two deltas are summed in another order, and four bf16
    # blocks carry that to the velocity at the model's own floor (~7e-3 here
    # against the oracle), so the model bar applies; the adapter itself moves
    # the output 30x further
    mh = m.Model.load(ctx, files["w4"], [(files["ad"]["diffusers"], 0.5),
                                        (files["ad"]["kohya"], 0.5)])
    assert mh.lora_modules(0) == CAPACITY and mh.lora_modules(1) == CAPACITY
    two = run(mh)
    err = orc.rel_l2(f32(two), f32(first))
    moved = orc.rel_l2(f32(base), f32(first))
    print(f"two slots at 0.5 vs one at 1: rel-L2 {err:.3e} (the adapter moves {moved:.3e})")
    assert err <= 2e-2 and moved > 10 * err
    mh.close()


def test_foreign_and_wrong_shape_adapters_are_refused_and_said(ctx, files):
    base_model = m.Model.load(ctx, files["w4"])
    base = run(base_model)
    base_model.close()
    msgs = []
    m.set_log_sink(lambda lvl, s: msgs.append((lvl, s)))
    try:
        for k in ("foreign", "wrong"):
            msgs.clear()
            model = m.Model.load(ctx, files["w4"], [(files["ad"][k], 1.0)])
            rep = model.lora_report(0)
            assert model.lora_modules(0) == 0
            assert model.lora_skipped(0) == (0 if k == "foreign" else 1)
            if k == "foreign":
                assert "matched zero modules" in rep
            else:
                assert "left unbound" in rep and "other shapes (1 fit)" in rep
            assert any(lvl == m.LOG_WARN and s == rep for lvl, s in msgs)
            ctx.reset_engagement()
            assert np.array_equal(run(model), base)
            assert ctx.engagement()["lora_proj"] == 0
            model.close()
        model = m.Model.load(ctx, files["w4"], [(files["ad"]["foreign"] + ".missing", 1.0)])
        assert model.lora_modules(0) == 0 and "could not be read" in model.lora_report(0)
        model.close()
    finally:
        m.set_log_sink(None)


def test_stop_and_block_progress(ctx, files):
    model = m.Model.load(ctx, files["w4"])
    base = run(model)
    seen = []
    model.set_block_progress(lambda d, t: seen.append((d, t)))
    model.set_caption_cache(False)
    assert np.array_equal(run(model), base)
    assert seen == [(i, 4) for i in range(4)]
    seen.clear()
    calls = []

    def stop():
        calls.append(1)
        return len(calls) > 2          # stop before the third block

    model.set_stream_stop(stop)
    assert run(model) is None
    assert m.lib().ming_last_error() == b""
    assert seen == [(i, 4) for i in range(len(seen))] and len(seen) <= 2
    model.set_stream_stop(None)
    model.set_block_progress(None)
    assert np.array_equal(run(model), base)  # a stopped forward leaves nothing behind
    model.close()


def test_caption_cache(ctx, files):
    model = m.Model.load(ctx, files["w4"], [(files["ad"]["diffusers"], 1.0)])
    inp = inputs()
    ctx.reset_engagement()
    a = run(model, inp)
    assert ctx.engagement()["cap_cache_hits"] == 0
    b = run(model, inp)
    assert ctx.engagement()["cap_cache_hits"] == 1 and np.array_equal(a, b)
    # another caption (same image): a miss, then the first is still cached
    lay, img, lat, cap, cs = inp
    cap2 = cap.copy()
    cap2[QROWS + 1, 5] ^= 1
    run(model, (lay, img, lat, cap2, cs))
    assert ctx.engagement()["cap_cache_hits"] == 1
    assert np.array_equal(run(model, inp), a)
    assert ctx.engagement()["cap_cache_hits"] == 2
    # a strength change on a slot bound in the context refiner drops it
    model.set_lora_scale(0, 0.5)
    half = run(model, inp)
    assert ctx.engagement()["cap_cache_hits"] == 2
    model.set_caption_cache(False)
    assert np.array_equal(run(model, inp), half)
    model.set_lora_scale(0, 1.0)
    assert np.array_equal(run(model, inp), a)
    assert ctx.engagement()["cap_cache_hits"] == 2
    model.close()


def test_load_refuses_what_it_does_not_run(ctx, tmp_path):
    d = str(tmp_path / "learned")
    make_checkpoint(d, seed=12, cfg=config(alignment_padding_mode="learned"), shards=1)
    with pytest.raises(m.MingError, match="learned caption padding"):
        m.Model.load(ctx, d)
    d = str(tmp_path / "short")
    make_checkpoint(d, seed=12, cfg=CFG, shards=1, drop=("layers.1.ffn_norm2.weight",))
    with pytest.raises(m.MingError, match="layers.1.ffn_norm2.weight' is absent from the checkpoint"):
        m.Model.load(ctx, d)


def reference_loop(ctx, model, lat0, cap, lay, steps, shift, g, trunc=1.0,
                   stop_after=None):
    """The generator's loop (ming-generator.cc:505-577) restated in numpy
    f32 over the same model's forwards: bf16 latent per step (NaN -> 0x7fc0),
    v = pos (+ g (pos - neg) while (1 - sigma) <= trunc, negative = the
    caption times zero), latent += (sigma[i+1] - sigma[i]) * -v."""
    lay_, img, _, cap_h, cs = lay
    sig = np.asarray(orc.schedule_sigmas(steps, shift), np.float32)
    x = lat0.copy()
    zero = np.zeros_like(cap_h)
    for i in range(steps if stop_after is None else stop_after):
        inp = (lay_, img, orc.f32_to_bf16(x), cap_h, cs)
        v = f32(run(model, inp, float(sig[i])))
        if g > 1.0 and (1.0 - float(sig[i])) <= trunc:
            vn = f32(run(model, (lay_, img, orc.f32_to_bf16(x), zero, cs), float(sig[i])))
            v = (v + np.float32(g) * (v - vn)).astype(np.float32)
        dt = np.float32(sig[i + 1] - sig[i])
        x = (x + dt * -v).astype(np.float32)
    return x


@pytest.mark.parametrize("g,trunc", [(1.0, 1.0), (4.0, 1.0), (3.0, 0.2)])
def test_denoise_loop_equals_its_restatement(ctx, files, g, trunc):
    model = m.Model.load(ctx, files["w4"], [(files["ad"]["diffusers"], 0.7)])
    lay, img, lat, cap, cs = inputs()
    lat0 = randn(71, (img, PD))
    steps = 3
    want = reference_loop(ctx, model, lat0, None, (lay, img, None, cap, cs), steps, 6.0, g,
                          trunc)
    x = lat0.copy()
    cd = to_dev(cap)
    model.set_caption_cache(False)     # cold: the restatement's forwards filled it
    model.set_caption_cache(True)
    ctx.reset_engagement()
    assert model.denoise(x, cd, cs, CAP, QROWS, (lay["pos_t"], lay["pos_h"], lay["pos_w"]),
                         img, steps, 6.0, g, trunc)
    assert np.array_equal(x, want)
    # the caption cache serves the context refiner after the first step, for
    # the positive and (while guided) the zero negative
    sig = orc.schedule_sigmas(steps, 6.0)
    guided = [g > 1.0 and (1.0 - float(s)) <= trunc for s in sig[:steps]]
    assert ctx.engagement()["cap_cache_hits"] == (steps - 1) + max(sum(guided) - 1, 0)
    model.close()


def test_denoise_stops_and_clamps(ctx, files):
    model = m.Model.load(ctx, files["w4"])
    lay, img, lat, cap, cs = inputs()
    lat0 = randn(73, (img, PD))
    pos = (lay["pos_t"], lay["pos_h"], lay["pos_w"])
    cd = to_dev(cap)
    seen = []
    x = lat0.copy()
    assert not model.denoise(x, cd, cs, CAP, QROWS, pos, img, 4, 6.0, 4.0,
                             progress=lambda i, n: seen.append((i, n)) or i < 2)
    assert seen == [(1, 4), (2, 4)]
    want = reference_loop(ctx, model, lat0, None, (lay, img, None, cap, cs), 4, 6.0, 4.0,
                          stop_after=2)
    assert np.array_equal(x, want)
    # the norm clamp: |guided| <= cfg_normalization x |positive| on the one step
    sig = orc.schedule_sigmas(1, 6.0)
    x1, x2 = lat0.copy(), lat0.copy()
    assert model.denoise(x1, cd, cs, CAP, QROWS, pos, img, 1, 6.0, 4.0)
    assert model.denoise(x2, cd, cs, CAP, QROWS, pos, img, 1, 6.0, 4.0, cfg_normalization=1.0)
    v_free = (x1 - lat0) / np.float32(sig[0])      # the guided velocity
    v_clamp = (x2 - lat0) / np.float32(sig[0])
    vp = f32(run(model, (lay, img, orc.f32_to_bf16(lat0), cap, cs), float(sig[0])))
    assert np.linalg.norm(v_free) > 1.05 * np.linalg.norm(vp)
    assert abs(np.linalg.norm(v_clamp) / np.linalg.norm(vp) - 1.0) < 1e-3
    model.close()
