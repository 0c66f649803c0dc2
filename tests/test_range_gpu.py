"""Projection inputs beyond fp16's range, and weights whose scales fp16 cannot
hold.

The fast and general routes multiply fp16 activations that carry the bf16
values exactly while |x| < 2^16 (65280 is bf16's largest magnitude below it
and an fp16 value). A value of 2^16 or more would saturate to 65504, so every
writer of an fp16 copy reports one, and the next synchronization returns
MING_ERR_RANGE instead of results; the wide route computes such inputs in
bf16 end to end (bf16 activations, each weight a bf16 pair). The reference's
bf16 path has no such limit (ming-dit.cc:1721-1771), which is what the wide
route restores. A weight whose scales or biases are not exact in fp16 leaves
the fast route for the general kernel automatically, within the same bar.
"""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import (CFG2_RANKS, CFG2_SCALES, bf16, build_block, build_model, empty_bf16,
                     f32, from_dev, grid_positions, make_lora, make_weight, randn, sync,
                     to_dev)

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(autouse=True)
def auto_route(ctx):
    ctx.set_route("auto")
    yield
    ctx.set_route("auto")


def _qw(ctx, pack, bits, loras=()):
    qw = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)
    for slot, (A, B) in loras:
        qw.bind_lora(slot, A, B)
    return qw


def _lin(ctx, qw, xd, M, scales=None):
    """y on the context's stream, waited for device-wide (torch reads y on its
    own stream); the range word is left for ctx.synchronize() to report."""
    y = empty_bf16(M, qw.N)
    sync()
    ctx.lin(qw, xd, y, M, scales)
    sync()
    return y


def _refused(ctx):
    with pytest.raises(m.MingError) as e:
        ctx.synchronize()
    assert e.value.code == m.ERR_RANGE and "65536" in str(e.value)


@pytest.mark.parametrize("live", [False, True])
def test_largest_carried_value_is_not_a_fault(ctx, orc, live):
    """+-65280 (bf16's largest below 2^16) passes through both fp16 routes
    exactly: no fault, and the result within the bar. With a live adapter the
    fast route's fp16 copy of x is written by the x.A launch (no conversion
    launch), without one by the conversion kernel."""
    M, N, K = 300, 512, 640
    x = randn(1, (M, K))
    x[::7, ::5] = 65280.0
    x[3::11, 1::9] = -65280.0
    xb = bf16(x)
    pack, w = make_weight(2, N, K, 4)
    lo = [(1, make_lora(8, N, K, 32))] if live else []
    qw = _qw(ctx, pack, 4, lo)
    sc = [0.0, 0.5] if live else None
    ref = orc.proj(xb, w, [(A, B, 0.5) for _, (A, B) in lo])
    for route in ("auto", "general"):
        ctx.set_route(route)
        ctx.reset_engagement()
        ctx.set_profiling(True)
        ctx.profile_collect()
        y = _lin(ctx, qw, to_dev(xb), M, sc)
        ctx.synchronize()
        prof = ctx.profile_collect()
        ctx.set_profiling(False)
        assert ctx.engagement()["range_faults"] == 0
        assert orc.rel_l2(f32(from_dev(y)), ref) <= TOL
        if route == "auto":
            assert prof.get("cvt_f16", {}).get("launches", 0) == (0 if live else 1)
            assert prof.get("lora_xa", {}).get("launches", 0) == (1 if live else 0)


@pytest.mark.parametrize("big", [65536.0, -1.0e6, np.inf])
def test_beyond_fp16_is_refused_and_the_wide_route_computes_it(ctx, orc, big):
    M, N, K = 300, 512, 640
    print(f"case big={big}", flush=True)
    x = randn(3, (M, K))
    x[17, 33] = big
    x[250, 600] = big
    xb = bf16(x)
    pack, w = make_weight(4, N, K, 4)
    lo = [(0, make_lora(5, N, K, 16)), (3, make_lora(7, N, K, 64))]
    qw = _qw(ctx, pack, 4, lo)
    sc = [0.7, 0, 0, -0.4]
    for route in ("auto", "general"):
        ctx.set_route(route)
        ctx.reset_engagement()
        _lin(ctx, qw, to_dev(xb), M, sc)
        _refused(ctx)
        assert ctx.engagement()["range_faults"] == 1
        ctx.synchronize()                      # reported once, then cleared
    ctx.set_route("wide")
    ctx.reset_engagement()
    y = from_dev(_lin(ctx, qw, to_dev(xb), M, sc))
    ctx.synchronize()
    eng = ctx.engagement()
    assert eng["range_faults"] == 0 and eng["gemm_fast"] == 0 and eng["lora_proj"] == 1
    if np.isfinite(big):
        ref = orc.proj(xb, w, [(lo[0][1][0], lo[0][1][1], 0.7), (lo[1][1][0], lo[1][1][1], -0.4)])
        assert orc.rel_l2(f32(y), ref) <= TOL
    else:
        # the rows that hold an inf are not finite; every other row is the base
        bad = np.zeros(M, bool)
        bad[[17, 250]] = True
        assert np.all(np.isfinite(f32(y)[~bad])) and not np.all(np.isfinite(f32(y)[bad]))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K", [(300, 512, 640), (520, 1024, 1024)])
def test_wide_route_parity(ctx, orc, bits, M, N, K):
    """The wide route is the same function: within the bar of the fp32
    reference with the config-2 adapter set, at least as close to it as the
    fast route (its weights carry ~16 bits where the fast route's fp16 tiles
    carry 11), and within the bar of the fast route's output."""
    x = bf16(randn(11, (M, K)))
    pack, w = make_weight(12, N, K, bits)
    lo = [(s, make_lora(100 + 2 * s, N, K, r)) for s, r in enumerate(CFG2_RANKS)]
    qw = _qw(ctx, pack, bits, lo)
    ctx.set_route("wide")
    ctx.reset_engagement()
    yw = f32(from_dev(_lin(ctx, qw, to_dev(x), M, CFG2_SCALES)))
    ctx.synchronize()
    eng = ctx.engagement()
    assert eng["gemm_fast"] == 0 and eng["lora_proj"] == 1 and eng["lora_xa"] == 1
    ref = orc.proj(x, w, [(A, B, CFG2_SCALES[s]) for s, (A, B) in lo])
    rel = orc.rel_l2(yw, ref)
    ctx.set_route("auto")
    ya = f32(from_dev(_lin(ctx, qw, to_dev(x), M, CFG2_SCALES)))
    ctx.synchronize()
    rel_fast = orc.rel_l2(ya, ref)
    print(f"wide w{bits} {M}x{N}x{K}: rel-L2 {rel:.3e} (fast {rel_fast:.3e}), "
          f"vs fast {orc.rel_l2(yw, ya):.3e}")
    assert rel <= TOL and rel <= 1.02 * rel_fast and orc.rel_l2(yw, ya) <= TOL


def test_ffn_fault_in_the_fused_epilogue_and_wide_ffn(ctx, orc):
    """h = silu(g) * u beyond 2^16 (large w1/w3): the fp16 copy of h that w3's
    fused epilogue writes for w2 reports it; the wide route runs the FFN in
    bf16, w2 within the bar of the fp32 reference on its own h."""
    M, H, F = 300, 384, 640
    ws = []
    packs = []
    for i, (N, K, std) in enumerate(((F, H, 15.0), (F, H, 15.0), (H, F, 0.02))):
        pack, wd = make_weight(40 + i, N, K, 4, std=std)
        packs.append(wd)
        ws.append(_qw(ctx, pack, 4, [(0, make_lora(50 + 2 * i, N, K, 16))]))
    x = to_dev(bf16(randn(45, (M, H))))
    y = empty_bf16(M, H)
    h = empty_bf16(M, F)
    sc = [0.5]
    sync()
    ctx.ffn(ws[0], ws[1], ws[2], x, y, M, sc, h=h)
    _refused(ctx)
    ctx.set_route("wide")
    ctx.ffn(ws[0], ws[1], ws[2], x, y, M, sc, h=h)
    ctx.synchronize()
    sync()
    hh, yy = from_dev(h), from_dev(y)
    assert np.abs(f32(hh)).max() > 65536.0
    rows = np.arange(0, M, 13)
    A, B = make_lora(54, H, F, 16)
    ref = orc.proj(np.ascontiguousarray(hh[rows]), packs[2], [(A, B, 0.5)])
    assert orc.rel_l2(f32(yy[rows]), ref) <= TOL


def test_block_fault_in_the_norm_copy_and_wide_block(ctx, orc):
    """A pre-norm gain of 1e5 puts the RMSNorm output (which also writes the
    fp16 copy q, k and v read) past 2^16: refused on the auto route; the wide
    route runs the block, within the block bars of the oracle."""
    H, NH, F, ADA, rows = 256, 2, 512, 64, 130
    ob, gp, desc = build_block(ctx, 321, H, F, ADA, 4, False)
    big = bf16(np.full(H, 1.0e5, np.float32))
    ob["an1"] = big
    gp["an1"].copy_(to_dev(big))
    x = bf16(randn(46, (rows, H)))
    c, s = orc.rope_table(*grid_positions(rows))
    cd, sd = to_dev(np.ascontiguousarray(c)), to_dev(np.ascontiguousarray(s))
    scales = (1.0, 0, 0, -0.5)
    xd = to_dev(x)
    sync()
    ctx.block_forward(desc, m.BlockDims(H, NH, F, ADA, 1e-5), xd, rows, cd, sd, None, scales)
    _refused(ctx)
    ctx.set_route("wide")
    xd = to_dev(x)
    sync()
    ctx.block_forward(desc, m.BlockDims(H, NH, F, ADA, 1e-5), xd, rows, cd, sd, None, scales)
    ctx.synchronize()
    sync()
    got = from_dev(xd)
    ref = orc.block_forward(x, ob, NH, c, s, None, scales)
    upd = orc.rel_l2(f32(got) - f32(x), f32(ref) - f32(x))
    print(f"wide block with a 1e5 gain: output {orc.rel_l2(f32(got), f32(ref)):.3e}, "
          f"update {upd:.3e}")
    assert orc.rel_l2(f32(got), f32(ref)) <= 1e-2 and upd <= 2e-2


def test_dense_block_writes_no_fault(ctx, orc):
    """A block of dense projections multiplies bf16 activations: the fp16
    copies the block driver still writes are never read, so the same 1e5
    pre-norm gain raises no range fault on the auto route, and the block
    meets the oracle's block bars."""
    H, NH, F, ADA, rows = 256, 2, 512, 64, 130
    ob, gp, desc = build_block(ctx, 321, H, F, ADA, 16, False)
    big = bf16(np.full(H, 1.0e5, np.float32))
    ob["an1"] = big
    gp["an1"].copy_(to_dev(big))
    x = bf16(randn(46, (rows, H)))
    c, s = orc.rope_table(*grid_positions(rows))
    cd, sd = to_dev(np.ascontiguousarray(c)), to_dev(np.ascontiguousarray(s))
    scales = (1.0, 0, 0, -0.5)
    xd = to_dev(x)
    ctx.set_route("auto")
    ctx.reset_engagement()
    sync()
    ctx.block_forward(desc, m.BlockDims(H, NH, F, ADA, 1e-5), xd, rows, cd, sd, None, scales)
    ctx.synchronize()                      # raises MingError on a range fault
    sync()
    eng = ctx.engagement()
    assert eng["range_faults"] == 0 and eng["gemm_dense"] == 7
    got = from_dev(xd)
    ref = orc.block_forward(x, ob, NH, c, s, None, scales)
    upd = orc.rel_l2(f32(got) - f32(x), f32(ref) - f32(x))
    print(f"dense block with a 1e5 gain: output {orc.rel_l2(f32(got), f32(ref)):.3e}, "
          f"update {upd:.3e}")
    assert orc.rel_l2(f32(got), f32(ref)) <= 1e-2 and upd <= 2e-2
    # the same block quantized still refuses (the copies feed fp16 routes)
    obq, gpq, descq = build_block(ctx, 321, H, F, ADA, 4, False)
    gpq["an1"].copy_(to_dev(big))
    xd = to_dev(x)
    sync()
    ctx.block_forward(descq, m.BlockDims(H, NH, F, ADA, 1e-5), xd, rows, cd, sd, None, scales)
    _refused(ctx)


def test_model_forward_fault_and_wide_forward(ctx, orc):
    """The forward itself returns MING_ERR_RANGE; the caption-cache entry that
    forward filled never becomes valid; on the wide route the forward runs,
    within the forward bar of the oracle."""
    from test_model_gpu import CAP, QROWS, SCALES, inputs, run
    mo, model = build_model(ctx, 17)
    for i, v in enumerate(SCALES):
        model.set_lora_scale(i, v)
    gp = next(k for k in model._keep if isinstance(k, dict) and "ada" in k)
    blk = next(b for b in mo["blocks"])
    big = bf16(np.full(mo["hidden"], 1.0e5, np.float32))
    blk["an1"] = big
    gp["an1"].copy_(to_dev(big))
    lay, img, lat, cap, cs = inputs()
    ctx.reset_engagement()
    with pytest.raises(m.MingError) as e:
        run(model, lay, img, lat, cap, cs, 0.4)
    assert e.value.code == m.ERR_RANGE
    ctx.set_route("wide")
    got = run(model, lay, img, lat, cap, cs, 0.4)
    assert ctx.engagement()["cap_cache_hits"] == 0       # the faulted fill was dropped
    again = run(model, lay, img, lat, cap, cs, 0.4)
    assert ctx.engagement()["cap_cache_hits"] == 1 and np.array_equal(got, again)
    ref = orc.model_forward(mo, lat, cap, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                            lay["pos_w"], 0.4, SCALES)
    err = orc.rel_l2(f32(got), f32(ref))
    print(f"wide forward with a 1e5 gain: velocity rel-L2 {err:.3e}")
    assert err <= 2e-2
    model.close()


def test_scales_not_exact_in_fp16_take_the_general_route(ctx, orc):
    """A group of tiny spread has a scale and bias fp16 cannot hold (deep in
    its subnormals): the weight leaves the fast route by itself, and the
    projection stays within the bar."""
    M, N, K = 300, 512, 640
    wf = randn(60, (N, K), 0.02)
    wf[5, 64:128] = randn(61, (64,), 1e-6)
    wf[400, 0:64] = randn(62, (64,), 3e-7)
    import oracle as o
    codes, sc, bi = o.quantize(wf, 4)
    wd = o.dequant(codes, sc, bi, 4)
    qw = m.QWeight.quantized(ctx, codes, sc, bi, 4)
    assert not qw.fast
    A, B = make_lora(63, N, K, 32)
    qw.bind_lora(2, A, B)
    x = bf16(randn(64, (M, K)))
    ctx.reset_engagement()
    y = f32(from_dev(_lin(ctx, qw, to_dev(x), M, [0, 0, 0.9])))
    ctx.synchronize()
    eng = ctx.engagement()
    assert eng["gemm_q4"] == 1 and eng["gemm_fast"] == 0 and eng["lora_proj"] == 1
    assert orc.rel_l2(y, orc.proj(x, wd, [(A, B, 0.9)])) <= TOL
