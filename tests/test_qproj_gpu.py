"""GPU parity of the projection path (ming_lin) against the CPU oracle.

Bar (north_star): rel-L2 <= 2e-3 against the fp32 dequant+GEMM+LoRA
reference, and bit-identity with the unadapted run when every strength is
0. Engagement counters are asserted before accuracy (ming-dit.h:55-103).
"""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import (CFG2_RANKS, CFG2_SCALES, CFG5_RANKS, CFG5_SCALES, bf16,
                     empty_bf16, from_dev, make_lora, make_weight, randn, sync,
                     to_dev)

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(params=["auto", "general"], autouse=True)
def route(request, ctx):
    """Every projection test runs on both kernel routes."""
    ctx.set_route(request.param)
    ctx._route_param = request.param
    yield request.param
    ctx.set_route("auto")


def _qw(ctx, pack, bits):
    if bits == 16:
        return m.QWeight.dense(ctx, pack["w"])
    return m.QWeight.quantized(ctx, pack["codes"], pack["scales"],
                               pack["biases"], bits)


def _run(ctx, qw, x_dev, M, scales=None):
    y = empty_bf16(M, qw.N)
    sync()
    ctx.lin(qw, x_dev, y, M, scales)
    sync()
    return from_dev(y)


def route_is_auto(ctx):
    return getattr(ctx, "_route_param", None) != "general"


def _rel(orc, y_bf16, ref):
    return orc.rel_l2(orc.bf16_to_f32(y_bf16), ref)


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("M,N,K", [(300, 512, 640), (1, 264, 64),
                                   (257, 256, 3840), (64, 1024, 192)])
def test_base_projection_parity(ctx, orc, bits, M, N, K):
    print(f"case bits={bits} M={M} N={N} K={K}", flush=True)
    x = bf16(randn(1000 + M, (M, K)))
    pack, w = make_weight(2000 + N, N, K, bits)
    qw = _qw(ctx, pack, bits)
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M)
    eng = ctx.engagement()
    key = {4: "gemm_q4", 8: "gemm_q8", 16: "gemm_dense"}[bits]
    assert eng[key] == 1 and eng["lora_proj"] == 0 and eng["lora_xa"] == 0
    # at M <= 8 with no live adapter the auto route runs the GEMV
    want_gemv = route_is_auto(ctx) and M <= 8
    want_fast = bits != 16 and route_is_auto(ctx) and not want_gemv
    assert qw.fast == (bits != 16)
    assert eng["gemm_fast"] == (1 if want_fast else 0)
    assert eng["gemv"] == (1 if want_gemv else 0)
    ref = orc.proj(x, w)
    assert _rel(orc, y, ref) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K", [(320, 768, 1024), (520, 8192, 512)])
def test_lora_eight_slots_parity(ctx, orc, bits, M, N, K):
    """BASELINE config 2's adapter set on one projection (an 8-chunk LoRA
    tail): on a few tiles (6: the fast route splits K) and on a grid of 96
    tiles with a ragged last tile-row (the unsplit fast kernel)."""
    print(f"case eight slots bits={bits} M={M} N={N} K={K}", flush=True)
    x = bf16(randn(11, (M, K)))
    pack, w = make_weight(12, N, K, bits)
    qw = _qw(ctx, pack, bits)
    loras = []
    for s, r in enumerate(CFG2_RANKS):
        A, B = make_lora(100 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        loras.append((A, B, CFG2_SCALES[s]))
    assert [qw.lora_rank(s) for s in range(8)] == list(CFG2_RANKS)
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M, CFG2_SCALES)
    eng = ctx.engagement()
    assert eng["lora_proj"] == 1 and eng["lora_xa"] == 1
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    assert eng["gemm_fast"] == (1 if route_is_auto(ctx) else 0)
    assert eng["gemm_split"] == (1 if route_is_auto(ctx) and tiles < 64 else 0)
    ref = orc.proj(x, w, loras)
    base = orc.proj(x, w)
    rel = _rel(orc, y, ref)
    assert rel <= TOL
    # the adapter MOVED the output far past the bar (not a vacuous match)
    assert orc.rel_l2(ref, base) > 10 * TOL


@pytest.mark.parametrize("bits,K", [(4, 64), (4, 128), (4, 192), (8, 64)])
def test_short_k_parity(ctx, orc, bits, K):
    """One, two and three 64-wide K stages (the ring's prologue and its
    remainder stages with no full trip) on a 64-tile grid, so the unsplit
    fast kernel runs, followed by the 8-chunk LoRA tail of config 2's set."""
    M, N = 2048, 2048
    print(f"case short K bits={bits} M={M} N={N} K={K}", flush=True)
    x = bf16(randn(31 + K, (M, K)))
    pack, w = make_weight(32 + K, N, K, bits)
    qw = _qw(ctx, pack, bits)
    loras = []
    for s, r in enumerate(CFG2_RANKS):
        A, B = make_lora(300 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        loras.append((A, B, CFG2_SCALES[s]))
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M, CFG2_SCALES)
    eng = ctx.engagement()
    assert eng["lora_proj"] == 1 and eng["gemm_split"] == 0
    assert eng["gemm_fast"] == (1 if route_is_auto(ctx) else 0)
    ref = orc.proj(x, w, loras)
    assert _rel(orc, y, ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w)) > 10 * TOL


ODD_RANKS = (3, 12, 20, 5, 36, 1, 7, 9)
ODD_SCALES = (0.9, -0.6, 0.4, 1.3, 0.25, -1.1, 0.0, 0.7)


@pytest.mark.parametrize("M,N,K", [(2085, 2048, 256), (300, 768, 1024)])
def test_ranks_off_the_group_grid_parity(ctx, orc, M, N, K):
    """Ranks that are no multiple of the 8-rank packing group, so zero rows
    pad groups in the middle of the stack and a slot's groups straddle the
    tails' 32-rank chunks: on an unsplit grid (72 tiles) and a split one."""
    print(f"case odd ranks M={M} N={N} K={K}", flush=True)
    x = bf16(randn(41 + M, (M, K)))
    pack, w = make_weight(42, N, K, 4)
    qw = _qw(ctx, pack, 4)
    loras = []
    for s, r in enumerate(ODD_RANKS):
        A, B = make_lora(300 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        loras.append((A, B, ODD_SCALES[s]))
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M, ODD_SCALES)
    eng = ctx.engagement()
    assert eng["lora_proj"] == 1 and eng["lora_xa"] == 1
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    assert eng["gemm_split"] == (1 if route_is_auto(ctx) and tiles < 64 else 0)
    ref = orc.proj(x, w, loras)
    assert _rel(orc, y, ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w)) > 10 * TOL
    qw.close()


def test_zero_strength_is_bit_identical(ctx, orc):
    """All eight strengths 0 == the unadapted projection, memcmp
    (ming-dit-test.cc:1249-1273)."""
    M, N, K = 300, 512, 640
    x = to_dev(bf16(randn(21, (M, K))))
    pack, _ = make_weight(22, N, K, 4)
    qw = _qw(ctx, pack, 4)
    plain = _qw(ctx, pack, 4)
    for s, r in enumerate(CFG2_RANKS):
        A, B = make_lora(200 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
    ctx.reset_engagement()
    y0 = _run(ctx, qw, x, M, [0.0] * 8)
    assert ctx.engagement()["lora_proj"] == 0
    assert np.array_equal(y0, _run(ctx, plain, x, M))
    assert np.array_equal(y0, _run(ctx, qw, x, M, None))


def test_live_strength_change_and_back(ctx, orc):
    """Strengths change between calls without rebinding, and going back
    reproduces the first bits (ming-dit-test.cc:1257-1264)."""
    M, N, K = 256, 512, 512
    x = to_dev(bf16(randn(31, (M, K))))
    pack, w = make_weight(32, N, K, 8)
    qw = _qw(ctx, pack, 8)
    A, B = make_lora(33, N, K, 16)
    qw.bind_lora(0, A, B)
    y1 = _run(ctx, qw, x, M, [0.8])
    y2 = _run(ctx, qw, x, M, [-0.5])
    y3 = _run(ctx, qw, x, M, [0.8])
    assert np.array_equal(y1, y3)
    assert not np.array_equal(y1, y2)
    xh = from_dev(x)
    assert _rel(orc, y2, orc.proj(xh, w, [(A, B, -0.5)])) <= TOL


def test_slots_are_positional(ctx, orc):
    """An adapter alone in slot 2 or slot 8 computes the bits it computes
    alone in slot 1 (ming-dit-test.cc:1294-1339)."""
    M, N, K = 200, 256, 384
    x = to_dev(bf16(randn(41, (M, K))))
    pack, _ = make_weight(42, N, K, 4)
    A, B = make_lora(43, N, K, 32)
    outs = []
    for slot in (0, 1, 7):
        qw = _qw(ctx, pack, 4)
        qw.bind_lora(slot, A, B)
        sc = [0.0] * 8
        sc[slot] = 0.7
        outs.append(_run(ctx, qw, x, M, sc))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_two_halves_make_one(ctx, orc):
    M, N, K = 128, 256, 256
    x = to_dev(bf16(randn(51, (M, K))))
    pack, _ = make_weight(52, N, K, 8)
    A, B = make_lora(53, N, K, 16)
    one = _qw(ctx, pack, 8)
    one.bind_lora(0, A, B)
    two = _qw(ctx, pack, 8)
    two.bind_lora(0, A, B)
    two.bind_lora(1, A, B)
    y1 = _run(ctx, one, x, M, [1.0])
    y2 = _run(ctx, two, x, M, [0.5, 0.5])
    assert orc.rel_l2(orc.bf16_to_f32(y2), orc.bf16_to_f32(y1)) < 1e-3


def test_fold_scales_the_delta(ctx, orc):
    M, N, K = 96, 256, 256
    xh = bf16(randn(61, (M, K)))
    pack, w = make_weight(62, N, K, 4)
    A, B = make_lora(63, N, K, 8)
    qw = _qw(ctx, pack, 4)
    qw.bind_lora(3, A, B, fold=2.0)   # alpha 16 / rank 8
    y = _run(ctx, qw, to_dev(xh), M, [0, 0, 0, 0.5])
    assert _rel(orc, y, orc.proj(xh, w, [(A, B, 1.0)])) <= TOL


def test_fused_qkv_equals_separate(ctx, orc):
    """q|k|v fused along N, each with its own adapters, gives the bits of
    three separate projections."""
    M, H, K = 300, 512, 512
    x = to_dev(bf16(randn(71, (M, K))))
    parts, sep = [], []
    for i in range(3):
        pack, _ = make_weight(72 + i, H, K, 4)
        p = _qw(ctx, pack, 4)
        A, B = make_lora(80 + 2 * i, H, K, 16 * (i + 1))
        p.bind_lora(i, A, B)
        parts.append(p)
    fused = m.QWeight.concat(ctx, parts)
    assert fused.N == 3 * H and fused.n_segments == 3
    sc = [0.9, -0.4, 0.6]
    ctx.reset_engagement()
    yf = _run(ctx, fused, x, M, sc)
    eng = ctx.engagement()
    assert eng["lora_xa"] == 1 and eng["lora_proj"] == 3
    for i, p in enumerate(parts):
        yi = _run(ctx, p, x, M, sc)
        assert np.array_equal(yf[:, i * H:(i + 1) * H], yi)


def test_strided_rows_in_and_out(ctx, orc):
    """Element strides on x and y (the reference's element offsets)."""
    M, N, K = 130, 256, 256
    xh = bf16(randn(91, (M, 2 * K)))
    pack, w = make_weight(92, N, K, 8)
    qw = _qw(ctx, pack, 8)
    xd = to_dev(xh)
    y = empty_bf16(M, 3 * N)
    y.zero_()
    sync()
    ctx.lin(qw, xd[:, K:], y[:, N:], M, None, ldx=2 * K, ldy=3 * N)
    sync()
    yh = from_dev(y)
    ref = orc.proj(np.ascontiguousarray(xh[:, K:]), w)
    assert _rel(orc, np.ascontiguousarray(yh[:, N:2 * N]), ref) <= TOL
    assert np.all(yh[:, :N] == 0) and np.all(yh[:, 2 * N:] == 0)


def test_bad_shapes_are_refused(ctx):
    pack, _ = make_weight(95, 64, 128, 4)
    qw = _qw(ctx, pack, 4)
    y = empty_bf16(8, 64)
    x = empty_bf16(8, 128)
    with pytest.raises(m.MingError):
        ctx.lin(qw, x, y, 8, None, ldx=100)      # ldx < K
    with pytest.raises(m.MingError):
        qw.bind_lora(8, np.zeros((4, 128), np.uint16), np.zeros((64, 4), np.uint16))
    with pytest.raises(m.MingError):      # bits 5 is not a pack
        m.QWeight.quantized(ctx, pack["codes"], pack["scales"],
                            pack["biases"], 5)
    with pytest.raises(m.MingError):      # K % 64 != 0
        m.QWeight.dense(ctx, np.zeros((64, 96), np.uint16))


def test_config1_full_size(ctx, orc):
    """to_q w8g64, X [4096, 3840], one r16 slot at 0.8,
    then 0 (memcmp with the unadapted run). The fp32 reference runs on a
    row sample spread over every M tile."""
    M, N, K = 4096, 3840, 3840
    x = bf16(randn(1001, (M, K)))
    w = randn(1002, (N, K), 0.02)
    codes, sc, bi = orc.quantize(w, 8)
    wd = orc.dequant(codes, sc, bi, 8)
    A = bf16(randn(1003, (16, K), 1.0 / np.sqrt(K)))
    B = bf16(randn(1004, (N, 16), 0.01))
    qw = m.QWeight.quantized(ctx, codes, sc, bi, 8)
    plain = m.QWeight.quantized(ctx, codes, sc, bi, 8)
    qw.bind_lora(0, A, B)
    xd = to_dev(x)
    y = _run(ctx, qw, xd, M, [0.8])
    rows = np.arange(0, M, 61)
    ref = orc.proj(np.ascontiguousarray(x[rows]), wd, [(A, B, 0.8)])
    assert _rel(orc, np.ascontiguousarray(y[rows]), ref) <= TOL
    y0 = _run(ctx, qw, xd, M, [0.0])
    assert np.array_equal(y0, _run(ctx, plain, xd, M))


@pytest.mark.parametrize("bits", [4, 8])
def test_routes_agree(ctx, orc, bits, route):
    """The fast and the general route compute the same function: both within
    the bar, and within a fraction of it of each other."""
    if route != "auto":
        pytest.skip("compares the routes once")
    M, N, K = 515, 768, 2048
    x = to_dev(bf16(randn(101, (M, K))))
    pack, w = make_weight(102, N, K, bits)
    qw = _qw(ctx, pack, bits)
    for s, r in enumerate((16, 64)):
        A, B = make_lora(110 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
    sc = [0.7, -0.4]
    ctx.set_route("auto")
    yf = _run(ctx, qw, x, M, sc)
    ctx.set_route("general")
    yg = _run(ctx, qw, x, M, sc)
    ctx.set_route("auto")
    assert orc.rel_l2(orc.bf16_to_f32(yf), orc.bf16_to_f32(yg)) < 5e-4


def _ffn_weights(ctx, seed, H, F, bits=4, slots=CFG2_RANKS):
    ws = []
    for i, (N, K) in enumerate(((F, H), (F, H), (H, F))):
        pack, _ = make_weight(seed + i, N, K, bits)
        qw = _qw(ctx, pack, bits)
        for s, r in enumerate(slots):
            A, B = make_lora(seed + 10 * i + 2 * s + 100, N, K, r)
            qw.bind_lora(s, A, B)
        ws.append(qw)
    return ws


@pytest.mark.parametrize("inplace", [False, True])
def test_lin_swiglu_equals_lin_then_swiglu(ctx, orc, inplace):
    """The SwiGLU fused into the projection epilogue gives the bits of
    ming_lin followed by ming_swiglu (gpu_ff, ming-dit.cc:2151-2158)."""
    M, H, F = 300, 384, 640
    w1, w3, _ = _ffn_weights(ctx, 610, H, F)
    x = to_dev(bf16(randn(611, (M, H))))
    g = to_dev(bf16(randn(612, (M, F))))
    u = _run(ctx, w3, x, M, CFG2_SCALES)
    ref = empty_bf16(M, F)
    ud = to_dev(u)
    sync()
    ctx.swiglu(g, ud, ref, M, F)
    sync()
    out = g.clone() if inplace else empty_bf16(M, F)
    sync()
    ctx.lin_swiglu(w3, x, out if inplace else g, out, M, CFG2_SCALES)
    sync()
    assert np.array_equal(from_dev(out), from_dev(ref))


def _ffn_four_calls(ctx, w1, w3, w2, x, M, F, scales):
    g = to_dev(_run(ctx, w1, x, M, scales))
    u = to_dev(_run(ctx, w3, x, M, scales))
    a = empty_bf16(M, F)
    sync()
    ctx.swiglu(g, u, a, M, F)
    sync()
    return from_dev(a), _run(ctx, w2, a, M, scales)


@pytest.mark.parametrize("M,H,F,bits,w3_slots,scales", [
    (260, 384, 640, 4, 8, CFG2_SCALES),     # the config-2 set on all three
    (300, 256, 320, 8, 8, CFG2_SCALES),     # w8, F not a whole 128-column tile
    (513, 256, 448, 4, 8, None),            # no live adapter: no tail at all
    (260, 384, 640, 4, 6, CFG2_SCALES),     # w3 with fewer tail chunks than w1
    # 17 x 16 = 272 paired tiles: the second round holds one tile row, which
    # runs as 128-row tiles in a launch of its own
    (4352, 256, 2048, 4, 8, CFG2_SCALES),
    (4300, 256, 2048, 8, 8, CFG2_SCALES),   # w8, the half-tile rows ragged
    # one and two 64-wide K stages in the paired launch (its ring's
    # prologue and remainder with no full trip)
    (4352, 64, 2048, 4, 8, CFG2_SCALES),
    (4352, 128, 2048, 4, 8, CFG2_SCALES),
])
def test_ffn_equals_the_four_calls(ctx, orc, M, H, F, bits, w3_slots, scales):
    """ming_ffn == lin(w1), lin(w3), swiglu, lin(w2) bit for bit, h included.
    On the fast route w1 and w3 run as one paired launch (128 columns of each
    per tile, the SwiGLU taken in LDS) unless their LoRA tails differ in
    length; either way the bits are the separate calls'."""
    print(f"case ffn M={M} H={H} F={F} bits={bits} w3_slots={w3_slots}", flush=True)
    w1, w3, w2 = _ffn_weights(ctx, 620, H, F, bits)
    for s in range(w3_slots, 8):
        w3.unbind_lora(s)
    x = to_dev(bf16(randn(621, (M, H))))
    h_ref, ref = _ffn_four_calls(ctx, w1, w3, w2, x, M, F, scales)
    y = empty_bf16(M, H)
    sync()
    e0 = ctx.engagement()
    h = ctx.ffn(w1, w3, w2, x, y, M, scales)
    sync()
    e1 = ctx.engagement()
    assert e1["gemm_q4" if bits == 4 else "gemm_q8"] - e0["gemm_q4" if bits == 4 else "gemm_q8"] == 3
    assert e1["lora_proj"] - e0["lora_proj"] == (3 if scales else 0)
    # the config-2 set ends in its rank-128 slot 7, so unbinding slots 6-7
    # leaves w3 fewer 32-rank chunks than w1
    paired = route_is_auto(ctx) and w3_slots == 8
    assert e1["gemm_paired"] - e0["gemm_paired"] == (1 if paired else 0)
    assert np.array_equal(from_dev(h), h_ref)
    assert np.array_equal(from_dev(y), ref)


def test_ffn_rejects_mismatched_shapes(ctx):
    M, H, F = 64, 256, 512
    w1, w3, w2 = _ffn_weights(ctx, 630, H, F)
    x = to_dev(bf16(randn(631, (M, H))))
    y = empty_bf16(M, H)
    with pytest.raises(m.MingError):
        ctx.ffn(w1, w2, w2, x, y, M)


@pytest.mark.parametrize("M,N,K", [(256, 3840, 2560), (4096, 64, 3840), (200, 192, 1024)])
def test_dense_few_tiles_parity(ctx, orc, M, N, K):
    """Dense weights whose output is a few 256 x 256 tiles (the caption
    embedder, the final layer) take the split-K GEMM on the auto route: to
    the bar against the fp32 reference, with row strides, writing only the
    M x N block (the route fixture runs the general kernel on it as well)."""
    print(f"case dense M={M} N={N} K={K}", flush=True)
    x = bf16(randn(700 + M, (M, K + 64)))
    pack, w = make_weight(701 + N, N, K, 16)
    qw = _qw(ctx, pack, 16)
    ldy = N + 36
    y = to_dev(np.full((M, ldy), 0x2345, np.uint16))
    sync()
    ctx.reset_engagement()
    ctx.lin(qw, to_dev(x), y, M, ldx=K + 64, ldy=ldy)
    sync()
    eng = ctx.engagement()
    assert eng["gemm_dense"] == 1 and eng["gemm_fast"] == 0 and eng["gemv"] == 0
    out = from_dev(y)
    assert (out[:, N:] == 0x2345).all()
    ref = orc.proj(np.ascontiguousarray(x[:, :K]), w)
    assert _rel(orc, np.ascontiguousarray(out[:, :N]), ref) <= TOL
    qw.close()


@pytest.mark.parametrize("bits", [4, 8])
def test_few_tiles_split_k_parity(ctx, orc, bits):
    """A fast-route projection over 256 rows (the context refiner's caption
    rows: 15 tiles of 256 x 256) splits K across the chip, the last slice
    carrying the LoRA tail: to the bar against the fp32 reference with the
    config-2 adapter set (the route fixture runs the unsplit general kernel
    on it as well)."""
    M, N, K = 256, 3840, 3840
    print(f"case split bits={bits} M={M} N={N} K={K}", flush=True)
    x = bf16(randn(41, (M, K)))
    pack, w = make_weight(42, N, K, bits)
    qw = _qw(ctx, pack, bits)
    loras = []
    for s, r in enumerate(CFG2_RANKS):
        A, B = make_lora(300 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        loras.append((A, B, CFG2_SCALES[s]))
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M, CFG2_SCALES)
    eng = ctx.engagement()
    assert eng["lora_proj"] == 1 and eng["gemm_fast"] == (1 if route_is_auto(ctx) else 0)
    assert eng["gemm_split"] == eng["gemm_fast"]
    ref = orc.proj(x, w, loras)
    assert _rel(orc, y, ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w)) > 10 * TOL
    qw.close()


def test_few_tiles_ffn_equals_the_four_calls(ctx):
    """ming_ffn over 256 rows at full width (w1, w3: 40 tiles, w2: 15, all
    split on the fast route; the split reduce applies w3's SwiGLU and writes
    the fp16 copy of h) == lin(w1), lin(w3), swiglu, lin(w2) bit for bit."""
    M, H, F = 256, 3840, 10240
    w1, w3, w2 = _ffn_weights(ctx, 640, H, F)
    x = to_dev(bf16(randn(641, (M, H))))
    g = to_dev(_run(ctx, w1, x, M, CFG2_SCALES))
    u = to_dev(_run(ctx, w3, x, M, CFG2_SCALES))
    a = empty_bf16(M, F)
    sync()
    ctx.swiglu(g, u, a, M, F)
    sync()
    ref = _run(ctx, w2, a, M, CFG2_SCALES)
    y = empty_bf16(M, H)
    ctx.ffn(w1, w3, w2, x, y, M, CFG2_SCALES)
    sync()
    assert np.array_equal(from_dev(y), ref)
    assert np.all(np.isfinite(orc_f32(from_dev(y))))
    for wt in (w1, w3, w2):
        wt.close()


# The stacked x.A over thousands of rows: stacked widths of 64 to 896
# columns (half-filled 128-column blocks included), ragged row counts, and K
# of one to three 64-wide steps (fewer than the stage ring holds).
MANY_ROWS_XA_CASES = [
    (2085, 256, 192, [16], [0.7]),
    (2085, 256, 192, [128, 64, 32, 16, 8, 4], [0.3, -0.5, 1.1, 0.9, 0.0, 1.4]),
    (4352, 256, 192, list(CFG2_RANKS), list(CFG2_SCALES)),
    (4300, 256, 128, [128, 128, 128, 128, 64], [0.4, -0.2, 0.0, 0.3, 1.0]),
    (4300, 256, 64, [128] * 7, [0.2, -0.3, 0.25, 0.0, 0.15, -0.1, 0.3]),
]


@pytest.mark.parametrize("M,N,K,ranks,scales", MANY_ROWS_XA_CASES)
def test_many_rows_xa_parity(ctx, orc, M, N, K, ranks, scales):
    """One projection with up to seven live adapters over 2085-4352 rows
    against the oracle."""
    print(f"case many-rows x.A M={M} N={N} K={K} ranks={ranks}", flush=True)
    x = bf16(randn(3000 + M + K, (M, K)))
    pack, w = make_weight(3001 + len(ranks), N, K, 4)
    qw = _qw(ctx, pack, 4)
    loras = []
    for s, r in enumerate(ranks):
        A, B = make_lora(3100 + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        loras.append((A, B, scales[s]))
    sc = list(scales) + [0.0] * (8 - len(scales))
    ctx.reset_engagement()
    y = _run(ctx, qw, to_dev(x), M, sc)
    eng = ctx.engagement()
    assert eng["lora_xa"] == 1 and eng["lora_proj"] == 1
    ref = orc.proj(x, w, loras)
    assert _rel(orc, y, ref) <= TOL
    assert orc.rel_l2(ref, orc.proj(x, w)) > 10 * TOL
    qw.close()


def test_many_rows_xa_stacking_moves_no_bits(ctx):
    """Over 2085 rows q|k|v fused (768 stacked T columns) gives the bits of
    the three projections run alone (256 columns each), and ming_ffn (w1|w3
    stacked) the bits of the four calls."""
    M, H, K = 2085, 256, 256
    x = to_dev(bf16(randn(3201, (M, K))))
    parts = []
    for i in range(3):
        pack, _ = make_weight(3202 + i, H, K, 4)
        p = _qw(ctx, pack, 4)
        for s in range(2):
            A, B = make_lora(3210 + 4 * i + 2 * s, H, K, 128)
            p.bind_lora(s, A, B)
        parts.append(p)
    fused = m.QWeight.concat(ctx, parts)
    sc = [0.8, -0.6]
    yf = _run(ctx, fused, x, M, sc)
    for i, p in enumerate(parts):
        assert np.array_equal(yf[:, i * H:(i + 1) * H], _run(ctx, p, x, M, sc))
    for p in parts + [fused]:
        p.close()

    Hf, F = 384, 640
    w1, w3, w2 = _ffn_weights(ctx, 3220, Hf, F)
    x = to_dev(bf16(randn(3221, (M, Hf))))
    g = to_dev(_run(ctx, w1, x, M, CFG2_SCALES))
    u = to_dev(_run(ctx, w3, x, M, CFG2_SCALES))
    a = empty_bf16(M, F)
    sync()
    ctx.swiglu(g, u, a, M, F)
    sync()
    ref = _run(ctx, w2, a, M, CFG2_SCALES)
    y = empty_bf16(M, Hf)
    ctx.ffn(w1, w3, w2, x, y, M, CFG2_SCALES)
    sync()
    assert np.array_equal(from_dev(y), ref)
    for wt in (w1, w3, w2):
        wt.close()


def orc_f32(v):
    return (v.astype(np.uint32) << 16).view(np.float32)


def _cfg2_rows(M, tile=256):
    """A row sample covering every 256-row M tile: its first and last row
    and one interior row that moves from tile to tile."""
    rows = []
    for t in range((M + tile - 1) // tile):
        lo, hi = t * tile, min(M, (t + 1) * tile) - 1
        rows += [lo, min(hi, lo + 1 + (37 * t) % (tile - 2)), hi]
    return np.array(sorted(set(rows)), np.int64)


def _ffn_full_size(ctx, orc, bits, ranks, scales, seed, label):
    """One block's SwiGLU FFN at the configs' full size through ming_ffn (the
    bench's step): X [4352, 3840] ~ N(0, 1) bf16, w1/w3 3840 -> 10240 and w2
    10240 -> 3840 as w{bits}g64 packs of N(0, 0.02) weights, the adapter set
    (ranks, strengths) on all three. On the fast route w1 and w3 run as one
    paired launch (17 x 80 tiles of 128 columns of each, the SwiGLU taken in
    LDS) and w2 as the unsplit kernel (17 x 15 tiles), each with the tail of
    the live ranks in 32-rank chunks. Held on a row sample over all 17 M tiles
    against the oracle (gpu_ff, ming-dit.cc:2151-2162):
      * each stage on its own input, to the projection bar (2e-3): h (w3's
        fused epilogue) vs swiglu(bf16(x.W1'), bf16(x.W3')), and y vs the
        f32 w2 on the kernel's own h;
      * the whole chain by the reference's rule for a result that passes
        through more than one bf16 rounding (ming-dit-test.cc:2125-2131;
        ming-quant-test.cc:826-831): y within twice the distance of the
        bf16-rounded oracle chain (g, u, h and y each rounded) from the f32
        chain (nothing rounded), floored at the projection bar."""
    M, H, F = 4352, 3840, 10240
    x = bf16(randn(seed + 1, (M, H)))
    packs, loras = [], []
    for i, (N, K) in enumerate(((F, H), (F, H), (H, F))):
        codes, sc, bi = orc.quantize(randn(seed + 10 + i, (N, K), 0.02), bits)
        packs.append((codes, sc, bi))
        lo = []
        for s, r in enumerate(ranks):
            A = bf16(randn(seed + 100 + 20 * i + 2 * s, (r, K), 1.0 / np.sqrt(K)))
            B = bf16(randn(seed + 101 + 20 * i + 2 * s, (N, r), 0.01))
            lo.append((A, B, scales[s]))
        loras.append(lo)
    ws = []
    for (codes, sc, bi), lo in zip(packs, loras):
        qw = m.QWeight.quantized(ctx, codes, sc, bi, bits)
        for s, (A, B, _) in enumerate(lo):
            qw.bind_lora(s, A, B)
        ws.append(qw)
    xd = to_dev(x)
    y = empty_bf16(M, H)
    h = empty_bf16(M, F)
    sync()
    ctx.reset_engagement()
    ctx.ffn(ws[0], ws[1], ws[2], xd, y, M, scales, h=h)
    sync()
    eng = ctx.engagement()
    auto = route_is_auto(ctx)
    live = sum(r for r, s in zip(ranks, scales) if s != 0.0)
    assert eng["gemm_q%d" % bits] == 3 and eng["lora_proj"] == 3 and eng["lora_xa"] == 2
    assert eng["gemm_fast"] == (3 if auto else 0) and eng["gemm_split"] == 0
    assert eng["gemm_paired"] == (1 if auto else 0)
    # the live stack the tails walk: every live rank, counted in the FLOP
    assert eng["gemm_flops"] == 3 * 2 * M * H * F + 3 * 2 * M * live * (H + F)
    rows = _cfg2_rows(M)
    assert len(rows) == 51 and rows[-1] == M - 1
    yh, hh = from_dev(y)[rows], from_dev(h)[rows]
    xs = np.ascontiguousarray(x[rows])

    def qp(inp, i):
        codes, sc, bi = packs[i]
        return orc.qproj_packed(np.ascontiguousarray(inp), codes, sc, bi, bits, loras[i])

    g = qp(xs, 0)
    u = qp(xs, 1)
    h_ref = orc.swiglu(orc.f32_to_bf16(g), orc.f32_to_bf16(u))
    rel_h = orc.rel_l2(orc.bf16_to_f32(hh), orc.bf16_to_f32(h_ref))
    rel_y_own = _rel(orc, yh, qp(hh, 2))
    # the f32 chain: SiLU(g) * u and w2 (dequantized, with its adapters) on it
    # in f64, nothing rounded to bf16
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    h32 = g64 / (1.0 + np.exp(-g64)) * u64
    w2 = orc.dequant(*packs[2], bits).astype(np.float64)
    y32 = h32 @ w2.T
    for A, B, s in loras[2]:
        if s != 0.0:
            y32 += np.float64(np.float32(s)) * ((h32 @ orc.bf16_to_f32(A).astype(np.float64).T)
                                                @ orc.bf16_to_f32(B).astype(np.float64).T)
    y_bf = orc.bf16_to_f32(orc.f32_to_bf16(qp(h_ref, 2)))
    floor = orc.rel_l2(y_bf, y32)
    bar = max(TOL, 2.0 * floor)
    rel_y = orc.rel_l2(orc.bf16_to_f32(yh), y32)
    base = orc.qproj_packed(xs, *packs[0], bits)
    moved = orc.rel_l2(g, base)
    print(f"{label} ffn ({'auto' if auto else 'general'}): h rel-L2 {rel_h:.3e}, "
          f"y vs w2(own h) {rel_y_own:.3e}, y vs f32 chain {rel_y:.3e} (bf16 chain "
          f"{floor:.3e}, bar {bar:.3e}), adapters move w1 by {moved:.3e}", flush=True)
    assert rel_h <= TOL and rel_y_own <= TOL and rel_y <= bar
    assert moved > 10 * TOL
    for w in ws:
        w.close()


def test_config2_ffn_full_size(ctx, orc):
    """BASELINE configs[1] exactly: w4g64, the eight slots {4, 8, 16, 16, 32,
    32, 64, 128} at strengths {1, .5, 0, -.3, .8, 0, 1.2, .25} on all three
    weights (252 live ranks: an 8-chunk tail)."""
    _ffn_full_size(ctx, orc, 4, CFG2_RANKS, CFG2_SCALES, 2000, "configs[1]")


def test_config5_ffn_w8_full_size(ctx, orc):
    """BASELINE configs[4]'s arithmetic on one block's FFN: w8g64 packs with
    eight rank-64 slots at strengths uniform in [-1, 1.5] (all live: 512
    ranks, a 16-chunk tail) on all three weights, through the w8 paired and
    unsplit kernels."""
    _ffn_full_size(ctx, orc, 8, CFG5_RANKS, CFG5_SCALES, 5000, "configs[4]")


def test_config5_projection_w8_full_size(ctx, orc):
    """One w8 3840 x 3840 projection over 4352 rows with configs[4]'s eight
    rank-64 slots (255 tiles: the unsplit fast kernel, a 16-chunk tail),
    against the oracle on a row sample over all 17 M tiles; all strengths 0
    gives the unadapted bits."""
    M, N, K = 4352, 3840, 3840
    x = bf16(randn(5101, (M, K)))
    codes, sc, bi = orc.quantize(randn(5102, (N, K), 0.02), 8)
    qw = m.QWeight.quantized(ctx, codes, sc, bi, 8)
    plain = m.QWeight.quantized(ctx, codes, sc, bi, 8)
    loras = []
    for s, r in enumerate(CFG5_RANKS):
        A = bf16(randn(5110 + 2 * s, (r, K), 1.0 / np.sqrt(K)))
        B = bf16(randn(5111 + 2 * s, (N, r), 0.01))
        qw.bind_lora(s, A, B)
        loras.append((A, B, CFG5_SCALES[s]))
    xd = to_dev(x)
    ctx.reset_engagement()
    y = _run(ctx, qw, xd, M, CFG5_SCALES)
    eng = ctx.engagement()
    auto = route_is_auto(ctx)
    assert eng["gemm_q8"] == 1 and eng["lora_proj"] == 1 and eng["lora_xa"] == 1
    assert eng["gemm_fast"] == (1 if auto else 0) and eng["gemm_split"] == 0
    assert eng["gemm_flops"] == 2 * M * N * K + 2 * M * 512 * (K + N)
    rows = _cfg2_rows(M)
    ref = orc.qproj_packed(np.ascontiguousarray(x[rows]), codes, sc, bi, 8, loras)
    rel = _rel(orc, np.ascontiguousarray(y[rows]), ref)
    moved = orc.rel_l2(ref, orc.qproj_packed(np.ascontiguousarray(x[rows]), codes, sc, bi, 8))
    print(f"configs[4] w8 projection ({'auto' if auto else 'general'}): rel-L2 {rel:.3e}, "
          f"adapters move it by {moved:.3e}", flush=True)
    assert rel <= TOL and moved > 10 * TOL
    y0 = _run(ctx, qw, xd, M, [0.0] * 8)
    assert np.array_equal(y0, _run(ctx, plain, xd, M))
    qw.close()
    plain.close()
