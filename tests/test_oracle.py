"""Pins the CPU oracle (oracle/oracle.c) before anything is compared with it.

Each check is against something the oracle does not compute itself: the
reference's own known answers (ming-config-test.cc), a library routine
(torch's randn and bf16 cast, numpy float64 matmul), a closed form, or an
invariant a plausible mistake would break.
"""
import numpy as np
import pytest
import torch

from helpers import bf16, f32, make_lora, make_weight, randn


# ---- bf16 ---------------------------------------------------------------------
def test_bf16_rne_matches_torch_cast(orc):
    v = np.concatenate([
        randn(7, (4096,)) * 100,
        np.array([1.0, -1.0, 0.0, -0.0, 1.00390625, 1.01171875, 3.4e38,
                  -3.4e38, 1e-40, np.inf, -np.inf], np.float32),
        # exact ties: mantissa ...1 1000..., ...0 1000...
        np.array([np.uint32(0x3F808000).view(np.float32),
                  np.uint32(0x3F818000).view(np.float32)], np.float32)])
    ours = bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(ours, ref.view(np.uint16))


def test_bf16_ties_and_nan(orc):
    L = orc.lib()
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa wins -> 1.0
    assert L.or_bf16_rne(float(np.float32(1.0 + 2.0 ** -8))) == 0x3F80
    # 1 + 3*2^-8 ties between 1+2^-7 (odd) and 1+2^-6 (even) -> up
    assert L.or_bf16_rne(float(np.float32(1.0 + 3 * 2.0 ** -8))) == 0x3F82
    # the generator's copy maps NaN to the quiet NaN 0x7fc0
    assert L.or_bf16_rne_nan(float("nan")) == 0x7FC0
    assert L.or_bf16_to_f32(0x4049) == pytest.approx(3.140625)


# ---- torch randn ------------------------------------------------------------------
def test_randn_known_answers(orc):
    """ming-config-test.cc:99-108, bit for bit."""
    x = orc.randn(42, 1024)
    assert x[0] == np.float32(1.9269150495529175)
    assert x[1] == np.float32(1.4872841835021973)
    assert x[3] == np.float32(-2.1055214405059814)
    assert x[1023] == np.float32(1.5817502737045288)


@pytest.mark.parametrize("seed,n", [(42, 16), (0, 20), (1234, 1000),
                                    (2**33 + 5, 4099)])
def test_randn_matches_torch(orc, seed, n):
    """Same mt19937 stream and sixteen-wide Box-Muller as torch: a wrong
    stream, pairing or tail redraw differs by O(1). torch on x86 takes its
    AVX2 path whose sin/cos/log differ in the last bits (up to ~1.6e-6
    absolute); the bits themselves are pinned by the reference's known
    answers above, which follow the scalar path."""
    g = torch.Generator().manual_seed(seed)
    ref = torch.randn(n, generator=g).numpy()
    assert np.max(np.abs(orc.randn(seed, n) - ref)) <= 2e-6


def test_randn_refuses_below_16(orc):
    with pytest.raises(ValueError):
        orc.randn(1, 15)


# ---- layout, schedule, timestep ---------------------------------------------------
def test_layout_known_answers(orc):
    """ming-config-test.cc:61-84."""
    L = orc.build_layout(32, 32, 256, 34)
    assert (L["img_tokens"], L["cap_len"], L["cap_total"]) == (1024, 290, 320)
    assert L["joint_len"] == 1024 + 290
    pt, ph, pw = L["pos_t"], L["pos_h"], L["pos_w"]
    assert (pt[0], ph[0], pw[0]) == (321, 0, 0)
    assert (pt[33], ph[33], pw[33]) == (321, 1, 1)
    assert (pt[1024], ph[1024]) == (1, 0)
    assert (pt[1024 + 289], pw[1024 + 289]) == (290, 0)
    L2 = orc.build_layout(2, 2, 256, 32)
    assert L2["cap_total"] == 288 and L2["pos_t"][0] == 289
    assert orc.build_layout(2, 2, 256, 20300) is None


def test_layout_config3_grid(orc):
    """64x64 patches + 256 text rows."""
    L = orc.build_layout(64, 64, 0, 256)
    assert L["joint_len"] == 4352 and L["cap_total"] == 256
    assert np.all(L["pos_t"][:4096] == 257)
    assert L["pos_h"][4095] == 63 and L["pos_w"][4095] == 63
    assert np.array_equal(L["pos_t"][4096:], np.arange(1, 257))


def test_schedule_closed_form(orc):
    """ming-config-test.cc:45-59: sigma = 6m/(11+5m), m = 11-k."""
    s = orc.schedule_sigmas(11, 6.0)
    assert s.shape == (12,)
    for k in range(11):
        m = 11 - k
        assert abs(float(s[k]) - 6 * m / (11 + 5 * m)) <= 1e-7
    assert s[0] == 1.0 and s[10] == np.float32(0.375) and s[11] == 0.0
    assert abs(float(s[1]) - 60.0 / 61.0) <= 1e-7


def test_time_proj_closed_form(orc):
    t = orc.time_proj(0.25, 1000.0, 256)
    i = np.arange(128)
    f = np.exp(-np.log(10000.0) * i / 128.0)
    a = 750.0 * f
    assert np.array_equal(t[:128], np.cos(a).astype(np.float32))
    assert np.array_equal(t[128:], np.sin(a).astype(np.float32))
    # sigma 1: t = 0 -> cos 1, sin 0
    t1 = orc.time_proj(1.0)
    assert np.all(t1[:128] == 1.0) and np.all(t1[128:] == 0.0)


# ---- the pack -------------------------------------------------------------------------
def test_pack_hand_built_words(orc):
    """LSB-first codes: w4 codes 1..8 -> 0x87654321; w8 codes -> bytes."""
    K = 64
    # w4 affine: a row whose group spans [0, 15] exactly in steps of 1 -> q = w
    w = np.zeros((1, K), np.float32)
    w[0, :16] = np.arange(16)
    w[0, 16:] = 15.0
    codes, sc, bi = orc.quantize(w, 4)
    assert f32(sc)[0, 0] == 1.0 and f32(bi)[0, 0] == 0.0
    assert codes[0, 0] == 0x76543210 and codes[0, 1] == 0xFEDCBA98
    assert codes[0, 2] == 0xFFFFFFFF
    # w8 symmetric: max |w| = 127 -> s = 1, code = q + 128
    w8 = np.zeros((1, K), np.float32)
    w8[0, :4] = [1, -1, 127, -127]
    codes8, sc8, bi8 = orc.quantize(w8, 8)
    assert f32(sc8)[0, 0] == 1.0 and f32(bi8)[0, 0] == -128.0
    assert codes8[0, 0] == (129 | (127 << 8) | (255 << 16) | (1 << 24))
    assert codes8[0, 1] == 0x80808080


def test_pack_get_code_round_trip(orc):
    rng = np.random.default_rng(3)
    for bits in (4, 8):
        K = 128
        codes = rng.integers(0, 2**32, size=(1, K * bits // 32),
                             dtype=np.uint64).astype(np.uint32)
        row = np.ascontiguousarray(codes[0])
        for k in range(K):
            word = int(row[k * bits // 32])
            sh = (k % (32 // bits)) * bits
            want = (word >> sh) & ((1 << bits) - 1)
            assert orc.lib().or_get_code(row, k, bits) == want


def test_quant_w8_symmetric_exact(orc):
    w = randn(11, (64, 256), 0.02)
    codes, sc, bi = orc.quantize(w, 8)
    dq = orc.dequant(codes, sc, bi, 8)
    s = np.repeat(f32(sc), 64, axis=1)
    # the bias is exactly -128*s, so dq = s*q exactly with |q| <= 127
    assert np.array_equal(f32(bi), -128.0 * f32(sc))
    q = dq / s
    assert np.array_equal(q, np.rint(q)) and np.abs(q).max() <= 127
    # quantization error within half a step (the scale rounds to bf16, so
    # the clamp at 127 can add at most 2^-8 of the group max)
    gmax = np.repeat(np.abs(w.reshape(64, 4, 64)).max(-1), 64, axis=1)
    assert np.all(np.abs(dq - w) <= s / 2 + gmax * 2.0**-8 + 1e-12)


def test_quant_w4_affine_bounds(orc):
    w = randn(12, (32, 512), 0.02)
    codes, sc, bi = orc.quantize(w, 4)
    dq = orc.dequant(codes, sc, bi, 4)
    s = np.repeat(f32(sc), 64, axis=1)
    b = np.repeat(f32(bi), 64, axis=1)
    q = (dq - b) / s
    assert np.allclose(q, np.rint(q), atol=1e-3) and q.min() >= -1e-3
    assert q.max() <= 15 + 1e-3
    # error: half a step plus the bf16 rounding of the scale times 15 and
    # of the bias
    gw = w.reshape(32, 8, 64)
    span = np.repeat(gw.max(-1) - gw.min(-1), 64, axis=1)
    bound = s / 2 + span * 2.0**-8 * 1.01 + np.abs(b) * 2.0**-8 + 1e-9
    assert np.all(np.abs(dq - w) <= bound)


def test_dequant_against_numpy(orc):
    for bits in (4, 8):
        pack, dq = make_weight(5, 16, 192, bits)
        codes = pack["codes"]
        per = 32 // bits
        k = np.arange(192)
        words = codes[:, k // per].astype(np.uint64)
        q = (words >> ((k % per) * bits).astype(np.uint64)) & ((1 << bits) - 1)
        s = np.repeat(f32(pack["scales"]), 64, axis=1)
        b = np.repeat(f32(pack["biases"]), 64, axis=1)
        assert np.array_equal(dq, (s * q.astype(np.float32) + b)
                              .astype(np.float32))


# ---- the projection -----------------------------------------------------------------
def _np_proj(x, w, loras):
    ref = f32(x).astype(np.float64) @ w.astype(np.float64).T
    for A, B, c in loras:
        ref += c * (f32(x).astype(np.float64) @ f32(A).astype(np.float64).T) \
            @ f32(B).astype(np.float64).T
    return ref


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_proj_against_numpy(orc, bits):
    M, N, K = 37, 96, 320
    x = bf16(randn(1, (M, K)))
    pack, w = make_weight(2, N, K, bits)
    loras = []
    for i, r in enumerate((4, 16)):
        A, B = make_lora(10 + 2 * i, N, K, r)
        loras.append((A, B, 0.7 - i))
    y = orc.proj(x, w, loras)
    ref = _np_proj(x, w, loras)
    assert np.max(np.abs(y - ref)) <= 1e-6 * (np.abs(ref).max() + 1)
    if bits != 16:
        yp = orc.qproj_packed(x, pack["codes"], pack["scales"],
                              pack["biases"], bits, loras)
        assert np.array_equal(yp, y)


def test_proj_brute_force_tiny(orc):
    M, N, K = 3, 5, 64
    x = bf16(randn(3, (M, K)))
    w = randn(4, (N, K))
    y = orc.proj(x, w)
    xf = f32(x)
    for m in range(M):
        for n in range(N):
            s = sum(float(xf[m, k]) * float(w[n, k]) for k in range(K))
            assert abs(y[m, n] - s) <= 1e-5


def test_proj_linearity_and_zero(orc):
    M, N, K = 9, 32, 128
    x = bf16(randn(5, (M, K)))
    w1, w2 = randn(6, (N, K)), randn(7, (N, K))
    y12 = orc.proj(x, (w1 + w2).astype(np.float32))
    assert np.allclose(y12, orc.proj(x, w1) + orc.proj(x, w2), atol=1e-4)
    assert np.all(orc.proj(x, np.zeros((N, K), np.float32)) == 0)


def test_lora_zero_strength_is_absent(orc):
    """A 0-strength slot contributes nothing at all (ming-dit.h:150-154)."""
    M, N, K = 11, 64, 192
    x = bf16(randn(8, (M, K)))
    _, w = make_weight(9, N, K, 4)
    A, B = make_lora(20, N, K, 8)
    A2, B2 = make_lora(22, N, K, 16)
    base = orc.proj(x, w)
    assert np.array_equal(orc.proj(x, w, [(A, B, 0.0)]), base)
    assert np.array_equal(orc.proj(x, w, [(A, B, 0.0), (A2, B2, 0.5)]),
                          orc.proj(x, w, [None, (A2, B2, 0.5)]))


def test_lora_two_halves_make_one(orc):
    """One adapter in two slots at 0.5 ~ one slot at 1 (ming-dit-test.cc:1276-1293)."""
    M, N, K = 7, 64, 128
    x = bf16(randn(30, (M, K)))
    _, w = make_weight(31, N, K, 8)
    A, B = make_lora(32, N, K, 16)
    one = orc.proj(x, w, [(A, B, 1.0)])
    two = orc.proj(x, w, [(A, B, 0.5), (A, B, 0.5)])
    assert orc.rel_l2(two, one) < 1e-7
    assert orc.rel_l2(one, orc.proj(x, w)) > 1e-3   # and it moved


# ---- norms ------------------------------------------------------------------------------
def test_rmsnorm_against_numpy(orc):
    x = bf16(randn(40, (50, 3840)))
    w = bf16(1.0 + randn(41, (3840,), 0.1))
    y = orc.rmsnorm(x, w)
    xf = f32(x).astype(np.float64)
    inv = (1.0 / np.sqrt((np.float32((xf * xf).mean(-1)) + np.float32(1e-5))
                         .astype(np.float32))).astype(np.float32)
    ref = (f32(x) * inv[:, None]).astype(np.float32) * f32(w)
    assert np.array_equal(y, bf16(ref))


def test_rmsnorm_power_of_two_invariance(orc):
    x = bf16(randn(42, (8, 128)))
    w = bf16(np.ones(128, np.float32))
    x4 = bf16(f32(x) * 4.0)
    assert np.array_equal(orc.rmsnorm(x, w, eps=0.0), orc.rmsnorm(x4, w, eps=0.0))
    y = f32(orc.rmsnorm(x, w, eps=0.0))
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0,
                       atol=4e-3)


def test_fold_gain_special_cases(orc):
    """nw = norm_w * (1 + scale) (ming-dit.cc:2266-2273): scale 0 is the
    identity, -1 the zero gain, 1 and 3 the exact doublings; a dropped "1 +",
    a swapped operand or an added shift fails one of them."""
    nw = bf16(randn(43, (64,)))
    z = bf16(np.zeros(64, np.float32))
    assert np.array_equal(orc.fold_gain(nw, z), nw)
    assert np.all(f32(orc.fold_gain(nw, bf16(np.full(64, -1.0, np.float32)))) == 0.0)
    assert np.array_equal(orc.fold_gain(nw, bf16(np.ones(64, np.float32))), bf16(2 * f32(nw)))
    assert np.array_equal(orc.fold_gain(nw, bf16(np.full(64, 3.0, np.float32))),
                          bf16(4 * f32(nw)))
    # a per-element scale: one rounding of the f32 product (torch's bf16
    # multiply of exact operands: 1 + s is exact for these s); the fold adds
    # a zero shift, so a -0 product reads +0 (values compared)
    sc = bf16(np.round(randn(44, (64,)) * 8) / 8)
    want = (torch.from_numpy(f32(nw)).to(torch.bfloat16)
            * (1.0 + torch.from_numpy(f32(sc))).to(torch.bfloat16))
    assert np.array_equal(f32(orc.fold_gain(nw, sc)), want.float().numpy())


# ---- rotary -------------------------------------------------------------------------------
def test_rope_table_closed_form_and_axes(orc):
    n = 5
    pt = np.array([0, 5, 321, 20000, 7], np.int32)
    ph = np.array([0, 3, 63, 511, 7], np.int32)
    pw = np.array([0, 9, 1, 0, 7], np.int32)
    c, s = orc.rope_table(pt, ph, pw)
    assert c.shape == (n, 64)
    # position 0 on every axis: identity
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # pair p: axis 0 for p < 16 (d 32), axis 1 for p < 40 (d 48), else axis 2
    for t in range(1, n):
        for p in range(64):
            if p < 16:
                pos, j, d = pt[t], p, 32
            elif p < 40:
                pos, j, d = ph[t], p - 16, 48
            else:
                pos, j, d = pw[t], p - 40, 48
            ang = float(pos) * (1.0 / 256.0 ** (2.0 * j / d))
            assert c[t, p] == np.float32(np.cos(ang))
            assert s[t, p] == np.float32(np.sin(ang))


def test_rope_apply_is_complex_rotation(orc):
    rows, H = 6, 2
    x = bf16(randn(50, (rows, H * 128)))
    L = orc.build_layout(2, 2, 0, 2)
    c, s = orc.rope_table(L["pos_t"], L["pos_h"], L["pos_w"])
    y = orc.rope_apply(x, 0, H, 128, c, s)
    xf = f32(x).reshape(rows, H, 64, 2)
    z = xf[..., 0].astype(np.float32) + 1j * xf[..., 1].astype(np.float32)
    rot = (c + 1j * s)[:, None, :]
    want = z * rot
    yf = f32(y).reshape(rows, H, 64, 2)
    got = yf[..., 0] + 1j * yf[..., 1]
    assert np.max(np.abs(got - want)) <= 2 ** -7 * np.abs(want).max()
    # rotation preserves each pair's norm (to bf16 rounding)
    assert np.allclose(np.abs(got), np.abs(z), rtol=1e-2, atol=1e-2)


def test_qk_norm_rope_is_norm_then_rotation(orc):
    rows, H = 9, 3
    x = bf16(randn(60, (rows, 2 * H * 128)))
    wq = bf16(1.0 + randn(61, (128,), 0.1))
    wk = bf16(1.0 + randn(62, (128,), 0.1))
    L = orc.build_layout(3, 3, 0, 0 + 9 - 9 + 1)
    c, s = orc.rope_table(L["pos_t"][:rows], L["pos_h"][:rows], L["pos_w"][:rows])
    y = orc.qk_norm_rope(x, 0, H * 128, H, 128, wq, wk, c, s)
    q = orc.rmsnorm(x[:, :H * 128].reshape(rows * H, 128), wq).reshape(rows, -1)
    k = orc.rmsnorm(x[:, H * 128:].reshape(rows * H, 128), wk).reshape(rows, -1)
    want = np.concatenate([orc.rope_apply(q, 0, H, 128, c, s),
                           orc.rope_apply(k, 0, H, 128, c, s)], axis=1)
    assert np.array_equal(y, want)


def _angle_tables(rows, R, seed):
    ang = randn(seed, (rows, R)).astype(np.float64) * 3.0
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@pytest.mark.parametrize("rot_half", [32, 64])
def test_llm_qk_norm_rope_is_rotate_half(orc, rot_half):
    """LlmOps::qk_norm_rope (ming_llm.metal:100-178): per-head RMSNorm with
    the q weight on heads [0, n_q) and the k weight on the next n_k, then the
    rotation of the split halves (x_j, x_{j+R}) as one complex number times
    e^{i angle_j}, rounded once; checked against numpy complex128 on the
    normalized values, the earlier-pinned per-head RMSNorm, and the identities
    the definition fixes (rot_half 0, zero angles, the pass-through dims, the
    value columns)."""
    rows, nq, nk, R = 7, 3, 2, rot_half
    nh = nq + nk
    ld = (nh + 2) * 128 + 8                      # value heads after, a ragged tail
    x = bf16(randn(80, (rows, ld)))
    qw = bf16(1.0 + randn(81, (128,), 0.2))
    kw = bf16(0.5 + randn(82, (128,), 0.2))
    c, s = _angle_tables(rows, R, 83 + R)
    y = orc.llm_qk_norm_rope(x, qw, kw, c, s, nq, nk, R)
    assert np.array_equal(y[:, nh * 128:], x[:, nh * 128:])
    # no rotation, no weights: the identity
    assert np.array_equal(orc.llm_qk_norm_rope(x, None, None, None, None, nq, nk, 0), x)
    # normalization alone is the per-head RMSNorm, q weight then k weight
    # (within one rounding of its product order: x * (inv * w) here)
    n0 = orc.llm_qk_norm_rope(x, qw, kw, None, None, nq, nk, 0)
    heads = x[:, :nh * 128].reshape(rows, nh, 128)
    want0 = np.concatenate(
        [orc.rmsnorm(np.ascontiguousarray(heads[:, :nq]).reshape(-1, 128), qw).reshape(rows, nq, 128),
         orc.rmsnorm(np.ascontiguousarray(heads[:, nq:]).reshape(-1, 128), kw).reshape(rows, nk, 128)],
        axis=1)
    u = _ulps(n0[:, :nh * 128].reshape(rows, nh, 128), want0)
    assert u.max() <= 1 and (u > 0).mean() < 0.01
    # zero angles: the normalized heads unchanged, bit for bit
    one, zero = np.ones((rows, R), np.float32), np.zeros((rows, R), np.float32)
    assert np.array_equal(orc.llm_qk_norm_rope(x, qw, kw, one, zero, nq, nk, R), n0)
    # the rotation of the split halves, against complex128 on the normalized values
    v = f32(heads).astype(np.float64)
    inv = 1.0 / np.sqrt((v * v).mean(-1, keepdims=True) + 1e-5)
    w = np.concatenate([np.repeat(f32(qw)[None], nq, 0), np.repeat(f32(kw)[None], nk, 0)])
    xn = v * inv * w[None].astype(np.float64)
    z = xn[..., :R] + 1j * xn[..., R:2 * R]
    want = z * (c.astype(np.float64) + 1j * s.astype(np.float64))[:, None, :]
    yh = f32(y[:, :nh * 128].reshape(rows, nh, 128)).astype(np.float64)
    got = yh[..., :R] + 1j * yh[..., R:2 * R]
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(z) + 1e-30)
    assert np.allclose(np.abs(got), np.abs(z), rtol=1e-2)
    # half-width 32 leaves dims 64..127 as the norm left them
    if R == 32:
        assert np.array_equal(y[:, :nh * 128].reshape(rows, nh, 128)[..., 64:],
                              n0[:, :nh * 128].reshape(rows, nh, 128)[..., 64:])
    if R == 64:      # the DiT's interleaved-pair rotation is another function
        assert not np.array_equal(y, orc.rope_apply(n0, 0, nh, 128, c, s))
    with pytest.raises(ValueError):
        orc.llm_qk_norm_rope(x, qw, kw, c, s, nq, nk, 16)


# ---- block glue ------------------------------------------------------------------------------
def test_attention_against_numpy(orc):
    rows, H, D = 33, 2, 128
    q = bf16(randn(70, (rows, H * D)))
    k = bf16(randn(71, (rows, H * D)))
    v = bf16(randn(72, (rows, H * D)))
    o = f32(orc.attention(q, k, v, H, D))
    qf, kf, vf = (f32(t).reshape(rows, H, D).transpose(1, 0, 2).astype(np.float64)
                  for t in (q, k, v))
    sc = qf @ kf.transpose(0, 2, 1) / np.sqrt(D)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = (p @ vf).transpose(1, 0, 2).reshape(rows, H * D)
    assert np.max(np.abs(o - ref)) <= 2 ** -7 * np.abs(ref).max()


def test_attention_special_cases(orc):
    H, D = 1, 128
    v = bf16(randn(73, (1, D)))
    q = bf16(randn(74, (1, D)))
    # one key: the output is that key's value
    assert np.array_equal(orc.attention(q, q, v, H, D), v)
    # zero queries: uniform weights -> the mean of v
    rows = 16
    v2 = bf16(randn(75, (rows, D)))
    z = bf16(np.zeros((rows, D), np.float32))
    o = f32(orc.attention(z, bf16(randn(76, (rows, D))), v2, H, D))
    assert np.allclose(o, f32(v2).mean(0, keepdims=True), atol=2e-2)


def _ulps(a, b):
    """bf16 distance in units of the last place (sign-aware, -0 == +0)."""
    def key(u):
        v = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(v >= 0x8000, -(v & 0x7FFF), v)
    return np.abs(key(a) - key(b))


def _t(a):
    """bf16 bit patterns -> a float64 torch tensor of their values."""
    return torch.from_numpy(f32(a).astype(np.float64))


def _tb(t):
    """A float torch tensor -> bf16 bit patterns by torch's own cast."""
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_swiglu_against_torch_silu(orc):
    """silu(g) * u rounded once (ming_ops.metal:97-112) against torch's
    F.silu in float64: within one bf16 ulp (f32 expf against f64), and
    the zero and saturation cases exactly."""
    g = bf16(randn(80, (16, 256)) * 3)
    u = bf16(randn(81, (16, 256)))
    got = orc.swiglu(g, u)
    want = _tb(torch.nn.functional.silu(_t(g)) * _t(u))
    d = _ulps(got, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    # silu(0) = 0; u = 0 gives 0; silu(g) -> g for large g, -> 0 for very negative g
    assert np.all(f32(orc.swiglu(bf16(np.zeros(64, np.float32)), u[0, :64])) == 0)
    assert np.all(f32(orc.swiglu(g[0, :64], bf16(np.zeros(64, np.float32)))) == 0)
    big = bf16(np.full(8, 40.0, np.float32))
    one = bf16(np.ones(8, np.float32))
    assert np.array_equal(orc.swiglu(big, one), big)
    assert np.all(np.abs(f32(orc.swiglu(bf16(np.full(8, -40.0, np.float32)), one))) < 1e-15)


def test_gated_residual_against_torch_tanh(orc):
    """h + tanh(gate) * sub rounded once (ming_ops.metal:59-74) against torch's
    tanh in float64; gate 0 leaves h; a gate of +-inf adds +-sub once."""
    h = bf16(randn(82, (8, 128)))
    sub = bf16(randn(81, (8, 128)))
    gate = bf16(randn(83, (128,)))
    got = orc.gated_residual(h, gate, sub)
    want = _tb(_t(h) + torch.tanh(_t(gate))[None, :] * _t(sub))
    d = _ulps(got, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    assert np.array_equal(orc.gated_residual(h, bf16(np.zeros(128, np.float32)), sub), h)
    inf = bf16(np.full(128, np.inf, np.float32))
    assert np.array_equal(orc.gated_residual(h, inf, sub), orc.residual_add(h, sub))


def test_residual_add_is_torch_bf16_add(orc):
    """h + sub rounded once (ming_ops.metal:43-52) is torch's bf16 add (f32 sum,
    round to nearest even) bit for bit; h + (-h) = 0 and h + 0 = h."""
    h = bf16(randn(84, (32, 384)) * 4)
    sub = bf16(randn(85, (32, 384)))
    got = orc.residual_add(h, sub)
    th = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16)
    ts = torch.from_numpy(sub.view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(got, (th + ts).view(torch.int16).numpy().view(np.uint16))
    assert np.all(f32(orc.residual_add(h, bf16(-f32(h)))) == 0)
    assert np.array_equal(orc.residual_add(h, bf16(np.zeros_like(f32(h)))), h)


def test_bias_act_and_silu_against_torch(orc):
    """The timestep MLP's bias (+ SiLU) (ming-dit.cc:2276-2281): the bias add
    is torch's bf16 add bit for bit; SiLU of that bf16 sum is torch's F.silu
    in float64 within one bf16 ulp; silu_bf16 is the same with a zero bias."""
    y = bf16(randn(86, (4, 1024)) * 2)
    b = bf16(randn(87, (1024,)) * 0.5)
    ty = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    s = ty + tb[None, :]
    assert np.array_equal(orc.bias_act(y, b), s.view(torch.int16).numpy().view(np.uint16))
    got = orc.bias_act(y, b, silu=True)
    want = _tb(torch.nn.functional.silu(s.double()))
    d = _ulps(got, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    d = _ulps(orc.silu_bf16(y), _tb(torch.nn.functional.silu(_t(y))))
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    special = bf16(np.array([0.0, 40.0, -40.0, 1.0], np.float32))
    sv = f32(orc.silu_bf16(special))
    assert sv[0] == 0 and sv[1] == 40.0 and -1e-15 < sv[2] <= 0
    assert sv[3] == f32(bf16(np.float32(1.0 / (1.0 + np.exp(-1.0)))))


def test_ln_modulate_against_torch_layer_norm(orc):
    """The final layer's LayerNorm without affine (eps 1e-6), rounded to bf16,
    then * (1 + scale) (ming-dit.cc:2553-2563): with scale 0, torch's
    layer_norm in float64 within one ulp on rows of non-zero mean and spread,
    each row zero-mean and unit-variance; a row whose variance is far below
    eps (the eps placement decides it); scale -1 gives 0, scale 1 doubles."""
    D = 3840
    mu = np.array([0.0, 3.0, -7.5, 100.0], np.float32)[:, None]
    sd = np.array([1.0, 0.25, 4.0, 2.0], np.float32)[:, None]
    x = bf16(randn(88, (4, D)) * sd + mu)
    tiny = bf16(randn(89, (1, D)) * 1e-4)       # variance 1e-8 << eps
    x = np.concatenate([x, tiny])
    zero = bf16(np.zeros(D, np.float32))
    y0 = orc.ln_modulate(x, zero, eps=1e-6)
    want = _tb(torch.nn.functional.layer_norm(_t(x), (D,), eps=1e-6))
    d = _ulps(y0, want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    yf = f32(y0[:4]).astype(np.float64)
    assert np.all(np.abs(yf.mean(-1)) < 1e-2) and np.all(np.abs(yf.var(-1) - 1) < 1e-2)
    # the tiny row is scaled by 1/sqrt(var + eps) ~ 995, not 1/sqrt(var) ~ 1e4
    assert 0.05 < np.sqrt((f32(y0[4]).astype(np.float64) ** 2).mean()) < 0.15
    # at D = 16 the n vs n - 1 variance differs by 3% (~8 ulps): torch's is n
    xs = bf16(randn(90, (64, 16)) * 2 + 1)
    d = _ulps(orc.ln_modulate(xs, zero[:16], eps=1e-6),
              _tb(torch.nn.functional.layer_norm(_t(xs), (16,), eps=1e-6)))
    assert d.max() <= 1
    assert np.all(f32(orc.ln_modulate(x, bf16(np.full(D, -1.0, np.float32)), eps=1e-6)) == 0)
    assert np.array_equal(orc.ln_modulate(x, bf16(np.ones(D, np.float32)), eps=1e-6),
                          bf16(2 * f32(y0)))
