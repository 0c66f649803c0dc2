"""A seeded sweep over projection shapes and adapter sets the other tests do
not pick: M, N and K drawn over ragged tile edges (M any, N a multiple of 8,
K a multiple of 64), w4 and w8, one to eight slots of ranks 1-40 at random
strengths (some 0). Each case runs on the auto and the general route and is
held to the oracle at the projection bar; the all-zero strengths give the
unadapted weight's bits."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import bf16, empty_bf16, from_dev, make_lora, make_weight, randn, sync, to_dev

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _cases(n=16, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.integers(1, 2600))
        N = 8 * int(rng.integers(1, 200))
        K = 64 * int(rng.integers(1, 40))
        bits = int(rng.choice([4, 8]))
        nslots = int(rng.integers(1, 9))
        slots = sorted(rng.choice(8, nslots, replace=False).tolist())
        ranks = [int(rng.integers(1, 41)) for _ in slots]
        scales = [float(rng.choice([0.0, rng.uniform(-1.5, 1.5)], p=[0.2, 0.8])) for _ in slots]
        out.append((i, M, N, K, bits, slots, ranks, scales))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"s{c[0]}-M{c[1]}-N{c[2]}-K{c[3]}-w{c[4]}")
def test_projection_sweep(ctx, orc, case):
    i, M, N, K, bits, slots, ranks, scales = case
    print(f"case sweep {case}", flush=True)
    x = bf16(randn(5000 + i, (M, K)))
    pack, w = make_weight(5100 + i, N, K, bits)
    qw = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)
    plain = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)
    sc8 = [0.0] * 8
    loras = [None] * 8
    for s, r, v in zip(slots, ranks, scales):
        A, B = make_lora(5200 + 20 * i + 2 * s, N, K, r)
        qw.bind_lora(s, A, B)
        sc8[s] = v
        loras[s] = (A, B, v)
    xd = to_dev(x)
    ref = orc.proj(x, w, [l for l in loras if l is not None])
    outs = {}
    for route in ("auto", "general"):
        ctx.set_route(route)
        y = empty_bf16(M, N)
        sync()
        ctx.lin(qw, xd, y, M, sc8)
        sync()
        outs[route] = from_dev(y)
        rel = orc.rel_l2(orc.bf16_to_f32(outs[route]), ref)
        assert rel <= TOL, (route, rel)
    ctx.set_route("auto")
    # all strengths 0: the unadapted bits
    y0, yp = empty_bf16(M, N), empty_bf16(M, N)
    sync()
    ctx.lin(qw, xd, y0, M, [0.0] * 8)
    ctx.lin(plain, xd, yp, M, None)
    sync()
    assert np.array_equal(from_dev(y0), from_dev(yp))
    qw.close()
    plain.close()


def _ffn_cases(n=10, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        # half the draws reach 64 tiles (no K split); the rest split K
        # where H holds 12 stages
        big = i % 2 == 0
        M = int(rng.integers(2000, 4400) if big else rng.integers(1, 1500))
        F = 64 * int(rng.integers(24, 48) if big else rng.integers(1, 30))
        H = 64 * int(rng.integers(1, 16))
        bits = int(rng.choice([4, 8]))
        nslots = int(rng.integers(0, 9))
        slots = sorted(rng.choice(8, nslots, replace=False).tolist())
        ranks = [int(rng.integers(1, 41)) for _ in slots]
        scales = [float(rng.uniform(-1.5, 1.5)) for _ in slots]
        out.append((i, M, H, F, bits, slots, ranks, scales))
    return out


def _lin(ctx, qw, x, M, sc8):
    y = empty_bf16(M, qw.N)
    sync()
    ctx.lin(qw, x, y, M, sc8)
    sync()
    return y


@pytest.mark.parametrize("case", _ffn_cases(), ids=lambda c: f"f{c[0]}-M{c[1]}-H{c[2]}-F{c[3]}-w{c[4]}")
def test_ffn_sweep(ctx, case):
    """ming_ffn == lin(w1), lin(w3), swiglu, lin(w2) bit for bit, h and y,
    on both routes; on the auto route w1 and w3 pair exactly when neither is
    split along K (the same slots on both, so the same tail)."""
    i, M, H, F, bits, slots, ranks, scales = case
    print(f"case ffn sweep {case}", flush=True)
    ws = []
    for j, (N, K) in enumerate(((F, H), (F, H), (H, F))):
        pack, _ = make_weight(6000 + 10 * i + j, N, K, bits)
        qw = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], bits)
        for s, r in zip(slots, ranks):
            A, B = make_lora(6400 + 100 * i + 20 * j + 2 * s, N, K, r)
            qw.bind_lora(s, A, B)
        ws.append(qw)
    sc8 = [0.0] * 8
    for s, v in zip(slots, scales):
        sc8[s] = v
    x = to_dev(bf16(randn(8900 + i, (M, H))))
    tiles = ((M + 255) // 256) * ((F + 255) // 256)
    for route in ("auto", "general"):
        ctx.set_route(route)
        g = _lin(ctx, ws[0], x, M, sc8)
        u = _lin(ctx, ws[1], x, M, sc8)
        a = empty_bf16(M, F)
        sync()
        ctx.swiglu(g, u, a, M, F)
        sync()
        y_ref = from_dev(_lin(ctx, ws[2], a, M, sc8))
        y = empty_bf16(M, H)
        e0 = ctx.engagement()
        h = ctx.ffn(ws[0], ws[1], ws[2], x, y, M, sc8)
        sync()
        e1 = ctx.engagement()
        # few tiles split K (>= 2 slices of >= 6 64-wide stages), which
        # rules the pair out
        split = tiles < 64 and min(256 // tiles, (H // 64) // 6) >= 2
        paired = route == "auto" and not split
        assert e1["gemm_paired"] - e0["gemm_paired"] == (1 if paired else 0)
        assert np.array_equal(from_dev(h), from_dev(a)), route
        assert np.array_equal(from_dev(y), y_ref), route
    ctx.set_route("auto")
    for qw in ws:
        qw.close()
