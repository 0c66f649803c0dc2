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
