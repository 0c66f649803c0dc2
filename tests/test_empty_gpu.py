"""Zero-row calls: every entry point that takes a row count accepts 0, returns
MING_OK, launches nothing (the engagement counters do not move) and writes
nothing (sentinel outputs keep their bits) -- the empty batch the reference's
callers may hand over (a caption of query rows only, an empty chunk)."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import (CFG2_RANKS, CFG2_SCALES, bf16, from_dev, make_lora, make_weight,
                     randn, sync, to_dev)

pytestmark = pytest.mark.gpu


def _sentinel(rows, cols):
    return to_dev(np.full((rows, cols), 0x2345, np.uint16))


def test_zero_rows_launch_and_write_nothing(ctx):
    import torch
    H, F = 256, 512
    ws = []
    for i, (N, K) in enumerate(((F, H), (F, H), (H, F))):
        pack, _ = make_weight(800 + i, N, K, 4)
        q = m.QWeight.quantized(ctx, pack["codes"], pack["scales"], pack["biases"], 4)
        for s, r in enumerate(CFG2_RANKS):
            A, B = make_lora(820 + 10 * i + 2 * s, N, K, r)
            q.bind_lora(s, A, B)
        ws.append(q)
    x = to_dev(bf16(randn(850, (8, H))))
    y, h = _sentinel(8, H), _sentinel(8, F)
    w = to_dev(bf16(1.0 + randn(851, (H,), 0.1)))
    qkv = _sentinel(8, 3 * 128 * 2)
    tab = torch.zeros((8, 64), dtype=torch.float32, device="cuda")
    nw = to_dev(bf16(1.0 + randn(852, (128,), 0.1)))
    dpack, _ = make_weight(853, F, H, 16)
    wd = m.QWeight.dense(ctx, dpack["w"])
    bias = to_dev(bf16(randn(854, (F,))))
    sync()
    ctx.reset_engagement()
    before = ctx.engagement()
    for route in ("auto", "general", "wide"):
        ctx.set_route(route)
        ctx.lin(ws[0], x, h, 0, CFG2_SCALES)
        ctx.lin_bias(wd, x, h, 0, bias)
        ctx.lin_noalloc(ws[0], x, h, 0, CFG2_SCALES)
        ctx.lin_swiglu(ws[1], x, h, h, 0, CFG2_SCALES)
        ctx.ffn(ws[0], ws[1], ws[2], x, y, 0, CFG2_SCALES, h=h)
    ctx.set_route("auto")
    ctx.rmsnorm(x, w, y, 0, H)
    ctx.qk_norm_rope(qkv, 3 * 256, 0, 256, 0, 2, nw, nw, tab, tab)
    ctx.llm_qk_norm_rope(qkv, nw, nw, tab, tab, 0, 3 * 256, 2, 2, 64, 1e-6)
    ctx.llm_qk_norm_rope(qkv, nw, nw, tab, tab, 8, 3 * 256, 0, 0, 64, 1e-6)   # no heads
    ctx.attention(qkv, 3 * 256, 0, 256, 512, y, H, 0, 2)
    ctx.swiglu(h, h, h, 0, F)
    ctx.synchronize()
    sync()
    assert ctx.engagement() == before
    assert (from_dev(y) == 0x2345).all() and (from_dev(h) == 0x2345).all()
    assert (from_dev(qkv) == 0x2345).all()
    # and a negative count is refused, not treated as empty
    with pytest.raises(m.MingError):
        ctx.lin(ws[0], x, h, -1, CFG2_SCALES)
    with pytest.raises(m.MingError):
        ctx.rmsnorm(x, w, y, -1, H)
    with pytest.raises(m.MingError):
        ctx.lin_bias(wd, x, h, -1, bias)
    for q in ws:
        q.close()
    wd.close()
