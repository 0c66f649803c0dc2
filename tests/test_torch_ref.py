"""Pins the torch reference (tests/torch_ref.py) against the CPU oracle at
reduced width, on the CPU, before the full-size GPU tests use it as their
fp32 reference.

The "bf16" mode rounds where the oracle rounds; what separates them is f32
against f64 accumulation, which flips a few bf16 roundings that later norms
and residuals carry on. The "f32" mode keeps every intermediate in fp32 and
so sits at the oracle's rounding floor. A plausible mistake (a pair rotated
the wrong way, w1 and w3 swapped, a norm dropped, a tanh gate missing) moves
either far past these bars (O(0.1-1)).
"""
import numpy as np
import pytest
import torch

import oracle as orc
import torch_ref as tr
from helpers import bf16, build_block, build_model, f32, grid_positions, make_weight, randn

H, NH, F, ADA = 256, 2, 512, 64
SCALES = (1.0, 0.0, 0.0, -0.5, 0.0, 0.0, 0.0, 0.0)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_is_the_oracles(bits):
    pack, w = make_weight(5, 96, 320, bits)
    got = tr.dequant(pack["codes"], pack["scales"], pack["biases"], bits, "cpu")
    assert torch.equal(got, torch.from_numpy(w))


def test_rope_is_the_oracles():
    rows = 40
    x = bf16(randn(7, (rows, 2 * 128)))
    pt, ph, pw = grid_positions(rows)
    c, s = orc.rope_table(pt, ph, pw)
    want = orc.rope_apply(x, 0, 2, 128, c, s)
    R = tr.Ref("bf16", "cpu")
    got = R.rope(tr.bf(x, "cpu").reshape(rows, 2, 128), torch.from_numpy(c),
                 torch.from_numpy(s)).reshape(rows, -1)
    assert torch.equal(got, torch.from_numpy(f32(want)))


@pytest.mark.parametrize("modulated,rows", [(True, 200), (False, 96)])
def test_block_matches_oracle(modulated, rows):
    ob, _, _ = build_block(None, 500 + rows, H, F, ADA, 4, modulated)
    x = bf16(randn(41, (rows, H)))
    temb = bf16(randn(43, (ADA,))) if modulated else None
    c, s = orc.rope_table(*grid_positions(rows))
    ref = orc.block_forward(x, ob, NH, c, s, temb, SCALES)
    xt = tr.bf(x, "cpu")
    want_out, want_upd = torch.from_numpy(f32(ref)), torch.from_numpy(f32(ref) - f32(x))
    bars = {"bf16": (5e-3, 1e-2), "f32": (1e-2, 2e-2)}
    for mode, (b_out, b_upd) in bars.items():
        R = tr.Ref(mode, "cpu")
        y = R.block(xt, ob, NH, torch.from_numpy(c), torch.from_numpy(s),
                    None if temb is None else tr.bf(temb, "cpu"), SCALES)
        out, upd = tr.rel_l2(y, want_out), tr.rel_l2(y - xt, want_upd)
        print(f"torch ref block ({mode}, modulated={modulated}): output {out:.3e}, "
              f"update {upd:.3e}")
        assert out <= b_out and upd <= b_upd


def test_forward_matches_oracle():
    from test_model_gpu import CAP, QROWS, inputs
    mo, _ = build_model(None, 7)
    lay, img, lat, cap, cs = inputs()
    ref = orc.model_forward(mo, lat, cap, img, CAP, QROWS, lay["pos_t"], lay["pos_h"],
                            lay["pos_w"], 0.6, SCALES)
    c, s = orc.rope_table(lay["pos_t"], lay["pos_h"], lay["pos_w"])
    tin = orc.time_proj(0.6, 1000.0, mo["time_freq"])
    for mode, bar in (("bf16", 1e-2), ("f32", 2e-2)):
        y = tr.Ref(mode, "cpu").forward(mo, lat, cap, img, CAP, QROWS, c, s, 0.6, SCALES,
                                        tin)
        rel = tr.rel_l2(y, torch.from_numpy(f32(ref)))
        print(f"torch ref forward ({mode}): velocity rel-L2 {rel:.3e}")
        assert rel <= bar


def test_a_planted_mistake_is_caught():
    """w1 and w3 swapped in one block moves the torch block far past the bar."""
    rows = 64
    ob, _, _ = build_block(None, 321, H, F, ADA, 4, True)
    x = bf16(randn(44, (rows, H)))
    temb = bf16(randn(45, (ADA,)))
    c, s = orc.rope_table(*grid_positions(rows))
    ref = orc.block_forward(x, ob, NH, c, s, temb, SCALES)
    bad = dict(ob, w1=ob["w3"], w3=ob["w1"])
    xt = tr.bf(x, "cpu")
    y = tr.Ref("f32", "cpu").block(xt, bad, NH, torch.from_numpy(c), torch.from_numpy(s),
                                   tr.bf(temb, "cpu"), SCALES)
    assert tr.rel_l2(y - xt, torch.from_numpy(f32(ref) - f32(x))) > 0.2
