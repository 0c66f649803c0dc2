"""A projection whose input is larger than 4 GiB: 600,000 rows x 3840 bf16
(4.6 GB). The fast route addresses x's fp16 copy with 32-bit byte offsets
from a 64-bit base and takes operands within 2 GiB only, so the host must
refuse it there and run the general kernels, which index in 64 bits; the x.A
takes its general kernel the same way. Held to the oracle on rows spread
over the whole input, rows past the 2 GiB and 4 GiB marks among them."""
import numpy as np
import pytest

import ming_dit_amd as m
from helpers import bf16, from_dev, make_lora, randn

pytestmark = pytest.mark.gpu
TOL = 2e-3


def test_input_beyond_4_gib_runs_the_general_kernels(ctx, orc):
    import torch
    M, N, K = 600_000, 256, 3840
    assert M * K * 2 > 1 << 32
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    w = randn(7001, (N, K), 0.02)
    codes, sc, bi = orc.quantize(w, 4)
    qw = m.QWeight.quantized(ctx, codes, sc, bi, 4)
    A, B = make_lora(7002, N, K, 16)
    qw.bind_lora(0, A, B)
    y = torch.empty((M, N), dtype=torch.int16, device="cuda")
    ctx.set_route("auto")
    torch.cuda.synchronize()
    ctx.reset_engagement()
    ctx.lin(qw, x, y, M, [0.8])
    ctx.synchronize()
    torch.cuda.synchronize()
    eng = ctx.engagement()
    assert eng["gemm_q4"] == 1 and eng["lora_proj"] == 1
    assert eng["gemm_fast"] == 0                    # past the fast route's offset range
    rows = np.array([0, 1, 12_345, 280_000, 559_239, 559_240, 599_000, M - 2, M - 1])
    ri = torch.from_numpy(rows).cuda()
    xs = from_dev(x.index_select(0, ri))
    ys = from_dev(y.index_select(0, ri))
    ref = orc.qproj_packed(xs, codes, sc, bi, 4, [(A, B, 0.8)])
    rel = orc.rel_l2(orc.bf16_to_f32(ys), ref)
    print(f"600k-row projection: rel-L2 {rel:.3e} on rows {rows.tolist()}", flush=True)
    assert rel <= TOL
    del x, y
    qw.close()
