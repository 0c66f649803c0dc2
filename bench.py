#!/usr/bin/env python3
"""Benchmark of the DiT block-projection path on one MI355X.

Metric: w4g64 + 8-LoRA projection TFLOP/s and MFMA
utilisation at 4352 tokens. The workload is BASELINE configs[1]: one
block's SwiGLU FFN, w1/w3 3840->10240 and w2 10240->3840 as w4 group-64
packs, eight runtime-LoRA slots (ranks 4..128, strengths
{1, .5, 0, -.3, .8, 0, 1.2, .25}) on all three, X [4352, 3840] bf16.
A step = lin(w1) + lin(w3) + swiglu + lin(w2), each lin being the stacked
x.A GEMM and the quantized GEMM with the LoRA tail; it runs as one ming_ffn
call (SwiGLU fused into w3's epilogue, x converted to fp16 once). Inputs are synthetic
(seeded torch draws on the GPU, quantized on the GPU by the library's pack
writer) and resident in HBM before the timed region.

`roofline` is for the dominant kernel (qproj.w4): its algorithmic FLOPs
(2MNK + the LoRA tail's 2M*r*N per launch) over its launches' summed
duration, from HIP events the library records around each launch on the
stream it launches on, during the timed steps. `cpu_baseline` times the
scalar C oracle (the same dequant + GEMM + LoRA + SwiGLU, f64 accumulate)
on a bounded row sample on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "vpipe-ming-image_amd")]

M_TOK, HID, FFN = 4352, 3840, 10240
RANKS = (4, 8, 16, 16, 32, 32, 64, 128)
SCALES = (1.0, 0.5, 0.0, -0.3, 0.8, 0.0, 1.2, 0.25)
PEAK_TFLOPS = 2500.0          # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0


def live_rank(ranks=RANKS, scales=SCALES):
    return sum(r for r, s in zip(ranks, scales) if s != 0.0)


def ffn_flops(M):
    R = live_rank()
    base = 2 * M * FFN * HID * 3
    lora = 2 * (2 * M * R * (HID + FFN)) + 2 * M * R * (FFN + HID)
    return base, lora


def build(ctx, m, torch, gen):
    """Synthetic config-2 inputs, resident on the GPU."""
    dev = "cuda"

    def qweight(N, K):
        w = torch.randn((N, K), generator=gen, device=dev) * 0.02
        codes = torch.empty((N, K // 8), dtype=torch.int32, device=dev)
        sc = torch.empty((N, K // 64), dtype=torch.int16, device=dev)
        bi = torch.empty((N, K // 64), dtype=torch.int16, device=dev)
        torch.cuda.synchronize()
        ctx.quantize_pack(w, N, K, 4, codes, sc, bi)
        ctx.synchronize()
        qw = m.QWeight.quantized(ctx, codes, sc, bi, 4, on_device=True)
        host = {"codes": codes.cpu().numpy().view("uint32"),
                "scales": sc.cpu().numpy().view("uint16"),
                "biases": bi.cpu().numpy().view("uint16"), "loras": []}
        for s, r in enumerate(RANKS):
            A = (torch.randn((r, K), generator=gen, device=dev) / K ** 0.5
                 ).to(torch.bfloat16)
            B = (torch.randn((N, r), generator=gen, device=dev) * 0.01
                 ).to(torch.bfloat16)
            torch.cuda.synchronize()
            qw.bind_lora(s, A, B, on_device=True)
            host["loras"].append((A.cpu().view(torch.int16).numpy().view("uint16"),
                                  B.cpu().view(torch.int16).numpy().view("uint16")))
        return qw, host

    w1, h1 = qweight(FFN, HID)
    w3, h3 = qweight(FFN, HID)
    w2, h2 = qweight(HID, FFN)
    x = torch.randn((M_TOK, HID), generator=gen, device=dev).to(torch.bfloat16)
    return (w1, w3, w2), (h1, h3, h2), x


def cpu_baseline(hosts, x_host, target_s, threads):
    """The scalar oracle on a row sample of the same FFN, scaled to TFLOP/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as orc

    h1, h3, h2 = hosts

    def lo(h):
        return [(A, B, s) for (A, B), s in zip(h["loras"], SCALES)]

    def ffn(rows):
        xs = np.ascontiguousarray(x_host[:rows])
        g = orc.qproj_packed(xs, h1["codes"], h1["scales"], h1["biases"], 4,
                             lo(h1), nthreads=threads)
        u = orc.qproj_packed(xs, h3["codes"], h3["scales"], h3["biases"], 4,
                             lo(h3), nthreads=threads)
        a = orc.swiglu(orc.f32_to_bf16(g), orc.f32_to_bf16(u))
        orc.qproj_packed(a, h2["codes"], h2["scales"], h2["biases"], 4,
                         lo(h2), nthreads=threads)

    rows = threads
    t0 = time.perf_counter()
    ffn(rows)
    dt = time.perf_counter() - t0
    if dt < target_s / 3:
        rows = max(rows, min(512, int(rows * target_s / max(dt, 1e-3))))
        rows = max(threads, rows // threads * threads)
        t0 = time.perf_counter()
        ffn(rows)
        dt = time.perf_counter() - t0
    base, lora = ffn_flops(rows)
    cpu = host_cpu()
    return {"value": round((base + lora) / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"{rows} of {M_TOK} token rows of the same FFN step "
                      f"(w1, w3, swiglu, w2 with the 8 LoRA slots), scalar C "
                      f"oracle (f64 accumulation, -O3, no intrinsics), {threads} threads "
                      f"({cpu['affinity']} cores in the process's affinity, nproc "
                      f"{cpu['nproc']}), {dt:.1f} s",
            "cpu_model": cpu["model"], "cpu_mhz": cpu["mhz"], "nproc": cpu["nproc"],
            "affinity_cores": cpu["affinity"], "accumulate": "f64"}


def forward_flops(img, cap, ranks=RANKS, scales=SCALES):
    """Algorithmic FLOP of one 34-block forward (GEMM + live LoRA +
    attention): 2 context-refiner blocks over the caption, 2 noise-refiner
    blocks over the image, 30 layers over the joint sequence."""
    R = live_rank(ranks, scales)
    JT = img + cap
    per_row = 2 * (4 * HID * HID + 3 * HID * FFN)          # q,k,v,o,w1,w3,w2
    lora_row = 2 * R * (4 * (HID + HID) + 3 * (HID + FFN))
    rows = 30 * JT + 2 * img + 2 * cap
    attn = 4 * 30 * 128 * (30 * JT * JT + 2 * img * img + 2 * cap * cap)
    return rows * (per_row + lora_row) + attn


def build_forward_model(ctx, m, torch, gen, n_layers=30, n_refiner=2, bits=4,
                        ranks=RANKS, ref=None):
    """A 34-block w{bits}g64 model with random-init weights (quantized on the
    GPU by the library's pack writer), an adapter of each rank in `ranks`
    bound on all seven projections of every block (slot i = ranks[i]; the
    config-2 set by default), dense embedders and final layer. The model's
    projection weights are listed in model.projections. When `ref` is a
    dict, it is filled with the same weights as device tensors in the layout
    an fp32 reference of the forward reads (the tests' torch reference)."""
    dev = "cuda"
    keep = []
    projections = []
    packs = {}

    def qw(N, K):
        w = torch.randn((N, K), generator=gen, device=dev) * 0.02
        codes = torch.empty((N, K * bits // 32), dtype=torch.int32, device=dev)
        sc = torch.empty((N, K // 64), dtype=torch.int16, device=dev)
        bi = torch.empty((N, K // 64), dtype=torch.int16, device=dev)
        torch.cuda.synchronize()
        ctx.quantize_pack(w, N, K, bits, codes, sc, bi)
        ctx.synchronize()
        q = m.QWeight.quantized(ctx, codes, sc, bi, bits, on_device=True)
        if ref is not None:
            packs[id(q)] = {"codes": codes, "scales": sc, "biases": bi, "bits": bits}
        return q

    def lora(q, N, K):
        projections.append(q)
        kept = []
        for slot, r in enumerate(ranks):
            A = (torch.randn((r, K), generator=gen, device=dev) / K ** 0.5
                 ).to(torch.bfloat16).view(torch.int16)
            B = (torch.randn((N, r), generator=gen, device=dev) * 0.01
                 ).to(torch.bfloat16).view(torch.int16)
            torch.cuda.synchronize()
            q.bind_lora(slot, A, B, on_device=True)
            kept.append((A, B, 1.0))
        return kept

    def vec(n, base, std):
        v = (base + std * torch.randn((n,), generator=gen, device=dev))
        v = v.to(torch.bfloat16).view(torch.int16).contiguous()
        keep.append(v)
        return v

    def dense(N, K):
        w = (torch.randn((N, K), generator=gen, device=dev) / K ** 0.5
             ).to(torch.bfloat16).view(torch.int16).contiguous()
        torch.cuda.synchronize()
        q = m.QWeight.dense(ctx, w, on_device=True)
        if ref is not None:
            packs[id(q)] = {"w": w}
        return q

    def block(modulated):
        parts = {}
        rb = {"loras": {}}
        for name, (N, K) in {"q": (HID, HID), "k": (HID, HID),
                             "v": (HID, HID), "o": (HID, HID),
                             "w1": (FFN, HID), "w3": (FFN, HID),
                             "w2": (HID, FFN)}.items():
            parts[name] = qw(N, K)
            rb["loras"][name] = lora(parts[name], N, K)
        if modulated:
            parts["ada"] = qw(4 * HID, 256)
            parts["ada_b"] = vec(4 * HID, 0.0, 0.1)
        for g in ("an1", "an2", "fn1", "fn2"):
            parts[g] = vec(HID, 1.0, 0.1)
        parts["nq"] = vec(128, 1.0, 0.1)
        parts["nk"] = vec(128, 1.0, 0.1)
        if ref is not None:
            for k, v in parts.items():
                rb[k] = packs.pop(id(v)) if isinstance(v, m.QWeight) else v
            (ref["blocks"] if modulated else ref["ctx_blocks"]).append(rb)
        return m.block_desc(**parts)

    if ref is not None:
        ref.update({"hidden": HID, "n_heads": 30, "n_refiner": n_refiner, "cap_dim": 2560,
                    "time_freq": 256, "t_scale": 1000.0, "eps": 1e-5,
                    "ctx_blocks": [], "blocks": []})
    cb, mb = [], []
    for i in range(2 * n_refiner + n_layers):
        (cb if i < n_refiner else mb).append(block(i >= n_refiner))
        print(f"bench: forward model block {i + 1}/{2 * n_refiner + n_layers}",
              file=sys.stderr, flush=True)
    d = m.ModelDesc()
    d.hidden, d.n_heads, d.ffn = HID, 30, FFN
    d.n_layers, d.n_refiner, d.adaln_dim = n_layers, n_refiner, 256
    d.time_freq, d.time_mid, d.patch_dim, d.cap_dim = 256, 1024, 64, 2560
    d.eps, d.rope_theta, d.t_scale = 1e-5, 256.0, 1000.0
    d.axes[:] = [32, 48, 48]
    d.axes_lens[:] = [1536, 512, 512]
    tw = {"time_1": dense(1024, 256), "time_1b": vec(1024, 0.0, 0.05),
          "time_2": dense(256, 1024), "time_2b": vec(256, 0.0, 0.05),
          "x_in": dense(HID, 64), "x_in_b": vec(HID, 0.0, 0.05),
          "cap_norm": vec(2560, 1.0, 0.1), "cap_in": dense(HID, 2560),
          "cap_in_b": vec(HID, 0.0, 0.05), "final_ada": dense(HID, 256),
          "final_ada_b": vec(HID, 0.0, 0.05), "final_lin": dense(64, HID),
          "final_lin_b": vec(64, 0.0, 0.05)}
    for k, v in tw.items():
        setattr(d, k, m._h(v))
        if ref is not None:
            ref[k] = packs.pop(id(v)) if isinstance(v, m.QWeight) else v
    model = m.Model(ctx, d, cb, mb, keep=keep + [tw, cb, mb])
    model.projections = projections
    return model


def layout_2048():
    """Positions of the 2048^2 joint sequence: a 128 x 128 patch grid (16384
    image tokens) at t = 257, then 256 caption rows at (1 + i, 0, 0)."""
    import numpy as np
    img, cap, grid = 16384, 256, 128
    pt = np.concatenate([np.full(img, cap + 1), 1 + np.arange(cap)]).astype(np.int32)
    ph = np.concatenate([np.arange(img) // grid, np.zeros(cap)]).astype(np.int32)
    pw = np.concatenate([np.arange(img) % grid, np.zeros(cap)]).astype(np.int32)
    return img, cap, (pt, ph, pw)


def run_forward2048(ctx, m, torch, gen, steps):
    """the 34-block w4 forward at 2048^2 with the config-2 adapters
    on all 238 modules; ms per forward after two untimed ones."""
    model = build_forward_model(ctx, m, torch, gen)
    model.set_caption_cache(False)
    for i, sc in enumerate(SCALES):
        model.set_lora_scale(i, sc)
    img, cap, pos = layout_2048()
    lat = torch.randn((img, 64), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    for _ in range(2):
        model.forward(lat, capt, 2560, img, cap, cap, *pos, 0.5, out)
    each = []
    for _ in range(steps):
        t0 = time.perf_counter()
        model.forward(lat, capt, 2560, img, cap, cap, *pos, 0.5, out)
        each.append((time.perf_counter() - t0) * 1e3)
    model.close()
    flops = forward_flops(img, cap)
    med = sorted(each)[len(each) // 2]
    return {"metric": "34-block w4g64 forward @2048^2 (configs[3])", "value": round(med, 2),
            "unit": "ms", "higher_is_better": False, "ms_each": [round(t, 2) for t in each],
            "tflops": round(flops / (med * 1e-3) / 1e12, 2),
            "forward_tflop": round(flops / 1e12, 2), "tokens": img + cap}


def run_cfg2048(ctx, m, torch, gen, steps=11):
    """classifier-free guidance at 2048^2, w8g64, eight r64 slots
    with strengths uniform in [-1, 1.5], `steps` denoise steps (a positive and a
    zero-negative forward each) on the shift-6 schedule; the per-forward ms and
    the sustained TFLOP/s."""
    import numpy as np
    ranks = (64,) * 8
    rng = np.random.default_rng(5)
    scales = tuple(float(v) for v in rng.uniform(-1.0, 1.5, 8))
    model = build_forward_model(ctx, m, torch, gen, bits=8, ranks=ranks)
    for i, sc in enumerate(scales):
        model.set_lora_scale(i, sc)
    img, cap, pos = layout_2048()
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    lat = (torch.randn((img, 64), generator=gen, device="cuda")).float().cpu().numpy()
    torch.cuda.synchronize()
    # one untimed step first (workspaces, both caption cache entries)
    warm = lat.copy()
    model.denoise(warm, capt, 2560, cap, cap, pos, img, 1, 6.0, 4.0)
    marks = [time.perf_counter()]
    model.denoise(lat, capt, 2560, cap, cap, pos, img, steps, 6.0, 4.0,
                  progress=lambda i, n: marks.append(time.perf_counter()) or True)
    model.close()
    per_step = [(b - a) * 1e3 for a, b in zip(marks, marks[1:])]
    flops = 2 * forward_flops(img, cap, ranks, scales)      # positive + negative
    total_s = (marks[-1] - marks[0])
    med = sorted(per_step)[len(per_step) // 2]
    return {"metric": "CFG x2 w8g64 denoise @2048^2 (configs[4])",
            "value": round(flops * steps / total_s / 1e12, 2), "unit": "TFLOP/s sustained",
            "higher_is_better": True, "steps": steps, "guidance": 4.0,
            "ms_per_step_each": [round(t, 1) for t in per_step],
            "ms_per_forward_median": round(med / 2, 2),
            "step_tflop": round(flops / 1e12, 2), "lora_scales": [round(v, 3) for v in scales],
            "finite": bool(np.isfinite(lat).all())}


def time_forward(ctx, m, torch, gen, steps, warmup):
    """34-block forward at 1024^2 (4096 image + 256 caption tokens): ms per
    forward, host clock around ming_model_forward (synchronous)."""
    import numpy as np
    model = build_forward_model(ctx, m, torch, gen)
    # every forward runs all 34 blocks: the caption cache (which would serve
    # the context refiner from the previous forward) is off
    model.set_caption_cache(False)
    for i, sc in enumerate(SCALES):
        model.set_lora_scale(i, sc)
    img, cap, grid = 4096, 256, 64
    # positions: image (cap + 1, row, col), caption (1 + i, 0, 0)
    pt = np.concatenate([np.full(img, cap + 1), 1 + np.arange(cap)]).astype(np.int32)
    ph = np.concatenate([np.arange(img) // grid, np.zeros(cap)]).astype(np.int32)
    pw = np.concatenate([np.arange(img) % grid, np.zeros(cap)]).astype(np.int32)
    lat = torch.randn((img, 64), generator=gen, device="cuda").to(
        torch.bfloat16).view(torch.int16)
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(
        torch.bfloat16).view(torch.int16)
    out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    for _ in range(warmup):
        model.forward(lat, capt, 2560, img, cap, cap, pt, ph, pw, 0.5, out)
    each = []
    for _ in range(steps):
        t0 = time.perf_counter()
        model.forward(lat, capt, 2560, img, cap, cap, pt, ph, pw, 0.5, out)
        each.append((time.perf_counter() - t0) * 1e3)
    flops = forward_flops(img, cap)
    return each, flops, model


def run_forward1024(ctx, m, torch, gen, steps):
    """The 1024^2 forward alone: ms per forward (host clock, after two untimed
    forwards), then the same forwards with the library's per-launch HIP events,
    summed per kernel family -- the reference's profile buckets
    (ming-dit.cc:1689-1717) -- as ms and TFLOP/s per forward."""
    each, flops, model = time_forward(ctx, m, torch, gen, steps, 2)
    img, cap, grid = 4096, 256, 64
    import numpy as np
    pt = np.concatenate([np.full(img, cap + 1), 1 + np.arange(cap)]).astype(np.int32)
    ph = np.concatenate([np.arange(img) // grid, np.zeros(cap)]).astype(np.int32)
    pw = np.concatenate([np.arange(img) % grid, np.zeros(cap)]).astype(np.int32)
    lat = torch.randn((img, 64), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
    ctx.set_profiling(True)
    ctx.profile_collect()
    for _ in range(steps):
        model.forward(lat, capt, 2560, img, cap, cap, pt, ph, pw, 0.5, out)
    prof = ctx.profile_collect()
    ctx.set_profiling(False)
    model.close()
    tot = sum(b["ms"] for b in prof.values())
    fams = {k: {"ms_per_forward": round(v["ms"] / steps, 3),
                "launches_per_forward": v["launches"] // steps,
                "share": round(v["ms"] / tot, 4),
                "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1) if v["flops"] else None,
                "gbps": round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1) if not v["flops"] else None}
            for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])}
    med = sorted(each)[len(each) // 2]
    return {"metric": "34-block w4g64 forward @1024^2", "value": round(med, 2), "unit": "ms",
            "higher_is_better": False, "ms_each": [round(t, 2) for t in each],
            "tflops": round(flops / (med * 1e-3) / 1e12, 2),
            "kernel_ms_per_forward": round(tot / steps, 3), "families": fams}


def time_forward_2048(model, torch, gen, steps):
    """configs[3] on an already-built model (the same 34 blocks and adapters
    as the 1024^2 forward): ms per 2048^2 forward after one untimed one."""
    img, cap, pos = layout_2048()
    lat = torch.randn((img, 64), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    capt = torch.randn((cap, 2560), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty((img, 64), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    model.forward(lat, capt, 2560, img, cap, cap, *pos, 0.5, out)
    each = []
    for _ in range(steps):
        t0 = time.perf_counter()
        model.forward(lat, capt, 2560, img, cap, cap, *pos, 0.5, out)
        each.append((time.perf_counter() - t0) * 1e3)
    return each, forward_flops(img, cap)


def time_norms(ctx, torch, gen, rounds=4):
    """The HBM-bound feeds at configs[2]'s shape (4352 rows, H 3840, 30 heads):
    RMSNorm [4352, 3840] out of place, and qk-norm + RoPE in place on the
    token-major [4352, 3*3840] qkv plane -- the DiT's interleaved-pair form,
    and the encoder's LlmOps form on the same plane (30 query then 30 key
    heads from column 0, both weights, rotate-half width 64). Each kernel walks a ring of
    buffers totalling more than the 256 MB Infinity Cache (MALL), so every
    launch reads its input from HBM, not from a cache the previous launch
    filled; the launches of a round are bracketed by two events on the
    context's stream. achieved = algorithmic bytes (activations read + written
    once, gains; the rotary tables excluded) / average launch time, against
    8 TB/s."""
    import numpy as np
    rows, H, NH = M_TOK, HID, HID // 128
    n_rms = 6                      # 6 x (33.4 MB in + 33.4 MB out) = 401 MB
    n_qk = 4                       # 4 x 100.3 MB qkv planes = 401 MB
    xs = [torch.randn((rows, H), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
          for _ in range(n_rms)]
    ys = [torch.empty_like(xs[0]) for _ in range(n_rms)]
    w = (1.0 + 0.1 * torch.randn((H,), generator=gen, device="cuda")).to(torch.bfloat16).view(torch.int16)
    qkvs = [torch.randn((rows, 3 * H), generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
            for _ in range(n_qk)]
    nq = (1.0 + 0.1 * torch.randn((128,), generator=gen, device="cuda")).to(torch.bfloat16).view(torch.int16)
    nk = (1.0 + 0.1 * torch.randn((128,), generator=gen, device="cuda")).to(torch.bfloat16).view(torch.int16)
    img, cap, grid = 4096, 256, 64
    pt = torch.from_numpy(np.concatenate([np.full(img, cap + 1), 1 + np.arange(cap)]).astype(np.int32)).cuda()
    ph = torch.from_numpy(np.concatenate([np.arange(img) // grid, np.zeros(cap)]).astype(np.int32)).cuda()
    pw = torch.from_numpy(np.concatenate([np.arange(img) % grid, np.zeros(cap)]).astype(np.int32)).cuda()
    cos_t = torch.empty((rows, 64), dtype=torch.float32, device="cuda")
    sin_t = torch.empty_like(cos_t)
    ctx.rope_table(pt, ph, pw, rows, cos_t, sin_t)
    cstream = torch.cuda.ExternalStream(ctx_stream(ctx))

    def run_rms(i):
        ctx.rmsnorm(xs[i % n_rms], w, ys[i % n_rms], rows, H)

    def run_qk(i):
        ctx.qk_norm_rope(qkvs[i % n_qk], 3 * H, 0, H, rows, NH, nq, nk, cos_t, sin_t)

    def run_llm_qk(i):
        ctx.llm_qk_norm_rope(qkvs[i % n_qk], nq, nk, cos_t, sin_t, rows, 3 * H, NH, NH, 64,
                             1e-6)

    out = {}
    for name, fn, nbuf, shape, nbytes, ring in (
            ("rmsnorm", run_rms, n_rms, [rows, H], 4.0 * rows * H + 2.0 * H,
             n_rms * 4 * rows * H),
            ("qk_norm_rope", run_qk, n_qk, [rows, 2 * H], 8.0 * rows * H + 512.0,
             n_qk * 6 * rows * H),
            ("llm_qk_norm_rope", run_llm_qk, n_qk, [rows, 2 * H], 8.0 * rows * H + 512.0,
             n_qk * 6 * rows * H)):
        for i in range(2 * nbuf):                 # warm: every buffer touched
            fn(i)
        ctx.synchronize()
        n = rounds * nbuf
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(cstream)
        for i in range(n):
            fn(i)
        e1.record(cstream)
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / n
        gbps = nbytes / (us * 1e-6) / 1e9
        out[name] = {"shape": shape, "launches": n, "ring_bytes": int(ring),
                     "avg_us": round(us, 2), "bytes_per_launch": round(nbytes),
                     "achieved_gbps": round(gbps, 1), "peak_gbps": PEAK_HBM_GBS,
                     "frac": round(gbps / PEAK_HBM_GBS, 4)}
    return out


def ctx_stream(ctx):
    """The context's HIP stream handle (an int)."""
    import ming_dit_amd as m
    return int(m.lib().ming_ctx_stream(ctx.h) or 0)


def host_cpu():
    """The host's CPU as the baseline ran on it: model, clock, counts."""
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "model": None, "mhz": None}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "model name" and info["model"] is None:
                    info["model"] = v.strip()
                elif k == "cpu MHz" and info["mhz"] is None:
                    info["mhz"] = float(v)
    except OSError:
        pass
    return info


TRAFFIC_MD = os.path.join(ROOT, "profiles", "qproj_w4_ffn_config2_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed PMC
    summary (FETCH_SIZE and WRITE_SIZE passes scaled by a known-size copy);
    None when absent."""
    try:
        with open(TRAFFIC_MD) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


TIMELINE_MD = os.path.join(ROOT, "profiles", "ffn_step_timeline_config2.md")


def steady_pair_launch_us():
    """The paired launch's duration in the event-free pass (its two kernels
    back to back), from the committed rocprofv3 kernel trace of this bench's
    default FFN command; None when absent."""
    try:
        with open(TIMELINE_MD) as f:
            for line in f:
                if line.startswith("steady_pair_launch_us:"):
                    return float(line.split(":")[1])
    except OSError:
        pass
    return None


def mfma_ceiling(torch, seconds=2.0, variants=("f16_random", "bf16_random", "f16_zero")):
    """The sustained MFMA rate of a kernel that does nothing else (see
    vpipe-ming-image_amd/calib/mfma_ceiling.hip): per variant, launches of
    ~25 ms back to back for about `seconds`, the median of the second half."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                   "vpipe-ming-image_amd", "libming_calib.so"))
    lib.ming_calib_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.Stream()
    out = torch.empty(cus * 256, dtype=torch.float32, device="cuda")
    iters = 50000
    flop = cus * 4 * iters * 16 * 32768.0
    res = {"metric": "mfma_ceiling", "unit": "TFLOP/s", "cus": cus, "blocks": cus,
           "iters_per_launch": iters, "flop_per_launch": flop,
           "peak_nominal_tflops": {"f16": 2516.6, "bf16": 2516.6}}
    for name, bf16, zero in (("f16_random", 0, 0), ("bf16_random", 1, 0), ("f16_zero", 0, 1)):
        if name not in variants:
            continue
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 6:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            rc = lib.ming_calib_mfma(bf16, cus, iters, zero, 12345 + len(times),
                                     out.data_ptr(), ctypes.c_void_p(stream.cuda_stream))
            assert rc == 0, rc
            e1.record(stream)
            e1.synchronize()
            times.append(e0.elapsed_time(e1))
        late = sorted(times[len(times) // 2:])
        ms = late[len(late) // 2]
        tf = flop / (ms * 1e-3) / 1e12
        res[name] = {"ms_per_launch": round(ms, 3), "tflops": round(tf, 1),
                     "launches": len(times),
                     # the clock at which 1024 FLOP/clk per SIMD gives this rate
                     "equiv_ghz": round(tf * 1e12 / (cus * 4 * 1024) / 1e9, 3)}
        assert torch.isfinite(out).all()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-forward", action="store_true",
                    help="skip the 34-block forwards (1024^2 and 2048^2)")
    ap.add_argument("--no-cfg", action="store_true",
                    help="skip configs[4] (the CFG x 2 w8 denoise at 2048^2)")
    ap.add_argument("--forward-steps", type=int, default=5)
    ap.add_argument("--workload", choices=("ffn", "forward1024", "forward2048", "cfg2048"),
                    default="ffn",
                    help="ffn: the headline line (configs[1], the forwards, configs[4]); "
                         "forward1024: the 1024^2 forward alone, with its kernel-family "
                         "breakdown; forward2048: configs[3]; cfg2048: configs[4]")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="measure the MFMA throughput this board sustains under its power "
                         "limit: back-to-back 32x32x16 f16/bf16 MFMAs on register operands, "
                         "the projection kernels' occupancy, random and zero operands")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB device-to-device three times (the "
                         "known-size kernel the HBM byte counters are scaled by)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path runs on ONE GPU (asked for {args.gpus}); "
              "token-row sharding across GPUs is a design note, not a build "
              "target here", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.mfma_ceiling:
        print(json.dumps(mfma_ceiling(torch)))
        return
    if args.copy_calibration:
        n = 256 * 1024 * 1024 // 4
        src = torch.randint(0, 1 << 30, (n,), dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("copy calibration: 268435456 bytes read and written per copy")
        return
    import ming_dit_amd as m

    torch.cuda.init()
    stream = torch.cuda.Stream()
    ctx = m.Ctx(0, stream.cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(2)
    if args.workload == "forward1024":
        res = run_forward1024(ctx, m, torch, gen, args.forward_steps)
        ctx.close()
        print(json.dumps(res))
        return
    if args.workload != "ffn":
        fn = run_forward2048 if args.workload == "forward2048" else run_cfg2048
        res = fn(ctx, m, torch, gen, args.forward_steps) if args.workload == "forward2048" \
            else fn(ctx, m, torch, gen)
        res.update({"n_gpus": 1, "data": "synthetic", "dtype": "w4/w8 g64 -> fp16 MFMA"})
        ctx.close()
        print(json.dumps(res))
        return
    (w1, w3, w2), hosts, x = build(ctx, m, torch, gen)
    M = M_TOK
    g = torch.empty((M, FFN), dtype=torch.int16, device="cuda")
    y = torch.empty((M, HID), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    def step():
        # gpu_ff as one call: lin(w1), lin(w3) with the SwiGLU fused into its
        # epilogue, lin(w2) -- the same bits as the four separate calls
        ctx.ffn(w1, w3, w2, x, y, M, SCALES, h=g)

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    ctx.reset_engagement()
    torch.cuda.synchronize()
    # the timed steps: nothing but the work (no per-launch events)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    e1.synchronize()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    eng = ctx.engagement()
    # the same steps again with the library's per-launch HIP events, for the
    # kernel breakdown and the roofline (events cost ~5% of step time, so
    # they stay out of the timed pass above)
    ctx.set_profiling(True)
    ctx.profile_collect()
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    prof = ctx.profile_collect()
    ctx.set_profiling(False)
    base, lora = ffn_flops(M)
    step_flops = base + lora
    assert eng["gemm_q4"] == 3 * args.steps and eng["lora_proj"] == 3 * args.steps, eng
    value = step_flops / (ms * 1e-3) / 1e12

    qname = max((k for k in prof if k.startswith("qproj")),
                key=lambda k: prof[k]["ms"])
    q = prof[qname]
    achieved = q["flops"] / (q["ms"] * 1e-3) / 1e12
    kernels = {k: {"launches": v["launches"],
                   "avg_us": round(1e3 * v["ms"] / v["launches"], 2),
                   "share": round(v["ms"] / sum(b["ms"] for b in prof.values()), 4)}
               for k, v in prof.items()}
    out = {
        "metric": "w4g64+8-LoRA proj TFLOP/s & MFMA util @4352 tok; "
                  "34-block fwd ms @1024²",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4g64 codes -> fp16 MFMA (base), bf16 MFMA (LoRA), f32 acc",
        "data": "synthetic",
        "config": {"workload": "configs[1]: one block's SwiGLU FFN, w4g64, "
                               "8 LoRA slots on w1/w3/w2, 4352 tokens",
                   "tokens": M, "hidden": HID, "ffn": FFN,
                   "lora_ranks": list(RANKS), "lora_scales": list(SCALES),
                   "step_gflop": round(step_flops / 1e9, 2),
                   "parallelism": "1 GPU"},
        "mfma_util": round(value / PEAK_TFLOPS, 4),
        "forward_ms_1024": None,
        "forward_tflops_1024": None,
        "roofline": {"bound": "mfma", "kernel": qname,
                     "achieved": round(achieved, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(),
                     "traffic_source": ("profiles/qproj_w4_ffn_config2_traffic.md (rocprofv3 "
                                        "FETCH_SIZE + WRITE_SIZE passes of this command, scaled "
                                        "by a 256 MiB copy)"),
                     "avg_launch_us": round(1e3 * q["ms"] / q["launches"], 2),
                     "flop_per_launch": round(q["flops"] / q["launches"])},
        "kernels": kernels,
    }
    steady = steady_pair_launch_us()
    if steady and qname.startswith("qproj_pair"):
        # the same kernel in the event-free pass that `value` is timed on,
        # where nothing between launches lets the clock recover (read from
        # the committed trace; the profiled pass above has ~10 us of idle
        # before every launch)
        fl = q["flops"] / q["launches"]
        out["roofline"]["frac_steady"] = round(fl / (steady * 1e-6) / 1e12 / PEAK_TFLOPS, 4)
        out["roofline"]["steady_launch_us"] = steady
        out["roofline"]["steady_source"] = ("profiles/ffn_step_timeline_config2.md (rocprofv3 "
                                            "kernel trace of the event-free pass)")
    for w in (w1, w3, w2):
        w.close()
    # the MFMA rate this board sustains on random fp16 operands under its
    # power limit (the projection's own MFMA type and occupancy), measured
    # here so the fraction below compares two numbers from one box
    ceil = mfma_ceiling(torch, seconds=1.0, variants=("f16_random",))["f16_random"]
    out["roofline"]["measured_ceiling"] = {
        "what": "back-to-back fp16 32x32x16 MFMAs on random register operands, one "
                "256-thread block per CU (bench.py --mfma-ceiling)",
        "tflops": ceil["tflops"], "equiv_ghz": ceil["equiv_ghz"],
        "frac": round(achieved / ceil["tflops"], 4)}
    out["hbm_kernels"] = time_norms(ctx, torch, gen)
    if not args.no_forward:
        # two untimed forwards (the first allocates the forward's workspaces,
        # ~110 ms); the timed ones are reported one by one, with their median
        # as the figure: an occasional forward on these boxes takes ~40 ms
        # longer, and the list shows when one did
        each, fflops, model = time_forward(ctx, m, torch, gen, args.forward_steps, 2)
        fms = sorted(each)[len(each) // 2]
        out["forward_ms_1024"] = round(fms, 2)
        out["forward_ms_mean"] = round(sum(each) / len(each), 2)
        out["forward_ms_each"] = [round(t, 2) for t in each]
        out["forward_tflops_1024"] = round(fflops / (fms * 1e-3) / 1e12, 2)
        out["forward_tflop"] = round(fflops / 1e12, 2)
        # the same model at 2048^2 (16384 image + 256 caption tokens)
        each2, fflops2 = time_forward_2048(model, torch, gen, 3)
        model.close()
        fms2 = sorted(each2)[len(each2) // 2]
        out["forward_ms_2048"] = round(fms2, 2)
        out["forward_ms_2048_each"] = [round(t, 2) for t in each2]
        out["forward_tflops_2048"] = round(fflops2 / (fms2 * 1e-3) / 1e12, 2)
    if not args.no_cfg:
        # CFG x 2, w8, eight r64 slots, 11 denoise steps at 2048^2
        cfg = run_cfg2048(ctx, m, torch, gen)
        out["cfg2048_tflops_sustained"] = cfg["value"]
        out["cfg2048_ms_per_forward_median"] = cfg["ms_per_forward_median"]
        out["cfg2048_ms_per_step_each"] = cfg["ms_per_step_each"]
        out["cfg2048_finite"] = cfg["finite"]
    if not args.no_cpu:
        import numpy as np
        xh = x.cpu().view(torch.int16).numpy().view(np.uint16)
        # every core of the process's affinity, up to the one-GPU box's CPU
        # share of 16
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        out["cpu_baseline"] = cpu_baseline(hosts, xh, args.cpu_seconds, threads)
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
