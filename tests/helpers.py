"""Shared helpers for the tests: seeded inputs (BASELINE recipes), host <->
device moves of bf16 bit patterns, and the projection problem builder."""
from __future__ import annotations

import numpy as np

import oracle as orc

# BASELINE config 2's adapter set.
CFG2_RANKS = (4, 8, 16, 16, 32, 32, 64, 128)
CFG2_SCALES = (1.0, 0.5, 0.0, -0.3, 0.8, 0.0, 1.2, 0.25)
# BASELINE config 5's set: eight rank-64 slots, strengths uniform in [-1, 1.5]
# (the draw the bench's CFG run uses).
CFG5_RANKS = (64,) * 8
CFG5_SCALES = tuple(float(v) for v in np.random.default_rng(5).uniform(-1.0, 1.5, 8))


def randn(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """TorchCpuRandn draw (ming-torch-randn.h) reshaped, times std."""
    n = int(np.prod(shape))
    v = orc.randn(seed, max(n, 16))[:n]
    return (v * np.float32(std)).astype(np.float32).reshape(shape)


def bf16(a) -> np.ndarray:
    return orc.f32_to_bf16(a)


def f32(a) -> np.ndarray:
    return orc.bf16_to_f32(a)


def make_weight(seed: int, N: int, K: int, bits: int, std: float = 0.02):
    """(pack, dequantized f32) for bits 4/8; dense bf16 for bits 16."""
    w = randn(seed, (N, K), std)
    if bits == 16:
        wb = bf16(w)
        return {"w": wb}, f32(wb)
    codes, sc, bi = orc.quantize(w, bits)
    return {"codes": codes, "scales": sc, "biases": bi}, orc.dequant(
        codes, sc, bi, bits)


def make_lora(seed: int, N: int, K: int, rank: int):
    """A ~ N(0, 1/sqrt(K)) [rank, K], B ~ N(0, 0.01) [N, rank], bf16."""
    A = bf16(randn(seed, (rank, K), 1.0 / np.sqrt(K)))
    B = bf16(randn(seed + 1, (N, rank), 0.01))
    return A, B


# ---- device moves (torch owns the memory) ------------------------------------
def to_dev(a: np.ndarray):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def from_dev(t) -> np.ndarray:
    import torch
    t = t.detach().cpu()
    if t.dtype in (torch.int16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def empty_bf16(*shape):
    import torch
    return torch.empty(shape, dtype=torch.int16, device="cuda")


def sync():
    import torch
    torch.cuda.synchronize()


# ---- blocks and models (small dims for the oracle, GPU objects beside) ----------
BLOCK_PROJS = ("q", "k", "v", "o", "w1", "w3", "w2")


def block_proj_shapes(H, F):
    return {"q": (H, H), "k": (H, H), "v": (H, H), "o": (H, H),
            "w1": (F, H), "w3": (F, H), "w2": (H, F)}


def build_block(ctx, seed, H, F, adaln, bits=4, modulated=True,
                slots=((0, 4, 1.0), (3, 16, 0.5))):
    """A random block as (oracle dict, gpu dict, BlockDesc). Weights ~ N(0, .02)
    quantized by the oracle's packer (bits 4 / 8) or dense bf16 (bits 16);
    gains ~ 1 + N(0, .1); adaLN bias ~ N(0, .1); LoRA (slot, rank, fold) bound on all seven projections. Every
    tensor has a fixed seed of its own, so the same seed with other slots
    gives the same base block. With ctx None only the oracle dict is made
    (gp and the desc are None)."""
    gpu = ctx is not None
    if gpu:
        import ming_dit_amd as m
    ob = {"loras": {}}
    gp = {}
    for i, (name, (N, K)) in enumerate(block_proj_shapes(H, F).items()):
        pack, _ = make_weight(seed + 100 * i, N, K, bits)
        ob[name] = dict(pack, bits=bits)
        qw = None
        if gpu:
            qw = m.QWeight.dense(ctx, pack["w"]) if bits == 16 else m.QWeight.quantized(
                ctx, pack["codes"], pack["scales"], pack["biases"], bits)
        lor = [None] * 8
        for slot, rank, fold in slots:
            A, B = make_lora(seed + 100 * i + 10 + 2 * slot, N, K, rank)
            if gpu:
                qw.bind_lora(slot, A, B, fold)
            lor[slot] = (A, B, fold)
        ob["loras"][name] = lor
        gp[name] = qw
    if modulated:
        pack, _ = make_weight(seed + 1000, 4 * H, adaln, bits)
        ob["ada"] = dict(pack, bits=bits)
        if gpu:
            gp["ada"] = m.QWeight.dense(ctx, pack["w"]) if bits == 16 else m.QWeight.quantized(
                ctx, pack["codes"], pack["scales"], pack["biases"], bits)
        ob["ada_b"] = bf16(randn(seed + 1001, (4 * H,), 0.1))
        if gpu:
            gp["ada_b"] = to_dev(ob["ada_b"])
    for j, (g, n) in enumerate((("an1", H), ("an2", H), ("fn1", H),
                                ("fn2", H), ("nq", 128), ("nk", 128))):
        ob[g] = bf16(1.0 + randn(seed + 1002 + j, (n,), 0.1))
        if gpu:
            gp[g] = to_dev(ob[g])
    if not gpu:
        return ob, None, None
    return ob, gp, m.block_desc(**gp)


def grid_positions(rows, width=16, t=257):
    """Image-like rotary positions (t, row, col) for `rows` tokens."""
    i = np.arange(rows, dtype=np.int32)
    return (np.full(rows, t, np.int32), i // width, i % width)


def build_model(ctx, seed, H=256, NH=2, F=512, n_layers=2, n_refiner=1,
                adaln=64, time_freq=64, time_mid=128, patch_dim=64,
                cap_dim=128, bits=4, slots=((0, 4, 1.0), (3, 16, 0.5))):
    """A random model: (oracle dict for oracle.model_forward, Model). The
    non-block weights are dense bf16, as the reference leaves them
    (MingQuantFamily excludes the embedders and the final layer). With ctx
    None only the oracle dict is made (the Model is None)."""
    gpu = ctx is not None
    if gpu:
        import ming_dit_amd as m
    mo = {"hidden": H, "n_heads": NH, "n_refiner": n_refiner,
          "cap_dim": cap_dim, "time_freq": time_freq, "t_scale": 1000.0,
          "rope_theta": 256.0, "axes": (32, 48, 48), "eps": 1e-5}
    keep = []
    mo["ctx_blocks"], cb = [], []
    for i in range(n_refiner):
        ob, gp, d = build_block(ctx, seed + 10000 * (i + 1), H, F, adaln, bits,
                                False, slots)
        mo["ctx_blocks"].append(ob)
        cb.append(d)
        keep.append(gp)
    mo["blocks"], mb = [], []
    for i in range(n_refiner + n_layers):
        ob, gp, d = build_block(ctx, seed + 10000 * (i + 11), H, F, adaln, bits,
                                True, slots)
        mo["blocks"].append(ob)
        mb.append(d)
        keep.append(gp)
    dev = {}
    for j, (name, N, K) in enumerate((("time_1", time_mid, time_freq),
                                      ("time_2", adaln, time_mid),
                                      ("x_in", H, patch_dim),
                                      ("cap_in", H, cap_dim),
                                      ("final_ada", H, adaln),
                                      ("final_lin", patch_dim, H))):
        pack, _ = make_weight(seed + 500 + 2 * j, N, K, 16, std=1.0 / np.sqrt(K))
        mo[name] = pack
        b = bf16(randn(seed + 501 + 2 * j, (N,), 0.05))
        mo[name + "b" if name.startswith("time") else name + "_b"] = b
        if gpu:
            dev[name] = m.QWeight.dense(ctx, pack["w"])
            dev[name + "b" if name.startswith("time") else name + "_b"] = to_dev(b)
    mo["cap_norm"] = bf16(1.0 + randn(seed + 600, (cap_dim,), 0.1))
    if not gpu:
        return mo, None
    dev["cap_norm"] = to_dev(mo["cap_norm"])
    d = m.ModelDesc()
    d.hidden, d.n_heads, d.ffn, d.n_layers, d.n_refiner = H, NH, F, n_layers, n_refiner
    d.adaln_dim, d.time_freq, d.time_mid = adaln, time_freq, time_mid
    d.patch_dim, d.cap_dim = patch_dim, cap_dim
    d.eps, d.rope_theta, d.t_scale = 1e-5, 256.0, 1000.0
    d.axes[:] = [32, 48, 48]
    d.axes_lens[:] = [4096, 512, 512]
    for name, obj in dev.items():
        setattr(d, name, m._h(obj))
    model = m.Model(ctx, d, cb, mb, keep=keep + [dev, cb, mb])
    return mo, model
