"""Shared helpers for the tests: seeded inputs (BASELINE recipes), host <->
device moves of bf16 bit patterns, and the projection problem builder."""
from __future__ import annotations

import numpy as np

import oracle as orc

# BASELINE config 2's adapter set.
CFG2_RANKS = (4, 8, 16, 16, 32, 32, 64, 128)
CFG2_SCALES = (1.0, 0.5, 0.0, -0.3, 0.8, 0.0, 1.2, 0.25)


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
