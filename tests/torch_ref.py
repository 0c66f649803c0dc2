"""A torch restatement of one DiT block and the whole forward -- TEST
INFRASTRUCTURE ONLY, the fp32 reference for the full-size configs.

The CPU oracle (oracle/oracle.c) is f64 and scalar: it finishes the reduced
width tests in seconds but not a 4352-row block or a 16640-token forward
(~344 TFLOP). This module computes the same functions with torch matmuls on
whatever device its tensors live on (the GPU for the full-size tests, the CPU
for its own validation), in one of two modes:

  * "f32": every intermediate stays fp32 -- the reference's f32 compute that
    its real-size test holds a forward against (ming-dit-test.cc:2107-2131);
  * "bf16": each value is rounded to bf16 where the library and the oracle
    round it (each projection, norm, modulation and residual output) -- the
    analogue of the reference's own bf16 run, whose distance from f32 sets
    the bar (twice it, floored at kSmallTol = 0.035, ming-dit-test.cc:815,
    2131).

It is pinned against the oracle at reduced width (tests/test_torch_ref.py):
the bf16 mode reproduces oracle.block_forward / oracle.model_forward to within
f32-vs-f64 accumulation, and the f32 mode stays within the rounding floor of
it. Weights come in the pack layout (LSB-first codes, bf16 scales and biases
per 64 columns: load_qw_, ming-dit.cc:802-831) and are dequantized here in
fp32. Inputs may be numpy bit patterns (uint16/uint32) or torch tensors.
"""
from __future__ import annotations

import numpy as np
import torch

# fp32 means fp32: no reduced-precision (xf32) matmuls in the reference
torch.backends.cuda.matmul.allow_tf32 = False
torch.set_float32_matmul_precision("highest")


def _tensor(a, dev, dtype):
    """numpy (bit patterns) or torch -> a torch tensor of `dtype` bits on dev."""
    if isinstance(a, np.ndarray):
        a = np.ascontiguousarray(a)
        a = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else
                             a.view(np.int32) if a.dtype == np.uint32 else a)
    return a.to(dev).view(dtype)


def bf(a, dev) -> torch.Tensor:
    """bf16 bit patterns -> their fp32 values."""
    return _tensor(a, dev, torch.int16).view(torch.bfloat16).float()


def dequant(codes, scales, biases, bits: int, dev) -> torch.Tensor:
    """w = scale * q + bias per 64-column group, q the unsigned LSB-first code
    (ming-dit.cc:802-831; the MLX affine convention), fp32 [N, K]."""
    c = _tensor(codes, dev, torch.int32)
    N, W = c.shape
    per = 32 // bits
    shifts = torch.arange(per, device=dev, dtype=torch.int32) * bits
    q = ((c[:, :, None] >> shifts) & ((1 << bits) - 1)).reshape(N, W * per).float()
    s = bf(scales, dev).repeat_interleave(64, dim=1)
    b = bf(biases, dev).repeat_interleave(64, dim=1)
    return torch.addcmul(b, q, s)


class Ref:
    """The reference computations in one mode ("f32" or "bf16") on `dev`."""

    def __init__(self, mode: str, dev):
        assert mode in ("f32", "bf16")
        self.mode, self.dev = mode, dev
        self._w = {}

    def r(self, t):
        return t.to(torch.bfloat16).float() if self.mode == "bf16" else t

    def weight(self, w):
        """w: {"codes","scales","biases","bits"} or {"w"} (dense bf16)."""
        key = id(w)
        if key not in self._w:
            if "w" in w:
                self._w[key] = bf(w["w"], self.dev)
            else:
                self._w[key] = dequant(w["codes"], w["scales"], w["biases"], w["bits"],
                                       self.dev)
        return self._w[key]

    def drop_weights(self):
        self._w.clear()

    # lin() = lin_base + lora::Applier (ming-dit.cc:1763-1771): y = x W^T +
    # sum over live slots of coef * (x A^T) B^T, coef = fold * strength, a slot
    # live when bound and its strength is non-zero (ming-dit.cc:3007-3022)
    def lin(self, x, w, loras=None, scales=None):
        W = self.weight(w)
        y = x @ W.t()
        if loras is not None and scales is not None:
            for i, l in enumerate(loras):
                if l is None or float(scales[i]) == 0.0:
                    continue
                A, B, fold = l
                coef = float(np.float32(fold) * np.float32(scales[i]))
                y = y + coef * ((x @ bf(A, self.dev).t()) @ bf(B, self.dev).t())
        return self.r(y)

    def rms(self, x, w, eps):
        """rms_norm_fast (ming-dit.cc:1780-1787): x * rsqrt(mean x^2 + eps) * w."""
        inv = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
        return self.r(x * inv * w)

    def rope(self, x, cos_t, sin_t):
        """Interleaved pairs (x[2k], x[2k+1]) rotated by the row's angle k
        (ming-dit.cc:1885-1895); x [rows, heads, 128], tables [rows, 64]."""
        x0, x1 = x[..., 0::2], x[..., 1::2]
        c, s = cos_t[:, None, :], sin_t[:, None, :]
        return self.r(torch.stack((x0 * c - x1 * s, x0 * s + x1 * c), -1).flatten(-2))

    def attention(self, q, k, v, n_heads, scale):
        """Dense, bidirectional, maskless softmax(q k^T * scale) v per head
        (ming-dit.cc:1905-2039), fp32 throughout, one head at a time."""
        rows = q.shape[0]
        out = torch.empty_like(q)
        for h in range(n_heads):
            sl = slice(128 * h, 128 * (h + 1))
            s = (q[:, sl] @ k[:, sl].t()) * scale
            p = torch.softmax(s, dim=-1)
            out[:, sl] = p @ v[:, sl]
            del s, p
        return self.r(out.reshape(rows, -1))

    def block(self, x, blk, n_heads, cos_t, sin_t, temb=None, scales=None, eps=1e-5):
        """run_block (ming-dit.cc:2065-2263) with fill_mod's folded gains
        (2266-2273): blk as oracle.block_forward takes it."""
        dev = self.dev
        rows, H = x.shape
        L = blk.get("loras", {})

        def P(name, inp):
            return self.lin(inp, blk[name], L.get(name), scales)

        g1, g3 = bf(blk["an1"], dev), bf(blk["fn1"], dev)
        mods = None
        if blk.get("ada") is not None:
            mods = self.r(self.lin(temb.reshape(1, -1), blk["ada"])[0] + bf(blk["ada_b"], dev))
            g1 = self.r(g1 * (1.0 + mods[:H]))
            g3 = self.r(g3 * (1.0 + mods[2 * H:3 * H]))
        nrm = self.rms(x, g1, eps)
        q, k, v = P("q", nrm), P("k", nrm), P("v", nrm)
        nq, nk = bf(blk["nq"], dev), bf(blk["nk"], dev)
        q = self.rope(self.rms(q.reshape(rows, n_heads, 128), nq, eps), cos_t, sin_t)
        k = self.rope(self.rms(k.reshape(rows, n_heads, 128), nk, eps), cos_t, sin_t)
        ao = self.attention(q.reshape(rows, -1), k.reshape(rows, -1), v, n_heads,
                            1.0 / np.sqrt(128.0))
        del q, k, v
        ob = self.rms(P("o", ao), bf(blk["an2"], dev), eps)
        x = self._residual(x, ob, None if mods is None else mods[H:2 * H])
        nrm = self.rms(x, g3, eps)
        g = P("w1", nrm)
        a = self.r(torch.nn.functional.silu(g) * P("w3", nrm))
        del g
        ob = self.rms(P("w2", a), bf(blk["fn2"], dev), eps)
        return self._residual(x, ob, None if mods is None else mods[3 * H:])

    def _residual(self, x, sub, gate):
        """h + tanh(gate) * sub on modulated blocks, h + sub on the context
        refiner's (ming_ops.metal:43-74)."""
        if gate is None:
            return self.r(x + sub)
        return self.r(x + torch.tanh(gate) * sub)

    def forward(self, m, latents, cap, img, cap_len, query_rows, cos_t, sin_t, sigma,
                scales=None, time_in=None):
        """MingDit::forward (ming-dit.cc:1490-2563), m as oracle.model_forward
        takes it; latents [img][patch_dim] and cap [cap_len][>= cap_dim, H]
        bf16; cos_t / sin_t the rotary tables of the joint sequence (f32
        [JT][64]); time_in the time_proj vector (f32 [time_freq]). Returns the
        velocity [img][patch_dim] (fp32 values; bf16-exact in "bf16")."""
        dev = self.dev
        H, NH, eps = m["hidden"], m["n_heads"], m.get("eps", 1e-5)
        Q, JT = query_rows, img + cap_len
        cos_t = torch.as_tensor(cos_t).to(dev)
        sin_t = torch.as_tensor(sin_t).to(dev)
        tin = torch.as_tensor(time_in).to(dev).float()
        tin = tin.to(torch.bfloat16).float()    # the timestep vector enters as bf16
        te1 = torch.nn.functional.silu(self.r(self.lin(tin[None], m["time_1"])
                                              + bf(m["time_1b"], dev)))
        te1 = self.r(te1)
        temb = self.r(self.lin(te1, m["time_2"]) + bf(m["time_2b"], dev))[0]
        tsilu = self.r(torch.nn.functional.silu(temb))
        cap_v = bf(cap, dev)
        joint = torch.zeros((JT, H), device=dev)
        joint[:img] = self.r(self.lin(bf(latents, dev), m["x_in"]) + bf(m["x_in_b"], dev))
        if Q > 0:
            capn = self.rms(cap_v[:Q, :m["cap_dim"]], bf(m["cap_norm"], dev), eps)
            joint[img:img + Q] = self.r(self.lin(capn, m["cap_in"]) + bf(m["cap_in_b"], dev))
        if Q < cap_len:
            joint[img + Q:] = cap_v[Q:cap_len, :H]
        for blk in m["ctx_blocks"]:
            joint[img:] = self.block(joint[img:], blk, NH, cos_t[img:], sin_t[img:], None,
                                     scales, eps)
            self.drop_weights()
        for i, blk in enumerate(m["blocks"]):
            rows = img if i < m["n_refiner"] else JT
            joint[:rows] = self.block(joint[:rows], blk, NH, cos_t[:rows], sin_t[:rows],
                                      temb, scales, eps)
            self.drop_weights()
        outmod = self.r(self.lin(tsilu[None], m["final_ada"])[0] + bf(m["final_ada_b"], dev))
        x = joint[:img]
        ln = self.r(torch.nn.functional.layer_norm(x, (H,), eps=1e-6))
        nrm = self.r(ln * (1.0 + outmod))
        return self.r(self.lin(nrm, m["final_lin"]) + bf(m["final_lin_b"], dev))


def rel_l2(a, b) -> float:
    """||a - b|| / ||b|| in float64 (ming-test.h:54-72)."""
    a = torch.as_tensor(a).double().reshape(-1)
    b = torch.as_tensor(b).double().reshape(-1)
    return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))
