"""ctypes face of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker -- never by the product library.
bf16 values travel as numpy uint16 arrays (their bit patterns), exactly as
the reference's SharedBuffers hold them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    args = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = C.CDLL(_LIB_PATH)
    L.or_bf16_rne.argtypes = [C.c_float]
    L.or_bf16_rne.restype = C.c_uint16
    L.or_bf16_rne_nan.argtypes = [C.c_float]
    L.or_bf16_rne_nan.restype = C.c_uint16
    L.or_bf16_to_f32.argtypes = [C.c_uint16]
    L.or_bf16_to_f32.restype = C.c_float
    L.or_f32_to_bf16_n.argtypes = [_f32p, _u16p, C.c_size_t]
    L.or_bf16_to_f32_n.argtypes = [_u16p, _f32p, C.c_size_t]
    L.or_torch_randn.argtypes = [C.c_uint64, C.c_size_t, _f32p]
    L.or_torch_randn.restype = C.c_int
    for fn in (L.or_quant_w8_sym, L.or_quant_w4_affine):
        fn.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, _u32p, _u16p, _u16p]
        fn.restype = C.c_int
    L.or_get_code.argtypes = [_u32p, C.c_int, C.c_int]
    L.or_get_code.restype = C.c_uint32
    L.or_dequant.argtypes = [_u32p, _u16p, _u16p, C.c_int, C.c_int, C.c_int,
                             C.c_int, _f32p]
    L.or_dequant.restype = C.c_int
    vpp = C.POINTER(C.c_void_p)
    L.or_proj.argtypes = [_u16p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int,
                          C.c_int, _i32p, vpp, vpp, _f32p, _f32p, C.c_int,
                          C.c_int]
    L.or_proj.restype = C.c_int
    L.or_qproj_packed.argtypes = [_u16p, C.c_int, C.c_int, C.c_int, _u32p,
                                  _u16p, _u16p, C.c_int, C.c_int, C.c_int,
                                  C.c_int, _i32p, vpp, vpp, _f32p, _f32p,
                                  C.c_int, C.c_int]
    L.or_qproj_packed.restype = C.c_int
    L.or_rmsnorm.argtypes = [_u16p, C.c_int, _u16p, _u16p, C.c_int, C.c_int,
                             C.c_int, C.c_float]
    L.or_fold_gain.argtypes = [_u16p, _u16p, _u16p, C.c_int]
    L.or_rope_table.argtypes = [_i32p, _i32p, _i32p, C.c_int, _i32p, C.c_int,
                                C.c_double, _f32p, _f32p]
    L.or_rope_table.restype = C.c_int
    L.or_rope_apply.argtypes = [_u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_int, _f32p, _f32p, C.c_int]
    L.or_qk_norm_rope.argtypes = [_u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_int, _u16p, _u16p, _f32p,
                                  _f32p, C.c_int, C.c_float]
    # the weights and tables are optional (NULL): passed as raw addresses
    L.or_llm_qk_norm_rope.argtypes = [_u16p, C.c_int, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                      C.c_int, C.c_int, C.c_float]
    L.or_llm_qk_norm_rope.restype = C.c_int
    L.or_build_layout.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_void_p, C.c_void_p, C.c_void_p, _i32p]
    L.or_build_layout.restype = C.c_int
    L.or_schedule_sigmas.argtypes = [C.c_int, C.c_float, _f32p]
    L.or_schedule_sigmas.restype = C.c_int
    L.or_time_proj.argtypes = [C.c_float, C.c_float, C.c_int, _f32p]
    L.or_gated_residual.argtypes = [_u16p, C.c_int, _u16p, _u16p, C.c_int,
                                    C.c_int, C.c_int]
    L.or_swiglu.argtypes = [_u16p, _u16p, _u16p, C.c_size_t]
    L.or_bias_act.argtypes = [_u16p, C.c_int, _u16p, C.c_int, C.c_int,
                              C.c_int]
    L.or_ln_modulate.argtypes = [_u16p, C.c_int, _u16p, _u16p, C.c_int,
                                 C.c_int, C.c_int, C.c_float]
    L.or_attention.argtypes = [_u16p, C.c_int, _u16p, C.c_int, _u16p, C.c_int,
                               _u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                               C.c_float]
    _lib = L
    return L


# ---- bf16 ------------------------------------------------------------------
def f32_to_bf16(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().or_f32_to_bf16_n(a.reshape(-1), out.reshape(-1), a.size)
    return out


def bf16_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().or_bf16_to_f32_n(a.reshape(-1), out.reshape(-1), a.size)
    return out


def randn(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    if lib().or_torch_randn(seed, n, out) != 0:
        raise ValueError("torch randn needs n >= 16")
    return out


# ---- pack ----------------------------------------------------------------------
def quantize(w: np.ndarray, bits: int, group: int = 64):
    """(codes u32 [N, K*bits/32], scales bf16 [N, K/g], biases bf16 [N, K/g])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    codes = np.zeros((N, K * bits // 32), np.uint32)
    sc = np.zeros((N, K // group), np.uint16)
    bi = np.zeros((N, K // group), np.uint16)
    fn = lib().or_quant_w8_sym if bits == 8 else lib().or_quant_w4_affine
    if bits not in (4, 8) or fn(w, N, K, group, codes, sc, bi) != 0:
        raise ValueError("bad quantize arguments")
    return codes, sc, bi


def dequant(codes, scales, biases, bits: int, group: int = 64) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint32)
    N = codes.shape[0]
    K = codes.shape[1] * 32 // bits
    w = np.empty((N, K), np.float32)
    if lib().or_dequant(codes, np.ascontiguousarray(scales, np.uint16),
                        np.ascontiguousarray(biases, np.uint16), N, K, bits,
                        group, w) != 0:
        raise ValueError("bad dequant arguments")
    return w


def _lora_args(loras):
    """loras: list of (A bf16 [r,K], B bf16 [N,r], coef) or None per slot."""
    loras = list(loras or [])
    n = len(loras)
    ranks = np.zeros(max(n, 1), np.int32)
    aps = (C.c_void_p * max(n, 1))()
    bps = (C.c_void_p * max(n, 1))()
    coef = np.zeros(max(n, 1), np.float32)
    keep = []
    for i, l in enumerate(loras):
        if l is None:
            continue
        A, B, c = l
        A = np.ascontiguousarray(A, np.uint16)
        B = np.ascontiguousarray(B, np.uint16)
        keep += [A, B]
        ranks[i] = A.shape[0]
        aps[i] = A.ctypes.data
        bps[i] = B.ctypes.data
        coef[i] = c
    return n, ranks, aps, bps, coef, keep


def proj(x_bf16: np.ndarray, w: np.ndarray, loras=None,
         nthreads: int = 8) -> np.ndarray:
    """fp32 (f64-accumulated) y = x W^T + sum coef_i B_i (A_i x)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    w = np.ascontiguousarray(w, np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    n, ranks, aps, bps, coef, _keep = _lora_args(loras)
    rc = lib().or_proj(x, M, K, K, w, N, n, ranks, aps, bps, coef, y, N,
                       nthreads)
    if rc != 0:
        raise RuntimeError("or_proj failed")
    return y


def qproj_packed(x_bf16, codes, scales, biases, bits, loras=None,
                 nthreads: int = 8, group: int = 64) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, np.uint16)
    codes = np.ascontiguousarray(codes, np.uint32)
    M, K = x.shape
    N = codes.shape[0]
    y = np.empty((M, N), np.float32)
    n, ranks, aps, bps, coef, _keep = _lora_args(loras)
    rc = lib().or_qproj_packed(x, M, K, K, codes,
                               np.ascontiguousarray(scales, np.uint16),
                               np.ascontiguousarray(biases, np.uint16), bits,
                               group, N, n, ranks, aps, bps, coef, y, N,
                               nthreads)
    if rc != 0:
        raise RuntimeError("or_qproj_packed failed")
    return y


# ---- norms, rope ---------------------------------------------------------------
def rmsnorm(x_bf16, w_bf16, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, np.uint16)
    rows, D = x.shape
    y = np.empty_like(x)
    lib().or_rmsnorm(x, D, np.ascontiguousarray(w_bf16, np.uint16), y, D,
                     rows, D, eps)
    return y


def fold_gain(norm_w, scale) -> np.ndarray:
    nw = np.ascontiguousarray(norm_w, np.uint16)
    out = np.empty_like(nw)
    lib().or_fold_gain(nw, np.ascontiguousarray(scale, np.uint16), out,
                       nw.size)
    return out


def rope_table(pos_t, pos_h, pos_w, axes=(32, 48, 48), head_dim=128,
               theta=256.0):
    n = len(pos_t)
    c = np.empty((n, head_dim // 2), np.float32)
    s = np.empty((n, head_dim // 2), np.float32)
    rc = lib().or_rope_table(np.ascontiguousarray(pos_t, np.int32),
                             np.ascontiguousarray(pos_h, np.int32),
                             np.ascontiguousarray(pos_w, np.int32), n,
                             np.asarray(axes, np.int32), head_dim, theta, c,
                             s)
    if rc != 0:
        raise ValueError("rope table: axes do not cover head_dim")
    return c, s


def rope_apply(x_bf16, col0, n_heads, head_dim, cos_t, sin_t,
               table_row0=0) -> np.ndarray:
    x = np.array(x_bf16, np.uint16, copy=True, order="C")
    rows, ld = x.shape
    lib().or_rope_apply(x, ld, col0, rows, n_heads, head_dim,
                        np.ascontiguousarray(cos_t, np.float32),
                        np.ascontiguousarray(sin_t, np.float32), table_row0)
    return x


def qk_norm_rope(x_bf16, q_col, k_col, n_heads, head_dim, wq, wk, cos_t,
                 sin_t, table_row0=0, eps=1e-5) -> np.ndarray:
    x = np.array(x_bf16, np.uint16, copy=True, order="C")
    rows, ld = x.shape
    lib().or_qk_norm_rope(x, ld, q_col, k_col, rows, n_heads, head_dim,
                          np.ascontiguousarray(wq, np.uint16),
                          np.ascontiguousarray(wk, np.uint16),
                          np.ascontiguousarray(cos_t, np.float32),
                          np.ascontiguousarray(sin_t, np.float32), table_row0,
                          eps)
    return x


def llm_qk_norm_rope(qkv_bf16, q_w, k_w, cos_t, sin_t, n_q, n_k, rot_half,
                     eps=1e-5) -> np.ndarray:
    """LlmOps::qk_norm_rope (ming-ops.h:118-122): heads [0, n_q) queries from
    column 0, then n_k keys; norm only when both weights are given; rotate-half
    of width rot_half (0, 32, 64) by cos/sin [rows][rot_half]."""
    x = np.array(qkv_bf16, np.uint16, copy=True, order="C")
    rows, ld = x.shape
    norm = q_w is not None and k_w is not None
    qw = np.ascontiguousarray(q_w, np.uint16) if norm else None
    kw = np.ascontiguousarray(k_w, np.uint16) if norm else None
    c = np.ascontiguousarray(cos_t, np.float32) if rot_half else None
    s = np.ascontiguousarray(sin_t, np.float32) if rot_half else None
    if rot_half not in (0, 32, 64):
        raise ValueError("rot_half must be 0, 32 or 64")
    if n_q < 0 or n_k < 0 or (n_q + n_k) * 128 > ld:
        raise ValueError("heads past the row")
    if rot_half and (c.shape != (rows, rot_half) or s.shape != (rows, rot_half)):
        raise ValueError("tables must be [rows][rot_half]")

    def addr(a):
        return None if a is None else a.ctypes.data

    rc = lib().or_llm_qk_norm_rope(x, ld, addr(qw), addr(kw), addr(c), addr(s), rows,
                                   n_q, n_k, rot_half, eps)
    if rc != 0:
        raise ValueError("rot_half must be 0, 32 or 64")
    return x


# ---- layout, schedule, timestep ------------------------------------------------
def build_layout(grid_h, grid_w, query_rows, text_rows, axis0_len=20480):
    info = np.zeros(4, np.int32)
    if lib().or_build_layout(grid_h, grid_w, query_rows, text_rows, axis0_len,
                             None, None, None, info) != 0:
        return None
    n = int(info[3])
    pt = np.zeros(n, np.int32)
    ph = np.zeros(n, np.int32)
    pw = np.zeros(n, np.int32)
    lib().or_build_layout(grid_h, grid_w, query_rows, text_rows, axis0_len,
                          pt.ctypes.data, ph.ctypes.data, pw.ctypes.data,
                          info)
    return {"img_tokens": int(info[0]), "cap_len": int(info[1]),
            "cap_total": int(info[2]), "joint_len": int(info[3]),
            "pos_t": pt, "pos_h": ph, "pos_w": pw}


def schedule_sigmas(steps: int, shift: float) -> np.ndarray:
    out = np.zeros(steps + 1, np.float32)
    if lib().or_schedule_sigmas(steps, shift, out) != 0:
        raise ValueError("steps must be positive")
    return out


def time_proj(sigma: float, t_scale: float = 1000.0, D: int = 256):
    out = np.zeros(D, np.float32)
    lib().or_time_proj(sigma, t_scale, D, out)
    return out


def gated_residual(h_bf16, gate_bf16, sub_bf16) -> np.ndarray:
    h = np.array(h_bf16, np.uint16, copy=True, order="C")
    rows, N = h.shape
    sub = np.ascontiguousarray(sub_bf16, np.uint16)
    lib().or_gated_residual(h, N, np.ascontiguousarray(gate_bf16, np.uint16),
                            sub, sub.shape[1], rows, N)
    return h


def swiglu(g_bf16, u_bf16) -> np.ndarray:
    g = np.ascontiguousarray(g_bf16, np.uint16)
    out = np.empty_like(g)
    lib().or_swiglu(g.reshape(-1), np.ascontiguousarray(u_bf16,
                                                         np.uint16).reshape(-1),
                    out.reshape(-1), g.size)
    return out


def bias_act(y_bf16, b_bf16, silu=False) -> np.ndarray:
    y = np.array(y_bf16, np.uint16, copy=True, order="C")
    rows, N = y.shape
    lib().or_bias_act(y, N, np.ascontiguousarray(b_bf16, np.uint16), rows, N,
                      int(silu))
    return y


def ln_modulate(x_bf16, scale_bf16, eps=1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, np.uint16)
    rows, D = x.shape
    y = np.empty_like(x)
    lib().or_ln_modulate(x, D, np.ascontiguousarray(scale_bf16, np.uint16), y,
                         D, rows, D, eps)
    return y


def attention(q, k, v, n_heads, head_dim, scale=None) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint16)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    rows = q.shape[0]
    o = np.zeros((rows, n_heads * head_dim), np.uint16)
    if scale is None:
        scale = 1.0 / np.sqrt(head_dim)
    lib().or_attention(q, q.shape[1], k, k.shape[1], v, v.shape[1], o,
                       o.shape[1], rows, n_heads, head_dim, scale)
    return o


def rel_l2(a, b) -> float:
    """||a-b||_2 / ||b||_2 in f64 (ming-test.h:54-72)."""
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = float(np.sqrt(np.sum(b * b)))
    num = float(np.sqrt(np.sum((a - b) ** 2)))
    return num / den if den > 0 else num


# ---- block and model, composed from the pieces above ---------------------------
# The reference's run_block (ming-dit.cc:2065-2263), fill_mod (2266-2273), time
# MLP (2276-2281), embeddings (2283-2304) and final layer (2557-2563), with
# bf16 values at the same boundaries as the library: each projection output,
# norm output, modulation and residual is a bf16 plane.
def lin(x_bf16, w, loras=None, scales=None) -> np.ndarray:
    """One projection, rounded to bf16 once. w: {"codes","scales","biases",
    "bits"} (a pack) or {"w": bf16 [N,K]}; loras: per slot (A, B, fold) or
    None; scales: the 8 live strengths. A slot is live when bound and its
    strength is non-zero (lora_for_ + Stack::add, ming-dit.cc:3007-3022);
    its coefficient is fold * strength."""
    live = []
    if loras is not None and scales is not None:
        for i, l in enumerate(loras):
            if l is not None and float(scales[i]) != 0.0:
                A, B, fold = l
                live.append((A, B, np.float32(fold) * np.float32(scales[i])))
    x = np.ascontiguousarray(x_bf16, np.uint16)
    if "w" in w:
        y = proj(x, bf16_to_f32(w["w"]), live)
    else:
        y = qproj_packed(x, w["codes"], w["scales"], w["biases"], w["bits"],
                         live)
    return f32_to_bf16(y)


def residual_add(h_bf16, sub_bf16) -> np.ndarray:
    """h = bf16(h + sub), the f32 sum rounded once (ming_ops.metal resid)."""
    s = bf16_to_f32(h_bf16) + bf16_to_f32(sub_bf16)
    return f32_to_bf16(s.astype(np.float32))


def silu_bf16(x_bf16) -> np.ndarray:
    """bf16(silu(x)) through the bias+silu path with a zero bias."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    return bias_act(x.reshape(1, -1), np.zeros(x.size, np.uint16),
                    silu=True).reshape(x.shape)


def block_forward(x_bf16, blk, n_heads, cos_t, sin_t, temb=None, scales=None,
                  eps=1e-5) -> np.ndarray:
    """One block. blk: "q","k","v","o","w1","w3","w2" weights (see lin),
    "loras": {name: [8 x (A, B, fold) or None]}, gains "an1","an2","fn1",
    "fn2" [H], "nq","nk" [128], and "ada" + "ada_b" on modulated blocks."""
    x = np.array(x_bf16, np.uint16, copy=True, order="C")
    rows, H = x.shape
    L = blk.get("loras", {})

    def P(name, inp):
        return lin(inp, blk[name], L.get(name), scales)

    modulated = blk.get("ada") is not None
    g1, g3 = blk["an1"], blk["fn1"]
    if modulated:
        mods = bias_act(lin(np.asarray(temb, np.uint16).reshape(1, -1),
                            blk["ada"]), blk["ada_b"])[0]
        g1 = fold_gain(blk["an1"], mods[:H])
        g3 = fold_gain(blk["fn1"], mods[2 * H:3 * H])
    nrm = rmsnorm(x, g1, eps)
    qkv = np.concatenate([P("q", nrm), P("k", nrm), P("v", nrm)], axis=1)
    qkv = qk_norm_rope(qkv, 0, H, n_heads, 128, blk["nq"], blk["nk"], cos_t,
                       sin_t, 0, eps)
    ao = attention(qkv[:, :H], qkv[:, H:2 * H], qkv[:, 2 * H:], n_heads, 128)
    ob = rmsnorm(P("o", ao), blk["an2"], eps)
    if modulated:
        x = gated_residual(x, mods[H:2 * H], ob)
    else:
        x = residual_add(x, ob)
    nrm = rmsnorm(x, g3, eps)
    a = swiglu(P("w1", nrm), P("w3", nrm))
    ob = rmsnorm(P("w2", a), blk["fn2"], eps)
    if modulated:
        x = gated_residual(x, mods[3 * H:], ob)
    else:
        x = residual_add(x, ob)
    return x


def model_forward(m, latents, cap, img, cap_len, query_rows, pos_t, pos_h,
                  pos_w, sigma, scales=None) -> np.ndarray:
    """MingDit::forward. m: dims ("hidden","n_heads","n_refiner","cap_dim",
    "time_freq","t_scale","rope_theta","axes","eps"), "ctx_blocks" and
    "blocks" (block dicts), and the time / embedding / final-layer weights
    and biases. Returns the velocity [img][patch_dim] (bf16)."""
    H, NH, eps = m["hidden"], m["n_heads"], m.get("eps", 1e-5)
    Q, JT = query_rows, img + cap_len
    cos_t, sin_t = rope_table(pos_t, pos_h, pos_w, m["axes"], 128,
                              m["rope_theta"])
    tin = f32_to_bf16(time_proj(sigma, m["t_scale"], m["time_freq"]))
    te1 = bias_act(lin(tin.reshape(1, -1), m["time_1"]), m["time_1b"],
                   silu=True)
    temb = bias_act(lin(te1, m["time_2"]), m["time_2b"])[0]
    tsilu = silu_bf16(temb)
    joint = np.zeros((JT, H), np.uint16)
    joint[:img] = bias_act(lin(latents, m["x_in"]), m["x_in_b"])
    if Q > 0:
        capn = rmsnorm(np.ascontiguousarray(cap[:Q, :m["cap_dim"]]),
                       m["cap_norm"], eps)
        joint[img:img + Q] = bias_act(lin(capn, m["cap_in"]), m["cap_in_b"])
    joint[img + Q:] = cap[Q:cap_len, :H]
    for blk in m["ctx_blocks"]:
        joint[img:] = block_forward(joint[img:], blk, NH, cos_t[img:],
                                    sin_t[img:], None, scales, eps)
    for i, blk in enumerate(m["blocks"]):
        rows = img if i < m["n_refiner"] else JT
        joint[:rows] = block_forward(joint[:rows], blk, NH, cos_t[:rows],
                                     sin_t[:rows], temb, scales, eps)
    outmod = bias_act(lin(tsilu.reshape(1, -1), m["final_ada"]),
                      m["final_ada_b"])[0]
    nrm = ln_modulate(joint[:img], outmod)
    return bias_act(lin(nrm, m["final_lin"]), m["final_lin_b"])
