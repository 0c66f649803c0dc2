"""Python face of libming_dit_amd.so (the C-ABI in include/ming_dit_amd.h).

Thin ctypes plumbing for tests, bench.py and the graft entry: device
memory is whatever the caller owns (torch tensors here, passed by
data_ptr()). Every entry point raises MingError with the library's own
reason on a non-zero status. There is no fallback: if the library is not
built, importing it raises.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import sys
import weakref

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libming_dit_amd.so")
HEADER = os.path.join(os.path.dirname(_HERE), "include", "ming_dit_amd.h")
MAX_SLOTS = 8

_lib = None

# Every open handle, so that the ones still open when the interpreter exits
# are closed by an atexit hook -- before module teardown and before the HIP
# runtime's own exit handlers -- and never by a finalizer running during
# interpreter shutdown, when the runtime may already be gone.
_open = weakref.WeakSet()
_atexit_registered = False


def _track(obj):
    global _atexit_registered
    _open.add(obj)
    if not _atexit_registered:
        atexit.register(close_all)
        _atexit_registered = True


def close_all():
    """Closes every handle still open: models before the weights they borrow,
    weights before their contexts. Registered with atexit when the first
    handle opens; safe to call at any time."""
    objs = list(_open)
    for kind in (Model, QWeight, Pack, Ctx):
        for o in objs:
            if isinstance(o, kind):
                try:
                    o.close()
                except Exception:
                    pass


def _finalize(obj, _finalizing=sys.is_finalizing):
    """__del__ body: close, unless the interpreter is shutting down (then the
    atexit hook has closed what was open, and a late call into the HIP
    runtime could run after its teardown). What it calls is bound at
    definition: module globals read None during interpreter teardown."""
    if _finalizing():
        return
    try:
        obj.close()
    except Exception:
        pass


ERR_SHAPE, ERR_STATE, ERR_RANGE = 2, 6, 7
NOALLOC_SCRATCH_BYTES = 64 << 20


class MingError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Engagement(C.Structure):
    _fields_ = [("gemm_q4", C.c_int64), ("gemm_q8", C.c_int64),
                ("gemm_dense", C.c_int64), ("lora_proj", C.c_int64),
                ("lora_xa", C.c_int64), ("rmsnorm", C.c_int64),
                ("qk_norm_rope", C.c_int64), ("rope_table", C.c_int64),
                ("attention", C.c_int64), ("elementwise", C.c_int64),
                ("gemm_flops", C.c_uint64), ("gemm_fast", C.c_int64),
                ("cap_cache_hits", C.c_int64), ("gemv", C.c_int64),
                ("gemm_split", C.c_int64), ("range_faults", C.c_int64),
                ("gemm_paired", C.c_int64)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class ProfileBucket(C.Structure):
    _fields_ = [("name", C.c_char * 24), ("launches", C.c_int64),
                ("ms", C.c_double), ("flops", C.c_double),
                ("bytes", C.c_double)]


class BlockDesc(C.Structure):
    """ming_block_desc: borrowed weights (qweight handles) and bf16 gains."""
    _fields_ = [(n, C.c_void_p) for n in
                ("q", "k", "v", "o", "w1", "w3", "w2", "ada", "ada_b", "an1",
                 "an2", "fn1", "fn2", "nq", "nk")]


class BlockDims(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_heads", C.c_int), ("ffn", C.c_int),
                ("adaln_dim", C.c_int), ("eps", C.c_float)]


class ModelDesc(C.Structure):
    _fields_ = ([(n, C.c_int) for n in
                 ("hidden", "n_heads", "ffn", "n_layers", "n_refiner",
                  "adaln_dim", "time_freq", "time_mid", "patch_dim",
                  "cap_dim")]
                + [("eps", C.c_float), ("rope_theta", C.c_float),
                   ("t_scale", C.c_float), ("axes", C.c_int * 3),
                   ("axes_lens", C.c_int * 3),
                   ("ctx_blocks", C.POINTER(BlockDesc)),
                   ("blocks", C.POINTER(BlockDesc))]
                + [(n, C.c_void_p) for n in
                   ("time_1", "time_1b", "time_2", "time_2b", "x_in",
                    "x_in_b", "cap_norm", "cap_in", "cap_in_b", "final_ada",
                    "final_ada_b", "final_lin", "final_lin_b")])


class DitConfig(C.Structure):
    """ming_dit_config: transformer/config.json as the loader read it."""
    _fields_ = ([(n, C.c_int) for n in
                 ("dim", "n_layers", "n_refiner_layers", "n_heads",
                  "n_kv_heads", "in_channels", "patch", "f_patch",
                  "cap_feat_dim", "qk_norm")]
                + [("norm_eps", C.c_float), ("rope_theta", C.c_float),
                   ("t_scale", C.c_float), ("axes_dims", C.c_int * 3),
                   ("axes_lens", C.c_int * 3)]
                + [(n, C.c_int) for n in
                   ("zero_masked", "multi_frame_output", "ffn_inner",
                    "adaln_dim", "time_mid", "time_freq", "patch_dim")])

    def as_dict(self):
        out = {}
        for k, _ in self._fields_:
            v = getattr(self, k)
            out[k] = list(v) if isinstance(v, C.Array) else v
        return out


class LoraSpec(C.Structure):
    _fields_ = [("path", C.c_char_p), ("scale", C.c_float)]


class DenoiseArgs(C.Structure):
    _fields_ = [("cap", C.c_void_p), ("cap_stride", C.c_int64),
                ("cap_len", C.c_int), ("query_rows", C.c_int),
                ("pos_t", C.POINTER(C.c_int32)), ("pos_h", C.POINTER(C.c_int32)),
                ("pos_w", C.POINTER(C.c_int32)),
                ("cap_neg", C.c_void_p), ("neg_len", C.c_int),
                ("neg_query_rows", C.c_int),
                ("neg_pos_t", C.POINTER(C.c_int32)),
                ("neg_pos_h", C.POINTER(C.c_int32)),
                ("neg_pos_w", C.POINTER(C.c_int32)),
                ("img_tokens", C.c_int), ("steps", C.c_int), ("shift", C.c_float),
                ("guidance", C.c_float), ("cfg_truncation", C.c_double),
                ("cfg_normalization", C.c_double)]


LOG_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_char_p)
STEP_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int)
STOP_FN = C.CFUNCTYPE(C.c_int, C.c_void_p)
PROGRESS_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_int)
STOPPED = -1
LOG_WARN, LOG_INFO = 1, 2


def lib():
    """Load the built library (raises if it is not there)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    L = C.CDLL(LIB_PATH)
    vp, i32, i64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_float
    sig = {
        "ming_last_error": ([], C.c_char_p),
        "ming_abi_version": ([], i32),
        "ming_ctx_create": ([i32, vp, C.POINTER(vp)], i32),
        "ming_ctx_destroy": ([vp], i32),
        "ming_ctx_set_stream": ([vp, vp], i32),
        "ming_ctx_stream": ([vp], vp),
        "ming_ctx_synchronize": ([vp], i32),
        "ming_ctx_engagement": ([vp, C.POINTER(Engagement)], i32),
        "ming_ctx_reset_engagement": ([vp], i32),
        "ming_qweight_create": ([vp, i32, i32, i32, i32, vp, vp, vp, i32,
                                 C.POINTER(vp)], i32),
        "ming_qweight_create_dense": ([vp, i32, i32, vp, i32, C.POINTER(vp)],
                                      i32),
        "ming_qweight_concat": ([vp, i32, C.POINTER(vp), C.POINTER(vp)], i32),
        "ming_qweight_destroy": ([vp], i32),
        "ming_qweight_bits": ([vp], i32),
        "ming_qweight_shape": ([vp, C.POINTER(i32), C.POINTER(i32),
                                C.POINTER(i32)], i32),
        "ming_qweight_bind_lora": ([vp, i32, i32, i32, vp, vp, f32, i32], i32),
        "ming_qweight_unbind_lora": ([vp, i32, i32], i32),
        "ming_qweight_lora_rank": ([vp, i32, i32], i32),
        "ming_lin": ([vp, vp, vp, i64, vp, i64, i32, C.POINTER(f32)], i32),
        "ming_lin_bias": ([vp, vp, vp, i64, vp, i64, i32, C.POINTER(f32), vp], i32),
        "ming_lin_noalloc": ([vp, vp, vp, i64, vp, i64, i32, C.POINTER(f32)], i32),
        "ming_rmsnorm": ([vp, vp, i64, vp, vp, i64, i32, i32, f32], i32),
        "ming_rope_table": ([vp, vp, vp, vp, i32, C.POINTER(i32), i32,
                             C.c_double, vp, vp], i32),
        "ming_attention": ([vp, vp, i64, i32, i32, i32, vp, i64, i32, i32, i32,
                            f32], i32),
        "ming_qk_norm_rope": ([vp, vp, i64, i32, i32, i32, i32, i32, vp, vp,
                               vp, vp, f32], i32),
        "ming_llm_qk_norm_rope": ([vp, vp, vp, vp, vp, vp, i32, i64, i32, i32,
                                   i32, f32], i32),
        "ming_ctx_set_profiling": ([vp, i32], i32),
        "ming_ctx_set_route": ([vp, i32], i32),
        "ming_qweight_fast": ([vp], i32),
        "ming_ctx_profile_collect": ([vp, C.POINTER(ProfileBucket), i32,
                                      C.POINTER(i32)], i32),
        "ming_swiglu": ([vp, vp, i64, vp, i64, vp, i64, i32, i32], i32),
        "ming_gated_residual": ([vp, vp, i64, vp, vp, i64, i32, i32], i32),
        "ming_residual_add": ([vp, vp, i64, vp, i64, i32, i32], i32),
        "ming_modulate": ([vp, vp, i64, vp, vp, i64, i32, i32], i32),
        "ming_bias_act": ([vp, vp, i64, vp, i32, i32, i32], i32),
        "ming_silu": ([vp, vp, vp, i32], i32),
        "ming_ln_modulate": ([vp, vp, i64, vp, vp, i64, i32, i32, f32], i32),
        "ming_quantize_pack": ([vp, vp, i32, i32, i32, i32, vp, vp, vp], i32),
        "ming_lin_swiglu": ([vp, vp, vp, i64, vp, i64, vp, i64, i32,
                             C.POINTER(f32)], i32),
        "ming_ffn": ([vp, vp, vp, vp, vp, i64, vp, i64, i32, C.POINTER(f32),
                      vp, i64], i32),
        "ming_block_workspace_bytes": ([C.POINTER(BlockDims), i32], C.c_size_t),
        "ming_block_forward": ([vp, C.POINTER(BlockDesc), C.POINTER(BlockDims),
                                vp, i32, vp, vp, vp, C.POINTER(f32), vp,
                                C.c_size_t], i32),
        "ming_model_create": ([vp, C.POINTER(ModelDesc), C.POINTER(vp)], i32),
        "ming_model_destroy": ([vp], i32),
        "ming_model_set_lora_scale": ([vp, i32, f32], i32),
        "ming_model_lora_scale": ([vp, i32], f32),
        "ming_model_forward": ([vp, vp, vp, i64, i32, i32, i32,
                                C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                                C.POINTER(C.c_int32), f32, vp], i32),
        "ming_set_log_sink": ([LOG_FN, vp], None),
        "ming_model_set_stream_stop": ([vp, STOP_FN, vp], i32),
        "ming_model_set_block_progress": ([vp, PROGRESS_FN, vp], i32),
        "ming_model_set_caption_cache": ([vp, i32], i32),
        "ming_pack_open": ([C.c_char_p, C.POINTER(vp)], i32),
        "ming_pack_close": ([vp], i32),
        "ming_pack_config": ([vp, C.POINTER(DitConfig)], i32),
        "ming_pack_quant_bits": ([vp], i32),
        "ming_pack_group": ([vp], i32),
        "ming_pack_tensor_count": ([vp], i32),
        "ming_pack_tensor_name": ([vp, i32], C.c_char_p),
        "ming_pack_tensor_info": ([vp, C.c_char_p, C.c_char_p,
                                   C.POINTER(i64), C.POINTER(i32)], i32),
        "ming_pack_quantized_count": ([vp], i32),
        "ming_pack_write": ([C.c_char_p, C.c_char_p, i32, i32], i32),
        "ming_lora_module_capacity": ([C.POINTER(DitConfig)], i32),
        "ming_model_load": ([vp, C.c_char_p, C.POINTER(LoraSpec), i32,
                             C.POINTER(vp)], i32),
        "ming_model_bind_loras": ([vp, C.POINTER(LoraSpec), i32], i32),
        "ming_model_lora_modules": ([vp, i32], i32),
        "ming_model_lora_skipped": ([vp, i32], i32),
        "ming_model_lora_report": ([vp, i32], C.c_char_p),
        "ming_schedule_sigmas": ([i32, f32, C.POINTER(f32)], i32),
        "ming_model_denoise": ([vp, C.POINTER(DenoiseArgs), C.POINTER(f32), STEP_FN,
                                vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(rc: int):
    if rc != 0:
        msg = lib().ming_last_error().decode(errors="replace")
        raise MingError(rc, msg)


def _ptr(t) -> int:
    """Device (or host numpy) pointer of a tensor / array / int."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def _scales(scales):
    arr = (C.c_float * MAX_SLOTS)()
    if scales is not None:
        for i, s in enumerate(list(scales)[:MAX_SLOTS]):
            arr[i] = float(s)
    return arr


class Ctx:
    """A device + stream context (ming_ctx)."""

    def __init__(self, device: int = 0, stream: int | None = None):
        h = C.c_void_p()
        _check(lib().ming_ctx_create(device, stream, C.byref(h)))
        self.h = h
        self._weights = weakref.WeakSet()
        _track(self)

    def close(self):
        """Destroys the context's live weights first (the C-ABI refuses a
        context that still has weights)."""
        if self.h:
            for w in list(self._weights):
                w.close()
            _check(lib().ming_ctx_destroy(self.h))
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)

    def set_stream(self, stream: int | None):
        _check(lib().ming_ctx_set_stream(self.h, stream))

    def synchronize(self):
        _check(lib().ming_ctx_synchronize(self.h))

    def engagement(self) -> dict:
        e = Engagement()
        _check(lib().ming_ctx_engagement(self.h, C.byref(e)))
        return e.as_dict()

    def reset_engagement(self):
        _check(lib().ming_ctx_reset_engagement(self.h))

    def set_route(self, route: str = "auto"):
        """'auto' (fast route when the weight allows it), 'general' (the general
        kernel) or 'wide' (bf16 activations and bf16-pair weights: no fp16
        range limit)."""
        _check(lib().ming_ctx_set_route(self.h, {"auto": 0, "general": 1, "wide": 2}[route]))

    def set_profiling(self, on: bool = True):
        _check(lib().ming_ctx_set_profiling(self.h, int(on)))

    def profile_collect(self) -> dict:
        """{bucket: {launches, ms, flops, bytes}} since the last collect."""
        arr = (ProfileBucket * 32)()
        n = C.c_int()
        _check(lib().ming_ctx_profile_collect(self.h, arr, 32, C.byref(n)))
        return {arr[i].name.decode(): {"launches": arr[i].launches,
                                       "ms": arr[i].ms,
                                       "flops": arr[i].flops,
                                       "bytes": arr[i].bytes}
                for i in range(n.value)}

    # ---- ops ----
    def lin(self, qw: "QWeight", x, y, M: int, scales=None, ldx=None,
            ldy=None):
        ldx = qw.K if ldx is None else ldx
        ldy = qw.N if ldy is None else ldy
        _check(lib().ming_lin(self.h, qw.h, _ptr(x), ldx, _ptr(y), ldy, M,
                              _scales(scales)))

    def lin_bias(self, qw: "QWeight", x, y, M: int, bias, scales=None, ldx=None,
                 ldy=None):
        """ming_lin_bias (LlmOps::linear with a bias): the bias added before
        the output's one rounding; dense weights."""
        ldx = qw.K if ldx is None else ldx
        ldy = qw.N if ldy is None else ldy
        _check(lib().ming_lin_bias(self.h, qw.h, _ptr(x), ldx, _ptr(y), ldy, M,
                                   _scales(scales), _ptr(bias)))

    def lin_noalloc(self, qw: "QWeight", x, y, M: int, scales=None, ldx=None,
                    ldy=None):
        """ming_lin with the device's static scratch: allocates nothing."""
        ldx = qw.K if ldx is None else ldx
        ldy = qw.N if ldy is None else ldy
        _check(lib().ming_lin_noalloc(self.h, qw.h, _ptr(x), ldx, _ptr(y), ldy, M,
                                      _scales(scales)))

    def lin_swiglu(self, w: "QWeight", x, g, out, M: int, scales=None,
                   ldx=None, ldg=None, ldo=None):
        """out = bf16(silu(g) * lin(x, w)); g may be out."""
        _check(lib().ming_lin_swiglu(self.h, w.h, _ptr(x), ldx or w.K, _ptr(g),
                                     ldg or w.N, _ptr(out), ldo or w.N, M,
                                     _scales(scales)))

    def ffn(self, w1: "QWeight", w3: "QWeight", w2: "QWeight", x, y, M: int,
            scales=None, h=None, ldx=None, ldy=None, ldh=None):
        """gpu_ff: y = lin(swiglu(lin(x, w1), lin(x, w3)), w2); h is the
        [M][ffn] intermediate plane (allocated here when None)."""
        if h is None:
            import torch
            h = torch.empty((M, w1.N), dtype=torch.int16, device="cuda")
        _check(lib().ming_ffn(self.h, w1.h, w3.h, w2.h, _ptr(x), ldx or w1.K,
                              _ptr(y), ldy or w2.N, M, _scales(scales), _ptr(h),
                              ldh or w1.N))
        return h

    def rmsnorm(self, x, w, y, rows: int, D: int, eps: float = 1e-5,
                ldx=None, ldy=None):
        _check(lib().ming_rmsnorm(self.h, _ptr(x), D if ldx is None else ldx,
                                  _ptr(w), _ptr(y), D if ldy is None else ldy,
                                  rows, D, eps))

    def rope_table(self, pos_t, pos_h, pos_w, n: int, cos_out, sin_out,
                   axes=(32, 48, 48), head_dim: int = 128,
                   theta: float = 256.0):
        ax = (C.c_int * 3)(*axes)
        _check(lib().ming_rope_table(self.h, _ptr(pos_t), _ptr(pos_h),
                                     _ptr(pos_w), n, ax, head_dim, theta,
                                     _ptr(cos_out), _ptr(sin_out)))

    def qk_norm_rope(self, x, ld: int, q_col: int, k_col: int, rows: int,
                     n_heads: int, wq, wk, cos_t, sin_t, eps: float = 1e-5,
                     head_dim: int = 128):
        _check(lib().ming_qk_norm_rope(self.h, _ptr(x), ld, q_col, k_col, rows,
                                       n_heads, head_dim, _ptr(wq), _ptr(wk),
                                       _ptr(cos_t), _ptr(sin_t), eps))

    def llm_qk_norm_rope(self, qkv, q_w, k_w, cos_t, sin_t, rows: int,
                         row_stride: int, n_q: int, n_k: int, rot_half: int,
                         eps: float):
        """LlmOps::qk_norm_rope (ming-ops.h:118-122), its argument order:
        q_w / k_w None for no norm, cos_t / sin_t None when rot_half is 0."""
        def opt(t):
            return None if t is None else _ptr(t)
        _check(lib().ming_llm_qk_norm_rope(self.h, _ptr(qkv), opt(q_w), opt(k_w),
                                           opt(cos_t), opt(sin_t), rows, row_stride,
                                           n_q, n_k, rot_half, eps))

    def attention(self, qkv, ld: int, q_col: int, k_col: int, v_col: int,
                  out, ldo: int, rows: int, n_heads: int, scale=None,
                  head_dim: int = 128):
        if scale is None:
            scale = 1.0 / head_dim ** 0.5
        _check(lib().ming_attention(self.h, _ptr(qkv), ld, q_col, k_col, v_col,
                                    _ptr(out), ldo, rows, n_heads, head_dim,
                                    float(scale)))

    def block_forward(self, desc: "BlockDesc", dims: "BlockDims", x, rows: int,
                      cos_t, sin_t, temb=None, scales=None, ws=None):
        """ming_block_forward in place on x [rows][H]; ws (a device tensor
        of at least block_workspace_bytes) is allocated here when None."""
        need = self.block_workspace_bytes(dims, rows)
        if ws is None:
            import torch
            ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        sc = _scales(scales) if scales is not None else None
        _check(lib().ming_block_forward(self.h, C.byref(desc), C.byref(dims),
                                        _ptr(x), rows, _ptr(cos_t), _ptr(sin_t),
                                        _ptr(temb), sc, _ptr(ws), need))
        return ws

    @staticmethod
    def block_workspace_bytes(dims: "BlockDims", rows: int) -> int:
        return int(lib().ming_block_workspace_bytes(C.byref(dims), rows))

    def swiglu(self, g, u, out, rows: int, n: int, ldg=None, ldu=None,
               ldo=None):
        _check(lib().ming_swiglu(self.h, _ptr(g), ldg or n, _ptr(u), ldu or n,
                                 _ptr(out), ldo or n, rows, n))

    def gated_residual(self, h, gate, sub, rows: int, n: int, ldh=None,
                       lds=None):
        _check(lib().ming_gated_residual(self.h, _ptr(h), ldh or n, _ptr(gate),
                                         _ptr(sub), lds or n, rows, n))

    def residual_add(self, h, sub, rows: int, n: int, ldh=None, lds=None):
        _check(lib().ming_residual_add(self.h, _ptr(h), ldh or n, _ptr(sub),
                                       lds or n, rows, n))

    def modulate(self, x, scale, y, rows: int, n: int, ldx=None, ldy=None):
        _check(lib().ming_modulate(self.h, _ptr(x), ldx or n, _ptr(scale),
                                   _ptr(y), ldy or n, rows, n))

    def bias_act(self, y, bias, rows: int, n: int, silu: bool = False,
                 ldy=None):
        _check(lib().ming_bias_act(self.h, _ptr(y), ldy or n, _ptr(bias), rows,
                                   n, int(silu)))

    def silu(self, x, y, n: int):
        _check(lib().ming_silu(self.h, _ptr(x), _ptr(y), n))

    def ln_modulate(self, x, scale, y, rows: int, D: int, eps: float = 1e-6,
                    ldx=None, ldy=None):
        _check(lib().ming_ln_modulate(self.h, _ptr(x), ldx or D, _ptr(scale),
                                      _ptr(y), ldy or D, rows, D, eps))

    def quantize_pack(self, w_f32, N: int, K: int, bits: int, codes, scales,
                      biases, group: int = 64):
        _check(lib().ming_quantize_pack(self.h, _ptr(w_f32), N, K, bits, group,
                                        _ptr(codes), _ptr(scales),
                                        _ptr(biases)))


class QWeight:
    """A resident projection weight (ming_qweight)."""

    def __init__(self, ctx: Ctx, h):
        self.ctx = ctx
        self.h = h
        ctx._weights.add(self)
        _track(self)
        N, K, S = C.c_int(), C.c_int(), C.c_int()
        _check(lib().ming_qweight_shape(h, C.byref(N), C.byref(K),
                                        C.byref(S)))
        self.N, self.K, self.n_segments = N.value, K.value, S.value
        self.bits = lib().ming_qweight_bits(h)
        self.fast = bool(lib().ming_qweight_fast(h))

    @classmethod
    def quantized(cls, ctx: Ctx, codes, scales, biases, bits: int,
                  group: int = 64, on_device: bool = False):
        N = int(codes.shape[0])
        K = int(codes.shape[1]) * 32 // bits
        h = C.c_void_p()
        _check(lib().ming_qweight_create(ctx.h, N, K, bits, group,
                                         _ptr(codes), _ptr(scales),
                                         _ptr(biases), int(on_device),
                                         C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def dense(cls, ctx: Ctx, w, on_device: bool = False):
        N, K = int(w.shape[0]), int(w.shape[1])
        h = C.c_void_p()
        _check(lib().ming_qweight_create_dense(ctx.h, N, K, _ptr(w),
                                               int(on_device), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def concat(cls, ctx: Ctx, parts):
        arr = (C.c_void_p * len(parts))(*[p.h.value for p in parts])
        h = C.c_void_p()
        _check(lib().ming_qweight_concat(ctx.h, len(parts), arr, C.byref(h)))
        return cls(ctx, h)

    def bind_lora(self, slot: int, A, B, fold: float = 1.0, segment: int = 0,
                  on_device: bool = False):
        rank = int(A.shape[0])
        _check(lib().ming_qweight_bind_lora(self.h, segment, slot, rank,
                                            _ptr(A), _ptr(B), fold,
                                            int(on_device)))

    def unbind_lora(self, slot: int, segment: int = 0):
        _check(lib().ming_qweight_unbind_lora(self.h, segment, slot))

    def lora_rank(self, slot: int, segment: int = 0) -> int:
        return lib().ming_qweight_lora_rank(self.h, segment, slot)

    def close(self):
        if self.h:
            lib().ming_qweight_destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def _h(obj) -> int | None:
    """Handle (QWeight) or device pointer (tensor) or None, as an int."""
    if obj is None:
        return None
    if isinstance(obj, QWeight):
        return obj.h.value
    return _ptr(obj)


def block_desc(**parts) -> BlockDesc:
    """BlockDesc from QWeights (q, k, v, o, w1, w3, w2, ada) and bf16 device
    tensors (ada_b, an1, an2, fn1, fn2, nq, nk)."""
    d = BlockDesc()
    for name, _ in BlockDesc._fields_:
        setattr(d, name, _h(parts.get(name)))
    d._keep = dict(parts)      # the handles stay valid while the desc lives
    return d


_log_keep = None


def schedule_sigmas(steps: int, shift: float):
    import numpy as np
    out = np.zeros(steps + 1, np.float32)
    _check(lib().ming_schedule_sigmas(int(steps), float(shift),
                                      out.ctypes.data_as(C.POINTER(C.c_float))))
    return out


def set_log_sink(fn=None):
    """Route the library's session log to fn(level, message) (None: drop)."""
    global _log_keep
    if fn is None:
        _log_keep = None
        lib().ming_set_log_sink(LOG_FN(), None)
        return
    cb = LOG_FN(lambda _u, level, msg: fn(int(level),
                                           msg.decode(errors="replace")))
    _log_keep = cb
    lib().ming_set_log_sink(cb, None)


def _specs(loras):
    """[(path or None, scale), ...] -> (LoraSpec array, n, keep)."""
    loras = list(loras or [])
    arr = (LoraSpec * max(len(loras), 1))()
    keep = []
    for i, (path, scale) in enumerate(loras):
        b = os.fsencode(path) if path else None
        keep.append(b)
        arr[i].path = b
        arr[i].scale = float(scale)
    return arr, len(loras), keep


class Pack:
    """A transformer directory opened by ming_pack_open (config + tensors)."""

    def __init__(self, transformer_dir: str):
        h = C.c_void_p()
        _check(lib().ming_pack_open(os.fsencode(transformer_dir), C.byref(h)))
        self.h = h
        _track(self)

    def config(self) -> dict:
        c = DitConfig()
        _check(lib().ming_pack_config(self.h, C.byref(c)))
        return c.as_dict()

    def config_struct(self) -> DitConfig:
        c = DitConfig()
        _check(lib().ming_pack_config(self.h, C.byref(c)))
        return c

    @property
    def quant_bits(self) -> int:
        return int(lib().ming_pack_quant_bits(self.h))

    @property
    def group(self) -> int:
        return int(lib().ming_pack_group(self.h))

    def names(self) -> list:
        n = lib().ming_pack_tensor_count(self.h)
        return [lib().ming_pack_tensor_name(self.h, i).decode() for i in range(n)]

    def info(self, name: str):
        dt = C.create_string_buffer(8)
        shape = (C.c_int64 * 8)()
        nd = C.c_int()
        _check(lib().ming_pack_tensor_info(self.h, name.encode(), dt, shape,
                                           C.byref(nd)))
        return dt.value.decode(), tuple(shape[i] for i in range(nd.value))

    def quantized_count(self) -> int:
        return int(lib().ming_pack_quantized_count(self.h))

    def close(self):
        if self.h:
            lib().ming_pack_close(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def pack_write(src_dir: str, dst_dir: str, bits: int, threads: int = 0):
    _check(lib().ming_pack_write(os.fsencode(src_dir), os.fsencode(dst_dir),
                                 int(bits), int(threads)))


def lora_module_capacity(cfg: DitConfig) -> int:
    return int(lib().ming_lora_module_capacity(C.byref(cfg)))


class Model:
    """ming_model. Made over borrowed weights (the caller keeps every QWeight
    and tensor in `desc` alive for the model's lifetime; held here too), or
    loaded from a transformer directory with Model.load (the model owns what
    it loaded)."""

    def __init__(self, ctx: Ctx, desc: ModelDesc | None, ctx_blocks=(),
                 blocks=(), keep=(), _handle=None):
        self.ctx = ctx
        self._cbs = {}
        self._keep = list(keep)
        if _handle is not None:
            self.desc = None
            self.h = _handle
        else:
            self._cb = (BlockDesc * max(len(ctx_blocks), 1))(*ctx_blocks)
            self._mb = (BlockDesc * max(len(blocks), 1))(*blocks)
            desc.ctx_blocks = C.cast(self._cb, C.POINTER(BlockDesc))
            desc.blocks = C.cast(self._mb, C.POINTER(BlockDesc))
            self.desc = desc
            h = C.c_void_p()
            _check(lib().ming_model_create(ctx.h, C.byref(desc), C.byref(h)))
            self.h = h
        ctx._weights.add(self)
        _track(self)

    @classmethod
    def load(cls, ctx: Ctx, transformer_dir: str, loras=None) -> "Model":
        arr, n, keep = _specs(loras)
        h = C.c_void_p()
        _check(lib().ming_model_load(ctx.h, os.fsencode(transformer_dir), arr,
                                     n, C.byref(h)))
        return cls(ctx, None, _handle=h)

    def bind_loras(self, loras):
        arr, n, keep = _specs(loras)
        _check(lib().ming_model_bind_loras(self.h, arr, n))

    def lora_modules(self, slot: int) -> int:
        return int(lib().ming_model_lora_modules(self.h, slot))

    def lora_skipped(self, slot: int) -> int:
        return int(lib().ming_model_lora_skipped(self.h, slot))

    def lora_report(self, slot: int) -> str:
        return lib().ming_model_lora_report(self.h, slot).decode(errors="replace")

    def set_lora_scale(self, slot: int, s: float):
        _check(lib().ming_model_set_lora_scale(self.h, slot, float(s)))

    def lora_scale(self, slot: int) -> float:
        return float(lib().ming_model_lora_scale(self.h, slot))

    def set_stream_stop(self, fn=None):
        """fn() -> bool, polled before every block (None clears it)."""
        cb = STOP_FN(lambda _u: 1 if fn() else 0) if fn else STOP_FN()
        self._cbs["stop"] = cb
        _check(lib().ming_model_set_stream_stop(self.h, cb, None))

    def set_block_progress(self, fn=None):
        """fn(done, total) once per block, in order (None clears it)."""
        cb = (PROGRESS_FN(lambda _u, d, t: fn(int(d), int(t))) if fn
              else PROGRESS_FN())
        self._cbs["progress"] = cb
        _check(lib().ming_model_set_block_progress(self.h, cb, None))

    def set_caption_cache(self, on: bool):
        _check(lib().ming_model_set_caption_cache(self.h, int(bool(on))))

    def denoise(self, latents, cap, cap_stride: int, cap_len: int,
                query_rows: int, pos, img_tokens: int, steps: int,
                shift: float = 6.0, guidance: float = 1.0,
                cfg_truncation: float = 1.0, cfg_normalization: float = 0.0,
                cap_neg=None, neg_len: int = 0, neg_query_rows: int = 0,
                neg_pos=None, progress=None) -> bool:
        """The generator's Euler loop; latents: host f32 [img][patch_dim],
        updated in place. pos / neg_pos: (pos_t, pos_h, pos_w). True when
        every step ran, False when stopped."""
        import numpy as np
        assert latents.dtype == np.float32 and latents.flags.c_contiguous
        keep = [np.ascontiguousarray(p, np.int32) for p in pos]
        a = DenoiseArgs()
        a.cap, a.cap_stride, a.cap_len, a.query_rows = _ptr(cap), cap_stride, cap_len, query_rows
        a.pos_t, a.pos_h, a.pos_w = [k.ctypes.data_as(C.POINTER(C.c_int32)) for k in keep]
        if cap_neg is not None:
            nk = [np.ascontiguousarray(p, np.int32) for p in neg_pos]
            keep += nk
            a.cap_neg, a.neg_len, a.neg_query_rows = _ptr(cap_neg), neg_len, neg_query_rows
            a.neg_pos_t, a.neg_pos_h, a.neg_pos_w = [
                k.ctypes.data_as(C.POINTER(C.c_int32)) for k in nk]
        a.img_tokens, a.steps, a.shift, a.guidance = img_tokens, steps, shift, guidance
        a.cfg_truncation, a.cfg_normalization = cfg_truncation, cfg_normalization
        cb = (STEP_FN(lambda _u, i, n: 1 if progress(int(i), int(n)) else 0)
              if progress else STEP_FN())
        rc = lib().ming_model_denoise(self.h, C.byref(a),
                                      latents.ctypes.data_as(C.POINTER(C.c_float)),
                                      cb, None)
        if rc == STOPPED:
            return False
        _check(rc)
        return True

    def forward(self, latents, cap, cap_stride: int, img_tokens: int,
                cap_len: int, query_rows: int, pos_t, pos_h, pos_w,
                sigma: float, out) -> bool:
        """True when the forward ran, False on a cooperative stop."""
        import numpy as np
        arrs = [np.ascontiguousarray(a, np.int32) for a in (pos_t, pos_h, pos_w)]
        ptrs = [a.ctypes.data_as(C.POINTER(C.c_int32)) for a in arrs]
        rc = lib().ming_model_forward(self.h, _ptr(latents), _ptr(cap),
                                      cap_stride, img_tokens, cap_len,
                                      query_rows, *ptrs, float(sigma),
                                      _ptr(out))
        if rc == STOPPED:
            return False
        _check(rc)
        return True

    def close(self):
        if self.h:
            lib().ming_model_destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self)


def header_symbols(path: str = HEADER):
    """Every function the public header declares."""
    import re
    txt = open(path).read()
    return sorted(set(re.findall(r"\b(ming_[a-z0-9_]+)\s*\(", txt)))
