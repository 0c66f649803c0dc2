// Block and model drivers over the library's entry points: the reference's
// run_block (ming-dit.cc:2065-2263), fill_mod (2266-2273), the timestep MLP
// (2276-2281), the embeddings (2283-2304) and the block sequence and final
// layer of MingDit::forward (2366-2563). Host code only: every kernel runs
// through ming_lin / ming_rmsnorm / ming_attention / ..., on the context's
// stream, in the reference's order.
//
// Layout choices that differ from the reference (same arithmetic):
//   * q, k and v land side by side in ONE token-major [rows][3H] plane, so
//     qk-norm + RoPE run in place on it and attention reads the heads at a
//     column offset -- the reference's head-major transposes of q, k and the
//     attention output (2083-2092) do not exist here;
//   * the adaLN scale is always folded into the pre-norm gains (the
//     reference's _fold_mod path, 1602-1606): nw = norm_w * (1 + scale).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "model.h"
#include "rt.h"

namespace {

using ming::rt_fail;
using ming::rt_ok;

#define RC(call)                      \
  do {                                \
    const int rc_ = (call);           \
    if (rc_ != MING_OK) return rc_;   \
  } while (0)

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct BlockWs {
  uint16_t *nrm, *qkv, *ob, *ffg, *mods, *nw1, *nw3;
  float* tg;  // tanh of the two residual gates, f32 [2H]
};

size_t block_ws_layout(const ming_block_dims& d, int rows, char* base, BlockWs* w) {
  const size_t H = (size_t)d.hidden, F = (size_t)d.ffn, R = (size_t)rows;
  const size_t sz[7] = {R * H * 2, R * 3 * H * 2, R * H * 2, R * F * 2,
                        4 * H * 2, H * 2,         H * 2};
  uint16_t** dst[7] = {&w->nrm, &w->qkv, &w->ob, &w->ffg, &w->mods, &w->nw1, &w->nw3};
  size_t off = 0;
  for (int i = 0; i < 7; ++i) {
    if (base) *dst[i] = reinterpret_cast<uint16_t*>(base + off);
    off += align256(sz[i]);
  }
  if (base) w->tg = reinterpret_cast<float*>(base + off);
  off += align256(2 * H * 4);
  return off;
}

bool shape_is(const ming_qweight* q, int N, int K) {
  int n = 0, k = 0, s = 0;
  return q && ming_qweight_shape(q, &n, &k, &s) == MING_OK && n == N && k == K;
}

int check_dims(const ming_block_dims* d) {
  if (!d) return rt_fail(MING_ERR_ARG, "block dims: null");
  if (d->n_heads <= 0 || d->hidden != d->n_heads * 128 || d->ffn <= 0 ||
      d->ffn % 64 != 0 || d->adaln_dim <= 0 || d->adaln_dim % 64 != 0 ||
      !(d->eps > 0.0f))
    return rt_fail(MING_ERR_SHAPE,
                   "block dims: need hidden = 128 * n_heads, ffn and adaln_dim "
                   "multiples of 64, eps > 0");
  return MING_OK;
}

int check_block(const ming_block_desc* b, const ming_block_dims& d, bool modulated,
                const char* who) {
  const int H = d.hidden, F = d.ffn;
  const std::string w(who);
  if (!b) return rt_fail(MING_ERR_ARG, w + ": null block");
  if (!shape_is(b->q, H, H) || !shape_is(b->k, H, H) || !shape_is(b->v, H, H) ||
      !shape_is(b->o, H, H))
    return rt_fail(MING_ERR_SHAPE, w + ": q/k/v/o must be [H][H]");
  if (!shape_is(b->w1, F, H) || !shape_is(b->w3, F, H) || !shape_is(b->w2, H, F))
    return rt_fail(MING_ERR_SHAPE, w + ": w1/w3 must be [ffn][H] and w2 [H][ffn]");
  if (!b->an1 || !b->an2 || !b->fn1 || !b->fn2 || !b->nq || !b->nk)
    return rt_fail(MING_ERR_ARG, w + ": a norm gain is missing");
  if (modulated) {
    if (!shape_is(b->ada, 4 * H, d.adaln_dim) || !b->ada_b)
      return rt_fail(MING_ERR_SHAPE, w + ": adaLN must be [4H][adaln_dim] with a bias");
  } else if (b->ada || b->ada_b) {
    return rt_fail(MING_ERR_ARG, w + ": a context-refiner block carries no adaLN");
  }
  return MING_OK;
}

// A modulated block's adaLN results, made ahead of the block.
struct Premod {
  uint16_t *mods, *nw1, *nw3;
  float* tg;
};

// run_block (ming-dit.cc:2065-2263) with fill_mod folded in; pm: the
// block's modulation already computed (rt_modulation_batch), else it is
// computed here. prenormed: the previous block's last pass already wrote
// this block's attention pre-norm (w.nrm and the context's fp16 copy);
// next_g1: the next block's attention pre-norm weight over the same rows,
// applied by this block's last pass (then the next block runs prenormed).
int block_forward(ming_ctx* c, const ming_block_desc* b, const ming_block_dims& d,
                  uint16_t* x, int rows, const float* cos_t, const float* sin_t,
                  const uint16_t* temb, const float* scales, const BlockWs& w,
                  const Premod* pm = nullptr, bool prenormed = false,
                  const uint16_t* next_g1 = nullptr) {
  const int H = d.hidden, F = d.ffn, NH = d.n_heads;
  const bool modulated = b->ada != nullptr;
  const float eps = d.eps;
  // The fp16 copies this block writes (the pre-norms', attention's O, the
  // SwiGLU's h) feed only its projections. Over dense projections (bf16
  // activations) they are never read, so a value they cannot hold raises
  // no range fault.
  struct CopiesUnread {
    ming_ctx* c;
    bool was;
    ~CopiesUnread() { ming::rt_set_copies_unread(c, was); }
  };
  bool dense = true;
  for (const ming_qweight* q : {b->q, b->k, b->v, b->o, b->w1, b->w3, b->w2})
    dense = dense && ming_qweight_bits(q) == 16;
  const CopiesUnread unread{c, ming::rt_set_copies_unread(c, dense)};
  const uint16_t* g1 = b->an1;
  const uint16_t* g3 = b->fn1;
  const float* tg = nullptr;
  if (modulated && pm) {
    g1 = pm->nw1;
    g3 = pm->nw3;
    tg = pm->tg;
  } else if (modulated) {
    // mods = ada(temb) + ada_b = (scale_msa | gate_msa | scale_mlp | gate_mlp)
    RC(ming_lin(c, b->ada, temb, d.adaln_dim, w.mods, 4 * H, 1, nullptr));
    // + bias, the two gain folds and the tanh of the two gates, one launch
    RC(ming::rt_adaln_glue(c, w.mods, H, b->ada_b, b->an1, b->fn1, w.nw1, w.nw3, w.tg));
    g1 = w.nw1;
    g3 = w.nw3;
    tg = w.tg;
  }
  // ---- attention half ----
  // the norm also writes the fp16 copy q, k and v read (one conversion, not three)
  if (!prenormed) RC(ming::rt_rmsnorm_f16(c, x, H, g1, w.nrm, H, rows, H, eps));
  {
    const ming_qweight* qkv[3] = {b->q, b->k, b->v};
    uint16_t* out[3] = {w.qkv, w.qkv + H, w.qkv + 2 * H};
    RC(ming::rt_lin3_xh(c, qkv, w.nrm, H, out, 3 * H, rows, scales));
  }
  // qk-norm + RoPE: k in one pass, q inside the attention kernel. The
  // attention output reuses the normed-input plane (its q/k/v are done);
  // its fp16 copy is the o-projection's input
  RC(ming::rt_attention_qknorm_xh(c, w.qkv, 3 * H, 0, H, 2 * H, w.nrm, H, rows, NH,
                                  1.0f / std::sqrt(128.0f), b->nq, b->nk, cos_t, sin_t, eps));
  RC(ming::rt_lin_xh(c, b->o, w.nrm, H, w.ob, H, rows, scales));
  // post-norm and the (gated) residual, then the feed-forward half's pre-norm
  // (and its fp16 copy) of the new stream rows, in one pass
  RC(ming::rt_norm_residual_norm(c, x, H, w.ob, H, b->an2, tg, g3, w.nrm, H, rows, H, eps));
  // ---- feed-forward half (gpu_ff, 2151-2162; SwiGLU fused into w3) ----
  RC(ming::rt_ffn_xh(c, b->w1, b->w3, b->w2, w.nrm, H, w.ob, H, rows, scales, w.ffg, F));
  if (next_g1)
    RC(ming::rt_norm_residual_norm(c, x, H, w.ob, H, b->fn2, tg ? tg + H : nullptr, next_g1,
                                   w.nrm, H, rows, H, eps));
  else
    RC(ming::rt_norm_residual(c, x, H, w.ob, H, b->fn2, tg ? tg + H : nullptr, rows, H, eps));
  return MING_OK;
}

// Round-to-nearest-even f32 -> bf16, NaN -> 0x7fc0 (ming-dit.cc:173-181).
uint16_t host_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

}  // namespace


namespace {

// A modulated block's adaLN results: mods [4H], nw1 [H], nw3 [H] (bf16), tg
// [2H] (f32), each 256-byte aligned.
size_t premod_bytes(size_t H) {
  return align256(8 * H) + 2 * align256(2 * H) + align256(8 * H);
}

Premod premod_of(void* base, size_t H, int i) {
  char* p = static_cast<char*>(base) + (size_t)i * premod_bytes(H);
  Premod r;
  r.mods = reinterpret_cast<uint16_t*>(p);
  r.nw1 = reinterpret_cast<uint16_t*>(p + align256(8 * H));
  r.nw3 = reinterpret_cast<uint16_t*>(p + align256(8 * H) + align256(2 * H));
  r.tg = reinterpret_cast<float*>(p + align256(8 * H) + 2 * align256(2 * H));
  return r;
}

// One allocation for every per-forward plane of a joint length JT and Q query rows.
int ensure_model_ws(ming_model* m, int JT, int Q) {
  if (JT <= m->ws_rows && Q <= m->ws_q) return MING_OK;
  const ming_model_desc& d = m->d;
  const size_t H = (size_t)d.hidden;
  const size_t NM = (size_t)(d.n_refiner + d.n_layers);
  const size_t sz[11] = {(size_t)JT * H * 2,         (size_t)std::max(Q, 1) * d.cap_dim * 2,
                         (size_t)d.time_freq * 2,    (size_t)d.time_mid * 2,
                         (size_t)d.adaln_dim * 2,    (size_t)d.adaln_dim * 2,
                         H * 2,                      (size_t)JT * 64 * 4,
                         (size_t)JT * 64 * 4,        (size_t)JT * 3 * 4,
                         NM * premod_bytes(H)};
  size_t total = 0;
  for (size_t s : sz) total += align256(s);
  ming_block_dims bd{d.hidden, d.n_heads, d.ffn, d.adaln_dim, d.eps};
  const size_t blk = ming_block_workspace_bytes(&bd, JT);
  (void)hipStreamSynchronize((hipStream_t)ming_ctx_stream(m->ctx));
  if (m->ws) (void)hipFree(m->ws);
  m->ws = nullptr;
  m->ws_bytes = 0;
  m->ws_rows = m->ws_q = -1;
  if (hipMalloc(&m->ws, total + blk) != hipSuccess)
    return rt_fail(MING_ERR_ALLOC, "ming_model_forward: workspace allocation failed");
  m->ws_bytes = total + blk;
  char* p = static_cast<char*>(m->ws);
  void** dst[11] = {(void**)&m->joint, (void**)&m->capn, (void**)&m->tin,   (void**)&m->te1,
                    (void**)&m->temb,  (void**)&m->tsilu, (void**)&m->outmod,
                    (void**)&m->cos_t, (void**)&m->sin_t, (void**)&m->pos,
                    (void**)&m->premod};
  for (int i = 0; i < 11; ++i) {
    *dst[i] = p;
    p += align256(sz[i]);
  }
  m->blk_ws = p;
  m->blk_bytes = blk;
  m->ws_rows = JT;
  m->ws_q = Q;
  return MING_OK;
}

// flag = 1 when the n bytes (n % 16 == 0, both 16-byte aligned) differ.
__global__ void bytes_differ_kernel(const uint4* a, const uint4* b, size_t n16, int* flag) {
  bool diff = false;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint4 x = a[i], y = b[i];
    diff |= (x.x != y.x) | (x.y != y.y) | (x.z != y.z) | (x.w != y.w);
  }
  if (diff) *flag = 1;  // every writer stores the same value
}

void free_cap_entry(ming_model::CapEntry& e) {
  if (e.key) (void)hipFree(e.key);
  if (e.out) (void)hipFree(e.out);
  e = ming_model::CapEntry{};
}

// Grows a device buffer to `bytes` (contents not kept). false when it cannot.
bool grow(void** p, size_t* cap, size_t bytes) {
  if (*cap >= bytes && *p) return true;
  if (*p) (void)hipFree(*p);
  *p = nullptr;
  *cap = 0;
  if (hipMalloc(p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    *p = nullptr;
    return false;
  }
  *cap = bytes;
  return true;
}

// The context refiner's adapter state: the sum of its projections' bind
// generations, which grows with every bind or unbind of any of them (through
// ming_model_bind_loras or directly on a borrowed weight).
uint64_t caption_bind_sig(const ming_model* m) {
  uint64_t sig = 0;
  for (const ming_block_desc& b : m->ctx_blocks)
    for (const ming_qweight* q : {b.q, b.k, b.v, b.o, b.w1, b.w3, b.w2})
      sig += ming::rt_qweight_bind_gen(q);
  return sig;
}

// The caption-cache entry holding exactly these caption bytes, refined with
// the current adapter bindings, or null (ming-dit.cc:1543-1560): shape fields
// and binding signature first, then the bytes, compared on the device.
int cap_lookup(ming_model* m, const uint16_t* cap, int CAP, int Q, int64_t stride,
               uint64_t sig, hipStream_t s, ming_model::CapEntry** hit) {
  *hit = nullptr;
  const size_t bytes = (size_t)CAP * (size_t)stride * 2;
  int cand[2], nc = 0;
  for (int i = 0; i < 2; ++i) {
    const ming_model::CapEntry& e = m->cap[i];
    if (e.valid && e.q == Q && e.len == CAP && e.stride == stride && e.key_bytes == bytes &&
        e.bind_sig == sig)
      cand[nc++] = i;
  }
  if (nc == 0) return MING_OK;
  if (!m->cap_flag) {
    if (hipMalloc(&m->cap_flag, 2 * sizeof(int)) != hipSuccess) {
      (void)hipGetLastError();
      m->cap_flag = nullptr;
      return MING_OK;  // no comparison, no hit: the caption path runs
    }
  }
  if (hipMemsetAsync(m->cap_flag, 0, 2 * sizeof(int), s) != hipSuccess)
    return rt_fail(MING_ERR_HIP, "ming_model_forward: caption cache flag reset failed");
  const size_t n16 = bytes / 16;
  const unsigned grid = (unsigned)std::min<size_t>((n16 + 255) / 256, 1024);
  for (int k = 0; k < nc; ++k) {
    hipLaunchKernelGGL(bytes_differ_kernel, dim3(grid > 0 ? grid : 1), dim3(256), 0, s,
                       static_cast<const uint4*>(m->cap[cand[k]].key),
                       reinterpret_cast<const uint4*>(cap), n16, m->cap_flag + k);
    if (hipGetLastError() != hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: caption compare launch failed");
  }
  int differ[2] = {1, 1};
  if (hipMemcpyAsync(differ, m->cap_flag, 2 * sizeof(int), hipMemcpyDeviceToHost, s) !=
          hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return rt_fail(MING_ERR_HIP, "ming_model_forward: caption compare failed");
  for (int k = 0; k < nc; ++k)
    if (!differ[k]) {
      *hit = &m->cap[cand[k]];
      break;
    }
  return MING_OK;
}

// Block progress (set_block_progress): report k goes out once blocks [0, k)
// have finished, in order, each k once, on the calling thread.
struct Progress {
  ming_model* m = nullptr;
  int total = 0, recorded = 0, reported = 0;
  bool on() const { return m && m->progress; }
  int init(ming_model* mm, int n) {
    m = mm;
    total = n;
    if (!on()) return MING_OK;
    while ((int)m->block_events.size() < n) {
      hipEvent_t e;
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
        return rt_fail(MING_ERR_HIP, "ming_model_forward: progress event creation failed");
      m->block_events.push_back(static_cast<void*>(e));
    }
    return MING_OK;
  }
  int done_block(hipStream_t s) {
    if (!on()) return MING_OK;
    if (hipEventRecord(static_cast<hipEvent_t>(m->block_events[(size_t)recorded]), s) !=
        hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: progress event record failed");
    ++recorded;
    return MING_OK;
  }
  void poll(bool wait) {
    if (!on()) return;
    while (reported < total && reported <= recorded) {
      if (reported > 0) {
        hipEvent_t e = static_cast<hipEvent_t>(m->block_events[(size_t)reported - 1]);
        if (wait) {
          if (hipEventSynchronize(e) != hipSuccess) return;
        } else if (hipEventQuery(e) != hipSuccess) {
          (void)hipGetLastError();  // "not ready" is not an error to keep
          return;
        }
      }
      m->progress(m->progress_user, reported, total);
      ++reported;
    }
  }
};

// A cooperative stop: the queued work drains, the forward reports MING_STOPPED
// with no error (ming-dit.h:170-189).
bool stop_requested(ming_model* m) { return m->stop && m->stop(m->stop_user) != 0; }
int stopped(hipStream_t s) {
  (void)hipStreamSynchronize(s);
  ming::rt_ok();
  return MING_STOPPED;
}

// Whether `slot` is bound on any context-refiner projection: only then does a
// strength change touch the cached caption rows (ming-dit.cc:3031-3038).
bool slot_in_ctx_refiner(const ming_model* m, int slot) {
  for (const ming_block_desc& b : m->ctx_blocks)
    for (const ming_qweight* q : {b.q, b.k, b.v, b.o, b.w1, b.w3, b.w2}) {
      int N = 0, K = 0, ns = 0;
      if (!q || ming_qweight_shape(q, &N, &K, &ns) != MING_OK) continue;
      for (int sg = 0; sg < ns; ++sg)
        if (ming_qweight_lora_rank(q, sg, slot) > 0) return true;
    }
  return false;
}

}  // namespace

namespace ming {

std::vector<ModuleRef> model_modules(const ming_model* m) {
  std::vector<ModuleRef> v;
  const ming_model_desc& d = m->d;
  const int H = d.hidden, F = d.ffn;
  auto one = [&](const std::string& pre, const ming_block_desc& b, bool ctx) {
    const struct {
      const char* nm;
      const ming_qweight* q;
      int N, K;
    } p[7] = {{"attention.to_q", b.q, H, H},        {"attention.to_k", b.k, H, H},
              {"attention.to_v", b.v, H, H},        {"attention.to_out.0", b.o, H, H},
              {"feed_forward.w1", b.w1, F, H},      {"feed_forward.w3", b.w3, F, H},
              {"feed_forward.w2", b.w2, H, F}};
    for (const auto& x : p)
      v.push_back({pre + x.nm, const_cast<ming_qweight*>(x.q), x.N, x.K, ctx});
  };
  for (int L = 0; L < (int)m->blocks.size(); ++L) {
    const std::string pre = L < d.n_refiner
                                ? "noise_refiner." + std::to_string(L) + "."
                                : "layers." + std::to_string(L - d.n_refiner) + ".";
    one(pre, m->blocks[(size_t)L], false);
  }
  for (int i = 0; i < (int)m->ctx_blocks.size(); ++i)
    one("context_refiner." + std::to_string(i) + ".", m->ctx_blocks[(size_t)i], true);
  return v;
}

void model_drop_caption_cache(ming_model* m) {
  for (auto& e : m->cap) e.valid = false;
}

}  // namespace ming

extern "C" {

size_t ming_block_workspace_bytes(const ming_block_dims* dims, int rows) {
  if (!dims || rows < 0) return 0;
  BlockWs w{};
  return block_ws_layout(*dims, rows, nullptr, &w);
}

int ming_block_forward(ming_ctx* c, const ming_block_desc* b, const ming_block_dims* dims,
                       uint16_t* x, int rows, const float* cos_t, const float* sin_t,
                       const uint16_t* temb, const float* scales, void* ws,
                       size_t ws_bytes) {
  if (!c || !b || !x || !cos_t || !sin_t || !ws)
    return rt_fail(MING_ERR_ARG, "ming_block_forward: null argument");
  RC(check_dims(dims));
  const bool modulated = b->ada != nullptr;
  RC(check_block(b, *dims, modulated, "ming_block_forward"));
  if (modulated && !temb)
    return rt_fail(MING_ERR_ARG, "ming_block_forward: a modulated block needs temb");
  if (rows <= 0) return rows == 0 ? rt_ok() : rt_fail(MING_ERR_SHAPE, "ming_block_forward: rows < 0");
  BlockWs w{};
  const size_t need = block_ws_layout(*dims, rows, static_cast<char*>(ws), &w);
  if (ws_bytes < need || reinterpret_cast<uintptr_t>(ws) % 256 != 0)
    return rt_fail(MING_ERR_ARG, "ming_block_forward: workspace too small or not 256-byte aligned");
  RC(block_forward(c, b, *dims, x, rows, cos_t, sin_t, temb, scales, w));
  return rt_ok();
}

int ming_model_create(ming_ctx* c, const ming_model_desc* d, ming_model** out) {
  if (!c || !d || !out) return rt_fail(MING_ERR_ARG, "ming_model_create: null argument");
  *out = nullptr;
  ming_block_dims bd{d->hidden, d->n_heads, d->ffn, d->adaln_dim, d->eps};
  RC(check_dims(&bd));
  const int H = d->hidden;
  if (d->n_layers < 0 || d->n_refiner < 0 || d->time_freq <= 0 || d->time_freq % 64 ||
      d->time_mid <= 0 || d->time_mid % 64 || d->patch_dim <= 0 || d->patch_dim % 64 ||
      d->cap_dim <= 0 || d->cap_dim % 64 || d->cap_dim > 8192 || d->time_freq % 2)
    return rt_fail(MING_ERR_SHAPE,
                   "ming_model_create: time_freq, time_mid, patch_dim and cap_dim must be "
                   "multiples of 64 (cap_dim <= 8192)");
  if (d->axes[0] + d->axes[1] + d->axes[2] != 128 || d->axes[0] % 2 || d->axes[1] % 2 ||
      d->axes[2] % 2 || d->axes_lens[0] <= 0 || d->axes_lens[1] <= 0 || d->axes_lens[2] <= 0)
    return rt_fail(MING_ERR_SHAPE, "ming_model_create: rotary axes must be even and sum to 128");
  if ((d->n_refiner > 0 && !d->ctx_blocks) || (d->n_refiner + d->n_layers > 0 && !d->blocks))
    return rt_fail(MING_ERR_ARG, "ming_model_create: block list missing");
  for (int i = 0; i < d->n_refiner; ++i)
    RC(check_block(&d->ctx_blocks[i], bd, false, "ming_model_create (context refiner)"));
  for (int i = 0; i < d->n_refiner + d->n_layers; ++i)
    RC(check_block(&d->blocks[i], bd, true, "ming_model_create (modulated block)"));
  if (!shape_is(d->time_1, d->time_mid, d->time_freq) || !d->time_1b ||
      !shape_is(d->time_2, d->adaln_dim, d->time_mid) || !d->time_2b)
    return rt_fail(MING_ERR_SHAPE, "ming_model_create: timestep MLP shapes");
  if (!shape_is(d->x_in, H, d->patch_dim) || !d->x_in_b)
    return rt_fail(MING_ERR_SHAPE, "ming_model_create: x_embedder must be [H][patch_dim]");
  if (!shape_is(d->cap_in, H, d->cap_dim) || !d->cap_in_b || !d->cap_norm)
    return rt_fail(MING_ERR_SHAPE, "ming_model_create: cap_embedder must be [H][cap_dim]");
  if (!shape_is(d->final_ada, H, d->adaln_dim) || !d->final_ada_b ||
      !shape_is(d->final_lin, d->patch_dim, H) || !d->final_lin_b)
    return rt_fail(MING_ERR_SHAPE, "ming_model_create: final layer shapes");
  ming_model* m = new (std::nothrow) ming_model();
  if (!m) return rt_fail(MING_ERR_ALLOC, "ming_model_create: out of host memory");
  m->ctx = c;
  m->d = *d;
  m->ctx_blocks.assign(d->ctx_blocks, d->ctx_blocks + d->n_refiner);
  m->blocks.assign(d->blocks, d->blocks + d->n_refiner + d->n_layers);
  m->d.ctx_blocks = m->ctx_blocks.data();
  m->d.blocks = m->blocks.data();
  m->tin_host.assign((size_t)d->time_freq, 0);
  ming::rt_retain(c);
  *out = m;
  return rt_ok();
}

int ming_model_destroy(ming_model* m) {
  if (!m) return rt_ok();
  (void)hipStreamSynchronize((hipStream_t)ming_ctx_stream(m->ctx));
  if (m->ws) (void)hipFree(m->ws);
  for (auto& e : m->cap) free_cap_entry(e);
  if (m->cap_flag) (void)hipFree(m->cap_flag);
  for (void* e : m->block_events) (void)hipEventDestroy(static_cast<hipEvent_t>(e));
  for (ming_qweight* q : m->own_qw) (void)ming_qweight_destroy(q);
  for (void* p : m->own_dev) ming::rt_free(m->ctx, p);
  ming::rt_release(m->ctx);
  delete m;
  return rt_ok();
}

int ming_model_set_stream_stop(ming_model* m, ming_stop_fn fn, void* user) {
  if (!m) return rt_fail(MING_ERR_ARG, "ming_model_set_stream_stop: null model");
  m->stop = fn;
  m->stop_user = user;
  return rt_ok();
}

int ming_model_set_block_progress(ming_model* m, ming_progress_fn fn, void* user) {
  if (!m) return rt_fail(MING_ERR_ARG, "ming_model_set_block_progress: null model");
  m->progress = fn;
  m->progress_user = user;
  return rt_ok();
}

int ming_model_set_caption_cache(ming_model* m, int on) {
  if (!m) return rt_fail(MING_ERR_ARG, "ming_model_set_caption_cache: null model");
  m->cap_cache_on = on != 0;
  if (!m->cap_cache_on) {
    (void)hipStreamSynchronize((hipStream_t)ming_ctx_stream(m->ctx));
    for (auto& e : m->cap) free_cap_entry(e);
  }
  return rt_ok();
}

int ming_model_set_lora_scale(ming_model* m, int slot, float s) {
  if (!m) return rt_fail(MING_ERR_ARG, "ming_model_set_lora_scale: null model");
  if (slot < 0 || slot >= MING_MAX_LORA_SLOTS)
    return rt_fail(MING_ERR_ARG, "ming_model_set_lora_scale: slot out of range");
  if (!std::isfinite(s))
    return rt_fail(MING_ERR_ARG, "ming_model_set_lora_scale: strength must be finite");
  if (m->scales[slot] == s) return rt_ok();
  m->scales[slot] = s;
  // the cached caption rows were refined at the old strength
  if (slot_in_ctx_refiner(m, slot)) ming::model_drop_caption_cache(m);
  return rt_ok();
}

float ming_model_lora_scale(const ming_model* m, int slot) {
  if (!m || slot < 0 || slot >= MING_MAX_LORA_SLOTS) return 0.0f;
  return m->scales[slot];
}

int ming_model_forward(ming_model* m, const uint16_t* latents, const uint16_t* cap,
                       int64_t cap_stride, int IMG, int CAP, int Q, const int32_t* pos_t,
                       const int32_t* pos_h, const int32_t* pos_w, float sigma,
                       uint16_t* out) {
  if (!m || !latents || !cap || !pos_t || !pos_h || !pos_w || !out)
    return rt_fail(MING_ERR_ARG, "ming_model_forward: missing input");
  const ming_model_desc& d = m->d;
  ming_ctx* c = m->ctx;
  const int H = d.hidden, JT = IMG + CAP;
  // the layout is checked, not trusted (ming-dit.cc:1507-1523)
  if (IMG <= 0 || CAP <= 0 || Q < 0 || Q > CAP)
    return rt_fail(MING_ERR_SHAPE, "ming_model_forward: image and caption row counts must be "
                                   "positive, with 0 <= query rows <= caption rows");
  if ((Q > 0 && cap_stride < d.cap_dim) || (CAP > Q && cap_stride < H) || cap_stride % 8)
    return rt_fail(MING_ERR_SHAPE,
                   "ming_model_forward: cap_stride must be a multiple of 8 and at least "
                   "cap_dim (query rows) and the hidden width (pass-through rows)");
  for (int t = 0; t < JT; ++t)
    if (pos_t[t] < 0 || pos_h[t] < 0 || pos_w[t] < 0 || pos_t[t] >= d.axes_lens[0] ||
        pos_h[t] >= d.axes_lens[1] || pos_w[t] >= d.axes_lens[2])
      return rt_fail(MING_ERR_SHAPE,
                     "ming_model_forward: a position lies outside the rotary table's range on its axis (axes_lens)");
  if (!std::isfinite(sigma))
    return rt_fail(MING_ERR_ARG, "ming_model_forward: sigma must be finite");
  RC(ensure_model_ws(m, JT, Q));
  hipStream_t s = (hipStream_t)ming_ctx_stream(c);
  // positions -> device, then the joint rotary table (build_rope_, 1443-1486)
  {
    std::vector<int32_t> pos((size_t)JT * 3);
    std::memcpy(pos.data(), pos_t, sizeof(int32_t) * JT);
    std::memcpy(pos.data() + JT, pos_h, sizeof(int32_t) * JT);
    std::memcpy(pos.data() + 2 * JT, pos_w, sizeof(int32_t) * JT);
    if (hipMemcpyAsync(m->pos, pos.data(), pos.size() * 4, hipMemcpyHostToDevice, s) !=
        hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: position upload failed");
    if (hipStreamSynchronize(s) != hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: position upload failed");
  }
  RC(ming_rope_table(c, m->pos, m->pos + JT, m->pos + 2 * JT, JT, d.axes, 128,
                     (double)d.rope_theta, m->cos_t, m->sin_t));
  // timestep: cos-first sinusoid of t_scale * (1 - sigma) (time_proj_, 1418-1437)
  {
    const int half = d.time_freq / 2;
    const double t = (double)d.t_scale * (1.0 - (double)sigma);
    for (int i = 0; i < half; ++i) {
      const double f = std::exp(-std::log(10000.0) * (double)i / (double)half);
      m->tin_host[(size_t)i] = host_bf16((float)std::cos(t * f));
      m->tin_host[(size_t)(half + i)] = host_bf16((float)std::sin(t * f));
    }
    if (hipMemcpyAsync(m->tin, m->tin_host.data(), (size_t)d.time_freq * 2,
                       hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: timestep upload failed");
  }
  RC(ming_lin(c, d.time_1, m->tin, d.time_freq, m->te1, d.time_mid, 1, nullptr));
  RC(ming_bias_act(c, m->te1, d.time_mid, d.time_1b, 1, d.time_mid, 1));
  RC(ming_lin(c, d.time_2, m->te1, d.time_mid, m->temb, d.adaln_dim, 1, nullptr));
  RC(ming_bias_act(c, m->temb, d.adaln_dim, d.time_2b, 1, d.adaln_dim, 0));
  RC(ming_silu(c, m->temb, m->tsilu, d.adaln_dim));
  // embeddings: image rows through x_embedder; caption query rows through
  // cap_embedder (RMSNorm + Linear), the rest copied (2283-2304)
  // the caption cache (ming-dit.cc:1543-1577): a hit serves the whole caption
  // path; a miss refills an empty entry, else the least recently used one,
  // which becomes valid only when this forward completes
  ming_model::CapEntry* hit = nullptr;
  ming_model::CapEntry* fill = nullptr;
  const size_t cap_bytes = (size_t)CAP * (size_t)cap_stride * 2;
  const bool cacheable = m->cap_cache_on && reinterpret_cast<uintptr_t>(cap) % 16 == 0;
  const uint64_t bind_sig = caption_bind_sig(m);
  if (cacheable) {
    RC(cap_lookup(m, cap, CAP, Q, cap_stride, bind_sig, s, &hit));
    if (!hit) {
      fill = &m->cap[0];
      for (auto& e : m->cap) {
        if (!e.valid) {
          fill = &e;
          break;
        }
        if (e.tick < fill->tick) fill = &e;
      }
      fill->valid = false;
      if (!grow(&fill->key, &fill->key_cap, cap_bytes) ||
          !grow(&fill->out, &fill->out_cap, (size_t)CAP * H * 2))
        fill = nullptr;  // no room: this forward runs uncached
    }
  }
  RC(ming_lin(c, d.x_in, latents, d.patch_dim, m->joint, H, IMG, nullptr));
  RC(ming_bias_act(c, m->joint, H, d.x_in_b, IMG, H, 0));
  uint16_t* cap0 = m->joint + (size_t)IMG * H;
  if (hit) {
    if (hipMemcpyAsync(cap0, hit->out, (size_t)CAP * H * 2, hipMemcpyDeviceToDevice, s) !=
        hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: caption cache copy failed");
    hit->tick = ++m->cap_tick;
    ming::rt_note_cap_hit(c);
  } else {
  if (Q > 0) {
    if (hipMemcpy2DAsync(m->capn, (size_t)d.cap_dim * 2, cap, (size_t)cap_stride * 2,
                         (size_t)d.cap_dim * 2, Q, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: caption copy failed");
    RC(ming_rmsnorm(c, m->capn, d.cap_dim, d.cap_norm, m->capn, d.cap_dim, Q, d.cap_dim,
                    d.eps));
    RC(ming_lin(c, d.cap_in, m->capn, d.cap_dim, cap0, H, Q, nullptr));
    RC(ming_bias_act(c, cap0, H, d.cap_in_b, Q, H, 0));
  }
  if (CAP > Q &&
      hipMemcpy2DAsync(cap0 + (size_t)Q * H, (size_t)H * 2, cap + (size_t)Q * cap_stride,
                       (size_t)cap_stride * 2, (size_t)H * 2, CAP - Q,
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
    return rt_fail(MING_ERR_HIP, "ming_model_forward: caption copy failed");
  }
  // blocks: the context refiner over the caption rows (its table rows start
  // at IMG), then the noise refiner over the image rows and the main layers
  // over the joint sequence; stop polled and progress reported per block
  ming_block_dims bd{d.hidden, d.n_heads, d.ffn, d.adaln_dim, d.eps};
  BlockWs w{};
  block_ws_layout(bd, JT, static_cast<char*>(m->blk_ws), &w);
  const int NM = d.n_refiner + d.n_layers;
  Progress prog;
  RC(prog.init(m, d.n_refiner + NM));
  for (int i = 0; i < d.n_refiner; ++i) {
    if (stop_requested(m)) return stopped(s);
    prog.poll(false);
    if (!hit)
      RC(block_forward(c, &m->ctx_blocks[(size_t)i], bd, cap0, CAP,
                       m->cos_t + (size_t)IMG * 64, m->sin_t + (size_t)IMG * 64, nullptr,
                       m->scales, w));
    RC(prog.done_block(s));
  }
  if (fill) {
    // before the main stack rewrites these rows in place
    if (hipMemcpyAsync(fill->out, cap0, (size_t)CAP * H * 2, hipMemcpyDeviceToDevice, s) !=
            hipSuccess ||
        hipMemcpyAsync(fill->key, cap, cap_bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return rt_fail(MING_ERR_HIP, "ming_model_forward: caption cache fill failed");
  }
  // every modulated block's adaLN modulation depends on temb alone: one
  // batched GEMV + glue for all of them instead of two launches per block
  bool premod = false;
  {
    std::vector<const ming_qweight*> ada(NM);
    std::vector<const uint16_t*> ada_b(NM), an1(NM), fn1(NM);
    std::vector<uint16_t*> mods(NM), nw1(NM), nw3(NM);
    std::vector<float*> tg(NM);
    bool all = true;
    for (int L = 0; L < NM; ++L) {
      const ming_block_desc& b = m->blocks[(size_t)L];
      if (!b.ada) all = false;
      const Premod p = premod_of(m->premod, (size_t)H, L);
      ada[L] = b.ada; ada_b[L] = b.ada_b; an1[L] = b.an1; fn1[L] = b.fn1;
      mods[L] = p.mods; nw1[L] = p.nw1; nw3[L] = p.nw3; tg[L] = p.tg;
    }
    if (all)
      RC(ming::rt_modulation_batch(c, NM, ada.data(), ada_b.data(), an1.data(), fn1.data(),
                                   m->temb, H, mods.data(), nw1.data(), nw3.data(), tg.data(),
                                   nullptr, &premod));
  }
  bool prenormed = false;
  for (int L = 0; L < NM; ++L) {
    if (stop_requested(m)) return stopped(s);
    prog.poll(false);
    const int rows = L < d.n_refiner ? IMG : JT;
    const Premod pm = premod_of(m->premod, (size_t)H, L);
    // the next block's pre-norm rides on this block's last pass when it
    // covers the same rows and its weight is known already
    const uint16_t* next_g1 = nullptr;
    if (L + 1 < NM && (L + 1 < d.n_refiner ? IMG : JT) == rows) {
      const ming_block_desc& nb = m->blocks[(size_t)L + 1];
      if (!nb.ada) next_g1 = nb.an1;
      else if (premod) next_g1 = premod_of(m->premod, (size_t)H, L + 1).nw1;
    }
    RC(block_forward(c, &m->blocks[(size_t)L], bd, m->joint, rows, m->cos_t, m->sin_t,
                     m->temb, m->scales, w, premod ? &pm : nullptr, prenormed, next_g1));
    prenormed = next_g1 != nullptr;
    RC(prog.done_block(s));
    // with a stop wired, the host stays within 4 blocks of the GPU so that a
    // stop requested mid-forward is seen (ming-dit.cc:2530-2540)
    if (m->stop && (L + 1) % 4 == 0 && L + 1 < NM) {
      if (hipStreamSynchronize(s) != hipSuccess)
        return rt_fail(MING_ERR_HIP, "ming_model_forward: the GPU failed");
      prog.poll(false);
    }
  }
  // final layer: adaLN scale from silu(temb), LayerNorm (eps 1e-6) + modulate,
  // then the linear to the patch dimension (2557-2563)
  RC(ming_lin(c, d.final_ada, m->tsilu, d.adaln_dim, m->outmod, H, 1, nullptr));
  RC(ming_bias_act(c, m->outmod, H, d.final_ada_b, 1, H, 0));
  RC(ming_ln_modulate(c, m->joint, H, m->outmod, w.nrm, H, IMG, H, 1e-6f));
  RC(ming_lin(c, d.final_lin, w.nrm, H, out, d.patch_dim, IMG, nullptr));
  RC(ming_bias_act(c, out, d.patch_dim, d.final_lin_b, IMG, d.patch_dim, 0));
  prog.poll(true);
  if (hipStreamSynchronize(s) != hipSuccess)
    return rt_fail(MING_ERR_HIP, "ming_model_forward: the GPU failed");
  // an fp16 copy that could not hold its value fails the forward (and the
  // caption-cache entry it filled never becomes valid)
  RC(ming::rt_take_range_fault(c, "ming_model_forward"));
  if (fill) {
    fill->valid = true;
    fill->q = Q;
    fill->len = CAP;
    fill->stride = cap_stride;
    fill->key_bytes = cap_bytes;
    fill->bind_sig = bind_sig;
    fill->tick = ++m->cap_tick;
  }
  return rt_ok();
}

}  // extern "C"
