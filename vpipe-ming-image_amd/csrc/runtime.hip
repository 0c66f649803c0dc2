// Host runtime behind include/ming_dit_amd.h: contexts, resident
// projection weights, load-time adapter binding, and the lin() dispatch
// that builds the live LoRA stack per call.
//
// The live-stack rule is the reference's lora_for_ + Stack::add
// (ming-dit.cc:3007-3022): a slot enters the stack only when it is bound on
// the projection AND its strength is non-zero, in slot order, so an
// all-zero call runs the base kernel alone and a lone slot computes the
// same bits whichever slot index holds it.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ming_dit_amd.h"
#include "kernels.h"
#include "rt.h"

namespace {

thread_local std::string g_err;

// The process-wide session log (ming_set_log_sink).
std::mutex g_log_mu;
ming_log_fn g_log_fn = nullptr;
void* g_log_user = nullptr;

int fail(int code, const std::string& why) {
  g_err = why;
  return code;
}
int ok() {
  g_err.clear();
  return MING_OK;
}
int hip_fail(hipError_t e, const char* what) {
  return fail(MING_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define MING_HIP(call, what)                       \
  do {                                             \
    hipError_t e_ = (call);                        \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev)
      (void)hipSetDevice(prev);
  }
};

}  // namespace

struct ming_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  ming_engagement eng{};
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  void* xh = nullptr;          // fp16 copy of the projection input
  size_t xh_bytes = 0;
  void* xh2 = nullptr;         // fp16 copy of the SwiGLU output (w2's input)
  size_t xh2_bytes = 0;
  void* vt = nullptr;          // V^T [heads][128][keys] for attention
  size_t vt_bytes = 0;
  void* up = nullptr;          // general route + SwiGLU: the projection before the gate
  size_t up_bytes = 0;
  void* part = nullptr;        // split-K partials of the stacked x.A GEMM
  size_t part_bytes = 0;
  int route = MING_ROUTE_AUTO;
  // device word raised by any fp16 copy that could not hold its value
  // (range_report); read and cleared at synchronization points
  int* range = nullptr;
  // set by the block driver while the block's projections are dense: the fp16
  // copies it writes are then never read, so they raise nothing
  bool copies_unread = false;
  int live_weights = 0;   // a context outlives every weight made on it
  // Per-launch HIP-event timing (ming_ctx_set_profiling), by bucket.
  bool profiling = false;
  bool no_events = false;   // set while ming_lin_noalloc runs (creating one may allocate)
  struct Rec { int bucket; hipEvent_t a, b; double flops, bytes; };
  std::vector<Rec> recs;
  std::vector<hipEvent_t> pool;
};

namespace {

// Profile buckets: one per kernel family (the reference's per-category
// marks, ming-dit.cc:1689-1717, as HIP events around each launch).
enum Bucket {
  kBQ4, kBQ8, kBDense, kBF4, kBF8, kBCvt, kBXa, kBRms, kBQkRope, kBRopeTab, kBSwiglu, kBResid,
  kBModulate, kBBias, kBLn, kBQuant, kBAttn, kBNormRes, kBGemv, kBP4, kBP8, kBCount
};
const char* const kBucketName[kBCount] = {
    "qproj.w4", "qproj.w8", "qproj.dense", "qproj_fast.w4", "qproj_fast.w8",
    "cvt_f16", "lora_xa", "rmsnorm",
    "qk_norm_rope", "rope_table", "swiglu", "residual", "modulate",
    "bias_act", "ln_modulate", "quantize", "attention", "norm_residual", "gemv",
    "qproj_pair.w4", "qproj_pair.w8"};

hipEvent_t take_event(ming_ctx* c) {
  if (!c->pool.empty()) {
    hipEvent_t e = c->pool.back();
    c->pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Runs `launch` (returning hipError_t), bracketed by events when profiling.
template <class F>
hipError_t profiled(ming_ctx* c, int bucket, double flops, double bytes,
                    F&& launch) {
  if (!c->profiling || c->no_events) return launch();
  hipEvent_t a = take_event(c), b = take_event(c);
  if (!a || !b) return hipErrorOutOfMemory;
  hipError_t e = hipEventRecord(a, c->stream);
  if (e == hipSuccess) e = launch();
  if (e == hipSuccess) e = hipEventRecord(b, c->stream);
  if (e != hipSuccess) {
    c->pool.push_back(a);
    c->pool.push_back(b);
    return e;
  }
  c->recs.push_back({bucket, a, b, flops, bytes});
  return hipSuccess;
}

struct LoraBind {
  int rank = 0;     // as bound
  int rank8 = 0;    // padded to 8 (zero rows / columns)
  float fold = 1.0f;
  uint16_t* A = nullptr;  // [rank8][K]
  uint16_t* B = nullptr;  // [N_seg][rank8]
};

struct Segment {
  int n_begin = 0;
  int N = 0;
  LoraBind slot[MING_MAX_LORA_SLOTS];
};

int round_up(int v, int m) { return (v + m - 1) / m * m; }

}  // namespace

struct ming_qweight {
  ming_ctx* ctx = nullptr;
  int N = 0, K = 0, bits = 0, group = 64;
  uint32_t* codes_t = nullptr;   // general route: [kt][n][w] + bf16 (s, b)
  uint32_t* sb = nullptr;
  uint32_t* codes_f = nullptr;   // fast route: fragment-ordered codes
  uint32_t* sbf = nullptr;       //   + fp16 (s, b)
  bool fast = false;             // every scale and bias exact in fp16
  uint16_t* w16 = nullptr;
  std::vector<Segment> segs;
  // Stacked adapter factors, rebuilt when a binding changes:
  //   A_all [R8_all][K]     every (segment, slot) in order
  //   B_seg[s] [N_s][R8_s]  per segment, its slots in order
  bool stacks_dirty = true;
  uint16_t* A_all = nullptr;
  std::vector<uint16_t*> B_seg;
  std::vector<int> a_row0;   // [seg*8 + slot] row in A_all
  int a_rows = 0;            // rows of A_all
  std::vector<int> b_col0;   // [seg*8 + slot] column in B_seg[seg]
  std::vector<int> b_ld;     // per segment: R8 of the segment
  // bumped by every bind and unbind: a model's caption cache keys on the
  // context-refiner weights' generations, so a direct rebinding of one of
  // them is never served stale rows
  uint64_t bind_gen = 0;
};

namespace {

void free_stacks(ming_qweight* q) {
  if (q->A_all) (void)hipFree(q->A_all);
  q->A_all = nullptr;
  for (auto* b : q->B_seg)
    if (b) (void)hipFree(b);
  q->B_seg.clear();
  q->stacks_dirty = true;
}

int build_stacks(ming_qweight* q) {
  if (!q->stacks_dirty) return MING_OK;
  hipStream_t s = q->ctx->stream;
  // The old stacks may still be read by queued kernels.
  MING_HIP(hipStreamSynchronize(s), "stack rebuild sync");
  free_stacks(q);
  const int nseg = (int)q->segs.size();
  q->a_row0.assign(nseg * MING_MAX_LORA_SLOTS, -1);
  q->b_col0.assign(nseg * MING_MAX_LORA_SLOTS, -1);
  q->b_ld.assign(nseg, 0);
  q->B_seg.assign(nseg, nullptr);
  int rows_all = 0;
  for (int si = 0; si < nseg; ++si) {
    int col = 0;
    for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl) {
      const LoraBind& b = q->segs[si].slot[sl];
      if (b.rank <= 0) continue;
      q->a_row0[si * MING_MAX_LORA_SLOTS + sl] = rows_all;
      q->b_col0[si * MING_MAX_LORA_SLOTS + sl] = col;
      rows_all += b.rank8;
      col += b.rank8;
    }
    q->b_ld[si] = col;
  }
  q->a_rows = rows_all;
  if (rows_all == 0) {
    q->stacks_dirty = false;
    return MING_OK;
  }
  const size_t K = (size_t)q->K;
  MING_HIP(hipMalloc(&q->A_all, (size_t)rows_all * K * 2), "A stack alloc");
  for (int si = 0; si < nseg; ++si) {
    const Segment& sg = q->segs[si];
    if (q->b_ld[si] > 0)
      MING_HIP(hipMalloc(&q->B_seg[si], (size_t)sg.N * q->b_ld[si] * 2),
               "B stack alloc");
    for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl) {
      const LoraBind& b = sg.slot[sl];
      if (b.rank <= 0) continue;
      const int ar = q->a_row0[si * MING_MAX_LORA_SLOTS + sl];
      const int bc = q->b_col0[si * MING_MAX_LORA_SLOTS + sl];
      MING_HIP(hipMemcpyAsync(q->A_all + (size_t)ar * K, b.A,
                              (size_t)b.rank8 * K * 2,
                              hipMemcpyDeviceToDevice, s),
               "A stack copy");
      MING_HIP(hipMemcpy2DAsync(q->B_seg[si] + bc, (size_t)q->b_ld[si] * 2,
                                b.B, (size_t)b.rank8 * 2,
                                (size_t)b.rank8 * 2, (size_t)sg.N,
                                hipMemcpyDeviceToDevice, s),
               "B stack copy");
    }
  }
  q->stacks_dirty = false;
  return MING_OK;
}

int ensure_scratch(ming_ctx* c, size_t bytes) {
  if (bytes <= c->scratch_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->scratch) (void)hipFree(c->scratch);
  c->scratch = nullptr;
  c->scratch_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&c->scratch, want) != hipSuccess)
    return fail(MING_ERR_ALLOC, "LoRA scratch allocation failed");
  c->scratch_bytes = want;
  return MING_OK;
}

int ensure_part(ming_ctx* c, size_t bytes) {
  if (bytes <= c->part_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->part) (void)hipFree(c->part);
  c->part = nullptr;
  c->part_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&c->part, want) != hipSuccess)
    return fail(MING_ERR_ALLOC, "split-K partial scratch allocation failed");
  c->part_bytes = want;
  return MING_OK;
}

int ensure_xh(ming_ctx* c, size_t bytes) {
  if (bytes <= c->xh_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->xh) (void)hipFree(c->xh);
  c->xh = nullptr;
  c->xh_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&c->xh, want) != hipSuccess)
    return fail(MING_ERR_ALLOC, "fp16 activation scratch allocation failed");
  c->xh_bytes = want;
  return MING_OK;
}

int ensure_xh2(ming_ctx* c, size_t bytes) {
  if (bytes <= c->xh2_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->xh2) (void)hipFree(c->xh2);
  c->xh2 = nullptr;
  c->xh2_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&c->xh2, want) != hipSuccess)
    return fail(MING_ERR_ALLOC, "fp16 activation scratch allocation failed");
  c->xh2_bytes = want;
  return MING_OK;
}

int ensure_vt(ming_ctx* c, size_t bytes) {
  if (bytes <= c->vt_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->vt) (void)hipFree(c->vt);
  c->vt = nullptr;
  c->vt_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&c->vt, want) != hipSuccess)
    return fail(MING_ERR_ALLOC, "attention V^T scratch allocation failed");
  c->vt_bytes = want;
  return MING_OK;
}

int ensure_up(ming_ctx* c, size_t bytes) {
  if (bytes <= c->up_bytes) return MING_OK;
  MING_HIP(hipStreamSynchronize(c->stream), "scratch grow sync");
  if (c->up) (void)hipFree(c->up);
  c->up = nullptr;
  c->up_bytes = 0;
  if (hipMalloc(&c->up, bytes) != hipSuccess)
    return fail(MING_ERR_ALLOC, "SwiGLU scratch allocation failed");
  c->up_bytes = bytes;
  return MING_OK;
}

// Copy `bytes` from host or device into a fresh device buffer.
int upload(ming_ctx* c, void** dst, const void* src, size_t bytes,
           int src_on_device) {
  *dst = nullptr;
  if (hipMalloc(dst, bytes) != hipSuccess)
    return fail(MING_ERR_ALLOC, "device allocation failed");
  const hipError_t e = hipMemcpyAsync(
      *dst, src, bytes,
      src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
      c->stream);
  if (e != hipSuccess) {
    (void)hipFree(*dst);
    *dst = nullptr;
    return hip_fail(e, "upload");
  }
  return MING_OK;
}

void destroy_qweight(ming_qweight* q) {
  if (!q) return;
  DeviceGuard g(q->ctx->device);
  (void)hipStreamSynchronize(q->ctx->stream);
  if (q->codes_t) (void)hipFree(q->codes_t);
  if (q->sb) (void)hipFree(q->sb);
  if (q->codes_f) (void)hipFree(q->codes_f);
  if (q->sbf) (void)hipFree(q->sbf);
  if (q->w16) (void)hipFree(q->w16);
  for (auto& sg : q->segs)
    for (auto& b : sg.slot) {
      if (b.A) (void)hipFree(b.A);
      if (b.B) (void)hipFree(b.B);
    }
  free_stacks(q);
  q->ctx->live_weights -= 1;
  delete q;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// ---- scratch of the entry point that allocates nothing (ming_lin_noalloc) --
// One array per GPU, resident for the life of the process. Host code never
// uses its name as an address (in host code it is only a stand-in symbol):
// each device's address is taken with hipGetSymbolAddress when the first
// context on that device is created, with the device current.
static __device__ __align__(256) unsigned char scratch[MING_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once (device current).
int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return fail(MING_ERR_ARG, "no-alloc scratch: device index out of range");
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (g_noalloc_ptr[device]) return MING_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(MING_ERR_HIP, std::string("no-alloc scratch: hipGetSymbolAddress failed: ") +
                                  hipGetErrorString(e));
  g_noalloc_ptr[device] = p;
  return MING_OK;
}

void* noalloc_ptr(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  return g_noalloc_ptr[device];
}

// The range word the kernels raise: on the fp16 routes (auto, general);
// the wide route converts nothing to fp16, and whatever fp16 copies the block
// driver still writes there are not read; nor are the copies a block of dense
// projections writes (those multiply bf16 activations).
int* range_word(const ming_ctx* c) {
  return c->route == MING_ROUTE_WIDE || c->copies_unread ? nullptr : c->range;
}

// Reads the range word after the stream has drained: raised means some
// projection input on an fp16 route was >= 2^16 in magnitude or not finite,
// and its fp16 copy did not hold it. Cleared, counted and reported.
int take_range_fault(ming_ctx* c, const char* who) {
  int h = 0;
  MING_HIP(hipMemcpyAsync(&h, c->range, sizeof(int), hipMemcpyDeviceToHost, c->stream),
           "range word read");
  MING_HIP(hipStreamSynchronize(c->stream), "range word read");
  if (h == 0) return MING_OK;
  MING_HIP(hipMemsetAsync(c->range, 0, sizeof(int), c->stream), "range word reset");
  c->eng.range_faults += 1;
  return fail(MING_ERR_RANGE,
              std::string(who) +
                  ": a projection input on an fp16 route had a value of magnitude >= 65536 "
                  "or not finite, which its fp16 copy cannot hold; the results since the "
                  "last synchronization are not valid (MING_ROUTE_WIDE computes such inputs "
                  "in bf16)");
}

}  // namespace

extern "C" {

const char* ming_last_error(void) { return g_err.c_str(); }
int ming_abi_version(void) { return MING_ABI_VERSION; }

void ming_set_log_sink(ming_log_fn fn, void* user) {
  std::lock_guard<std::mutex> g(g_log_mu);
  g_log_fn = fn;
  g_log_user = user;
}

int ming_ctx_create(int device, void* hip_stream, ming_ctx** out) {
  if (!out) return fail(MING_ERR_ARG, "ming_ctx_create: null out");
  *out = nullptr;
  int ndev = 0;
  MING_HIP(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
  if (device < 0 || device >= ndev)
    return fail(MING_ERR_ARG, "ming_ctx_create: no such device");
  DeviceGuard g(device);
  // Resolve and validate every kernel on this device; refuse, never degrade.
  hipError_t e = ming::validate_qproj_kernels();
  if (e == hipSuccess) e = ming::validate_norm_kernels();
  if (e == hipSuccess) e = ming::validate_elementwise_kernels();
  if (e == hipSuccess) e = ming::validate_qproj_fast_kernels();
  if (e == hipSuccess) e = ming::validate_gemv_kernels();
  if (e == hipSuccess) e = ming::validate_attention_kernels();
  if (e != hipSuccess)
    return fail(MING_ERR_KERNEL,
                std::string("kernel validation failed on this device (the "
                            "library is built for gfx950): ") +
                    hipGetErrorString(e));
  // the device's no-alloc scratch address (its array is resident already)
  {
    const int rc = noalloc_setup(device);
    if (rc != MING_OK) return rc;
  }
  auto* c = new (std::nothrow) ming_ctx();
  if (!c) return fail(MING_ERR_ALLOC, "ming_ctx_create: out of memory");
  c->device = device;
  if (hip_stream) {
    c->stream = (hipStream_t)hip_stream;
  } else {
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
      delete c;
      return fail(MING_ERR_HIP, "ming_ctx_create: stream creation failed");
    }
    c->own_stream = true;
  }
  if (hipMalloc(&c->range, 256) != hipSuccess ||
      hipMemsetAsync(c->range, 0, sizeof(int), c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess) {
    if (c->range) (void)hipFree(c->range);
    if (c->own_stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(MING_ERR_HIP, "ming_ctx_create: range word allocation failed");
  }
  *out = c;
  return ok();
}

int ming_ctx_destroy(ming_ctx* c) {
  if (!c) return ok();
  if (c->live_weights > 0)
    return fail(MING_ERR_STATE,
                "ming_ctx_destroy: destroy the context's weights and models first");
  DeviceGuard g(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->scratch) (void)hipFree(c->scratch);
  if (c->xh) (void)hipFree(c->xh);
  if (c->xh2) (void)hipFree(c->xh2);
  if (c->vt) (void)hipFree(c->vt);
  if (c->up) (void)hipFree(c->up);
  if (c->part) (void)hipFree(c->part);
  if (c->range) (void)hipFree(c->range);
  for (auto& rec : c->recs) {
    (void)hipEventDestroy(rec.a);
    (void)hipEventDestroy(rec.b);
  }
  for (auto e : c->pool) (void)hipEventDestroy(e);
  if (c->own_stream) (void)hipStreamDestroy(c->stream);
  delete c;
  return ok();
}

int ming_ctx_set_stream(ming_ctx* c, void* hip_stream) {
  if (!c) return fail(MING_ERR_ARG, "null context");
  DeviceGuard g(c->device);
  MING_HIP(hipStreamSynchronize(c->stream), "set_stream sync");
  if (c->own_stream) (void)hipStreamDestroy(c->stream);
  c->own_stream = false;
  c->stream = (hipStream_t)hip_stream;
  return ok();
}

void* ming_ctx_stream(const ming_ctx* c) { return c ? (void*)c->stream : nullptr; }

int ming_ctx_synchronize(ming_ctx* c) {
  if (!c) return fail(MING_ERR_ARG, "null context");
  DeviceGuard g(c->device);
  MING_HIP(hipStreamSynchronize(c->stream), "synchronize");
  const int rc = take_range_fault(c, "ming_ctx_synchronize");
  if (rc != MING_OK) return rc;
  return ok();
}

int ming_ctx_engagement(const ming_ctx* c, ming_engagement* out) {
  if (!c || !out) return fail(MING_ERR_ARG, "null argument");
  *out = c->eng;
  return ok();
}

int ming_ctx_reset_engagement(ming_ctx* c) {
  if (!c) return fail(MING_ERR_ARG, "null context");
  c->eng = ming_engagement{};
  return ok();
}

int ming_qweight_create(ming_ctx* c, int N, int K, int bits, int group,
                        const uint32_t* codes, const uint16_t* scales,
                        const uint16_t* biases, int src_on_device,
                        ming_qweight** out) {
  if (!c || !out || !codes || !scales || !biases)
    return fail(MING_ERR_ARG, "ming_qweight_create: null argument");
  *out = nullptr;
  if (bits != 4 && bits != 8)
    return fail(MING_ERR_SHAPE, "ming_qweight_create: bits must be 4 or 8");
  if (group != 64)
    return fail(MING_ERR_SHAPE, "ming_qweight_create: group must be 64");
  if (N <= 0 || K <= 0 || K % 64 != 0 || N % 8 != 0)
    return fail(MING_ERR_SHAPE,
                "ming_qweight_create: need K % 64 == 0 and N % 8 == 0");
  DeviceGuard g(c->device);
  auto* q = new (std::nothrow) ming_qweight();
  if (!q) return fail(MING_ERR_ALLOC, "out of memory");
  q->ctx = c; q->N = N; q->K = K; q->bits = bits; q->group = group;
  c->live_weights += 1;
  q->segs.resize(1);
  q->segs[0].N = N;
  const size_t words = (size_t)N * K * bits / 32;
  const size_t G = (size_t)K / 64;
  void *dc = nullptr, *ds = nullptr, *db = nullptr;
  int rc = upload(c, &dc, codes, words * 4, src_on_device);
  if (rc == MING_OK) rc = upload(c, &ds, scales, (size_t)N * G * 2, src_on_device);
  if (rc == MING_OK) rc = upload(c, &db, biases, (size_t)N * G * 2, src_on_device);
  hipError_t e = hipSuccess;
  if (rc == MING_OK) {
    int* flag = nullptr;
    e = hipMalloc(&q->codes_t, words * 4);
    if (e == hipSuccess) e = hipMalloc(&q->sb, (size_t)N * G * 4);
    if (e == hipSuccess) e = hipMalloc(&q->codes_f, words * 4);
    if (e == hipSuccess) e = hipMalloc(&q->sbf, (size_t)N * G * 4);
    if (e == hipSuccess) e = hipMalloc(&flag, sizeof(int));
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, sizeof(int), c->stream);
    if (e == hipSuccess)
      e = ming::launch_repack(bits, (const uint32_t*)dc, (const uint16_t*)ds,
                              (const uint16_t*)db, N, K, q->codes_t, q->sb,
                              c->stream);
    if (e == hipSuccess)
      e = ming::launch_repack_fast(bits, (const uint32_t*)dc, (const uint16_t*)ds,
                                   (const uint16_t*)db, N, K, q->codes_f, q->sbf,
                                   flag, c->stream);
    int inexact = 1;
    if (e == hipSuccess)
      e = hipMemcpyAsync(&inexact, flag, sizeof(int), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (flag) (void)hipFree(flag);
    q->fast = (e == hipSuccess && inexact == 0);
    if (e != hipSuccess) rc = hip_fail(e, "ming_qweight_create: repack");
  }
  if (dc) (void)hipFree(dc);
  if (ds) (void)hipFree(ds);
  if (db) (void)hipFree(db);
  if (rc != MING_OK) {
    destroy_qweight(q);
    return rc;
  }
  *out = q;
  return ok();
}

int ming_qweight_create_dense(ming_ctx* c, int N, int K, const uint16_t* w,
                              int src_on_device, ming_qweight** out) {
  if (!c || !out || !w)
    return fail(MING_ERR_ARG, "ming_qweight_create_dense: null argument");
  *out = nullptr;
  if (N <= 0 || K <= 0 || K % 64 != 0 || N % 8 != 0)
    return fail(MING_ERR_SHAPE,
                "ming_qweight_create_dense: need K % 64 == 0 and N % 8 == 0");
  DeviceGuard g(c->device);
  auto* q = new (std::nothrow) ming_qweight();
  if (!q) return fail(MING_ERR_ALLOC, "out of memory");
  q->ctx = c; q->N = N; q->K = K; q->bits = 16;
  c->live_weights += 1;
  q->segs.resize(1);
  q->segs[0].N = N;
  void* d = nullptr;
  int rc = upload(c, &d, w, (size_t)N * K * 2, src_on_device);
  if (rc == MING_OK && hipStreamSynchronize(c->stream) != hipSuccess)
    rc = fail(MING_ERR_HIP, "ming_qweight_create_dense: upload sync");
  q->w16 = (uint16_t*)d;
  if (rc != MING_OK) {
    destroy_qweight(q);
    return rc;
  }
  *out = q;
  return ok();
}

int ming_qweight_concat(ming_ctx* c, int n_parts, ming_qweight* const* parts,
                        ming_qweight** out) {
  if (!c || !out || !parts || n_parts <= 0)
    return fail(MING_ERR_ARG, "ming_qweight_concat: bad arguments");
  *out = nullptr;
  if (n_parts > ming::kMaxSeg)
    return fail(MING_ERR_SHAPE, "ming_qweight_concat: at most 4 parts");
  int N = 0;
  for (int i = 0; i < n_parts; ++i) {
    const ming_qweight* p = parts[i];
    if (!p) return fail(MING_ERR_ARG, "ming_qweight_concat: null part");
    if (p->ctx != c || p->K != parts[0]->K || p->bits != parts[0]->bits ||
        p->segs.size() != 1)
      return fail(MING_ERR_SHAPE,
                  "ming_qweight_concat: parts must be single projections of "
                  "one context with equal K and bits");
    if (i + 1 < n_parts && p->N % ming::kQpBN != 0)
      return fail(MING_ERR_SHAPE,
                  "ming_qweight_concat: every part but the last needs "
                  "N % 256 == 0");
    N += p->N;
  }
  DeviceGuard g(c->device);
  auto* q = new (std::nothrow) ming_qweight();
  if (!q) return fail(MING_ERR_ALLOC, "out of memory");
  q->ctx = c; q->N = N; q->K = parts[0]->K; q->bits = parts[0]->bits;
  c->live_weights += 1;
  const int K = q->K, bits = q->bits;
  hipStream_t s = c->stream;
  int rc = MING_OK;
  auto chk = [&](hipError_t e, const char* what) {
    if (rc == MING_OK && e != hipSuccess) rc = hip_fail(e, what);
  };
  if (bits == 16) {
    chk(hipMalloc(&q->w16, (size_t)N * K * 2), "concat alloc");
  } else {
    chk(hipMalloc(&q->codes_t, (size_t)N * K * bits / 8), "concat alloc");
    chk(hipMalloc(&q->sb, (size_t)N * (K / 64) * 4), "concat alloc");
    chk(hipMalloc(&q->codes_f, (size_t)N * K * bits / 8), "concat alloc");
    chk(hipMalloc(&q->sbf, (size_t)N * (K / 64) * 4), "concat alloc");
    q->fast = true;
    for (int i = 0; i < n_parts; ++i) q->fast = q->fast && parts[i]->fast;
  }
  q->segs.resize(n_parts);
  int nb = 0;
  const int KT = K / 64, wpr = bits == 4 ? 8 : 16;
  for (int i = 0; i < n_parts && rc == MING_OK; ++i) {
    const ming_qweight* p = parts[i];
    Segment& sg = q->segs[i];
    sg.n_begin = nb;
    sg.N = p->N;
    if (bits == 16) {
      chk(hipMemcpyAsync(q->w16 + (size_t)nb * K, p->w16, (size_t)p->N * K * 2,
                         hipMemcpyDeviceToDevice, s), "concat copy");
    } else {
      chk(hipMemcpy2DAsync(q->codes_t + (size_t)nb * wpr, (size_t)N * wpr * 4,
                           p->codes_t, (size_t)p->N * wpr * 4,
                           (size_t)p->N * wpr * 4, (size_t)KT,
                           hipMemcpyDeviceToDevice, s), "concat copy");
      chk(hipMemcpy2DAsync(q->sb + nb, (size_t)N * 4, p->sb, (size_t)p->N * 4,
                           (size_t)p->N * 4, (size_t)KT,
                           hipMemcpyDeviceToDevice, s), "concat copy");
      chk(hipMemcpy2DAsync(q->codes_f + (size_t)nb * wpr, (size_t)N * wpr * 4,
                           p->codes_f, (size_t)p->N * wpr * 4,
                           (size_t)p->N * wpr * 4, (size_t)KT,
                           hipMemcpyDeviceToDevice, s), "concat copy");
      chk(hipMemcpy2DAsync(q->sbf + nb, (size_t)N * 4, p->sbf, (size_t)p->N * 4,
                           (size_t)p->N * 4, (size_t)KT,
                           hipMemcpyDeviceToDevice, s), "concat copy");
    }
    for (int sl = 0; sl < MING_MAX_LORA_SLOTS && rc == MING_OK; ++sl) {
      const LoraBind& b = p->segs[0].slot[sl];
      if (b.rank <= 0) continue;
      LoraBind& d = sg.slot[sl];
      d.rank = b.rank; d.rank8 = b.rank8; d.fold = b.fold;
      chk(hipMalloc(&d.A, (size_t)b.rank8 * K * 2), "concat lora alloc");
      chk(hipMalloc(&d.B, (size_t)p->N * b.rank8 * 2), "concat lora alloc");
      if (rc != MING_OK) break;
      chk(hipMemcpyAsync(d.A, b.A, (size_t)b.rank8 * K * 2,
                         hipMemcpyDeviceToDevice, s), "concat lora copy");
      chk(hipMemcpyAsync(d.B, b.B, (size_t)p->N * b.rank8 * 2,
                         hipMemcpyDeviceToDevice, s), "concat lora copy");
    }
    nb += p->N;
  }
  chk(hipStreamSynchronize(s), "concat sync");
  if (rc != MING_OK) {
    destroy_qweight(q);
    return rc;
  }
  *out = q;
  return ok();
}

int ming_qweight_destroy(ming_qweight* q) {
  destroy_qweight(q);
  return ok();
}

int ming_qweight_bits(const ming_qweight* q) { return q ? q->bits : 0; }

int ming_qweight_shape(const ming_qweight* q, int* N, int* K, int* n_segments) {
  if (!q) return fail(MING_ERR_ARG, "null weight");
  if (N) *N = q->N;
  if (K) *K = q->K;
  if (n_segments) *n_segments = (int)q->segs.size();
  return ok();
}

int ming_qweight_bind_lora(ming_qweight* q, int segment, int slot, int rank,
                           const uint16_t* A, const uint16_t* B, float fold,
                           int src_on_device) {
  if (!q || !A || !B) return fail(MING_ERR_ARG, "bind_lora: null argument");
  if (segment < 0 || segment >= (int)q->segs.size())
    return fail(MING_ERR_ARG, "bind_lora: no such segment");
  if (slot < 0 || slot >= MING_MAX_LORA_SLOTS)
    return fail(MING_ERR_ARG, "bind_lora: slot out of range");
  if (rank <= 0 || rank > MING_MAX_LORA_RANK)
    return fail(MING_ERR_SHAPE, "bind_lora: rank out of range");
  ming_ctx* c = q->ctx;
  DeviceGuard g(c->device);
  Segment& sg = q->segs[segment];
  const int r8 = round_up(rank, 8);
  const size_t K = (size_t)q->K;
  LoraBind nb;
  nb.rank = rank; nb.rank8 = r8; nb.fold = fold;
  if (hipMalloc(&nb.A, (size_t)r8 * K * 2) != hipSuccess ||
      hipMalloc(&nb.B, (size_t)sg.N * r8 * 2) != hipSuccess) {
    if (nb.A) (void)hipFree(nb.A);
    if (nb.B) (void)hipFree(nb.B);
    return fail(MING_ERR_ALLOC, "bind_lora: allocation failed");
  }
  const hipMemcpyKind kind =
      src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  hipError_t e = hipMemsetAsync(nb.A, 0, (size_t)r8 * K * 2, c->stream);
  if (e == hipSuccess) e = hipMemsetAsync(nb.B, 0, (size_t)sg.N * r8 * 2, c->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(nb.A, A, (size_t)rank * K * 2, kind, c->stream);
  if (e == hipSuccess)
    e = hipMemcpy2DAsync(nb.B, (size_t)r8 * 2, B, (size_t)rank * 2,
                         (size_t)rank * 2, (size_t)sg.N, kind, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    (void)hipFree(nb.A);
    (void)hipFree(nb.B);
    return hip_fail(e, "bind_lora: upload");
  }
  LoraBind& old = sg.slot[slot];
  if (old.A) (void)hipFree(old.A);
  if (old.B) (void)hipFree(old.B);
  old = nb;
  q->stacks_dirty = true;
  ++q->bind_gen;
  return ok();
}

int ming_qweight_unbind_lora(ming_qweight* q, int segment, int slot) {
  if (!q) return fail(MING_ERR_ARG, "unbind_lora: null weight");
  if (segment < 0 || segment >= (int)q->segs.size() || slot < 0 ||
      slot >= MING_MAX_LORA_SLOTS)
    return fail(MING_ERR_ARG, "unbind_lora: out of range");
  DeviceGuard g(q->ctx->device);
  (void)hipStreamSynchronize(q->ctx->stream);
  LoraBind& b = q->segs[segment].slot[slot];
  if (b.A) (void)hipFree(b.A);
  if (b.B) (void)hipFree(b.B);
  b = LoraBind{};
  q->stacks_dirty = true;
  ++q->bind_gen;
  return ok();
}

int ming_qweight_lora_rank(const ming_qweight* q, int segment, int slot) {
  if (!q || segment < 0 || segment >= (int)q->segs.size() || slot < 0 ||
      slot >= MING_MAX_LORA_SLOTS)
    return 0;
  return q->segs[segment].slot[slot].rank;
}

// One projection's output side: y [M][ldy]; `gate` fuses SwiGLU into the
// output (y = bf16(silu(gate) * bf16(lin(x)))); `yh`, when set, receives an
// fp16 copy of the output (row stride N) from the fast route's epilogue;
// *took_fast reports whether the fast route ran (only then was `yh` written).
struct LinOut {
  uint16_t* y = nullptr;
  int64_t ldy = 0;
  const uint16_t* gate = nullptr;
  int64_t ldg = 0;
  uint16_t* yh = nullptr;
  bool* took_fast = nullptr;
  const uint16_t* bias = nullptr;   // dense weights only (ming_lin_bias)
};

// n projections over the same x [M][K] (q, k, v; w1, w3): x is converted to
// fp16 once for all of them (`xh_src`, when set, is that copy already made,
// row stride K), and every live adapter of every one of them goes into ONE
// stacked x.A launch -- the stacks' 8-rank groups side by side in T, group
// entries naming their weight -- before each projection's GEMM reads its own
// columns of T. n == 1 is lin() (ming-dit.cc:1763-1771).
// Where one call's scratch comes from: the context's buffers, grown on
// demand (every entry point but one), or regions carved from the device's
// static no-alloc array (ming_lin_noalloc), sized before anything launches.
struct Carve {
  char* base = nullptr;
  size_t cap = 0, used = 0;
  static size_t aligned256(size_t b) { return (b + 255) & ~(size_t)255; }
  // a 256-byte-aligned region of `bytes` (callers check the total first)
  void* take(size_t bytes) {
    void* p = base + used;
    used += aligned256(bytes);
    return p;
  }
};

static int lin_multi(ming_ctx* c, int n, const ming_qweight* const* qs, const LinOut* outs,
                     const uint16_t* x, int64_t ldx, int M, const float* scales,
                     const uint16_t* xh_src, Carve* carve = nullptr) {
  for (int i = 0; i < n; ++i)
    if (outs[i].took_fast) *outs[i].took_fast = false;
  if (!c || !x || n < 1 || n > ming::kMaxXaSources)
    return fail(MING_ERR_ARG, "ming_lin: null argument");
  if (M < 0) return fail(MING_ERR_ARG, "ming_lin: M < 0");
  if (!aligned(x, 16)) return fail(MING_ERR_ARG, "ming_lin: x must be 16-byte and y 8-byte aligned");
  const int K = qs[0] ? qs[0]->K : 0;
  for (int i = 0; i < n; ++i) {
    const ming_qweight* q = qs[i];
    const LinOut& o = outs[i];
    if (!q || !o.y) return fail(MING_ERR_ARG, "ming_lin: null argument");
    if (q->ctx != c) return fail(MING_ERR_ARG, "ming_lin: weight of another context");
    if (q->K != K) return fail(MING_ERR_SHAPE, "ming_lin: projections over one x need one K");
    if (ldx < q->K || o.ldy < q->N || ldx % 8 != 0 || o.ldy % 4 != 0)
      return fail(MING_ERR_SHAPE,
                  "ming_lin: need ldx >= K, ldx % 8 == 0, ldy >= N, ldy % 4 == 0");
    if (!aligned(o.y, 8))
      return fail(MING_ERR_ARG, "ming_lin: x must be 16-byte and y 8-byte aligned");
    if (o.gate && (o.ldg < q->N || o.ldg % 8 != 0 || !aligned(o.gate, 16) || o.ldy % 8 != 0 ||
                   !aligned(o.y, 16)))
      return fail(MING_ERR_SHAPE,
                  "ming_lin_swiglu: gate and output need strides % 8 == 0 and 16-byte "
                  "alignment (ldg >= N)");
  }
  if (M == 0) return ok();
  DeviceGuard g(c->device);

  // A handful of rows and no live adapter (the adaLN and timestep
  // projections run at M = 1): the GEMV streams each weight once instead of
  // running a 256-row tile. It reads bf16 x in f32, so any route but the
  // general one takes it.
  if (c->route != MING_ROUTE_GENERAL && M <= ming::kGemvMaxM) {
    bool gemv = true;
    for (int i = 0; i < n && gemv; ++i) {
      const ming_qweight* q = qs[i];
      if (outs[i].gate || outs[i].yh) gemv = false;
      for (const Segment& sg : q->segs)
        for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl)
          if (sg.slot[sl].rank > 0 && scales && scales[sl] != 0.0f) gemv = false;
    }
    if (gemv) {
      for (int i = 0; i < n; ++i) {
        const ming_qweight* q = qs[i];
        const ming::GemvArgs ga{x, ldx, q->codes_t, q->sb, q->w16, outs[i].y, outs[i].ldy,
                                M, q->N, K, outs[i].bias};
        const double wbytes = q->bits == 16
                                  ? 2.0 * q->N * K
                                  : (double)q->N * K * q->bits / 8 + 4.0 * q->N * (K / 64);
        MING_HIP(profiled(c, kBGemv, 2.0 * M * (double)q->N * K,
                          wbytes + 2.0 * M * K + 2.0 * M * q->N,
                          [&] { return ming::launch_gemv(q->bits, ga, c->stream); }),
                 "gemv launch");
        if (q->bits == 4) c->eng.gemm_q4 += 1;
        else if (q->bits == 8) c->eng.gemm_q8 += 1;
        else c->eng.gemm_dense += 1;
        c->eng.gemv += 1;
        c->eng.gemm_flops += 2ull * (uint64_t)M * (uint64_t)q->N * (uint64_t)K;
      }
      return ok();
    }
  }

  // ---- plan: the live stacks, the routes, and every scratch size --------
  // The live stacks, per weight and segment, in slot order.
  ming::QprojArgs qa[ming::kMaxXaSources] = {};
  ming::LoraXaArgs xa{};
  int xa_groups = 0;   // 8-wide groups of T over every weight and segment
  uint64_t lora_flops[ming::kMaxXaSources] = {};
  int live_segs[ming::kMaxXaSources] = {};
  int qp_used[ming::kMaxXaSources] = {};   // entries of qa[i].grp in use
  double xa_flops = 0.0, tail_flops[ming::kMaxXaSources] = {};
  bool xa_fits = true;
  for (int i = 0; i < n; ++i) {
    ming_qweight* q = const_cast<ming_qweight*>(qs[i]);
    const int nseg = (int)q->segs.size();
    bool any_live = false;
    for (int si = 0; si < nseg; ++si)
      for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl)
        if (q->segs[si].slot[sl].rank > 0 && scales && scales[sl] != 0.0f) any_live = true;
    if (any_live) {
      if (carve && q->stacks_dirty)
        return fail(MING_ERR_STATE,
                    "ming_lin_noalloc: the weight's adapter stacks are not built since its "
                    "last binding change (one ming_lin call builds them)");
      int rc = build_stacks(q);
      if (rc != MING_OK) return rc;
      xa.A[i] = q->A_all;
      if ((uint64_t)q->a_rows * (uint64_t)q->K * 2 > (1ull << 31)) xa_fits = false;
    }
    int qp_groups = 0;
    for (int si = 0; si < nseg; ++si) {
      const Segment& sg = q->segs[si];
      ming::QprojSeg& d = qa[i].seg[si];
      d.n_begin = sg.n_begin;
      d.n_end = sg.n_begin + sg.N;
      d.t_col0 = xa_groups * 8;
      d.grp0 = qp_groups;
      d.chunks = 0;
      d.ldb = any_live ? q->b_ld[si] : 0;
      d.B = any_live ? q->B_seg[si] : nullptr;
      int seg_groups = 0;
      for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl) {
        const LoraBind& b = sg.slot[sl];
        if (b.rank <= 0 || !scales || scales[sl] == 0.0f) continue;
        const int ar = q->a_row0[si * MING_MAX_LORA_SLOTS + sl];
        const int bc = q->b_col0[si * MING_MAX_LORA_SLOTS + sl];
        for (int gi = 0; gi < b.rank8 / 8; ++gi) {
          if (xa_groups + seg_groups >= ming::kMaxGroups ||
              qp_groups + seg_groups >= ming::kMaxGroups)
            return fail(MING_ERR_SHAPE, "ming_lin: live adapter ranks exceed 4096");
          xa.grp[xa_groups + seg_groups] = (int16_t)((i << 12) | (ar / 8 + gi));
          xa.coef[xa_groups + seg_groups] = b.fold * scales[sl];
          qa[i].grp[qp_groups + seg_groups] = (int16_t)(bc / 8 + gi);
          ++seg_groups;
        }
        lora_flops[i] += 2ull * (uint64_t)M * (uint64_t)b.rank * (uint64_t)(q->K + sg.N);
        xa_flops += 2.0 * M * b.rank * (double)q->K;
        tail_flops[i] += 2.0 * M * b.rank * (double)sg.N;
      }
      if (seg_groups == 0) continue;
      ++live_segs[i];
      // pad the segment's T columns to whole 32-rank chunks with zero groups
      const int padded = round_up(seg_groups, 4);
      for (int gi = seg_groups; gi < padded; ++gi) {
        if (xa_groups + gi >= ming::kMaxGroups || qp_groups + gi >= ming::kMaxGroups)
          return fail(MING_ERR_SHAPE, "ming_lin: live adapter ranks exceed 4096");
        xa.grp[xa_groups + gi] = -1;
        xa.coef[xa_groups + gi] = 0.0f;
        qa[i].grp[qp_groups + gi] = -1;
      }
      d.chunks = padded / 4;
      xa_groups += padded;
      qp_groups += padded;
    }
    qp_used[i] = qp_groups;
  }
  // the x.A kernels write T in 64-column blocks: zero groups after the last
  // segment make the stack a whole number of them
  while (xa_groups % 8 != 0) {
    if (xa_groups >= ming::kMaxGroups)
      return fail(MING_ERR_SHAPE, "ming_lin: live adapter ranks exceed 4096");
    xa.grp[xa_groups] = -1;
    xa.coef[xa_groups] = 0.0f;
    ++xa_groups;
  }
  const int t_cols = xa_groups * 8;
  // the fast x.A addresses x and each A stack as 64-bit bases plus 32-bit
  // byte offsets; its K split (slices summed in f32 by a second launch)
  const bool xa_fast = t_cols > 0 && c->route != MING_ROUTE_GENERAL && ldx % 8 == 0 &&
                       (uint64_t)M * (uint64_t)ldx * 2 <= (1ull << 31) && xa_fits;
  const int xa_ks = xa_fast ? ming::lora_xa_fast_slices(M, t_cols, K) : 1;
  size_t part_bytes = ming::lora_xa_part_bytes(M, t_cols, xa_ks);
  // Which projections take the fast route. It addresses each operand as a
  // 64-bit base plus 32-bit byte offsets: x (fp16 copy, row stride K), T and
  // every B stack must fit.
  bool fast[ming::kMaxXaSources] = {};
  bool any_fast = false;
  for (int i = 0; i < n; ++i) {
    const ming_qweight* q = qs[i];
    bool fits32 = (uint64_t)M * (uint64_t)K * 2 <= (1ull << 31) &&
                  (uint64_t)M * (uint64_t)t_cols * 2 <= (1ull << 31);
    for (int si = 0; si < (int)q->segs.size() && t_cols > 0; ++si)
      if (qa[i].seg[si].chunks > 0 &&
          (uint64_t)q->segs[si].N * (uint64_t)q->b_ld[si] * 2 > (1ull << 31))
        fits32 = false;
    fast[i] = q->bits != 16 && q->fast && c->route == MING_ROUTE_AUTO && fits32;
    any_fast = any_fast || fast[i];
  }
  // Per projection: the fast route's K split on few tiles (the context
  // refiner's 256 caption rows: 15 or 40 tiles), about one round of the
  // chip at >= 6 K steps a slice; a dense weight with no live adapter on few
  // 256 x 256 tiles (the caption embedder: 15; the final layer's 64
  // columns: 16) runs as the x.A path's split-K bf16 GEMM (identity column
  // groups, coefficient 1); the general route writes a gated projection into
  // a plane of its own first, since y may be the gate itself.
  int split_ks[ming::kMaxXaSources] = {};
  int dense_ks[ming::kMaxXaSources] = {};
  size_t up_bytes = 0;
  for (int i = 0; i < n; ++i) {
    const ming_qweight* q = qs[i];
    const LinOut& o = outs[i];
    const int tiles = ((M + 255) / 256) * ((q->N + 255) / 256);
    if (fast[i] && tiles < 64 && c->route == MING_ROUTE_AUTO && q->N % 4 == 0) {
      int ks = 256 / tiles;
      if (ks > (K / 64) / 6) ks = (K / 64) / 6;
      if (ks >= 2) {
        split_ks[i] = ks;
        part_bytes = std::max(part_bytes, (size_t)ks * M * q->N * 4);
      }
    }
    const bool dense_sk =
        q->bits == 16 && c->route != MING_ROUTE_GENERAL && live_segs[i] == 0 && !o.gate &&
        !o.yh && tiles < 64 && q->N % 64 == 0 && q->N <= 8 * ming::kMaxGroups &&
        K % 64 == 0 && o.ldy <= (1 << 30) && (uint64_t)M * (uint64_t)ldx * 2 <= (1ull << 31) &&
        (uint64_t)q->N * (uint64_t)K * 2 <= (1ull << 31);
    if (dense_sk) {
      dense_ks[i] = ming::dense_xa_slices(M, q->N, K);
      part_bytes = std::max(part_bytes, ming::lora_xa_part_bytes(M, q->N, dense_ks[i]));
    }
    if (o.gate && !fast[i]) up_bytes = std::max(up_bytes, (size_t)M * q->N * 2);
  }
  // A SwiGLU's gate and up projections (the second gated by the first's
  // output, as ming_ffn runs w1 and w3) on the fast route run as one launch:
  // each tile computes 128 columns of both, and only the SwiGLU leaves the
  // chip. Same bits as the two launches. It needs one segment per weight,
  // the same number of LoRA tail chunks, no K split, and room for both
  // group tables in one.
  const bool pair = n == 2 && outs[1].gate && outs[1].gate == outs[0].y &&
                    outs[1].ldg == outs[0].ldy && !outs[0].gate && !outs[0].yh && fast[0] &&
                    fast[1] && split_ks[0] == 0 && split_ks[1] == 0 &&
                    qs[0]->bits == qs[1]->bits && qs[0]->N == qs[1]->N && qs[0]->N % 8 == 0 &&
                    outs[1].ldy % 8 == 0 && aligned(outs[1].y, 16) &&
                    (!outs[1].yh || aligned(outs[1].yh, 16)) &&
                    qs[0]->segs.size() == 1 && qs[1]->segs.size() == 1 &&
                    qa[0].seg[0].chunks == qa[1].seg[0].chunks &&
                    qp_used[0] + qp_used[1] <= ming::kMaxGroups;
  // The fast route reads x as fp16 carrying the same (bf16) values: one
  // conversion serves every projection here.
  const bool need_xh = any_fast && !xh_src;
  const size_t t_bytes = (size_t)M * t_cols * 2, xh_bytes = need_xh ? (size_t)M * K * 2 : 0;

  // ---- acquire: every scratch region before the first launch ------------
  uint16_t* T = nullptr;
  float* part = nullptr;
  uint16_t* up = nullptr;
  const uint16_t* xh = xh_src;
  if (carve) {
    if (up_bytes > 0) return fail(MING_ERR_ARG, "ming_lin_noalloc: no gated projection");
    const size_t need = Carve::aligned256(t_bytes) + Carve::aligned256(xh_bytes) +
                        Carve::aligned256(part_bytes);
    if (need > carve->cap - carve->used)
      return fail(MING_ERR_SHAPE,
                  "ming_lin_noalloc: the call needs " + std::to_string(need) +
                      " bytes of scratch; the no-alloc array holds " +
                      std::to_string(carve->cap) + " (MING_NOALLOC_SCRATCH_BYTES)");
    if (t_bytes) T = (uint16_t*)carve->take(t_bytes);
    if (xh_bytes) xh = (const uint16_t*)carve->take(xh_bytes);
    if (part_bytes) part = (float*)carve->take(part_bytes);
  } else {
    int rc = MING_OK;
    if (t_bytes) rc = ensure_scratch(c, t_bytes);
    if (rc == MING_OK && part_bytes) rc = ensure_part(c, part_bytes);
    if (rc == MING_OK && xh_bytes) rc = ensure_xh(c, xh_bytes);
    if (rc == MING_OK && up_bytes) rc = ensure_up(c, up_bytes);
    if (rc != MING_OK) return rc;
    if (t_bytes) T = (uint16_t*)c->scratch;
    if (xh_bytes) xh = (const uint16_t*)c->xh;
    if (part_bytes) part = (float*)c->part;
    if (up_bytes) up = (uint16_t*)c->up;
  }

  // ---- launch ------------------------------------------------------------
  // The fast x.A stages every element of x through LDS: its DMA waves
  // write the fp16 copy as they go, in place of the conversion launch.
  const bool xh_in_xa = need_xh && t_cols > 0 && xa_fast;
  if (t_cols > 0) {
    xa.x = x; xa.ldx = ldx; xa.K = K; xa.M = M;
    xa.n_cols = t_cols; xa.t = T; xa.ldt = t_cols;
    if (xh_in_xa) {
      xa.xh = const_cast<uint16_t*>(xh);
      xa.ldxh = K;
      xa.range = range_word(c);
    }
    double a_bytes = 0.0;
    for (int i = 0; i < n; ++i)
      if (xa.A[i]) a_bytes += 2.0 * qs[i]->a_rows * (double)K;
    MING_HIP(profiled(c, kBXa, xa_flops,
                      2.0 * M * K + a_bytes + 2.0 * M * t_cols + (xh_in_xa ? 2.0 * M * K : 0.0),
                      [&] {
                        return xa_fast ? ming::launch_lora_xa_fast(xa, part, xa_ks, c->stream)
                                       : ming::launch_lora_xa(xa, c->stream);
                      }),
             "lora_xa launch");
    c->eng.lora_xa += 1;
  }
  if (need_xh && !xh_in_xa) {
    uint16_t* dst = const_cast<uint16_t*>(xh);
    MING_HIP(profiled(c, kBCvt, 0.0, 4.0 * M * K,
                      [&] { return ming::launch_bf16_to_f16(x, ldx, dst, K, M, K,
                                                            c->stream, range_word(c)); }),
             "bf16->fp16 launch");
  }
  if (pair) {
    const ming_qweight* q = qs[0];
    const ming_qweight* u = qs[1];
    const LinOut& o = outs[1];
    ming::QprojArgs& a = qa[0];
    a.x = xh; a.ldx = K; a.codes = q->codes_f; a.sb = q->sbf; a.w16 = nullptr;
    a.y = o.y; a.ldy = o.ldy; a.M = M; a.N = q->N; a.K = K;
    a.t = T; a.ldt = t_cols > 0 ? t_cols : 0; a.nseg = 1;
    a.g = nullptr; a.ldg = 0;
    a.yh = o.yh; a.ldyh = q->N;
    a.range = range_word(c);
    a.codes_u = u->codes_f; a.sb_u = u->sbf;
    a.seg_u = qa[1].seg[0];
    a.seg_u.grp0 += qp_used[0];
    for (int gi = 0; gi < qp_used[1]; ++gi) a.grp[qp_used[0] + gi] = qa[1].grp[gi];
    const double flops = 2.0 * 2.0 * M * (double)q->N * K + tail_flops[0] + tail_flops[1];
    const double wbytes = 2.0 * ((double)q->N * K * q->bits / 8 + 4.0 * q->N * (K / 64));
    MING_HIP(profiled(c, q->bits == 4 ? kBP4 : kBP8, flops,
                      2.0 * M * K + wbytes + 2.0 * M * q->N,
                      [&] { return ming::launch_qproj_pair(q->bits, a, c->stream); }),
             "qproj pair launch");
    for (int i = 0; i < 2; ++i) {
      if (outs[i].took_fast) *outs[i].took_fast = true;
      c->eng.gemm_fast += 1;
      if (qs[i]->bits == 4) c->eng.gemm_q4 += 1;
      else c->eng.gemm_q8 += 1;
      c->eng.lora_proj += live_segs[i];
      c->eng.gemm_flops +=
          2ull * (uint64_t)M * (uint64_t)qs[i]->N * (uint64_t)K + lora_flops[i];
    }
    c->eng.elementwise += 1;
    c->eng.gemm_paired += 1;
    return ok();
  }
  for (int i = 0; i < n; ++i) {
    const ming_qweight* q = qs[i];
    const LinOut& o = outs[i];
    ming::QprojArgs& a = qa[i];
    a.x = x; a.ldx = ldx; a.codes = q->codes_t; a.sb = q->sb; a.w16 = q->w16;
    a.y = o.y; a.ldy = o.ldy; a.M = M; a.N = q->N; a.K = K;
    a.t = T; a.ldt = t_cols > 0 ? t_cols : 0; a.nseg = (int)q->segs.size();
    a.g = nullptr; a.ldg = 0;
    a.yh = nullptr; a.ldyh = 0;
    a.range = range_word(c);
    a.bias = o.bias;   // set for dense weights only: the general kernel adds it
    if (o.gate && !fast[i]) {
      a.y = up; a.ldy = q->N;
    }
    if (fast[i]) {
      a.x = xh; a.ldx = K; a.codes = q->codes_f; a.sb = q->sbf;
      a.g = o.gate; a.ldg = o.ldg;     // the fast epilogue fuses SwiGLU
      a.yh = o.yh; a.ldyh = q->N;      // and writes the fp16 copy the next projection reads
      if (split_ks[i] >= 2) {
        a.part = part;
        a.kslices = split_ks[i];
      }
    }
    const double base_flops = 2.0 * M * (double)q->N * K;
    const double wbytes = q->bits == 16
                              ? 2.0 * q->N * K
                              : (double)q->N * K * q->bits / 8 + 4.0 * q->N * (K / 64);
    const int bk = fast[i] ? (q->bits == 4 ? kBF4 : kBF8)
                           : (q->bits == 4 ? kBQ4 : (q->bits == 8 ? kBQ8 : kBDense));
    if (dense_ks[i] > 0) {
      ming::LoraXaArgs da{};
      da.x = x; da.ldx = ldx; da.A[0] = q->w16; da.K = K; da.M = M;
      da.n_cols = q->N; da.t = o.y; da.ldt = (int)o.ldy; da.bias = o.bias;
      for (int gi = 0; gi < q->N / 8; ++gi) {
        da.grp[gi] = (int16_t)gi;
        da.coef[gi] = 1.0f;
      }
      const int dks = dense_ks[i];
      MING_HIP(profiled(c, bk, base_flops, 2.0 * M * K + wbytes + 2.0 * M * q->N,
                        [&] { return ming::launch_lora_xa_fast(da, part, dks, c->stream); }),
               "dense split-K launch");
    } else {
      MING_HIP(profiled(c, bk, base_flops + tail_flops[i],
                        2.0 * M * K + wbytes + 2.0 * M * q->N,
                        [&] {
                          return fast[i] ? ming::launch_qproj_fast(q->bits, a, c->stream)
                                         : ming::launch_qproj(q->bits, a, c->stream,
                                                              c->route == MING_ROUTE_WIDE);
                        }),
               "qproj launch");
    }
    if (o.gate && !fast[i]) {
      // the general route writes the projection; SwiGLU follows
      MING_HIP(profiled(c, kBSwiglu, 0.0, 6.0 * M * q->N,
                        [&] { return ming::launch_swiglu(o.gate, o.ldg, up, q->N, o.y,
                                                         o.ldy, M, q->N, c->stream); }),
               "swiglu launch");
    }
    if (o.gate) c->eng.elementwise += 1;
    if (o.took_fast) *o.took_fast = fast[i];
    if (fast[i]) c->eng.gemm_fast += 1;
    if (fast[i] && a.kslices >= 2) c->eng.gemm_split += 1;
    if (q->bits == 4) c->eng.gemm_q4 += 1;
    else if (q->bits == 8) c->eng.gemm_q8 += 1;
    else c->eng.gemm_dense += 1;
    c->eng.lora_proj += live_segs[i];
    c->eng.gemm_flops += 2ull * (uint64_t)M * (uint64_t)q->N * (uint64_t)K + lora_flops[i];
  }
  return ok();
}

// One projection (see LinOut, lin_multi).
static int lin_impl(ming_ctx* c, const ming_qweight* qc, const uint16_t* x,
                    int64_t ldx, uint16_t* y, int64_t ldy, int M,
                    const float* scales, const uint16_t* gate, int64_t ldg,
                    const uint16_t* xh_src, bool* took_fast, uint16_t* yh = nullptr) {
  if (!qc) {
    if (took_fast) *took_fast = false;
    return fail(MING_ERR_ARG, "ming_lin: null argument");
  }
  LinOut o;
  o.y = y; o.ldy = ldy; o.gate = gate; o.ldg = ldg; o.yh = yh; o.took_fast = took_fast;
  return lin_multi(c, 1, &qc, &o, x, ldx, M, scales, xh_src);
}

int ming_lin(ming_ctx* c, const ming_qweight* qc, const uint16_t* x,
             int64_t ldx, uint16_t* y, int64_t ldy, int M,
             const float* scales) {
  return lin_impl(c, qc, x, ldx, y, ldy, M, scales, nullptr, 0, nullptr, nullptr);
}

int ming_lin_bias(ming_ctx* c, const ming_qweight* qc, const uint16_t* x, int64_t ldx,
                  uint16_t* y, int64_t ldy, int M, const float* scales, const uint16_t* bias) {
  if (!c || !qc || !bias) return fail(MING_ERR_ARG, "ming_lin_bias: null argument");
  if (qc->bits != 16)
    return fail(MING_ERR_ARG,
                "ming_lin_bias: the bias is for dense (bf16) weights, as LlmOps::linear's; "
                "a quantized weight takes ming_lin and ming_bias_act");
  if (!aligned(bias, 2)) return fail(MING_ERR_ARG, "ming_lin_bias: bias must be 2-byte aligned");
  LinOut o;
  o.y = y;
  o.ldy = ldy;
  o.bias = bias;
  return lin_multi(c, 1, &qc, &o, x, ldx, M, scales, nullptr);
}

int ming_lin_noalloc(ming_ctx* c, const ming_qweight* qc, const uint16_t* x,
                     int64_t ldx, uint16_t* y, int64_t ldy, int M, const float* scales) {
  if (!c || !qc) return fail(MING_ERR_ARG, "ming_lin_noalloc: null argument");
  void* base = noalloc_ptr(c->device);
  if (!base)
    return fail(MING_ERR_STATE, "ming_lin_noalloc: the device has no scratch address");
  Carve cv;
  cv.base = static_cast<char*>(base);
  cv.cap = MING_NOALLOC_SCRATCH_BYTES;
  struct NoEvents {
    ming_ctx* c;
    bool was;
    ~NoEvents() { c->no_events = was; }
  } ne{c, c->no_events};
  c->no_events = true;
  LinOut o;
  o.y = y;
  o.ldy = ldy;
  return lin_multi(c, 1, &qc, &o, x, ldx, M, scales, nullptr, &cv);
}

int ming_lin_swiglu(ming_ctx* c, const ming_qweight* w, const uint16_t* x,
                    int64_t ldx, const uint16_t* g, int64_t ldg, uint16_t* out,
                    int64_t ldo, int M, const float* scales) {
  if (!g) return fail(MING_ERR_ARG, "ming_lin_swiglu: null gate");
  return lin_impl(c, w, x, ldx, out, ldo, M, scales, g, ldg, nullptr, nullptr);
}

// gpu_ff; xh_ready: the context's fp16 copy already holds x (row stride H).
static int ffn_impl(ming_ctx* c, const ming_qweight* w1, const ming_qweight* w3,
                    const ming_qweight* w2, const uint16_t* x, int64_t ldx, uint16_t* y,
                    int64_t ldy, int M, const float* scales, uint16_t* h, int64_t ldh,
                    bool xh_ready) {
  if (!c || !w1 || !w3 || !w2 || !x || !y || !h)
    return fail(MING_ERR_ARG, "ming_ffn: null argument");
  const int F = w1->N, H = w1->K;
  if (w3->N != F || w3->K != H || w2->N != H || w2->K != F)
    return fail(MING_ERR_SHAPE, "ming_ffn: need w1, w3 [ffn][H] and w2 [H][ffn]");
  if (ldh < F || ldh % 8 != 0 || !aligned(h, 16))
    return fail(MING_ERR_SHAPE, "ming_ffn: h needs ldh >= ffn, ldh % 8 == 0, 16-byte alignment");
  // w1 and w3 read the same x: one fp16 conversion and one x.A launch for
  // both. w3's epilogue fuses the SwiGLU (gate = w1's output, in place) and
  // writes the fp16 copy of h that w2 reads, into a buffer of its own (w3's
  // other tiles still read x from the first).
  if (M > 0) {
    int rc = ensure_xh2(c, (size_t)M * F * 2);
    if (rc != MING_OK) return rc;
  }
  bool fast3 = false;
  const ming_qweight* pair[2] = {w1, w3};
  LinOut outs[2];
  outs[0].y = h; outs[0].ldy = ldh;
  outs[1].y = h; outs[1].ldy = ldh; outs[1].gate = h; outs[1].ldg = ldh;
  outs[1].yh = (uint16_t*)c->xh2; outs[1].took_fast = &fast3;
  int rc = lin_multi(c, 2, pair, outs, x, ldx, M, scales,
                     xh_ready ? (const uint16_t*)c->xh : nullptr);
  if (rc != MING_OK) return rc;
  return lin_impl(c, w2, h, ldh, y, ldy, M, scales, nullptr, 0,
                  fast3 ? (const uint16_t*)c->xh2 : nullptr, nullptr);
}

int ming_ffn(ming_ctx* c, const ming_qweight* w1, const ming_qweight* w3,
             const ming_qweight* w2, const uint16_t* x, int64_t ldx, uint16_t* y,
             int64_t ldy, int M, const float* scales, uint16_t* h, int64_t ldh) {
  return ffn_impl(c, w1, w3, w2, x, ldx, y, ldy, M, scales, h, ldh, false);
}

// The RMSNorm kernel's modes (see rmsnorm_kernel): 0 plain; 1 also the
// context's fp16 copy of y; 2 / 3 post-norm fused into the gated / plain
// residual h += (tanh(gate) *) y.
static int rms_impl(ming_ctx* c, int mode, const uint16_t* x, int64_t ldx,
                    const uint16_t* w, uint16_t* y, int64_t ldy, uint16_t* h,
                    int64_t ldh, const float* gate, int rows, int D, float eps,
                    const char* who) {
  if (!c || !x || !w || (mode <= 1 && !y) || (mode >= 2 && !h) || (mode == 2 && !gate))
    return fail(MING_ERR_ARG, std::string(who) + ": null argument");
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 8192)
    return fail(MING_ERR_SHAPE, std::string(who) + ": need D % 8 == 0 and D <= 8192");
  if (ldx < D || ldx % 8 != 0 || (mode <= 1 && (ldy < D || ldy % 8 != 0)) ||
      (mode >= 2 && (ldh < D || ldh % 8 != 0)))
    return fail(MING_ERR_SHAPE, std::string(who) + ": bad row strides");
  if (!aligned(x, 16) || !aligned(w, 16) || (mode <= 1 && !aligned(y, 16)) ||
      (mode >= 2 && !aligned(h, 16)) || (mode == 2 && !aligned(gate, 16)))
    return fail(MING_ERR_ARG, std::string(who) + ": pointers must be 16-byte aligned");
  if (rows == 0) return ok();
  DeviceGuard g(c->device);
  if (mode == 1) {
    int rc = ensure_xh(c, (size_t)rows * D * 2);
    if (rc != MING_OK) return rc;
    h = (uint16_t*)c->xh;
    ldh = D;
  }
  const double bytes = (mode == 0 ? 4.0 : 6.0) * rows * D + (mode == 2 ? 6.0 : 2.0) * D;
  MING_HIP(profiled(c, mode >= 2 ? kBNormRes : kBRms, 0.0, bytes,
                    [&] { return ming::launch_rmsnorm_ex(mode, x, ldx, w, y, ldy, h, ldh,
                                                         gate, rows, D, eps, c->stream,
                                                         range_word(c)); }),
           "rmsnorm launch");
  c->eng.rmsnorm += 1;
  if (mode >= 2) c->eng.elementwise += 1;
  return ok();
}

int ming_rmsnorm(ming_ctx* c, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 uint16_t* y, int64_t ldy, int rows, int D, float eps) {
  return rms_impl(c, 0, x, ldx, w, y, ldy, nullptr, 0, nullptr, rows, D, eps,
                  "ming_rmsnorm");
}

int ming_rope_table(ming_ctx* c, const int32_t* pos_t, const int32_t* pos_h,
                    const int32_t* pos_w, int n, const int* axes, int head_dim,
                    double theta, float* cos_out, float* sin_out) {
  if (!c || !pos_t || !pos_h || !pos_w || !axes || !cos_out || !sin_out)
    return fail(MING_ERR_ARG, "ming_rope_table: null argument");
  if (n < 0 || head_dim <= 0 || head_dim % 2 != 0 || axes[0] < 0 ||
      axes[1] < 0 || axes[2] < 0 || axes[0] % 2 || axes[1] % 2 || axes[2] % 2 ||
      axes[0] + axes[1] + axes[2] != head_dim)
    return fail(MING_ERR_SHAPE, "ming_rope_table: axes must be even and sum to head_dim");
  if (n == 0) return ok();
  DeviceGuard g(c->device);
  MING_HIP(profiled(c, kBRopeTab, 0.0, 12.0 * n + 4.0 * n * head_dim,
                    [&] { return ming::launch_rope_table(pos_t, pos_h, pos_w, n,
                                                         axes[0], axes[1], axes[2],
                                                         head_dim, theta, cos_out,
                                                         sin_out, c->stream); }),
           "rope_table launch");
  c->eng.rope_table += 1;
  return ok();
}

int ming_qk_norm_rope(ming_ctx* c, uint16_t* x, int64_t ld, int q_col, int k_col,
                      int rows, int n_heads, int head_dim, const uint16_t* wq,
                      const uint16_t* wk, const float* cos_t, const float* sin_t,
                      float eps) {
  if (!c || !x || !wq || !wk || !cos_t || !sin_t)
    return fail(MING_ERR_ARG, "ming_qk_norm_rope: null argument");
  if (head_dim != 128)
    return fail(MING_ERR_SHAPE, "ming_qk_norm_rope: head_dim must be 128");
  if (rows < 0 || n_heads <= 0 || q_col < 0 || k_col < 0 || q_col % 8 ||
      k_col % 8 || ld % 8 || q_col + n_heads * 128 > ld ||
      k_col + n_heads * 128 > ld)
    return fail(MING_ERR_SHAPE, "ming_qk_norm_rope: bad columns or stride");
  if (!aligned(x, 16) || !aligned(wq, 16) || !aligned(wk, 16) ||
      !aligned(cos_t, 16) || !aligned(sin_t, 16))
    return fail(MING_ERR_ARG, "ming_qk_norm_rope: pointers must be 16-byte aligned");
  if (rows == 0) return ok();
  DeviceGuard g(c->device);
  MING_HIP(profiled(c, kBQkRope, 0.0, 8.0 * rows * n_heads * 128 + 512.0,
                    [&] { return ming::launch_qk_norm_rope(x, ld, q_col, k_col, rows,
                                                           n_heads, wq, wk, cos_t,
                                                           sin_t, eps, c->stream); }),
           "qk_norm_rope launch");
  c->eng.qk_norm_rope += 1;
  return ok();
}

int ming_llm_qk_norm_rope(ming_ctx* c, uint16_t* qkv, const uint16_t* q_w,
                          const uint16_t* k_w, const float* cos_t, const float* sin_t,
                          int rows, int64_t row_stride, int n_q, int n_k, int rot_half,
                          float eps) {
  if (!c || !qkv) return fail(MING_ERR_ARG, "ming_llm_qk_norm_rope: null argument");
  if (rot_half != 0 && rot_half != 32 && rot_half != 64)
    return fail(MING_ERR_ARG, "ming_llm_qk_norm_rope: rot_half must be 0, 32 or 64");
  if (rot_half != 0 && (!cos_t || !sin_t))
    return fail(MING_ERR_ARG, "ming_llm_qk_norm_rope: a rotation needs its cos and sin tables");
  if (rows < 0 || n_q < 0 || n_k < 0 || row_stride % 8 ||
      (int64_t)(n_q + n_k) * 128 > row_stride)
    return fail(MING_ERR_SHAPE, "ming_llm_qk_norm_rope: heads past the row stride");
  const bool norm = q_w && k_w;
  if (!aligned(qkv, 16) || (norm && (!aligned(q_w, 16) || !aligned(k_w, 16))) ||
      (rot_half && (!aligned(cos_t, 16) || !aligned(sin_t, 16))))
    return fail(MING_ERR_ARG, "ming_llm_qk_norm_rope: pointers must be 16-byte aligned");
  if (rows == 0 || n_q + n_k == 0) return ok();
  DeviceGuard g(c->device);
  const double bytes = 4.0 * rows * (n_q + n_k) * 128 + 8.0 * rows * rot_half;
  MING_HIP(profiled(c, kBQkRope, 0.0, bytes,
                    [&] {
                      return ming::launch_llm_qk_norm_rope(
                          qkv, row_stride, rows, n_q, n_k, norm ? q_w : nullptr,
                          norm ? k_w : nullptr, cos_t, sin_t, rot_half, eps, c->stream);
                    }),
           "llm_qk_norm_rope launch");
  c->eng.qk_norm_rope += 1;
  return ok();
}

// oh: optional fp16 copy of the output (the context's xh plane, row stride
// n_heads * 128) for the o-projection's fast route.
// qn: q and k arrive as raw projection outputs; k is normed + rotated in
// place by one pass, q by the attention kernel as it loads it (the bits of
// ming_qk_norm_rope followed by ming_attention).
struct QkNorm {
  const uint16_t *wq, *wk;
  const float *cos_t, *sin_t;
  float eps;
};
static int attention_impl(ming_ctx* c, const uint16_t* qkv, int64_t ld, int q_col, int k_col,
                          int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                          int head_dim, float scale, bool fp16_copy,
                          const QkNorm* qn = nullptr) {
  if (!c || !qkv || !out) return fail(MING_ERR_ARG, "ming_attention: null argument");
  if (head_dim != 128)
    return fail(MING_ERR_SHAPE, "ming_attention: head_dim must be 128");
  const int64_t w = (int64_t)n_heads * 128;
  if (rows < 0 || n_heads <= 0 || q_col < 0 || k_col < 0 || v_col < 0 || q_col % 8 ||
      k_col % 8 || v_col % 8 || ld % 8 || ldo % 8 || q_col + w > ld || k_col + w > ld ||
      v_col + w > ld || ldo < w)
    return fail(MING_ERR_SHAPE, "ming_attention: bad columns or strides");
  if (!aligned(qkv, 16) || !aligned(out, 16))
    return fail(MING_ERR_ARG, "ming_attention: pointers must be 16-byte aligned");
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail(MING_ERR_ARG, "ming_attention: scale must be positive and finite");
  // the K tile DMA addresses 64 rows from a scalar base with 32-bit offsets
  if ((uint64_t)ld * 2 * 64 >= (1ull << 31))
    return fail(MING_ERR_SHAPE, "ming_attention: row stride too large");
  if (rows == 0) return ok();
  DeviceGuard g(c->device);
  const int ldv = (rows + 63) / 64 * 64;
  int rc = ensure_vt(c, (size_t)n_heads * 128 * ldv * 2);
  if (rc != MING_OK) return rc;
  ming::AttnArgs a{};
  a.q = qkv + q_col; a.ldq = ld;
  a.k = qkv + k_col; a.ldk = ld;
  a.vt = (const uint16_t*)c->vt; a.ldv = ldv;
  a.o = out; a.ldo = ldo;
  if (fp16_copy) {
    rc = ensure_xh(c, (size_t)rows * w * 2);
    if (rc != MING_OK) return rc;
    a.oh = (uint16_t*)c->xh;
    a.ldoh = w;
    a.range = range_word(c);
  }
  a.R = rows; a.NH = n_heads;
  a.sl2 = scale * 1.4426950408889634f;
  if (qn) {
    if (!qn->wq || !qn->wk || !qn->cos_t || !qn->sin_t || !aligned(qn->wq, 16) ||
        !aligned(qn->wk, 16) || !aligned(qn->cos_t, 16) || !aligned(qn->sin_t, 16))
      return fail(MING_ERR_ARG, "attention: bad qk-norm weights or tables");
    uint16_t* kx = const_cast<uint16_t*>(qkv);
    MING_HIP(profiled(c, kBQkRope, 0.0, 4.0 * rows * w + 256.0,
                      [&] { return ming::launch_k_norm_rope(kx, ld, k_col, rows, n_heads,
                                                            qn->wk, qn->cos_t, qn->sin_t,
                                                            qn->eps, c->stream); }),
             "k-norm launch");
    c->eng.qk_norm_rope += 1;
    a.qw = qn->wq; a.cos_t = qn->cos_t; a.sin_t = qn->sin_t; a.eps = qn->eps;
  }
  const double flops = 4.0 * (double)rows * rows * 128.0 * n_heads;
  MING_HIP(profiled(c, kBAttn, flops, 8.0 * rows * w,
                    [&] { return ming::launch_attention(a, qkv + v_col, ld, c->stream); }),
           "attention launch");
  c->eng.attention += 1;
  return ok();
}

int ming_attention(ming_ctx* c, const uint16_t* qkv, int64_t ld, int q_col, int k_col,
                   int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                   int head_dim, float scale) {
  return attention_impl(c, qkv, ld, q_col, k_col, v_col, out, ldo, rows, n_heads, head_dim,
                        scale, false);
}


int ming_ctx_set_route(ming_ctx* c, int route) {
  if (!c) return fail(MING_ERR_ARG, "null context");
  if (route != MING_ROUTE_AUTO && route != MING_ROUTE_GENERAL && route != MING_ROUTE_WIDE)
    return fail(MING_ERR_ARG, "ming_ctx_set_route: unknown route");
  c->route = route;
  return ok();
}

int ming_qweight_fast(const ming_qweight* q) { return q && q->fast ? 1 : 0; }

int ming_ctx_set_profiling(ming_ctx* c, int on) {
  if (!c) return fail(MING_ERR_ARG, "null context");
  c->profiling = on != 0;
  return ok();
}

int ming_ctx_profile_collect(ming_ctx* c, ming_profile_bucket* out, int max,
                             int* n_out) {
  if (!c || (!out && max > 0)) return fail(MING_ERR_ARG, "null argument");
  DeviceGuard g(c->device);
  MING_HIP(hipStreamSynchronize(c->stream), "profile sync");
  ming_profile_bucket acc[kBCount];
  std::memset(acc, 0, sizeof(acc));
  for (auto& rec : c->recs) {
    float ms = 0.0f;
    const hipError_t e = hipEventElapsedTime(&ms, rec.a, rec.b);
    if (e == hipSuccess) {
      acc[rec.bucket].launches += 1;
      acc[rec.bucket].ms += ms;
      acc[rec.bucket].flops += rec.flops;
      acc[rec.bucket].bytes += rec.bytes;
    }
    c->pool.push_back(rec.a);
    c->pool.push_back(rec.b);
  }
  c->recs.clear();
  int n = 0;
  for (int b = 0; b < kBCount; ++b) {
    if (acc[b].launches == 0) continue;
    if (n < max) {
      out[n] = acc[b];
      std::snprintf(out[n].name, sizeof(out[n].name), "%s", kBucketName[b]);
    }
    ++n;
  }
  if (n_out) *n_out = n < max ? n : max;
  return ok();
}

namespace {
int elt_check(ming_ctx* c, const void* a, const void* b, int rows, int n) {
  if (!c || !a || !b) return fail(MING_ERR_ARG, "null argument");
  if (rows < 0 || n <= 0) return fail(MING_ERR_SHAPE, "bad rows / width");
  return MING_OK;
}
}  // namespace

int ming_swiglu(ming_ctx* c, const uint16_t* g, int64_t ldg, const uint16_t* u,
                int64_t ldu, uint16_t* out, int64_t ldo, int rows, int n) {
  int rc = elt_check(c, g, u, rows, n);
  if (rc != MING_OK) return rc;
  if (!out || n % 8 || ldg % 8 || ldu % 8 || ldo % 8 || !aligned(g, 16) ||
      !aligned(u, 16) || !aligned(out, 16))
    return fail(MING_ERR_SHAPE, "ming_swiglu: widths, strides and pointers must be 8-element aligned");
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBSwiglu, 0.0, 6.0 * rows * n,
                    [&] { return ming::launch_swiglu(g, ldg, u, ldu, out, ldo, rows, n,
                                                     c->stream); }),
           "swiglu launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_gated_residual(ming_ctx* c, uint16_t* h, int64_t ldh,
                        const uint16_t* gate, const uint16_t* sub, int64_t lds,
                        int rows, int n) {
  int rc = elt_check(c, h, sub, rows, n);
  if (rc != MING_OK) return rc;
  if (!gate || n % 8 || ldh % 8 || lds % 8 || !aligned(h, 16) ||
      !aligned(sub, 16) || !aligned(gate, 16))
    return fail(MING_ERR_SHAPE, "ming_gated_residual: 8-element alignment required");
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBResid, 0.0, 6.0 * rows * n,
                    [&] { return ming::launch_residual(h, ldh, gate, sub, lds, rows, n,
                                                       1, c->stream); }),
           "gated_residual launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_residual_add(ming_ctx* c, uint16_t* h, int64_t ldh, const uint16_t* sub,
                      int64_t lds, int rows, int n) {
  int rc = elt_check(c, h, sub, rows, n);
  if (rc != MING_OK) return rc;
  if (n % 8 || ldh % 8 || lds % 8 || !aligned(h, 16) || !aligned(sub, 16))
    return fail(MING_ERR_SHAPE, "ming_residual_add: 8-element alignment required");
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBResid, 0.0, 6.0 * rows * n,
                    [&] { return ming::launch_residual(h, ldh, nullptr, sub, lds, rows,
                                                       n, 0, c->stream); }),
           "residual_add launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_modulate(ming_ctx* c, const uint16_t* x, int64_t ldx,
                  const uint16_t* scale, uint16_t* y, int64_t ldy, int rows,
                  int n) {
  int rc = elt_check(c, x, scale, rows, n);
  if (rc != MING_OK) return rc;
  if (!y) return fail(MING_ERR_ARG, "null argument");
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBModulate, 0.0, 4.0 * rows * n + 2.0 * n,
                    [&] { return ming::launch_modulate(x, ldx, scale, y, ldy, rows, n,
                                                       c->stream); }),
           "modulate launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_bias_act(ming_ctx* c, uint16_t* y, int64_t ldy, const uint16_t* bias,
                  int rows, int n, int silu) {
  int rc = elt_check(c, y, bias, rows, n);
  if (rc != MING_OK) return rc;
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBBias, 0.0, 4.0 * rows * n + 2.0 * n,
                    [&] { return ming::launch_bias_act(y, ldy, bias, nullptr, rows, n,
                                                       silu ? 1 : 0, c->stream); }),
           "bias_act launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_silu(ming_ctx* c, const uint16_t* x, uint16_t* y, int n) {
  int rc = elt_check(c, x, y, 1, n);
  if (rc != MING_OK) return rc;
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBBias, 0.0, 4.0 * n,
                    [&] { return ming::launch_bias_act(const_cast<uint16_t*>(x), n,
                                                       nullptr, y, 1, n, 2, c->stream); }),
           "silu launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_ln_modulate(ming_ctx* c, const uint16_t* x, int64_t ldx,
                     const uint16_t* scale, uint16_t* y, int64_t ldy, int rows,
                     int D, float eps) {
  int rc = elt_check(c, x, scale, rows, D);
  if (rc != MING_OK) return rc;
  if (!y) return fail(MING_ERR_ARG, "null argument");
  // the kernel holds a row in registers, 16-byte chunks
  if (D % 8 != 0 || D > 8192 || ldx < D || ldy < D || ldx % 8 != 0 || ldy % 8 != 0)
    return fail(MING_ERR_SHAPE, "ming_ln_modulate: need D % 8 == 0, D <= 8192, strides % 8 == 0");
  if (!aligned(x, 16) || !aligned(y, 16) || !aligned(scale, 16))
    return fail(MING_ERR_ARG, "ming_ln_modulate: pointers must be 16-byte aligned");
  if (rows == 0) return ok();
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBLn, 0.0, 4.0 * rows * D,
                    [&] { return ming::launch_ln_modulate(x, ldx, scale, y, ldy, rows, D,
                                                          eps, c->stream); }),
           "ln_modulate launch");
  c->eng.elementwise += 1;
  return ok();
}

int ming_quantize_pack(ming_ctx* c, const float* w, int N, int K, int bits,
                       int group, uint32_t* codes, uint16_t* scales,
                       uint16_t* biases) {
  if (!c || !w || !codes || !scales || !biases)
    return fail(MING_ERR_ARG, "ming_quantize_pack: null argument");
  if ((bits != 4 && bits != 8) || group != 64 || N <= 0 || K <= 0 || K % 64)
    return fail(MING_ERR_SHAPE, "ming_quantize_pack: bits 4/8, group 64, K % 64 == 0");
  DeviceGuard dg(c->device);
  MING_HIP(profiled(c, kBQuant, 0.0, 4.0 * N * K,
                    [&] { return ming::launch_quantize(w, N, K, bits, codes, scales,
                                                       biases, c->stream); }),
           "quantize launch");
  return ok();
}

}  // extern "C"

namespace ming {
int rt_fail(int code, const std::string& why) { return fail(code, why); }
int rt_ok() { return ok(); }
int rt_device(const ming_ctx* c) { return c ? c->device : -1; }
void rt_retain(ming_ctx* c) { c->live_weights += 1; }
void rt_release(ming_ctx* c) { c->live_weights -= 1; }

void rt_log(int level, const std::string& msg) {
  ming_log_fn fn;
  void* user;
  {
    std::lock_guard<std::mutex> g(g_log_mu);
    fn = g_log_fn;
    user = g_log_user;
  }
  if (fn) fn(user, level, msg.c_str());
}

int rt_upload(ming_ctx* c, const void* host, size_t bytes, void** dev) {
  *dev = nullptr;
  if (bytes == 0) return ok();
  DeviceGuard dg(c->device);
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MING_ERR_ALLOC, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  if (hipMemcpy(p, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(p);
    return fail(MING_ERR_HIP, "host to device copy failed");
  }
  *dev = p;
  return ok();
}

int rt_alloc(ming_ctx* c, size_t bytes, bool zero, void** dev) {
  *dev = nullptr;
  DeviceGuard dg(c->device);
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MING_ERR_ALLOC, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  if (zero && (hipMemsetAsync(p, 0, bytes, c->stream) != hipSuccess ||
               hipStreamSynchronize(c->stream) != hipSuccess)) {
    (void)hipFree(p);
    return fail(MING_ERR_HIP, "device memset failed");
  }
  *dev = p;
  return ok();
}

int rt_h2d(ming_ctx* c, void* dev, const void* host, size_t bytes) {
  DeviceGuard dg(c->device);
  if (hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return fail(MING_ERR_HIP, "host to device copy failed");
  return ok();
}

int rt_d2h(ming_ctx* c, void* host, const void* dev, size_t bytes) {
  DeviceGuard dg(c->device);
  if (hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess)
    return fail(MING_ERR_HIP, "device to host copy failed");
  return ok();
}

void rt_free(ming_ctx* c, void* dev) {
  if (!dev) return;
  DeviceGuard dg(c->device);
  (void)hipFree(dev);
}

void rt_note_cap_hit(ming_ctx* c) { c->eng.cap_cache_hits += 1; }
uint64_t rt_qweight_bind_gen(const ming_qweight* q) { return q ? q->bind_gen : 0; }

bool rt_set_copies_unread(ming_ctx* c, bool unread) {
  const bool was = c->copies_unread;
  c->copies_unread = unread;
  return was;
}

int rt_take_range_fault(ming_ctx* c, const char* who) {
  DeviceGuard dg(c->device);
  return take_range_fault(c, who);
}

int rt_rmsnorm_f16(ming_ctx* c, const uint16_t* x, int64_t ldx, const uint16_t* w,
                   uint16_t* y, int64_t ldy, int rows, int D, float eps) {
  return rms_impl(c, 1, x, ldx, w, y, ldy, nullptr, 0, nullptr, rows, D, eps, "rmsnorm");
}

int rt_norm_residual(ming_ctx* c, uint16_t* h, int64_t ldh, const uint16_t* sub,
                     int64_t lds, const uint16_t* w, const float* tgate, int rows, int D,
                     float eps) {
  return rms_impl(c, tgate ? 2 : 3, sub, lds, w, nullptr, 0, h, ldh, tgate, rows, D, eps,
                  "post-norm residual");
}

int rt_norm_residual_norm(ming_ctx* c, uint16_t* h, int64_t ldh, const uint16_t* sub,
                          int64_t lds, const uint16_t* wpost, const float* tgate,
                          const uint16_t* wpre, uint16_t* y, int64_t ldy, int rows, int D,
                          float eps) {
  if (!c || !h || !sub || !wpost || !wpre || !y)
    return fail(MING_ERR_ARG, "norm-residual-norm: null argument");
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 8192 || ldh < D || ldh % 8 != 0 || lds < D ||
      lds % 8 != 0 || ldy < D || ldy % 8 != 0)
    return fail(MING_ERR_SHAPE, "norm-residual-norm: bad shape or row strides");
  if (!aligned(h, 16) || !aligned(sub, 16) || !aligned(wpost, 16) || !aligned(wpre, 16) ||
      !aligned(y, 16) || (tgate && !aligned(tgate, 16)))
    return fail(MING_ERR_ARG, "norm-residual-norm: pointers must be 16-byte aligned");
  if (rows == 0) return ok();
  DeviceGuard g(c->device);
  int rc = ensure_xh(c, (size_t)rows * D * 2);
  if (rc != MING_OK) return rc;
  uint16_t* yh = (uint16_t*)c->xh;
  MING_HIP(profiled(c, kBNormRes, 0.0, 10.0 * rows * D + (tgate ? 8.0 : 4.0) * D,
                    [&] { return ming::launch_norm_residual_norm(sub, lds, wpost, h, ldh, tgate,
                                                                 wpre, y, ldy, yh, D, rows, D,
                                                                 eps, c->stream,
                                                                 range_word(c)); }),
           "norm-residual-norm launch");
  // counted as the two launches it replaces
  c->eng.rmsnorm += 2;
  c->eng.elementwise += 1;
  return ok();
}

int rt_adaln_glue(ming_ctx* c, uint16_t* mods, int n, const uint16_t* b, const uint16_t* an1,
                  const uint16_t* fn1, uint16_t* nw1, uint16_t* nw3, float* t) {
  DeviceGuard g(c->device);
  MING_HIP(profiled(c, kBModulate, 0.0, 2.0 * 8 * n + 2.0 * 4 * n + 4.0 * 2 * n,
                    [&] {
                      return ming::launch_adaln_glue(mods, n, b, an1, fn1, nw1, nw3, t,
                                                     c->stream);
                    }),
           "adaLN glue launch");
  c->eng.elementwise += 1;
  return ok();
}

int rt_modulation_batch(ming_ctx* c, int count, const ming_qweight* const* ada,
                        const uint16_t* const* ada_b, const uint16_t* const* an1,
                        const uint16_t* const* fn1, const uint16_t* temb, int H,
                        uint16_t* const* mods, uint16_t* const* nw1, uint16_t* const* nw3,
                        float* const* tg, const float* scales, bool* done) {
  *done = false;
  if (count <= 0 || c->route == MING_ROUTE_GENERAL || !ada[0]) return ok();
  const ming_qweight* q0 = ada[0];
  for (int i = 0; i < count; ++i) {
    const ming_qweight* q = ada[i];
    if (!q || q->ctx != c || q->bits != q0->bits || q->N != 4 * H || q->K != q0->K ||
        q->K % 64 != 0)
      return ok();
    // the per-block projection runs the GEMV only with no live adapter
    for (const Segment& sg : q->segs)
      for (int sl = 0; sl < MING_MAX_LORA_SLOTS; ++sl)
        if (sg.slot[sl].rank > 0 && scales && scales[sl] != 0.0f) return ok();
  }
  DeviceGuard g(c->device);
  const double wbytes = q0->bits == 16 ? 2.0 * q0->N * q0->K
                                       : (double)q0->N * q0->K * q0->bits / 8 +
                                             4.0 * q0->N * (q0->K / 64);
  for (int b0 = 0; b0 < count; b0 += ming::kGemvBatch) {
    const int nb = std::min(ming::kGemvBatch, count - b0);
    ming::GemvBatch gb{};
    gb.base.x = temb; gb.base.ldx = q0->K; gb.base.ldy = q0->N;
    gb.base.M = 1; gb.base.N = q0->N; gb.base.K = q0->K;
    gb.count = nb;
    ming::GlueBatch gl{};
    gl.n = H;
    gl.count = nb;
    for (int j = 0; j < nb; ++j) {
      const ming_qweight* q = ada[b0 + j];
      gb.e[j] = {q->codes_t, q->sb, q->w16, mods[b0 + j]};
      gl.e[j] = {mods[b0 + j], ada_b[b0 + j], an1[b0 + j], fn1[b0 + j],
                 nw1[b0 + j],  nw3[b0 + j],   tg[b0 + j]};
    }
    MING_HIP(profiled(c, kBGemv, 2.0 * nb * q0->N * (double)q0->K,
                      nb * (wbytes + 2.0 * q0->K + 2.0 * q0->N),
                      [&] { return ming::launch_gemv_batch(q0->bits, gb, c->stream); }),
             "batched gemv launch");
    MING_HIP(profiled(c, kBModulate, 0.0, nb * (2.0 * 8 * H + 2.0 * 4 * H + 4.0 * 2 * H),
                      [&] { return ming::launch_adaln_glue_batch(gl, c->stream); }),
             "batched adaLN glue launch");
    // counted as the per-block projections and glue are
    if (q0->bits == 4) c->eng.gemm_q4 += nb;
    else if (q0->bits == 8) c->eng.gemm_q8 += nb;
    else c->eng.gemm_dense += nb;
    c->eng.gemv += nb;
    c->eng.gemm_flops += 2ull * (uint64_t)nb * (uint64_t)q0->N * (uint64_t)q0->K;
    c->eng.elementwise += nb;
  }
  *done = true;
  return ok();
}

int rt_tanh_gates(ming_ctx* c, const uint16_t* mods, int n, float* t) {
  DeviceGuard g(c->device);
  MING_HIP(profiled(c, kBModulate, 0.0, 2.0 * 2 * n + 4.0 * 2 * n,
                    [&] { return ming::launch_tanh_gates(mods, n, t, c->stream); }),
           "tanh gates launch");
  c->eng.elementwise += 1;
  return ok();
}

int rt_attention_xh(ming_ctx* c, const uint16_t* qkv, int64_t ld, int q_col, int k_col,
                    int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                    float scale) {
  return attention_impl(c, qkv, ld, q_col, k_col, v_col, out, ldo, rows, n_heads, 128, scale,
                        true);
}

int rt_attention_qknorm_xh(ming_ctx* c, uint16_t* qkv, int64_t ld, int q_col, int k_col,
                           int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                           float scale, const uint16_t* wq, const uint16_t* wk,
                           const float* cos_t, const float* sin_t, float eps) {
  const QkNorm qn{wq, wk, cos_t, sin_t, eps};
  return attention_impl(c, qkv, ld, q_col, k_col, v_col, out, ldo, rows, n_heads, 128, scale,
                        true, &qn);
}

int rt_lin_xh(ming_ctx* c, const ming_qweight* qw, const uint16_t* x, int64_t ldx,
              uint16_t* y, int64_t ldy, int M, const float* scales) {
  return lin_impl(c, qw, x, ldx, y, ldy, M, scales, nullptr, 0, (const uint16_t*)c->xh,
                  nullptr);
}

int rt_lin3_xh(ming_ctx* c, const ming_qweight* const* qw, const uint16_t* x, int64_t ldx,
               uint16_t* const* y, int64_t ldy, int M, const float* scales) {
  LinOut outs[3];
  for (int i = 0; i < 3; ++i) {
    outs[i].y = y[i];
    outs[i].ldy = ldy;
  }
  return lin_multi(c, 3, qw, outs, x, ldx, M, scales, (const uint16_t*)c->xh);
}

int rt_ffn_xh(ming_ctx* c, const ming_qweight* w1, const ming_qweight* w3,
              const ming_qweight* w2, const uint16_t* x, int64_t ldx, uint16_t* y,
              int64_t ldy, int M, const float* scales, uint16_t* h, int64_t ldh) {
  return ffn_impl(c, w1, w3, w2, x, ldx, y, ldy, M, scales, h, ldh, true);
}
}  // namespace ming
