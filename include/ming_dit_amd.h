/*
 * ming_dit_amd.h -- the C-ABI of the MI355X-native DiT block-projection
 * path of Ming-Image (a drop-in for the reference's ming-dit / ming-ops /
 * ming-quant-family seams, tgo-app-dev/vpipe-ming-image).
 *
 * Plain C: opaque handles, plain pointers and sizes, integer status codes,
 * no exceptions across the boundary. Activations are bf16 bit patterns
 * (uint16_t) in device memory, token-major with an explicit row stride in
 * ELEMENTS (the reference passes element offsets, ming-dit.cc:1763; a
 * caller adds them to the pointer). One caller thread per context; work
 * is enqueued in order on the context's HIP stream and entry points return
 * without waiting unless they say otherwise.
 *
 * Status: 0 ok, > 0 error (ming_last_error() says why, per thread),
 * < 0 a cooperative stop (ming-dit.h:170-189: empty result, empty error).
 */
#ifndef MING_DIT_AMD_H
#define MING_DIT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MING_ABI_VERSION 5

/* Runtime-LoRA slots: lora::Stack::kMax (ming-dit.h:117) and the eight
 * `lora`..`lora8` keys (ming-model-config-stage.h:37-56). */
#define MING_MAX_LORA_SLOTS 8
/* Largest adapter rank one slot binds. */
#define MING_MAX_LORA_RANK 512

enum {
  MING_OK = 0,
  MING_ERR_ARG = 1,     /* a null handle/pointer or an out-of-range value */
  MING_ERR_SHAPE = 2,   /* a shape the path does not take */
  MING_ERR_HIP = 3,     /* the HIP runtime reported an error */
  MING_ERR_ALLOC = 4,   /* device memory could not be allocated */
  MING_ERR_KERNEL = 5,  /* a kernel failed validation at context creation */
  MING_ERR_STATE = 6,   /* the call does not fit the object's state */
  MING_ERR_RANGE = 7,   /* a projection input on an fp16 route was >= 65536 in
                           magnitude or not finite (see MING_ROUTE_WIDE) */
  MING_STOPPED = -1     /* a cooperative stop: not an error */
};

typedef struct ming_ctx ming_ctx;
typedef struct ming_qweight ming_qweight;

/* What the context DISPATCHED since its last reset, counted at the
 * dispatch site (the reference's DitEngagement, ming-dit.h:55-103): a
 * route that is configured but never ran passes every numeric bar, so
 * tests assert these before accuracy. */
typedef struct ming_engagement {
  int64_t gemm_q4;      /* quantized w4 projections (gemm_qmm, w4) */
  int64_t gemm_q8;      /* quantized w8 projections (gemm_qmm, w8) */
  int64_t gemm_dense;   /* dense bf16 projections */
  int64_t lora_proj;    /* projections that carried >= 1 live adapter */
  int64_t lora_xa;      /* stacked x.A GEMMs launched */
  int64_t rmsnorm;
  int64_t qk_norm_rope;
  int64_t rope_table;
  int64_t attention;
  int64_t elementwise;
  uint64_t gemm_flops;  /* 2*M*N*K + sum_live 2*M*r*(K+N) per projection */
  int64_t gemm_fast;    /* of the quantized projections, those on the fast route */
  int64_t cap_cache_hits; /* forwards whose caption path came from the caption cache */
  int64_t gemv;           /* of the projections, those run as a GEMV (M <= 8, no live adapter) */
  int64_t gemm_split;     /* of the fast-route projections, those split along K (< 64 tiles) */
  int64_t range_faults;   /* synchronizations that found a saturated fp16 input copy
                             (MING_ERR_RANGE; see MING_ROUTE_WIDE) */
  int64_t gemm_paired;    /* launches that ran a SwiGLU's gate and up projections together
                             (ming_ffn on the fast route; each projection also counts in
                             gemm_q4/q8 and gemm_fast) */
} ming_engagement;

/* Kernel routes for quantized projections. AUTO takes the fast route
 * (fp16 activations, DMA-fed LDS ring, fragment dequant) whenever the
 * weight's scales and biases are exact in fp16, and a GEMV (each weight
 * streamed once, f32 dot products) for M <= 8 rows with no live adapter, as
 * the adaLN and timestep projections run at M = 1. GENERAL always takes the
 * general kernel. Both multiply fp16 activations: bf16 values are carried
 * exactly at magnitudes in [2^-17, 2^16); smaller ones are cut toward zero
 * to fp16's subnormal step of 2^-24 (below 2^-24 they become 0; an absolute
 * error of at most 2^-24, not reported). A value of 2^16 or more, inf or NaN
 * cannot be carried, and the next ming_ctx_synchronize (or the forward that
 * met it) returns MING_ERR_RANGE instead of results. The report is pending
 * for the CONTEXT, not for the call that met it: it stays raised until the
 * next ming_ctx_synchronize or ming_model_forward collects it, so a caller
 * that waits for the stream some other way should call ming_ctx_synchronize
 * after a projection whose inputs it does not control. WIDE multiplies the
 * bf16 activations themselves with each dequantized weight split into a
 * bf16 pair (hi + lo, twice the MFMA work): no range limit, for inputs that
 * the fp16 routes refuse. All compute the same function to the same bar. */
enum { MING_ROUTE_AUTO = 0, MING_ROUTE_GENERAL = 1, MING_ROUTE_WIDE = 2 };

/* Per-launch kernel timing (HIP events around each launch, on the
 * context's stream), summed per kernel family -- the reference's profile
 * buckets (ming-dit.cc:1689-1717) without its commit+wait per mark. flops
 * and bytes are the ALGORITHMIC work of the timed launches: GEMM flops
 * 2*M*N*K (+ the LoRA's 2*M*r*K in lora_xa and 2*M*r*N in the tail),
 * bytes read + written once. */
typedef struct ming_profile_bucket {
  char name[24];
  int64_t launches;
  double ms;
  double flops;
  double bytes;
} ming_profile_bucket;

/* Last error of the CALLING thread; "" when the last call succeeded. */
const char* ming_last_error(void);
int ming_abi_version(void);

/* The session log (the reference's SessionContextIntf warn / log_normal):
 * binding reports and refusals that are not errors go here. level 1 warn,
 * 2 info. NULL restores the default, which drops the messages. The sink is
 * process-wide and called on the thread that makes the call being reported. */
#define MING_LOG_WARN 1
#define MING_LOG_INFO 2
typedef void (*ming_log_fn)(void* user, int level, const char* message);
void ming_set_log_sink(ming_log_fn fn, void* user);

/* ---- context --------------------------------------------------------------
 * Binds a device and a stream (NULL: the context creates and owns one).
 * Every kernel the path dispatches is resolved and VALIDATED here, and a
 * missing one refuses the context rather than degrading (the reference's
 * load-time refusal, ming-dit.cc:1141-1235). */
int ming_ctx_create(int device, void* hip_stream, ming_ctx** out);
/* Refused (MING_ERR_STATE) while weights made on the context are alive. */
int ming_ctx_destroy(ming_ctx* ctx);
int ming_ctx_set_stream(ming_ctx* ctx, void* hip_stream);
void* ming_ctx_stream(const ming_ctx* ctx);
/* Waits for the context's stream. MING_ERR_RANGE when a projection input on
 * an fp16 route could not be carried since the last synchronization (see
 * MING_ROUTE_WIDE); the condition is then cleared. */
int ming_ctx_synchronize(ming_ctx* ctx);
int ming_ctx_engagement(const ming_ctx* ctx, ming_engagement* out);
int ming_ctx_reset_engagement(ming_ctx* ctx);
int ming_ctx_set_route(ming_ctx* ctx, int route);
/* Profiling on/off; collect waits for the stream, fills up to `max`
 * non-empty buckets and clears the records. */
int ming_ctx_set_profiling(ming_ctx* ctx, int on);
int ming_ctx_profile_collect(ming_ctx* ctx, ming_profile_bucket* out, int max,
                             int* n_out);

/* ---- projection weights (the quant pack) ------------------------------------
 * A quantized projection in the reference's pack layout (load_qw_,
 * ming-dit.cc:802-831; pack detection 1115-1135): codes U32
 * [N, K*bits/32] (unsigned codes, LSB-first within a word), scales and
 * biases bf16 [N, K/group], w = scales*q + biases. bits 4 or 8, group 64,
 * K % 64 == 0, N % 8 == 0. `src_on_device` 0 reads host memory. The
 * weight is repacked into the kernels' resident tiled layout; the sources
 * may be freed when the call returns. */
int ming_qweight_create(ming_ctx* ctx, int N, int K, int bits, int group,
                        const uint32_t* codes, const uint16_t* scales,
                        const uint16_t* biases, int src_on_device,
                        ming_qweight** out);
/* A dense bf16 [N, K] projection (a dense checkpoint's `.weight`,
 * to_elt_ at ming-dit.cc:795-800). */
int ming_qweight_create_dense(ming_ctx* ctx, int N, int K, const uint16_t* w,
                              int src_on_device, ming_qweight** out);
/* Several projections over the SAME input fused along N (q|k|v;
 * w1|w3): the output is their concatenation, each part keeping its own
 * adapter bindings (part i = segment i). Parts must share K and bits, and
 * every part but the last must have N % 256 == 0. At most 4 parts. The
 * parts stay valid and independent. */
int ming_qweight_concat(ming_ctx* ctx, int n_parts,
                        ming_qweight* const* parts, ming_qweight** out);
int ming_qweight_destroy(ming_qweight* qw);
/* 4, 8 or 16 (dense bf16); 0 on a null handle. */
int ming_qweight_bits(const ming_qweight* qw);
/* 1 when the weight can take the fast route (scales, biases fp16-exact). */
int ming_qweight_fast(const ming_qweight* qw);
int ming_qweight_shape(const ming_qweight* qw, int* N, int* K, int* n_segments);

/* ---- runtime LoRA, bound at load (bind_loras_, ming-dit.cc:2918-3005) -------
 * Binds slot `slot`'s factors to segment `segment` of a projection:
 * A [rank, K] bf16 (down), B [N_seg, rank] bf16 (up), and `fold` the
 * adapter's alpha/rank (the factor the reference folds into A). The delta
 * is fold * scale * B (A x). Wrong shapes are refused (MING_ERR_SHAPE),
 * which the model level turns into refusing the WHOLE slot. */
int ming_qweight_bind_lora(ming_qweight* qw, int segment, int slot, int rank,
                           const uint16_t* A, const uint16_t* B, float fold,
                           int src_on_device);
int ming_qweight_unbind_lora(ming_qweight* qw, int segment, int slot);
/* Rank bound at (segment, slot), 0 when unbound. */
int ming_qweight_lora_rank(const ming_qweight* qw, int segment, int slot);

/* ---- the projection (lin, ming-dit.cc:1763-1771) -----------------------------
 * y[M, N] = x[M, K] . W^T + sum over live slots of
 *           fold * scales[slot] * B_slot (A_slot x)
 * `scales` holds MING_MAX_LORA_SLOTS live strengths (NULL: all 0). A slot
 * is live when it is bound on the segment AND its strength is non-zero;
 * strength 0 encodes nothing at all, so an all-zero call is bit-identical
 * to an unadapted one (ming-dit.h:150-154, ming-dit.cc:3015-3019).
 * ldx, ldy in elements (>= K, >= N; multiples of 8). x and y device. */
int ming_lin(ming_ctx* ctx, const ming_qweight* qw, const uint16_t* x,
             int64_t ldx, uint16_t* y, int64_t ldy, int M,
             const float* scales);

/* ming_lin with a bias: y = bf16(x . W^T + (live LoRA) + bias), the bias
 * added to the f32 result before the output's one rounding, as the LLM
 * encoder's LlmOps::linear(enc, x, xe, w, bias, y, ye, M, N, K) passes it to
 * its GEMM kernel (ming-ops.h:84-90, ming-ops.cc:119-141). For dense (bf16)
 * weights, that linear's kind: a quantized weight is refused (MING_ERR_ARG;
 * ming_lin then ming_bias_act adds a bias after the rounding). bias [N] bf16
 * on the device; the other arguments as ming_lin's. */
int ming_lin_bias(ming_ctx* ctx, const ming_qweight* qw, const uint16_t* x,
                  int64_t ldx, uint16_t* y, int64_t ldy, int M,
                  const float* scales, const uint16_t* bias);

/* ming_lin that allocates nothing. It has NO counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and bits as ming_lin; the call's scratch (the adapters'
 * x.A intermediate, the fp16 copy of x, split-K partials) comes from one
 * static array of MING_NOALLOC_SCRATCH_BYTES per GPU, resident from the first
 * context on that GPU until the process ends. Refusals, before anything is
 * launched: MING_ERR_SHAPE when a call needs more than the array holds (the
 * fp16 copy of x, M * K * 2 bytes; the adapters' x.A intermediate, M * padded
 * live ranks * 2 bytes; the f32 partials of a split-K launch, slices * M *
 * columns * 4 bytes; each region rounded up to 256 bytes); MING_ERR_STATE
 * when the weight's adapter bindings changed since its last ming_lin call
 * (that call builds the stacked factors, which allocates). Every call on a
 * GPU shares that GPU's array and it keeps the last call's contents (nothing
 * in it needs to start at zero): calls that overlap on one GPU -- other
 * streams, other contexts, other threads -- race. Profiling events are not
 * recorded for it. */
#define MING_NOALLOC_SCRATCH_BYTES (64u << 20)
int ming_lin_noalloc(ming_ctx* ctx, const ming_qweight* w, const uint16_t* x,
                     int64_t ldx, uint16_t* y, int64_t ldy, int M, const float* scales);

/* out = bf16(silu(g) * bf16(lin(x, w))): the w3 projection with the SwiGLU
 * of gpu_ff (ming-dit.cc:2151-2158; ming_ops.metal:97-112) fused into its
 * epilogue. Same bits as ming_lin then ming_swiglu. g may be out (in place).
 * g and out: strides multiples of 8, 16-byte aligned. */
int ming_lin_swiglu(ming_ctx* ctx, const ming_qweight* w, const uint16_t* x,
                    int64_t ldx, const uint16_t* g, int64_t ldg, uint16_t* out,
                    int64_t ldo, int M, const float* scales);
/* gpu_ff (ming-dit.cc:2151-2162): h = lin(x, w1); h = swiglu(h, lin(x, w3));
 * y = lin(h, w2), with the live LoRA of each projection. h is the caller's
 * [M][ffn] plane (ldh >= ffn, a multiple of 8, 16-byte aligned). Same bits
 * as the four separate calls; x is converted for the fast route once. */
int ming_ffn(ming_ctx* ctx, const ming_qweight* w1, const ming_qweight* w3,
             const ming_qweight* w2, const uint16_t* x, int64_t ldx, uint16_t* y,
             int64_t ldy, int M, const float* scales, uint16_t* h, int64_t ldh);
/* ---- norms and rotary ----------------------------------------------------------
 * rms (ming-dit.cc:1780-1787): y = bf16(x * rsqrt(mean(x^2)+eps) * w) per
 * row of D (D % 8 == 0, D <= 8192); in place when x == y. */
int ming_rmsnorm(ming_ctx* ctx, const uint16_t* x, int64_t ldx,
                 const uint16_t* w, uint16_t* y, int64_t ldy, int rows, int D,
                 float eps);
/* The rotary tables of build_rope_ (ming-dit.cc:1443-1486) from device
 * int32 positions [n] per axis: f32 cos/sin [n][head_dim/2], pairs split
 * over the three axes as axes[0]/2, axes[1]/2, axes[2]/2, angles in f64. */
int ming_rope_table(ming_ctx* ctx, const int32_t* pos_t, const int32_t* pos_h,
                    const int32_t* pos_w, int n, const int* axes, int head_dim,
                    double theta, float* cos_out, float* sin_out);
/* qk-norm + RoPE, in place on token-major rows (ming-dit.cc:2083-2088):
 * per head of 128, RMSNorm with wq / wk [128], then the interleaved-pair
 * rotation with table row `row` (the caller offsets the tables by row0).
 * q heads start at column q_col, k heads at k_col; n_heads each. */
int ming_qk_norm_rope(ming_ctx* ctx, uint16_t* x, int64_t ld, int q_col,
                      int k_col, int rows, int n_heads, int head_dim,
                      const uint16_t* wq, const uint16_t* wk,
                      const float* cos_t, const float* sin_t, float eps);

/* The LLM encoder's qk-norm + RoPE, LlmOps::qk_norm_rope (ming-ops.h:118-122,
 * ming-ops.cc:281-302; kernel ming_llm.metal:100-178), in place on the fused
 * token-major qkv rows [rows][row_stride] bf16: heads [0, n_q) are queries
 * from column 0, heads [n_q, n_q + n_k) keys right after them (128 wide each;
 * n_k may differ from n_q); the value columns past them are not touched.
 * With both q_w and k_w [128] given, each head is RMS-normalized (f32
 * statistics, eps) and scaled by its weight first; with either one NULL there
 * is no norm. rot_half is the rotate-half width: 64 rotates each pair
 * (j, j + 64) of the whole head, 32 the pairs (j, j + 32) of dims 0..63 and
 * leaves 64..127, 0 rotates nothing; cos_t / sin_t are f32 [rows][rot_half]
 * (angle j of row r; unused at 0). One bf16 rounding per element.
 * row_stride a multiple of 8 elements; pointers 16-byte aligned. */
int ming_llm_qk_norm_rope(ming_ctx* ctx, uint16_t* qkv, const uint16_t* q_w,
                          const uint16_t* k_w, const float* cos_t, const float* sin_t,
                          int rows, int64_t row_stride, int n_q, int n_k, int rot_half,
                          float eps);

/* Dense bidirectional attention (run_attn, ming-dit.cc:1905-2039, with the
 * head-major transposes around it, 2085-2092): for every head h,
 *   out[:, 128h + d] = softmax(scale * Q_h K_h^T) V_h,
 * Q_h = qkv[:, q_col + 128h ...], K_h and V_h likewise at k_col / v_col, all
 * token-major with row stride ld; out token-major with stride ldo. head_dim
 * must be 128; strides and columns multiples of 8, pointers 16-byte
 * aligned. No mask: every row attends to all `rows` keys. */
int ming_attention(ming_ctx* ctx, const uint16_t* qkv, int64_t ld, int q_col,
                   int k_col, int v_col, uint16_t* out, int64_t ldo, int rows,
                   int n_heads, int head_dim, float scale);

/* ---- block glue (ming_ops.metal; ming-dit.cc:1772-1884) -----------------------
 * All bf16, token-major, element strides; widths and strides multiples of
 * 8 and pointers 16-byte aligned where noted. */
/* out = bf16(silu(g) * u), silu(g) = g / (1 + exp(-g)): swiglu_v4_f16. */
int ming_swiglu(ming_ctx* ctx, const uint16_t* g, int64_t ldg,
                const uint16_t* u, int64_t ldu, uint16_t* out, int64_t ldo,
                int rows, int n);
/* h = bf16(h + tanh(gate[n]) * sub): gated_residual_tanh_v4_f16. */
int ming_gated_residual(ming_ctx* ctx, uint16_t* h, int64_t ldh,
                        const uint16_t* gate, const uint16_t* sub,
                        int64_t lds, int rows, int n);
/* h = bf16(h + sub): residual_add_v4_f16 (the context refiner). */
int ming_residual_add(ming_ctx* ctx, uint16_t* h, int64_t ldh,
                      const uint16_t* sub, int64_t lds, int rows, int n);
/* y = bf16(x * (1 + scale[n])): the model's modulation with its zero
 * shift; over one row it folds the block's scale into a norm gain
 * (fill_mod, ming-dit.cc:2266-2273). */
int ming_modulate(ming_ctx* ctx, const uint16_t* x, int64_t ldx,
                  const uint16_t* scale, uint16_t* y, int64_t ldy, int rows,
                  int n);
/* y = bf16(y + bias[n]), then silu when `silu` != 0 (bias, silu). */
int ming_bias_act(ming_ctx* ctx, uint16_t* y, int64_t ldy,
                  const uint16_t* bias, int rows, int n, int silu);
/* y = bf16(silu(x)) over n elements. */
int ming_silu(ming_ctx* ctx, const uint16_t* x, uint16_t* y, int n);
/* The final layer's LayerNorm (no affine) then * (1 + scale[n])
 * (ming-dit.cc:2553-2563, eps 1e-6 there). D % 8 == 0, D <= 8192, strides
 * % 8 == 0, pointers 16-byte aligned. */
int ming_ln_modulate(ming_ctx* ctx, const uint16_t* x, int64_t ldx,
                     const uint16_t* scale, uint16_t* y, int64_t ldy, int rows,
                     int D, float eps);

/* ---- the pack quantizer (ming-quant-family.cc:31-59's recipe target) -----------
 * Device f32 w [N, K] -> the pack layout ming_qweight_create reads: bits 8
 * symmetric (s = bf16(max|w|/127), code = clamp(rint(w/s), -127, 127) +
 * 128, bias = -128 s) or bits 4 affine (s = bf16((max-min)/15),
 * b = bf16(min), code = clamp(rint((w-b)/s), 0, 15)), group 64, codes
 * LSB-first. */
int ming_quantize_pack(ming_ctx* ctx, const float* w, int N, int K, int bits,
                       int group, uint32_t* codes, uint16_t* scales,
                       uint16_t* biases);

/* ---- block and model drivers ------------------------------------------------------
 * The reference's run_block, fill_mod and forward sequence (ming-dit.cc:2065-2273,
 * 2266-2281, 1490-2563) over the entry points above. Everything is borrowed:
 * weights, gains and biases stay owned by the caller and must outlive the
 * block call / the model. Gains and biases are bf16 device vectors. */
typedef struct ming_block_desc {
  /* [out][in]: q, k, v, o [H][H]; w1, w3 [ffn][H]; w2 [H][ffn] */
  const ming_qweight* q;
  const ming_qweight* k;
  const ming_qweight* v;
  const ming_qweight* o;
  const ming_qweight* w1;
  const ming_qweight* w3;
  const ming_qweight* w2;
  /* adaLN_modulation [4H][adaln_dim] + bias [4H] on modulated blocks (noise
   * refiner, layers); NULL on the context refiner, which is unmodulated */
  const ming_qweight* ada;
  const uint16_t* ada_b;
  /* attention_norm1/2, ffn_norm1/2 [H]; q/k norms [head_dim] */
  const uint16_t* an1;
  const uint16_t* an2;
  const uint16_t* fn1;
  const uint16_t* fn2;
  const uint16_t* nq;
  const uint16_t* nk;
} ming_block_desc;

typedef struct ming_block_dims {
  int hidden;      /* H; H / n_heads must be 128 */
  int n_heads;
  int ffn;
  int adaln_dim;
  float eps;       /* RMSNorm and qk-norm epsilon (1e-5) */
} ming_block_dims;

/* Workspace one ming_block_forward over `rows` rows needs (bytes). */
size_t ming_block_workspace_bytes(const ming_block_dims* dims, int rows);
/* One block, in place on x [rows][H] (row stride H): pre-norm (gain folded with
 * the adaLN scale on modulated blocks), q/k/v, qk-norm + RoPE (tables cos_t /
 * sin_t [rows][64] for these rows), attention, to_out, post-norm, gated (tanh)
 * or plain residual; then the SwiGLU feed-forward the same way. temb [adaln_dim]
 * is the adaLN input (modulated blocks only); scales are the 8 live strengths of
 * the LoRA slots bound on the projections (NULL: none). */
int ming_block_forward(ming_ctx* ctx, const ming_block_desc* b, const ming_block_dims* dims,
                       uint16_t* x, int rows, const float* cos_t, const float* sin_t,
                       const uint16_t* temb, const float* scales, void* ws,
                       size_t ws_bytes);

typedef struct ming_model ming_model;
typedef struct ming_model_desc {
  int hidden;        /* 3840 */
  int n_heads;       /* 30 (head_dim 128) */
  int ffn;           /* 10240 */
  int n_layers;      /* 30 main layers */
  int n_refiner;     /* 2 context-refiner and 2 noise-refiner blocks */
  int adaln_dim;     /* 256 */
  int time_freq;     /* 256 */
  int time_mid;      /* 1024 */
  int patch_dim;     /* 64 = patch^2 * in_channels */
  int cap_dim;       /* 2560: caption features of the query rows */
  float eps;         /* 1e-5 */
  float rope_theta;  /* 256 */
  float t_scale;     /* 1000 */
  int axes[3];       /* rotary dims per axis (32, 48, 48) */
  int axes_lens[3];  /* positions per axis must stay below these */
  const ming_block_desc* ctx_blocks;  /* [n_refiner], unmodulated */
  const ming_block_desc* blocks;      /* [n_refiner + n_layers]: noise refiner, layers */
  const ming_qweight* time_1;         /* t_embedder.mlp.0 [time_mid][time_freq] */
  const uint16_t* time_1b;
  const ming_qweight* time_2;         /* t_embedder.mlp.2 [adaln_dim][time_mid] */
  const uint16_t* time_2b;
  const ming_qweight* x_in;           /* x_embedder [H][patch_dim] */
  const uint16_t* x_in_b;
  const uint16_t* cap_norm;           /* cap_embedder.0 RMSNorm [cap_dim] */
  const ming_qweight* cap_in;         /* cap_embedder.1 [H][cap_dim] */
  const uint16_t* cap_in_b;
  const ming_qweight* final_ada;      /* final_layer.adaLN_modulation [H][adaln_dim] */
  const uint16_t* final_ada_b;
  const ming_qweight* final_lin;      /* final_layer.linear [patch_dim][H] */
  const uint16_t* final_lin_b;
} ming_model_desc;

/* MingDit::load over in-memory weights: validates the dimensions and every
 * weight's shape, refusing rather than degrading. */
int ming_model_create(ming_ctx* ctx, const ming_model_desc* d, ming_model** out);
int ming_model_destroy(ming_model* m);
/* set_lora_scale / lora_scale (ming-dit.cc:3024-3039): live between forwards. */
int ming_model_set_lora_scale(ming_model* m, int slot, float s);
float ming_model_lora_scale(const ming_model* m, int slot);
/* forward (ming-dit.cc:1490-2563): latents [img_tokens][patch_dim] and the
 * caption [cap_len][cap_stride] (rows < query_rows carry cap_dim features for
 * cap_embedder, the rest H-wide rows that bypass it) in device memory; the
 * joint layout's positions (host int32 [img_tokens + cap_len] per axis, image
 * rows first); out [img_tokens][patch_dim] device, the velocity before
 * negation. Synchronous: returns after the GPU finished. MING_ERR_RANGE when a
 * projection input could not be carried in fp16 on the context's route (the
 * output is then not valid; MING_ROUTE_WIDE runs such a forward). The range
 * report is the context's: one left pending by an earlier ming_lin / ming_ffn
 * that no ming_ctx_synchronize collected fails this forward too, so collect
 * it before. */
int ming_model_forward(ming_model* m, const uint16_t* latents, const uint16_t* cap,
                       int64_t cap_stride, int img_tokens, int cap_len, int query_rows,
                       const int32_t* pos_t, const int32_t* pos_h, const int32_t* pos_w,
                       float sigma, uint16_t* out);

/* ---- lifecycle (set_stream_stop, set_block_progress, set_caption_cache;
 * ming-dit.h:191-193, 221-223) ------------------------------------------------
 * stop: polled on the calling thread before every block; non-zero stops the
 * forward, which then returns MING_STOPPED with an empty error and leaves
 * `out` unwritten. While a stop callback is set the forward waits for the
 * GPU every 4 modulated blocks, so a stop is seen within a few blocks
 * (kStopDrainBlocks, ming-dit.cc:2530-2540). NULL clears it. */
typedef int (*ming_stop_fn)(void* user);
int ming_model_set_stream_stop(ming_model* m, ming_stop_fn fn, void* user);
/* progress(user, done, total): once per block, in order, done = 0 .. total-1
 * (blocks finished BEFORE that block; total = 2 * n_refiner + n_layers). A
 * report is made only after those blocks have finished on the GPU, on the
 * calling thread, before ming_model_forward returns. NULL clears it. */
typedef void (*ming_progress_fn)(void* user, int done, int total);
int ming_model_set_block_progress(ming_model* m, ming_progress_fn fn, void* user);
/* The per-caption cache (on by default): the context-refined caption rows of
 * the last two captions, keyed on the caption's exact bytes, length, query
 * rows and stride (ming-dit.cc:1543-1577). A hit skips cap_embedder and the
 * context refiner. A strength change on a slot bound in the context refiner,
 * and any rebinding, drops it. Off frees it. */
int ming_model_set_caption_cache(ming_model* m, int on);

/* ---- checkpoints and packs (load_qw_ + pack detection, ming-dit.cc:802-831,
 * 1115-1135; read_dit_config, ming-config.cc:90-137) -------------------------
 * A transformer directory: config.json (a DiffusionTransformer with the Ming
 * checkpoint contract) and one or more .safetensors files. A pack carries
 * `<name>.scales` beside its codes; quantization is read off the tensors,
 * not the config: group = dim / to_q.scales.cols, bits = codes.cols * 32 / K. */
typedef struct ming_dit_config {
  int dim, n_layers, n_refiner_layers, n_heads, n_kv_heads, in_channels;
  int patch, f_patch, cap_feat_dim, qk_norm;
  float norm_eps, rope_theta, t_scale;
  int axes_dims[3], axes_lens[3];
  int zero_masked;          /* alignment_padding_mode: 1 "zero_masked", 0 "learned" */
  int multi_frame_output;
  /* derived as the reference derives them (cfg_from_, ming-dit.cc:296-366) */
  int ffn_inner;            /* int(dim / 3 * 8) */
  int adaln_dim;            /* min(dim, 256) */
  int time_mid, time_freq;  /* 1024, 256 */
  int patch_dim;            /* f_patch * patch^2 * in_channels */
} ming_dit_config;

typedef struct ming_pack ming_pack;
/* Reads config.json and maps every .safetensors file (nothing is copied).
 * Refuses a directory that is not a Ming-Image transformer. */
int ming_pack_open(const char* transformer_dir, ming_pack** out);
int ming_pack_close(ming_pack* p);
int ming_pack_config(const ming_pack* p, ming_dit_config* out);
/* 4 or 8 for a pack, 0 for a dense checkpoint; group 64 for a pack. */
int ming_pack_quant_bits(const ming_pack* p);
int ming_pack_group(const ming_pack* p);
int ming_pack_tensor_count(const ming_pack* p);
/* Name of tensor i (file order), NULL past the end. */
const char* ming_pack_tensor_name(const ming_pack* p, int i);
/* dtype (e.g. "BF16", "U32"; 8 bytes with the NUL), shape (up to 8 dims). */
int ming_pack_tensor_info(const ming_pack* p, const char* name, char* dtype8,
                          int64_t* shape8, int* ndim);
/* Projections held quantized (codes + scales + biases): 270 in the 34-block model. */
int ming_pack_quantized_count(const ming_pack* p);
/* model-quantize for this family (ming-quant-family.cc:31-59): every 2-D float
 * tensor of the block stacks whose leaf is not a norm, at `bits` (4 affine or 8
 * symmetric, group 64, the recipe of ming_quantize_pack) as codes U32 + scales
 * + biases BF16; every other tensor BF16; config.json kept key for key with
 * "quantization": {"bits", "group_size": 64} and "_vpipe_component":
 * "ming-image-dit" added. Host only (no GPU); `threads` <= 0 uses all cores. */
int ming_pack_write(const char* src_dir, const char* dst_dir, int bits, int threads);

/* ---- runtime LoRA from adapter files (bind_loras_, ming-dit.cc:2918-3005) -----
 * One .safetensors per slot, POSITIONAL: spec i binds slot i, an empty or NULL
 * path leaves its slot unbound, specs past slot 8 are reported and ignored.
 * Module names are the model's own (`layers.<i>.attention.to_q`, ...,
 * `feed_forward.w2` over context_refiner / noise_refiner / layers), read under
 * the `transformer.`, `diffusion_model.` and `base_model.model.` prefixes,
 * with `.lora_A` / `.lora_B` (peft's `.lora_A.<adapter>` too) or kohya's
 * `lora_unet_<flattened>.lora_down` / `.lora_up`; an alpha (per module, or in
 * the file's metadata) folds alpha / rank into the delta. A name bound at the
 * wrong shape refuses the WHOLE slot; a slot that binds nothing is reported
 * loudly. Neither is an error: the base model runs. */
typedef struct ming_lora_spec {
  const char* path;
  float scale;
} ming_lora_spec;
/* The projections an adapter may bind: 7 x (2 * n_refiner + n_layers). */
int ming_lora_module_capacity(const ming_dit_config* cfg);
/* MingDit::load from a directory: config refusals (cfg_from_), shape checks,
 * every weight resident (quantized or dense as the checkpoint holds it), the
 * adapters bound. The model owns everything it loaded. */
int ming_model_load(ming_ctx* ctx, const char* transformer_dir, const ming_lora_spec* loras,
                    int n_loras, ming_model** out);
/* Binds adapter files to a model's projections (a loaded model, or one made by
 * ming_model_create, whose borrowed weights then carry the bindings). A slot a
 * spec names is unbound first; its strength is set to the spec's scale. */
int ming_model_bind_loras(ming_model* m, const ming_lora_spec* loras, int n_loras);
/* Projections slot `slot` bound; modules refused at the wrong shape; the
 * binding report (what the log said). */
int ming_model_lora_modules(const ming_model* m, int slot);
int ming_model_lora_skipped(const ming_model* m, int slot);
const char* ming_model_lora_report(const ming_model* m, int slot);

/* ---- the denoise loop (MingImageGenerator::generate, ming-generator.cc:352-577) -----
 * schedule_sigmas (ming-generator.cc:158-174): out[k] = f32(shift*u / (1 + (shift-1)*u)),
 * u = 1 - k/steps, k < steps, computed in double; out[steps] = 0. `out` holds steps+1. */
int ming_schedule_sigmas(int steps, float shift, float* out);

typedef struct ming_denoise_args {
  /* the positive caption (device bf16 [cap_len][cap_stride]) and its layout's
   * positions (host int32 [img_tokens + cap_len] per axis, image rows first) */
  const uint16_t* cap;
  int64_t cap_stride;
  int cap_len, query_rows;
  const int32_t *pos_t, *pos_h, *pos_w;
  /* the negative for classifier-free guidance: NULL is the reference's default,
   * the positive's shape times zero (then its layout is the positive's);
   * otherwise neg_len rows of the same stride and their own positions */
  const uint16_t* cap_neg;
  int neg_len, neg_query_rows;
  const int32_t *neg_pos_t, *neg_pos_h, *neg_pos_w;
  int img_tokens;
  int steps;                 /* forwards (11 by default in the reference) */
  float shift;               /* the checkpoint's static shift (6.0) */
  float guidance;            /* > 1 runs the negative and guides */
  double cfg_truncation;     /* guide while (1 - sigma) <= this (1.0: always) */
  double cfg_normalization;  /* > 0: clamp |guided| to this x |positive| */
} ming_denoise_args;

/* progress(user, step, steps) after each step; returning 0 stops the loop. */
typedef int (*ming_step_fn)(void* user, int step, int steps);

/* The flow-match Euler loop over the model, with the reference's host
 * arithmetic in f32: per step the latent is rounded to bf16 (NaN -> 0x7fc0),
 * v = forward(positive); when guided, v = p + g*(p - forward(negative)) with
 * the optional norm clamp; then latents += (sigma[i+1] - sigma[i]) * -v.
 * latents: host f32 [img_tokens][patch_dim], the packed noise in, the
 * denoised latent out. Returns MING_STOPPED when the model's stop callback or
 * `progress` stopped it (latents then hold the last completed step). */
int ming_model_denoise(ming_model* m, const ming_denoise_args* a, float* latents,
                       ming_step_fn progress, void* user);

#ifdef __cplusplus
}
#endif

#endif /* MING_DIT_AMD_H */
