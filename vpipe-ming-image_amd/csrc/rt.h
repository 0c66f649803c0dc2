// Internal host-side hooks shared by the runtime's source files: the
// thread-local last-error reporting behind ming_last_error, the session log,
// device uploads and the context's device. Plain C++ (no HIP types), so the
// host-only sources include it too.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/ming_dit_amd.h"

namespace ming {
int rt_fail(int code, const std::string& why);
int rt_ok();
int rt_device(const ming_ctx* c);
// models hold their context like weights do: it refuses to go first
void rt_retain(ming_ctx* c);
void rt_release(ming_ctx* c);
// the session log (ming_set_log_sink); level MING_LOG_WARN / MING_LOG_INFO
void rt_log(int level, const std::string& msg);
// a device copy of `bytes` host bytes on the context's device (NULL for 0)
int rt_upload(ming_ctx* c, const void* host, size_t bytes, void** dev);
void rt_free(ming_ctx* c, void* dev);
int rt_alloc(ming_ctx* c, size_t bytes, bool zero, void** dev);
// ordered on the context's stream, and waited for
int rt_h2d(ming_ctx* c, void* dev, const void* host, size_t bytes);
int rt_d2h(ming_ctx* c, void* host, const void* dev, size_t bytes);
void rt_note_cap_hit(ming_ctx* c);
// a weight's bind generation (bumped by every ming_qweight_bind_lora / unbind)
uint64_t rt_qweight_bind_gen(const ming_qweight* q);
// After the stream has drained: MING_ERR_RANGE (counted, reason set, word
// cleared) when an fp16 copy met a value it cannot hold since the last check.
int rt_take_range_fault(ming_ctx* c, const char* who);
// Marks the fp16 activation copies written from here on as unread (a block
// whose projections are all dense); returns the previous mark.
bool rt_set_copies_unread(ming_ctx* c, bool unread);

// Fused forms the block driver uses (same bits as the public calls they
// replace):
// y = rmsnorm(x) and the context's fp16 copy of y, which the next projections
// over y then read instead of converting y themselves (rt_lin_xh, rt_ffn_xh
// are only valid while that copy still holds y: no other projection between);
int rt_rmsnorm_f16(ming_ctx* c, const uint16_t* x, int64_t ldx, const uint16_t* w,
                   uint16_t* y, int64_t ldy, int rows, int D, float eps);
int rt_lin_xh(ming_ctx* c, const ming_qweight* qw, const uint16_t* x, int64_t ldx,
              uint16_t* y, int64_t ldy, int M, const float* scales);
// ming_attention that also leaves the fp16 copy of its output in the
// context's plane, for rt_lin_xh over that output (the o-projection)
int rt_attention_xh(ming_ctx* c, const uint16_t* qkv, int64_t ld, int q_col, int k_col,
                    int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                    float scale);
// rt_attention_xh on raw q and k projection outputs: ming_qk_norm_rope's per-
// head RMSNorm + RoPE is applied to k by one pass (in place) and to q inside
// the attention kernel as it loads it, with the same bits.
int rt_attention_qknorm_xh(ming_ctx* c, uint16_t* qkv, int64_t ld, int q_col, int k_col,
                           int v_col, uint16_t* out, int64_t ldo, int rows, int n_heads,
                           float scale, const uint16_t* wq, const uint16_t* wk,
                           const float* cos_t, const float* sin_t, float eps);
// the three projections q, k, v over the same normed x, one x.A launch for
// their adapters, outputs y[i] with one row stride
int rt_lin3_xh(ming_ctx* c, const ming_qweight* const* qw, const uint16_t* x, int64_t ldx,
               uint16_t* const* y, int64_t ldy, int M, const float* scales);
int rt_ffn_xh(ming_ctx* c, const ming_qweight* w1, const ming_qweight* w3,
              const ming_qweight* w2, const uint16_t* x, int64_t ldx, uint16_t* y,
              int64_t ldy, int M, const float* scales, uint16_t* h, int64_t ldh);
// h = bf16(h + tgate * rmsnorm(sub)) with tgate = tanh(gate) from
// rt_tanh_gates (tgate NULL: h + rmsnorm(sub)), sub left as it was:
// ming_rmsnorm in place followed by ming_gated_residual / ming_residual_add.
int rt_norm_residual(ming_ctx* c, uint16_t* h, int64_t ldh, const uint16_t* sub,
                     int64_t lds, const uint16_t* w, const float* tgate, int rows, int D,
                     float eps);
// rt_norm_residual followed by rt_rmsnorm_f16 on the new h (weight wpre, into
// y and the context's fp16 copy), bit for bit, in one pass over the rows.
int rt_norm_residual_norm(ming_ctx* c, uint16_t* h, int64_t ldh, const uint16_t* sub,
                          int64_t lds, const uint16_t* wpost, const float* tgate,
                          const uint16_t* wpre, uint16_t* y, int64_t ldy, int rows, int D,
                          float eps);
// t[0, n) = tanh(mods[n, 2n)), t[n, 2n) = tanh(mods[3n, 4n)) in f32: a block's
// two residual gates, once per block instead of once per element.
int rt_tanh_gates(ming_ctx* c, const uint16_t* mods, int n, float* t);
// ming_bias_act (mode 0) on the block's adaLN output, the two ming_modulate
// gain folds and rt_tanh_gates, in one launch (the same bits as those four)
int rt_adaln_glue(ming_ctx* c, uint16_t* mods, int n, const uint16_t* b, const uint16_t* an1,
                  const uint16_t* fn1, uint16_t* nw1, uint16_t* nw3, float* t);
// Every modulated block's adaLN modulation of a forward at once (it depends
// on temb alone): mods[i] = ada[i](temb) + ada_b[i] and the glue of
// rt_adaln_glue, as one batched GEMV and one batched glue launch per 32
// blocks, each block's bits those of ming_lin + rt_adaln_glue. *done is
// false (nothing launched) when the per-block projections would not run the
// GEMV: another route, a live adapter on an adaLN weight, mixed shapes.
int rt_modulation_batch(ming_ctx* c, int count, const ming_qweight* const* ada,
                        const uint16_t* const* ada_b, const uint16_t* const* an1,
                        const uint16_t* const* fn1, const uint16_t* temb, int H,
                        uint16_t* const* mods, uint16_t* const* nw1, uint16_t* const* nw3,
                        float* const* tg, const float* scales, bool* done);
}  // namespace ming
