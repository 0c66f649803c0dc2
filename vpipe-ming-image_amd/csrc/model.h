// The model object behind the ming_model_* entry points, shared by the
// drivers (model.hip), the checkpoint loader (pack.cc) and the adapter binder
// (lora_file.cc). Plain C++: device memory and HIP events are held as void*.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/ming_dit_amd.h"

struct ming_model {
  ming_ctx* ctx = nullptr;
  ming_model_desc d{};
  std::vector<ming_block_desc> ctx_blocks, blocks;
  float scales[MING_MAX_LORA_SLOTS] = {};
  // per-forward device planes, grown on demand
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int ws_rows = -1, ws_q = -1;
  uint16_t *joint = nullptr, *capn = nullptr, *tin = nullptr, *te1 = nullptr,
           *temb = nullptr, *tsilu = nullptr, *outmod = nullptr;
  float *cos_t = nullptr, *sin_t = nullptr;
  int32_t* pos = nullptr;
  void* premod = nullptr;   // every modulated block's adaLN results, made per forward
  void* blk_ws = nullptr;
  size_t blk_bytes = 0;
  std::vector<uint16_t> tin_host;

  // What a model loaded from a directory owns and frees (weights and the
  // device vectors of gains and biases); empty for ming_model_create.
  std::vector<ming_qweight*> own_qw;
  std::vector<void*> own_dev;

  // Runtime LoRA bound from files: per slot, projections bound, modules
  // refused at the wrong shape, and the binding report.
  int lora_modules[MING_MAX_LORA_SLOTS] = {};
  int lora_skipped[MING_MAX_LORA_SLOTS] = {};
  std::string lora_report[MING_MAX_LORA_SLOTS];

  // lifecycle
  ming_stop_fn stop = nullptr;
  void* stop_user = nullptr;
  ming_progress_fn progress = nullptr;
  void* progress_user = nullptr;
  std::vector<void*> block_events;  // hipEvent_t, one per block

  // the caption cache: two entries, least recently used refilled
  struct CapEntry {
    bool valid = false;
    int q = 0, len = 0;
    int64_t stride = 0;
    void* key = nullptr;  // the caption's bytes, on the device
    size_t key_bytes = 0, key_cap = 0;
    void* out = nullptr;  // the context-refined rows [len][H]
    size_t out_cap = 0;
    uint64_t tick = 0;
    // the caption path's weights' bind generations when it was filled
    uint64_t bind_sig = 0;
  };
  bool cap_cache_on = true;
  CapEntry cap[2];
  uint64_t cap_tick = 0;
  int* cap_flag = nullptr;  // device int for the key comparison
};

namespace ming {
// The model's adaptable projections by module name (the reference's
// bind_loras_ order: the modulated stack, then the context refiner), with
// each projection's weight and expected [N][K].
struct ModuleRef {
  std::string name;
  ming_qweight* qw;
  int N, K;
  bool ctx_refiner;
};
std::vector<ModuleRef> model_modules(const ming_model* m);
// Drops every caption cache entry (a rebinding or a strength change).
void model_drop_caption_cache(ming_model* m);
}  // namespace ming
