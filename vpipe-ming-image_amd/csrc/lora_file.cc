// Runtime LoRA from adapter files: bind_loras_ (ming-dit.cc:2918-3005) over
// the model's own module names. The file reader restates the conventions
// that function's comment lists (ming-dit.cc:2893-2916) for the adapter
// reader it calls (lora::Adapter in the vpipe SDK, not part of the reference
// tree):
//   * module = the base tensor's path without `.weight`, optionally under a
//     `transformer.`, `diffusion_model.` or `base_model.model.` prefix;
//   * factors `<module>.lora_A.weight` / `.lora_B.weight` (diffusers, the
//     pipeline's and peft's default), peft's `.lora_A.<adapter>.weight`, the
//     older `.lora.down.weight` / `.lora.up.weight`, and kohya's
//     `lora_unet_<module with '.' -> '_'>.lora_down.weight` / `.lora_up.weight`;
//   * an alpha per module (`<module>.alpha`, a scalar) or once in the file's
//     metadata (`lora_alpha`, `alpha`, `ss_network_alpha`, or the
//     `lora_alpha` inside a diffusers `*lora_adapter_metadata` JSON string);
//     the delta is scaled by alpha / rank (the factor the reference folds
//     into A). No alpha: 1.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "json.h"
#include "model.h"
#include "rt.h"
#include "safetensors.h"

using ming::rt_fail;
using ming::rt_ok;

namespace {

struct Factors {
  const ming::st::Tensor* a = nullptr;  // down [r, K]
  const ming::st::Tensor* b = nullptr;  // up [N, r]
  const ming::st::Tensor* alpha = nullptr;
};

bool ends_with(const std::string& s, const std::string& t) {
  return s.size() >= t.size() && s.compare(s.size() - t.size(), t.size(), t) == 0;
}

std::string strip_prefixes(std::string m) {
  static const char* kPre[] = {"base_model.model.", "transformer.", "diffusion_model.",
                               "model.diffusion_model."};
  for (bool again = true; again;) {
    again = false;
    for (const char* p : kPre) {
      const size_t n = std::strlen(p);
      if (m.size() > n && m.compare(0, n, p) == 0) {
        m = m.substr(n);
        again = true;
      }
    }
  }
  return m;
}

std::string flatten(const std::string& m) {
  std::string f = m;
  for (char& c : f)
    if (c == '.') c = '_';
  return f;
}

// Splits a tensor name into (module key, role): role 'A', 'B' or 'a' (alpha);
// false for names that are not adapter factors. Kohya modules are keyed
// "kohya:<flattened>".
bool classify(const std::string& name, std::string* module, char* role) {
  struct Suffix {
    const char* s;
    char r;
  };
  static const Suffix kSuf[] = {{".lora_A.weight", 'A'},    {".lora_B.weight", 'B'},
                                {".lora_down.weight", 'A'}, {".lora_up.weight", 'B'},
                                {".lora.down.weight", 'A'}, {".lora.up.weight", 'B'},
                                {".alpha", 'a'}};
  std::string base;
  *role = 0;
  for (const Suffix& x : kSuf)
    if (ends_with(name, x.s)) {
      base = name.substr(0, name.size() - std::strlen(x.s));
      *role = x.r;
      break;
    }
  if (!*role) {
    // peft: <module>.lora_A.<adapter>.weight
    for (const char* tag : {".lora_A.", ".lora_B."}) {
      const size_t at = name.rfind(tag);
      if (at == std::string::npos || !ends_with(name, ".weight")) continue;
      const std::string mid = name.substr(at + 8, name.size() - 7 - (at + 8));
      if (mid.empty() || mid.find('.') != std::string::npos) continue;
      base = name.substr(0, at);
      *role = tag[6];
      break;
    }
  }
  if (!*role || base.empty()) return false;
  if (base.rfind("lora_unet_", 0) == 0) {
    *module = "kohya:" + base.substr(10);
    return true;
  }
  if (base.rfind("lora_transformer_", 0) == 0) {
    *module = "kohya:" + base.substr(17);
    return true;
  }
  *module = strip_prefixes(base);
  return true;
}

// The file-level alpha, when its metadata states one.
bool metadata_alpha(const std::map<std::string, std::string>* meta, double* alpha) {
  if (!meta) return false;
  for (const char* k : {"lora_alpha", "alpha", "ss_network_alpha"}) {
    auto it = meta->find(k);
    if (it == meta->end()) continue;
    char* e = nullptr;
    const double v = std::strtod(it->second.c_str(), &e);
    if (e != it->second.c_str() && std::isfinite(v)) {
      *alpha = v;
      return true;
    }
  }
  for (const auto& kv : *meta) {
    if (!ends_with(kv.first, "lora_adapter_metadata")) continue;
    ming::json::Value j;
    if (!ming::json::parse(kv.second.data(), kv.second.size(), &j, nullptr)) continue;
    const ming::json::Value* a = j.get("lora_alpha");
    if (a && a->is_num()) {
      *alpha = a->num;
      return true;
    }
  }
  return false;
}

double scalar_of(const ming::st::Tensor& t) {
  std::vector<float> v;
  if (t.numel() != 1 || !ming::st::to_f32(t, &v, nullptr)) return std::nan("");
  return (double)v[0];
}

// One slot: bind every module the file carries at the right shape; any name
// at the wrong shape refuses the whole slot.
int bind_slot(ming_model* m, int slot, const ming_lora_spec& spec) {
  const std::string path = spec.path;
  const std::string who = "ming-image DiT: lora '" + path + "'";
  ming::st::Set file;
  std::string err;
  if (!file.open_file(path, &err)) {
    m->lora_report[slot] = who + " could not be read (" + err + "); this slot stays empty";
    ming::rt_log(MING_LOG_WARN, m->lora_report[slot]);
    return MING_OK;
  }
  std::map<std::string, Factors> mods;
  for (const ming::st::Tensor* t : file.all()) {
    std::string mod;
    char role;
    if (!classify(t->name, &mod, &role)) continue;
    Factors& f = mods[mod];
    (role == 'A' ? f.a : role == 'B' ? f.b : f.alpha) = t;
  }
  double file_alpha = 0.0;
  const bool has_file_alpha = metadata_alpha(file.metadata(), &file_alpha);
  const std::vector<ming::ModuleRef> refs = ming::model_modules(m);
  // pass 1: every module the file names, at the right shape or not
  struct Bind {
    const ming::ModuleRef* ref;
    const Factors* f;
    int rank;
    double alpha;
  };
  std::vector<Bind> fits;
  int skipped = 0;
  for (const ming::ModuleRef& r : refs) {
    auto it = mods.find(r.name);
    if (it == mods.end()) it = mods.find("kohya:" + flatten(r.name));
    if (it == mods.end()) continue;
    const Factors& f = it->second;
    const ming::st::Tensor *A = f.a, *B = f.b;
    const bool shape_ok = A && B && A->shape.size() == 2 && B->shape.size() == 2 &&
                          A->shape[1] == r.K && B->shape[0] == r.N &&
                          A->shape[0] == B->shape[1] && A->shape[0] >= 1 &&
                          A->shape[0] <= MING_MAX_LORA_RANK;
    double alpha = shape_ok ? (double)A->shape[0] : 0.0;
    if (shape_ok && f.alpha) alpha = scalar_of(*f.alpha);
    else if (shape_ok && has_file_alpha) alpha = file_alpha;
    if (!shape_ok || !std::isfinite(alpha)) {
      ++skipped;
      continue;
    }
    fits.push_back({&r, &f, (int)A->shape[0], alpha});
  }
  if (skipped > 0) {
    // a name that fits at the wrong shape: the modules that fit are half an
    // adapter, not a weaker one (ming-dit.cc:2966-2979)
    m->lora_skipped[slot] = skipped;
    m->lora_modules[slot] = 0;
    m->lora_report[slot] = who + " left unbound: " + std::to_string(skipped) +
                           " of its modules have this model's names but other shapes (" +
                           std::to_string(fits.size()) +
                           " fit), so it belongs to another model; this slot stays empty";
    ming::rt_log(MING_LOG_WARN, m->lora_report[slot]);
    return rt_ok();
  }
  // pass 2: bind
  int bound = 0, rmin = 0, rmax = 0;
  for (const Bind& b : fits) {
    std::vector<uint16_t> a16, b16;
    if (!ming::st::to_bf16(*b.f->a, &a16, &err) || !ming::st::to_bf16(*b.f->b, &b16, &err)) {
      for (const ming::ModuleRef& r : refs) (void)ming_qweight_unbind_lora(r.qw, 0, slot);
      return rt_fail(MING_ERR_SHAPE, "ming_model_bind_loras: " + err);
    }
    const int rc = ming_qweight_bind_lora(b.ref->qw, 0, slot, b.rank, a16.data(), b16.data(),
                                          (float)(b.alpha / (double)b.rank), 0);
    if (rc != MING_OK) {
      const std::string why = ming_last_error();
      for (const ming::ModuleRef& r : refs) (void)ming_qweight_unbind_lora(r.qw, 0, slot);
      return rt_fail(rc, why);
    }
    ++bound;
    rmin = bound == 1 ? b.rank : std::min(rmin, b.rank);
    rmax = std::max(rmax, b.rank);
  }
  m->lora_modules[slot] = bound;
  m->lora_skipped[slot] = 0;
  if (bound == 0) {
    // loud: an adapter for another model would otherwise say nothing
    m->lora_report[slot] = who +
                           " matched zero modules: none of its names is one of this model's "
                           "projections in a known spelling; this slot stays empty";
    ming::rt_log(MING_LOG_WARN, m->lora_report[slot]);
  } else {
    char buf[160];
    std::snprintf(buf, sizeof buf, " slot %d: bound %d of %d modules, rank %d..%d, strength %g",
                  slot, bound, (int)refs.size(), rmin, rmax, (double)spec.scale);
    m->lora_report[slot] = who + buf;
    ming::rt_log(MING_LOG_INFO, m->lora_report[slot]);
  }
  return rt_ok();
}

}  // namespace

extern "C" {

int ming_model_bind_loras(ming_model* m, const ming_lora_spec* loras, int n) {
  if (!m || n < 0 || (n > 0 && !loras))
    return rt_fail(MING_ERR_ARG, "ming_model_bind_loras: bad arguments");
  const std::vector<ming::ModuleRef> refs = ming::model_modules(m);
  for (int slot = 0; slot < n; ++slot) {
    const ming_lora_spec& spec = loras[slot];
    const bool named = spec.path && *spec.path;
    if (slot >= MING_MAX_LORA_SLOTS) {
      if (named)
        ming::rt_log(MING_LOG_WARN, "ming_model_bind_loras: slot " + std::to_string(slot) +
                                        " is past the " + std::to_string(MING_MAX_LORA_SLOTS) +
                                        " slots; '" + spec.path + "' is ignored");
      continue;
    }
    if (!std::isfinite(spec.scale))
      return rt_fail(MING_ERR_ARG, "ming_model_bind_loras: strength must be finite");
    // positional: this slot now holds this spec (or nothing)
    for (const ming::ModuleRef& r : refs) (void)ming_qweight_unbind_lora(r.qw, 0, slot);
    m->lora_modules[slot] = 0;
    m->lora_skipped[slot] = 0;
    m->lora_report[slot].clear();
    m->scales[slot] = spec.scale;
    if (!named) continue;
    const int rc = bind_slot(m, slot, spec);
    if (rc != MING_OK) return rc;
  }
  ming::model_drop_caption_cache(m);
  return rt_ok();
}

int ming_model_lora_modules(const ming_model* m, int slot) {
  if (!m || slot < 0 || slot >= MING_MAX_LORA_SLOTS) return 0;
  return m->lora_modules[slot];
}

int ming_model_lora_skipped(const ming_model* m, int slot) {
  if (!m || slot < 0 || slot >= MING_MAX_LORA_SLOTS) return 0;
  return m->lora_skipped[slot];
}

const char* ming_model_lora_report(const ming_model* m, int slot) {
  if (!m || slot < 0 || slot >= MING_MAX_LORA_SLOTS) return "";
  return m->lora_report[slot].c_str();
}

}  // extern "C"
