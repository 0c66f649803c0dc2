// Checkpoints and packs: the transformer directory's config.json
// (read_dit_config, ming-config.cc:90-137; cfg_from_, ming-dit.cc:296-366),
// pack detection (ming-dit.cc:1115-1135), load_qw_ (802-831) and the tensor
// names of the model (load_fixed_ 868-891, each_block_tensor_ 958-986,
// mod_prefix_ / ctx_prefix_ 676-694), the dense shape check (check_shapes_
// 900-942), and the pack writer for this family (ming-quant-family.cc:31-59).
// Host code only; weights reach the device through the library's own
// entry points (ming_qweight_create, rt_upload).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <new>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "json.h"
#include "model.h"
#include "rt.h"
#include "safetensors.h"

namespace fs = std::filesystem;
using ming::rt_fail;
using ming::rt_ok;

struct ming_pack {
  std::string dir;
  ming::json::Value config;  // config.json as read
  ming_dit_config cfg{};
  ming::st::Set tensors;
  int quant_bits = 0;   // read off block 0's to_q (0: dense)
  int quant_group = 0;
};

namespace {

#define RC(call)                    \
  do {                              \
    const int rc_ = (call);         \
    if (rc_ != MING_OK) return rc_; \
  } while (0)

// ---- config.json --------------------------------------------------------

int get_int(const ming::json::Value& o, const char* k, int d) {
  const ming::json::Value* v = o.get(k);
  return v && v->is_num() ? (int)v->num : d;
}
float get_real(const ming::json::Value& o, const char* k, float d) {
  const ming::json::Value* v = o.get(k);
  return v && v->is_num() ? (float)v->num : d;
}
bool get_bool(const ming::json::Value& o, const char* k, bool d) {
  const ming::json::Value* v = o.get(k);
  return v && v->is_bool() ? v->b : d;
}
std::string get_str(const ming::json::Value& o, const char* k) {
  const ming::json::Value* v = o.get(k);
  return v && v->is_str() ? v->str : std::string();
}
// An integer array, replaced wholesale when present.
std::vector<int> get_ints(const ming::json::Value& o, const char* k, std::vector<int> d) {
  const ming::json::Value* v = o.get(k);
  if (!v || !v->is_arr()) return d;
  std::vector<int> r;
  for (const auto& e : v->arr) r.push_back(e.is_num() ? (int)e.num : 0);
  return r;
}

bool read_json_file(const fs::path& p, ming::json::Value* out, std::string* why) {
  std::ifstream f(p, std::ios::binary);
  if (!f) return false;
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string t = ss.str();
  return ming::json::parse(t.data(), t.size(), out, why);
}

// read_dit_config (ming-config.cc:90-137) plus the derived widths of cfg_from_.
int read_config(const std::string& dir, ming::json::Value* t, ming_dit_config* d) {
  std::string jerr;
  if (!read_json_file(fs::path(dir) / "config.json", t, &jerr) || !t->is_obj())
    return rt_fail(MING_ERR_ARG, "'" + dir + "': config.json is missing or not a JSON object" +
                                     (jerr.empty() ? "" : " (" + jerr + ")"));
  if (get_str(*t, "_class_name") != "DiffusionTransformer")
    return rt_fail(MING_ERR_ARG, "config.json: _class_name must be DiffusionTransformer for this path");
  if (!t->get("alignment_padding_mode") || !t->get("multi_frame_output"))
    return rt_fail(MING_ERR_ARG,
                   "config.json: both alignment_padding_mode and multi_frame_output are "
                   "required keys of a Ming-Image DiT checkpoint, and one is absent");
  ming_dit_config c{};
  c.dim = get_int(*t, "dim", 3840);
  c.n_layers = get_int(*t, "n_layers", 30);
  c.n_refiner_layers = get_int(*t, "n_refiner_layers", 2);
  c.n_heads = get_int(*t, "n_heads", 30);
  c.n_kv_heads = get_int(*t, "n_kv_heads", 30);
  c.in_channels = get_int(*t, "in_channels", 16);
  c.cap_feat_dim = get_int(*t, "cap_feat_dim", 2560);
  c.norm_eps = get_real(*t, "norm_eps", 1e-5f);
  c.rope_theta = get_real(*t, "rope_theta", 256.0f);
  c.t_scale = get_real(*t, "t_scale", 1000.0f);
  c.qk_norm = get_bool(*t, "qk_norm", true) ? 1 : 0;
  const std::vector<int> ad = get_ints(*t, "axes_dims", {32, 48, 48});
  const std::vector<int> al = get_ints(*t, "axes_lens", {20480, 512, 512});
  const std::vector<int> ps = get_ints(*t, "all_patch_size", {2});
  const std::vector<int> fp = get_ints(*t, "all_f_patch_size", {1});
  c.patch = ps.empty() ? 2 : ps.front();
  c.f_patch = fp.empty() ? 1 : fp.front();
  const std::string pad = get_str(*t, "alignment_padding_mode");
  c.multi_frame_output = get_bool(*t, "multi_frame_output", false) ? 1 : 0;
  if (pad != "zero_masked" && pad != "learned")
    return rt_fail(MING_ERR_ARG, "config.json: alignment_padding_mode '" + pad +
                                     "' is neither zero_masked nor learned");
  c.zero_masked = pad == "zero_masked" ? 1 : 0;
  if (ad.size() != 3 || al.size() != 3 || c.n_heads <= 0 || c.dim % c.n_heads != 0)
    return rt_fail(MING_ERR_ARG, "config.json: axes need three dims and three lengths, and dim "
                                 "a positive multiple of n_heads");
  for (int i = 0; i < 3; ++i) {
    c.axes_dims[i] = ad[(size_t)i];
    c.axes_lens[i] = al[(size_t)i];
  }
  c.ffn_inner = (int)((double)c.dim / 3.0 * 8.0);
  c.adaln_dim = std::min(c.dim, 256);
  c.time_mid = 1024;
  c.time_freq = 256;
  c.patch_dim = c.f_patch * c.patch * c.patch * c.in_channels;
  *d = c;
  return MING_OK;
}

// The refusals of cfg_from_ (ming-dit.cc:296-366): everything this path does
// not run is refused by name.
int check_config(const ming_dit_config& d) {
  auto no = [](const std::string& m) { return rt_fail(MING_ERR_SHAPE, "ming_model_load: " + m); };
  if (d.n_heads <= 0 || d.dim <= 0 || d.dim % d.n_heads != 0)
    return no("the model width does not split evenly into its heads");
  if (d.n_kv_heads != d.n_heads)
    return no("grouped keys (n_kv_heads differing from n_heads) are outside this path");
  if (!d.zero_masked)
    return no("learned caption padding is outside this path (it runs zero_masked padding)");
  if (d.multi_frame_output) return no("a multi-frame checkpoint is outside this path (one frame)");
  if (!d.qk_norm) return no("a checkpoint without per-head q/k norms is outside this path");
  if (d.f_patch != 1 || d.patch <= 0)
    return no("the frame patch must be 1 and the spatial patch positive");
  if (d.axes_dims[0] + d.axes_dims[1] + d.axes_dims[2] != d.dim / d.n_heads)
    return no("the three rotary axis widths must add up to the head width");
  if (d.dim / d.n_heads != 128)
    return no("heads of width " + std::to_string(d.dim / d.n_heads) +
              ": the attention kernel takes 128-wide heads only");
  if (d.n_layers <= 0 || d.n_refiner_layers <= 0 || d.cap_feat_dim <= 0 || d.in_channels <= 0)
    return no("layer counts, caption width and input channels must all be above zero");
  return MING_OK;
}

std::string mod_prefix(const ming_dit_config& c, int i) {
  if (i < c.n_refiner_layers) return "noise_refiner." + std::to_string(i) + ".";
  return "layers." + std::to_string(i - c.n_refiner_layers) + ".";
}
std::string ctx_prefix(int i) { return "context_refiner." + std::to_string(i) + "."; }
std::string patch_key(const ming_dit_config& c) {
  return std::to_string(c.patch) + "-" + std::to_string(c.f_patch);
}

// Pack detection (ming-dit.cc:1115-1135): block 0's to_q carries `.scales`
// beside its codes in a pack; group = dim / scales.cols, bits = codes.cols *
// 32 / K, and anything but 4 or 8 reads as dense.
int detect(ming_pack* p) {
  const std::string p0 = mod_prefix(p->cfg, 0);
  const ming::st::Tensor* si = p->tensors.find(p0 + "attention.to_q.scales");
  const ming::st::Tensor* ci = p->tensors.find(p0 + "attention.to_q.weight");
  if (!ci)
    return rt_fail(MING_ERR_ARG, "the first block's query weight '" + p0 +
                                 "attention.to_q.weight' is absent: the tensors are not this "
                                 "model's transformer");
  p->quant_bits = 0;
  p->quant_group = 0;
  if (si && si->shape.size() == 2 && ci->shape.size() == 2 && si->shape[1] > 0) {
    int g = (int)(p->cfg.dim / si->shape[1]);
    if (g <= 0) g = 64;
    const long K = (long)si->shape[1] * g;
    const int bits = K > 0 ? (int)(ci->shape[1] * 32 / K) : 0;
    if (bits == 4 || bits == 8) {
      p->quant_bits = bits;
      p->quant_group = g;
    }
  }
  return MING_OK;
}

// check_shapes_ (ming-dit.cc:900-942): a DENSE checkpoint's model-level and
// block-0 widths against the config, by name.
int check_dense_shapes(const ming_pack* p) {
  if (p->quant_bits > 0) return MING_OK;
  const ming_dit_config& c = p->cfg;
  const std::string pk = patch_key(c), b0 = mod_prefix(c, 0);
  const struct {
    std::string name;
    long rows, cols;
  } want[] = {
      {"all_x_embedder." + pk + ".weight", c.dim, c.patch_dim},
      {"cap_embedder.1.weight", c.dim, c.cap_feat_dim},
      {"t_embedder.mlp.0.weight", c.time_mid, c.time_freq},
      {"t_embedder.mlp.2.weight", c.adaln_dim, c.time_mid},
      {"all_final_layer." + pk + ".linear.weight", c.patch_dim, c.dim},
      {b0 + "attention.to_q.weight", c.dim, c.dim},
      {b0 + "feed_forward.w1.weight", c.ffn_inner, c.dim},
      {b0 + "feed_forward.w2.weight", c.dim, c.ffn_inner},
      {b0 + "adaLN_modulation.0.weight", 4L * c.dim, c.adaln_dim},
  };
  for (const auto& x : want) {
    const ming::st::Tensor* t = p->tensors.find(x.name);
    if (!t || t->shape.size() != 2 || t->shape[0] != x.rows || t->shape[1] != x.cols)
      return rt_fail(MING_ERR_SHAPE,
                     x.name + (t ? ": expected " + std::to_string(x.rows) + " x " +
                                       std::to_string(x.cols) + " from config.json"
                                 : " is missing"));
  }
  return MING_OK;
}

// ---- the pack writer's quantizer ------------------------------------------
//
// The recipe of ming_quantize_pack, on the host: per row and 64-wide group,
// w8 symmetric (s = bf16(max|w| / 127), q = clamp(rint(w / s), -127, 127),
// code q + 128, bias = bf16(-128 s)) or w4 affine (s = bf16((max - min) / 15),
// b = bf16(min), q = clamp(rint((w - b) / s), 0, 15)); codes LSB-first.

uint16_t bf16_bits(float f) { return ming::st::f32_to_bf16_narrow(f); }
float bf16_f(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

void quantize_rows(const float* w, int r0, int r1, int K, int bits, uint32_t* codes,
                   uint16_t* scales, uint16_t* biases) {
  const int G = K / 64, words = K * bits / 32, gw = 64 * bits / 32;
  for (int n = r0; n < r1; ++n)
    for (int g = 0; g < G; ++g) {
      const float* wr = w + (size_t)n * K + (size_t)g * 64;
      uint32_t* cr = codes + (size_t)n * words + (size_t)g * gw;
      if (bits == 8) {
        float amax = 0.0f;
        for (int j = 0; j < 64; ++j) amax = std::fmax(amax, std::fabs(wr[j]));
        const uint16_t sb = bf16_bits(amax / 127.0f);
        const float s = bf16_f(sb);
        scales[(size_t)n * G + g] = sb;
        biases[(size_t)n * G + g] = bf16_bits(-128.0f * s);
        for (int wd = 0; wd < 16; ++wd) {
          uint32_t o = 0;
          for (int i = 0; i < 4; ++i) {
            float q = s > 0.0f ? std::rint(wr[4 * wd + i] / s) : 0.0f;
            q = std::fmin(std::fmax(q, -127.0f), 127.0f);
            o |= (uint32_t)((int)q + 128) << (8 * i);
          }
          cr[wd] = o;
        }
      } else {
        float mn = wr[0], mx = wr[0];
        for (int j = 1; j < 64; ++j) {
          mn = std::fmin(mn, wr[j]);
          mx = std::fmax(mx, wr[j]);
        }
        const uint16_t sb = bf16_bits((mx - mn) / 15.0f), bb = bf16_bits(mn);
        const float s = bf16_f(sb), b = bf16_f(bb);
        scales[(size_t)n * G + g] = sb;
        biases[(size_t)n * G + g] = bb;
        for (int wd = 0; wd < 8; ++wd) {
          uint32_t o = 0;
          for (int i = 0; i < 8; ++i) {
            float q = s > 0.0f ? std::rint((wr[8 * wd + i] - b) / s) : 0.0f;
            q = std::fmin(std::fmax(q, 0.0f), 15.0f);
            o |= (uint32_t)q << (4 * i);
          }
          cr[wd] = o;
        }
      }
    }
}

bool is_float(const std::string& dt) {
  return dt == "F32" || dt == "F16" || dt == "BF16" || dt == "F64";
}

// The family's selection (ming-quant-family.cc:31-59): scope "." (every
// tensor), 2-D float `.weight` tensors whose leaf is not a norm or an
// embedding and whose width 64 divides, minus the model level
// (all_x_embedder, cap_embedder, t_embedder., all_final_layer).
bool selected(const ming::st::Tensor& t) {
  static const char* kExclude[] = {"all_x_embedder", "cap_embedder", "t_embedder.",
                                   "all_final_layer"};
  const std::string& n = t.name;
  if (n.size() < 7 || n.compare(n.size() - 7, 7, ".weight") != 0) return false;
  if (t.shape.size() != 2 || !is_float(t.dtype) || t.shape[1] % 64 != 0 || t.shape[1] <= 0)
    return false;
  const std::string base = n.substr(0, n.size() - 7);
  if (base.find("norm") != std::string::npos || base.find("embed") != std::string::npos)
    return false;
  for (const char* e : kExclude)
    if (n.find(e) != std::string::npos) return false;
  return true;
}

// ---- loading --------------------------------------------------------------

struct Loader {
  ming_ctx* ctx;
  const ming_pack* p;
  std::vector<ming_qweight*> qw;
  std::vector<void*> dev;

  // Frees whatever was not handed to a model. The destroy calls reset the
  // thread's error string, so a failure's reason is kept across them.
  int release(int rc) {
    const std::string why = ming_last_error();
    for (ming_qweight* q : qw) (void)ming_qweight_destroy(q);
    for (void* d : dev) ming::rt_free(ctx, d);
    qw.clear();
    dev.clear();
    return rc == MING_OK ? rt_ok() : rt_fail(rc, why);
  }

  const ming::st::Tensor* need(const std::string& n, int* rc) {
    const ming::st::Tensor* t = p->tensors.find(n);
    if (!t) *rc = rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + n + "' is absent from the checkpoint");
    return t;
  }

  // load_qw_ (ming-dit.cc:802-831): codes + bf16 scales/biases when the pack
  // holds them, else the dense `.weight` narrowed to bf16.
  int qweight(const std::string& name, const ming_qweight** out) {
    int rc = MING_OK;
    const ming::st::Tensor* ci = need(name + ".weight", &rc);
    if (!ci) return rc;
    const ming::st::Tensor* si = p->tensors.find(name + ".scales");
    ming_qweight* q = nullptr;
    std::string why;
    if (p->quant_bits > 0 && si && si->shape.size() == 2 && ci->shape.size() == 2) {
      const long K = (long)si->shape[1] * p->quant_group;
      const int bits = K > 0 ? (int)(ci->shape[1] * 32 / K) : 0;
      if (bits != 4 && bits != 8)
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + name + "' is neither w4 nor w8 (" +
                                           std::to_string(ci->shape[1]) + " words per row)");
      if (ci->dtype != "U32")
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + name + ".weight' codes are " +
                                           ci->dtype + ", not U32");
      const ming::st::Tensor* bi = need(name + ".biases", &rc);
      if (!bi) return rc;
      if (si->shape[0] != ci->shape[0] || bi->shape != si->shape)
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + name +
                                           "' scales/biases do not match its codes");
      std::vector<uint16_t> sc, bs;
      if (!ming::st::to_bf16(*si, &sc, &why) || !ming::st::to_bf16(*bi, &bs, &why))
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: " + why);
      RC(ming_qweight_create(ctx, (int)ci->shape[0], (int)K, bits, p->quant_group,
                             reinterpret_cast<const uint32_t*>(ci->data), sc.data(), bs.data(),
                             0, &q));
    } else {
      if (ci->shape.size() != 2)
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + name + ".weight' is not 2-D");
      std::vector<uint16_t> w;
      if (!ming::st::to_bf16(*ci, &w, &why))
        return rt_fail(MING_ERR_SHAPE, "ming_model_load: " + why);
      RC(ming_qweight_create_dense(ctx, (int)ci->shape[0], (int)ci->shape[1], w.data(), 0, &q));
    }
    qw.push_back(q);
    *out = q;
    return MING_OK;
  }

  // A bf16 vector (a gain or a bias) of `len` elements, resident.
  int vec(const std::string& name, int64_t len, const uint16_t** out) {
    int rc = MING_OK;
    const ming::st::Tensor* t = need(name, &rc);
    if (!t) return rc;
    if (t->numel() != len)
      return rt_fail(MING_ERR_SHAPE, "ming_model_load: '" + name + "' has " +
                                         std::to_string(t->numel()) + " elements, not " +
                                         std::to_string(len));
    std::vector<uint16_t> v;
    std::string why;
    if (!ming::st::to_bf16(*t, &v, &why)) return rt_fail(MING_ERR_SHAPE, "ming_model_load: " + why);
    void* d = nullptr;
    RC(ming::rt_upload(ctx, v.data(), v.size() * 2, &d));
    dev.push_back(d);
    *out = static_cast<const uint16_t*>(d);
    return MING_OK;
  }

  // load_block_ (ming-dit.cc:843-866) over each_block_tensor_'s names.
  int block(const std::string& pre, bool with_ada, ming_block_desc* b) {
    const ming_dit_config& c = p->cfg;
    *b = ming_block_desc{};
    RC(qweight(pre + "attention.to_q", &b->q));
    RC(qweight(pre + "attention.to_k", &b->k));
    RC(qweight(pre + "attention.to_v", &b->v));
    RC(qweight(pre + "attention.to_out.0", &b->o));
    RC(vec(pre + "attention.norm_q.weight", c.dim / c.n_heads, &b->nq));
    RC(vec(pre + "attention.norm_k.weight", c.dim / c.n_heads, &b->nk));
    RC(qweight(pre + "feed_forward.w1", &b->w1));
    RC(qweight(pre + "feed_forward.w3", &b->w3));
    RC(qweight(pre + "feed_forward.w2", &b->w2));
    RC(vec(pre + "attention_norm1.weight", c.dim, &b->an1));
    RC(vec(pre + "attention_norm2.weight", c.dim, &b->an2));
    RC(vec(pre + "ffn_norm1.weight", c.dim, &b->fn1));
    RC(vec(pre + "ffn_norm2.weight", c.dim, &b->fn2));
    if (with_ada) {
      // `.0`: a bare Linear; the final layer's adaLN is `.1`
      RC(qweight(pre + "adaLN_modulation.0", &b->ada));
      RC(vec(pre + "adaLN_modulation.0.bias", 4LL * c.dim, &b->ada_b));
    }
    return MING_OK;
  }
};

int load_model(Loader& ld, ming_model** out);

int open_pack(const char* dir, ming_pack** out) {
  auto* p = new (std::nothrow) ming_pack();
  if (!p) return rt_fail(MING_ERR_ALLOC, "ming_pack_open: out of host memory");
  p->dir = dir;
  int rc = read_config(p->dir, &p->config, &p->cfg);
  std::string why;
  if (rc == MING_OK && !p->tensors.open_dir(p->dir, &why))
    rc = rt_fail(MING_ERR_ARG, "ming_pack_open: " + why);
  if (rc == MING_OK) rc = detect(p);
  if (rc != MING_OK) {
    delete p;
    return rc;
  }
  *out = p;
  return rt_ok();
}

}  // namespace

extern "C" {

int ming_pack_open(const char* transformer_dir, ming_pack** out) {
  if (!transformer_dir || !out) return rt_fail(MING_ERR_ARG, "ming_pack_open: null argument");
  *out = nullptr;
  return open_pack(transformer_dir, out);
}

int ming_pack_close(ming_pack* p) {
  delete p;
  return rt_ok();
}

int ming_pack_config(const ming_pack* p, ming_dit_config* out) {
  if (!p || !out) return rt_fail(MING_ERR_ARG, "ming_pack_config: null argument");
  *out = p->cfg;
  return rt_ok();
}

int ming_pack_quant_bits(const ming_pack* p) { return p ? p->quant_bits : 0; }
int ming_pack_group(const ming_pack* p) { return p ? p->quant_group : 0; }
int ming_pack_tensor_count(const ming_pack* p) { return p ? (int)p->tensors.all().size() : 0; }

const char* ming_pack_tensor_name(const ming_pack* p, int i) {
  if (!p || i < 0 || i >= (int)p->tensors.all().size()) return nullptr;
  return p->tensors.all()[(size_t)i]->name.c_str();
}

int ming_pack_tensor_info(const ming_pack* p, const char* name, char* dtype8, int64_t* shape8,
                          int* ndim) {
  if (!p || !name) return rt_fail(MING_ERR_ARG, "ming_pack_tensor_info: null argument");
  const ming::st::Tensor* t = p->tensors.find(name);
  if (!t) return rt_fail(MING_ERR_ARG, std::string("ming_pack_tensor_info: no tensor '") + name + "'");
  if (t->shape.size() > 8) return rt_fail(MING_ERR_SHAPE, "ming_pack_tensor_info: more than 8 dims");
  if (dtype8) {
    std::memset(dtype8, 0, 8);
    std::strncpy(dtype8, t->dtype.c_str(), 7);
  }
  if (shape8)
    for (size_t i = 0; i < t->shape.size(); ++i) shape8[i] = t->shape[i];
  if (ndim) *ndim = (int)t->shape.size();
  return rt_ok();
}

int ming_pack_quantized_count(const ming_pack* p) {
  if (!p) return 0;
  int n = 0;
  for (const ming::st::Tensor* t : p->tensors.all()) {
    const std::string& nm = t->name;
    if (nm.size() < 7 || nm.compare(nm.size() - 7, 7, ".weight") != 0) continue;
    const std::string base = nm.substr(0, nm.size() - 7);
    if (t->dtype == "U32" && p->tensors.find(base + ".scales") && p->tensors.find(base + ".biases"))
      ++n;
  }
  return n;
}

int ming_lora_module_capacity(const ming_dit_config* c) {
  if (!c) return 0;
  return 7 * (2 * c->n_refiner_layers + c->n_layers);
}

int ming_pack_write(const char* src_dir, const char* dst_dir, int bits, int threads) {
  if (!src_dir || !dst_dir) return rt_fail(MING_ERR_ARG, "ming_pack_write: null argument");
  if (bits != 4 && bits != 8) return rt_fail(MING_ERR_ARG, "ming_pack_write: bits must be 4 or 8");
  ming_pack* p = nullptr;
  RC(ming_pack_open(src_dir, &p));
  std::unique_ptr<ming_pack> hold(p);
  if (p->config.get("quantization") || p->quant_bits > 0)
    return rt_fail(MING_ERR_STATE, "ming_pack_write: '" + std::string(src_dir) +
                                       "' is already a pack");
  std::error_code ec;
  if (fs::exists(dst_dir, ec) && fs::equivalent(src_dir, dst_dir, ec))
    return rt_fail(MING_ERR_ARG, "ming_pack_write: the pack cannot overwrite its source");
  fs::create_directories(dst_dir, ec);
  if (ec) return rt_fail(MING_ERR_ARG, "ming_pack_write: cannot create '" + std::string(dst_dir) + "'");
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());

  // the plan: every output tensor's name, dtype, shape and source
  struct Out {
    std::string name, dtype;
    std::vector<int64_t> shape;
    size_t bytes;
    const ming::st::Tensor* src;
    int role;  // 0 copy narrowed to BF16, 1 codes, 2 scales, 3 biases, 4 raw copy
  };
  std::vector<Out> plan;
  for (const ming::st::Tensor* t : p->tensors.all()) {
    if (selected(*t)) {
      const std::string base = t->name.substr(0, t->name.size() - 7);
      const int64_t N = t->shape[0], K = t->shape[1];
      plan.push_back({t->name, "U32", {N, K * bits / 32}, (size_t)(N * K * bits / 8), t, 1});
      plan.push_back({base + ".scales", "BF16", {N, K / 64}, (size_t)(N * (K / 64) * 2), t, 2});
      plan.push_back({base + ".biases", "BF16", {N, K / 64}, (size_t)(N * (K / 64) * 2), t, 3});
    } else if (is_float(t->dtype)) {
      plan.push_back({t->name, "BF16", t->shape, (size_t)t->numel() * 2, t, 0});
    } else {
      plan.push_back({t->name, t->dtype, t->shape, t->bytes, t, 4});
    }
  }
  // header
  ming::json::Value h = ming::json::Value::object();
  {
    ming::json::Value m = ming::json::Value::object();
    m.set("format", ming::json::Value::string("pt"));
    h.set("__metadata__", std::move(m));
  }
  size_t off = 0;
  for (const Out& o : plan) {
    ming::json::Value e = ming::json::Value::object();
    e.set("dtype", ming::json::Value::string(o.dtype));
    ming::json::Value sh = ming::json::Value::array();
    for (int64_t d : o.shape) sh.arr.push_back(ming::json::Value::number((double)d));
    e.set("shape", std::move(sh));
    ming::json::Value ofs = ming::json::Value::array();
    ofs.arr.push_back(ming::json::Value::number((double)off));
    ofs.arr.push_back(ming::json::Value::number((double)(off + o.bytes)));
    e.set("data_offsets", std::move(ofs));
    h.set(o.name, std::move(e));
    off += o.bytes;
  }
  std::string hdr = ming::json::dump(h);
  while (hdr.size() % 8) hdr.push_back(' ');
  const fs::path out_file = fs::path(dst_dir) / "diffusion_pytorch_model.safetensors";
  std::ofstream f(out_file, std::ios::binary | std::ios::trunc);
  if (!f) return rt_fail(MING_ERR_ARG, "ming_pack_write: cannot write '" + out_file.string() + "'");
  const uint64_t hl = hdr.size();
  f.write(reinterpret_cast<const char*>(&hl), 8);
  f.write(hdr.data(), (std::streamsize)hdr.size());
  // data, one source tensor at a time (a quantized matrix writes its three
  // outputs from one pass)
  std::string why;
  for (size_t i = 0; i < plan.size(); ++i) {
    const Out& o = plan[i];
    if (o.role == 4) {
      f.write(reinterpret_cast<const char*>(o.src->data), (std::streamsize)o.bytes);
    } else if (o.role == 0) {
      std::vector<uint16_t> v;
      if (!ming::st::to_bf16(*o.src, &v, &why)) return rt_fail(MING_ERR_SHAPE, "ming_pack_write: " + why);
      f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)o.bytes);
    } else if (o.role == 1) {
      std::vector<float> w;
      if (!ming::st::to_f32(*o.src, &w, &why)) return rt_fail(MING_ERR_SHAPE, "ming_pack_write: " + why);
      const int N = (int)o.src->shape[0], K = (int)o.src->shape[1];
      std::vector<uint32_t> codes((size_t)N * K * bits / 32);
      std::vector<uint16_t> sc((size_t)N * (K / 64)), bs((size_t)N * (K / 64));
      const int nt = std::max(1, std::min(threads, N));
      std::vector<std::thread> pool;
      for (int t = 0; t < nt; ++t) {
        const int r0 = (int)((long)N * t / nt), r1 = (int)((long)N * (t + 1) / nt);
        pool.emplace_back(quantize_rows, w.data(), r0, r1, K, bits, codes.data(), sc.data(),
                          bs.data());
      }
      for (auto& th : pool) th.join();
      f.write(reinterpret_cast<const char*>(codes.data()), (std::streamsize)(codes.size() * 4));
      f.write(reinterpret_cast<const char*>(sc.data()), (std::streamsize)(sc.size() * 2));
      f.write(reinterpret_cast<const char*>(bs.data()), (std::streamsize)(bs.size() * 2));
      i += 2;  // scales and biases written with the codes
    }
  }
  f.close();
  if (!f) return rt_fail(MING_ERR_ARG, "ming_pack_write: '" + out_file.string() + "' could not be written in full");
  // config.json, every key kept, the quantization block and the component tag added
  ming::json::Value cfg = p->config;
  ming::json::Value q = ming::json::Value::object();
  q.set("bits", ming::json::Value::number(bits));
  q.set("group_size", ming::json::Value::number(64));
  cfg.set("quantization", std::move(q));
  cfg.set("_vpipe_component", ming::json::Value::string("ming-image-dit"));
  std::ofstream cf(fs::path(dst_dir) / "config.json", std::ios::trunc);
  cf << ming::json::dump(cfg, 2) << "\n";
  cf.close();
  if (!cf) return rt_fail(MING_ERR_ARG, "ming_pack_write: config.json could not be written");
  return rt_ok();
}

int ming_model_load(ming_ctx* ctx, const char* dir, const ming_lora_spec* loras, int n_loras,
                    ming_model** out) {
  if (!ctx || !dir || !out || n_loras < 0 || (n_loras > 0 && !loras))
    return rt_fail(MING_ERR_ARG, "ming_model_load: bad arguments");
  *out = nullptr;
  ming_pack* p = nullptr;
  RC(ming_pack_open(dir, &p));
  std::unique_ptr<ming_pack> hold(p);
  RC(check_config(p->cfg));
  RC(check_dense_shapes(p));
  if (p->quant_bits > 0 && p->quant_group != 64)
    return rt_fail(MING_ERR_SHAPE, "ming_model_load: group " + std::to_string(p->quant_group) +
                                       " -- the kernels here read group-64 packs");
  Loader ld{ctx, p, {}, {}};
  ming_model* m = nullptr;
  const int rc = load_model(ld, &m);
  if (rc != MING_OK) return ld.release(rc);
  if (n_loras > 0) {
    const int brc = ming_model_bind_loras(m, loras, n_loras);
    if (brc != MING_OK) {
      const std::string why = ming_last_error();
      (void)ming_model_destroy(m);
      return rt_fail(brc, why);
    }
  }
  *out = m;
  return rt_ok();
}

}  // extern "C"

namespace {

// Every weight of the model resident, then ming_model_create; on success the
// model owns what the loader made.
int load_model(Loader& ld, ming_model** out) {
  const ming_pack* p = ld.p;
  ming_ctx* ctx = ld.ctx;
  const ming_dit_config& c = p->cfg;
  std::vector<ming_block_desc> ctx_blocks((size_t)c.n_refiner_layers);
  std::vector<ming_block_desc> blocks((size_t)(c.n_refiner_layers + c.n_layers));
  for (int i = 0; i < c.n_refiner_layers; ++i)
    RC(ld.block(ctx_prefix(i), false, &ctx_blocks[(size_t)i]));
  for (int L = 0; L < c.n_refiner_layers + c.n_layers; ++L)
    RC(ld.block(mod_prefix(c, L), true, &blocks[(size_t)L]));
  ming_model_desc d{};
  d.hidden = c.dim;
  d.n_heads = c.n_heads;
  d.ffn = c.ffn_inner;
  d.n_layers = c.n_layers;
  d.n_refiner = c.n_refiner_layers;
  d.adaln_dim = c.adaln_dim;
  d.time_freq = c.time_freq;
  d.time_mid = c.time_mid;
  d.patch_dim = c.patch_dim;
  d.cap_dim = c.cap_feat_dim;
  d.eps = c.norm_eps;
  d.rope_theta = c.rope_theta;
  d.t_scale = c.t_scale;
  for (int i = 0; i < 3; ++i) {
    d.axes[i] = c.axes_dims[i];
    d.axes_lens[i] = c.axes_lens[i];
  }
  d.ctx_blocks = ctx_blocks.data();
  d.blocks = blocks.data();
  // load_fixed_ (ming-dit.cc:868-891)
  const std::string pk = patch_key(c);
  RC(ld.qweight("all_x_embedder." + pk, &d.x_in));
  RC(ld.vec("all_x_embedder." + pk + ".bias", c.dim, &d.x_in_b));
  RC(ld.vec("cap_embedder.0.weight", c.cap_feat_dim, &d.cap_norm));
  RC(ld.qweight("cap_embedder.1", &d.cap_in));
  RC(ld.vec("cap_embedder.1.bias", c.dim, &d.cap_in_b));
  RC(ld.qweight("t_embedder.mlp.0", &d.time_1));
  RC(ld.vec("t_embedder.mlp.0.bias", c.time_mid, &d.time_1b));
  RC(ld.qweight("t_embedder.mlp.2", &d.time_2));
  RC(ld.vec("t_embedder.mlp.2.bias", c.adaln_dim, &d.time_2b));
  RC(ld.qweight("all_final_layer." + pk + ".adaLN_modulation.1", &d.final_ada));
  RC(ld.vec("all_final_layer." + pk + ".adaLN_modulation.1.bias", c.dim, &d.final_ada_b));
  RC(ld.qweight("all_final_layer." + pk + ".linear", &d.final_lin));
  RC(ld.vec("all_final_layer." + pk + ".linear.bias", c.patch_dim, &d.final_lin_b));
  ming_model* m = nullptr;
  RC(ming_model_create(ctx, &d, &m));
  m->own_qw.swap(ld.qw);
  m->own_dev.swap(ld.dev);
  *out = m;
  return MING_OK;
}

}  // namespace
