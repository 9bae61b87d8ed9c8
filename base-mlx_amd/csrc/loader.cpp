// MLX-format checkpoint loading for the Qwen3 model: config.json and
// safetensors shards (host code).
//
// Restates the reference's loading path:
//   ModelConfig::from_path (crates/base-mlx-core/src/model/config.rs:149-167):
//     HuggingFace config.json; `quantization` and `quantization_config`
//     (mlx-lm writes both) merged; num_key_value_heads defaults to
//     num_attention_heads, head_dim to hidden_size / num_attention_heads
//     (config.rs:184-191), rms_norm_eps to 1e-6, rope_theta to 10000,
//     tie_word_embeddings to false (config.rs:109-135);
//   Qwen3::load (crates/base-mlx-core/src/model/qwen3.rs:194-295) with
//     read_all_shards (qwen3.rs:607-627): every *.safetensors file of the
//     directory in sorted order, later shards overriding earlier names;
//     each tensor taken by name (qwen3.rs:580-605), a missing one an error,
//     and tensors left over once the model is built an error naming the
//     first five;
//   the bits a projection's shapes imply, W_last * 32 / (S_last * gs)
//     (infer_bits, crates/base-mlx-core/src/model/gemma.rs:760-779).
// The safetensors format: an 8-byte little-endian header length, a JSON
// header {name: {dtype, shape, data_offsets [begin, end)}, "__metadata__":
// {...}}, then the data block the offsets index.  Packed weights must be
// U32 (I32 accepted: the same bits); scales, biases and norm weights BF16,
// or F16 / F32 rounded to bf16 (round to nearest even) on the way in.
// All headers are read and every tensor is checked against the config
// before anything is allocated on the GPU.
#include <dirent.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "bmx_internal.h"

namespace bmx {
namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const char* key) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* s, size_t n) : p_(s), end_(s + n) {}
  bool parse(Json* out, std::string* err) {
    if (!value(out, 0)) {
      *err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      *err = "trailing characters after the JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if (static_cast<size_t>(end_ - p_) < n || strncmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(uint32_t c, std::string* o) {
    if (c < 0x80) {
      o->push_back(static_cast<char>(c));
    } else if (c < 0x800) {
      o->push_back(static_cast<char>(0xC0 | (c >> 6)));
      o->push_back(static_cast<char>(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
      o->push_back(static_cast<char>(0xE0 | (c >> 12)));
      o->push_back(static_cast<char>(0x80 | ((c >> 6) & 0x3F)));
      o->push_back(static_cast<char>(0x80 | (c & 0x3F)));
    } else {
      o->push_back(static_cast<char>(0xF0 | (c >> 18)));
      o->push_back(static_cast<char>(0x80 | ((c >> 12) & 0x3F)));
      o->push_back(static_cast<char>(0x80 | ((c >> 6) & 0x3F)));
      o->push_back(static_cast<char>(0x80 | (c & 0x3F)));
    }
  }
  bool hex4(uint32_t* c) {
    if (end_ - p_ < 4) return false;
    *c = 0;
    for (int i = 0; i < 4; i++) {
      const char h = *p_++;
      *c <<= 4;
      if (h >= '0' && h <= '9') *c |= static_cast<uint32_t>(h - '0');
      else if (h >= 'a' && h <= 'f') *c |= static_cast<uint32_t>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') *c |= static_cast<uint32_t>(h - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string* o) {
    if (p_ >= end_ || *p_ != '"') return false;
    p_++;
    while (p_ < end_ && *p_ != '"') {
      const char c = *p_++;
      if (c != '\\') {
        o->push_back(c);
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': o->push_back('"'); break;
        case '\\': o->push_back('\\'); break;
        case '/': o->push_back('/'); break;
        case 'b': o->push_back('\b'); break;
        case 'f': o->push_back('\f'); break;
        case 'n': o->push_back('\n'); break;
        case 'r': o->push_back('\r'); break;
        case 't': o->push_back('\t'); break;
        case 'u': {
          uint32_t c1;
          if (!hex4(&c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2;
            uint32_t c2;
            if (!hex4(&c2)) return false;
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          }
          utf8(c1, o);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= end_) return false;
    p_++;
    return true;
  }
  bool value(Json* v, int depth) {
    if (depth > 64) {
      err_ = "JSON nested too deeply";
      return false;
    }
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      p_++;
      v->kind = Json::OBJ;
      ws();
      if (p_ < end_ && *p_ == '}') {
        p_++;
        return true;
      }
      for (;;) {
        ws();
        std::string key;
        if (!string(&key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return false;
        p_++;
        Json child;
        if (!value(&child, depth + 1)) return false;
        v->obj.emplace_back(std::move(key), std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          p_++;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      p_++;
      v->kind = Json::ARR;
      ws();
      if (p_ < end_ && *p_ == ']') {
        p_++;
        return true;
      }
      for (;;) {
        Json child;
        if (!value(&child, depth + 1)) return false;
        v->arr.push_back(std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          p_++;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v->kind = Json::STR;
      return string(&v->str);
    }
    if (lit("true")) {
      v->kind = Json::BOOL;
      v->b = true;
      return true;
    }
    if (lit("false")) {
      v->kind = Json::BOOL;
      return true;
    }
    if (lit("null")) return true;
    // number
    const char* q = p_;
    if (q < end_ && (*q == '-' || *q == '+')) q++;
    while (q < end_ && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' || *q == '+'))
      q++;
    if (q == p_) return false;
    const std::string t(p_, q);
    char* e = nullptr;
    v->num = strtod(t.c_str(), &e);
    if (!e || *e) return false;
    v->kind = Json::NUM;
    p_ = q;
    return true;
  }
};

bool read_file(const std::string& path, std::string* out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
  const bool ok = !ferror(f);
  fclose(f);
  return ok;
}

// An integer field of the config; `def` when absent (or null).
int cfg_int(const Json& j, const char* key, long def, bool required, long* out, std::string* err) {
  const Json* v = j.get(key);
  if (!v || v->kind == Json::NUL) {
    if (required) {
      *err = std::string("config.json: missing ") + key;
      return BMX_E_ARG;
    }
    *out = def;
    return BMX_OK;
  }
  if (v->kind != Json::NUM || v->num != floor(v->num) || v->num < 0 || v->num > 2147483647.0) {
    *err = std::string("config.json: ") + key + " is not a non-negative integer";
    return BMX_E_ARG;
  }
  *out = static_cast<long>(v->num);
  return BMX_OK;
}

int config_from_text(const std::string& text, bmx_qwen3_config* cfg) {
  Json j;
  std::string err;
  if (!JsonParser(text.data(), text.size()).parse(&j, &err)) return set_error(BMX_E_ARG, "config.json: %s", err.c_str());
  if (j.kind != Json::OBJ) return set_error(BMX_E_ARG, "config.json: not a JSON object");
  if (const Json* t = j.get("model_type"))
    if (t->kind == Json::STR && t->str != "qwen3")
      return set_error(BMX_E_UNSUPPORTED, "config.json: model_type \"%s\" (this library builds qwen3)", t->str.c_str());
  long hidden, inter, layers, heads, kv, hd, vocab;
  if (cfg_int(j, "hidden_size", 0, true, &hidden, &err) || cfg_int(j, "intermediate_size", 0, true, &inter, &err) ||
      cfg_int(j, "num_hidden_layers", 0, true, &layers, &err) ||
      cfg_int(j, "num_attention_heads", 0, true, &heads, &err) || cfg_int(j, "vocab_size", 0, true, &vocab, &err))
    return set_error(BMX_E_ARG, "%s", err.c_str());
  if (hidden == 0 || heads == 0)
    return set_error(BMX_E_ARG, "config.json: hidden_size and num_attention_heads must be non-zero");
  if (cfg_int(j, "num_key_value_heads", heads, false, &kv, &err) || cfg_int(j, "head_dim", -1, false, &hd, &err))
    return set_error(BMX_E_ARG, "%s", err.c_str());
  if (hd < 0) {
    if (hidden % heads)
      return set_error(BMX_E_ARG, "config.json: hidden_size (%ld) not divisible by num_attention_heads (%ld) and no "
                                  "explicit head_dim", hidden, heads);
    hd = hidden / heads;
  }
  double eps = 1e-6, theta = 10000.0;
  if (const Json* v = j.get("rms_norm_eps"); v && v->kind == Json::NUM) eps = v->num;
  if (const Json* v = j.get("rope_theta"); v && v->kind == Json::NUM) theta = v->num;
  bool tied = false;
  if (const Json* v = j.get("tie_word_embeddings"); v && v->kind == Json::BOOL) tied = v->b;
  // quantization: mlx-lm writes both keys; `quantization` wins
  const Json* q = j.get("quantization");
  if (!q || q->kind != Json::OBJ) q = j.get("quantization_config");
  if (!q || q->kind != Json::OBJ) return set_error(BMX_E_UNSUPPORTED, "config.json: only quantized models are supported");
  long bits, gs;
  if (cfg_int(*q, "bits", 0, true, &bits, &err) || cfg_int(*q, "group_size", 0, true, &gs, &err))
    return set_error(BMX_E_ARG, "%s (quantization)", err.c_str());
  cfg->hidden = static_cast<int>(hidden);
  cfg->inter = static_cast<int>(inter);
  cfg->layers = static_cast<int>(layers);
  cfg->n_heads = static_cast<int>(heads);
  cfg->n_kv_heads = static_cast<int>(kv);
  cfg->head_dim = static_cast<int>(hd);
  cfg->vocab = static_cast<int>(vocab);
  cfg->tied = tied ? 1 : 0;
  cfg->group_size = static_cast<int>(gs);
  cfg->bits = static_cast<int>(bits);
  cfg->eps = static_cast<float>(eps);
  cfg->rope_theta = static_cast<float>(theta);
  return BMX_OK;
}

// ---- safetensors ----
struct TensorRef {
  int file = 0;
  std::string dtype;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // absolute byte offsets in the file
};

int read_header(const std::string& path, int file, std::map<std::string, TensorRef>* out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return set_error(BMX_E_ARG, "safetensors: cannot open %s", path.c_str());
  std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
  unsigned char len8[8];
  if (fread(len8, 1, 8, f) != 8) return set_error(BMX_E_ARG, "safetensors: %s: truncated header", path.c_str());
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | len8[i];
  if (fseeko(f, 0, SEEK_END) != 0) return set_error(BMX_E_ARG, "safetensors: %s: cannot seek", path.c_str());
  const uint64_t fsize = static_cast<uint64_t>(ftello(f));
  if (hlen == 0 || hlen > (100ull << 20) || 8 + hlen > fsize)
    return set_error(BMX_E_ARG, "safetensors: %s: header length %llu invalid", path.c_str(),
                     static_cast<unsigned long long>(hlen));
  std::string h(hlen, '\0');
  if (fseeko(f, 8, SEEK_SET) != 0 || fread(&h[0], 1, hlen, f) != hlen)
    return set_error(BMX_E_ARG, "safetensors: %s: truncated header", path.c_str());
  Json j;
  std::string err;
  if (!JsonParser(h.data(), h.size()).parse(&j, &err) || j.kind != Json::OBJ)
    return set_error(BMX_E_ARG, "safetensors: %s: header: %s", path.c_str(), err.empty() ? "not an object" : err.c_str());
  const uint64_t data0 = 8 + hlen;
  for (const auto& kv : j.obj) {
    if (kv.first == "__metadata__") continue;
    const Json& t = kv.second;
    const Json* dt = t.get("dtype");
    const Json* sh = t.get("shape");
    const Json* off = t.get("data_offsets");
    if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off || off->kind != Json::ARR ||
        off->arr.size() != 2)
      return set_error(BMX_E_ARG, "safetensors: %s: bad entry for %s", path.c_str(), kv.first.c_str());
    TensorRef r;
    r.file = file;
    r.dtype = dt->str;
    for (const Json& d : sh->arr) {
      if (d.kind != Json::NUM || d.num < 0) return set_error(BMX_E_ARG, "safetensors: %s: bad shape", kv.first.c_str());
      r.shape.push_back(static_cast<int64_t>(d.num));
    }
    if (off->arr[0].kind != Json::NUM || off->arr[1].kind != Json::NUM || off->arr[1].num < off->arr[0].num)
      return set_error(BMX_E_ARG, "safetensors: %s: bad data_offsets", kv.first.c_str());
    r.begin = data0 + static_cast<uint64_t>(off->arr[0].num);
    r.end = data0 + static_cast<uint64_t>(off->arr[1].num);
    if (r.end > fsize)
      return set_error(BMX_E_ARG, "safetensors: %s: %s runs past the end of the file", path.c_str(), kv.first.c_str());
    (*out)[kv.first] = std::move(r);  // a later shard overrides an earlier one
  }
  return BMX_OK;
}

int elem_bytes(const std::string& dt) {
  if (dt == "U32" || dt == "I32" || dt == "F32") return 4;
  if (dt == "BF16" || dt == "F16") return 2;
  return 0;
}

uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1f;
  const uint32_t m = h & 0x3ffu;
  float v;
  if (e == 0) v = ldexpf(static_cast<float>(m), -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf(static_cast<float>(m | 0x400u), e - 25);
  uint32_t u;
  memcpy(&u, &v, 4);
  u |= sign;
  memcpy(&v, &u, 4);
  return v;
}

}  // namespace
}  // namespace bmx

using namespace bmx;

extern "C" int bmx_qwen3_config_from_json(const char* path, bmx_qwen3_config* out) {
  if (!path || !out) return set_error(BMX_E_ARG, "qwen3_config_from_json: null pointer");
  std::string text;
  if (!read_file(path, &text)) return set_error(BMX_E_ARG, "cannot read %s", path);
  bmx_qwen3_config cfg{};
  if (int rc = config_from_text(text, &cfg)) return rc;
  *out = cfg;
  return BMX_OK;
}

extern "C" int bmx_qwen3_load(const char* dir, int max_tokens, bmx_qwen3** out) {
  if (!dir || !out) return set_error(BMX_E_ARG, "qwen3_load: null pointer");
  *out = nullptr;
  const std::string d(dir);
  bmx_qwen3_config cfg{};
  if (int rc = bmx_qwen3_config_from_json((d + "/config.json").c_str(), &cfg)) return rc;
  // every shard's header, sorted by file name
  std::vector<std::string> files;
  if (DIR* dp = opendir(dir)) {
    while (dirent* e = readdir(dp)) {
      const std::string n(e->d_name);
      if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(d + "/" + n);
    }
    closedir(dp);
  } else {
    return set_error(BMX_E_ARG, "qwen3_load: cannot open directory %s", dir);
  }
  std::sort(files.begin(), files.end());
  if (files.empty()) return set_error(BMX_E_ARG, "no .safetensors in %s", dir);
  std::map<std::string, TensorRef> tensors;
  for (size_t i = 0; i < files.size(); i++)
    if (int rc = read_header(files[i], static_cast<int>(i), &tensors)) return rc;
  // the bits the embedding's shapes imply must agree with the config
  // (infer_bits: W_last * 32 / (S_last * gs))
  {
    auto w = tensors.find("model.embed_tokens.weight");
    auto s = tensors.find("model.embed_tokens.scales");
    if (w != tensors.end() && s != tensors.end() && !w->second.shape.empty() && !s->second.shape.empty() &&
        cfg.group_size > 0 && s->second.shape.back() > 0) {
      const int64_t num = w->second.shape.back() * 32, den = s->second.shape.back() * cfg.group_size;
      if (num % den == 0 && num / den != cfg.bits)
        return set_error(BMX_E_UNSUPPORTED, "qwen3_load: tensors hold %lld-bit weights, config says %d",
                         static_cast<long long>(num / den), cfg.bits);
    }
  }
  if (cfg.bits != 4 || cfg.group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "qwen3_load: only bits=4, group_size=64 (got %d, %d)", cfg.bits,
                     cfg.group_size);
  // check every expected tensor before touching the GPU: allocate a model
  // description only (the slot list needs the shapes, not the memory)
  struct Want {
    std::string name;
    int rows, cols;
    bool u32;
  };
  std::vector<Want> want;
  {
    const int H = cfg.hidden, I = cfg.inter, qd = cfg.n_heads * cfg.head_dim, kvd = cfg.n_kv_heads * cfg.head_dim;
    auto qlin = [&](const std::string& p, int N, int K) {
      want.push_back({p + ".weight", N, K / 8, true});
      want.push_back({p + ".scales", N, K / 64, false});
      want.push_back({p + ".biases", N, K / 64, false});
    };
    qlin("model.embed_tokens", cfg.vocab, H);
    static const char* const kProj[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                                         "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"};
    const int dims[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {I, H}, {I, H}, {H, I}};
    for (int l = 0; l < cfg.layers; l++) {
      const std::string p = "model.layers." + std::to_string(l) + ".";
      want.push_back({p + "input_layernorm.weight", 1, H, false});
      for (int s = 0; s < 7; s++) qlin(p + kProj[s], dims[s][0], dims[s][1]);
      want.push_back({p + "self_attn.q_norm.weight", 1, cfg.head_dim, false});
      want.push_back({p + "self_attn.k_norm.weight", 1, cfg.head_dim, false});
      want.push_back({p + "post_attention_layernorm.weight", 1, H, false});
    }
    want.push_back({"model.norm.weight", 1, H, false});
    if (!cfg.tied) qlin("lm_head", cfg.vocab, H);
  }
  for (const Want& w : want) {
    auto it = tensors.find(w.name);
    if (it == tensors.end()) return set_error(BMX_E_SHAPE, "missing tensor: %s", w.name.c_str());
    const TensorRef& t = it->second;
    const bool ok_dtype = w.u32 ? (t.dtype == "U32" || t.dtype == "I32")
                                : (t.dtype == "BF16" || t.dtype == "F16" || t.dtype == "F32");
    if (!ok_dtype) return set_error(BMX_E_UNSUPPORTED, "%s: dtype %s", w.name.c_str(), t.dtype.c_str());
    int64_t rows = 1, cols = t.shape.empty() ? 1 : t.shape.back();
    for (size_t i = 0; i + 1 < t.shape.size(); i++) rows *= t.shape[i];
    if (t.shape.empty() || rows != w.rows || cols != w.cols)
      return set_error(BMX_E_SHAPE, "%s: shape does not match the config (want [%d, %d])", w.name.c_str(), w.rows,
                       w.cols);
    if (t.end - t.begin != static_cast<uint64_t>(rows * cols * elem_bytes(t.dtype)))
      return set_error(BMX_E_SHAPE, "%s: %llu data bytes for its shape", w.name.c_str(),
                       static_cast<unsigned long long>(t.end - t.begin));
  }
  if (tensors.size() > want.size()) {
    std::vector<std::string> left;
    for (const auto& kv : tensors) {
      bool used = false;
      for (const Want& w : want)
        if (w.name == kv.first) {
          used = true;
          break;
        }
      if (!used) left.push_back(kv.first);
    }
    std::string first;
    for (size_t i = 0; i < left.size() && i < 5; i++) first += (i ? ", " : "") + left[i];
    return set_error(BMX_E_SHAPE, "%zu unmapped tensors remain (first 5: %s)", left.size(), first.c_str());
  }
  // allocate and copy
  bmx_qwen3* m = nullptr;
  if (int rc = qwen3_alloc(&cfg, max_tokens, &m)) return rc;
  std::vector<FILE*> fh(files.size(), nullptr);
  auto close_all = [&]() {
    for (FILE* f : fh)
      if (f) fclose(f);
  };
  std::vector<unsigned char> buf;
  std::vector<uint16_t> conv;
  int rc = BMX_OK;
  for (const WeightSlot& s : qwen3_weight_slots(m)) {
    const TensorRef& t = tensors.at(s.name);
    FILE*& f = fh[t.file];
    if (!f && !(f = fopen(files[t.file].c_str(), "rb"))) {
      rc = set_error(BMX_E_ARG, "cannot open %s", files[t.file].c_str());
      break;
    }
    const size_t n = t.end - t.begin;
    buf.resize(n);
    if (fseeko(f, static_cast<off_t>(t.begin), SEEK_SET) != 0 || fread(buf.data(), 1, n, f) != n) {
      rc = set_error(BMX_E_ARG, "%s: read failed", s.name.c_str());
      break;
    }
    const void* src = buf.data();
    size_t bytes = n;
    const size_t count = static_cast<size_t>(s.rows) * s.cols;
    if (!s.u32 && t.dtype != "BF16") {
      conv.resize(count);
      for (size_t i = 0; i < count; i++) {
        float v;
        if (t.dtype == "F32") {
          memcpy(&v, buf.data() + 4 * i, 4);
        } else {
          uint16_t h;
          memcpy(&h, buf.data() + 2 * i, 2);
          v = f16_to_f32(h);
        }
        conv[i] = f32_to_bf16(v);
      }
      src = conv.data();
      bytes = count * 2;
    }
    if ((rc = check_hip(hipMemcpy(s.dev, src, bytes, hipMemcpyHostToDevice), "hipMemcpy"))) break;
  }
  close_all();
  // copies from pageable memory may return before the data has landed:
  // the model is complete only once they have
  if (!rc) rc = check_hip(hipDeviceSynchronize(), "qwen3_load: sync");
  if (rc) {
    bmx_qwen3_destroy(m);
    return rc;
  }
  *out = m;
  return BMX_OK;
}
