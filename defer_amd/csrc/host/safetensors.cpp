// safetensors.cpp -- the model file loader (safetensors.rs:142-237 and
// model.rs:41-118, 285-347 of the reference): one front-to-back pass over
// the file (8-byte header length, JSON header, tensors in ascending offset
// order), every byte fed to SHA-256 for the model signature, F32 / F16 /
// BF16 / F64 converted exactly to f32; the config from the "defer.config"
// metadata entry or config.json beside the file; the tensors handed to
// libdefer_gpu in the canonical order.
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "defer_host.h"

using dh::fail;

namespace {

// ------------------------------------------------------------------ JSON
// Enough JSON for safetensors headers and HF configs: objects (key order
// kept), arrays, strings with escapes, numbers, true/false/null.

struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  bool is_int = false;
  unsigned long long u = 0;  // exact value of a non-negative integer
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(e - p) < n || memcmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  static void utf8(std::string& o, unsigned cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 0x3F));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(unsigned* v) {
    if (e - p < 4) return false;
    *v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      *v <<= 4;
      if (c >= '0' && c <= '9') *v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') *v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') *v |= (unsigned)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& o) {
    if (p >= e || *p != '"') return false;
    ++p;
    while (p < e && *p != '"') {
      if (*p != '\\') {
        o += *p++;
        continue;
      }
      if (++p >= e) return false;
      const char c = *p++;
      switch (c) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          unsigned cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            unsigned lo;
            if (!hex4(&lo)) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
    if (p >= e) return false;
    ++p;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p >= e) return false;
    if (*p == '{') {
      ++p;
      v.kind = JVal::OBJ;
      ws();
      if (p < e && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= e || *p != ':') return false;
        ++p;
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(x));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == '}') {
          ++p;
          return true;
        }
        return false;
      }
    }
    if (*p == '[') {
      ++p;
      v.kind = JVal::ARR;
      ws();
      if (p < e && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.arr.push_back(std::move(x));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == ']') {
          ++p;
          return true;
        }
        return false;
      }
    }
    if (*p == '"') {
      v.kind = JVal::STR;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = JVal::BOOL;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = JVal::BOOL;
      return true;
    }
    if (lit("null")) return true;
    const char* s = p;
    if (p < e && *p == '-') ++p;
    bool digits = false, frac = false;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                     *p == '+' || *p == '-')) {
      if (*p >= '0' && *p <= '9') digits = true;
      else frac = true;
      ++p;
    }
    if (!digits) return false;
    const std::string t(s, p);
    v.kind = JVal::NUM;
    v.num = strtod(t.c_str(), nullptr);
    if (!frac && t[0] != '-') {
      v.is_int = true;
      v.u = strtoull(t.c_str(), nullptr, 10);
    }
    return true;
  }
};

bool parse_json(const std::string& s, JVal& out) {
  JParser jp{s.data(), s.data() + s.size(), ""};
  if (!jp.value(out, 0)) return false;
  jp.ws();
  return jp.p == jp.e;
}

// --------------------------------------------------------- conversions

// IEEE 754 binary16 -> binary32, exact (the conversion safetensors.rs:47-72
// performs). From the definition: a finite half is (-1)^s * M * 2^(E - 25)
// with the integer significand M = 1024 + m for a biased exponent E >= 1
// and M = m (E taken as 1) for E = 0; both M and the power of two are exact
// in binary32, so their product is the value. Exponent 31 is infinity
// (m = 0) or NaN, whose payload moves to the top of binary32's fraction.
float f16_to_f32(uint16_t h) {
  const bool neg = (h & 0x8000u) != 0;
  const uint32_t E = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (E == 0x1Fu) {
    const uint32_t bits = (neg ? 0x80000000u : 0u) | 0x7F800000u | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
  }
  const float M = (float)(E ? 1024u + m : m);
  const float v = ldexpf(M, (int)(E ? E : 1u) - 25);
  return neg ? -v : v;
}
float bf16_to_f32(uint16_t h) {
  const uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

enum DType { DT_F32, DT_F16, DT_BF16, DT_F64 };
size_t dsize(DType t) { return t == DT_F32 ? 4 : (t == DT_F64 ? 8 : 2); }

void convert(DType t, const uint8_t* raw, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) {
    const uint8_t* c = raw + i * dsize(t);
    switch (t) {
      case DT_F32: memcpy(out + i, c, 4); break;
      case DT_F16: out[i] = f16_to_f32((uint16_t)(c[0] | c[1] << 8)); break;
      case DT_BF16: out[i] = bf16_to_f32((uint16_t)(c[0] | c[1] << 8)); break;
      case DT_F64: {
        double d;
        memcpy(&d, c, 8);
        out[i] = (float)d;
        break;
      }
    }
  }
}

}  // namespace

// ------------------------------------------------------------ the reader

struct defer_host_st {
  std::vector<std::string> names;  // on-disk order
  std::vector<std::vector<uint64_t>> shapes;
  std::vector<std::vector<float>> data;
  std::vector<std::pair<std::string, std::string>> meta;
  uint8_t signature[32];
};

namespace {

struct Entry {
  std::string name;
  DType dt;
  std::vector<uint64_t> shape;
  uint64_t start, end;
};

// Reads exactly n bytes (hashing them); false on a short read.
bool read_hashed(FILE* f, dh::Sha256& sha, uint8_t* dst, size_t n) {
  if (n && fread(dst, 1, n, f) != n) return false;
  sha.update(dst, n);
  return true;
}

}  // namespace

extern "C" int defer_host_st_open(const char* path, defer_host_st** out) {
  if (!path || !out) return fail(DEFER_HOST_E_INVALID, "null argument");
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return fail(DEFER_HOST_E_IO, "cannot open %s: %s", path, strerror(errno));
  std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
  if (fseeko(f, 0, SEEK_END) != 0) return fail(DEFER_HOST_E_IO, "%s: seek", path);
  const uint64_t file_len = (uint64_t)ftello(f);
  rewind(f);
  dh::Sha256 sha;
  uint8_t lb[8];
  if (!read_hashed(f, sha, lb, 8)) return fail(DEFER_HOST_E_MODEL, "invalid safetensors header length");
  uint64_t hl = 0;
  for (int i = 0; i < 8; ++i) hl |= (uint64_t)lb[i] << (8 * i);
  if (hl > 100ull * 1024 * 1024 || 8 + hl > file_len)
    return fail(DEFER_HOST_E_MODEL, "invalid safetensors header length");
  std::string hdr(hl, '\0');
  if (!read_hashed(f, sha, reinterpret_cast<uint8_t*>(&hdr[0]), hl))
    return fail(DEFER_HOST_E_IO, "%s: short read", path);
  JVal root;
  if (!parse_json(hdr, root)) return fail(DEFER_HOST_E_MODEL, "safetensors header is not valid JSON");
  if (root.kind != JVal::OBJ) return fail(DEFER_HOST_E_MODEL, "safetensors header is not an object");
  std::unique_ptr<defer_host_st> st(new defer_host_st());
  std::vector<Entry> entries;
  for (const auto& kv : root.obj) {
    const std::string& name = kv.first;
    const JVal& v = kv.second;
    if (name == "__metadata__") {
      if (v.kind == JVal::OBJ)
        for (const auto& m : v.obj)
          if (m.second.kind == JVal::STR) st->meta.emplace_back(m.first, m.second.str);
      continue;
    }
    const JVal* dt = v.get("dtype");
    const JVal* sh = v.get("shape");
    const JVal* of = v.get("data_offsets");
    if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !of ||
        of->kind != JVal::ARR || of->arr.size() != 2)
      return fail(DEFER_HOST_E_MODEL, "malformed header entry for %s", name.c_str());
    Entry e;
    e.name = name;
    if (dt->str == "F32") e.dt = DT_F32;
    else if (dt->str == "F16") e.dt = DT_F16;
    else if (dt->str == "BF16") e.dt = DT_BF16;
    else if (dt->str == "F64") e.dt = DT_F64;
    else return fail(DEFER_HOST_E_MODEL, "unsupported safetensors dtype %s", dt->str.c_str());
    uint64_t numel = 1;
    for (const JVal& d : sh->arr) {
      if (d.kind != JVal::NUM || !d.is_int)
        return fail(DEFER_HOST_E_MODEL, "malformed header entry for %s", name.c_str());
      e.shape.push_back(d.u);
      numel *= d.u;
    }
    for (const JVal& o : of->arr)
      if (o.kind != JVal::NUM || !o.is_int)
        return fail(DEFER_HOST_E_MODEL, "malformed header entry for %s", name.c_str());
    e.start = of->arr[0].u;
    e.end = of->arr[1].u;
    if (e.end < e.start || e.end - e.start != numel * dsize(e.dt))
      return fail(DEFER_HOST_E_MODEL, "size mismatch for tensor %s", name.c_str());
    entries.push_back(std::move(e));
  }
  // sequential on-disk order, ties by name
  std::sort(entries.begin(), entries.end(), [](const Entry& a, const Entry& b) {
    return a.start != b.start ? a.start < b.start : a.name < b.name;
  });
  const uint64_t data_len = file_len - 8 - hl;
  uint64_t pos = 0;
  std::vector<uint8_t> raw, skipbuf(1 << 16);
  auto skip = [&](uint64_t n) {
    while (n) {
      const size_t k = (size_t)std::min<uint64_t>(n, skipbuf.size());
      if (!read_hashed(f, sha, skipbuf.data(), k)) return false;
      n -= k;
    }
    return true;
  };
  for (const Entry& e : entries) {
    if (e.start < pos || e.end > data_len)
      return fail(DEFER_HOST_E_MODEL, "overlapping/out of range tensor %s", e.name.c_str());
    if (e.start > pos && !skip(e.start - pos)) return fail(DEFER_HOST_E_IO, "%s: short read", path);
    raw.resize(e.end - e.start);
    if (!read_hashed(f, sha, raw.data(), raw.size())) return fail(DEFER_HOST_E_IO, "%s: short read", path);
    pos = e.end;
    const size_t n = raw.size() / dsize(e.dt);
    std::vector<float> data(n);
    convert(e.dt, raw.data(), n, data.data());
    st->names.push_back(e.name);
    st->shapes.push_back(e.shape);
    st->data.push_back(std::move(data));
  }
  if (pos < data_len && !skip(data_len - pos)) return fail(DEFER_HOST_E_IO, "%s: short read", path);
  sha.finish(st->signature);
  *out = st.release();
  return DEFER_HOST_OK;
}

extern "C" void defer_host_st_close(defer_host_st* st) { delete st; }
extern "C" size_t defer_host_st_count(const defer_host_st* st) { return st ? st->names.size() : 0; }
extern "C" const char* defer_host_st_name(const defer_host_st* st, size_t i) {
  return st && i < st->names.size() ? st->names[i].c_str() : nullptr;
}
extern "C" size_t defer_host_st_shape(const defer_host_st* st, size_t i, uint64_t* dims,
                                      size_t max_dims) {
  if (!st || i >= st->shapes.size()) return 0;
  const auto& s = st->shapes[i];
  for (size_t k = 0; k < s.size() && k < max_dims; ++k) dims[k] = s[k];
  return s.size();
}
extern "C" const float* defer_host_st_data(const defer_host_st* st, size_t i, size_t* n) {
  if (!st || i >= st->data.size()) return nullptr;
  if (n) *n = st->data[i].size();
  return st->data[i].data();
}
extern "C" const char* defer_host_st_meta(const defer_host_st* st, const char* key) {
  if (!st || !key) return nullptr;
  for (const auto& kv : st->meta)
    if (kv.first == key) return kv.second.c_str();
  return nullptr;
}
extern "C" void defer_host_st_signature(const defer_host_st* st, uint8_t out[32]) {
  if (st) memcpy(out, st->signature, 32);
}

// --------------------------------------------------------- model config

namespace {

int find(const defer_host_st* st, const std::string& name) {
  for (size_t i = 0; i < st->names.size(); ++i)
    if (st->names[i] == name) return (int)i;
  return -1;
}

// Config::from_json (model.rs:41-118): sizes from the JSON, else inferred
// from the weights; the reference's defaults otherwise.
int config_from(const JVal& v, const defer_host_st* st, defer_gpu_config* c) {
  auto num = [&](const char* k, uint64_t* out) {
    const JVal* x = v.get(k);
    if (!x || x->kind != JVal::NUM || !x->is_int) return false;
    *out = x->u;
    return true;
  };
  auto flt = [&](const char* k, double* out) {
    const JVal* x = v.get(k);
    if (!x || x->kind != JVal::NUM) return false;
    *out = x->num;
    return true;
  };
  int ei = find(st, "model.embed_tokens.weight");
  if (ei < 0) ei = find(st, "embed_tokens.weight");
  uint64_t vocab = 0, hidden = 0, layers = 0, inter = 0, heads = 0, kvh = 0, hd = 0, mpe = 0;
  const bool embed2 = ei >= 0 && st->shapes[ei].size() == 2;
  if (!num("hidden_size", &hidden)) {
    if (!embed2) return fail(DEFER_HOST_E_MODEL, "config is missing `hidden_size`");
    hidden = st->shapes[ei][1];
  }
  if (!num("vocab_size", &vocab)) {
    if (!embed2) return fail(DEFER_HOST_E_MODEL, "config is missing `vocab_size`");
    vocab = st->shapes[ei][0];
  }
  if (!num("num_hidden_layers", &layers)) {
    while (find(st, "model.layers." + std::to_string(layers) + ".input_layernorm.weight") >= 0)
      ++layers;
    if (!layers) return fail(DEFER_HOST_E_MODEL, "config is missing `num_hidden_layers`");
  }
  if (!num("intermediate_size", &inter)) {
    const int gi = find(st, "model.layers.0.mlp.gate_proj.weight");
    if (gi < 0) return fail(DEFER_HOST_E_MODEL, "config is missing `intermediate_size`");
    inter = st->shapes[gi][0];
  }
  if (!num("num_attention_heads", &heads))
    return fail(DEFER_HOST_E_MODEL, "config is missing `num_attention_heads`");
  if (!num("num_key_value_heads", &kvh)) kvh = heads;
  if (!num("head_dim", &hd)) hd = heads ? hidden / heads : 0;
  const JVal* act = v.get("hidden_act");
  const std::string a = act && act->kind == JVal::STR ? act->str : "silu";
  uint32_t activation;
  if (a == "silu" || a == "swish") activation = 0;
  else if (a.compare(0, 4, "gelu") == 0) activation = 1;
  else return fail(DEFER_HOST_E_MODEL, "unsupported activation %s", a.c_str());
  double eps = 1e-6, theta = 10000.0;
  flt("rms_norm_eps", &eps);
  flt("rope_theta", &theta);
  if (!num("max_position_embeddings", &mpe)) mpe = 4096;
  const bool has_head = find(st, "lm_head.weight") >= 0;
  bool tie = !has_head;
  const JVal* t = v.get("tie_word_embeddings");
  if (t && t->kind == JVal::BOOL) tie = t->b;
  tie = tie || !has_head;
  if (kvh == 0 || heads % kvh != 0)
    return fail(DEFER_HOST_E_MODEL, "num_attention_heads must be a multiple of num_key_value_heads");
  if (hd % 2 != 0) return fail(DEFER_HOST_E_MODEL, "head_dim must be even for RoPE");
  memset(c, 0, sizeof(*c));
  c->vocab_size = (uint32_t)vocab;
  c->hidden_size = (uint32_t)hidden;
  c->intermediate_size = (uint32_t)inter;
  c->num_layers = (uint32_t)layers;
  c->num_heads = (uint32_t)heads;
  c->num_kv_heads = (uint32_t)kvh;
  c->head_dim = (uint32_t)hd;
  c->rms_norm_eps = (float)eps;
  c->rope_theta = (float)theta;
  c->max_seq_len = (uint32_t)mpe;
  c->tie_word_embeddings = tie ? 1 : 0;
  c->activation = activation;
  c->has_bias = find(st, "model.layers.0.self_attn.q_proj.bias") >= 0 ? 1 : 0;
  return DEFER_HOST_OK;
}

}  // namespace

extern "C" int defer_host_model_load(const char* path, uint32_t max_seq_len, defer_gpu_model** out,
                                     defer_gpu_config* cfg_out, uint8_t signature[32]) {
  if (!path || !out) return fail(DEFER_HOST_E_INVALID, "null argument");
  *out = nullptr;
  defer_host_st* st = nullptr;
  int rc = defer_host_st_open(path, &st);
  if (rc) return rc;
  std::unique_ptr<defer_host_st, void (*)(defer_host_st*)> guard(st, defer_host_st_close);
  // The config: the "defer.config" metadata entry, else config.json beside the file.
  JVal cv;
  cv.kind = JVal::OBJ;
  if (const char* s = defer_host_st_meta(st, "defer.config")) {
    if (!parse_json(s, cv)) return fail(DEFER_HOST_E_MODEL, "defer.config metadata is not valid JSON");
  } else {
    std::string p(path);
    const size_t slash = p.find_last_of('/');
    p = (slash == std::string::npos ? std::string() : p.substr(0, slash + 1)) + "config.json";
    FILE* f = fopen(p.c_str(), "rb");
    if (f) {
      std::string s;
      char b[4096];
      size_t k;
      while ((k = fread(b, 1, sizeof(b), f)) > 0) s.append(b, k);
      fclose(f);
      if (!parse_json(s, cv)) return fail(DEFER_HOST_E_MODEL, "config.json is not valid JSON");
    }
  }
  defer_gpu_config c;
  rc = config_from(cv, st, &c);
  if (rc) return rc;
  if (max_seq_len) c.max_seq_len = max_seq_len;
  // Tensors in the canonical order (model.rs:301-347), shapes checked.
  const uint64_t h = c.hidden_size, q = (uint64_t)c.num_heads * c.head_dim,
                 kv = (uint64_t)c.num_kv_heads * c.head_dim, ff = c.intermediate_size,
                 V = c.vocab_size;
  std::vector<const float*> ptrs;
  auto take = [&](const std::string& name, uint64_t n) -> int {
    const int i = find(st, name);
    if (i < 0) return fail(DEFER_HOST_E_MODEL, "missing tensor %s", name.c_str());
    if (st->data[i].size() != n)
      return fail(DEFER_HOST_E_MODEL, "tensor %s has %zu elements, expected %llu", name.c_str(),
                  st->data[i].size(), (unsigned long long)n);
    ptrs.push_back(st->data[i].data());
    return DEFER_HOST_OK;
  };
  const std::string embed =
      find(st, "model.embed_tokens.weight") >= 0 ? "model.embed_tokens.weight" : "embed_tokens.weight";
  if ((rc = take(embed, V * h))) return rc;
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l);
    if ((rc = take(p + ".input_layernorm.weight", h))) return rc;
    if ((rc = take(p + ".self_attn.q_proj.weight", q * h))) return rc;
    if (c.has_bias && (rc = take(p + ".self_attn.q_proj.bias", q))) return rc;
    if ((rc = take(p + ".self_attn.k_proj.weight", kv * h))) return rc;
    if (c.has_bias && (rc = take(p + ".self_attn.k_proj.bias", kv))) return rc;
    if ((rc = take(p + ".self_attn.v_proj.weight", kv * h))) return rc;
    if (c.has_bias && (rc = take(p + ".self_attn.v_proj.bias", kv))) return rc;
    if ((rc = take(p + ".self_attn.o_proj.weight", h * q))) return rc;
    if ((rc = take(p + ".post_attention_layernorm.weight", h))) return rc;
    if ((rc = take(p + ".mlp.gate_proj.weight", ff * h))) return rc;
    if ((rc = take(p + ".mlp.up_proj.weight", ff * h))) return rc;
    if ((rc = take(p + ".mlp.down_proj.weight", h * ff))) return rc;
  }
  if ((rc = take("model.norm.weight", h))) return rc;
  if (!c.tie_word_embeddings && (rc = take("lm_head.weight", V * h))) return rc;
  rc = defer_gpu_model_create(&c, ptrs.data(), ptrs.size(), 0, out);
  if (rc) return fail(DEFER_HOST_E_GPU, "defer_gpu error %d: %s", rc, defer_gpu_last_error());
  if (cfg_out) *cfg_out = c;
  if (signature) memcpy(signature, st->signature, 32);
  return DEFER_HOST_OK;
}
