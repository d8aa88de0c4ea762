// loader.cpp - the GPTQ / AutoRound int4 g64 checkpoint loader.
//
// Replaces the reference's loader for the decoders this build runs (src/loader/loader.cc: the
// name view and the per-tensor binding; src/loader/quant.cc: QuantConfig::parse and
// assert_quant_invariants, docs/13-loader.md "The three data checks"; src/common/repack.h:
// the interleave16 gate||up column map and the layout-1 expert tiles; src/loader/moe.cc: the
// expert blocks and the router || shared-gate rows). A checkpoint is a directory with
// config.json and one or more *.safetensors files of a Qwen3-style GQA decoder:
//   * int4 linears in GPTQ packing: qweight I32 [K/8][N] (8 nibbles per word, low first, the
//     stored value q + 8), scales F16 [K/64][N]; qzeros, when shipped, all 0x77777777 (GPTQ v1
//     stores the zero point minus one: symmetric); g_idx, when shipped, the identity k / 64;
//     every scale a finite f16 (subnormals are counted, not flushed);
//   * 16-bit (BF16 / F16 / F32) embeddings, norms, the MoE router and shared-expert gate;
//   * lm_head int4, or 16-bit (or tied to the embeddings) and then quantised here to int4 g64
//     with GPTQ's symmetric round-to-nearest (scale = f16(2 amax / 15), q = clamp(rint(w /
//     scale) + 8, 0, 15)), since the head GEMV reads int4.
// The safetensors files are memory-mapped and read as data only (an 8-byte header length, a
// JSON header, then the tensors): nothing in a checkpoint is executed.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "mi_capi_internal.h"

namespace mi {
namespace ld {

// ---- a small JSON reader (objects, arrays, strings, numbers, true / false / null) ----
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct Parser {
  const char* p;
  const char* end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
  }
  bool str(std::string& out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) return fail("bad escape");
        switch (*p) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {  // keep the code point's low byte; names and keys here are ASCII
            if (end - p < 5) return fail("bad \\u escape");
            out += static_cast<char>(std::strtol(std::string(p + 1, p + 5).c_str(), nullptr, 16) & 0x7F);
            p += 4;
            break;
          }
          default: out += *p;
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    if (*p == '{') {
      v.kind = Json::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') { ++p; return true; }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        Json c;
        if (!value(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == '}') { ++p; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      v.kind = Json::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') { ++p; return true; }
      for (;;) {
        Json c;
        if (!value(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == ']') { ++p; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') { v.kind = Json::Str; return str(v.str); }
    if (end - p >= 4 && !std::strncmp(p, "true", 4)) { v.kind = Json::Bool; v.b = true; p += 4; return true; }
    if (end - p >= 5 && !std::strncmp(p, "false", 5)) { v.kind = Json::Bool; v.b = false; p += 5; return true; }
    if (end - p >= 4 && !std::strncmp(p, "null", 4)) { v.kind = Json::Null; p += 4; return true; }
    char* q = nullptr;
    const std::string tok(p, std::min<size_t>(64, end - p));
    v.num = std::strtod(tok.c_str(), &q);
    if (q == tok.c_str()) return fail("bad value");
    v.kind = Json::Num;
    p += q - tok.c_str();
    return true;
  }
};

bool parse_json(const char* text, size_t n, Json& out, std::string& err) {
  Parser ps{text, text + n, {}};
  if (!ps.value(out, 0)) {
    err = ps.err;
    return false;
  }
  return true;
}

// ---- fp16 / bf16 conversions (round to nearest even; subnormals kept) ----
inline uint32_t fbits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
inline float bitsf(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline float f16_to_f32(uint16_t h) {
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0) v = float(m) * 5.9604644775390625e-08f;
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = bitsf(((e + 112u) << 23) | (m << 13));
  return (h & 0x8000u) ? -v : v;
}
inline float bf16_to_f32(uint16_t h) { return bitsf(uint32_t(h) << 16); }
// false when |f| rounds past 65504 (the value does not fit an f16) or f is not finite
inline bool f32_to_f16(float f, uint16_t& out) {
  uint32_t u = fbits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  u &= 0x7FFFFFFFu;
  if (u >= 0x7F800000u) return false;
  if (u >= 0x477FF000u) return false;  // rounds to 65520 or more
  if (u < 0x38800000u) {                // an f16 subnormal (or zero): m x 2^-24, rounded
    out = uint16_t(sign | uint32_t(std::nearbyint(bitsf(u) * 16777216.0f)));
    return true;
  }
  const uint32_t e = (u >> 23) - 112u, m = u & 0x7FFFFFu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  out = uint16_t(sign | h);
  return true;
}

// ---- memory-mapped safetensors ----
struct Tensor {
  std::string dtype;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  size_t numel() const {
    size_t n = 1;
    for (int64_t d : shape) n *= size_t(d);
    return n;
  }
};

struct Mapped {
  void* base = MAP_FAILED;
  size_t len = 0;
  ~Mapped() {
    if (base != MAP_FAILED) munmap(base, len);
  }
};

struct Checkpoint {
  std::vector<std::unique_ptr<Mapped>> maps;
  std::map<std::string, Tensor> t;
  std::map<std::string, bool> used;
  Json config;
  std::string err;

  bool fail(const std::string& m) {
    if (err.empty()) err = m;
    return false;
  }
  const Tensor* find(const std::string& n) const {
    auto it = t.find(n);
    return it == t.end() ? nullptr : &it->second;
  }
  const Tensor* take(const std::string& n) {
    const Tensor* x = find(n);
    if (x) used[n] = true;
    return x;
  }

  bool open_file(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail("cannot open " + path);
    struct stat st {};
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
      ::close(fd);
      return fail("not a safetensors file: " + path);
    }
    auto m = std::make_unique<Mapped>();
    m->len = size_t(st.st_size);
    m->base = mmap(nullptr, m->len, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m->base == MAP_FAILED) return fail("mmap failed: " + path);
    const uint8_t* b = static_cast<const uint8_t*>(m->base);
    uint64_t hlen = 0;
    std::memcpy(&hlen, b, 8);
    if (hlen > m->len - 8) return fail("bad header length: " + path);
    Json h;
    std::string jerr;
    if (!parse_json(reinterpret_cast<const char*>(b + 8), size_t(hlen), h, jerr) || h.kind != Json::Obj)
      return fail("bad safetensors header (" + jerr + "): " + path);
    const uint8_t* data = b + 8 + hlen;
    const size_t data_len = m->len - 8 - size_t(hlen);
    for (const auto& kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      const Json* dt = kv.second.get("dtype");
      const Json* sh = kv.second.get("shape");
      const Json* off = kv.second.get("data_offsets");
      if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
          off->arr.size() != 2)
        return fail("bad tensor entry " + kv.first + " in " + path);
      Tensor x;
      x.dtype = dt->str;
      for (const auto& d : sh->arr) x.shape.push_back(int64_t(d.num));
      const size_t b0 = size_t(off->arr[0].num), b1 = size_t(off->arr[1].num);
      if (b1 < b0 || b1 > data_len) return fail("tensor " + kv.first + " runs past the file");
      x.data = data + b0;
      x.nbytes = b1 - b0;
      if (t.count(kv.first)) return fail("tensor " + kv.first + " appears twice");
      t[kv.first] = x;
    }
    maps.push_back(std::move(m));
    return true;
  }

  bool open_dir(const std::string& dir) {
    DIR* d = opendir(dir.c_str());
    if (!d) return fail("cannot open directory " + dir);
    std::vector<std::string> files;
    while (dirent* e = readdir(d)) {
      const std::string n = e->d_name;
      if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(dir + "/" + n);
    }
    closedir(d);
    if (files.empty()) return fail("no .safetensors files in " + dir);
    std::sort(files.begin(), files.end());
    for (const auto& f : files)
      if (!open_file(f)) return false;
    // config.json
    const std::string cp = dir + "/config.json";
    FILE* f = std::fopen(cp.c_str(), "rb");
    if (!f) return fail("missing " + cp);
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    std::fclose(f);
    std::string jerr;
    if (!parse_json(text.data(), text.size(), config, jerr) || config.kind != Json::Obj)
      return fail("bad config.json (" + jerr + ")");
    return true;
  }
};

// config.json accessors (the language model's block may sit under "text_config")
const Json* cfg_root(const Json& c) {
  const Json* tc = c.get("text_config");
  return tc && tc->kind == Json::Obj ? tc : &c;
}
bool cfg_num(const Json& c, const char* k, double& v) {
  const Json* x = cfg_root(c)->get(k);
  if (!x) x = c.get(k);
  if (!x || x->kind != Json::Num) return false;
  v = x->num;
  return true;
}
bool cfg_bool(const Json& c, const char* k, bool dflt) {
  const Json* x = cfg_root(c)->get(k);
  if (!x) x = c.get(k);
  return x && x->kind == Json::Bool ? x->b : dflt;
}

// QuantConfig::parse (quant.cc; docs/13-loader.md): int4, group 64, symmetric, no activation
// order, GPTQ packing (auto_round:auto_gptq or plain GPTQ)
bool check_quant(const Json& c, std::string& err, bool& desc_act_declared) {
  const Json* q = c.get("quantization_config");
  if (!q) q = cfg_root(c)->get("quantization_config");
  if (!q || q->kind != Json::Obj) {
    err = "config.json has no quantization_config (an int4 GPTQ / AutoRound checkpoint is required)";
    return false;
  }
  const Json* m = q->get("quant_method");
  if (!m || m->kind != Json::Str || (m->str != "gptq" && m->str != "auto-round" && m->str != "intel/auto-round")) {
    err = "quant_method must be gptq or auto-round";
    return false;
  }
  const Json* pf = q->get("packing_format");
  if (pf && pf->kind == Json::Str && pf->str != "auto_round:auto_gptq" && pf->str != "auto_gptq") {
    err = "packing_format " + pf->str + " is not GPTQ packing";
    return false;
  }
  const Json* bits = q->get("bits");
  const Json* gs = q->get("group_size");
  const Json* sym = q->get("sym");
  if (!bits || bits->kind != Json::Num || bits->num != 4) { err = "bits must be 4"; return false; }
  if (!gs || gs->kind != Json::Num || gs->num != 64) { err = "group_size must be 64"; return false; }
  if (!sym || sym->kind != Json::Bool || !sym->b) { err = "sym must be true"; return false; }
  const Json* da = q->get("desc_act");
  desc_act_declared = da != nullptr;
  if (da && da->kind == Json::Bool && da->b) { err = "desc_act must be false"; return false; }
  return true;
}

struct Report {
  size_t linears = 0, qzeros = 0, g_idx = 0, subnormal_scales = 0, quantised_head = 0;
  size_t mtp_tensors = 0, mtp_quantised = 0;  // the MTP head's tensors; its linears quantised at load
};

// one int4 linear: qweight I32 [K/8][N], scales F16 [K/64][N]; the data checks of
// assert_quant_invariants on its qzeros, g_idx and scales
struct Linear4 {
  const uint32_t* q = nullptr;
  const uint16_t* s = nullptr;
  uint32_t K = 0, N = 0;
};
bool get_linear(Checkpoint& ck, const std::string& base, uint32_t K, uint32_t N, Linear4& out, Report& rep) {
  const Tensor* qw = ck.take(base + ".qweight");
  const Tensor* sc = ck.take(base + ".scales");
  if (!qw || !sc) return ck.fail("missing " + base + ".qweight / .scales");
  if (qw->dtype != "I32" || qw->shape.size() != 2 || qw->shape[0] != K / 8 || qw->shape[1] != N)
    return ck.fail(base + ".qweight: expected I32 [" + std::to_string(K / 8) + ", " + std::to_string(N) + "]");
  if (sc->dtype != "F16" || sc->shape.size() != 2 || sc->shape[0] != K / 64 || sc->shape[1] != N)
    return ck.fail(base + ".scales: expected F16 [" + std::to_string(K / 64) + ", " + std::to_string(N) + "]");
  if ((reinterpret_cast<uintptr_t>(qw->data) & 3) || (reinterpret_cast<uintptr_t>(sc->data) & 1))
    return ck.fail(base + ": misaligned tensor data");
  out.q = reinterpret_cast<const uint32_t*>(qw->data);
  out.s = reinterpret_cast<const uint16_t*>(sc->data);
  out.K = K;
  out.N = N;
  for (size_t i = 0, n = sc->numel(); i < n; ++i) {
    const uint16_t h = out.s[i];
    if (((h >> 10) & 0x1F) == 0x1F) {
      char b[160];
      std::snprintf(b, sizeof b, "%s.scales[%zu] = 0x%04X is not a finite f16", base.c_str(), i, h);
      return ck.fail(b);
    }
    if (((h >> 10) & 0x1F) == 0 && (h & 0x3FF)) ++rep.subnormal_scales;
  }
  if (const Tensor* qz = ck.take(base + ".qzeros")) {
    if (qz->dtype != "I32") return ck.fail(base + ".qzeros: expected I32");
    const uint32_t* z = reinterpret_cast<const uint32_t*>(qz->data);
    for (size_t i = 0, n = qz->nbytes / 4; i < n; ++i)
      if (z[i] != 0x77777777u) {
        char b[160];
        std::snprintf(b, sizeof b, "%s.qzeros[%zu] = 0x%08X (symmetric int4 stores 0x77777777)", base.c_str(), i, z[i]);
        return ck.fail(b);
      }
    ++rep.qzeros;
  }
  if (const Tensor* gi = ck.take(base + ".g_idx")) {
    if (gi->dtype != "I32" || gi->numel() != K) return ck.fail(base + ".g_idx: expected I32 [K]");
    const int32_t* g = reinterpret_cast<const int32_t*>(gi->data);
    for (uint32_t k = 0; k < K; ++k)
      if (g[k] != int32_t(k / 64)) {
        char b[160];
        std::snprintf(b, sizeof b, "%s.g_idx[%u] = %d (activation order is not supported)", base.c_str(), k, g[k]);
        return ck.fail(b);
      }
    ++rep.g_idx;
  }
  ++rep.linears;
  return true;
}

// a 16-bit (or F32) tensor of `n` elements as fp32
bool get_float(Checkpoint& ck, const std::string& name, size_t n, std::vector<float>& out) {
  const Tensor* x = ck.take(name);
  if (!x) return ck.fail("missing " + name);
  if (x->numel() != n) return ck.fail(name + ": expected " + std::to_string(n) + " elements");
  out.resize(n);
  if (x->dtype == "F32") {
    std::memcpy(out.data(), x->data, n * 4);
  } else if (x->dtype == "F16" || x->dtype == "BF16") {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(x->data);
    for (size_t i = 0; i < n; ++i) out[i] = x->dtype == "F16" ? f16_to_f32(h[i]) : bf16_to_f32(h[i]);
  } else {
    return ck.fail(name + ": expected F32, F16 or BF16, found " + x->dtype);
  }
  return true;
}
bool to_f16(Checkpoint& ck, const std::string& name, const std::vector<float>& v, std::vector<uint16_t>& out) {
  out.resize(v.size());
  for (size_t i = 0; i < v.size(); ++i)
    if (!f32_to_f16(v[i], out[i])) return ck.fail(name + ": a value does not fit an f16 (" + std::to_string(v[i]) + ")");
  return true;
}

// GPTQ's symmetric round-to-nearest int4 g64 of a row-major [N][K] fp32 matrix, in the GPTQ
// packing (qweight [K/8][N], scales [K/64][N])
void quantise_rtn(const std::vector<float>& w, uint32_t N, uint32_t K, std::vector<uint32_t>& qw,
                  std::vector<uint16_t>& sc) {
  qw.assign(size_t(K / 8) * N, 0u);
  sc.assign(size_t(K / 64) * N, 0u);
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t g = 0; g < K / 64; ++g) {
      const float* row = w.data() + size_t(n) * K + size_t(g) * 64;
      float amax = 0.f;
      for (int i = 0; i < 64; ++i) amax = std::fmax(amax, std::fabs(row[i]));
      uint16_t s16 = 0;
      f32_to_f16(2.0f * amax / 15.0f, s16);
      sc[size_t(g) * N + n] = s16;
      const float s = f16_to_f32(s16);
      for (int i = 0; i < 64; ++i) {
        float q = s == 0.f ? 8.f : std::nearbyint(row[i] / s) + 8.f;
        q = std::fmin(std::fmax(q, 0.f), 15.f);
        const uint32_t k = g * 64 + i;
        qw[size_t(k / 8) * N + n] |= uint32_t(q) << (4 * (k % 8));
      }
    }
}

// columns of several [rows][n_i] matrices side by side
template <typename T>
void concat_cols(const std::vector<std::pair<const T*, uint32_t>>& parts, uint32_t rows, std::vector<T>& out) {
  uint32_t N = 0;
  for (const auto& p : parts) N += p.second;
  out.resize(size_t(rows) * N);
  for (uint32_t r = 0; r < rows; ++r) {
    uint32_t c0 = 0;
    for (const auto& p : parts) {
      std::memcpy(out.data() + size_t(r) * N + c0, p.first + size_t(r) * p.second, size_t(p.second) * sizeof(T));
      c0 += p.second;
    }
  }
}
// repack.h's interleave16: column n of the fused gate||up is gate column (n / 32) 16 + n % 16
// when n % 32 < 16, else up column (n / 32) 16 + n % 16
template <typename T>
void interleave16(const T* a, const T* b, uint32_t rows, uint32_t Np, std::vector<T>& out) {
  const uint32_t NT = 2 * Np;
  out.resize(size_t(rows) * NT);
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t n = 0; n < NT; ++n) {
      const uint32_t src = (n / 32) * 16 + n % 16;
      out[size_t(r) * NT + n] = ((n % 32) >= 16 ? b : a)[size_t(r) * Np + src];
    }
}
// repack.h:17-30 layout 1: per (16-column tile, 64-k group) 136 words: the 128 nibble words
// [8 k-octets][16 columns], then the 16 scales as 8 words (low half first)
void layout1(const uint32_t* qw, const uint16_t* sc, uint32_t K, uint32_t N, uint32_t* out) {
  const uint32_t G = K / 64, NT = N / 16;
  for (uint32_t nt = 0; nt < NT; ++nt)
    for (uint32_t g = 0; g < G; ++g) {
      uint32_t* tile = out + (size_t(nt) * G + g) * 136;
      for (uint32_t j = 0; j < 8; ++j)
        for (uint32_t l = 0; l < 16; ++l) tile[j * 16 + l] = qw[size_t(g * 8 + j) * N + nt * 16 + l];
      for (uint32_t l = 0; l < 16; l += 2)
        tile[128 + l / 2] = uint32_t(sc[size_t(g) * N + nt * 16 + l]) | (uint32_t(sc[size_t(g) * N + nt * 16 + l + 1]) << 16);
    }
}
// the router's f16 tiles (gemv_bf16's layout): element (n, k) of the [N][K] matrix at
// ((n / 16) (K / 8) + k / 8) 128 + (k % 8) 16 + n % 16
void f16w_tile(const uint16_t* w, uint32_t K, uint32_t N, uint16_t* out) {
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t k = 0; k < K; ++k)
      out[(size_t(n / 16) * (K / 8) + k / 8) * 128 + (k % 8) * 16 + n % 16] = w[size_t(n) * K + k];
}

}  // namespace ld
}  // namespace mi

using namespace mi::ld;

namespace {
// the language model's tensor prefix: "model.language_model." or "model."
std::string lm_prefix(const Checkpoint& ck) {
  if (ck.find("model.language_model.embed_tokens.weight")) return "model.language_model.";
  return "model.";
}
int fail_ck(const Checkpoint& ck) { return mi_fail(MI_ERR_ARG, ck.err.c_str()); }
}  // namespace

extern "C" {

int mi_checkpoint_desc(const char* dir, uint32_t max_len, uint32_t max_rows, mi_model_desc* desc) {
  if (!dir || !desc || max_len == 0 || max_rows == 0) return mi_fail(MI_ERR_ARG, "checkpoint_desc: bad arguments");
  Checkpoint ck;
  if (!ck.open_dir(dir)) return fail_ck(ck);
  std::string err;
  bool dad = false;
  if (!check_quant(ck.config, err, dad)) return mi_fail(MI_ERR_SHAPE, err.c_str());
  double L, H, QH, KVH, HD = 0, I = 0, V, theta = 1e6, eps = 1e-6, E = 0, TOPK = 0, MI = 0, SI = 0, prf = 1;
  if (!cfg_num(ck.config, "num_hidden_layers", L) || !cfg_num(ck.config, "hidden_size", H) ||
      !cfg_num(ck.config, "num_attention_heads", QH) || !cfg_num(ck.config, "vocab_size", V))
    return mi_fail(MI_ERR_SHAPE, "config.json: num_hidden_layers, hidden_size, num_attention_heads, vocab_size required");
  if (!cfg_num(ck.config, "num_key_value_heads", KVH)) KVH = QH;
  if (!cfg_num(ck.config, "head_dim", HD)) HD = H / QH;
  cfg_num(ck.config, "intermediate_size", I);
  cfg_num(ck.config, "rope_theta", theta);
  cfg_num(ck.config, "rms_norm_eps", eps);
  cfg_num(ck.config, "partial_rotary_factor", prf);
  const bool moe = cfg_num(ck.config, "num_experts", E) && E > 0;
  if (moe) {
    cfg_num(ck.config, "num_experts_per_tok", TOPK);
    cfg_num(ck.config, "moe_intermediate_size", MI);
    cfg_num(ck.config, "shared_expert_intermediate_size", SI);
    if (SI != MI)
      return mi_fail(MI_ERR_SHAPE, "config.json: the MoE block needs one shared expert of moe_intermediate_size");
  }
  const std::string pre = lm_prefix(ck);
  mi_model_desc d{};
  d.layers = uint32_t(L);
  d.hidden = uint32_t(H);
  d.q_heads = uint32_t(QH);
  d.kv_heads = uint32_t(KVH);
  d.head_dim = uint32_t(HD);
  d.rot_dim = uint32_t(HD * prf);
  d.inter = moe ? 0u : uint32_t(I);
  d.vocab = uint32_t(V);
  d.vocab_used = uint32_t(V);
  d.max_len = max_len;
  d.qk_norm = ck.find(pre + "layers.0.self_attn.q_norm.weight") ? 1u : 0u;
  d.max_rows = max_rows;
  d.attn_tgt = 64;
  d.rope_theta = float(theta);
  d.rms_eps = float(eps);
  d.experts = moe ? uint32_t(E) : 0u;
  d.top_k = moe ? uint32_t(TOPK) : 0u;
  d.moe_inter = moe ? uint32_t(MI) : 0u;
  d.kv_int8 = 0;
  if (d.vocab % 64) {  // the head GEMV works in 64-column tiles: pad, and mask the tail
    d.vocab = (d.vocab + 63) / 64 * 64;
  }
  *desc = d;
  return 0;
}

int mi_checkpoint_check(const char* dir, char* report, size_t report_len) {
  if (!dir) return mi_fail(MI_ERR_ARG, "checkpoint_check: bad arguments");
  Checkpoint ck;
  if (!ck.open_dir(dir)) return fail_ck(ck);
  std::string err;
  bool dad = false;
  if (!check_quant(ck.config, err, dad)) return mi_fail(MI_ERR_SHAPE, err.c_str());
  Report rep;
  size_t gidx_seen = 0;
  for (const auto& kv : ck.t) {
    const std::string& n = kv.first;
    if (n.size() > 8 && n.compare(n.size() - 8, 8, ".qweight") == 0) {
      const Tensor& q = kv.second;
      if (q.shape.size() != 2) return mi_fail(MI_ERR_SHAPE, (n + ": expected a 2-d qweight").c_str());
      Linear4 l;
      if (!get_linear(ck, n.substr(0, n.size() - 8), uint32_t(q.shape[0] * 8), uint32_t(q.shape[1]), l, rep))
        return fail_ck(ck);
    }
    if (n.size() > 6 && n.compare(n.size() - 6, 6, ".g_idx") == 0) ++gidx_seen;
  }
  // quant.cc: an undeclared desc_act is inferred false only when no g_idx is shipped
  if (!dad && gidx_seen)
    return mi_fail(MI_ERR_SHAPE, ("config.json declares no desc_act but the checkpoint ships " +
                                  std::to_string(gidx_seen) + " g_idx tensors").c_str());
  if (report && report_len)
    std::snprintf(report, report_len, "%zu int4 linears; %zu qzeros + %zu g_idx checked; %zu subnormal scales",
                  rep.linears, rep.qzeros, rep.g_idx, rep.subnormal_scales);
  return 0;
}

int mi_engine_load(mi_engine* e, const char* dir, char* report, size_t report_len) {
  if (!e || !dir) return mi_fail(MI_ERR_ARG, "engine_load: bad arguments");
  Checkpoint ck;
  if (!ck.open_dir(dir)) return fail_ck(ck);
  std::string err;
  bool dad = false;
  if (!check_quant(ck.config, err, dad)) return mi_fail(MI_ERR_SHAPE, err.c_str());
  if (int rc = mi_checkpoint_check(dir, nullptr, 0)) return rc;
  // the engine's shape, from its tensors
  mi_model_desc want{};
  if (int rc = mi_checkpoint_desc(dir, 1, 1, &want)) return rc;
  void* st = mi_engine_stream(e);
  // the engine's lm_head form (its descriptor's lm_head_int8): whether it holds an int8 head
  bool head_i8 = false;
  {
    void* p8 = nullptr;
    size_t b8 = 0;
    if (int rc = mi_engine_tensor(e, MI_T_LM_I8, 0, &p8, &b8)) return rc;
    head_i8 = b8 != 0;
  }
  // the MTP head's form (its descriptor's mtp_w16): whether it holds 16-bit linears
  bool head_w16 = false;
  {
    void* p16 = nullptr;
    size_t b16 = 0;
    if (int rc = mi_engine_tensor(e, MI_T_MTP_W16_FC, 0, &p16, &b16)) return rc;
    head_w16 = b16 != 0;
  }
  const std::string pre = lm_prefix(ck);
  const uint32_t H = want.hidden, QH = want.q_heads, KVH = want.kv_heads, HD = want.head_dim;
  const uint32_t I = want.inter, Vp = want.vocab;
  uint32_t V = 0;
  {
    double v = 0;
    cfg_num(ck.config, "vocab_size", v);
    V = uint32_t(v);
  }
  Report rep;
  std::vector<std::vector<uint8_t>> keep;  // host staging kept alive until the stream drains
  auto upload = [&](uint32_t kind, uint32_t layer, const void* src, size_t bytes, const char* what) -> int {
    void* p = nullptr;
    size_t cap = 0;
    if (int rc = mi_engine_tensor(e, kind, layer, &p, &cap)) return rc;
    if (!p || cap != bytes) {
      char b[200];
      std::snprintf(b, sizeof b, "engine_load: %s (layer %u) is %zu bytes in the checkpoint, %zu in the engine "
                    "(the engine's model description does not match config.json)", what, layer, bytes, cap);
      return mi_fail(MI_ERR_SHAPE, b);
    }
    keep.emplace_back(static_cast<const uint8_t*>(src), static_cast<const uint8_t*>(src) + bytes);
    return mi_memcpy_h2d(p, keep.back().data(), bytes, st);
  };
  auto flush = [&]() -> int {
    const int rc = mi_stream_sync(st);
    keep.clear();
    return rc;
  };
  std::vector<float> f32;
  std::vector<uint16_t> f16;
  std::vector<uint32_t> qcat;
  std::vector<uint16_t> scat;
  // embeddings
  if (!get_float(ck, pre + "embed_tokens.weight", size_t(V) * H, f32)) return fail_ck(ck);
  if (mi_engine_act_bf16(e)) {  // bf16 activations: the table in bf16 (common/bf16.h:12-16's rounding)
    f16.resize(f32.size());
    for (size_t i = 0; i < f32.size(); ++i) {
      uint32_t u;
      std::memcpy(&u, &f32[i], 4);
      f16[i] = uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
  } else if (!to_f16(ck, "embed_tokens", f32, f16)) {
    return fail_ck(ck);
  }
  f16.resize(size_t(Vp) * H, 0);
  if (int rc = upload(MI_T_EMBED, 0, f16.data(), f16.size() * 2, "embed_tokens")) return rc;
  if (!get_float(ck, pre + "norm.weight", H, f32)) return fail_ck(ck);
  if (int rc = upload(MI_T_FINAL_NORM, 0, f32.data(), f32.size() * 4, "norm")) return rc;
  // lm_head: int4 as shipped, or a 16-bit head (or the tied embeddings) quantised here to int4
  // g64 - or, for an engine built with the int8 head, to int8 rows (lm_head_int8.cc: a packed
  // head is refused there as here)
  if (head_i8) {
    if (ck.find("lm_head.qweight"))
      return mi_fail(MI_ERR_ARG, "engine_load: the int8 lm_head is made from a 16-bit head, this one is packed");
    const std::string src = ck.find("lm_head.weight") ? "lm_head.weight" : pre + "embed_tokens.weight";
    if (src != "lm_head.weight" && !cfg_bool(ck.config, "tie_word_embeddings", false))
      return mi_fail(MI_ERR_ARG, "engine_load: no lm_head and tie_word_embeddings is not set");
    if (!get_float(ck, src, size_t(V) * H, f32)) return fail_ck(ck);
    f32.resize(size_t(Vp) * H, 0.f);  // padded vocabulary rows: scale 0, q 0 (masked by vocab_used)
    std::vector<int8_t> q8(size_t(Vp) * H);
    std::vector<float> s8(Vp);
    if (int rc = mi_lm_head_int8_quantise(f32.data(), H, Vp, q8.data(), s8.data())) return rc;
    rep.quantised_head = 1;
    if (int rc = upload(MI_T_LM_I8, 0, q8.data(), q8.size(), "lm_head (int8)")) return rc;
    if (int rc = upload(MI_T_LM_I8_S, 0, s8.data(), s8.size() * 4, "lm_head scales (int8)")) return rc;
  } else {
    Linear4 lm;
    std::vector<uint32_t> lq;
    std::vector<uint16_t> ls;
    if (ck.find("lm_head.qweight")) {
      if (!get_linear(ck, "lm_head", H, V, lm, rep)) return fail_ck(ck);
      lq.assign(lm.q, lm.q + size_t(H / 8) * V);
      ls.assign(lm.s, lm.s + size_t(H / 64) * V);
    } else {
      const std::string src = ck.find("lm_head.weight") ? "lm_head.weight" : pre + "embed_tokens.weight";
      if (src != "lm_head.weight" && !cfg_bool(ck.config, "tie_word_embeddings", false))
        return mi_fail(MI_ERR_ARG, "engine_load: no lm_head and tie_word_embeddings is not set");
      if (!get_float(ck, src, size_t(V) * H, f32)) return fail_ck(ck);
      quantise_rtn(f32, V, H, lq, ls);
      rep.quantised_head = 1;
    }
    if (Vp != V) {  // padded vocabulary columns: zero weights (masked by vocab_used)
      std::vector<uint32_t> q2(size_t(H / 8) * Vp, 0x88888888u);
      std::vector<uint16_t> s2(size_t(H / 64) * Vp, 0);
      for (uint32_t r = 0; r < H / 8; ++r) std::memcpy(&q2[size_t(r) * Vp], &lq[size_t(r) * V], size_t(V) * 4);
      for (uint32_t r = 0; r < H / 64; ++r) std::memcpy(&s2[size_t(r) * Vp], &ls[size_t(r) * V], size_t(V) * 2);
      lq.swap(q2);
      ls.swap(s2);
    }
    if (int rc = upload(MI_T_LM_Q, 0, lq.data(), lq.size() * 4, "lm_head.qweight")) return rc;
    if (int rc = upload(MI_T_LM_S, 0, ls.data(), ls.size() * 2, "lm_head.scales")) return rc;
  }
  if (int rc = flush()) return rc;
  const bool moe = want.experts > 0;
  const uint32_t E = want.experts, MI = want.moe_inter;
  // one int4 linear as shipped, or (rtn: the MTP head's 16-bit linears) quantised here by rtn.h's
  // rule from its 16-bit weight
  auto linear_or_rtn = [&](const std::string& base, uint32_t K, uint32_t N, bool rtn, std::vector<uint32_t>& q,
                           std::vector<uint16_t>& sc) -> bool {
    if (!rtn || ck.find(base + ".qweight")) {
      Linear4 l;
      if (!get_linear(ck, base, K, N, l, rep)) return false;
      q.assign(l.q, l.q + size_t(K / 8) * N);
      sc.assign(l.s, l.s + size_t(K / 64) * N);
      return true;
    }
    if (!ck.find(base + ".weight"))
      return ck.fail("engine_load: the engine has an MTP head and the checkpoint has no " + base + " (.weight or .qweight)");
    if (!get_float(ck, base + ".weight", size_t(N) * K, f32)) return false;
    quantise_rtn(f32, N, K, q, sc);
    ++rep.mtp_quantised;
    return true;
  };
  // an MoE layer's FFN under prefix lp into layer index li: router || shared gate as f16 tiles
  // (rows 0..E-1 the router, row E the shared expert's gate, zero rows up to a multiple of 16,
  // moe.cc), the experts and the shared expert (last) as layout-1 blocks
  auto load_moe_ffn = [&](const std::string& lp, uint32_t li, bool rtn) -> int {
    const uint32_t RN = (E + 1 + 15) / 16 * 16;
    std::vector<float> rt;
    if (!get_float(ck, lp + "mlp.gate.weight", size_t(E) * H, rt)) return fail_ck(ck);
    if (!get_float(ck, lp + "mlp.shared_expert_gate.weight", H, f32)) return fail_ck(ck);
    rt.insert(rt.end(), f32.begin(), f32.end());
    rt.resize(size_t(RN) * H, 0.f);
    if (!to_f16(ck, lp + "mlp.gate", rt, f16)) return fail_ck(ck);
    std::vector<uint16_t> tiles(f16.size());
    f16w_tile(f16.data(), H, RN, tiles.data());
    if (int rc = upload(MI_T_ROUTER, li, tiles.data(), tiles.size() * 2, "router")) return rc;
    const size_t gub = size_t(2 * MI / 16) * (H / 64) * 136, dnb = size_t(H / 16) * (MI / 64) * 136;
    std::vector<uint32_t> gu((E + 1) * gub), dn((E + 1) * dnb), gq, uq, dq;
    std::vector<uint16_t> gs, us, ds;
    for (uint32_t ex = 0; ex <= E; ++ex) {
      const std::string ep = ex < E ? lp + "mlp.experts." + std::to_string(ex) + "." : lp + "mlp.shared_expert.";
      if (!linear_or_rtn(ep + "gate_proj", H, MI, rtn, gq, gs) || !linear_or_rtn(ep + "up_proj", H, MI, rtn, uq, us) ||
          !linear_or_rtn(ep + "down_proj", MI, H, rtn, dq, ds))
        return fail_ck(ck);
      interleave16(gq.data(), uq.data(), H / 8, MI, qcat);
      interleave16(gs.data(), us.data(), H / 64, MI, scat);
      layout1(qcat.data(), scat.data(), H, 2 * MI, gu.data() + ex * gub);
      layout1(dq.data(), ds.data(), MI, H, dn.data() + ex * dnb);
    }
    if (int rc = upload(MI_T_MOE_GU, li, gu.data(), gu.size() * 4, "expert gate||up blocks")) return rc;
    return upload(MI_T_MOE_DN, li, dn.data(), dn.size() * 4, "expert down blocks");
  };
  for (uint32_t li = 0; li < want.layers; ++li) {
    const std::string lp = pre + "layers." + std::to_string(li) + ".";
    Linear4 q, k, v, o;
    if (!get_linear(ck, lp + "self_attn.q_proj", H, QH * HD, q, rep) ||
        !get_linear(ck, lp + "self_attn.k_proj", H, KVH * HD, k, rep) ||
        !get_linear(ck, lp + "self_attn.v_proj", H, KVH * HD, v, rep) ||
        !get_linear(ck, lp + "self_attn.o_proj", QH * HD, H, o, rep))
      return fail_ck(ck);
    concat_cols<uint32_t>({{q.q, q.N}, {k.q, k.N}, {v.q, v.N}}, H / 8, qcat);
    concat_cols<uint16_t>({{q.s, q.N}, {k.s, k.N}, {v.s, v.N}}, H / 64, scat);
    if (int rc = upload(MI_T_QKV_Q, li, qcat.data(), qcat.size() * 4, "q||k||v qweight")) return rc;
    if (int rc = upload(MI_T_QKV_S, li, scat.data(), scat.size() * 2, "q||k||v scales")) return rc;
    if (int rc = upload(MI_T_O_Q, li, o.q, size_t(o.K / 8) * o.N * 4, "o_proj.qweight")) return rc;
    if (int rc = upload(MI_T_O_S, li, o.s, size_t(o.K / 64) * o.N * 2, "o_proj.scales")) return rc;
    if (!get_float(ck, lp + "input_layernorm.weight", H, f32)) return fail_ck(ck);
    if (int rc = upload(MI_T_IN_NORM, li, f32.data(), f32.size() * 4, "input_layernorm")) return rc;
    if (!get_float(ck, lp + "post_attention_layernorm.weight", H, f32)) return fail_ck(ck);
    if (int rc = upload(MI_T_POST_NORM, li, f32.data(), f32.size() * 4, "post_attention_layernorm")) return rc;
    if (want.qk_norm) {
      if (!get_float(ck, lp + "self_attn.q_norm.weight", HD, f32)) return fail_ck(ck);
      if (int rc = upload(MI_T_Q_NORM, li, f32.data(), f32.size() * 4, "q_norm")) return rc;
      if (!get_float(ck, lp + "self_attn.k_norm.weight", HD, f32)) return fail_ck(ck);
      if (int rc = upload(MI_T_K_NORM, li, f32.data(), f32.size() * 4, "k_norm")) return rc;
    }
    if (!moe) {
      Linear4 g, u, dn;
      if (!get_linear(ck, lp + "mlp.gate_proj", H, I, g, rep) || !get_linear(ck, lp + "mlp.up_proj", H, I, u, rep) ||
          !get_linear(ck, lp + "mlp.down_proj", I, H, dn, rep))
        return fail_ck(ck);
      interleave16(g.q, u.q, H / 8, I, qcat);
      interleave16(g.s, u.s, H / 64, I, scat);
      if (int rc = upload(MI_T_GU_Q, li, qcat.data(), qcat.size() * 4, "gate||up qweight")) return rc;
      if (int rc = upload(MI_T_GU_S, li, scat.data(), scat.size() * 2, "gate||up scales")) return rc;
      if (int rc = upload(MI_T_DOWN_Q, li, dn.q, size_t(I / 8) * H * 4, "down_proj.qweight")) return rc;
      if (int rc = upload(MI_T_DOWN_S, li, dn.s, size_t(I / 64) * H * 2, "down_proj.scales")) return rc;
    } else {
      if (int rc = load_moe_ffn(lp, li, false)) return rc;
    }
    if (int rc = flush()) return rc;
  }
  // The MTP head, for an engine created with one (desc.mtp; the reference loads it only when
  // asked, loader.cc:521-670): the 15 tensors of a dense head under `mtp.`. A linear shipped
  // in 16 bits (the published checkpoints ship the head in bf16) is quantised here to int4 g64
  // by rtn.h's round-to-nearest rule - the reference does that for its MoE head's experts;
  // the head only drafts, so its quantisation moves acceptance, never output; a packed int4
  // linear is taken as shipped. Layouts as the main layers': q||k||v by columns, gate/up
  // interleaved in 16-column blocks; fc reads cat(pre_fc_norm_embedding(e),
  // pre_fc_norm_hidden(h)), K = 2 hidden.
  if (mi_engine_has_mtp(e)) {
    const uint32_t HL = want.layers;  // the per-layer kinds at layer = layers are the head's
    auto mtp_linear = [&](const std::string& base, uint32_t K, uint32_t N, std::vector<uint32_t>& q,
                          std::vector<uint16_t>& sc) -> bool {
      ++rep.mtp_tensors;
      return linear_or_rtn(base, K, N, true, q, sc);
    };
    auto mtp_norm = [&](const std::string& name, uint32_t n, uint32_t kind, uint32_t layer) -> int {
      ++rep.mtp_tensors;
      if (!ck.find(name)) {
        ck.fail("engine_load: the engine has an MTP head and the checkpoint has no " + name);
        return fail_ck(ck);
      }
      if (!get_float(ck, name, n, f32)) return fail_ck(ck);
      return upload(kind, layer, f32.data(), f32.size() * 4, name.c_str());
    };
    std::vector<uint32_t> q1, q2, q3;
    std::vector<uint16_t> s1, s2, s3;
    // the 16-bit head (desc.mtp_w16, loader.cc:586-597): the linears' [N][K] weights (q||k||v
    // and gate||up by output rows, gate/up interleaved in 16-row blocks) as f16 in gemv_f16w's
    // tiles
    const bool w16 = head_w16;
    auto mtp_w16 = [&](const std::vector<std::string>& bases, const std::vector<uint32_t>& ns, uint32_t K, bool gu,
                       uint32_t kind) -> int {
      std::vector<float> all;
      uint32_t N = 0;
      for (size_t i = 0; i < bases.size(); ++i) {
        ++rep.mtp_tensors;
        if (!ck.find(bases[i] + ".weight")) {
          ck.fail("engine_load: a 16-bit MTP head needs " + bases[i] + ".weight (the checkpoint's head is not 16-bit)");
          return fail_ck(ck);
        }
        if (!get_float(ck, bases[i] + ".weight", size_t(ns[i]) * K, f32)) return fail_ck(ck);
        all.insert(all.end(), f32.begin(), f32.end());
        N += ns[i];
      }
      if (gu) {  // repack.h's interleave16 by rows: row n is gate row (n / 32) 16 + n % 16 (n % 32 < 16), else up's
        const uint32_t I2 = N / 2;
        std::vector<float> r(all.size());
        for (uint32_t n = 0; n < N; ++n) {
          const uint32_t src = (n % 32 < 16 ? 0u : I2) + (n / 32) * 16 + n % 16;
          std::memcpy(&r[size_t(n) * K], &all[size_t(src) * K], size_t(K) * 4);
        }
        all.swap(r);
      }
      std::vector<uint16_t> h16, tiles;
      if (!to_f16(ck, bases[0], all, h16)) return fail_ck(ck);
      tiles.resize(h16.size());
      f16w_tile(h16.data(), K, N, tiles.data());
      return upload(kind, 0, tiles.data(), tiles.size() * 2, bases[0].c_str());
    };
    if (w16) {
      if (int rc = mtp_w16({"mtp.fc"}, {H}, 2 * H, false, MI_T_MTP_W16_FC)) return rc;
    } else {
      if (!mtp_linear("mtp.fc", 2 * H, H, q1, s1)) return fail_ck(ck);
      if (int rc = upload(MI_T_MTP_FC_Q, 0, q1.data(), q1.size() * 4, "mtp.fc qweight")) return rc;
      if (int rc = upload(MI_T_MTP_FC_S, 0, s1.data(), s1.size() * 2, "mtp.fc scales")) return rc;
    }
    if (int rc = mtp_norm("mtp.pre_fc_norm_embedding.weight", H, MI_T_MTP_PRE_E, 0)) return rc;
    if (int rc = mtp_norm("mtp.pre_fc_norm_hidden.weight", H, MI_T_MTP_PRE_H, 0)) return rc;
    if (int rc = mtp_norm("mtp.norm.weight", H, MI_T_MTP_FINAL, 0)) return rc;
    if (int rc = flush()) return rc;
    const std::string lp = "mtp.layers.0.";
    if (w16) {
      if (int rc = mtp_w16({lp + "self_attn.q_proj", lp + "self_attn.k_proj", lp + "self_attn.v_proj"},
                          {QH * HD, KVH * HD, KVH * HD}, H, false, MI_T_MTP_W16_QKV))
        return rc;
      if (int rc = mtp_w16({lp + "self_attn.o_proj"}, {H}, QH * HD, false, MI_T_MTP_W16_O)) return rc;
    } else {
      std::vector<uint32_t> qq, kq, vq;
      std::vector<uint16_t> qs, ks, vs;
      if (!mtp_linear(lp + "self_attn.q_proj", H, QH * HD, qq, qs) ||
          !mtp_linear(lp + "self_attn.k_proj", H, KVH * HD, kq, ks) ||
          !mtp_linear(lp + "self_attn.v_proj", H, KVH * HD, vq, vs))
        return fail_ck(ck);
      concat_cols<uint32_t>({{qq.data(), QH * HD}, {kq.data(), KVH * HD}, {vq.data(), KVH * HD}}, H / 8, qcat);
      concat_cols<uint16_t>({{qs.data(), QH * HD}, {ks.data(), KVH * HD}, {vs.data(), KVH * HD}}, H / 64, scat);
      if (int rc = upload(MI_T_QKV_Q, HL, qcat.data(), qcat.size() * 4, "mtp q||k||v qweight")) return rc;
      if (int rc = upload(MI_T_QKV_S, HL, scat.data(), scat.size() * 2, "mtp q||k||v scales")) return rc;
      if (!mtp_linear(lp + "self_attn.o_proj", QH * HD, H, q1, s1)) return fail_ck(ck);
      if (int rc = upload(MI_T_O_Q, HL, q1.data(), q1.size() * 4, "mtp o_proj qweight")) return rc;
      if (int rc = upload(MI_T_O_S, HL, s1.data(), s1.size() * 2, "mtp o_proj scales")) return rc;
    }
    if (int rc = mtp_norm(lp + "input_layernorm.weight", H, MI_T_IN_NORM, HL)) return rc;
    if (int rc = mtp_norm(lp + "post_attention_layernorm.weight", H, MI_T_POST_NORM, HL)) return rc;
    if (want.qk_norm) {
      if (int rc = mtp_norm(lp + "self_attn.q_norm.weight", HD, MI_T_Q_NORM, HL)) return rc;
      if (int rc = mtp_norm(lp + "self_attn.k_norm.weight", HD, MI_T_K_NORM, HL)) return rc;
    }
    if (int rc = flush()) return rc;
    if (moe) {  // an MoE model's head (spec 15e): one MoE layer in the main layers' device form
      if (int rc = load_moe_ffn(lp, HL, true)) return rc;
      rep.mtp_tensors += 2 + 3 * (size_t(E) + 1);  // router, shared gate, the experts' linears
    } else if (w16) {
      if (int rc = mtp_w16({lp + "mlp.gate_proj", lp + "mlp.up_proj"}, {I, I}, H, true, MI_T_MTP_W16_GU)) return rc;
      if (int rc = mtp_w16({lp + "mlp.down_proj"}, {H}, I, false, MI_T_MTP_W16_DN)) return rc;
    } else {
      if (!mtp_linear(lp + "mlp.gate_proj", H, I, q1, s1) || !mtp_linear(lp + "mlp.up_proj", H, I, q2, s2) ||
          !mtp_linear(lp + "mlp.down_proj", I, H, q3, s3))
        return fail_ck(ck);
      interleave16(q1.data(), q2.data(), H / 8, I, qcat);
      interleave16(s1.data(), s2.data(), H / 64, I, scat);
      if (int rc = upload(MI_T_GU_Q, HL, qcat.data(), qcat.size() * 4, "mtp gate||up qweight")) return rc;
      if (int rc = upload(MI_T_GU_S, HL, scat.data(), scat.size() * 2, "mtp gate||up scales")) return rc;
      if (int rc = upload(MI_T_DOWN_Q, HL, q3.data(), q3.size() * 4, "mtp down_proj qweight")) return rc;
      if (int rc = upload(MI_T_DOWN_S, HL, s3.data(), s3.size() * 2, "mtp down_proj scales")) return rc;
    }
    if (int rc = flush()) return rc;
  }
  // every tensor of the language model must have been bound (qzeros / g_idx are checked and
  // dropped; other namespaces - vision towers, an MTP head the engine does not hold - are not
  // this engine's)
  size_t unused = 0;
  std::string first;
  for (const auto& kv : ck.t) {
    const std::string& n = kv.first;
    if (ck.used.count(n)) continue;
    if (n.compare(0, pre.size(), pre) != 0 && n.compare(0, 8, "lm_head.") != 0) continue;
    if (n.find(".rotary_emb.") != std::string::npos) continue;  // recomputed from rope_theta
    if (n == pre + "embed_tokens.weight") continue;
    ++unused;
    if (first.empty()) first = n;
  }
  if (unused) return mi_fail(MI_ERR_SHAPE, ("engine_load: " + std::to_string(unused) + " unbound tensors, first " + first).c_str());
  if (report && report_len) {
    std::snprintf(report, report_len,
                  "loaded %zu int4 linears; dropped %zu qzeros + %zu g_idx (invariants asserted); %zu subnormal "
                  "scales kept; lm_head %s; MTP head: %zu tensors, %zu linears quantised to int4 g64 at load%s",
                  rep.linears, rep.qzeros, rep.g_idx, rep.subnormal_scales,
                  rep.quantised_head ? (head_i8 ? "quantised to int8 rows at load" : "quantised to int4 g64 at load")
                                     : "int4 as shipped",
                  rep.mtp_tensors, rep.mtp_quantised, head_w16 ? " (its linears kept 16-bit)" : "");
  }
  return 0;
}

}  // extern "C"
