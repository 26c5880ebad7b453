// pgw_convert.cc -- HuggingFace checkpoint -> PGW1 Q4 file, in C++.
//
// The reference converts with Python (tools/convert_hf_to_pgw.py,
// tools/convert_gpt2_to_pgw.py): load the model through transformers, quantise
// every matrix with quant_q4, append the tensors to one payload in a fixed
// order, and write a 256-byte header, a compact JSON table and the payload.
// This restates that packaging for checkpoints already on disk (safetensors),
// without Python, torch or a network: the same weights give the same bytes.
//
// Built twice from this file: libpgwconvert.so (the C ABI of
// include/pgw_convert.h) and, with -DPGW_CONVERT_MAIN, the pgw_convert
// command.
#include "pgw_convert.h"

#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return 1;
}

// ---------------------------------------------------------------- JSON
// Enough JSON for config.json and safetensors headers: objects, arrays,
// strings (with \uXXXX escapes), numbers, true / false / null.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json *get(const std::string &k) const {
    if (kind != Obj) return nullptr;
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char *p, *end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *s) {
    const size_t n = strlen(s);
    if ((size_t)(end - p) < n || memcmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  static void utf8(std::string &o, unsigned c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xC0 | (c >> 6));
      o += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      o += (char)(0xE0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    } else {
      o += (char)(0xF0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 0x3F));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(unsigned &v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string &o) {
    if (p >= end || *p != '"') return false;
    ++p;
    while (p < end && *p != '"') {
      if (*p != '\\') {
        o += *p++;
        continue;
      }
      if (++p >= end) return false;
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
          unsigned v;
          if (!hex4(v)) return false;
          if (v >= 0xD800 && v < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            unsigned lo;
            if (!hex4(lo)) return false;
            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, v);
          break;
        }
        default: return false;
      }
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool value(Json &v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p >= end) return false;
    if (*p == '{') {
      ++p;
      v.kind = Json::Obj;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= end || *p != ':') return false;
        ++p;
        Json c;
        if (!value(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return false;
      }
    }
    if (*p == '[') {
      ++p;
      v.kind = Json::Arr;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        Json c;
        if (!value(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return false;
      }
    }
    if (*p == '"') {
      v.kind = Json::Str;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = Json::Bool;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = Json::Bool;
      return true;
    }
    if (lit("null")) return true;
    // number
    const char *s = p;
    if (p < end && (*p == '-' || *p == '+')) ++p;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) ++p;
    if (p == s) return false;
    const std::string t(s, p);
    char *e = nullptr;
    v.num = strtod(t.c_str(), &e);
    v.kind = Json::Num;
    return e && *e == '\0';
  }
};

bool parse_json(const char *s, size_t n, Json &out) {
  JsonParser jp{s, s + n, {}};
  if (!jp.value(out, 0)) return false;
  jp.ws();
  return jp.p == jp.end;
}

bool read_file(const std::string &path, std::string &out) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t n;
  out.clear();
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
  const bool ok = !ferror(f);
  fclose(f);
  return ok;
}

// ---------------------------------------------------------------- safetensors
// A file: u64 header length, a JSON header {name: {dtype, shape,
// data_offsets: [begin, end]}, "__metadata__": ...}, then the data.  Mapped
// read-only; tensors are widened to f32 on request (torch's .to(float32):
// exact from f16 and bf16, rounded to nearest even from f64).
struct Mapped {
  void *base = nullptr;
  size_t size = 0;
  ~Mapped() {
    if (base && base != MAP_FAILED) munmap(base, size);
  }
};

struct TensorRef {
  std::shared_ptr<Mapped> file;
  std::string dtype;
  std::vector<int64_t> shape;
  const uint8_t *data = nullptr;
  size_t nbytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {  // subnormal: renormalise
      int sh = 0;
      uint32_t mm = m;
      while (!(mm & 1024)) {
        mm <<= 1;
        ++sh;
      }
      u = s | ((uint32_t)(127 - 15 - sh + 1) << 23) | ((mm & 1023) << 13);
    }
  } else if (e == 31) {
    u = s | 0x7F800000u | (m << 13);
  } else {
    u = s | ((e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

class Checkpoint {
 public:
  int open_dir(const std::string &dir) {
    std::string idx;
    if (read_file(dir + "/model.safetensors.index.json", idx)) {
      Json j;
      if (!parse_json(idx.data(), idx.size(), j)) return fail("bad JSON in model.safetensors.index.json");
      const Json *wm = j.get("weight_map");
      if (!wm || wm->kind != Json::Obj) return fail("model.safetensors.index.json has no weight_map");
      std::vector<std::string> files;
      for (const auto &kv : wm->obj)
        if (kv.second.kind == Json::Str) {
          bool seen = false;
          for (const auto &f : files) seen = seen || f == kv.second.str;
          if (!seen) files.push_back(kv.second.str);
        }
      for (const auto &f : files)
        if (int rc = open_file(dir + "/" + f)) return rc;
      return 0;
    }
    return open_file(dir + "/model.safetensors");
  }

  const TensorRef *find(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }

  // The tensor as a row-major f32 matrix (1-D tensors as one row).
  int to_f32(const TensorRef &t, std::vector<float> &out) const {
    const int64_t n = t.numel();
    out.resize((size_t)n);
    if (t.dtype == "F32") {
      if (t.nbytes != (size_t)n * 4) return fail("tensor size mismatch");
      memcpy(out.data(), t.data, t.nbytes);
    } else if (t.dtype == "BF16" || t.dtype == "F16") {
      if (t.nbytes != (size_t)n * 2) return fail("tensor size mismatch");
      const bool bf = t.dtype == "BF16";
      for (int64_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, t.data + 2 * i, 2);
        out[(size_t)i] = bf ? bf16_to_f32(h) : f16_to_f32(h);
      }
    } else if (t.dtype == "F64") {
      if (t.nbytes != (size_t)n * 8) return fail("tensor size mismatch");
      for (int64_t i = 0; i < n; ++i) {
        double d;
        memcpy(&d, t.data + 8 * i, 8);
        out[(size_t)i] = (float)d;
      }
    } else {
      return fail("unsupported dtype %s", t.dtype.c_str());
    }
    return 0;
  }

 private:
  int open_file(const std::string &path) {
    auto m = std::make_shared<Mapped>();
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) return fail("cannot open %s", path.c_str());
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
      close(fd);
      return fail("%s is not a safetensors file", path.c_str());
    }
    m->size = (size_t)st.st_size;
    m->base = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->base == MAP_FAILED) return fail("cannot map %s", path.c_str());
    const uint8_t *b = static_cast<const uint8_t *>(m->base);
    uint64_t hn;
    memcpy(&hn, b, 8);
    if (hn > m->size - 8) return fail("%s: header length %llu past the file", path.c_str(), (unsigned long long)hn);
    Json h;
    if (!parse_json(reinterpret_cast<const char *>(b + 8), (size_t)hn, h) || h.kind != Json::Obj)
      return fail("%s: bad header", path.c_str());
    const uint8_t *data = b + 8 + hn;
    const size_t avail = m->size - 8 - (size_t)hn;
    for (const auto &kv : h.obj) {
      if (kv.first == "__metadata__") continue;
      const Json *dt = kv.second.get("dtype"), *sh = kv.second.get("shape"), *off = kv.second.get("data_offsets");
      if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
          off->arr.size() != 2)
        return fail("%s: bad entry %s", path.c_str(), kv.first.c_str());
      TensorRef t;
      t.file = m;
      t.dtype = dt->str;
      for (const auto &d : sh->arr) t.shape.push_back((int64_t)d.num);
      const double b0 = off->arr[0].num, b1 = off->arr[1].num;
      if (b0 < 0 || b1 < b0 || b1 > (double)avail) return fail("%s: %s out of the file", path.c_str(), kv.first.c_str());
      t.data = data + (size_t)b0;
      t.nbytes = (size_t)(b1 - b0);
      tensors_[kv.first] = t;
    }
    return 0;
  }

  std::map<std::string, TensorRef> tensors_;
};

// ---------------------------------------------------------------- PGW1 writer
// Tensors appended in call order (convert_hf_to_pgw.py:37-72): a q4 tensor is
// its scales then its packed nibbles; the JSON entry keys in the reference's
// order, serialised as json.dumps(..., separators=(",", ":")) does.
struct Writer {
  std::vector<uint8_t> payload;
  std::string table = "[";

  void put(const void *p, size_t n) {
    const uint8_t *b = static_cast<const uint8_t *>(p);
    payload.insert(payload.end(), b, b + n);
  }
  static std::string jstr(const std::string &s) {  // ensure_ascii JSON string
    std::string o = "\"";
    char buf[8];
    for (unsigned char c : s) {
      if (c == '"') o += "\\\"";
      else if (c == '\\') o += "\\\\";
      else if (c == '\n') o += "\\n";
      else if (c == '\r') o += "\\r";
      else if (c == '\t') o += "\\t";
      else if (c == '\b') o += "\\b";
      else if (c == '\f') o += "\\f";
      else if (c < 0x20 || c >= 0x80) {
        snprintf(buf, sizeof buf, "\\u%04x", c);  // names here are ASCII
        o += buf;
      } else o += (char)c;
    }
    return o + "\"";
  }
  void sep() {
    if (table.size() > 1) table += ",";
  }
  int add_q4(const std::string &name, const float *m, int64_t rows, int64_t cols) {
    if (cols % 32) return fail("%s: %lld columns are not a multiple of 32", name.c_str(), (long long)cols);
    std::vector<uint8_t> packed((size_t)(rows * cols / 2));
    std::vector<float> scales((size_t)(rows * cols / 32));
    if (int rc = pgwc_quant_q4(m, rows, cols, packed.data(), scales.data())) return rc;
    const size_t soff = payload.size();
    put(scales.data(), scales.size() * 4);
    const size_t doff = payload.size();
    put(packed.data(), packed.size());
    sep();
    char buf[512];
    snprintf(buf, sizeof buf,
             "{\"name\":%s,\"shape\":[%lld,%lld],\"kind\":\"q4\",\"storage\":\"q4\",\"group\":32,"
             "\"scaleOffset\":%zu,\"scaleNbytes\":%zu,\"offset\":%zu,\"nbytes\":%zu}",
             jstr(name).c_str(), (long long)rows, (long long)cols, soff, scales.size() * 4, doff, packed.size());
    table += buf;
    return 0;
  }
  void add_f32(const std::string &name, const float *v, const std::vector<int64_t> &shape) {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    const size_t off = payload.size();
    put(v, (size_t)n * 4);
    sep();
    std::string sh = "[";
    for (size_t i = 0; i < shape.size(); ++i) sh += (i ? "," : "") + std::to_string(shape[i]);
    sh += "]";
    char buf[512];
    snprintf(buf, sizeof buf, "{\"name\":%s,\"shape\":%s,\"kind\":\"q4\",\"storage\":\"f32\",\"offset\":%zu,\"nbytes\":%zu}",
             jstr(name).c_str(), sh.c_str(), off, (size_t)n * 4);
    table += buf;
  }
  // Header (convert_hf_to_pgw.py:124-141): "PGW1", dtype 4, arch, eight u32
  // at 8, table offset / length / payload offset at 40, ropeTheta and
  // ropePct as f64 at 56 and 64; the table padded to 16 bytes with zeros.
  int finish(const std::string &path, int arch, const uint32_t (&dims)[8], double rope_theta) {
    table += "]";
    uint8_t h[256] = {0};
    memcpy(h, "PGW1", 4);
    h[4] = 4;
    h[5] = (uint8_t)arch;
    memcpy(h + 8, dims, 32);
    const uint32_t toff = 256, tlen = (uint32_t)table.size();
    const uint32_t pad = (16 - ((toff + tlen) % 16)) % 16, poff = toff + tlen + pad;
    const uint32_t t3[3] = {toff, tlen, poff};
    memcpy(h + 40, t3, 12);
    const double pct = 1.0;
    memcpy(h + 56, &rope_theta, 8);
    memcpy(h + 64, &pct, 8);
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) return fail("cannot write %s", path.c_str());
    const uint8_t zeros[16] = {0};
    bool ok = fwrite(h, 1, 256, f) == 256 && fwrite(table.data(), 1, table.size(), f) == table.size() &&
              fwrite(zeros, 1, pad, f) == pad && fwrite(payload.data(), 1, payload.size(), f) == payload.size();
    ok = (fclose(f) == 0) && ok;
    return ok ? 0 : fail("short write to %s", path.c_str());
  }
};

int load_config(const std::string &dir, Json &cfg) {
  std::string text;
  if (!read_file(dir + "/config.json", text)) return fail("cannot read %s/config.json", dir.c_str());
  if (!parse_json(text.data(), text.size(), cfg) || cfg.kind != Json::Obj) return fail("bad config.json");
  return 0;
}

int cfg_int(const Json &cfg, const char *key, int64_t *out, const char *fallback = nullptr) {
  const Json *v = cfg.get(key);
  if ((!v || v->kind != Json::Num) && fallback) v = cfg.get(fallback);
  if (!v || v->kind != Json::Num) return fail("config.json: no %s", key);
  *out = (int64_t)v->num;
  return 0;
}

// A named matrix [rows][cols] as f32 (torch .to(float32)), checked for shape.
int matrix(const Checkpoint &ck, const std::string &name, int64_t rows, int64_t cols, std::vector<float> &out) {
  const TensorRef *t = ck.find(name);
  if (!t) return fail("missing tensor %s", name.c_str());
  if (t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != cols)
    return fail("%s: shape is not [%lld, %lld]", name.c_str(), (long long)rows, (long long)cols);
  return ck.to_f32(*t, out);
}

int vector_f32(const Checkpoint &ck, const std::string &name, int64_t n, std::vector<float> &out) {
  const TensorRef *t = ck.find(name);
  if (!t) return fail("missing tensor %s", name.c_str());
  if (t->numel() != n) return fail("%s: %lld elements, expected %lld", name.c_str(), (long long)t->numel(), (long long)n);
  return ck.to_f32(*t, out);
}

// The first of the names that the checkpoint holds ("" if none).
std::string first_of(const Checkpoint &ck, std::initializer_list<std::string> names) {
  for (const auto &n : names)
    if (ck.find(n)) return n;
  return "";
}

void transpose(const std::vector<float> &in, int64_t rows, int64_t cols, std::vector<float> &out) {
  out.resize(in.size());
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) out[(size_t)(c * rows + r)] = in[(size_t)(r * cols + c)];
}

}  // namespace

extern "C" const char *pgwc_last_error(void) { return g_err.c_str(); }

extern "C" int pgwc_quant_q4(const float *mat, int64_t rows, int64_t cols, uint8_t *packed, float *scales) {
  if (!mat || !packed || !scales) return fail("null pointer");
  if (rows < 0 || cols <= 0 || cols % 32) return fail("shape %lld x %lld (cols must be a multiple of 32)",
                                                      (long long)rows, (long long)cols);
  const int64_t ng = cols / 32;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t g = 0; g < ng; ++g) {
      const float *x = mat + r * cols + g * 32;
      // np.max propagates NaN; `amax > 0` is then false and sc = 1
      float amax = 0.f;
      for (int k = 0; k < 32; ++k) amax = isnan(x[k]) || isnan(amax) ? NAN : fmaxf(amax, fabsf(x[k]));
      // sc = amax / 8.0 in double (a Python float), stored as f32; NumPy
      // divides the f32 chunk by it in f32 (NEP 50), so by the f32 value
      const float sc = amax > 0.f ? (float)((double)amax / 8.0) : 1.0f;
      scales[r * ng + g] = sc;
      uint8_t q[32];
      for (int k = 0; k < 32; ++k) {
        float v = nearbyintf(x[k] / sc) + 8.0f;  // np.rint: ties to even
        v = v < 0.f ? 0.f : (v > 15.f ? 15.f : v);
        q[k] = isnan(v) ? 0 : (uint8_t)v;  // NaN -> uint8 is 0 on x86
      }
      uint8_t *dst = packed + r * (cols / 2) + g * 16;
      for (int k = 0; k < 16; ++k) dst[k] = (uint8_t)(q[2 * k] | (q[2 * k + 1] << 4));
    }
  return 0;
}

extern "C" int pgwc_convert_llama(const char *hf_dir, const char *out_path, int max_seq) {
  if (!hf_dir || !out_path) return fail("null argument");
  if (max_seq <= 0) return fail("max_seq %d", max_seq);
  Json cfg;
  if (int rc = load_config(hf_dir, cfg)) return rc;
  int64_t L, D, NH, FF, V, NKV;
  if (cfg_int(cfg, "num_hidden_layers", &L) || cfg_int(cfg, "hidden_size", &D) ||
      cfg_int(cfg, "num_attention_heads", &NH) || cfg_int(cfg, "intermediate_size", &FF) ||
      cfg_int(cfg, "vocab_size", &V))
    return 1;
  if (cfg_int(cfg, "num_key_value_heads", &NKV)) NKV = NH;  // getattr(cfg, "num_key_value_heads", n_heads)
  // rope_theta: getattr(cfg, "rope_theta", 10000.0) or 10000.0
  const Json *rt = cfg.get("rope_theta");
  const double theta = rt && rt->kind == Json::Num && rt->num != 0.0 ? rt->num : 10000.0;
  if (D % NH) return fail("d_model %lld not divisible by n_heads %lld", (long long)D, (long long)NH);
  const int64_t hd = D / NH, kvd = NKV * hd;
  Checkpoint ck;
  if (int rc = ck.open_dir(hf_dir)) return rc;
  Writer w;
  std::vector<float> a, b, c;
  // lm_head (tied checkpoints store only the embedding)
  const std::string lm = first_of(ck, {"lm_head.weight", "model.embed_tokens.weight"});
  if (lm.empty()) return fail("missing tensor lm_head.weight / model.embed_tokens.weight");
  if (int rc = matrix(ck, lm, V, D, a)) return rc;
  if (int rc = w.add_q4("lm_head", a.data(), V, D)) return rc;
  for (int64_t i = 0; i < L; ++i) {
    const std::string p = "model.layers." + std::to_string(i) + ".", o = "blocks." + std::to_string(i) + ".";
    if (int rc = vector_f32(ck, p + "input_layernorm.weight", D, a)) return rc;
    w.add_f32(o + "norm1", a.data(), {D});
    // q ‖ k ‖ v rows (np.concatenate axis 0)
    std::vector<float> qkv;
    for (const char *n : {"q_proj", "k_proj", "v_proj"}) {
      const int64_t rows = n[0] == 'q' ? D : kvd;
      if (int rc = matrix(ck, p + "self_attn." + n + ".weight", rows, D, a)) return rc;
      qkv.insert(qkv.end(), a.begin(), a.end());
    }
    if (int rc = w.add_q4(o + "attn.qkv", qkv.data(), D + 2 * kvd, D)) return rc;
    if (int rc = matrix(ck, p + "self_attn.o_proj.weight", D, D, a)) return rc;
    if (int rc = w.add_q4(o + "attn.proj", a.data(), D, D)) return rc;
    if (int rc = vector_f32(ck, p + "post_attention_layernorm.weight", D, a)) return rc;
    w.add_f32(o + "norm2", a.data(), {D});
    if (int rc = matrix(ck, p + "mlp.gate_proj.weight", FF, D, a)) return rc;
    if (int rc = w.add_q4(o + "mlp.w1", a.data(), FF, D)) return rc;
    if (int rc = matrix(ck, p + "mlp.up_proj.weight", FF, D, a)) return rc;
    if (int rc = w.add_q4(o + "mlp.w3", a.data(), FF, D)) return rc;
    if (int rc = matrix(ck, p + "mlp.down_proj.weight", D, FF, a)) return rc;
    if (int rc = w.add_q4(o + "mlp.w2", a.data(), D, FF)) return rc;
  }
  if (int rc = vector_f32(ck, "model.norm.weight", D, a)) return rc;
  w.add_f32("norm_f", a.data(), {D});
  const uint32_t dims[8] = {(uint32_t)V, (uint32_t)L, (uint32_t)D, (uint32_t)NH, (uint32_t)NKV, (uint32_t)FF,
                            (uint32_t)max_seq, 32u};
  return w.finish(out_path, 0, dims, theta);
}

extern "C" int pgwc_convert_gpt2(const char *hf_dir, const char *out_path, int max_seq, const float *scale_factors,
                                 int n_scale) {
  if (!hf_dir || !out_path) return fail("null argument");
  if (max_seq <= 0) return fail("max_seq %d", max_seq);
  Json cfg;
  if (int rc = load_config(hf_dir, cfg)) return rc;
  int64_t L, D, NH, V, NPOS;
  if (cfg_int(cfg, "n_layer", &L) || cfg_int(cfg, "n_embd", &D) || cfg_int(cfg, "n_head", &NH) ||
      cfg_int(cfg, "vocab_size", &V) || cfg_int(cfg, "n_positions", &NPOS))
    return 1;
  const int64_t nctx = NPOS < max_seq ? NPOS : max_seq, FF = 4 * D;
  Checkpoint ck;
  if (int rc = ck.open_dir(hf_dir)) return rc;
  // GPT2LMHeadModel checkpoints name the trunk "transformer." or nothing
  const std::string tp = ck.find("transformer.wte.weight") ? "transformer." : "";
  std::vector<float> sf((size_t)D, 1.0f);
  if (scale_factors) {
    if (n_scale != D) return fail("%d scale factors for n_embd %lld", n_scale, (long long)D);
    sf.assign(scale_factors, scale_factors + D);
  }
  Writer w;
  std::vector<float> a, t, b2;
  w.add_f32("scale_factors", sf.data(), {D});
  // lm_head * scale[None, :] (float32)
  const std::string lm = first_of(ck, {"lm_head.weight", tp + "wte.weight"});
  if (lm.empty()) return fail("missing tensor lm_head.weight / %swte.weight", tp.c_str());
  if (int rc = matrix(ck, lm, V, D, a)) return rc;
  for (int64_t r = 0; r < V; ++r)
    for (int64_t c = 0; c < D; ++c) a[(size_t)(r * D + c)] = a[(size_t)(r * D + c)] * sf[(size_t)c];
  if (int rc = w.add_q4("lm_head", a.data(), V, D)) return rc;
  if (int rc = matrix(ck, tp + "wpe.weight", NPOS, D, a)) return rc;
  w.add_f32("wpe", a.data(), {nctx, D});
  // ln_f: gamma / scale ‖ beta / scale
  if (int rc = vector_f32(ck, tp + "ln_f.weight", D, a)) return rc;
  if (int rc = vector_f32(ck, tp + "ln_f.bias", D, t)) return rc;
  b2.resize((size_t)(2 * D));
  for (int64_t c = 0; c < D; ++c) {
    b2[(size_t)c] = a[(size_t)c] / sf[(size_t)c];
    b2[(size_t)(D + c)] = t[(size_t)c] / sf[(size_t)c];
  }
  w.add_f32("ln_f", b2.data(), {2 * D});
  auto ln = [&](const std::string &p, const std::string &name) -> int {
    if (int rc = vector_f32(ck, p + ".weight", D, a)) return rc;
    if (int rc = vector_f32(ck, p + ".bias", D, t)) return rc;
    b2.assign(a.begin(), a.end());
    b2.insert(b2.end(), t.begin(), t.end());
    w.add_f32(name, b2.data(), {2 * D});
    return 0;
  };
  // HF Conv1D weight [in, out] -> [out, in]
  auto conv = [&](const std::string &p, int64_t in, int64_t out, const std::string &name) -> int {
    if (int rc = matrix(ck, p + ".weight", in, out, a)) return rc;
    transpose(a, in, out, t);
    if (int rc = w.add_q4(name, t.data(), out, in)) return rc;
    if (int rc = vector_f32(ck, p + ".bias", out, a)) return rc;
    w.add_f32(name + "_bias", a.data(), {out});
    return 0;
  };
  for (int64_t i = 0; i < L; ++i) {
    const std::string p = tp + "h." + std::to_string(i) + ".", o = "blocks." + std::to_string(i) + ".";
    if (int rc = ln(p + "ln_1", o + "ln1")) return rc;
    if (int rc = conv(p + "attn.c_attn", D, 3 * D, o + "attn.qkv")) return rc;
    if (int rc = conv(p + "attn.c_proj", D, D, o + "attn.proj")) return rc;
    if (int rc = ln(p + "ln_2", o + "ln2")) return rc;
    if (int rc = conv(p + "mlp.c_fc", D, FF, o + "mlp.fc")) return rc;
    if (int rc = conv(p + "mlp.c_proj", FF, D, o + "mlp.proj")) return rc;
  }
  const uint32_t dims[8] = {(uint32_t)V, (uint32_t)L, (uint32_t)D, (uint32_t)NH, (uint32_t)NH, (uint32_t)FF,
                            (uint32_t)nctx, 1u};
  return w.finish(out_path, 1, dims, 10000.0);
}

#ifdef PGW_CONVERT_MAIN
// pgw_convert llama|gpt2 <hf_dir> <out.bin> [--max-seq N] [--scale-factors f32_file]
int main(int argc, char **argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s llama|gpt2 <hf_dir> <out.bin> [--max-seq N] [--scale-factors file]\n", argv[0]);
    return 2;
  }
  const std::string arch = argv[1];
  int max_seq = arch == "gpt2" ? 1024 : 2048;
  std::vector<float> sf;
  for (int i = 4; i < argc; ++i) {
    if (!strcmp(argv[i], "--max-seq") && i + 1 < argc) {
      max_seq = atoi(argv[++i]);
    } else if (!strcmp(argv[i], "--scale-factors") && i + 1 < argc) {
      std::string raw;
      if (!read_file(argv[++i], raw) || raw.size() % 4) {
        fprintf(stderr, "cannot read scale factors from %s\n", argv[i]);
        return 1;
      }
      sf.resize(raw.size() / 4);
      memcpy(sf.data(), raw.data(), raw.size());
    } else {
      fprintf(stderr, "unknown argument %s\n", argv[i]);
      return 2;
    }
  }
  int rc;
  if (arch == "llama") rc = pgwc_convert_llama(argv[2], argv[3], max_seq);
  else if (arch == "gpt2")
    rc = pgwc_convert_gpt2(argv[2], argv[3], max_seq, sf.empty() ? nullptr : sf.data(), (int)sf.size());
  else {
    fprintf(stderr, "unknown arch %s\n", arch.c_str());
    return 2;
  }
  if (rc) {
    fprintf(stderr, "pgw_convert: %s\n", pgwc_last_error());
    return 1;
  }
  return 0;
}
#endif
