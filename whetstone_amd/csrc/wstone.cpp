// The .wstone container: header parse and validation, payload verification,
// and the model loader with load-time projection fusion.
//
// reference: crates/whetstone-quant/src/format.rs (container, 1-547),
// docs/FORMAT.md (layout, integrity, validation on load),
// crates/whetstone-core/src/model.rs:454-638,779-967 (loader),
// crates/whetstone-core/src/config.rs:26-262 (config.json fields, validate).
//
// The file is treated as hostile until validated: every declared range is
// checked against the file length (with overflow checks) and for 256-byte
// alignment before anything indexes with it, and a malformed file is an error,
// never an out-of-bounds read. Loading is an mmap plus device copies: q|k|v and
// gate|up are fused by copying each part straight to its row offset in the
// fused device matrix (the int4-hier layout is row-major with a fixed stride,
// so a row append is a byte append of qw, si and sb alike).
#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <utility>
#include <vector>

#include "engine_internal.hpp"

using namespace wse;

namespace {

constexpr uint64_t kPrefix = 32;  // magic, version, flags, header_len, header_hash
constexpr uint64_t kAlign = 256;
constexpr uint32_t kVersion = 1;
constexpr const char *kRescoreSuffix = ".rescore";  // format.rs:218
constexpr int kHeadRescoreK = 64;                    // model.rs:814

// format.rs:225-232: FNV-1a's offset basis with the multiplier 0x1000000001B3
// (one hex digit longer than the FNV prime; kept, as the reference keeps it,
// because every existing file carries hashes made with it).
uint64_t fnv(const uint8_t *p, uint64_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (uint64_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x1000000001B3ull;
  }
  return h;
}

wst_status_t fail(wst_status_t st, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return st;
}
#define FMT_ERR(...) fail(WST_ERR_INVALID_ARG, __VA_ARGS__)

// ------------------------------------------------------------------- JSON
//
// RFC 8259 values. Numbers keep their source text, so an integer field is read
// exactly (u64) and a float field as a double.
struct JVal {
  enum Type { NUL, BOOL, NUM, STR, ARR, OBJ } t = NUL;
  bool b = false;
  std::string s;  // string value, or the number's text
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;
  const JVal *get(const char *key) const {
    if (t != OBJ) return nullptr;
    for (const auto &kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *end;
  int depth = 0;
  std::string err;

  bool error(const char *what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(end - p) < n || memcmp(p, w, n)) return error("invalid literal");
    p += n;
    return true;
  }
  static int hexv(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  bool hex4(uint32_t &u) {
    if (end - p < 4) return error("truncated \\u escape");
    u = 0;
    for (int i = 0; i < 4; ++i) {
      const int v = hexv(p[i]);
      if (v < 0) return error("bad \\u escape");
      u = u * 16 + (uint32_t)v;
    }
    p += 4;
    return true;
  }
  static void utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool string(std::string &out) {
    if (p >= end || *p != '"') return error("expected a string");
    ++p;
    while (true) {
      if (p >= end) return error("unterminated string");
      const unsigned char ch = (unsigned char)*p++;
      if (ch == '"') return true;
      if (ch < 0x20) return error("control character in string");
      if (ch != '\\') {
        out += (char)ch;
        continue;
      }
      if (p >= end) return error("unterminated escape");
      const char e = *p++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t u;
          if (!hex4(u)) return false;
          if (u >= 0xD800 && u < 0xDC00) {  // high surrogate: a low one must follow
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return error("lone surrogate");
            p += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return error("lone surrogate");
            u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
          } else if (u >= 0xDC00 && u < 0xE000) {
            return error("lone surrogate");
          }
          utf8(out, u);
          break;
        }
        default:
          return error("bad escape");
      }
    }
  }
  bool number(std::string &out) {
    const char *s0 = p;
    if (p < end && *p == '-') ++p;
    if (p >= end) return error("truncated number");
    if (*p == '0') {
      ++p;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') ++p;
    } else {
      return error("bad number");
    }
    if (p < end && *p == '.') {
      ++p;
      if (p >= end || *p < '0' || *p > '9') return error("bad number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || *p < '0' || *p > '9') return error("bad number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    out.assign(s0, p);
    return true;
  }
  bool value(JVal &v) {
    if (++depth > 64) return error("nesting too deep");
    ws();
    if (p >= end) return error("unexpected end of input");
    bool ok = true;
    switch (*p) {
      case '{': {
        v.t = JVal::OBJ;
        ++p;
        ws();
        if (p < end && *p == '}') {
          ++p;
          break;
        }
        while (ok) {
          ws();
          std::pair<std::string, JVal> kv;
          ok = string(kv.first);
          if (!ok) break;
          ws();
          if (p >= end || *p != ':') {
            ok = error("expected ':'");
            break;
          }
          ++p;
          ok = value(kv.second);
          if (!ok) break;
          v.o.push_back(std::move(kv));
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == '}') {
            ++p;
            break;
          }
          ok = error("expected ',' or '}'");
        }
        break;
      }
      case '[': {
        v.t = JVal::ARR;
        ++p;
        ws();
        if (p < end && *p == ']') {
          ++p;
          break;
        }
        while (ok) {
          JVal e;
          ok = value(e);
          if (!ok) break;
          v.a.push_back(std::move(e));
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == ']') {
            ++p;
            break;
          }
          ok = error("expected ',' or ']'");
        }
        break;
      }
      case '"':
        v.t = JVal::STR;
        ok = string(v.s);
        break;
      case 't':
        v.t = JVal::BOOL;
        v.b = true;
        ok = lit("true");
        break;
      case 'f':
        v.t = JVal::BOOL;
        ok = lit("false");
        break;
      case 'n':
        v.t = JVal::NUL;
        ok = lit("null");
        break;
      default:
        v.t = JVal::NUM;
        ok = number(v.s);
    }
    --depth;
    return ok;
  }
};

bool json_parse(const char *p, size_t n, JVal &out, std::string &err) {
  JParser ps{p, p + n};
  if (!ps.value(out)) {
    err = ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    err = "trailing characters after the header";
    return false;
  }
  return true;
}

// A JSON integer that fits u64 (serde's usize/u64: no sign, fraction or exponent).
bool as_u64(const JVal &v, uint64_t &out) {
  if (v.t != JVal::NUM || v.s.empty()) return false;
  uint64_t x = 0;
  for (char c : v.s) {
    if (c < '0' || c > '9') return false;
    const uint64_t d = (uint64_t)(c - '0');
    if (x > (UINT64_MAX - d) / 10) return false;
    x = x * 10 + d;
  }
  out = x;
  return true;
}

bool as_f64(const JVal &v, double &out) {
  if (v.t != JVal::NUM) return false;
  out = strtod(v.s.c_str(), nullptr);
  return true;
}

// ------------------------------------------------------------------ header

struct Blob {
  uint64_t offset = 0, len = 0, hash = 0;
};

enum Kind { K_FP16, K_FP32, K_INT4_G128, K_INT4_HIER };

struct Tensor {
  std::string name;
  Kind kind = K_FP16;
  std::vector<uint64_t> shape;
  std::vector<std::pair<std::string, Blob>> blobs;
  const Blob *blob(const char *n) const {
    for (const auto &b : blobs)
      if (b.first == n) return &b.second;
    return nullptr;
  }
  uint64_t numel() const {
    uint64_t n = 1;
    for (uint64_t d : shape) n *= d;
    return n;
  }
};

struct Header {
  JVal root;
  const JVal *model_config = nullptr;
  std::vector<Tensor> tensors;
  std::vector<std::pair<std::string, Blob>> extras;
  const Tensor *tensor(const std::string &n) const {
    for (const auto &t : tensors)
      if (t.name == n) return &t;
    return nullptr;
  }
};

uint64_t le64(const uint8_t *p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}

wst_status_t parse_blob(const JVal &v, const std::string &what, Blob &b) {
  const JVal *o = v.get("offset"), *l = v.get("len"), *h = v.get("hash");
  if (v.t != JVal::OBJ || !o || !l || !h || !as_u64(*o, b.offset) || !as_u64(*l, b.len) ||
      !as_u64(*h, b.hash))
    return FMT_ERR("malformed header JSON: %s: a blob needs integer offset, len and hash",
                   what.c_str());
  return WST_OK;
}

// format.rs:427-516.
wst_status_t parse_header(const uint8_t *bytes, uint64_t file_len, Header &h) {
  if (file_len < kPrefix) return FMT_ERR("file is too short to be a .wstone");
  if (memcmp(bytes, "WHETSTON", 8)) return FMT_ERR("bad magic; not a .wstone file");
  const uint32_t version = (uint32_t)bytes[8] | (uint32_t)bytes[9] << 8 |
                           (uint32_t)bytes[10] << 16 | (uint32_t)bytes[11] << 24;
  if (version != kVersion)
    return FMT_ERR("file is format version %u, this build understands %u", version, kVersion);
  // bytes 12..16: flags, reserved for additions a reader may ignore
  const uint64_t header_len = le64(bytes + 16), want_hash = le64(bytes + 24);
  if (header_len > UINT64_MAX - kPrefix) return FMT_ERR("header length overflows");
  if (kPrefix + header_len > file_len)
    return FMT_ERR("header claims %llu bytes but the file holds %llu",
                   (unsigned long long)header_len, (unsigned long long)file_len);
  const uint8_t *json = bytes + kPrefix;
  if (fnv(json, header_len) != want_hash)
    return FMT_ERR("header checksum mismatch; file is corrupt");
  std::string err;
  if (!json_parse((const char *)json, (size_t)header_len, h.root, err))
    return FMT_ERR("malformed header JSON: %s", err.c_str());
  const JVal &r = h.root;
  if (r.t != JVal::OBJ) return FMT_ERR("malformed header JSON: not an object");
  // The Header struct's fields (format.rs:139-161); unknown fields are ignored.
  const JVal *fmt = r.get("format"), *ver = r.get("version"), *prod = r.get("producer");
  const JVal *quant = r.get("quant"), *tensors = r.get("tensors"), *extras = r.get("extras");
  h.model_config = r.get("model_config");
  uint64_t v64 = 0;
  if (!fmt || fmt->t != JVal::STR || !ver || !as_u64(*ver, v64) || v64 > UINT32_MAX || !prod ||
      prod->t != JVal::STR || !h.model_config || !quant || quant->t != JVal::OBJ || !tensors ||
      tensors->t != JVal::ARR)
    return FMT_ERR("malformed header JSON: format, version, producer, model_config, quant and "
                   "tensors are required");
  for (const auto &kv : quant->o)
    if (kv.second.t != JVal::STR) return FMT_ERR("malformed header JSON: quant values are strings");
  if (extras && extras->t != JVal::NUL) {  // #[serde(default)]: absent in older files
    if (extras->t != JVal::OBJ) return FMT_ERR("malformed header JSON: extras is not an object");
    for (const auto &kv : extras->o) {
      Blob b;
      TRY(parse_blob(kv.second, "extra " + kv.first, b));
      if (b.offset > UINT64_MAX - b.len) return FMT_ERR("extra \"%s\": range overflows", kv.first.c_str());
      if (b.offset + b.len > file_len)
        return FMT_ERR("extra \"%s\" ends at %llu but the file is %llu bytes", kv.first.c_str(),
                       (unsigned long long)(b.offset + b.len), (unsigned long long)file_len);
      h.extras.emplace_back(kv.first, b);
    }
  }
  for (const JVal &tv : tensors->a) {
    Tensor t;
    const JVal *nm = tv.get("name"), *kd = tv.get("kind"), *sh = tv.get("shape"),
               *bl = tv.get("blobs");
    if (!nm || nm->t != JVal::STR || !kd || kd->t != JVal::STR || !sh || sh->t != JVal::ARR ||
        !bl || bl->t != JVal::OBJ)
      return FMT_ERR("malformed header JSON: a tensor needs name, kind, shape and blobs");
    t.name = nm->s;
    if (kd->s == "fp16") t.kind = K_FP16;
    else if (kd->s == "fp32") t.kind = K_FP32;
    else if (kd->s == "int4_g128") t.kind = K_INT4_G128;
    else if (kd->s == "int4_hier_g32") t.kind = K_INT4_HIER;
    else return FMT_ERR("malformed header JSON: %s: unknown kind \"%s\"", t.name.c_str(), kd->s.c_str());
    for (const JVal &d : sh->a) {
      uint64_t x;
      if (!as_u64(d, x)) return FMT_ERR("malformed header JSON: %s: bad shape", t.name.c_str());
      t.shape.push_back(x);
    }
    for (const auto &kv : bl->o) {
      Blob b;
      TRY(parse_blob(kv.second, t.name + "/" + kv.first, b));
      if (b.offset > UINT64_MAX - b.len)
        return FMT_ERR("%s/%s: range overflows", t.name.c_str(), kv.first.c_str());
      if (b.offset + b.len > file_len)
        return FMT_ERR("%s/%s ends at %llu but the file is %llu bytes (truncated or corrupt)",
                       t.name.c_str(), kv.first.c_str(), (unsigned long long)(b.offset + b.len),
                       (unsigned long long)file_len);
      if (b.offset % kAlign)
        return FMT_ERR("%s/%s is at %llu which is not %llu-byte aligned", t.name.c_str(),
                       kv.first.c_str(), (unsigned long long)b.offset,
                       (unsigned long long)kAlign);
      t.blobs.emplace_back(kv.first, b);
    }
    static const char *const need_g128[] = {"qw", "sz", nullptr};
    static const char *const need_hier[] = {"qw", "si", "sb", nullptr};
    static const char *const need_dense[] = {"data", nullptr};
    const char *const *need = t.kind == K_INT4_G128   ? need_g128
                              : t.kind == K_INT4_HIER ? need_hier
                                                      : need_dense;
    for (; *need; ++need)
      if (!t.blob(*need))
        return FMT_ERR("%s: kind %s requires a \"%s\" blob", t.name.c_str(), kd->s.c_str(), *need);
    h.tensors.push_back(std::move(t));
  }
  return WST_OK;
}

// format.rs:518-547.
wst_status_t verify_payloads(const Header &h, const uint8_t *bytes, uint64_t file_len) {
  for (const auto &e : h.extras) {
    const Blob &b = e.second;
    if (b.offset + b.len > file_len) return FMT_ERR("extra \"%s\": range past end of file", e.first.c_str());
    if (fnv(bytes + b.offset, b.len) != b.hash)
      return FMT_ERR("extra \"%s\": checksum mismatch", e.first.c_str());
  }
  for (const Tensor &t : h.tensors)
    for (const auto &e : t.blobs) {
      const Blob &b = e.second;
      if (b.offset + b.len > file_len)
        return FMT_ERR("%s/%s: range past end of file", t.name.c_str(), e.first.c_str());
      if (fnv(bytes + b.offset, b.len) != b.hash)
        return FMT_ERR("%s/%s: checksum mismatch; the file is corrupt", t.name.c_str(),
                       e.first.c_str());
    }
  return WST_OK;
}

// A read-only mapping of the whole file.
struct Mapped {
  const uint8_t *p = nullptr;
  uint64_t n = 0;
  ~Mapped() {
    if (p && n) munmap((void *)p, (size_t)n);
  }
  wst_status_t open(const char *path) {
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return FMT_ERR("could not open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
      ::close(fd);
      return FMT_ERR("could not stat %s: %s", path, strerror(errno));
    }
    n = (uint64_t)st.st_size;
    if (n < kPrefix) {
      ::close(fd);
      n = 0;
      return FMT_ERR("%s: file is too short to be a .wstone", path);
    }
    void *m = mmap(nullptr, (size_t)n, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
      n = 0;
      return FMT_ERR("could not mmap %s: %s", path, strerror(errno));
    }
    p = (const uint8_t *)m;
    return WST_OK;
  }
};

// ------------------------------------------------------------------ config
//
// config.rs:26-262: the fields the decode path reads, their defaults, and
// validate() (including the architecture whitelist). Refusals name the field.

wst_status_t cfg_err(const char *fmt, const char *what) {
  char buf[400];
  snprintf(buf, sizeof(buf), fmt, what);
  return fail(WST_ERR_INVALID_ARG, "embedded config is unusable: %s", buf);
}

wst_status_t cfg_u64(const JVal &mc, const char *key, bool required, uint64_t dflt,
                     uint64_t &out, bool *present = nullptr) {
  const JVal *v = mc.get(key);
  if (present) *present = v && v->t != JVal::NUL;
  if (!v || (v->t == JVal::NUL && !required)) {
    if (required) return cfg_err("missing field `%s`", key);
    out = dflt;
    return WST_OK;
  }
  if (!as_u64(*v, out)) return cfg_err("field `%s` is not a non-negative integer", key);
  return WST_OK;
}

wst_status_t cfg_f64(const JVal &mc, const char *key, double dflt, double &out,
                     bool *present = nullptr) {
  const JVal *v = mc.get(key);
  if (present) *present = v && v->t != JVal::NUL;
  if (!v || v->t == JVal::NUL) {
    out = dflt;
    return WST_OK;
  }
  if (!as_f64(*v, out)) return cfg_err("field `%s` is not a number", key);
  return WST_OK;
}

wst_status_t cfg_str(const JVal &mc, const char *key, const char *dflt, std::string &out) {
  const JVal *v = mc.get(key);
  if (!v || v->t == JVal::NUL) {
    out = dflt;
    return WST_OK;
  }
  if (v->t != JVal::STR) return cfg_err("field `%s` is not a string", key);
  out = v->s;
  return WST_OK;
}

wst_status_t parse_config(const JVal *mcp, wse_config_t &c) {
  if (!mcp || mcp->t != JVal::OBJ) return cfg_err("%s", "model_config is not an object");
  const JVal &mc = *mcp;
  uint64_t hidden, layers, heads, kv, inter, vocab, head_dim;
  bool kv_given = false, hd_given = false;
  TRY(cfg_u64(mc, "hidden_size", true, 0, hidden));
  TRY(cfg_u64(mc, "num_hidden_layers", true, 0, layers));
  TRY(cfg_u64(mc, "num_attention_heads", true, 0, heads));
  TRY(cfg_u64(mc, "num_key_value_heads", false, 0, kv, &kv_given));
  TRY(cfg_u64(mc, "intermediate_size", true, 0, inter));
  TRY(cfg_u64(mc, "vocab_size", true, 0, vocab));
  TRY(cfg_u64(mc, "head_dim", false, 0, head_dim, &hd_given));
  double eps, theta;
  TRY(cfg_f64(mc, "rms_norm_eps", 1e-6, eps));
  TRY(cfg_f64(mc, "rope_theta", 10000.0, theta));
  std::string model_type, act;
  TRY(cfg_str(mc, "model_type", "", model_type));
  TRY(cfg_str(mc, "hidden_act", "silu", act));
  bool tied = false;
  if (const JVal *t = mc.get("tie_word_embeddings")) {
    if (t->t == JVal::BOOL) tied = t->b;
    else if (t->t != JVal::NUL) return cfg_err("field `%s` is not a bool", "tie_word_embeddings");
  }
  // validate() (config.rs:206-247)
  if (hidden == 0 || heads == 0)
    return cfg_err("%s", "hidden_size and num_attention_heads must be non-zero");
  if (!hd_given && hidden % heads)
    return cfg_err("%s", "hidden_size is not divisible by num_attention_heads and no head_dim "
                         "is given");
  if (!kv_given) kv = heads;  // MHA when unspecified
  if (kv == 0 || heads % kv) return cfg_err("%s", "num_attention_heads must be a multiple of "
                                                  "num_key_value_heads");
  if (act != "silu" && act != "swish")
    return cfg_err("unsupported activation \"%s\"; the block is SwiGLU with SiLU", act.c_str());
  static const char *const families[] = {"", "qwen2", "qwen3", "llama", "mistral",
                                         "smollm", "smollm2", "olmo2", nullptr};
  bool known = false;
  for (const char *const *f = families; *f; ++f) known = known || model_type == *f;
  if (!known)
    return cfg_err("unsupported model_type \"%s\": the block executed is pre-norm RMSNorm, "
                   "RoPE, grouped-query attention and SwiGLU (qwen2, qwen3, llama, mistral and "
                   "their distillations); mixture-of-experts and MLA families are refused",
                   model_type.c_str());
  // Mixture-of-experts configs parse as dense ones; the expert path is not
  // part of this build, so their presence is refused rather than ignored.
  for (const char *k : {"num_experts", "num_local_experts"}) {
    const JVal *v = mc.get(k);
    uint64_t ne = 0;
    if (v && v->t != JVal::NUL && as_u64(*v, ne) && ne > 0)
      return cfg_err("%s: mixture-of-experts models are not part of this build", k);
  }
  c.rope_llama3 = 0;
  c.rope_factor = 8.0;
  c.rope_low_freq = 1.0;
  c.rope_high_freq = 4.0;
  c.rope_orig_max = 8192;
  if (const JVal *rs = mc.get("rope_scaling")) {
    if (rs->t == JVal::OBJ) {
      std::string type;
      const JVal *tv = rs->get("rope_type");
      if (!tv || tv->t == JVal::NUL) tv = rs->get("type");  // older configs (serde alias)
      if (tv && tv->t == JVal::STR) type = tv->s;
      else if (tv && tv->t != JVal::NUL) return cfg_err("%s", "rope_scaling.rope_type is not a string");
      if (type != "" && type != "default" && type != "llama3")
        return cfg_err("rope_scaling type \"%s\" is not implemented (the llama3 schedule and "
                       "unscaled RoPE are)", type.c_str());
      if (type == "llama3") {
        uint64_t orig;
        c.rope_llama3 = 1;
        TRY(cfg_f64(*rs, "factor", 8.0, c.rope_factor));
        TRY(cfg_f64(*rs, "low_freq_factor", 1.0, c.rope_low_freq));
        TRY(cfg_f64(*rs, "high_freq_factor", 4.0, c.rope_high_freq));
        TRY(cfg_u64(*rs, "original_max_position_embeddings", false, 8192, orig));
        if (orig > INT32_MAX) return cfg_err("%s", "original_max_position_embeddings too large");
        c.rope_orig_max = (int32_t)orig;
      }
    } else if (rs->t != JVal::NUL) {
      return cfg_err("%s", "rope_scaling is not an object");
    }
  }
  const uint64_t hd = hd_given ? head_dim : hidden / heads;
  const uint64_t lim = INT32_MAX;
  if (hidden > lim || layers > lim || heads > lim || kv > lim || inter > lim || vocab > lim ||
      hd > lim || heads * hd > lim)
    return cfg_err("%s", "a dimension exceeds 2^31");
  c.n_layers = (int32_t)layers;
  c.hidden = (int32_t)hidden;
  c.n_q = (int32_t)heads;
  c.n_kv = (int32_t)kv;
  c.head_dim = (int32_t)hd;
  c.inter = (int32_t)inter;
  c.vocab = (int32_t)vocab;
  c.tied = tied ? 1 : 0;
  c.eps = (float)eps;                       // rms_norm_eps: f32
  c.rope_theta = (double)(float)theta;      // rope_theta: f32, widened for the table
  return WST_OK;
}

// ------------------------------------------------------------------ loading

struct Loader {
  const uint8_t *base;
  const Header &h;
  Arena &a;

  const Tensor *need(const std::string &name) {
    const Tensor *t = h.tensor(name);
    if (!t) fail(WST_ERR_INVALID_ARG, "missing tensor %s", name.c_str());
    return t;
  }

  // A dense f16 vector of n elements (norm gains, biases, QK-norm gains).
  wst_status_t vec(const Tensor &t, uint64_t n, void **out) {
    const Blob *d = t.blob("data");
    if (t.kind != K_FP16)
      return FMT_ERR("%s: stored as a quantised kind; vectors are f16", t.name.c_str());
    if (t.numel() != n || d->len != 2 * n)
      return fail(WST_ERR_SHAPE, "%s: %llu elements, expected %llu", t.name.c_str(),
                  (unsigned long long)t.numel(), (unsigned long long)n);
    TRY(a.alloc(out, (size_t)(2 * n), false));
    return wst_memcpy_h2d(*out, base + d->offset, (size_t)d->len);
  }

  // Matrices appended along the output dimension into one int4-hier matrix
  // (model.rs:860-930): all share in_f and the kind; no repacking.
  wst_status_t fused(const std::vector<std::string> &names, const std::vector<int64_t> &rows,
                     int64_t in_f, Mat &m) {
    int64_t total = 0;
    std::vector<const Tensor *> ts;
    for (size_t i = 0; i < names.size(); ++i) {
      const Tensor *t = need(names[i]);
      if (!t) return WST_ERR_INVALID_ARG;
      if (t->kind != K_INT4_HIER)
        return FMT_ERR("%s: this build runs int4_hier_g32 projections; re-convert with the "
                       "int4-hier body", t->name.c_str());
      if (t->shape.size() != 2 || (int64_t)t->shape[0] != rows[i] || (int64_t)t->shape[1] != in_f)
        return fail(WST_ERR_SHAPE, "%s: shape does not match the config (expected [%lld, %lld])",
                    t->name.c_str(), (long long)rows[i], (long long)in_f);
      const uint64_t r = t->shape[0], c = t->shape[1];
      if (t->blob("qw")->len != r * c / 2 || t->blob("si")->len != r * c / 32 ||
          t->blob("sb")->len != r * 4)
        return FMT_ERR("%s: blob sizes do not match its shape", t->name.c_str());
      ts.push_back(t);
      total += rows[i];
    }
    TRY(alloc_mat(a, m, in_f, total));
    int64_t r0 = 0;
    for (const Tensor *t : ts) {
      const Blob *qw = t->blob("qw"), *si = t->blob("si"), *sb = t->blob("sb");
      TRY(wst_memcpy_h2d((char *)m.qw + (size_t)(r0 * in_f / 2), base + qw->offset, qw->len));
      TRY(wst_memcpy_h2d((char *)m.si + (size_t)(r0 * in_f / 32), base + si->offset, si->len));
      TRY(wst_memcpy_h2d((char *)m.sb + (size_t)(r0 * 4), base + sb->offset, sb->len));
      r0 += (int64_t)t->shape[0];
    }
    return WST_OK;
  }

  // The embedding or the output projection: int4-hier or dense f16.
  wst_status_t table(const std::string &name, int64_t rows, int64_t cols, Mat &m) {
    const Tensor *t = need(name);
    if (!t) return WST_ERR_INVALID_ARG;
    if (t->kind == K_INT4_HIER) return fused({name}, {rows}, cols, m);
    if (t->kind != K_FP16)
      return FMT_ERR("%s: stored as %s; the embedding and head are int4_hier_g32 or fp16 here",
                     name.c_str(), t->kind == K_FP32 ? "fp32" : "int4_g128");
    if (t->shape.size() != 2 || (int64_t)t->shape[0] != rows || (int64_t)t->shape[1] != cols)
      return fail(WST_ERR_SHAPE, "%s: shape does not match the config (expected [%lld, %lld])",
                  name.c_str(), (long long)rows, (long long)cols);
    const Blob *d = t->blob("data");
    if (d->len != (uint64_t)rows * (uint64_t)cols * 2)
      return FMT_ERR("%s: blob size does not match its shape", name.c_str());
    m.in_f = cols;
    m.out_f = rows;
    TRY(a.alloc(&m.w16, (size_t)d->len, false));
    return wst_memcpy_h2d(m.w16, base + d->offset, (size_t)d->len);
  }
};

wst_status_t load_model(const uint8_t *bytes, const Header &h, int32_t rescore_k, wse_model *m) {
  wse_config_t &c = m->c;
  TRY(parse_config(h.model_config, c));
  const int64_t H = c.hidden, hd = c.head_dim, I = c.inter, V = c.vocab;
  const int64_t nq = (int64_t)c.n_q * hd, nk = (int64_t)c.n_kv * hd;
  // Presence decides biases and QK-norm (model.rs:779-806, fuse_biases), as
  // the reference decides; they are then required of every layer alike.
  const std::string p0 = "model.layers.0.";
  c.qkv_bias = (h.tensor(p0 + "self_attn.q_proj.bias") || h.tensor(p0 + "self_attn.k_proj.bias") ||
                h.tensor(p0 + "self_attn.v_proj.bias"))
                   ? 1
                   : 0;
  c.qk_norm = h.tensor(p0 + "self_attn.q_norm.weight") ? 1 : 0;
  const std::string head_name = c.tied ? "model.embed_tokens.weight" : "lm_head.weight";
  const Tensor *head_t = h.tensor(head_name);
  const Tensor *resc = h.tensor(head_name + kRescoreSuffix);
  const bool head_quant = head_t && head_t->kind == K_INT4_HIER;
  c.rescore_k = (resc && head_quant && rescore_k != 0) ? (rescore_k < 0 ? kHeadRescoreK : rescore_k) : 0;
  TRY(check_config(&c));

  Loader ld{bytes, h, m->arena};
  TRY(ld.table("model.embed_tokens.weight", V, H, m->embed));
  if (!c.tied) TRY(ld.table("lm_head.weight", V, H, m->lm_head));
  {
    const Tensor *t = ld.need("model.norm.weight");
    if (!t) return WST_ERR_INVALID_ARG;
    TRY(ld.vec(*t, (uint64_t)H, &m->final_norm));
  }
  if (c.rescore_k > 0) {
    if (resc->kind != K_FP16 || resc->shape.size() != 2 || (int64_t)resc->shape[0] != V ||
        (int64_t)resc->shape[1] != H || resc->blob("data")->len != (uint64_t)(V * H * 2))
      return fail(WST_ERR_SHAPE, "%s%s: expected an f16 [vocab, hidden] head copy",
                  head_name.c_str(), kRescoreSuffix);
    TRY(m->arena.alloc(&m->rescore, (size_t)(V * H * 2), false));
    TRY(wst_memcpy_h2d(m->rescore, bytes + resc->blob("data")->offset, (size_t)(V * H * 2)));
  }
  m->layers.resize((size_t)c.n_layers);
  for (int l = 0; l < c.n_layers; ++l) {
    Layer &L = m->layers[(size_t)l];
    const std::string p = "model.layers." + std::to_string(l) + ".";
    TRY(ld.fused({p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight",
                  p + "self_attn.v_proj.weight"},
                 {nq, nk, nk}, H, L.qkv));
    TRY(ld.fused({p + "self_attn.o_proj.weight"}, {H}, nq, L.o));
    TRY(ld.fused({p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"}, {I, I}, H, L.gate_up));
    TRY(ld.fused({p + "mlp.down_proj.weight"}, {H}, I, L.down));
    for (auto &nv : {std::make_pair(std::string("input_layernorm.weight"), &L.in_norm),
                     std::make_pair(std::string("post_attention_layernorm.weight"), &L.post_norm)}) {
      const Tensor *t = ld.need(p + nv.first);
      if (!t) return WST_ERR_INVALID_ARG;
      TRY(ld.vec(*t, (uint64_t)H, nv.second));
    }
    // q|k|v biases, zero-filled where one is absent (model.rs fuse_biases).
    const Tensor *bq = h.tensor(p + "self_attn.q_proj.bias"),
                 *bk = h.tensor(p + "self_attn.k_proj.bias"),
                 *bv = h.tensor(p + "self_attn.v_proj.bias");
    if ((bq || bk || bv) != (c.qkv_bias != 0))
      return FMT_ERR("%s: q/k/v biases present in some layers and not others", p.c_str());
    if (c.qkv_bias) {
      TRY(m->arena.alloc(&L.qkv_bias, (size_t)(nq + 2 * nk) * 2, true));
      const Tensor *parts[3] = {bq, bk, bv};
      const int64_t width[3] = {nq, nk, nk};
      int64_t off = 0;
      for (int i = 0; i < 3; ++i) {
        if (parts[i]) {
          const Tensor &t = *parts[i];
          const Blob *d = t.blob("data");
          if (t.kind != K_FP16 || t.numel() != (uint64_t)width[i] || d->len != (uint64_t)width[i] * 2)
            return fail(WST_ERR_SHAPE, "%s: %llu elements, expected %lld", t.name.c_str(),
                        (unsigned long long)t.numel(), (long long)width[i]);
          TRY(wst_memcpy_h2d((char *)L.qkv_bias + off * 2, bytes + d->offset, (size_t)d->len));
        }
        off += width[i];
      }
    }
    // QK-norm: both gains or neither (model.rs:779-806).
    const Tensor *qn = h.tensor(p + "self_attn.q_norm.weight"),
                 *kn = h.tensor(p + "self_attn.k_norm.weight");
    if ((qn != nullptr) != (kn != nullptr))
      return FMT_ERR("%shas %s but not the other. QK-norm needs both gains", p.c_str(),
                     qn ? "q_norm" : "k_norm");
    if ((qn != nullptr) != (c.qk_norm != 0))
      return FMT_ERR("%s: QK-norm gains present in some layers and not others", p.c_str());
    if (qn) {
      TRY(ld.vec(*qn, (uint64_t)hd, &L.q_norm));
      TRY(ld.vec(*kn, (uint64_t)hd, &L.k_norm));
    }
  }
  return wst_device_synchronize();
}

}  // namespace

extern "C" {

uint64_t wse_fnv1a(const void *bytes, size_t n) {
  return bytes || !n ? fnv((const uint8_t *)bytes, n) : 0;
}

wst_status_t wse_wstone_check(const char *path, int32_t verify, int32_t *n_tensors) {
  if (!path) return FMT_ERR("null path");
  Mapped f;
  TRY(f.open(path));
  Header h;
  TRY(parse_header(f.p, f.n, h));
  if (verify) TRY(verify_payloads(h, f.p, f.n));
  if (n_tensors) *n_tensors = (int32_t)h.tensors.size();
  return WST_OK;
}

wst_status_t wse_wstone_config(const char *path, wse_config_t *out) {
  if (!path || !out) return FMT_ERR("null argument");
  Mapped f;
  TRY(f.open(path));
  Header h;
  TRY(parse_header(f.p, f.n, h));
  wse_config_t c{};
  TRY(parse_config(h.model_config, c));
  *out = c;
  return WST_OK;
}

wst_status_t wse_config_from_json(const char *json, wse_config_t *out) {
  if (!json || !out) return FMT_ERR("null argument");
  JVal v;
  std::string err;
  if (!json_parse(json, strlen(json), v, err)) return FMT_ERR("could not parse config.json: %s", err.c_str());
  wse_config_t c{};
  TRY(parse_config(&v, c));
  *out = c;
  return WST_OK;
}

wst_status_t wse_model_load_wstone(const char *path, int32_t rescore_k, wse_model_t **out) {
  if (!path || !out) return FMT_ERR("null argument");
  *out = nullptr;
  Mapped f;
  TRY(f.open(path));
  Header h;
  {
    const wst_status_t st = parse_header(f.p, f.n, h);
    if (st != WST_OK) {
      std::string msg = g_msg;
      return fail(st, "%s: %s", path, msg.c_str());
    }
  }
  wse_model *m = new wse_model();
  const wst_status_t st = load_model(f.p, h, rescore_k, m);
  if (st != WST_OK) {
    wse_model_free(m);
    return st;
  }
  *out = m;
  return WST_OK;
}

wst_status_t wse_model_config(const wse_model_t *m, wse_config_t *out) {
  if (!m || !out) return WST_ERR_INVALID_ARG;
  *out = m->c;
  return WST_OK;
}

}  // extern "C"
