// On-disk format of the quantized weights: MLX-style safetensors archives.
//
// Reference:
//   crates/cider-press-models/src/safetensors_io.rs:43-134  read_quantized_weight
//   crates/cider-press-models/src/safetensors_io.rs:25-32   read_dense_tensor
//   crates/cider-press-models/src/safetensors_io.rs:136-146 map_dtype
//   crates/cider-press-models/src/qwen2/weights.rs:316-376  pad_quantized_k
//   crates/cider-press-models/src/qwen2/weights.rs:297-307  build_padded_twin
//   crates/cider-press-models/src/qwen2/weights.rs:412-420  derive_quantization
//   crates/cider-press-models/src/qwen2/config.rs:65-73     {"quantization": {group_size, bits}}
//   crates/cider-press-models/src/error.rs:9-60             error kinds
//
// Archive layout (safetensors): an 8-byte little-endian header length H, H
// bytes of JSON {name: {"dtype", "shape", "data_offsets": [begin, end)}, and
// an optional "__metadata__" string map}, then the byte buffer the offsets
// index.  The file is memory-mapped; tensor bytes are uploaded straight from
// the mapping, so a multi-GB checkpoint is never copied on the host.
//
// Validation follows the format's rules: the header must be a JSON object,
// every entry a known dtype with a non-negative integer shape whose byte size
// equals end - begin, and the entries, sorted by offset, must tile the byte
// buffer exactly (no gap, no overlap, nothing left over).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "cpq_internal.hpp"

namespace cpq {
namespace {

// ---------------------------------------------------------------------------
// Minimal JSON reader (objects, arrays, strings with escapes, numbers,
// true/false/null) -- enough for safetensors headers and config.json.
// ---------------------------------------------------------------------------
struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  bool integral = false;     // the literal had no fraction or exponent
  unsigned long long u = 0;  // value of a non-negative integral literal
  bool negative = false;
  std::string str;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;  // document order

  const Json* get(const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool parse(Json& out, std::string& err) {
    if (!value(out, 0)) {
      err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      err = "trailing characters after JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* m) {
    if (err_.empty()) err_ = m;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return fail("invalid literal");
    p_ += n;
    return true;
  }
  static void utf8(std::string& s, unsigned cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(unsigned& v) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= end_ || *p_ != '"') return fail("expected string");
    ++p_;
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const unsigned char c = (unsigned char)*p_++;
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        s += (char)c;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          unsigned cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            unsigned lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("unpaired surrogate");
            p_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("unpaired surrogate");
          }
          utf8(s, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(Json& v) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
    if (*p_ == '0') {
      ++p_;
    } else {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(s, p_);
    v.kind = Json::Number;
    v.num = std::strtod(text.c_str(), nullptr);
    v.negative = text[0] == '-';
    v.integral = integral;
    if (integral && !v.negative) {
      unsigned long long u = 0;
      for (char c : text) {
        const unsigned d = (unsigned)(c - '0');
        if (u > (~0ull - d) / 10) return fail("integer out of range");
        u = u * 10 + d;
      }
      v.u = u;
    }
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    ws();
    if (p_ >= end_) return fail("unexpected end of JSON");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Json::Object;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
        ++p_;
        Json item;
        if (!value(item, depth + 1)) return false;
        v.members.emplace_back(std::move(key), std::move(item));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = Json::Array;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        Json item;
        if (!value(item, depth + 1)) return false;
        v.items.push_back(std::move(item));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Json::String;
      return string(v.str);
    }
    if (c == 't') {
      v.kind = Json::Bool;
      v.b = true;
      return lit("true");
    }
    if (c == 'f') {
      v.kind = Json::Bool;
      return lit("false");
    }
    if (c == 'n') {
      v.kind = Json::Null;
      return lit("null");
    }
    return number(v);
  }
};

// safetensors dtype names and element sizes (the format's closed list).
struct DtypeInfo {
  const char* name;
  size_t size;
};
constexpr DtypeInfo kDtypes[] = {
    {"BOOL", 1}, {"U8", 1},  {"I8", 1},   {"F8_E5M2", 1}, {"F8_E4M3", 1}, {"I16", 2},
    {"U16", 2},  {"F16", 2}, {"BF16", 2}, {"I32", 4},     {"U32", 4},     {"F32", 4},
    {"F64", 8},  {"I64", 8}, {"U64", 8},
};

size_t dtype_bytes(const std::string& name) {
  for (const auto& d : kDtypes)
    if (name == d.name) return d.size;
  return 0;
}

std::string shape_str(const std::vector<size_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

}  // namespace
}  // namespace cpq

struct cpq_safetensors {
  struct Entry {
    std::string name, dtype;
    std::vector<size_t> shape;
    size_t begin = 0, end = 0;
  };
  // Backing bytes: a private read-only mapping of the file, or an owned copy.
  const unsigned char* base = nullptr;
  size_t size = 0;
  void* map = nullptr;
  std::vector<unsigned char> owned;
  size_t data_start = 0;  // 8 + header length
  std::vector<Entry> entries;  // sorted by name
  std::vector<std::pair<std::string, std::string>> metadata;

  ~cpq_safetensors() {
    if (map) munmap(map, size);
  }
  const Entry* find(const char* key) const {
    auto it = std::lower_bound(entries.begin(), entries.end(), key,
                               [](const Entry& e, const char* k) { return e.name < k; });
    return it != entries.end() && it->name == key ? &*it : nullptr;
  }
  const unsigned char* data(const Entry& e) const { return base + data_start + e.begin; }
};

namespace cpq {
namespace {

cpq_status parse_archive(cpq_safetensors* st) {
  const auto bad = [](const std::string& m) { return fail(CPQ_ERR_SAFETENSORS, "safetensors: " + m); };
  if (st->size < 8) return bad("file shorter than the 8-byte header length");
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | st->base[i];
  if (hlen > 100ull * 1024 * 1024) return bad("header length " + std::to_string(hlen) + " too large");
  if (hlen > st->size - 8) return bad("header length " + std::to_string(hlen) + " exceeds the file");
  st->data_start = 8 + (size_t)hlen;
  const size_t buffer_len = st->size - st->data_start;
  Json root;
  std::string err;
  JsonParser jp(reinterpret_cast<const char*>(st->base + 8), (size_t)hlen);
  if (!jp.parse(root, err)) return bad("header is not valid JSON: " + err);
  if (root.kind != Json::Object) return bad("header is not a JSON object");
  for (const auto& m : root.members) {
    if (m.first == "__metadata__") {
      if (m.second.kind == Json::Null) continue;
      if (m.second.kind != Json::Object) return bad("__metadata__ is not an object");
      for (const auto& kv : m.second.members) {
        if (kv.second.kind != Json::String) return bad("__metadata__ values must be strings");
        st->metadata.emplace_back(kv.first, kv.second.str);
      }
      continue;
    }
    const Json& t = m.second;
    if (t.kind != Json::Object) return bad("entry \"" + m.first + "\" is not an object");
    const Json* dt = t.get("dtype");
    const Json* sh = t.get("shape");
    const Json* off = t.get("data_offsets");
    if (!dt || dt->kind != Json::String || !sh || sh->kind != Json::Array || !off || off->kind != Json::Array ||
        off->items.size() != 2)
      return bad("entry \"" + m.first + "\" needs dtype, shape and data_offsets [begin, end]");
    cpq_safetensors::Entry e;
    e.name = m.first;
    e.dtype = dt->str;
    const size_t esz = dtype_bytes(e.dtype);
    if (!esz) return bad("entry \"" + m.first + "\" has unknown dtype \"" + e.dtype + "\"");
    size_t numel = 1;
    for (const Json& d : sh->items) {
      if (d.kind != Json::Number || !d.integral || d.negative) return bad("entry \"" + m.first + "\": bad shape");
      size_t v = (size_t)d.u;
      if (v && numel > SIZE_MAX / v) return bad("entry \"" + m.first + "\": shape overflows");
      numel *= v;
      e.shape.push_back(v);
    }
    for (const Json& o : off->items)
      if (o.kind != Json::Number || !o.integral || o.negative) return bad("entry \"" + m.first + "\": bad data_offsets");
    e.begin = (size_t)off->items[0].u;
    e.end = (size_t)off->items[1].u;
    if (e.begin > e.end || e.end > buffer_len)
      return bad("entry \"" + m.first + "\": data_offsets [" + std::to_string(e.begin) + ", " +
                 std::to_string(e.end) + ") outside the " + std::to_string(buffer_len) + "-byte buffer");
    if (numel > SIZE_MAX / esz || numel * esz != e.end - e.begin)
      return bad("entry \"" + m.first + "\": " + std::to_string(e.end - e.begin) + " bytes for shape " +
                 shape_str(e.shape) + " of " + e.dtype);
    st->entries.push_back(std::move(e));
  }
  // The entries must tile the buffer: sorted by offset, each starts where the
  // previous ended, and the last ends at the buffer's end.
  std::vector<const cpq_safetensors::Entry*> by_off;
  for (const auto& e : st->entries) by_off.push_back(&e);
  std::sort(by_off.begin(), by_off.end(), [](const cpq_safetensors::Entry* a, const cpq_safetensors::Entry* b) {
    return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
  });
  size_t at = 0;
  for (const auto* e : by_off) {
    if (e->begin != at) return bad("entry \"" + e->name + "\" does not start where the previous one ends");
    at = e->end;
  }
  if (at != buffer_len) return bad("the byte buffer has " + std::to_string(buffer_len - at) + " unindexed trailing bytes");
  std::sort(st->entries.begin(), st->entries.end(),
            [](const cpq_safetensors::Entry& a, const cpq_safetensors::Entry& b) { return a.name < b.name; });
  for (size_t i = 1; i < st->entries.size(); ++i)
    if (st->entries[i].name == st->entries[i - 1].name) return bad("duplicate entry \"" + st->entries[i].name + "\"");
  return CPQ_OK;
}

cpq_status finish_open(std::unique_ptr<cpq_safetensors> st, cpq_safetensors** out) {
  const cpq_status s = parse_archive(st.get());
  if (s != CPQ_OK) return s;
  *out = st.release();
  return CPQ_OK;
}

// Shared by the plain and the K-padded loaders: the reference's checks of
// read_quantized_weight (safetensors_io.rs:55-123), in its order.
struct TripleView {
  const cpq_safetensors::Entry *w, *s, *b;
  size_t n, k;
  cpq_dtype dtype;
};

cpq_status check_triple(const cpq_safetensors* st, const char* base, uint32_t bits, uint32_t group_size,
                        TripleView& tv) {
  const std::string wk = std::string(base) + ".weight", sk = std::string(base) + ".scales",
                    bk = std::string(base) + ".biases";
  const auto missing = [](const std::string& k) {
    return fail(CPQ_ERR_MISSING_KEY, "safetensors: missing tensor key \"" + k + "\"");
  };
  const auto unsupported = [](const std::string& k, const std::string& d) {
    return fail(CPQ_ERR_UNSUPPORTED_DTYPE, "safetensors: unsupported dtype " + d + " for key \"" + k + "\"");
  };
  tv.w = st->find(wk.c_str());
  if (!tv.w) return missing(wk);
  tv.s = st->find(sk.c_str());
  if (!tv.s) return missing(sk);
  tv.b = st->find(bk.c_str());
  if (!tv.b) return missing(bk);
  if (tv.w->dtype != "U32") return unsupported(wk, tv.w->dtype);
  // The reference accepts BF16 scales and biases; F16 (both) is accepted too,
  // since the kernels run either element type.
  if (tv.s->dtype != "BF16" && tv.s->dtype != "F16") return unsupported(sk, tv.s->dtype);
  if (tv.b->dtype != tv.s->dtype) return unsupported(bk, tv.b->dtype);
  tv.dtype = tv.s->dtype == "BF16" ? CPQ_DTYPE_BF16 : CPQ_DTYPE_F16;
  if (tv.w->shape.size() != 2)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized weight \"" + wk + "\" must be rank-2 [N, packed_K]; got shape " +
                                              shape_str(tv.w->shape));
  cpq_status q = cpq_quantization_validate(bits, group_size);
  if (q != CPQ_OK) return q;
  tv.n = tv.w->shape[0];
  const size_t packed_k = tv.w->shape[1];
  if (packed_k > SIZE_MAX / 32)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized weight \"" + wk + "\": packed_K * 32 overflows usize");
  const size_t bit_total = packed_k * 32;
  if (bit_total % bits != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized weight \"" + wk + "\": packed_K (" + std::to_string(packed_k) +
                                              ") x 32 not divisible by bits (" + std::to_string(bits) + ")");
  tv.k = bit_total / bits;
  if (tv.k % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized weight \"" + wk + "\": recovered K (" + std::to_string(tv.k) +
                                              ") not divisible by group_size (" + std::to_string(group_size) + ")");
  const std::vector<size_t> aux{tv.n, tv.k / group_size};
  if (tv.s->shape != aux)
    return fail(CPQ_ERR_SHAPE_MISMATCH, "safetensors: shape mismatch for \"" + sk + "\": expected " + shape_str(aux) +
                                            ", got " + shape_str(tv.s->shape));
  if (tv.b->shape != aux)
    return fail(CPQ_ERR_SHAPE_MISMATCH, "safetensors: shape mismatch for \"" + bk + "\": expected " + shape_str(aux) +
                                            ", got " + shape_str(tv.b->shape));
  return CPQ_OK;
}

}  // namespace
}  // namespace cpq

using cpq::fail;

extern "C" {

cpq_status cpq_safetensors_open(const char* path, cpq_safetensors** out) {
  if (!path || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_open: NULL argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(CPQ_ERR_SAFETENSORS, std::string("safetensors: cannot open ") + path + ": " + std::strerror(errno));
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    const int e = errno;
    close(fd);
    return fail(CPQ_ERR_SAFETENSORS, std::string("safetensors: cannot stat ") + path + ": " + std::strerror(e));
  }
  auto st = std::make_unique<cpq_safetensors>();
  st->size = (size_t)sb.st_size;
  if (st->size > 0) {
    void* m = mmap(nullptr, st->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      const int e = errno;
      close(fd);
      return fail(CPQ_ERR_SAFETENSORS, std::string("safetensors: cannot map ") + path + ": " + std::strerror(e));
    }
    st->map = m;
    st->base = static_cast<const unsigned char*>(m);
  }
  close(fd);
  return cpq::finish_open(std::move(st), out);
}

cpq_status cpq_safetensors_deserialize(const void* bytes, size_t len, cpq_safetensors** out) {
  if ((!bytes && len) || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_deserialize: NULL argument");
  *out = nullptr;
  auto st = std::make_unique<cpq_safetensors>();
  st->owned.assign(static_cast<const unsigned char*>(bytes), static_cast<const unsigned char*>(bytes) + len);
  st->base = st->owned.data();
  st->size = len;
  return cpq::finish_open(std::move(st), out);
}

void cpq_safetensors_close(cpq_safetensors* st) { delete st; }

cpq_status cpq_safetensors_len(const cpq_safetensors* st, size_t* n) {
  if (!st || !n) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_len: NULL argument");
  *n = st->entries.size();
  return CPQ_OK;
}

cpq_status cpq_safetensors_name(const cpq_safetensors* st, size_t i, const char** name) {
  if (!st || !name) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_name: NULL argument");
  if (i >= st->entries.size()) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_name: index out of range");
  *name = st->entries[i].name.c_str();
  return CPQ_OK;
}

cpq_status cpq_safetensors_tensor(const cpq_safetensors* st, const char* key, const char** dtype, size_t* dims,
                                  size_t cap, size_t* ndim, const void** data, size_t* nbytes) {
  if (!st || !key || !dtype || !ndim || !data || !nbytes || (cap && !dims))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_tensor: NULL argument");
  const auto* e = st->find(key);
  if (!e) return fail(CPQ_ERR_MISSING_KEY, std::string("safetensors: missing tensor key \"") + key + "\"");
  *ndim = e->shape.size();
  if (e->shape.size() > cap) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_tensor: dims capacity too small");
  for (size_t i = 0; i < e->shape.size(); ++i) dims[i] = e->shape[i];
  *dtype = e->dtype.c_str();
  *data = st->data(*e);
  *nbytes = e->end - e->begin;
  return CPQ_OK;
}

cpq_status cpq_safetensors_metadata(const cpq_safetensors* st, const char* key, const char** value) {
  if (!st || !key || !value) return fail(CPQ_ERR_INVALID_ARGUMENT, "safetensors_metadata: NULL argument");
  for (const auto& kv : st->metadata)
    if (kv.first == key) {
      *value = kv.second.c_str();
      return CPQ_OK;
    }
  return fail(CPQ_ERR_MISSING_KEY, std::string("safetensors: missing metadata key \"") + key + "\"");
}

cpq_status cpq_read_quantized_weight(cpq_device* dev, const cpq_safetensors* st, const char* base_name,
                                     uint32_t bits, uint32_t group_size, cpq_qweight** out) {
  if (!st || !base_name || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight: NULL argument");
  *out = nullptr;
  cpq::TripleView tv;
  cpq_status s = cpq::check_triple(st, base_name, bits, group_size, tv);
  if (s != CPQ_OK) return s;
  if (!dev) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight: NULL device");
  return cpq_qweight_from_bytes(dev, tv.dtype, tv.n, tv.k, tv.k, bits, group_size, st->data(*tv.w),
                                tv.w->end - tv.w->begin, st->data(*tv.s), tv.s->end - tv.s->begin,
                                st->data(*tv.b), tv.b->end - tv.b->begin, out);
}

cpq_status cpq_pad_quantized_k(const void* weights, const void* scales, const void* biases, size_t n, size_t k,
                               size_t k_pad, uint32_t bits, uint32_t group_size, size_t sb_elem_bytes,
                               void* w_out, void* s_out, void* b_out) {
  if (!weights || !scales || !biases || !w_out || !s_out || !b_out)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: NULL argument");
  cpq_status q = cpq_quantization_validate(bits, group_size);
  if (q != CPQ_OK) return q;
  if (sb_elem_bytes != 2) return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: scales/biases must be 16-bit");
  if (k % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: k=" + std::to_string(k) +
                                              " must be a multiple of group_size=" + std::to_string(group_size));
  if (k_pad < k)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: k_pad=" + std::to_string(k_pad) + " must be >= k=" +
                                              std::to_string(k));
  if (k_pad % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: k_pad=" + std::to_string(k_pad) +
                                              " must be a multiple of group_size=" + std::to_string(group_size));
  // Row strides: packed bytes k*bits/8 (whole words, since gs*bits % 32 == 0),
  // scale/bias bytes (k/gs)*2.  Pad columns are zero words and zero s, b.
  const size_t w_src = k * bits / 8, w_dst = k_pad * bits / 8;
  const size_t sb_src = (k / group_size) * sb_elem_bytes, sb_dst = (k_pad / group_size) * sb_elem_bytes;
  if (n && (w_dst > SIZE_MAX / n || sb_dst > SIZE_MAX / n))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "pad_quantized_k: padded size overflows usize");
  auto* wo = static_cast<unsigned char*>(w_out);
  auto* so = static_cast<unsigned char*>(s_out);
  auto* bo = static_cast<unsigned char*>(b_out);
  const auto* wi = static_cast<const unsigned char*>(weights);
  const auto* si = static_cast<const unsigned char*>(scales);
  const auto* bi = static_cast<const unsigned char*>(biases);
  for (size_t r = 0; r < n; ++r) {
    std::memcpy(wo + r * w_dst, wi + r * w_src, w_src);
    std::memset(wo + r * w_dst + w_src, 0, w_dst - w_src);
    std::memcpy(so + r * sb_dst, si + r * sb_src, sb_src);
    std::memset(so + r * sb_dst + sb_src, 0, sb_dst - sb_src);
    std::memcpy(bo + r * sb_dst, bi + r * sb_src, sb_src);
    std::memset(bo + r * sb_dst + sb_src, 0, sb_dst - sb_src);
  }
  return CPQ_OK;
}

cpq_status cpq_read_quantized_weight_k_padded(cpq_device* dev, const cpq_safetensors* st, const char* base_name,
                                              uint32_t bits, uint32_t group_size, size_t k_pad,
                                              cpq_qweight** out) {
  if (!st || !base_name || !out)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight_k_padded: NULL argument");
  *out = nullptr;
  cpq::TripleView tv;
  cpq_status s = cpq::check_triple(st, base_name, bits, group_size, tv);
  if (s != CPQ_OK) return s;
  if (k_pad < tv.k || k_pad % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight_k_padded: k_pad=" + std::to_string(k_pad) +
                                              " must be >= K=" + std::to_string(tv.k) +
                                              " and a multiple of group_size=" + std::to_string(group_size));
  if (!dev) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight_k_padded: NULL device");
  if (tv.n > SIZE_MAX / k_pad) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_quantized_weight_k_padded: N*K overflows");
  std::vector<unsigned char> w(tv.n * (k_pad * bits / 8)), sc(tv.n * (k_pad / group_size) * 2),
      bi(tv.n * (k_pad / group_size) * 2);
  s = cpq_pad_quantized_k(st->data(*tv.w), st->data(*tv.s), st->data(*tv.b), tv.n, tv.k, k_pad, bits, group_size, 2,
                          w.data(), sc.data(), bi.data());
  if (s != CPQ_OK) return s;
  return cpq_qweight_from_bytes(dev, tv.dtype, tv.n, k_pad, tv.k, bits, group_size, w.data(), w.size(), sc.data(),
                                sc.size(), bi.data(), bi.size(), out);
}

cpq_status cpq_read_dense_tensor(cpq_device* dev, const cpq_safetensors* st, const char* key, cpq_tensor** out) {
  if (!st || !key || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_dense_tensor: NULL argument");
  *out = nullptr;
  const auto* e = st->find(key);
  if (!e) return fail(CPQ_ERR_MISSING_KEY, std::string("safetensors: missing tensor key \"") + key + "\"");
  cpq_dtype dt;
  if (e->dtype == "BF16") dt = CPQ_DTYPE_BF16;
  else if (e->dtype == "F16") dt = CPQ_DTYPE_F16;
  else return fail(CPQ_ERR_UNSUPPORTED_DTYPE, "safetensors: unsupported dtype " + e->dtype + " for key \"" + key + "\"");
  if (!dev) return fail(CPQ_ERR_INVALID_ARGUMENT, "read_dense_tensor: NULL device");
  return cpq_tensor_from_host(dev, dt, e->shape.data(), e->shape.size(), st->data(*e), out);
}

cpq_status cpq_quantization_from_config(const char* json, size_t len, int* present, uint32_t* bits,
                                        uint32_t* group_size) {
  if ((!json && len) || !present || !bits || !group_size)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantization_from_config: NULL argument");
  *present = 0;
  *bits = *group_size = 0;
  cpq::Json root;
  std::string err;
  cpq::JsonParser jp(json, len);
  if (!jp.parse(root, err)) return fail(CPQ_ERR_JSON, "json: " + err);
  if (root.kind != cpq::Json::Object) return fail(CPQ_ERR_JSON, "json: config is not an object");
  const cpq::Json* q = root.get("quantization");
  if (!q || q->kind == cpq::Json::Null) return CPQ_OK;
  if (q->kind != cpq::Json::Object) return fail(CPQ_ERR_JSON, "json: \"quantization\" is not an object");
  const cpq::Json* g = q->get("group_size");
  const cpq::Json* b = q->get("bits");
  if (!g) return fail(CPQ_ERR_JSON, "json: missing field `group_size`");
  if (!b) return fail(CPQ_ERR_JSON, "json: missing field `bits`");
  // group_size: u32, bits: u8 (config.rs:65-73).
  if (g->kind != cpq::Json::Number || !g->integral || g->negative || g->u > 0xFFFFFFFFull)
    return fail(CPQ_ERR_JSON, "json: `group_size` is not a u32");
  if (b->kind != cpq::Json::Number || !b->integral || b->negative || b->u > 0xFFull)
    return fail(CPQ_ERR_JSON, "json: `bits` is not a u8");
  *present = 1;
  *bits = (uint32_t)b->u;
  *group_size = (uint32_t)g->u;
  return CPQ_OK;
}

}  // extern "C"
