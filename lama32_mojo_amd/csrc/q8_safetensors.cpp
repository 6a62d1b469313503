// q8_safetensors.cpp -- safetensors reader and writer (host code).
//
// Reader: the reference's multi-shard SafeTensors (src/safetensors.mojo:36-
// 95): with `model.safetensors.index.json` in a directory the shards are the
// weight_map's files in order of first appearance, otherwise the one
// `model.safetensors` (or the file named).  Each shard's header -- an 8-byte
// little-endian length, then a JSON object name -> {dtype, shape,
// data_offsets} with an optional "__metadata__" -- gives the absolute byte
// range of every tensor.  Tensors are listed shard by shard in header order.
//
// Writer: the layout of the safetensors library's serializer (the format
// qwen3_mojo/scripts/quantize.py:59-61 writes with save_file): tensors sorted
// by dtype, descending in the library's dtype order (U64 first, BOOL last),
// then by name; compact JSON with "__metadata__" first when given; the
// header padded with spaces to a multiple of 8 bytes; tensor bytes back to
// back in that order.  So a file written here from the same tensors is
// byte-identical to the library's.
//
// Header text comes from files and is untrusted: the parser checks every
// index against the text's end, limits nesting, and rejects offsets that
// fall outside the file.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/q8hip.h"

namespace {

constexpr int kReadAttempts = 15;     // reads of one tensor range, first included
constexpr int kReadRetryMs = 2000;    // between two attempts

thread_local std::string g_err;

int st_fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// ---- JSON (the subset safetensors headers use) ------------------------------
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  bool integral = false;
  int64_t i = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;   // in text order
  const JVal *get(const char *key) const {
    for (const auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *end;
  std::string err;
  int depth = 0;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  static void put_utf8(std::string &o, uint32_t c) {
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
  bool hex4(uint32_t &v) {
    if (end - p < 4) return fail("truncated \\u escape");
    v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool str(std::string &o) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (true) {
      if (p >= end) return fail("unterminated string");
      const char c = *p++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        o += c;
        continue;
      }
      if (p >= end) return fail("unterminated escape");
      const char e = *p++;
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00) {          // surrogate pair
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            uint32_t c2;
            if (!hex4(c2)) return false;
            if (c2 < 0xDC00 || c2 >= 0xE000) return fail("bad surrogate pair");
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          } else if (c1 >= 0xDC00 && c1 < 0xE000) {
            return fail("lone surrogate");
          }
          put_utf8(o, c1);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool num(JVal &v) {
    const char *s = p;
    if (p < end && *p == '-') ++p;
    bool digits = false, frac = false;
    while (p < end && *p >= '0' && *p <= '9') { ++p; digits = true; }
    if (p < end && *p == '.') {
      frac = true;
      ++p;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      frac = true;
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (!digits) return fail("bad number");
    v.kind = JVal::NUM;
    v.integral = !frac;
    if (!frac) {
      // integers: exact, with overflow detection
      const bool neg = *s == '-';
      uint64_t acc = 0;
      for (const char *q = s + (neg ? 1 : 0); q < p; ++q) {
        const uint64_t d = (uint64_t)(*q - '0');
        if (acc > (UINT64_MAX - d) / 10) return fail("integer out of range");
        acc = acc * 10 + d;
      }
      if (acc > (uint64_t)INT64_MAX) return fail("integer out of range");
      v.i = neg ? -(int64_t)acc : (int64_t)acc;
    }
    return true;
  }
  bool lit(const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool val(JVal &v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    bool ok = true;
    const char c = *p;
    if (c == '{') {
      v.kind = JVal::OBJ;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
      } else {
        while (ok) {
          ws();
          std::string k;
          JVal x;
          ok = str(k);
          if (!ok) break;
          ws();
          if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
          ++p;
          ok = val(x);
          if (!ok) break;
          v.obj.emplace_back(std::move(k), std::move(x));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == '}') { ++p; break; }
          ok = fail("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      v.kind = JVal::ARR;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
      } else {
        while (ok) {
          JVal x;
          ok = val(x);
          if (!ok) break;
          v.arr.push_back(std::move(x));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == ']') { ++p; break; }
          ok = fail("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v.kind = JVal::STR;
      ok = str(v.s);
    } else if (c == 't') {
      v.kind = JVal::BOOL;
      v.b = true;
      ok = lit("true");
    } else if (c == 'f') {
      v.kind = JVal::BOOL;
      ok = lit("false");
    } else if (c == 'n') {
      ok = lit("null");
    } else {
      ok = num(v);
    }
    --depth;
    return ok;
  }
};

bool parse_json(const std::string &text, JVal &out, std::string &err) {
  JParser jp{text.data(), text.data() + text.size(), {}};
  if (!jp.val(out)) {
    err = jp.err;
    return false;
  }
  jp.ws();
  if (jp.p != jp.end) {
    err = "trailing characters";
    return false;
  }
  return true;
}

// ---- dtypes ----------------------------------------------------------------
struct DtypeInfo {
  const char *name;
  int bits;
  int rank;   // the library's sort order (higher first)
};
const DtypeInfo kDtypes[] = {
    {"BOOL", 8, 0},     {"U8", 8, 1},    {"I8", 8, 2},    {"F8_E5M2", 8, 3},
    {"F8_E4M3", 8, 4},  {"I16", 16, 5},  {"U16", 16, 6},  {"F16", 16, 7},
    {"BF16", 16, 8},    {"I32", 32, 9},  {"U32", 32, 10}, {"F32", 32, 11},
    {"F64", 64, 12},    {"I64", 64, 13}, {"U64", 64, 14},
};
const DtypeInfo *dtype_of(const std::string &s) {
  for (const auto &d : kDtypes)
    if (s == d.name) return &d;
  return nullptr;
}

bool shape_bytes(const std::vector<int64_t> &shape, int bits, uint64_t &bytes) {
  uint64_t n = 1;
  for (int64_t d : shape) {
    if (d < 0) return false;
    if (d != 0 && n > UINT64_MAX / (uint64_t)d) return false;
    n *= (uint64_t)d;
  }
  if (n > UINT64_MAX / 8) return false;
  bytes = n * (uint64_t)bits / 8;
  return true;
}

// Reads n bytes at off, advancing *done past what arrived; returns 0, the
// errno of a failed read, or -1 when the file ends first.
int read_some(int fd, uint64_t off, void *dst, uint64_t n, uint64_t *done) {
  char *d = static_cast<char *>(dst);
  while (*done < n) {
    const uint64_t left = n - *done;
    const ssize_t r = pread(fd, d + *done, left > (1u << 30) ? (1u << 30) : left,
                            (off_t)(off + *done));
    if (r < 0 && errno == EINTR) continue;
    if (r < 0) return errno ? errno : EIO;
    if (r == 0) return -1;
    *done += (uint64_t)r;
  }
  return 0;
}

bool read_all(int fd, uint64_t off, void *dst, uint64_t n) {
  uint64_t done = 0;
  return read_some(fd, off, dst, n, &done) == 0;
}

// A read failure that can pass (an I/O error, a timeout, a stale network
// file handle, a busy or exhausted resource), as opposed to a file that
// ends inside a tensor or a bad descriptor.
bool transient_read_error(int err) {
  return err == EIO || err == EAGAIN || err == ETIMEDOUT || err == ESTALE || err == EBUSY ||
         err == ENOMEM || err == ENOBUFS;
}

bool write_all(int fd, uint64_t off, const void *src, uint64_t n) {
  const char *s = static_cast<const char *>(src);
  while (n > 0) {
    const ssize_t r = pwrite(fd, s, n > (1u << 30) ? (1u << 30) : n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    s += r;
    off += (uint64_t)r;
    n -= (uint64_t)r;
  }
  return true;
}

std::string json_escape(const std::string &s) {
  // serde_json's escaping: quote, backslash and control characters
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          char b[8];
          snprintf(b, sizeof b, "\\u%04x", c);
          o += b;
        } else {
          o += (char)c;
        }
    }
  }
  return o + "\"";
}

bool is_dir(const std::string &path) {
  struct stat sb;
  return stat(path.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode);
}

bool file_exists(const std::string &path) {
  struct stat sb;
  return stat(path.c_str(), &sb) == 0 && S_ISREG(sb.st_mode);
}

bool slurp(const std::string &path, std::string &out) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return false;
  struct stat sb;
  bool ok = fstat(fd, &sb) == 0 && sb.st_size >= 0 && sb.st_size < (1 << 28);
  if (ok) {
    out.resize((size_t)sb.st_size);
    ok = read_all(fd, 0, &out[0], (uint64_t)sb.st_size);
  }
  close(fd);
  return ok;
}

}  // namespace

// ---- reader -----------------------------------------------------------------
struct q8_st {
  struct Tensor {
    std::string name, dtype;
    std::vector<int64_t> shape;
    int file;
    uint64_t begin, end;   // absolute byte offsets in the file
  };
  std::vector<std::string> paths;
  // (reopened by a read that retries, under reopen_mu)
  mutable std::vector<int> fds;
  mutable std::mutex reopen_mu;
  std::vector<Tensor> tensors;
  std::map<std::string, int64_t> index;
  std::vector<std::pair<std::string, std::string>> metadata;   // first shard's
  ~q8_st() {
    for (int fd : fds)
      if (fd >= 0) close(fd);
  }
};

namespace {

int read_shard(q8_st *st, const std::string &path) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return st_fail(Q8_ERR_ARG, "cannot open %s: %s", path.c_str(), strerror(errno));
  const int file = (int)st->fds.size();
  st->fds.push_back(fd);
  st->paths.push_back(path);
  struct stat sb;
  if (fstat(fd, &sb) != 0) return st_fail(Q8_ERR_ARG, "cannot stat %s", path.c_str());
  const uint64_t fsize = (uint64_t)sb.st_size;
  unsigned char lenb[8];
  if (fsize < 8 || !read_all(fd, 0, lenb, 8))
    return st_fail(Q8_ERR_SHAPE, "%s: shorter than a safetensors header", path.c_str());
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | lenb[k];
  if (n > (uint64_t)100 << 20 || 8 + n > fsize)
    return st_fail(Q8_ERR_SHAPE, "%s: header length %llu does not fit the file", path.c_str(),
                   (unsigned long long)n);
  std::string text((size_t)n, '\0');
  if (n && !read_all(fd, 8, &text[0], n))
    return st_fail(Q8_ERR_ARG, "%s: cannot read the header", path.c_str());
  JVal hdr;
  std::string err;
  if (!parse_json(text, hdr, err) || hdr.kind != JVal::OBJ)
    return st_fail(Q8_ERR_SHAPE, "%s: bad header JSON (%s)", path.c_str(),
                   err.empty() ? "not an object" : err.c_str());
  const uint64_t data0 = 8 + n;
  for (const auto &kv : hdr.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JVal::OBJ)
        return st_fail(Q8_ERR_SHAPE, "%s: __metadata__ is not an object", path.c_str());
      if (file == 0)
        for (const auto &m : kv.second.obj) {
          if (m.second.kind != JVal::STR)
            return st_fail(Q8_ERR_SHAPE, "%s: metadata values must be strings", path.c_str());
          st->metadata.emplace_back(m.first, m.second.s);
        }
      continue;
    }
    const JVal &t = kv.second;
    const JVal *dt = t.kind == JVal::OBJ ? t.get("dtype") : nullptr;
    const JVal *sh = t.kind == JVal::OBJ ? t.get("shape") : nullptr;
    const JVal *of = t.kind == JVal::OBJ ? t.get("data_offsets") : nullptr;
    if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !of ||
        of->kind != JVal::ARR || of->arr.size() != 2)
      return st_fail(Q8_ERR_SHAPE, "%s: tensor '%s' lacks dtype, shape or data_offsets",
                     path.c_str(), kv.first.c_str());
    const DtypeInfo *di = dtype_of(dt->s);
    if (!di)
      return st_fail(Q8_ERR_UNSUPPORTED, "%s: tensor '%s' has dtype %s", path.c_str(),
                     kv.first.c_str(), dt->s.c_str());
    q8_st::Tensor ti;
    ti.name = kv.first;
    ti.dtype = dt->s;
    ti.file = file;
    for (const auto &d : sh->arr) {
      if (d.kind != JVal::NUM || !d.integral || d.i < 0)
        return st_fail(Q8_ERR_SHAPE, "%s: tensor '%s' has a bad shape", path.c_str(),
                       kv.first.c_str());
      ti.shape.push_back(d.i);
    }
    const JVal &o0 = of->arr[0], &o1 = of->arr[1];
    if (o0.kind != JVal::NUM || o1.kind != JVal::NUM || !o0.integral || !o1.integral ||
        o0.i < 0 || o1.i < o0.i)
      return st_fail(Q8_ERR_SHAPE, "%s: tensor '%s' has bad data_offsets", path.c_str(),
                     kv.first.c_str());
    uint64_t bytes = 0;
    if (!shape_bytes(ti.shape, di->bits, bytes) || bytes != (uint64_t)(o1.i - o0.i))
      return st_fail(Q8_ERR_SHAPE, "%s: tensor '%s': %llu data bytes for its shape and dtype",
                     path.c_str(), kv.first.c_str(), (unsigned long long)(o1.i - o0.i));
    ti.begin = data0 + (uint64_t)o0.i;
    ti.end = data0 + (uint64_t)o1.i;
    if (ti.end > fsize || ti.end < ti.begin)
      return st_fail(Q8_ERR_SHAPE, "%s: tensor '%s' runs past the end of the file",
                     path.c_str(), kv.first.c_str());
    if (st->index.count(ti.name))
      return st_fail(Q8_ERR_SHAPE, "tensor '%s' appears twice", ti.name.c_str());
    st->index[ti.name] = (int64_t)st->tensors.size();
    st->tensors.push_back(std::move(ti));
  }
  return Q8_OK;
}

}  // namespace

extern "C" {

const char *q8_st_error(void) { return g_err.c_str(); }

int q8_st_open(const char *path, q8_st **out) {
  if (!path || !out) return st_fail(Q8_ERR_ARG, "q8_st_open: null argument");
  *out = nullptr;
  std::unique_ptr<q8_st> st(new (std::nothrow) q8_st());
  if (!st) return st_fail(Q8_ERR_NOMEM, "q8_st_open: out of host memory");
  std::vector<std::string> shards;
  const std::string p(path);
  if (is_dir(p)) {
    const std::string idx = p + "/model.safetensors.index.json";
    if (file_exists(idx)) {
      std::string text;
      JVal j;
      std::string err;
      if (!slurp(idx, text)) return st_fail(Q8_ERR_ARG, "cannot read %s", idx.c_str());
      if (!parse_json(text, j, err) || j.kind != JVal::OBJ)
        return st_fail(Q8_ERR_SHAPE, "%s: bad JSON (%s)", idx.c_str(), err.c_str());
      const JVal *wm = j.get("weight_map");
      if (!wm || wm->kind != JVal::OBJ)
        return st_fail(Q8_ERR_SHAPE, "%s: no weight_map object", idx.c_str());
      for (const auto &kv : wm->obj) {
        if (kv.second.kind != JVal::STR || kv.second.s.empty() ||
            kv.second.s.find('/') != std::string::npos)
          return st_fail(Q8_ERR_SHAPE, "%s: bad shard name for '%s'", idx.c_str(),
                         kv.first.c_str());
        const std::string f = p + "/" + kv.second.s;
        if (std::find(shards.begin(), shards.end(), f) == shards.end()) shards.push_back(f);
      }
    } else {
      shards.push_back(p + "/model.safetensors");
    }
  } else {
    shards.push_back(p);
  }
  for (const auto &s : shards)
    if (int rc = read_shard(st.get(), s)) return rc;
  *out = st.release();
  return Q8_OK;
}

void q8_st_close(q8_st *st) { delete st; }

int64_t q8_st_count(const q8_st *st) { return st ? (int64_t)st->tensors.size() : -1; }

int64_t q8_st_find(const q8_st *st, const char *name) {
  if (!st || !name) return -1;
  const auto it = st->index.find(name);
  return it == st->index.end() ? -1 : it->second;
}

int q8_st_info(const q8_st *st, int64_t i, const char **name, const char **dtype, int *ndim,
               const int64_t **shape, const char **path, uint64_t *begin, uint64_t *nbytes) {
  if (!st || i < 0 || i >= (int64_t)st->tensors.size())
    return st_fail(Q8_ERR_ARG, "q8_st_info: no tensor %lld", (long long)i);
  const q8_st::Tensor &t = st->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype.c_str();
  if (ndim) *ndim = (int)t.shape.size();
  if (shape) *shape = t.shape.data();
  if (path) *path = st->paths[(size_t)t.file].c_str();
  if (begin) *begin = t.begin;
  if (nbytes) *nbytes = t.end - t.begin;
  return Q8_OK;
}

int64_t q8_st_metadata_count(const q8_st *st) { return st ? (int64_t)st->metadata.size() : -1; }

int q8_st_metadata(const q8_st *st, int64_t i, const char **key, const char **value) {
  if (!st || i < 0 || i >= (int64_t)st->metadata.size())
    return st_fail(Q8_ERR_ARG, "q8_st_metadata: no entry %lld", (long long)i);
  if (key) *key = st->metadata[(size_t)i].first.c_str();
  if (value) *value = st->metadata[(size_t)i].second.c_str();
  return Q8_OK;
}

int q8_st_read(const q8_st *st, int64_t i, uint64_t byte_off, void *dst, uint64_t nbytes) {
  if (!st || i < 0 || i >= (int64_t)st->tensors.size())
    return st_fail(Q8_ERR_ARG, "q8_st_read: no tensor %lld", (long long)i);
  const q8_st::Tensor &t = st->tensors[(size_t)i];
  const uint64_t size = t.end - t.begin;
  if (byte_off > size || nbytes > size - byte_off)
    return st_fail(Q8_ERR_RANGE, "q8_st_read: [%llu, +%llu) exceeds '%s' (%llu bytes)",
                   (unsigned long long)byte_off, (unsigned long long)nbytes, t.name.c_str(),
                   (unsigned long long)size);
  if (nbytes && !dst) return st_fail(Q8_ERR_ARG, "q8_st_read: null destination");
  // A failed read is tried again, as the reference's loader does (15
  // attempts 2 s apart, reopening the file each time: src/resident.mojo:41-54),
  // when the failure can pass; the bytes already read are kept.  A file that
  // ends inside the tensor fails at once.
  uint64_t done = 0;
  for (int attempt = 1;; ++attempt) {
    int fd;
    {
      std::lock_guard<std::mutex> lock(st->reopen_mu);
      fd = st->fds[(size_t)t.file];
    }
    const int err = read_some(fd, t.begin + byte_off, dst, nbytes, &done);
    if (err == 0) return Q8_OK;
    if (err < 0 || !transient_read_error(err) || attempt >= kReadAttempts)
      return st_fail(Q8_ERR_ARG, "q8_st_read: read of '%s' failed after %d attempt%s: %s",
                     t.name.c_str(), attempt, attempt > 1 ? "s" : "",
                     err < 0 ? "the file ends inside the tensor" : strerror(err));
    fprintf(stderr, "q8_st_read: read of '%s' failed (%s), retry %d\n", t.name.c_str(),
            strerror(err), attempt);
    std::this_thread::sleep_for(std::chrono::milliseconds(kReadRetryMs));
    std::lock_guard<std::mutex> lock(st->reopen_mu);
    const int nfd = open(st->paths[(size_t)t.file].c_str(), O_RDONLY | O_CLOEXEC);
    if (nfd >= 0) {
      close(st->fds[(size_t)t.file]);
      st->fds[(size_t)t.file] = nfd;
    }
  }
}

// ---- writer -----------------------------------------------------------------
struct q8_stw {
  int fd = -1;
  std::string path;
  std::vector<uint64_t> offset, size;   // absolute file offset, bytes (caller order)
  std::vector<bool> done;
  ~q8_stw() {
    if (fd >= 0) close(fd);
  }
};

int q8_stw_open(const char *path, int64_t count, const char *const *names,
                const char *const *dtypes, const int *ndims, const int64_t *shapes,
                int64_t nmeta, const char *const *meta_keys, const char *const *meta_values,
                q8_stw **out) {
  if (!path || !out || count < 0 || nmeta < 0 || (count && (!names || !dtypes || !ndims)) ||
      (nmeta && (!meta_keys || !meta_values)))
    return st_fail(Q8_ERR_ARG, "q8_stw_open: bad arguments");
  *out = nullptr;
  struct Item {
    std::string name;
    const DtypeInfo *dt;
    std::vector<int64_t> shape;
    uint64_t bytes;
    int64_t caller;
  };
  std::vector<Item> items((size_t)count);
  const int64_t *sp = shapes;
  std::map<std::string, int> seen;
  for (int64_t i = 0; i < count; ++i) {
    Item &it = items[(size_t)i];
    if (!names[i] || !dtypes[i] || ndims[i] < 0 || ndims[i] > 16 || (ndims[i] && !sp))
      return st_fail(Q8_ERR_ARG, "q8_stw_open: bad entry %lld", (long long)i);
    it.name = names[i];
    if (it.name == "__metadata__" || seen[it.name]++)
      return st_fail(Q8_ERR_ARG, "q8_stw_open: bad or repeated name '%s'", names[i]);
    it.dt = dtype_of(dtypes[i]);
    if (!it.dt) return st_fail(Q8_ERR_UNSUPPORTED, "q8_stw_open: dtype %s", dtypes[i]);
    it.shape.assign(sp, sp + ndims[i]);
    sp += ndims[i];
    if (!shape_bytes(it.shape, it.dt->bits, it.bytes))
      return st_fail(Q8_ERR_SHAPE, "q8_stw_open: bad shape for '%s'", names[i]);
    it.caller = i;
  }
  // the library's order: dtype descending, then name
  std::vector<size_t> order((size_t)count);
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    if (items[a].dt->rank != items[b].dt->rank) return items[a].dt->rank > items[b].dt->rank;
    return items[a].name < items[b].name;
  });
  std::string h = "{";
  bool first = true;
  if (nmeta) {
    h += "\"__metadata__\":{";
    for (int64_t k = 0; k < nmeta; ++k) {
      if (!meta_keys[k] || !meta_values[k])
        return st_fail(Q8_ERR_ARG, "q8_stw_open: null metadata entry");
      if (k) h += ",";
      h += json_escape(meta_keys[k]) + ":" + json_escape(meta_values[k]);
    }
    h += "}";
    first = false;
  }
  std::unique_ptr<q8_stw> w(new (std::nothrow) q8_stw());
  if (!w) return st_fail(Q8_ERR_NOMEM, "q8_stw_open: out of host memory");
  w->offset.assign((size_t)count, 0);
  w->size.assign((size_t)count, 0);
  w->done.assign((size_t)count, false);
  uint64_t off = 0;
  std::vector<uint64_t> rel((size_t)count);
  for (size_t k : order) {
    const Item &it = items[k];
    if (!first) h += ",";
    first = false;
    h += json_escape(it.name) + ":{\"dtype\":\"" + it.dt->name + "\",\"shape\":[";
    for (size_t d = 0; d < it.shape.size(); ++d) {
      if (d) h += ",";
      h += std::to_string(it.shape[d]);
    }
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + it.bytes) +
         "]}";
    rel[k] = off;
    off += it.bytes;
  }
  h += "}";
  while (h.size() % 8) h += ' ';
  const uint64_t data0 = 8 + h.size();
  for (size_t k = 0; k < items.size(); ++k) {
    w->offset[(size_t)items[k].caller] = data0 + rel[k];
    w->size[(size_t)items[k].caller] = items[k].bytes;
  }
  w->path = path;
  w->fd = open(path, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (w->fd < 0) return st_fail(Q8_ERR_ARG, "cannot create %s: %s", path, strerror(errno));
  unsigned char lenb[8];
  uint64_t n = h.size();
  for (int k = 0; k < 8; ++k) lenb[k] = (unsigned char)(n >> (8 * k));
  if (!write_all(w->fd, 0, lenb, 8) || !write_all(w->fd, 8, h.data(), h.size()) ||
      ftruncate(w->fd, (off_t)(data0 + off)) != 0)
    return st_fail(Q8_ERR_ARG, "%s: write failed: %s", path, strerror(errno));
  for (size_t k = 0; k < items.size(); ++k)
    if (items[k].bytes == 0) w->done[(size_t)items[k].caller] = true;
  *out = w.release();
  return Q8_OK;
}

int q8_stw_put(q8_stw *w, int64_t i, const void *data, uint64_t nbytes) {
  if (!w || i < 0 || i >= (int64_t)w->offset.size())
    return st_fail(Q8_ERR_ARG, "q8_stw_put: no tensor %lld", (long long)i);
  if (nbytes != w->size[(size_t)i])
    return st_fail(Q8_ERR_SHAPE, "q8_stw_put: tensor %lld takes %llu bytes, not %llu",
                   (long long)i, (unsigned long long)w->size[(size_t)i],
                   (unsigned long long)nbytes);
  if (nbytes && !data) return st_fail(Q8_ERR_ARG, "q8_stw_put: null data");
  if (!write_all(w->fd, w->offset[(size_t)i], data, nbytes))
    return st_fail(Q8_ERR_ARG, "%s: write failed: %s", w->path.c_str(), strerror(errno));
  w->done[(size_t)i] = true;
  return Q8_OK;
}

int q8_stw_close(q8_stw *w) {
  if (!w) return st_fail(Q8_ERR_ARG, "q8_stw_close: null writer");
  int rc = Q8_OK;
  for (size_t i = 0; i < w->done.size(); ++i)
    if (!w->done[i]) {
      rc = st_fail(Q8_ERR_ARG, "%s: tensor %zu was never written", w->path.c_str(), i);
      break;
    }
  if (w->fd >= 0 && close(w->fd) != 0 && rc == Q8_OK)
    rc = st_fail(Q8_ERR_ARG, "%s: close failed: %s", w->path.c_str(), strerror(errno));
  w->fd = -1;
  delete w;
  return rc;
}

}  // extern "C"
