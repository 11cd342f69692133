// shards.hip -- safetensors checkpoint index (Shards, safetensors.rs:215-488) and the MXFP4 expert
// loader into the HBM pool (ExpertCache::ensure_loaded with ExpertNaming::{Qwen38Mxfp4,
// KimiK3Mxfp4}, expert_cache.rs:93-208,1227-1256). Host code only.
//
// A shard file is an 8-byte little-endian header length, the JSON header
//   { name: {"dtype": str, "shape": [u64...], "data_offsets": [start, end]}, "__metadata__": {...} }
// and the data region; offsets are relative to the data region's start. open() indexes every
// *.safetensors file of a directory in file-name order, with the reference's checks (header no
// longer than the file, two u64 offsets, end >= start, end inside the file, a known dtype).
//
// The loader reads each expert's packed and scale tensors verbatim (the on-disk MXFP4 layout is the
// kernels' layout) into a pool slot, validating byte lengths as mxfp4_from_raw does, through a
// pinned double-buffered staging ring (pread into one buffer while the other is copied to HBM).
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "rbt_internal.h"

namespace {

thread_local std::string g_shards_err;

int shards_fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_shards_err = buf;
  return code;
}

// ---- a small JSON reader: enough for safetensors headers --------------------------------------
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool is_u64 = false;  // a non-negative integer literal that fits u64 (serde_json's as_u64)
  uint64_t u = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
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
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
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
    for (int i = 0; i < 4; i++) {
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
    p++;
    while (p < end && *p != '"') {
      if ((unsigned char)*p < 0x20) return fail("control character in a string");
      if (*p != '\\') {
        o += *p++;
        continue;
      }
      if (++p >= end) return fail("truncated escape");
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
          uint32_t v;
          if (!hex4(v)) return false;
          if (v >= 0xD800 && v < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            uint32_t lo;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo > 0xDFFF) return fail("bad surrogate pair");
            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, v);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    p++;
    return true;
  }
  bool num(JVal &v) {
    const char *s = p;
    if (p < end && *p == '-') p++;
    const char *ds = p;
    while (p < end && *p >= '0' && *p <= '9') p++;
    if (p == ds) return fail("bad number");
    bool integer = true;
    if (p < end && *p == '.') {
      integer = false;
      p++;
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      integer = false;
      p++;
      if (p < end && (*p == '+' || *p == '-')) p++;
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    v.kind = JVal::NUM;
    if (integer && *s != '-') {
      uint64_t u = 0;
      bool ok = true;
      for (const char *q = ds; q < p; q++) {
        const uint64_t d = (uint64_t)(*q - '0');
        if (u > (UINT64_MAX - d) / 10) {
          ok = false;
          break;
        }
        u = u * 10 + d;
      }
      v.is_u64 = ok;
      v.u = u;
    }
    return true;
  }
  bool lit(const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(end - p) < n || strncmp(p, w, n) != 0) return fail("bad literal");
    p += n;
    return true;
  }
  bool value(JVal &v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end of header");
    bool ok;
    if (*p == '{') {
      v.kind = JVal::OBJ;
      p++;
      ws();
      ok = true;
      if (p < end && *p == '}') {
        p++;
      } else {
        for (;;) {
          ws();
          std::string k;
          if (!str(k)) {
            ok = false;
            break;
          }
          ws();
          if (p >= end || *p != ':') {
            ok = fail("expected ':'");
            break;
          }
          p++;
          JVal x;
          if (!value(x)) {
            ok = false;
            break;
          }
          v.obj.emplace_back(std::move(k), std::move(x));
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == '}') {
            p++;
            break;
          }
          ok = fail("expected ',' or '}'");
          break;
        }
      }
    } else if (*p == '[') {
      v.kind = JVal::ARR;
      p++;
      ws();
      ok = true;
      if (p < end && *p == ']') {
        p++;
      } else {
        for (;;) {
          JVal x;
          if (!value(x)) {
            ok = false;
            break;
          }
          v.arr.push_back(std::move(x));
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == ']') {
            p++;
            break;
          }
          ok = fail("expected ',' or ']'");
          break;
        }
      }
    } else if (*p == '"') {
      v.kind = JVal::STR;
      ok = str(v.s);
    } else if (*p == 't') {
      v.kind = JVal::BOOL;
      ok = lit("true");
    } else if (*p == 'f') {
      v.kind = JVal::BOOL;
      ok = lit("false");
    } else if (*p == 'n') {
      ok = lit("null");
    } else {
      ok = num(v);
    }
    depth--;
    return ok;
  }
};

bool known_dtype(const std::string &d) {
  // DType::from_str (safetensors.rs:42-51)
  return d == "BF16" || d == "F16" || d == "F32" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "float8_e4m3fn";
}

bool pread_all(int fd, void *dst, size_t n, uint64_t off) {
  uint8_t *d = (uint8_t *)dst;
  while (n) {
    const ssize_t r = pread(fd, d, n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

}  // namespace

struct rbt_shards {
  std::vector<std::string> paths;
  std::vector<int> fds;
  std::vector<rbt_tensor_info> tensors;
  std::vector<std::string> names;
  std::unordered_map<std::string, size_t> index;
  ~rbt_shards() {
    for (int fd : fds)
      if (fd >= 0) close(fd);
  }
};

extern "C" {

const char *rbt_shards_last_error(void) { return g_shards_err.c_str(); }

int rbt_shards_open(const char *dir, rbt_shards **out) {
  if (!out) return shards_fail(RBT_E_INVALID, "null out");
  *out = nullptr;
  if (!dir) return shards_fail(RBT_E_INVALID, "null dir");
  DIR *d = opendir(dir);
  if (!d) return shards_fail(RBT_E_IO, "io: cannot open directory %s: %s", dir, strerror(errno));
  std::vector<std::string> files;
  while (struct dirent *e = readdir(d)) {
    const std::string n = e->d_name;
    if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0) files.push_back(n);
  }
  closedir(d);
  std::sort(files.begin(), files.end());  // file-name order (safetensors.rs:262)
  auto sh = new rbt_shards();
  for (const std::string &f : files) {
    const std::string path = std::string(dir) + "/" + f;
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
      delete sh;
      return shards_fail(RBT_E_IO, "io: %s: %s", path.c_str(), strerror(errno));
    }
    sh->fds.push_back(fd);
    sh->paths.push_back(path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
      delete sh;
      return shards_fail(RBT_E_IO, "io: %s: %s", path.c_str(), strerror(errno));
    }
    const uint64_t file_len = (uint64_t)st.st_size;
    uint8_t hb[8];
    if (!pread_all(fd, hb, 8, 0)) {
      delete sh;
      return shards_fail(RBT_E_IO, "io: %s: cannot read the header length", path.c_str());
    }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | hb[i];
    if (hlen > file_len) {
      delete sh;
      return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: header length %llu exceeds file size %llu",
                         path.c_str(), (unsigned long long)hlen, (unsigned long long)file_len);
    }
    std::string hdr((size_t)hlen, '\0');
    if (hlen && !pread_all(fd, &hdr[0], (size_t)hlen, 8)) {
      delete sh;
      return shards_fail(RBT_E_IO, "io: %s: cannot read the header", path.c_str());
    }
    JParser jp{hdr.data(), hdr.data() + hdr.size()};
    JVal root;
    bool ok = jp.value(root);
    if (ok) {
      jp.ws();
      if (jp.p != jp.end) ok = jp.fail("trailing characters");
    }
    if (!ok) {
      delete sh;
      return shards_fail(RBT_E_FORMAT, "header json: %s: %s", path.c_str(), jp.err.c_str());
    }
    if (root.kind != JVal::OBJ) {
      delete sh;
      return shards_fail(RBT_E_FORMAT, "bad safetensors header: top-level value is not an object");
    }
    const uint64_t data_start = 8 + hlen;
    const int file_index = (int)sh->fds.size() - 1;
    for (const auto &kv : root.obj) {
      const std::string &name = kv.first;
      const JVal &m = kv.second;
      if (name == "__metadata__") continue;
      const JVal *dt = m.get("dtype");
      if (!dt || dt->kind != JVal::STR) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: missing dtype", name.c_str());
      }
      if (!known_dtype(dt->s)) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "unknown dtype: %s", dt->s.c_str());
      }
      const JVal *off = m.get("data_offsets");
      if (!off || off->kind != JVal::ARR) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: missing data_offsets", name.c_str());
      }
      if (off->arr.size() != 2) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: data_offsets must have 2 elements",
                           name.c_str());
      }
      if (!off->arr[0].is_u64 || !off->arr[1].is_u64) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: data_offsets[%d] is not a u64", name.c_str(),
                           off->arr[0].is_u64 ? 1 : 0);
      }
      const uint64_t a0 = off->arr[0].u, b0 = off->arr[1].u;
      if (b0 < a0) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: data_offsets end %llu precedes start %llu",
                           name.c_str(), (unsigned long long)b0, (unsigned long long)a0);
      }
      if (data_start > file_len || b0 > file_len - data_start) {
        delete sh;
        return shards_fail(RBT_E_FORMAT,
                           "bad safetensors header: %s: data_offsets end %llu extends past end of file (%llu bytes "
                           "available)",
                           name.c_str(), (unsigned long long)b0,
                           (unsigned long long)(data_start > file_len ? 0 : file_len - data_start));
      }
      const JVal *shp = m.get("shape");
      if (!shp || shp->kind != JVal::ARR) {
        delete sh;
        return shards_fail(RBT_E_FORMAT, "bad safetensors header: %s: missing shape", name.c_str());
      }
      rbt_tensor_info ti{};
      ti.file_index = file_index;
      ti.offset = data_start + a0;
      ti.nbytes = b0 - a0;
      snprintf(ti.dtype, sizeof ti.dtype, "%s", dt->s.c_str());
      // non-u64 shape entries are dropped, as the reference's filter_map(as_u64) does
      for (const JVal &e : shp->arr)
        if (e.is_u64 && ti.ndim < (int32_t)(sizeof ti.shape / sizeof ti.shape[0])) ti.shape[ti.ndim++] = e.u;
      // a later shard's tensor of the same name wins (HashMap::insert)
      auto it = sh->index.find(name);
      if (it != sh->index.end()) {
        sh->tensors[it->second] = ti;
      } else {
        sh->index.emplace(name, sh->tensors.size());
        sh->tensors.push_back(ti);
        sh->names.push_back(name);
      }
    }
  }
  *out = sh;
  return RBT_OK;
}

void rbt_shards_close(rbt_shards *sh) { delete sh; }

size_t rbt_shards_count(const rbt_shards *sh) { return sh ? sh->tensors.size() : 0; }

int rbt_shards_find(const rbt_shards *sh, const char *name, rbt_tensor_info *info) {
  if (!sh || !name) return shards_fail(RBT_E_INVALID, "null shards or name");
  auto it = sh->index.find(name);
  if (it == sh->index.end()) return shards_fail(RBT_E_NOT_FOUND, "missing tensor: %s", name);
  if (info) *info = sh->tensors[it->second];
  return RBT_OK;
}

int rbt_shards_read(const rbt_shards *sh, const char *name, void *dst, size_t cap) {
  rbt_tensor_info ti;
  const int rc = rbt_shards_find(sh, name, &ti);
  if (rc != RBT_OK) return rc;
  if (!dst) return shards_fail(RBT_E_INVALID, "null dst");
  if (cap < ti.nbytes)
    return shards_fail(RBT_E_SHAPE, "%s: %llu bytes do not fit in %zu", name, (unsigned long long)ti.nbytes, cap);
  if (!pread_all(sh->fds[ti.file_index], dst, (size_t)ti.nbytes, ti.offset))
    return shards_fail(RBT_E_IO, "io: %s: short read", name);
  return RBT_OK;
}

int rbt_shards_read_range(const rbt_shards *sh, const char *name, uint64_t offset, void *dst, size_t n) {
  rbt_tensor_info ti;
  const int rc = rbt_shards_find(sh, name, &ti);
  if (rc != RBT_OK) return rc;
  if (!dst && n) return shards_fail(RBT_E_INVALID, "null dst");
  if (offset > ti.nbytes || n > ti.nbytes - offset)
    return shards_fail(RBT_E_SHAPE, "%s: range [%llu, +%zu) outside its %llu bytes", name, (unsigned long long)offset,
                       n, (unsigned long long)ti.nbytes);
  if (n && !pread_all(sh->fds[ti.file_index], dst, n, ti.offset + offset))
    return shards_fail(RBT_E_IO, "io: %s: short read", name);
  return RBT_OK;
}

}  // extern "C"

// ---- the MXFP4 expert loader ---------------------------------------------------------------------
namespace rbt {

// ExpertNaming::tensor_specs for the two MXFP4 namings (expert_cache.rs:176-208), with
// packed_suffix (:154-159): base names and shapes in read order gate, up, down.
int mxfp4_specs(int naming, uint32_t layer, uint32_t eid, size_t hidden, size_t moe_inter, std::string base[3],
                size_t rows[3], size_t cols[3], const char **packed_suffix) {
  const char *mats[3];
  std::string pre;
  if (naming == RBT_NAMING_QWEN38_MXFP4) {
    pre = "model.layers." + std::to_string(layer) + ".mlp.experts." + std::to_string(eid) + ".";
    mats[0] = "gate_proj";
    mats[1] = "up_proj";
    mats[2] = "down_proj";
    *packed_suffix = ".weight";
  } else if (naming == RBT_NAMING_KIMI_K3_MXFP4) {
    pre = "language_model.model.layers." + std::to_string(layer) + ".block_sparse_moe.experts." + std::to_string(eid) + ".";
    mats[0] = "w1";
    mats[1] = "w3";
    mats[2] = "w2";
    *packed_suffix = ".weight_packed";
  } else {
    return RBT_E_INVALID;
  }
  for (int m = 0; m < 3; m++) {
    base[m] = pre + mats[m];
    rows[m] = m < 2 ? moe_inter : hidden;
    cols[m] = m < 2 ? hidden : moe_inter;
  }
  return RBT_OK;
}

}  // namespace rbt
