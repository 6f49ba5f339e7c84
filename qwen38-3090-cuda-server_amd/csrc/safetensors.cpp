// Safetensors reader (host C++) and the checkpoint -> repacked-weights loader.
//
// File format: [u64 little-endian header length][JSON header][tensor data];
// the header maps each tensor name to {"dtype", "shape", "data_offsets":
// [begin, end)} relative to the data section, plus an optional
// "__metadata__" object of strings. Files are mmap'd read-only; views point
// into the mapping (the reference's design, src/loader/safetensors.h:1-7).
//
// qw4_load_ct_fused is the reference's fuse() (src/model/model.cu:103-128):
// the compressed-tensors tensors <prefix>.weight_packed / .weight_scale /
// .weight_zero_point of one or more projections are uploaded and repacked
// side by side into one W4A16 tensor.
#include <dirent.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qwen_safetensors.hpp"
#include "../../include/qwen_w4a16.h"

namespace qwen {

size_t dtype_size(Dtype d) {
  switch (d) {
    case Dtype::BF16: case Dtype::F16: case Dtype::I16: return 2;
    case Dtype::F32: case Dtype::I32: return 4;
    case Dtype::F64: case Dtype::I64: return 8;
    case Dtype::I8: case Dtype::U8: case Dtype::BOOL: case Dtype::F8_E4M3: case Dtype::F8_E5M2:
      return 1;
  }
  return 0;
}

const char* dtype_name(Dtype d) {
  static const char* const names[] = {"BF16", "F16", "F32", "F64", "I8", "U8",
                                      "I16", "I32", "I64", "BOOL", "F8_E4M3", "F8_E5M2"};
  const unsigned i = static_cast<unsigned>(d);
  return i < sizeof(names) / sizeof(names[0]) ? names[i] : "?";
}

namespace {

bool dtype_from_name(const std::string& s, Dtype& d) {
  for (unsigned i = 0; i <= static_cast<unsigned>(Dtype::F8_E5M2); ++i)
    if (s == dtype_name(static_cast<Dtype>(i))) {
      d = static_cast<Dtype>(i);
      return true;
    }
  return false;
}

// ---------------------------------------------------------------- JSON
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  bool integral = false;
  long long i = 0;
  double d = 0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;

  const JVal* member(const char* key) const {
    for (const auto& kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonReader {
 public:
  JsonReader(const char* p, size_t n, const std::string& where)
      : p_(p), e_(p + n), where_(where) {}

  JVal document() {
    JVal v = value(0);
    space();
    if (p_ != e_) fail("trailing characters after the header object");
    return v;
  }

 private:
  const char* p_;
  const char* e_;
  const std::string& where_;

  [[noreturn]] void fail(const char* what) const {
    throw LoaderError(where_ + ": bad safetensors header: " + what);
  }
  void space() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool eat(char c) {
    space();
    if (p_ < e_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) fail("unexpected character");
  }
  bool word(const char* w) {
    const size_t n = std::strlen(w);
    if ((size_t)(e_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }

  static void put_utf8(std::string& out, unsigned cp) {
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

  unsigned hex4() {
    if (e_ - p_ < 4) fail("short \\u escape");
    unsigned v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else fail("bad \\u escape");
    }
    return v;
  }

  std::string string() {
    space();
    if (p_ >= e_ || *p_ != '"') fail("expected a string");
    ++p_;
    std::string out;
    while (true) {
      if (p_ >= e_) fail("unterminated string");
      const char c = *p_++;
      if (c == '"') break;
      if ((unsigned char)c < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= e_) fail("unterminated escape");
      const char x = *p_++;
      switch (x) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {   // surrogate pair
            if (!(e_ - p_ >= 2 && p_[0] == '\\' && p_[1] == 'u')) fail("lone surrogate");
            p_ += 2;
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("unknown escape");
      }
    }
    return out;
  }

  JVal number() {
    const char* s = p_;
    bool integral = true;
    if (p_ < e_ && *p_ == '-') ++p_;
    if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) fail("bad number");
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    if (p_ < e_ && *p_ == '.') {
      integral = false;
      ++p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(s, p_);
    JVal v;
    v.kind = JVal::Num;
    v.integral = integral;
    if (integral) {
      errno = 0;
      v.i = std::strtoll(text.c_str(), nullptr, 10);
      if (errno == ERANGE) fail("integer out of range");
      v.d = (double)v.i;
    } else {
      v.d = std::strtod(text.c_str(), nullptr);
    }
    return v;
  }

  JVal value(int depth) {
    if (depth > 64) fail("nesting too deep");
    space();
    if (p_ >= e_) fail("unexpected end");
    JVal v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JVal::Obj;
      if (eat('}')) return v;
      do {
        std::string k = string();
        expect(':');
        v.o.emplace_back(std::move(k), value(depth + 1));
      } while (eat(','));
      expect('}');
    } else if (c == '[') {
      ++p_;
      v.kind = JVal::Arr;
      if (eat(']')) return v;
      do {
        v.a.push_back(value(depth + 1));
      } while (eat(','));
      expect(']');
    } else if (c == '"') {
      v.kind = JVal::Str;
      v.s = string();
    } else if (word("true")) {
      v.kind = JVal::Bool;
      v.b = true;
    } else if (word("false")) {
      v.kind = JVal::Bool;
    } else if (word("null")) {
      v.kind = JVal::Null;
    } else {
      v = number();
    }
    return v;
  }
};

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = std::strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

}  // namespace

// The open files (read-only mappings) and the index of every tensor in them.
struct SafeTensors::Files {
  struct Region {
    const uint8_t* base = nullptr;
    size_t bytes = 0;
  };
  std::vector<Region> regions;
  std::unordered_map<std::string, TensorView> index;

  void add_file(const std::string& path);
  void release() {
    for (const Region& r : regions)
      if (r.base) munmap(const_cast<uint8_t*>(r.base), r.bytes);
    regions.clear();
    index.clear();
  }
};

SafeTensors::SafeTensors() : files_(new Files) {}
SafeTensors::~SafeTensors() { close(); }

void SafeTensors::close() { files_->release(); }

void SafeTensors::open_files(const std::vector<std::string>& paths) {
  for (const auto& p : paths) files_->add_file(p);
}

void SafeTensors::open_dir(const std::string& dir) {
  DIR* d = opendir(dir.c_str());
  if (!d) throw LoaderError(dir + ": cannot open directory");
  std::vector<std::string> found;
  while (dirent* ent = readdir(d)) {
    const std::string name = ent->d_name;
    if (ends_with(name, ".safetensors")) found.push_back(dir + "/" + name);
  }
  closedir(d);
  if (found.empty()) throw LoaderError(dir + ": no *.safetensors files");
  std::sort(found.begin(), found.end());
  open_files(found);
}

void SafeTensors::Files::add_file(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw LoaderError(path + ": cannot open");
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    ::close(fd);
    throw LoaderError(path + ": not a safetensors file (too short)");
  }
  const size_t len = (size_t)st.st_size;
  void* addr = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (addr == MAP_FAILED) throw LoaderError(path + ": mmap failed");
  const uint8_t* base = static_cast<const uint8_t*>(addr);
  regions.push_back({base, len});
  const int shard = (int)regions.size() - 1;
  uint64_t hlen = 0;
  for (int k = 0; k < 8; ++k) hlen |= (uint64_t)base[k] << (8 * k);
  if (hlen > len - 8 || hlen > (100ull << 20))
    throw LoaderError(path + ": header length " + std::to_string(hlen) + " exceeds the file");
  const size_t data0 = 8 + (size_t)hlen;
  const size_t data_len = len - data0;
  const JVal hdr = JsonReader(reinterpret_cast<const char*>(base + 8), (size_t)hlen, path).document();
  if (hdr.kind != JVal::Obj) throw LoaderError(path + ": header is not an object");

  for (const auto& kv : hdr.o) {
    if (kv.first == "__metadata__") continue;
    const JVal& t = kv.second;
    const JVal* dt = t.member("dtype");
    const JVal* sh = t.member("shape");
    const JVal* off = t.member("data_offsets");
    if (t.kind != JVal::Obj || !dt || dt->kind != JVal::Str || !sh || sh->kind != JVal::Arr ||
        !off || off->kind != JVal::Arr || off->a.size() != 2)
      throw LoaderError(path + ": malformed entry for tensor '" + kv.first + "'");
    TensorView v;
    if (!dtype_from_name(dt->s, v.dtype))
      throw LoaderError(path + ": tensor '" + kv.first + "' has unsupported dtype " + dt->s);
    for (const JVal& e : sh->a) {
      if (e.kind != JVal::Num || !e.integral || e.i < 0)
        throw LoaderError(path + ": tensor '" + kv.first + "' has a bad shape");
      v.shape.push_back(e.i);
    }
    const JVal& b = off->a[0];
    const JVal& e = off->a[1];
    if (b.kind != JVal::Num || e.kind != JVal::Num || !b.integral || !e.integral || b.i < 0 ||
        e.i < b.i || (uint64_t)e.i > data_len)
      throw LoaderError(path + ": tensor '" + kv.first + "' lies outside the file");
    v.nbytes = (size_t)(e.i - b.i);
    // numel * size must equal the byte range (guarding the product against overflow)
    unsigned __int128 want = dtype_size(v.dtype);
    for (int64_t dim : v.shape) want *= (unsigned __int128)dim;
    if (want != (unsigned __int128)v.nbytes)
      throw LoaderError(path + ": tensor '" + kv.first + "' size does not match its shape");
    v.data = base + data0 + (size_t)b.i;
    v.shard = shard;
    if (!index.emplace(kv.first, std::move(v)).second)
      throw LoaderError(path + ": tensor '" + kv.first + "' appears twice");
  }
}

bool SafeTensors::has(const std::string& name) const { return files_->index.count(name) != 0; }

const std::unordered_map<std::string, TensorView>& SafeTensors::all() const {
  return files_->index;
}

size_t SafeTensors::size() const { return files_->index.size(); }

const TensorView& SafeTensors::get(const std::string& name) const {
  const TensorView* v = find(name);
  if (!v) throw LoaderError("tensor not found: " + name);
  return *v;
}

const TensorView* SafeTensors::find(const std::string& name) const {
  auto it = files_->index.find(name);
  return it == files_->index.end() ? nullptr : &it->second;
}

size_t SafeTensors::mapped_bytes() const {
  size_t n = 0;
  for (const auto& r : files_->regions) n += r.bytes;
  return n;
}

size_t SafeTensors::bytes_with_prefix(const std::string& prefix) const {
  size_t n = 0;
  for (const auto& kv : files_->index)
    if (kv.first.compare(0, prefix.size(), prefix) == 0) n += kv.second.nbytes;
  return n;
}

}  // namespace qwen

// ------------------------------------------------------------------ C-ABI
namespace qw4 {
void set_hip_error(int e);
}

struct qw4_st {
  qwen::SafeTensors st;
};

namespace {
thread_local std::string g_st_error;

int st_fail(const std::string& msg, int code) {
  g_st_error = msg;
  return code;
}

void fill(const qwen::TensorView& v, qw4_st_tensor* out) {
  std::memset(out, 0, sizeof(*out));
  out->dtype = (int32_t)v.dtype;
  out->ndim = (int32_t)std::min<size_t>(v.shape.size(), 8);
  for (int k = 0; k < out->ndim; ++k) out->shape[k] = v.shape[k];
  out->data = v.data;
  out->nbytes = v.nbytes;
}
}  // namespace

extern "C" {

const char* qw4_st_last_error(void) { return g_st_error.c_str(); }

int qw4_st_open(qw4_st** st, const char* const* paths, int npaths) {
  if (!st || !paths || npaths <= 0) return QW4_ERR_NULL;
  *st = nullptr;
  qw4_st* h = new qw4_st;
  try {
    std::vector<std::string> v;
    for (int k = 0; k < npaths; ++k) {
      if (!paths[k]) {
        delete h;
        return QW4_ERR_NULL;
      }
      v.emplace_back(paths[k]);
    }
    h->st.open_files(v);
  } catch (const std::exception& e) {
    delete h;
    return st_fail(e.what(), QW4_ERR_IO);
  }
  *st = h;
  return QW4_OK;
}

int qw4_st_open_dir(qw4_st** st, const char* dir) {
  if (!st || !dir) return QW4_ERR_NULL;
  *st = nullptr;
  qw4_st* h = new qw4_st;
  try {
    h->st.open_dir(dir);
  } catch (const std::exception& e) {
    delete h;
    return st_fail(e.what(), QW4_ERR_IO);
  }
  *st = h;
  return QW4_OK;
}

int qw4_st_close(qw4_st* st) {
  delete st;
  return QW4_OK;
}

int qw4_st_count(const qw4_st* st) { return st ? (int)st->st.size() : 0; }

int qw4_st_find(const qw4_st* st, const char* name, qw4_st_tensor* out) {
  if (!st || !name || !out) return QW4_ERR_NULL;
  const qwen::TensorView* v = st->st.find(name);
  if (!v) return st_fail(std::string("tensor not found: ") + name, QW4_ERR_NOTFOUND);
  fill(*v, out);
  return QW4_OK;
}

int qw4_load_ct_fused(qw4_weights* w, const qw4_st* st, const char* const* prefixes,
                      int nparts, int in_f, int group_size, void* stream) {
  if (!w || !st || !prefixes || nparts <= 0) return QW4_ERR_NULL;
  if (group_size != 128) return QW4_ERR_GROUP;
  if (in_f <= 0 || in_f % group_size) return QW4_ERR_SHAPE;
  const int G = in_f / group_size;
  struct Part {
    const qwen::TensorView *p, *s, *z;
    int rows;
  };
  std::vector<Part> parts;
  long long total = 0;
  for (int k = 0; k < nparts; ++k) {
    if (!prefixes[k]) return QW4_ERR_NULL;
    const std::string b = prefixes[k];
    Part pt;
    pt.p = st->st.find(b + ".weight_packed");
    pt.s = st->st.find(b + ".weight_scale");
    pt.z = st->st.find(b + ".weight_zero_point");
    if (!pt.p || !pt.s || !pt.z)
      return st_fail(b + ": weight_packed / weight_scale / weight_zero_point missing",
                     QW4_ERR_NOTFOUND);
    // compressed-tensors pack-quantized layout (src/loader/w4a16_unpack.h:1-18)
    if (pt.p->dtype != qwen::Dtype::I32 || pt.s->dtype != qwen::Dtype::BF16 ||
        pt.z->dtype != qwen::Dtype::I32 || pt.p->shape.size() != 2 || pt.s->shape.size() != 2 ||
        pt.z->shape.size() != 2)
      return st_fail(b + ": expected I32 weight_packed, BF16 weight_scale, I32 weight_zero_point",
                     QW4_ERR_SHAPE);
    pt.rows = (int)pt.s->shape[0];
    if (pt.p->shape[0] != pt.rows || pt.p->shape[1] != in_f / 8 || pt.s->shape[1] != G ||
        pt.rows % 8 || pt.z->shape[0] != pt.rows / 8 || pt.z->shape[1] != G)
      return st_fail(b + ": tensor shapes do not match in_f " + std::to_string(in_f),
                     QW4_ERR_SHAPE);
    total += pt.rows;
    parts.push_back(pt);
  }
  if (total > (1 << 30)) return QW4_ERR_SHAPE;
  int rc = qw4_weights_alloc(w, (int)total, in_f, group_size, stream);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  int off = 0;
  for (const Part& pt : parts) {
    void *dp = nullptr, *ds = nullptr, *dz = nullptr;
    hipError_t e = hipMalloc(&dp, pt.p->nbytes);
    if (e == hipSuccess) e = hipMalloc(&ds, pt.s->nbytes);
    if (e == hipSuccess) e = hipMalloc(&dz, pt.z->nbytes);
    if (e == hipSuccess) e = hipMemcpyAsync(dp, pt.p->data, pt.p->nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(ds, pt.s->data, pt.s->nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(dz, pt.z->data, pt.z->nbytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
      rc = qw4_repack_ct_into(w, off, static_cast<const uint32_t*>(dp),
                              static_cast<const uint16_t*>(ds), static_cast<const uint32_t*>(dz),
                              pt.rows, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s);   // the sources are freed next
    if (dp) (void)hipFree(dp);
    if (ds) (void)hipFree(ds);
    if (dz) (void)hipFree(dz);
    if (e != hipSuccess || rc != QW4_OK) {
      (void)hipGetLastError();
      qw4_weights_free(w);
      if (rc != QW4_OK) return rc;
      qw4::set_hip_error((int)e);
      return st_fail(hipGetErrorString(e), QW4_ERR_HIP);
    }
    off += pt.rows;
  }
  return QW4_OK;
}

}  // extern "C"
