// GGUF reader and device weight upload (include/ferrum_gguf.h).
//
// The decoder restates Ferrum's crates/gguf/src/parse.rs: the same reads in the same
// order, each count bounded by the bytes still left before anything is allocated for
// it, and the same FerrumError::Gguf messages. The file is memory-mapped read-only and
// tensor bytes are never copied on the host except through the upload's pinned
// staging buffers.
#include <errno.h>
#include <fcntl.h>
#include <sched.h>
#include <hip/hip_runtime_api.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <string>
#include <system_error>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/ferrum_gguf.h"
#include "fkv_internal.h"

namespace {

struct GgufError {
  std::string msg;
};

[[noreturn]] void bad(const std::string& msg) { throw GgufError{msg}; }

// Metadata value tree (MetadataValue, crates/core-types/src/metadata.rs).
struct Value {
  uint32_t type = 0;
  uint32_t elem_type = 0;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  std::string str;
  std::vector<Value> arr;
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t ggml_type = 0;
  uint64_t data_offset = 0;
  uint64_t nbytes = 0;
};

constexpr uint64_t kMinKvBytes = 13;          // parse.rs:24: key len + type + smallest value
constexpr uint64_t kMinTensorInfoBytes = 24;  // parse.rs:28
constexpr uint32_t kMaxArrayDepth = 64;       // parse.rs:32

// (ggml type id, elements a block, bytes a block): crates/gguf/src/layout.rs:12-45.
struct Layout {
  uint32_t id;
  uint64_t block, bytes;
};
constexpr Layout kLayouts[] = {
    {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},
    {7, 32, 24},    {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110},
    {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {16, 256, 66},
    {17, 256, 74},  {18, 256, 98},  {19, 256, 50},  {20, 32, 18},   {21, 256, 110},
    {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},     {26, 1, 4},
    {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {34, 256, 54},
    {35, 256, 66},  {39, 32, 17},
};

// ggml_type_name (crates/core-types/src/dtype.rs:47-85).
const char* ggml_type_name(uint32_t id) {
  switch (id) {
    case 0: return "f32";     case 1: return "f16";     case 2: return "q4_0";
    case 3: return "q4_1";    case 4: return "q4_2";    case 5: return "q4_3";
    case 6: return "q5_0";    case 7: return "q5_1";    case 8: return "q8_0";
    case 9: return "q8_1";    case 10: return "q2_K";   case 11: return "q3_K";
    case 12: return "q4_K";   case 13: return "q5_K";   case 14: return "q6_K";
    case 15: return "q8_K";   case 16: return "iq2_xxs"; case 17: return "iq2_xs";
    case 18: return "iq3_xxs"; case 19: return "iq1_s";  case 20: return "iq4_nl";
    case 21: return "iq3_s";  case 22: return "iq2_s";  case 23: return "iq4_xs";
    case 24: return "i8";     case 25: return "i16";    case 26: return "i32";
    case 27: return "i64";    case 28: return "f64";    case 29: return "iq1_m";
    case 30: return "bf16";   case 34: return "tq1_0";  case 35: return "tq2_0";
    case 39: return "mxfp4";
    default: return nullptr;
  }
}

bool mul_ovf(uint64_t a, uint64_t b, uint64_t* r) { return __builtin_mul_overflow(a, b, r); }

// bound_count (parse.rs:368-379): count * min_elem must fit in what is left.
uint64_t bound_count(uint64_t count, uint64_t min_elem, uint64_t remaining) {
  if (min_elem == 0) bad("element size is zero");
  if (count > remaining / min_elem) bad("count exceeds remaining bytes");
  return count;
}

// Rust's str::from_utf8: well-formed UTF-8 only (no overlong forms, no surrogates,
// nothing past U+10FFFF).
bool valid_utf8(const uint8_t* p, uint64_t n) {
  uint64_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) { i++; continue; }
    uint64_t len;
    uint8_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) len = 2;
    else if (c == 0xE0) { len = 3; lo = 0xA0; }
    else if ((c >= 0xE1 && c <= 0xEC) || c == 0xEE || c == 0xEF) len = 3;
    else if (c == 0xED) { len = 3; hi = 0x9F; }
    else if (c == 0xF0) { len = 4; lo = 0x90; }
    else if (c >= 0xF1 && c <= 0xF3) len = 4;
    else if (c == 0xF4) { len = 4; hi = 0x8F; }
    else return false;
    if (n - i < len) return false;
    if (p[i + 1] < lo || p[i + 1] > hi) return false;
    for (uint64_t k = 2; k < len; k++)
      if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
    i += len;
  }
  return true;
}

struct Reader {
  const uint8_t* data;
  uint64_t len;
  uint64_t pos = 0;
  uint64_t remaining() const { return len > pos ? len - pos : 0; }
  const uint8_t* read_exact(uint64_t n) {
    if (n > len - pos) bad("unexpected end of gguf file");
    const uint8_t* p = data + pos;
    pos += n;
    return p;
  }
  template <typename T>
  T read_le() {
    T v;
    memcpy(&v, read_exact(sizeof(T)), sizeof(T));  // the host is little-endian
    return v;
  }
  bool read_bool() {
    const uint8_t b = read_le<uint8_t>();
    if (b > 1) bad("invalid bool byte");
    return b == 1;
  }
  std::string read_string() {
    const uint64_t n = bound_count(read_le<uint64_t>(), 1, remaining());
    const uint8_t* p = read_exact(n);
    if (!valid_utf8(p, n)) bad("invalid utf-8");
    return std::string((const char*)p, (size_t)n);
  }
};

bool known_meta_type(uint32_t t) { return t <= 12; }

uint64_t min_value_bytes(uint32_t t) {  // parse.rs:325-338
  switch (t) {
    case FKV_GGUF_UINT8: case FKV_GGUF_INT8: case FKV_GGUF_BOOL: return 1;
    case FKV_GGUF_UINT16: case FKV_GGUF_INT16: return 2;
    case FKV_GGUF_UINT32: case FKV_GGUF_INT32: case FKV_GGUF_FLOAT32: return 4;
    case FKV_GGUF_ARRAY: return 12;
    default: return 8;  // u64, i64, f64, string
  }
}

Value read_value(Reader& r, uint32_t type, uint32_t depth);

Value read_array(Reader& r, uint32_t depth) {  // parse.rs:306-323
  if (depth >= kMaxArrayDepth) bad("metadata array nested too deeply");
  const uint32_t elem = r.read_le<uint32_t>();
  if (!known_meta_type(elem)) bad("unknown metadata type " + std::to_string(elem));
  const uint64_t n = bound_count(r.read_le<uint64_t>(), min_value_bytes(elem), r.remaining());
  Value v;
  v.type = FKV_GGUF_ARRAY;
  v.elem_type = elem;
  v.arr.reserve((size_t)n);
  for (uint64_t k = 0; k < n; k++) v.arr.push_back(read_value(r, elem, depth + 1));
  return v;
}

Value read_value(Reader& r, uint32_t type, uint32_t depth) {  // parse.rs:285-304
  Value v;
  v.type = type;
  switch (type) {
    case FKV_GGUF_UINT8: v.u = r.read_le<uint8_t>(); break;
    case FKV_GGUF_INT8: v.i = r.read_le<int8_t>(); break;
    case FKV_GGUF_UINT16: v.u = r.read_le<uint16_t>(); break;
    case FKV_GGUF_INT16: v.i = r.read_le<int16_t>(); break;
    case FKV_GGUF_UINT32: v.u = r.read_le<uint32_t>(); break;
    case FKV_GGUF_INT32: v.i = r.read_le<int32_t>(); break;
    case FKV_GGUF_FLOAT32: v.f = r.read_le<float>(); break;
    case FKV_GGUF_BOOL: v.u = r.read_bool() ? 1u : 0u; break;
    case FKV_GGUF_STRING: v.str = r.read_string(); break;
    case FKV_GGUF_UINT64: v.u = r.read_le<uint64_t>(); break;
    case FKV_GGUF_INT64: v.i = r.read_le<int64_t>(); break;
    case FKV_GGUF_FLOAT64: v.f = r.read_le<double>(); break;
    default: return read_array(r, depth);  // FKV_GGUF_ARRAY
  }
  return v;
}

uint64_t validate_alignment(uint64_t a) {  // parse.rs:351-356
  if (a == 0 || a % 8 != 0) bad("alignment must be a non-zero multiple of 8");
  return a;
}

// shape_elements (dtype.rs:87-103).
uint64_t shape_elements(const std::vector<uint64_t>& shape) {
  if (shape.empty() || shape.size() > 4) bad("tensor rank must be from 1 to 4 inclusive");
  uint64_t n = 1;
  for (uint64_t d : shape) {
    if (d == 0) bad("tensor dimension is zero");
    if (mul_ovf(n, d, &n)) bad("tensor element count overflow");
  }
  return n;
}

// stored_nbytes (layout.rs:57-72).
uint64_t stored_nbytes(uint32_t type, uint64_t elements) {
  const Layout* lay = nullptr;
  for (const Layout& l : kLayouts)
    if (l.id == type) lay = &l;
  if (!lay) bad("ggml type " + std::to_string(type) + " has no stored size");
  if (lay->block == 0 || elements % lay->block != 0)
    bad("tensor element count is not a multiple of the block size");
  uint64_t n;
  if (mul_ovf(elements / lay->block, lay->bytes, &n)) bad("tensor size overflow");
  return n;
}

// TensorDesc::try_new (source.rs:25-56) for the compute types F32, F16, Q8_0; every
// other type only needs a non-zero size.
void check_tensor_desc(const Tensor& t) {
  const uint64_t elements = shape_elements(t.shape);
  if (t.ggml_type == 0 || t.ggml_type == 1 || t.ggml_type == 8) {
    uint64_t expected;
    if (t.ggml_type == 8) {
      if (elements % 32 != 0) bad("q8_0 element count is not a multiple of 32");
      if (mul_ovf(elements / 32, 34, &expected)) bad("tensor size overflow");
    } else if (mul_ovf(elements, t.ggml_type == 0 ? 4 : 2, &expected)) {
      bad("tensor size overflow");
    }
    if (expected != t.nbytes)
      bad("tensor " + t.name + " byte count " + std::to_string(t.nbytes) +
          " does not match layout " + std::to_string(expected));
  } else if (t.nbytes == 0) {
    bad("unsupported tensor has zero bytes");
  }
}

}  // namespace

struct fkv_gguf {
  int fd = -1;
  const uint8_t* map = nullptr;
  uint64_t len = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_start = 0;
  std::unordered_map<std::string, Value> metadata;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, uint64_t> by_name;
  ~fkv_gguf() {
    if (map && len) munmap((void*)map, len);
    if (fd >= 0) close(fd);
  }
};

namespace {

// parse_view (parse.rs:100-181).
void parse(fkv_gguf* g) {
  Reader r{g->map, g->len};
  static const uint8_t kMagic[4] = {0x47, 0x47, 0x55, 0x46};
  if (memcmp(r.read_exact(4), kMagic, 4) != 0) bad("bad gguf magic");
  g->version = r.read_le<uint32_t>();
  if (g->version != 2 && g->version != 3)
    bad("unsupported gguf version " + std::to_string(g->version));
  const uint64_t tensor_count = r.read_le<uint64_t>();
  const uint64_t kv_count = r.read_le<uint64_t>();

  const uint64_t n_kv = bound_count(kv_count, kMinKvBytes, r.remaining());
  for (uint64_t k = 0; k < n_kv; k++) {  // read_metadata, parse.rs:183-205
    std::string key = r.read_string();
    const uint32_t type = r.read_le<uint32_t>();
    if (!known_meta_type(type)) bad("unknown metadata type " + std::to_string(type));
    Value v = read_value(r, type, 0);
    if (g->metadata.count(key)) bad("duplicate metadata key " + key);
    g->metadata.emplace(std::move(key), std::move(v));
  }
  // alignment_of (parse.rs:340-349)
  auto al = g->metadata.find("general.alignment");
  if (al == g->metadata.end()) g->alignment = 32;
  else if (al->second.type == FKV_GGUF_UINT32 || al->second.type == FKV_GGUF_UINT64)
    g->alignment = validate_alignment(al->second.u);
  else bad("general.alignment must be uint32 or uint64");

  const uint64_t n_t = bound_count(tensor_count, kMinTensorInfoBytes, r.remaining());
  std::unordered_set<std::string> seen;
  for (uint64_t k = 0; k < n_t; k++) {  // read_tensor_info, parse.rs:224-258
    Tensor t;
    t.name = r.read_string();
    if (!seen.insert(t.name).second) bad("duplicate tensor name " + t.name);
    const uint32_t n_dims = r.read_le<uint32_t>();
    if (n_dims == 0 || n_dims > 4) bad("tensor rank must be from 1 to 4 inclusive");
    bound_count(n_dims, 8, r.remaining());
    for (uint32_t d = 0; d < n_dims; d++) t.shape.push_back(r.read_le<uint64_t>());
    t.ggml_type = r.read_le<uint32_t>();
    t.data_offset = r.read_le<uint64_t>();
    t.nbytes = stored_nbytes(t.ggml_type, shape_elements(t.shape));
    g->tensors.push_back(std::move(t));
  }

  const uint64_t info_end = r.pos;  // align_offset, parse.rs:358-366
  const uint64_t a = validate_alignment(g->alignment);
  const uint64_t pad = (a - info_end % a) % a;
  if (info_end > UINT64_MAX - pad) bad("aligned offset overflows");
  g->data_start = info_end + pad;
  if (g->data_start > g->len) bad("alignment padding exceeds file");
  for (uint64_t p = info_end; p < g->data_start; p++)
    if (g->map[p] != 0) bad("alignment padding is not zero");

  const uint64_t data_len = g->len - g->data_start;
  for (const Tensor& t : g->tensors) {  // parse.rs:141-171
    if (t.data_offset % g->alignment != 0) bad("tensor " + t.name + " data_offset is not aligned");
    if (t.data_offset > UINT64_MAX - t.nbytes) bad("tensor " + t.name + " data range overflows");
    if (t.data_offset + t.nbytes > data_len) bad("tensor " + t.name + " extends past end of file");
    check_tensor_desc(t);
  }
  for (uint64_t k = 0; k < g->tensors.size(); k++) g->by_name.emplace(g->tensors[k].name, k);
}

// io::Error's Display of an OS error: "<strerror> (os error N)". strerror_r (GNU form)
// because upload workers format errors concurrently.
std::string os_error_text(int err) {
  char buf[256];
  return std::string(strerror_r(err, buf, sizeof(buf))) + " (os error " + std::to_string(err) + ")";
}

std::string io_error(const char* what, const char* path, int err) {
  return std::string("failed to ") + what + " " + path + ": " + os_error_text(err);
}

void fill_value(const Value& v, fkv_gguf_value* out) {
  memset(out, 0, sizeof(*out));
  out->type = v.type;
  out->elem_type = v.elem_type;
  out->u = v.u;
  out->i = v.i;
  out->f = v.f;
  if (v.type == FKV_GGUF_STRING) {
    out->str = v.str.c_str();
    out->str_len = v.str.size();
  }
  if (v.type == FKV_GGUF_ARRAY) out->count = v.arr.size();
}

}  // namespace

extern "C" {

int32_t fkv_gguf_open(const char* path, fkv_gguf** out) {
  if (!path || !out) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  *out = nullptr;
  std::unique_ptr<fkv_gguf> g(new fkv_gguf());
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (g->fd < 0) return fkv::api_fail(FKV_ERR_GGUF, io_error("open", path, errno));
  struct stat st;
  if (fstat(g->fd, &st) != 0) return fkv::api_fail(FKV_ERR_GGUF, io_error("map", path, errno));
  if (S_ISDIR(st.st_mode)) return fkv::api_fail(FKV_ERR_GGUF, io_error("map", path, EISDIR));
  g->len = (uint64_t)st.st_size;
  if (g->len) {
    void* m = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fkv::api_fail(FKV_ERR_GGUF, io_error("map", path, errno));
    g->map = (const uint8_t*)m;
    madvise(m, g->len, MADV_SEQUENTIAL);
  }
  try {
    parse(g.get());
  } catch (const GgufError& e) {
    return fkv::api_fail(FKV_ERR_GGUF, e.msg);
  } catch (const std::bad_alloc&) {
    return fkv::api_fail(FKV_ERR_GGUF, "metadata allocation failed");
  }
  *out = g.release();
  return fkv::api_ok();
}

int32_t fkv_gguf_close(fkv_gguf* g) {
  fkv::KeepLastError keep;
  delete g;
  return fkv::api_ok();
}

int32_t fkv_gguf_info(const fkv_gguf* g, uint32_t* version, uint64_t* alignment,
                      uint64_t* n_metadata, uint64_t* n_tensors, uint64_t* data_start,
                      uint64_t* data_bytes) {
  if (!g) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  if (version) *version = g->version;
  if (alignment) *alignment = g->alignment;
  if (n_metadata) *n_metadata = g->metadata.size();
  if (n_tensors) *n_tensors = g->tensors.size();
  if (data_start) *data_start = g->data_start;
  if (data_bytes) *data_bytes = g->len - g->data_start;
  return fkv::api_ok();
}

int32_t fkv_gguf_tensor(const fkv_gguf* g, uint64_t index, fkv_gguf_tensor_info* out) {
  if (!g || !out) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  if (index >= g->tensors.size()) return fkv::api_fail(FKV_ERR_INVALID, "tensor index out of range");
  const Tensor& t = g->tensors[index];
  memset(out, 0, sizeof(*out));
  out->name = t.name.c_str();
  out->name_len = t.name.size();
  out->n_dims = (uint32_t)t.shape.size();
  for (size_t d = 0; d < t.shape.size(); d++) out->shape[d] = t.shape[d];
  out->ggml_type = t.ggml_type;
  out->data_offset = t.data_offset;
  out->nbytes = t.nbytes;
  return fkv::api_ok();
}

int32_t fkv_gguf_find(const fkv_gguf* g, const char* name, uint64_t name_len, uint64_t* index) {
  if (!g || (name_len && !name) || !index) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  const std::string key(name ? name : "", (size_t)name_len);
  auto it = g->by_name.find(key);
  if (it == g->by_name.end()) return fkv::api_fail(FKV_ERR_GGUF, "missing tensor " + key);
  *index = it->second;
  return fkv::api_ok();
}

int32_t fkv_gguf_meta(const fkv_gguf* g, const char* key, uint64_t key_len, fkv_gguf_value* out) {
  if (!g || (key_len && !key) || !out) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  const std::string k(key ? key : "", (size_t)key_len);
  auto it = g->metadata.find(k);
  if (it == g->metadata.end()) return fkv::api_fail(FKV_ERR_INVALID, "missing metadata key " + k);
  fill_value(it->second, out);
  return fkv::api_ok();
}

int32_t fkv_gguf_meta_array_elem(const fkv_gguf* g, const char* key, uint64_t key_len,
                                 uint64_t i, fkv_gguf_value* out) {
  if (!g || (key_len && !key) || !out) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  const std::string k(key ? key : "", (size_t)key_len);
  auto it = g->metadata.find(k);
  if (it == g->metadata.end()) return fkv::api_fail(FKV_ERR_INVALID, "missing metadata key " + k);
  if (it->second.type != FKV_GGUF_ARRAY)
    return fkv::api_fail(FKV_ERR_INVALID, "metadata key " + k + " is not an array");
  if (i >= it->second.arr.size())
    return fkv::api_fail(FKV_ERR_INVALID, "array index out of range");
  fill_value(it->second.arr[i], out);
  return fkv::api_ok();
}

int32_t fkv_gguf_dump(const fkv_gguf* g, char* buf, uint64_t cap, uint64_t* len) {
  if (!g || !len || (cap && !buf)) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  std::string s = "ferrum-gguf version=" + std::to_string(g->version) +
                  " alignment=" + std::to_string(g->alignment) +
                  " metadata=" + std::to_string(g->metadata.size()) +
                  " tensors=" + std::to_string(g->tensors.size()) + "\n";
  for (const Tensor& t : g->tensors) {
    s += t.name + " [";
    for (size_t d = 0; d < t.shape.size(); d++) {
      if (d) s += ", ";
      s += std::to_string(t.shape[d]);
    }
    const char* dt = ggml_type_name(t.ggml_type);
    s += std::string("] ") + (dt ? dt : "unknown") + "\n";
  }
  *len = s.size();
  if (cap) {
    const uint64_t n = std::min<uint64_t>(cap - 1, s.size());
    memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return fkv::api_ok();
}

// Granularity of the copies an upload queues (a chunk is read and sent in pieces of this).
constexpr uint64_t kUploadPiece = 2ull << 20;

// Host threads for an upload when the caller passes 0: 4, or fewer when the process may
// run on fewer CPUs. Four 8 MiB pipelines keep the PCIe link busy (measured on MI355X:
// 2 threads 42 GB/s, 3-4 threads 50-52 GB/s, 8 threads 46 GB/s, 16 threads 33-35 GB/s).
static uint32_t default_upload_threads() {
  cpu_set_t set;
  CPU_ZERO(&set);
  int n = sched_getaffinity(0, sizeof(set), &set) == 0 ? CPU_COUNT(&set) : 4;
  return (uint32_t)std::max(1, std::min(n, 4));
}

int32_t fkv_gguf_upload(const fkv_gguf* g, void* dst, uint64_t dst_bytes, uint64_t chunk_bytes,
                        uint32_t threads) {
  if (!g) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  const uint64_t data_bytes = g->len - g->data_start;
  if (data_bytes == 0) return fkv::api_ok();
  if (!dst) return fkv::api_fail(FKV_ERR_INVALID, "null argument");
  if (dst_bytes < data_bytes)
    return fkv::api_fail(FKV_ERR_INVALID, "device buffer smaller than the data section");
  const uint64_t chunk = chunk_bytes ? chunk_bytes : (8ull << 20);
  const uint64_t n_chunks = (data_bytes + chunk - 1) / chunk;
  const uint32_t nthr = (uint32_t)std::min<uint64_t>(
      std::max(1u, std::min(threads ? threads : default_upload_threads(), 64u)), n_chunks);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fkv::api_fail(FKV_ERR_INTERNAL, "hip: current device");

  // Worker t owns one pinned buffer and one stream and moves chunks t, t + nthr, ...: it
  // waits for its own previous copy, preads the next chunk into the buffer (the kernel
  // copies from the page cache, no page faults on the map) and queues its copy. Workers
  // never wait for each other: with one shared stream a worker's wait also covered every
  // copy queued before its own (measured 43 GB/s against 52 GB/s with a stream each).
  struct Failure {
    int32_t code = FKV_OK;
    std::string msg;
  };
  std::vector<Failure> fail(nthr);
  std::atomic<bool> stop{false};
  auto worker = [&](uint32_t t) {
    Failure& f = fail[t];
    auto hip = [&](hipError_t e, const char* what) {
      if (e != hipSuccess && f.code == FKV_OK) {
        f.code = FKV_ERR_INTERNAL;
        f.msg = std::string("hip: ") + what + ": " + hipGetErrorString(e);
      }
      return e == hipSuccess;
    };
    uint8_t* buf = nullptr;
    hipEvent_t ev = nullptr;
    hipStream_t s = nullptr;
    bool queued = false;
    bool ok = hip(hipSetDevice(dev), "set device") &&
              hip(hipHostMalloc((void**)&buf, chunk, hipHostMallocDefault), "pinned staging") &&
              hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "event") &&
              hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
    for (uint64_t k = t; ok && k < n_chunks && !stop.load(std::memory_order_relaxed); k += nthr) {
      if (queued && !(ok = hip(hipEventSynchronize(ev), "event wait"))) break;
      const uint64_t off = k * chunk;
      const uint64_t n = std::min(chunk, data_bytes - off);
      // each piece is queued as soon as it is read, so the link starts after the first piece
      // rather than after a whole chunk
      for (uint64_t p0 = 0; ok && p0 < n; p0 += kUploadPiece) {
        const uint64_t pn = std::min(kUploadPiece, n - p0);
        for (uint64_t got = 0; got < pn;) {
          const ssize_t r = pread(g->fd, buf + p0 + got, (size_t)(pn - got),
                                  (off_t)(g->data_start + off + p0 + got));
          if (r < 0 && errno == EINTR) continue;
          if (r <= 0) {
            const int e = r < 0 ? errno : EIO;
            f.code = FKV_ERR_GGUF;
            f.msg = "failed to read tensor data: " + os_error_text(e);
            ok = false;
            break;
          }
          got += (uint64_t)r;
        }
        ok = ok && hip(hipMemcpyAsync((uint8_t*)dst + off + p0, buf + p0, pn, hipMemcpyHostToDevice, s),
                       "copy to device");
        queued = queued || ok;
      }
      ok = ok && hip(hipEventRecord(ev, s), "event record");
    }
    if (!ok) stop.store(true, std::memory_order_relaxed);
    // the buffer is freed only once no copy can still read it
    if (!ok && s) (void)hipStreamSynchronize(s);
    else if (queued) hip(hipEventSynchronize(ev), "event wait");
    if (ev) (void)hipEventDestroy(ev);
    if (buf) (void)hipHostFree(buf);
    if (s) (void)hipStreamDestroy(s);
  };
  std::vector<std::thread> pool;
  pool.reserve(nthr);
  bool spawned = true;
  try {
    for (uint32_t t = 0; t < nthr; t++) pool.emplace_back(worker, t);
  } catch (const std::system_error&) {
    // the workers started so far stop after their current chunk
    stop.store(true, std::memory_order_relaxed);
    spawned = false;
  }
  for (auto& th : pool) th.join();
  if (!spawned) return fkv::api_fail(FKV_ERR_INTERNAL, "failed to start upload threads");
  for (const Failure& f : fail)
    if (f.code != FKV_OK) return fkv::api_fail(f.code, f.msg);
  return fkv::api_ok();
}

}  // extern "C"
