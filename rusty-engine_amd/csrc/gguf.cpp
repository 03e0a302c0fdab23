// GGUF container reader (src/gguf.rs:17-330, src/loader.rs:17-110): the file is mapped read-only
// and its header parsed (magic, version 2/3, metadata key/values of every kind including nested
// arrays, the tensor-info table, the aligned data start); tensor data is handed out as pointers
// into the mapping (the reference's MmapModel::tensor_bytes, without `to_vec`). The device
// upload of a tensor into a QMat (re_qmat_from_gguf, api.hip) copies those bytes to the GPU
// unchanged and repacks them there.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/rehip.h"
#include "common.hpp"

namespace rehip {
int report_error(int code, const char* fmt, ...);   // api.hip: sets re_last_error()
}

using rehip::report_error;

namespace {

constexpr uint64_t kDefaultAlignment = 32;   // gguf.rs:18

struct Kv {
  std::string key;
  uint32_t kind = 0;
  // scalars widened; strings as (offset, length) into the map; arrays: element kind and count
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  size_t s_off = 0, s_len = 0;
  uint32_t arr_kind = 0;
  uint64_t arr_count = 0;
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint32_t type = 0;
  uint64_t offset = 0;
};

// bytes of numel elements of a GGML type; false when the count is not whole blocks or the type
// is unsized (quant.rs:75-101)
bool bytes_for_numel(uint32_t type, uint64_t numel, uint64_t* out) {
  uint64_t el = 0, by = 0;
  switch (type) {
    case 0: el = 1; by = 4; break;             // F32
    case 1: case 30: el = 1; by = 2; break;    // F16, BF16
    case 2: el = 32; by = 18; break;
    case 6: el = 32; by = 22; break;
    case 8: el = 32; by = 34; break;
    case 12: el = 256; by = 144; break;
    case 13: el = 256; by = 176; break;
    case 14: el = 256; by = 210; break;
    default: return false;
  }
  if (numel % el) return false;
  *out = numel / el * by;
  return true;
}

// UTF-8 check with the error report of Rust's str::from_utf8 (the reference decodes every key,
// tensor name and string value with it, gguf.rs:255-265): on failure, `valid_up_to` and the
// length of the invalid sequence (0 = the input ends inside a sequence).
bool utf8_ok(const uint8_t* s, size_t n, size_t* valid_up_to, int* bad_len) {
  auto cont = [&](size_t k) { return k < n && (s[k] & 0xC0) == 0x80; };
  size_t i = 0;
  while (i < n) {
    const uint8_t b = s[i];
    if (b < 0x80) { ++i; continue; }
    int w = 0;
    if (b >= 0xC2 && b <= 0xDF) w = 2;
    else if (b >= 0xE0 && b <= 0xEF) w = 3;
    else if (b >= 0xF0 && b <= 0xF4) w = 4;
    *valid_up_to = i;
    if (!w) { *bad_len = 1; return false; }
    if (i + 1 >= n) { *bad_len = 0; return false; }
    const uint8_t c = s[i + 1];
    bool second;
    if (w == 2) second = (c & 0xC0) == 0x80;
    else if (w == 3) second = b == 0xE0 ? (c >= 0xA0 && c <= 0xBF) : b == 0xED ? (c >= 0x80 && c <= 0x9F)
                                                                                : (c & 0xC0) == 0x80;
    else second = b == 0xF0 ? (c >= 0x90 && c <= 0xBF) : b == 0xF4 ? (c >= 0x80 && c <= 0x8F)
                                                                    : (c & 0xC0) == 0x80;
    if (!second) { *bad_len = 1; return false; }
    for (int k = 2; k < w; ++k) {
      if (i + k >= n) { *bad_len = 0; return false; }
      if (!cont(i + k)) { *bad_len = k; return false; }
    }
    i += w;
  }
  return true;
}

struct Reader {
  const uint8_t* b;
  size_t n, pos = 0;
  std::string err;
  size_t err_at = 0;
  bool fail(const char* msg) {
    if (err.empty()) {
      err = msg;
      err_at = pos;
    }
    return false;
  }
  bool need(size_t k) {
    if (pos + k > n || pos + k < pos) {
      char m[96];
      snprintf(m, sizeof m, "unexpected EOF, need %zu bytes", k);
      return fail(m);
    }
    return true;
  }
  bool u8(uint8_t& v) { if (!need(1)) return false; v = b[pos++]; return true; }
  bool u16(uint16_t& v) { if (!need(2)) return false; std::memcpy(&v, b + pos, 2); pos += 2; return true; }
  bool u32(uint32_t& v) { if (!need(4)) return false; std::memcpy(&v, b + pos, 4); pos += 4; return true; }
  bool u64(uint64_t& v) { if (!need(8)) return false; std::memcpy(&v, b + pos, 8); pos += 8; return true; }
  bool str(size_t& off, size_t& len) {
    uint64_t l;
    if (!u64(l)) return false;
    if (l > n - pos) {
      char m[96];
      snprintf(m, sizeof m, "unexpected EOF, need %llu bytes", (unsigned long long)l);
      return fail(m);
    }
    size_t upto = 0;
    int bad = 0;
    if (!utf8_ok(b + pos, (size_t)l, &upto, &bad)) {
      char m[128];
      if (bad) snprintf(m, sizeof m, "invalid utf-8 string: invalid utf-8 sequence of %d bytes from index %zu", bad, upto);
      else snprintf(m, sizeof m, "invalid utf-8 string: incomplete utf-8 byte sequence from index %zu", upto);
      return fail(m);
    }
    off = pos;
    len = (size_t)l;
    pos += (size_t)l;
    return true;
  }
  // one value of `kind` (gguf.rs:274-312); scalars land in kv when given
  bool value(uint32_t kind, Kv* kv, int depth) {
    if (depth > 16) return fail("array nesting too deep");
    switch (kind) {
      case 0: { uint8_t v; if (!u8(v)) return false; if (kv) { kv->u = v; kv->i = v; } return true; }
      case 1: { uint8_t v; if (!u8(v)) return false; if (kv) { kv->i = (int8_t)v; kv->u = (uint64_t)kv->i; } return true; }
      case 2: { uint16_t v; if (!u16(v)) return false; if (kv) { kv->u = v; kv->i = v; } return true; }
      case 3: { uint16_t v; if (!u16(v)) return false; if (kv) { kv->i = (int16_t)v; kv->u = (uint64_t)kv->i; } return true; }
      case 4: { uint32_t v; if (!u32(v)) return false; if (kv) { kv->u = v; kv->i = v; } return true; }
      case 5: { uint32_t v; if (!u32(v)) return false; if (kv) { kv->i = (int32_t)v; kv->u = (uint64_t)kv->i; } return true; }
      case 6: { uint32_t v; if (!u32(v)) return false; if (kv) { float f; std::memcpy(&f, &v, 4); kv->f = f; } return true; }
      case 7: { uint8_t v; if (!u8(v)) return false; if (kv) { kv->u = v != 0; kv->i = v != 0; } return true; }
      case 8: { size_t o, l; if (!str(o, l)) return false; if (kv) { kv->s_off = o; kv->s_len = l; } return true; }
      case 9: {
        uint32_t ek;
        uint64_t count;
        if (!u32(ek)) return false;
        if (ek > 12) {
          char m[96];
          snprintf(m, sizeof m, "unknown array element kind %u", ek);
          return fail(m);
        }
        if (!u64(count)) return false;
        if (count > (uint64_t)(n - pos)) {      // every element is at least one byte
          char m[96];
          snprintf(m, sizeof m, "array count %llu exceeds remaining bytes", (unsigned long long)count);
          return fail(m);
        }
        if (kv) { kv->arr_kind = ek; kv->arr_count = count; }
        for (uint64_t j = 0; j < count; ++j)
          if (!value(ek, nullptr, depth + 1)) return false;
        return true;
      }
      case 10: { uint64_t v; if (!u64(v)) return false; if (kv) { kv->u = v; kv->i = (int64_t)v; } return true; }
      case 11: { uint64_t v; if (!u64(v)) return false; if (kv) { kv->i = (int64_t)v; kv->u = v; } return true; }
      case 12: { uint64_t v; if (!u64(v)) return false; if (kv) { double d; std::memcpy(&d, &v, 8); kv->f = d; } return true; }
      default: return fail("unknown value kind");
    }
  }
};

}  // namespace

struct re_gguf {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  std::vector<Kv> kvs;
  std::vector<Tensor> tensors;
  uint64_t alignment = kDefaultAlignment;
  size_t data_offset = 0, data_start = 0;
  std::vector<char> name_scratch;
};

extern "C" {

void re_gguf_close(re_gguf* g) {
  if (!g) return;
  if (g->map && g->size) munmap((void*)g->map, g->size);
  if (g->fd >= 0) close(g->fd);
  delete g;
}

// Parse a GGUF header held in memory (gguf.rs:322-392); `g` gets the tables.
static int parse_header(re_gguf* g) {
  if (g->size < 4 || std::memcmp(g->map, "GGUF", 4) != 0)
    return report_error(RE_ERR_ARG, "gguf parse error at 0: missing GGUF magic");
  Reader r{g->map, g->size};
  r.pos = 4;
  uint32_t version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  auto bad = [&]() {
    return report_error(RE_ERR_ARG, "gguf parse error at %zu: %s", r.err_at, r.err.c_str());
  };
  if (!r.u32(version)) return bad();
  if (version < 2 || version > 3)
    return report_error(RE_ERR_ARG, "gguf parse error at 4: unsupported GGUF version %u (need 2 or 3)", version);
  if (version >= 3) {
    if (!r.u64(n_tensors) || !r.u64(n_kv)) return bad();
  } else {
    uint32_t a, b;
    if (!r.u32(a) || !r.u32(b)) return bad();
    n_tensors = a;
    n_kv = b;
  }
  g->version = version;
  for (uint64_t k = 0; k < n_kv; ++k) {
    Kv kv;
    size_t ko, kl;
    if (!r.str(ko, kl)) return bad();
    kv.key.assign((const char*)g->map + ko, kl);
    if (!r.u32(kv.kind)) return bad();
    if (kv.kind > 12)
      return report_error(RE_ERR_ARG, "gguf parse error at %zu: unknown value kind %u for key %s", r.pos, kv.kind,
                          kv.key.c_str());
    if (!r.value(kv.kind, &kv, 0)) return bad();
    g->kvs.push_back(std::move(kv));
  }
  for (uint64_t k = 0; k < n_tensors; ++k) {
    Tensor t;
    size_t no, nl;
    if (!r.str(no, nl)) return bad();
    t.name.assign((const char*)g->map + no, nl);
    if (!r.u32(t.n_dims)) return bad();
    if (t.n_dims > 8)
      return report_error(RE_ERR_ARG, "gguf parse error at %zu: tensor %s declares %u dims (max 8)", r.pos,
                          t.name.c_str(), t.n_dims);
    for (uint32_t d = 0; d < t.n_dims; ++d)
      if (!r.u64(t.dims[d])) return bad();
    if (!r.u32(t.type) || !r.u64(t.offset)) return bad();
    g->tensors.push_back(std::move(t));
  }
  g->data_offset = r.pos;
  // general.alignment as U32 or U64, else 32 (gguf.rs:143-150); data start rounded up to it
  for (const Kv& kv : g->kvs)
    if (kv.key == "general.alignment") {
      if (kv.kind == 4 || kv.kind == 10) g->alignment = kv.u;
      break;
    }
  const uint64_t a = g->alignment ? g->alignment : 1;
  g->data_start = (size_t)((g->data_offset + a - 1) / a * a);
  return RE_OK;
}

int re_gguf_open(const char* path, re_gguf** out) {
  if (!path || !out) return report_error(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  re_gguf* g = new (std::nothrow) re_gguf();
  if (!g) return report_error(RE_ERR_ARG, "out of memory");
  g->fd = open(path, O_RDONLY);
  if (g->fd < 0) {
    re_gguf_close(g);
    return report_error(RE_ERR_ARG, "cannot open %s: %s", path, strerror(errno));
  }
  struct stat st;
  if (fstat(g->fd, &st) != 0 || st.st_size <= 0) {
    re_gguf_close(g);
    return report_error(RE_ERR_ARG, "cannot map %s: empty or unreadable", path);
  }
  g->size = (size_t)st.st_size;
  void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (m == MAP_FAILED) {
    g->map = nullptr;
    re_gguf_close(g);
    return report_error(RE_ERR_ARG, "mmap of %s failed: %s", path, strerror(errno));
  }
  g->map = (const uint8_t*)m;
  int rc = parse_header(g);
  if (rc) {
    re_gguf_close(g);
    return rc;
  }
  *out = g;
  return RE_OK;
}

uint32_t re_gguf_version(const re_gguf* g) { return g ? g->version : 0; }
size_t re_gguf_kv_count(const re_gguf* g) { return g ? g->kvs.size() : 0; }
size_t re_gguf_tensor_count(const re_gguf* g) { return g ? g->tensors.size() : 0; }
uint64_t re_gguf_alignment(const re_gguf* g) { return g ? g->alignment : 0; }
size_t re_gguf_data_offset(const re_gguf* g) { return g ? g->data_offset : 0; }
size_t re_gguf_data_start(const re_gguf* g) { return g ? g->data_start : 0; }

int re_gguf_kv(const re_gguf* g, size_t i, const char** key, uint32_t* kind) {
  if (!g || i >= g->kvs.size()) return report_error(RE_ERR_ARG, "kv index out of range");
  if (key) *key = g->kvs[i].key.c_str();
  if (kind) *kind = g->kvs[i].kind;
  return RE_OK;
}

static const Kv* find_kv(const re_gguf* g, const char* key) {
  for (const Kv& kv : g->kvs)
    if (kv.key == key) return &kv;   // first match (gguf.rs:139-141)
  return nullptr;
}

int re_gguf_get_int(const re_gguf* g, const char* key, int64_t* v) {
  if (!g || !key || !v) return report_error(RE_ERR_ARG, "null pointer");
  const Kv* kv = find_kv(g, key);
  if (!kv) return report_error(RE_ERR_ARG, "key %s not found", key);
  if (kv->kind > 5 && kv->kind != 7 && kv->kind != 10 && kv->kind != 11)
    return report_error(RE_ERR_ARG, "key %s is not an integer (kind %u)", key, kv->kind);
  *v = kv->i;
  return RE_OK;
}

int re_gguf_get_float(const re_gguf* g, const char* key, double* v) {
  if (!g || !key || !v) return report_error(RE_ERR_ARG, "null pointer");
  const Kv* kv = find_kv(g, key);
  if (!kv) return report_error(RE_ERR_ARG, "key %s not found", key);
  if (kv->kind != 6 && kv->kind != 12) return report_error(RE_ERR_ARG, "key %s is not a float (kind %u)", key, kv->kind);
  *v = kv->f;
  return RE_OK;
}

int re_gguf_get_str(const re_gguf* g, const char* key, const char** s, size_t* len) {
  if (!g || !key || !s || !len) return report_error(RE_ERR_ARG, "null pointer");
  const Kv* kv = find_kv(g, key);
  if (!kv) return report_error(RE_ERR_ARG, "key %s not found", key);
  if (kv->kind != 8) return report_error(RE_ERR_ARG, "key %s is not a string (kind %u)", key, kv->kind);
  *s = (const char*)g->map + kv->s_off;
  *len = kv->s_len;
  return RE_OK;
}

int re_gguf_get_array(const re_gguf* g, const char* key, uint32_t* elem_kind, uint64_t* count) {
  if (!g || !key || !elem_kind || !count) return report_error(RE_ERR_ARG, "null pointer");
  const Kv* kv = find_kv(g, key);
  if (!kv) return report_error(RE_ERR_ARG, "key %s not found", key);
  if (kv->kind != 9) return report_error(RE_ERR_ARG, "key %s is not an array (kind %u)", key, kv->kind);
  *elem_kind = kv->arr_kind;
  *count = kv->arr_count;
  return RE_OK;
}

int re_gguf_tensor_info(const re_gguf* g, size_t i, const char** name, uint32_t* type, uint32_t* n_dims,
                        uint64_t* dims, uint64_t* offset) {
  if (!g || i >= g->tensors.size()) return report_error(RE_ERR_ARG, "tensor index out of range");
  const Tensor& t = g->tensors[i];
  if (name) *name = t.name.c_str();
  if (type) *type = t.type;
  if (n_dims) *n_dims = t.n_dims;
  if (dims) for (uint32_t d = 0; d < 8; ++d) dims[d] = d < t.n_dims ? t.dims[d] : 0;
  if (offset) *offset = t.offset;
  return RE_OK;
}

int re_gguf_find_tensor(const re_gguf* g, const char* name, size_t* index) {
  if (!g || !name || !index) return report_error(RE_ERR_ARG, "null pointer");
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) {
      *index = i;
      return RE_OK;
    }
  return report_error(RE_ERR_ARG, "tensor '%s' not found", name);
}

// [data_start + offset, + nbytes) inside the mapping (loader.rs:95-101), numel = product of dims
int re_gguf_tensor_data(const re_gguf* g, size_t i, const uint8_t** data, size_t* nbytes) {
  if (!g || !data || !nbytes) return report_error(RE_ERR_ARG, "null pointer");
  if (i >= g->tensors.size()) return report_error(RE_ERR_ARG, "tensor index out of range");
  const Tensor& t = g->tensors[i];
  uint64_t numel = 1;
  for (uint32_t d = 0; d < t.n_dims; ++d) {
    if (t.dims[d] && numel > UINT64_MAX / t.dims[d])
      return report_error(RE_ERR_SIZE, "tensor '%s': element count overflows", t.name.c_str());
    numel *= t.dims[d];
  }
  uint64_t nb = 0;
  if (!bytes_for_numel(t.type, numel, &nb))
    return report_error(RE_ERR_TYPE, "tensor '%s': type %u is unsized or %llu elements are not whole blocks",
                        t.name.c_str(), t.type, (unsigned long long)numel);
  const uint64_t start = (uint64_t)g->data_start + t.offset;
  if (start < t.offset || start > g->size || nb > g->size - start)
    return report_error(RE_ERR_SIZE, "tensor '%s' bytes out of bounds", t.name.c_str());
  *data = g->map + start;
  *nbytes = (size_t)nb;
  return RE_OK;
}

// QMat::from_model (qmat.rs:310-330): the named tensor's mapped bytes go to the device as they
// are (no host copy of the whole tensor) and are repacked there. A tensor holding several
// equal matrices (experts, dims [n, m, count]) becomes a stacked QMat.
int re_qmat_from_gguf(const re_gguf* g, const char* name, size_t m, size_t n, re_qmat** out) {
  if (!g || !name || !out) return report_error(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  size_t i = 0;
  bool found = false;
  for (size_t k = 0; k < g->tensors.size() && !found; ++k)
    if (g->tensors[k].name == name) {
      i = k;
      found = true;
    }
  if (!found) return report_error(RE_ERR_ARG, "QMat: tensor '%s' missing", name);
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  if (re_gguf_tensor_data(g, i, &data, &nbytes) != RE_OK)
    return report_error(RE_ERR_SIZE, "QMat: tensor '%s' bytes out of bounds", name);
  const Tensor& t = g->tensors[i];
  if (t.n_dims < 2 || t.dims[0] != n || t.dims[1] != m)
    return report_error(RE_ERR_SIZE, "QMat: tensor '%s' dims do not start with [n=%zu, m=%zu]", name, n, m);
  uint64_t count = 1;
  for (uint32_t d = 2; d < t.n_dims; ++d) count *= t.dims[d];
  return re_qmat_create_stacked(t.type, data, nbytes, m, n, (size_t)count, out);
}

// Stacked expert tensors of one MoE layer (model.rs:372-389: ffn_{gate,up}_exps [hidden, inter,
// E], ffn_down_exps [inter, hidden, E]) uploaded from the mapping and repacked on the device.
int re_moe_from_gguf(const re_gguf* g, const char* gate, const char* up, const char* down, size_t n_experts,
                     size_t hidden, size_t inter, re_moe** out) {
  if (!g || !gate || !up || !down || !out) return report_error(RE_ERR_ARG, "null pointer");
  *out = nullptr;
  const char* names[3] = {gate, up, down};
  const uint64_t want[3][3] = {{hidden, inter, n_experts}, {hidden, inter, n_experts}, {inter, hidden, n_experts}};
  const uint8_t* data[3];
  size_t nbytes[3];
  uint32_t type[3];
  for (int p = 0; p < 3; ++p) {
    size_t i;
    if (re_gguf_find_tensor(g, names[p], &i) != RE_OK) return report_error(RE_ERR_ARG, "tensor '%s' missing", names[p]);
    const Tensor& t = g->tensors[i];
    if (t.n_dims != 3 || t.dims[0] != want[p][0] || t.dims[1] != want[p][1] || t.dims[2] != want[p][2])
      return report_error(RE_ERR_SIZE, "tensor '%s' dims are not [%llu, %llu, %llu]", names[p],
                          (unsigned long long)want[p][0], (unsigned long long)want[p][1],
                          (unsigned long long)want[p][2]);
    if (re_gguf_tensor_data(g, i, &data[p], &nbytes[p]) != RE_OK)
      return report_error(RE_ERR_SIZE, "tensor '%s' bytes out of bounds", names[p]);
    type[p] = t.type;
  }
  return re_moe_create(type[0], data[0], nbytes[0], type[1], data[1], nbytes[1], type[2], data[2], nbytes[2],
                       n_experts, hidden, inter, out);
}

}  // extern "C"
