// weights.cpp — the weight file (engine/src/weights.rs:38-74; format tools/convert.py:117-150):
// a 32-byte header (magic "VIOLETTO", version 1, tensor count, data-region offset), 128-byte
// records (name, dtype, shape, offset into the data region, bytes), then the tensors. The
// records are read and checked on the host; sv_weights_upload copies the data region into one
// device buffer through two pinned staging buffers on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "sv_internal.h"

using namespace sv;

#define SV_TRY(x)                  \
  do {                             \
    const sv_status st_ = (x);     \
    if (st_ != SV_OK) return st_;  \
  } while (0)
#define SV_TRY_HIP(x, what) SV_TRY(check_hip((x), (what)))

struct sv_weights {
  std::string path;
  uint64_t data_offset = 0, end = 0, file_size = 0;
  std::vector<sv_tensor_info> tensors;
  std::unordered_map<std::string, uint32_t> index;
  void* device = nullptr;
};

namespace {

uint32_t u32_at(const uint8_t* b) {
  uint32_t v;
  memcpy(&v, b, 4);
  return v;
}
uint64_t u64_at(const uint8_t* b) {
  uint64_t v;
  memcpy(&v, b, 8);
  return v;
}
size_t dtype_size(uint32_t d) { return d == 0 ? 4 : d == 1 ? 2 : 1; }
const char* dtype_name(uint32_t d) { return d == 0 ? "F32" : d == 1 ? "Bf16" : "I8"; }

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) fclose(f);
  }
};

}  // namespace

extern "C" sv_status sv_weights_open(const char* path, sv_weights** out) {
  if (!path || !out) return fail(SV_ERR_ARG, "weights_open: null pointer");
  *out = nullptr;
  File fh;
  fh.f = fopen(path, "rb");
  if (!fh.f) return fail(SV_ERR_ARG, "%s: cannot open", path);
  if (fseek(fh.f, 0, SEEK_END) != 0) return fail(SV_ERR_ARG, "%s: cannot seek", path);
  const long size = ftell(fh.f);
  rewind(fh.f);
  uint8_t head[32];
  if (size < 32 || fread(head, 1, 32, fh.f) != 32 || memcmp(head, "VIOLETTO", 8) != 0 || u32_at(head + 8) != 1)
    return fail(SV_ERR_ARG, "%s: not a version-1 violetto weight file", path);
  const uint32_t n = u32_at(head + 12);
  const uint64_t data_offset = u64_at(head + 16);
  if ((uint64_t)size < 32 + (uint64_t)n * 128 || data_offset < 32 + (uint64_t)n * 128 || data_offset > (uint64_t)size)
    return fail(SV_ERR_ARG, "%s: %u records do not fit the file", path, n);
  std::vector<uint8_t> rec((size_t)n * 128);
  if (n && fread(rec.data(), 1, rec.size(), fh.f) != rec.size()) return fail(SV_ERR_ARG, "%s: short read", path);
  sv_weights* w = new sv_weights();
  w->path = path;
  w->data_offset = data_offset;
  w->file_size = (uint64_t)size;
  for (uint32_t i = 0; i < n; i++) {
    const uint8_t* r = rec.data() + (size_t)i * 128;
    sv_tensor_info t{};
    size_t len = 0;
    while (len < 64 && r[len]) len++;
    // sv_tensor_info.name holds 63 bytes and a NUL; the reference writer's names are shorter
    // (tools/convert.py:137), and a longer one could not be looked up under its real name.
    if (len == 64) {
      delete w;
      return fail(SV_ERR_ARG, "%s: record %u has a 64-byte name with no NUL", path, i);
    }
    memcpy(t.name, r, len);
    t.name[len] = 0;
    t.dtype = u32_at(r + 64);
    t.ndim = u32_at(r + 68);
    for (int d = 0; d < 4; d++) t.shape[d] = u32_at(r + 72 + 4 * d);
    t.offset = u64_at(r + 88);
    t.nbytes = u64_at(r + 96);
    auto bad = [&](sv_status st) {
      delete w;
      return st;
    };
    if (t.dtype > 2) return bad(fail(SV_ERR_ARG, "%s: unknown dtype %u", t.name, t.dtype));
    if (t.ndim > 4) return bad(fail(SV_ERR_ARG, "%s: %u dimensions", t.name, t.ndim));
    // Overflow-safe: the element count is built against the file's data region, so neither
    // the product of the dims nor offset + nbytes can wrap.
    const uint64_t avail = (uint64_t)size - data_offset;
    uint64_t elems = 1;
    bool too_big = false;
    for (uint32_t d = 0; d < t.ndim; d++) {
      if (t.shape[d] != 0 && elems > avail / t.shape[d]) too_big = true;
      if (!too_big) elems *= t.shape[d];
    }
    if (too_big || elems * dtype_size(t.dtype) != t.nbytes)
      return bad(fail(SV_ERR_ARG, "%s: %llu bytes for a [%u, %u, %u, %u] %s shape", t.name, (unsigned long long)t.nbytes,
                      t.shape[0], t.shape[1], t.shape[2], t.shape[3], dtype_name(t.dtype)));
    if (t.offset > avail || t.nbytes > avail - t.offset)
      return bad(fail(SV_ERR_ARG, "%s: bytes past the end of the file", t.name));
    // The writer aligns every tensor to 256 bytes (tools/convert.py:17,133); the kernels read
    // weights, scales and tables with 8- and 16-byte vector loads from the device copy.
    if (t.offset % 256 != 0)
      return bad(fail(SV_ERR_ARG, "%s: offset %llu is not a multiple of 256", t.name, (unsigned long long)t.offset));
    if (w->index.count(t.name)) return bad(fail(SV_ERR_ARG, "%s: two tensors of this name", t.name));
    w->index[t.name] = i;
    w->tensors.push_back(t);
    w->end = std::max<uint64_t>(w->end, t.offset + t.nbytes);
  }
  *out = w;
  return SV_OK;
}

extern "C" uint32_t sv_weights_count(const sv_weights* w) { return w ? (uint32_t)w->tensors.size() : 0; }

extern "C" sv_status sv_weights_info(const sv_weights* w, uint32_t i, sv_tensor_info* out) {
  if (!w || !out) return fail(SV_ERR_ARG, "weights_info: null pointer");
  if (i >= w->tensors.size()) return fail(SV_ERR_ARG, "weights_info: tensor %u of %zu", i, w->tensors.size());
  *out = w->tensors[i];
  return SV_OK;
}

// weights.rs:89-91 tensor().
extern "C" sv_status sv_weights_find(const sv_weights* w, const char* name, sv_tensor_info* out) {
  if (!w || !name || !out) return fail(SV_ERR_ARG, "weights_find: null pointer");
  auto it = w->index.find(name);
  if (it == w->index.end()) return fail(SV_ERR_ARG, "weight file has no tensor %s", name);
  *out = w->tensors[it->second];
  return SV_OK;
}

extern "C" sv_status sv_weights_read(const sv_weights* w, const char* name, void* host, size_t bytes) {
  sv_tensor_info t;
  const sv_status st = sv_weights_find(w, name, &t);
  if (st != SV_OK) return st;
  if (!host || bytes != t.nbytes) return fail(SV_ERR_ARG, "weights_read: %s holds %llu bytes", name, (unsigned long long)t.nbytes);
  File fh;
  fh.f = fopen(w->path.c_str(), "rb");
  if (!fh.f || fseek(fh.f, (long)(w->data_offset + t.offset), SEEK_SET) != 0 || fread(host, 1, bytes, fh.f) != bytes)
    return fail(SV_ERR_ARG, "%s: cannot read %s", w->path.c_str(), name);
  return SV_OK;
}

extern "C" sv_status sv_weights_upload(sv_weights* w, void* stream) {
  if (!w) return fail(SV_ERR_ARG, "weights_upload: null pointer");
  if (w->device) return SV_OK;
  const hipStream_t s = (hipStream_t)stream;
  constexpr size_t CHUNK = (size_t)64 << 20;
  void* dev = nullptr;
  SV_TRY_HIP(hipMalloc(&dev, std::max<uint64_t>(w->end, 1)), "weights: device buffer");
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  sv_status st = SV_OK;
  File fh;
  fh.f = fopen(w->path.c_str(), "rb");
  if (!fh.f || fseek(fh.f, (long)w->data_offset, SEEK_SET) != 0) st = fail(SV_ERR_ARG, "%s: cannot read", w->path.c_str());
  for (int i = 0; i < 2 && st == SV_OK; i++) {
    st = check_hip(hipHostMalloc(&stage[i], CHUNK, hipHostMallocDefault), "weights: staging buffer");
    if (st == SV_OK) st = check_hip(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "weights: event");
  }
  for (uint64_t off = 0, i = 0; st == SV_OK && off < w->end; off += CHUNK, i++) {
    const size_t b = (size_t)std::min<uint64_t>(CHUNK, w->end - off);
    const int k = (int)(i & 1);
    if (i >= 2) st = check_hip(hipEventSynchronize(done[k]), "weights: staging");  // its last copy is done
    if (st == SV_OK && fread(stage[k], 1, b, fh.f) != b) st = fail(SV_ERR_ARG, "%s: short read", w->path.c_str());
    if (st == SV_OK) st = check_hip(hipMemcpyAsync((char*)dev + off, stage[k], b, hipMemcpyHostToDevice, s), "weights: copy");
    if (st == SV_OK) st = check_hip(hipEventRecord(done[k], s), "weights: event");
  }
  if (st == SV_OK) st = check_hip(hipStreamSynchronize(s), "weights: copy");
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  if (st != SV_OK) {
    (void)hipFree(dev);
    return st;
  }
  w->device = dev;
  return SV_OK;
}

extern "C" sv_status sv_weights_device(const sv_weights* w, const char* name, void** d_ptr) {
  sv_tensor_info t;
  const sv_status st = sv_weights_find(w, name, &t);
  if (st != SV_OK) return st;
  if (!d_ptr) return fail(SV_ERR_ARG, "weights_device: null pointer");
  if (!w->device) return fail(SV_ERR_STATE, "weights_device: not uploaded");
  *d_ptr = (char*)w->device + t.offset;
  return SV_OK;
}

// model.rs:80-103 bf16_matrix / matrix: bf16 [m][k], or int8 [m][k] with `<name>.scale` bf16
// [m][groups], groups of a power of two from 8 to 256 k; also one group per row (the
// benchmark configurations' per-output-channel format, which the reference's check refuses).
extern "C" sv_status sv_weights_matrix(const sv_weights* w, const char* name, uint32_t m, uint32_t k, sv_matrix* out) {
  if (!w || !name || !out) return fail(SV_ERR_ARG, "weights_matrix: null pointer");
  sv_tensor_info t;
  SV_TRY(sv_weights_find(w, name, &t));
  if (t.ndim != 2 || t.shape[0] != m || t.shape[1] != k || t.dtype == 0)
    return fail(SV_ERR_ARG, "%s: expected %s [%u, %u], found %s [%u, %u]", name, t.dtype == 2 ? "I8" : "Bf16", m, k,
                dtype_name(t.dtype), t.shape[0], t.ndim > 1 ? t.shape[1] : 0);
  const std::string scale = std::string(name) + ".scale";
  uint32_t gshift = 0;
  if (t.dtype == 2) {
    sv_tensor_info s;
    SV_TRY(sv_weights_find(w, scale.c_str(), &s));
    const uint32_t groups = s.ndim > 1 ? s.shape[1] : 0;
    const uint32_t group = k / std::max(groups, 1u);
    if (groups != 1 && (group < 8 || group > 256 || (group & (group - 1)) || group * groups != k))
      return fail(SV_ERR_ARG, "%s: %u groups per row of %u", scale.c_str(), groups, k);
    if (s.dtype != 1 || s.ndim != 2 || s.shape[0] != m)
      return fail(SV_ERR_ARG, "%s: expected Bf16 [%u, %u]", scale.c_str(), m, groups);
    gshift = groups == 1 ? 31u : (uint32_t)__builtin_ctz(group);
  }
  void* d = nullptr;
  SV_TRY(sv_weights_device(w, name, &d));
  *out = sv_matrix{d, nullptr, m, k, t.dtype == 2 ? (uint32_t)SV_FMT_I8 : (uint32_t)SV_FMT_BF16, gshift};
  if (t.dtype == 2) {
    void* ds = nullptr;
    SV_TRY(sv_weights_device(w, scale.c_str(), &ds));
    out->d_scales = (const uint16_t*)ds;
  }
  return SV_OK;
}

extern "C" void sv_weights_close(sv_weights* w) {
  if (!w) return;
  if (w->device) (void)hipFree(w->device);
  delete w;
}
