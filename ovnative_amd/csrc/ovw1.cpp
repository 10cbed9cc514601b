// OVW1 weight-file reader (cpp/include/ovnative/ov_weights.h, cpp/src/core/
// weight_file.cpp; format in docs/weight-format.en.md): the file is mapped
// read-only and every tensor is exposed as an OvhTensorView pointing into the
// mapping, so opening a checkpoint costs one mmap plus the index walk.  The
// views feed ovh_lm_create(), which uploads what the HIP runner needs.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdint>
#include <cstring>
#include <deque>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ovnative_amd.h"

namespace ovh {
int set_error(int code, const std::string& msg);
}

struct OvhWeightFile {
  void* base = nullptr;
  size_t size = 0;
  uint64_t n_params = 0;
  int dtype_mode = 0;
  std::deque<std::string> names;  // stable storage for view.name
  std::vector<OvhTensorView> views;
  std::unordered_map<std::string, int> index;
  ~OvhWeightFile() {
    if (base) ::munmap(base, size);
  }
};

namespace {

// On-disk records, little-endian (docs/weight-format.en.md "Header" and
// "TensorDesc"); the header block is 128 bytes of which these 72 are used.
#pragma pack(push, 1)
struct FileHeader {
  char magic[8];
  uint32_t version, dtype_mode, n_tensors, header_bytes;
  uint64_t index_off, names_off, data_off, file_size, flags, n_params;
};
struct FileDesc {
  uint32_t name_off, name_len;
  uint8_t dtype, ndim, layout, quant;
  uint32_t dims[4];
  uint32_t aux_n;
  uint64_t hash, data_off, nbytes, aux_off;
};
#pragma pack(pop)
static_assert(sizeof(FileHeader) == 72, "OVW1 header layout");
static_assert(sizeof(FileDesc) == 64, "OVW1 descriptor layout");

constexpr char kMagic[8] = {'O', 'M', 'N', 'I', 'V', 'O', 'I', 'C'};

int bad(const std::string& msg) { return ovh::set_error(OV_ERR_IO, "OVW1: " + msg); }

int64_t dtype_bytes(int dt) {
  switch (dt) {
    case 0: return 4;  // f32
    case 1: return 1;  // i8
    case 2: return 2;  // f16
    case 3: return 8;  // i64
    default: return 0;
  }
}

// CRC-32 (IEEE 802.3, reflected, poly 0xEDB88320): zlib.crc32, which the
// converter stores per payload.
uint32_t crc32(const uint8_t* p, size_t n) {
  static uint32_t table[256];
  static bool ready = false;
  if (!ready) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c >> 1) ^ (0xEDB88320u & (0u - (c & 1u)));
      table[i] = c;
    }
    ready = true;
  }
  uint32_t c = 0xFFFFFFFFu;
  for (size_t i = 0; i < n; ++i) c = table[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
  return ~c;
}

int parse(OvhWeightFile& wf) {
  const char* base = static_cast<const char*>(wf.base);
  const size_t size = wf.size;
  FileHeader h;
  std::memcpy(&h, base, sizeof h);
  if (std::memcmp(h.magic, kMagic, 8) != 0) return bad("bad magic (not an OVW1 file)");
  if (h.version != 1) return bad("unsupported version " + std::to_string(h.version));
  if (h.file_size != size)
    return bad("file size mismatch: header says " + std::to_string(h.file_size) + ", actual " +
               std::to_string(size));
  const uint64_t index_end = h.index_off + (uint64_t)h.n_tensors * sizeof(FileDesc);
  if (h.index_off < sizeof(FileHeader) || index_end > size || index_end < h.index_off)
    return bad("index out of bounds");
  wf.n_params = h.n_params;
  wf.dtype_mode = (int)h.dtype_mode;
  wf.views.reserve(h.n_tensors);
  for (uint32_t i = 0; i < h.n_tensors; ++i) {
    FileDesc d;
    std::memcpy(&d, base + h.index_off + (uint64_t)i * sizeof(FileDesc), sizeof d);
    const uint64_t nb = h.names_off + d.name_off;
    if (h.names_off > size || nb > size || d.name_len > size - nb) return bad("tensor name out of bounds");
    if (d.data_off > size || d.nbytes > size - d.data_off) return bad("tensor payload out of bounds");
    if (d.ndim > 4) return bad("tensor rank > 4");
    wf.names.emplace_back(base + nb, d.name_len);
    OvhTensorView v{};
    v.name = wf.names.back().c_str();
    v.dtype = d.dtype;
    v.ndim = d.ndim;
    int64_t numel = 1;
    for (int k = 0; k < 4; ++k) {
      v.dims[k] = k < d.ndim ? (int64_t)d.dims[k] : 0;
      if (k < d.ndim) numel *= (int64_t)d.dims[k];
    }
    v.transposed = d.layout == 1;
    v.quantized = d.quant == 1;
    v.data = base + d.data_off;
    v.nbytes = (int64_t)d.nbytes;
    v.crc = (uint32_t)(d.hash & 0xFFFFFFFFu);
    if (v.quantized) {
      if (d.aux_off > size || (uint64_t)d.aux_n * 4 > size - d.aux_off) return bad("scales out of bounds");
      if (d.aux_off % 4 != 0) return bad("misaligned scales");
      v.scales = reinterpret_cast<const float*>(base + d.aux_off);
      v.n_scales = d.aux_n;
    }
    const int64_t esz = dtype_bytes(d.dtype);
    if (esz == 0) return bad("unknown dtype for '" + wf.names.back() + "'");
    if (numel * esz != v.nbytes)
      return bad("size mismatch for '" + wf.names.back() + "': shape needs " +
                 std::to_string(numel * esz) + " bytes, descriptor says " + std::to_string(v.nbytes));
    wf.index.emplace(wf.names.back(), (int)wf.views.size());
    wf.views.push_back(v);
  }
  return OV_OK;
}

}  // namespace

extern "C" {

int ovh_ovw1_open(const char* path, OvhWeightFile** out) {
  if (!out) return ovh::set_error(OV_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!path) return ovh::set_error(OV_ERR_INVALID_ARG, "path is null");
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return bad(std::string("cannot open '") + path + "': " + std::strerror(errno));
  struct stat st {};
  if (::fstat(fd, &st) != 0) {
    ::close(fd);
    return bad(std::string("cannot stat '") + path + "'");
  }
  const size_t size = (size_t)st.st_size;
  if (size < sizeof(FileHeader)) {
    ::close(fd);
    return bad(std::string("'") + path + "' is smaller than a header");
  }
  void* base = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (base == MAP_FAILED) return bad(std::string("mmap failed for '") + path + "'");
  auto* wf = new (std::nothrow) OvhWeightFile();
  if (!wf) {
    ::munmap(base, size);
    return ovh::set_error(OV_ERR_INTERNAL, "out of host memory");
  }
  wf->base = base;
  wf->size = size;
  const int rc = parse(*wf);
  if (rc != OV_OK) {
    delete wf;
    return rc;
  }
  *out = wf;
  return OV_OK;
}

void ovh_ovw1_close(OvhWeightFile* wf) { delete wf; }

int ovh_ovw1_count(const OvhWeightFile* wf) { return wf ? (int)wf->views.size() : 0; }

const OvhTensorView* ovh_ovw1_tensors(const OvhWeightFile* wf) {
  return wf && !wf->views.empty() ? wf->views.data() : nullptr;
}

const OvhTensorView* ovh_ovw1_find(const OvhWeightFile* wf, const char* name) {
  if (!wf || !name) return nullptr;
  auto it = wf->index.find(name);
  return it == wf->index.end() ? nullptr : &wf->views[(size_t)it->second];
}

uint64_t ovh_ovw1_n_params(const OvhWeightFile* wf) { return wf ? wf->n_params : 0; }

uint32_t ovh_ovw1_compute_crc(const OvhWeightFile* wf, int index) {
  if (!wf || index < 0 || index >= (int)wf->views.size()) return 0;
  const OvhTensorView& v = wf->views[(size_t)index];
  return crc32(static_cast<const uint8_t*>(v.data), (size_t)v.nbytes);
}

}  // extern "C"
