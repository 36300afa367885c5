// pack.hip -- opening and reading a Hale expert pack (src/expert/pack.rs).
//
// Layout (PackWriter::create, src/expert/pack.rs:148-164):
//   offset 0      "HALEPACK"
//   offset 8      u64 LE length of the JSON header
//   offset 16     JSON PackHeader
//   data_offset   record (moe layer ordinal 0, expert 0), (0, 1), ...
// Every record is gate | up | down in the pack dtype, record_stride apart.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>

#include "pack.h"

namespace hale {

namespace {

constexpr char MAGIC[8] = {'H', 'A', 'L', 'E', 'P', 'A', 'C', 'K'};
constexpr uint32_t FORMAT_VERSION = 1;
constexpr size_t ALIGN = 16 * 1024;  // record alignment, src/expert/pack.rs:50

}  // namespace

bool pack_pread(const hale_pack* p, void* dst, size_t n, uint64_t off, std::string* err) {
  char* d = (char*)dst;
  while (n > 0) {
    const ssize_t r = ::pread(p->fd, d, n, (off_t)off);
    if (r < 0) {
      if (errno == EINTR) continue;
      *err = p->path + ": " + strerror(errno);
      return false;
    }
    if (r == 0) {
      *err = p->path + ": unexpected end of file";
      return false;
    }
    d += r;
    n -= (size_t)r;
    off += (uint64_t)r;
  }
  return true;
}

}  // namespace hale

using hale::ctx_fail;

extern "C" int hale_pack_open(const char* path, hale_pack** out) {
  hale_ctx* const c = nullptr;  // context-free: failures go to the calling thread's message
  if (!path || !out) return ctx_fail(c, HALE_EINVAL, "pack_open: NULL argument");
  *out = nullptr;
  hale_pack* p = new (std::nothrow) hale_pack;
  if (!p) return ctx_fail(c, HALE_ENOMEM, "out of host memory");
  p->path = path;
  auto bail = [&](int code, const std::string& msg) {
    if (p->fd >= 0) ::close(p->fd);
    delete p;
    return ctx_fail(c, code, "%s", msg.c_str());
  };
  p->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (p->fd < 0) return bail(HALE_EIO, std::string(path) + ": " + strerror(errno));
  struct stat st;
  if (fstat(p->fd, &st) != 0) return bail(HALE_EIO, std::string(path) + ": " + strerror(errno));
  const size_t actual = (size_t)st.st_size;
  unsigned char prefix[16];
  std::string err;
  if (actual < 16 || !hale::pack_pread(p, prefix, 16, 0, &err) ||
      memcmp(prefix, hale::MAGIC, 8) != 0)
    return bail(HALE_EPACK, std::string(path) + " is not a Hale expert pack");
  uint64_t json_len = 0;
  for (int i = 7; i >= 0; i--) json_len = (json_len << 8) | prefix[8 + i];
  if (json_len > hale::ALIGN * 64) return bail(HALE_EPACK, std::string(path) + ": header too large");
  std::string json((size_t)json_len, '\0');
  if (!hale::pack_pread(p, &json[0], (size_t)json_len, 16, &err)) return bail(HALE_EPACK, err);
  if (!hale::parse_pack_header(json.data(), json.size(), &p->h, &err))
    return bail(HALE_EPACK, std::string(path) + ": header: " + err);
  if (p->h.version != hale::FORMAT_VERSION)
    return bail(HALE_EPACK, std::string(path) + ": pack version " + std::to_string(p->h.version) +
                                " is not supported (expected 1)");
  if (actual < p->h.file_size())
    return bail(HALE_EPACK, std::string(path) + ": truncated pack (" + std::to_string(actual) +
                                " bytes, expected " + std::to_string(p->h.file_size()) + ")");
  if (p->h.record_stride < p->h.record_bytes)
    return bail(HALE_EPACK, std::string(path) + ": record_stride below record_bytes");
  *out = p;
  return HALE_OK;
}

extern "C" int hale_pack_info(const hale_pack* p, int* dtype, size_t* hidden, size_t* inter,
                              size_t* num_experts, size_t* num_moe_layers, size_t* record_bytes,
                              size_t* record_stride, size_t* data_offset) {
  if (!p) return HALE_EINVAL;
  if (dtype) *dtype = p->h.dtype;
  if (hidden) *hidden = p->h.hidden;
  if (inter) *inter = p->h.inter;
  if (num_experts) *num_experts = p->h.num_experts;
  if (num_moe_layers) *num_moe_layers = p->h.moe_layers.size();
  if (record_bytes) *record_bytes = p->h.record_bytes;
  if (record_stride) *record_stride = p->h.record_stride;
  if (data_offset) *data_offset = p->h.data_offset;
  return HALE_OK;
}

extern "C" int hale_pack_moe_layer(const hale_pack* p, size_t ordinal, uint32_t* layer) {
  if (!p || !layer) return HALE_EINVAL;
  if (ordinal >= p->h.moe_layers.size())
    return ctx_fail(nullptr, HALE_EINVAL, "MoE layer ordinal %zu of %zu", ordinal, p->h.moe_layers.size());
  *layer = (uint32_t)p->h.moe_layers[ordinal];
  return HALE_OK;
}

extern "C" int hale_pack_offset_of(const hale_pack* p, uint32_t layer, uint32_t expert,
                                   uint64_t* offset) {
  if (!p || !offset) return HALE_EINVAL;
  std::string err;
  if (!hale::pack_offset_of(p->h, layer, expert, offset, &err))
    return ctx_fail(nullptr, HALE_EPACK, "%s", err.c_str());
  return HALE_OK;
}

extern "C" int hale_pack_read_expert(hale_pack* p, uint32_t layer, uint32_t expert, void* buf,
                                     size_t nbytes) {
  if (!p || !buf) return ctx_fail(nullptr, HALE_EINVAL, "pack_read_expert: NULL argument");
  if (nbytes != p->h.record_bytes)
    return ctx_fail(nullptr, HALE_EINVAL, "record is %zu bytes, buffer %zu", p->h.record_bytes, nbytes);
  uint64_t off = 0;
  std::string err;
  if (!hale::pack_offset_of(p->h, layer, expert, &off, &err))
    return ctx_fail(nullptr, HALE_EPACK, "%s", err.c_str());
  if (!hale::pack_pread(p, buf, nbytes, off, &err)) return ctx_fail(nullptr, HALE_EIO, "%s", err.c_str());
  return HALE_OK;
}
