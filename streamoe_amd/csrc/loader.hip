// loader.hip — expert arena loader (host code): layer-file layout detection
// and file -> device copies through pinned staging buffers.
#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/smoe.h"
#include "handle.h"

namespace {

constexpr uint64_t kStageBytes = 32ull << 20;  // per staging buffer

uint64_t blob_bytes(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t bits) {
  const smoe_expert_shape s{hidden, inter, group, bits};
  return smoe_expert_bytes(&s);
}

// ExpertLayout::from_expert_size (variants.rs:442-450): 4-bit, then 3-bit.
uint32_t bits_of_size(uint64_t size, uint32_t hidden, uint32_t inter, uint32_t group) {
  if (size == blob_bytes(hidden, inter, group, 4)) return 4;
  if (size == blob_bytes(hidden, inter, group, 3)) return 3;
  return 0;
}

int ensure_staging(smoe_handle* h) {
  if (h->stage[0]) return SMOE_OK;
  for (int i = 0; i < 2; ++i) {
    if (hipHostMalloc(&h->stage[i], kStageBytes, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&h->stage_done[i], hipEventDisableTiming) != hipSuccess) {
      release_staging(h);
      return SMOE_ERR_HIP;
    }
  }
  h->stage_bytes = kStageBytes;
  return SMOE_OK;
}

// Reads exactly n bytes at off (retrying short reads); false on error/EOF.
bool read_full(int fd, void* buf, uint64_t n, uint64_t off) {
  uint8_t* p = static_cast<uint8_t*>(buf);
  while (n) {
    const ssize_t r = pread(fd, p, n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    p += r;
    n -= (uint64_t)r;
    off += (uint64_t)r;
  }
  return true;
}

}  // namespace

void release_staging(smoe_handle* h) {
  for (int i = 0; i < 2; ++i) {
    if (h->stage_done[i]) (void)hipEventSynchronize(h->stage_done[i]);
    if (h->stage_done[i]) (void)hipEventDestroy(h->stage_done[i]);
    if (h->stage[i]) (void)hipHostFree(h->stage[i]);
    h->stage[i] = nullptr;
    h->stage_done[i] = nullptr;
  }
  h->stage_bytes = 0;
}

extern "C" int smoe_layer_file_layout(uint64_t file_bytes, uint32_t n_experts, uint32_t hidden,
                                      uint32_t inter, uint32_t group, uint64_t declared_size,
                                      uint64_t declared_stride, smoe_file_layout* out) {
  if (!out || !n_experts || !hidden || !inter || !group || hidden % group) return SMOE_ERR_INVALID_ARG;
  // layout_and_stride (expert_io.rs:253-267): a declared padded stride.
  if (declared_stride > declared_size) {
    const uint32_t b = bits_of_size(declared_size, hidden, inter, group);
    if (b && file_bytes == (uint64_t)n_experts * declared_stride) {
      *out = smoe_file_layout{b, 0, declared_size, declared_stride};
      return SMOE_OK;
    }
  }
  // layout_of_len (expert_io.rs:229-237): the layout whose n blobs fill the
  // file, else 4-bit.
  uint32_t b = 0;
  if (file_bytes % n_experts == 0) b = bits_of_size(file_bytes / n_experts, hidden, inter, group);
  if (!b) b = 4;
  const uint64_t size = blob_bytes(hidden, inter, group, b);
  *out = smoe_file_layout{b, 0, size, size};
  return SMOE_OK;
}

extern "C" int smoe_load_file(smoe_handle* h, const char* path, uint64_t offset, uint64_t bytes,
                              void* dst, uint64_t dst_bytes, uint64_t* bytes_read) {
  if (bytes_read) *bytes_read = 0;
  if (!h || !path || !dst) return SMOE_ERR_INVALID_ARG;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return SMOE_ERR_IO;
  struct stat st;
  if (fstat(fd, &st) != 0 || (uint64_t)st.st_size < offset) {
    close(fd);
    return SMOE_ERR_IO;
  }
  if (bytes == 0) bytes = (uint64_t)st.st_size - offset;
  if (offset + bytes > (uint64_t)st.st_size) {
    close(fd);
    return SMOE_ERR_IO;
  }
  if (bytes > dst_bytes) {
    close(fd);
    return SMOE_ERR_INVALID_ARG;
  }
  if (hipSetDevice(h->device) != hipSuccess) {
    close(fd);
    return SMOE_ERR_HIP;
  }
  if (int rc = ensure_staging(h)) {
    close(fd);
    return rc;
  }
  // Double buffering: the read into one staging buffer overlaps the copy
  // out of the other; a buffer is refilled only after its copy finished.
  int rc = SMOE_OK;
  uint64_t done = 0;
  for (uint64_t i = 0; done < bytes; ++i) {
    const int b = (int)(i & 1);
    const uint64_t n = bytes - done < h->stage_bytes ? bytes - done : h->stage_bytes;
    if (hipEventSynchronize(h->stage_done[b]) != hipSuccess) {
      rc = SMOE_ERR_HIP;
      break;
    }
    if (!read_full(fd, h->stage[b], n, offset + done)) {
      rc = SMOE_ERR_IO;
      break;
    }
    if (hipMemcpyAsync(static_cast<uint8_t*>(dst) + done, h->stage[b], n, hipMemcpyHostToDevice, h->stream) !=
            hipSuccess ||
        hipEventRecord(h->stage_done[b], h->stream) != hipSuccess) {
      rc = SMOE_ERR_HIP;
      break;
    }
    done += n;
  }
  close(fd);
  for (int b = 0; b < 2; ++b)
    if (hipEventSynchronize(h->stage_done[b]) != hipSuccess && rc == SMOE_OK) rc = SMOE_ERR_HIP;
  if (rc == SMOE_OK && bytes_read) *bytes_read = done;
  return rc;
}
