// pack.hip - the pack reader's I/O: a byte range of a pack shard file streamed into device memory. Replaces the shard
// upload loop of the reference's PackStore.upload (engine/core/store.js:221-244), which reads a shard in 16 MB chunks
// (with one read ahead) and writes each into the GPU buffer. Here two pinned host buffers alternate: while one chunk
// is copied to the device (an asynchronous copy on the library's stream), the next is read from the file into the
// other, so disk reads overlap the PCIe copies. The manifest (names, shards, offsets, encodings) is the host's
// business (p0pc0rn_amd/js/core/store.mjs); this is the part that moves the bytes.
#include "common.hpp"

#include <fcntl.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

namespace p0 {

constexpr size_t kPackChunk = 16u << 20;   // engine/core/store.js:224 (CH)

struct Staging {
  void* host[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int device = -1;
};
static Staging g_stage;

static int staging_ready(const char* op) {
  Staging& s = g_stage;
  if (s.device == ctx().device && s.host[0]) return P0_OK;
  for (int i = 0; i < 2; ++i) {   // pinned memory allocated as such (never registered after the fact)
    if (!s.host[i]) P0_HIP(hipHostMalloc(&s.host[i], kPackChunk, hipHostMallocDefault), op);
    if (!s.done[i]) P0_HIP(hipEventCreateWithFlags(&s.done[i], hipEventDisableTiming), op);
  }
  s.device = ctx().device;
  return P0_OK;
}

}  // namespace p0

using namespace p0;

extern "C" int p0_upload_file(const char* path, int64_t offset, int64_t bytes, void* dst, int64_t dst_off) {
  if (!path || !dst) { set_error("upload_file: no path or destination"); return P0_EINVAL; }
  if (offset < 0 || bytes < 0 || dst_off < 0) { set_error("upload_file: negative offset or size"); return P0_EINVAL; }
  if (int r = require_open("upload_file")) return r;
  if (bytes == 0) return P0_OK;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) { set_error("upload_file: %s: %s", path, strerror(errno)); return P0_EINVAL; }
  int rc = staging_ready("upload_file");
  Staging& s = g_stage;
  int64_t done_b = 0;
  for (int i = 0; rc == P0_OK && done_b < bytes; i ^= 1) {
    const size_t len = (size_t)(bytes - done_b < (int64_t)kPackChunk ? bytes - done_b : (int64_t)kPackChunk);
    hipError_t e = hipEventSynchronize(s.done[i]);   // the copy that last used this staging buffer is finished
    if (e != hipSuccess) { rc = fail_hip(e, "upload_file"); break; }
    size_t got = 0;
    while (got < len) {
      const ssize_t n = pread(fd, (uint8_t*)s.host[i] + got, len - got, (off_t)(offset + done_b + (int64_t)got));
      if (n < 0 && errno == EINTR) continue;
      if (n <= 0) {
        set_error("upload_file: %s: %s at byte %lld", path, n < 0 ? strerror(errno) : "end of file",
                  (long long)(offset + done_b + (int64_t)got));
        rc = P0_EINVAL;
        break;
      }
      got += (size_t)n;
    }
    if (rc != P0_OK) break;
    e = hipMemcpyAsync((uint8_t*)dst + dst_off + done_b, s.host[i], len, hipMemcpyHostToDevice, ctx().cur);
    if (e == hipSuccess) e = hipEventRecord(s.done[i], ctx().cur);
    if (e != hipSuccess) { rc = fail_hip(e, "upload_file"); break; }
    done_b += (int64_t)len;
  }
  close(fd);
  // the staging buffers are reused by the next call: wait for this call's copies either way
  hipError_t e0 = hipEventSynchronize(s.done[0]), e1 = hipEventSynchronize(s.done[1]);
  if (rc == P0_OK && e0 != hipSuccess) rc = fail_hip(e0, "upload_file");
  if (rc == P0_OK && e1 != hipSuccess) rc = fail_hip(e1, "upload_file");
  return rc;
}
