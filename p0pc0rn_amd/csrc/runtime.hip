// runtime.hip - device context, buffers, stream and timing: the part of the reference's Gpu object
// (engine/core/gpu.js:18-147) that the q4 ops need, on one gfx950 device.
#include "common.hpp"

#include <cstring>

namespace p0 {

Ctx& ctx() {
  static Ctx* c = new Ctx();   // never destroyed: nothing of it is released after the HIP runtime at process exit
  return *c;
}

void keep_for_recording(const Keep& k) {
  Ctx& c = ctx();
  if (c.recording && k) c.rec_keeps.push_back(k);
}

// a recording: the instantiated graph and the library memory its kernels read
struct Rec {
  hipGraphExec_t exec = nullptr;
  std::vector<Keep> keeps;
  int32_t nodes = 0;
};

static thread_local std::string g_err;

int ensure_xstage(size_t bytes, const char* op) {
  Ctx& c = ctx();
  if (bytes <= c.xstage_bytes) return P0_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(c.cur, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
    set_error("%s: the activation staging workspace needs %zu B; run the call once before recording it", op, bytes);
    return P0_EINVAL;
  }
  size_t want = bytes < (256ull << 20) ? (256ull << 20) : (bytes + (1ull << 20) - 1) / (1ull << 20) * (1ull << 20);
  P0_HIP(hipStreamSynchronize(c.cur), op);   // the old buffer may still be read by enqueued work
  // the old buffer is released here unless a recording captured a kernel that reads it: then it lives on until the
  // last such recording is freed (p0_record_free)
  c.xstage_keep.reset();
  c.xstage = nullptr;
  c.xstage_bytes = 0;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    set_error("%s: activation staging workspace of %zu B: %s", op, want, hipGetErrorString(e));
    return P0_ENOMEM;
  }
  c.xstage_keep = Keep(p, [](void* q) { hipFree(q); });
  c.xstage = p;
  c.xstage_bytes = want;
  return P0_OK;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
}

// 32-bit pattern fill (the NaN-fill that proves a kernel wrote its output, engine/tune/autotune.js:1-7)
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint32_t v, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

// buffer copy (engine/core/gpu.js:237-242 runner.copy). 16 bytes per lane when source, destination and size allow it:
// the same request shape as the GEMV's record loads, which makes it the calibration kernel for HBM byte counters.
__global__ void copy16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = src[i];
}
__global__ void copy4_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = src[i];
}

}  // namespace p0

using namespace p0;

// Split-K workspace: 64 MiB of partial sums and 1 Mi arrival counters per device, in uncached device memory. The
// partials then reach memory when their stores are acknowledged and are read from memory, so the arrival protocol
// needs no L2 write-back or invalidate (a device-scope fence costs a write-back of the XCD's whole L2). Uncached memory
// that a kernel has read is never freed while the process runs (allocations made after such a free have been seen
// holding wrong values), so each device's workspace is allocated once and kept across p0_close / p0_open.
static constexpr size_t kPartBytes = 64ull << 20;
static constexpr size_t kCounters = 1ull << 20;
static constexpr int kWsDevices = 64;
static float* g_ws_part[kWsDevices] = {};
static unsigned* g_ws_cnt[kWsDevices] = {};

extern "C" {

const char* p0_last_error(void) { return g_err.c_str(); }
int p0_version(void) { return P0_ABI_VERSION; }

int p0_open(int device) {
  Ctx& c = ctx();
  if (c.device >= 0) {
    if (c.device == device) return P0_OK;
    set_error("p0_open: already open on device %d", c.device);
    return P0_EINVAL;
  }
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= device || device < 0) {
    set_error("p0_open: no HIP device %d (%d visible)", device, e == hipSuccess ? n : 0);
    return P0_ENODEV;
  }
  if (device >= kWsDevices) {
    set_error("p0_open: device %d (this build keeps workspaces for devices 0 .. %d)", device, kWsDevices - 1);
    return P0_ENODEV;
  }
  P0_HIP(hipSetDevice(device), "p0_open");
  P0_HIP(hipGetDeviceProperties(&c.prop, device), "p0_open");
  if (std::strncmp(c.prop.gcnArchName, "gfx950", 6) != 0) {
    set_error("p0_open: device %d is %s; this library is built for gfx950 (MI355X) only", device, c.prop.gcnArchName);
    return P0_ENODEV;
  }
  P0_HIP(hipStreamCreate(&c.own), "p0_open");   // default priority
  P0_HIP(hipEventCreate(&c.ev0), "p0_open");
  P0_HIP(hipEventCreate(&c.ev1), "p0_open");
  if (!g_ws_part[device]) {
    P0_HIP(hipExtMallocWithFlags((void**)&g_ws_part[device], kPartBytes, hipDeviceMallocUncached), "p0_open: workspace");
  }
  if (!g_ws_cnt[device]) {
    P0_HIP(hipExtMallocWithFlags((void**)&g_ws_cnt[device], kCounters * sizeof(unsigned), hipDeviceMallocUncached),
           "p0_open: workspace");
  }
  c.part = g_ws_part[device];
  c.counters = g_ws_cnt[device];
  P0_HIP(hipMemset(c.counters, 0, kCounters * sizeof(unsigned)), "p0_open: workspace");
  P0_HIP(hipDeviceSynchronize(), "p0_open");
  if (int r = gemm_init()) return r;
  if (int r = gemv_init()) return r;
  if (int r = misc_init()) return r;
  c.part_floats = kPartBytes / sizeof(float);
  c.n_counters = kCounters;
  c.cur = c.own;
  c.cu_count = c.prop.multiProcessorCount;
  c.device = device;
  return P0_OK;
}

int p0_close(void) {
  Ctx& c = ctx();
  if (c.device < 0) return P0_OK;
  (void)hipStreamSynchronize(c.own);   // the split-K workspace stays allocated (see g_ws_part)
  c.xstage_keep.reset();   // freed unless a recording still holds it
  hipEventDestroy(c.ev0);
  hipEventDestroy(c.ev1);
  hipStreamDestroy(c.own);
  c = Ctx{};
  return P0_OK;
}

int p0_device_info(p0_device_info_t* out) {
  if (int r = require_open("p0_device_info")) return r;
  Ctx& c = ctx();
  std::memset(out, 0, sizeof *out);
  std::strncpy(out->name, c.prop.gcnArchName, sizeof out->name - 1);
  out->device = c.device;
  out->cu_count = c.cu_count;
  out->xcd_count = c.cu_count / 32;
  out->hbm_bytes = (int64_t)c.prop.totalGlobalMem;
  out->lds_bytes_per_cu = (int64_t)c.prop.maxSharedMemoryPerMultiProcessor;
  out->clock_khz = c.prop.clockRate;
  out->workspace_bytes = (int64_t)(kPartBytes + kCounters * sizeof(unsigned));
  return P0_OK;
}

int p0_set_stream(void* stream) {
  if (int r = require_open("p0_set_stream")) return r;
  ctx().cur = stream ? (hipStream_t)stream : ctx().own;
  return P0_OK;
}
void* p0_get_stream(void) { return (void*)ctx().cur; }

int p0_buffer(size_t bytes, void** out) {   // Gpu.buffer: at least 16 B, rounded up to 16 B
  if (int r = require_open("p0_buffer")) return r;
  size_t size = bytes < 16 ? 16 : (bytes + 15) / 16 * 16;
  hipError_t e = hipMalloc(out, size);
  if (e != hipSuccess) {
    *out = nullptr;
    set_error("buffer %zu B: %s", size, hipGetErrorString(e));
    return P0_ENOMEM;
  }
  return P0_OK;
}

int p0_free(void* buf) {
  if (int r = require_open("p0_free")) return r;
  if (!buf) return P0_OK;
  P0_HIP(hipStreamSynchronize(ctx().cur), "p0_free");   // never free under a running op
  P0_HIP(hipFree(buf), "p0_free");
  return P0_OK;
}

int p0_upload(void* dst, size_t dst_off, const void* src, size_t bytes) {
  if (int r = require_open("p0_upload")) return r;
  if (!bytes) return P0_OK;
  P0_HIP(hipMemcpyAsync((char*)dst + dst_off, src, bytes, hipMemcpyHostToDevice, ctx().cur), "p0_upload");
  P0_HIP(hipStreamSynchronize(ctx().cur), "p0_upload");   // the host copy may be reused when this returns
  return P0_OK;
}

int p0_read(void* host_dst, const void* src, size_t src_off, size_t bytes) {
  if (int r = require_open("p0_read")) return r;
  if (!bytes) return P0_OK;
  P0_HIP(hipMemcpyAsync(host_dst, (const char*)src + src_off, bytes, hipMemcpyDeviceToHost, ctx().cur), "p0_read");
  P0_HIP(hipStreamSynchronize(ctx().cur), "p0_read");
  return P0_OK;
}

int p0_fill(void* dst, size_t dst_off, uint32_t value, size_t words) {
  if (int r = require_open("p0_fill")) return r;
  if ((dst_off & 3) || ((uintptr_t)dst & 3)) {
    set_error("p0_fill: destination must be 4-byte aligned");
    return P0_EINVAL;
  }
  if (!words) return P0_OK;
  size_t blocks = (words + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx().cur,
                     (uint32_t*)((char*)dst + dst_off), value, words);
  P0_LAUNCHED("p0_fill");
  return P0_OK;
}

int p0_copy(const void* src, size_t src_off, void* dst, size_t dst_off, size_t bytes) {
  if (int r = require_open("p0_copy")) return r;
  const char* a = (const char*)src + src_off;
  char* b = (char*)dst + dst_off;
  if (((uintptr_t)a | (uintptr_t)b | bytes) & 3) {   // copyBufferToBuffer's rule: offsets and size multiples of 4
    set_error("p0_copy: offsets and size must be multiples of 4");
    return P0_EINVAL;
  }
  if (!bytes) return P0_OK;
  if ((a < b + bytes) && (b < a + bytes)) {
    set_error("p0_copy: source and destination overlap");
    return P0_EINVAL;
  }
  if (building_chain()) return chain_add_copy(a, b, (int64_t)(bytes / 4));   // a chain op (chain_aux.hpp)
  const bool wide = !(((uintptr_t)a | (uintptr_t)b | bytes) & 15);
  const size_t n = wide ? bytes / 16 : bytes / 4;
  size_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (wide) hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx().cur, (const uint4*)a, (uint4*)b, n);
  else hipLaunchKernelGGL(copy4_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx().cur, (const uint32_t*)a, (uint32_t*)b, n);
  P0_LAUNCHED("p0_copy");
  return P0_OK;
}

int p0_done(void) {   // Gpu.done: wait for everything enqueued; faults of earlier ops surface here
  if (int r = require_open("p0_done")) return r;
  P0_HIP(hipStreamSynchronize(ctx().cur), "p0_done");
  return P0_OK;
}

// ---- recorded op sequences (engine/llm/drunner.js:1-8, 83-101: one decode token recorded once, submitted per token)
int p0_record_begin(void) {
  if (int r = require_open("p0_record_begin")) return r;
  Ctx& c = ctx();
  if (c.recording) { set_error("p0_record_begin: a recording is already being made"); return P0_EINVAL; }
  P0_HIP(hipStreamBeginCapture(c.cur, hipStreamCaptureModeThreadLocal), "p0_record_begin");
  c.recording = true;
  c.rec_keeps.clear();
  return P0_OK;
}

int p0_record_end(void** out) {
  if (int r = require_open("p0_record_end")) return r;
  Ctx& c = ctx();
  std::vector<Keep> keeps;
  keeps.swap(c.rec_keeps);
  c.recording = false;
  hipGraph_t graph = nullptr;
  P0_HIP(hipStreamEndCapture(c.cur, &graph), "p0_record_end");
  size_t nodes = 0;
  hipGraphGetNodes(graph, nullptr, &nodes);
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  hipGraphDestroy(graph);
  if (e != hipSuccess) return fail_hip(e, "p0_record_end: instantiate");
  Rec* rec = new Rec();
  rec->exec = exec;
  rec->keeps = std::move(keeps);
  rec->nodes = (int32_t)nodes;
  *out = (void*)rec;
  return P0_OK;
}

int p0_replay(void* rec) {
  if (int r = require_open("p0_replay")) return r;
  if (!rec) { set_error("p0_replay: no recording"); return P0_EINVAL; }
  P0_HIP(hipGraphLaunch(((Rec*)rec)->exec, ctx().cur), "p0_replay");
  return P0_OK;
}

int p0_record_info(void* rec, int32_t* nodes) {
  if (!rec || !nodes) { set_error("p0_record_info: no recording or output"); return P0_EINVAL; }
  *nodes = ((Rec*)rec)->nodes;
  return P0_OK;
}

int p0_record_free(void* rec) {
  if (!rec) return P0_OK;
  Rec* r = (Rec*)rec;
  if (ctx().device >= 0) hipStreamSynchronize(ctx().cur);   // replays still enqueued read what the recording holds
  hipError_t e = hipGraphExecDestroy(r->exec);
  delete r;   // releases the memory only this recording still held
  if (e != hipSuccess) return fail_hip(e, "p0_record_free");
  return P0_OK;
}

int p0_timer_start(void) {
  if (int r = require_open("p0_timer_start")) return r;
  P0_HIP(hipEventRecord(ctx().ev0, ctx().cur), "p0_timer_start");
  return P0_OK;
}

int p0_timer_stop(float* ms) {
  if (int r = require_open("p0_timer_stop")) return r;
  P0_HIP(hipEventRecord(ctx().ev1, ctx().cur), "p0_timer_stop");
  P0_HIP(hipEventSynchronize(ctx().ev1), "p0_timer_stop");
  P0_HIP(hipEventElapsedTime(ms, ctx().ev0, ctx().ev1), "p0_timer_stop");
  return P0_OK;
}

}  // extern "C"
