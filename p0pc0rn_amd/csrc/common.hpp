// common.hpp - shared state and helpers of the gfx950 q4 matmul library (see include/p0pc0rn.h for the C ABI).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <memory>
#include <string>
#include <vector>

#include "../../include/p0pc0rn.h"

namespace p0 {

// Device memory of the library's own that kernels read (the activation staging workspace, a chain's op table and
// state), held by shared ownership: a recording (p0_record_*) whose captured kernels read such memory holds a
// reference, so the memory outlives a later growth of the workspace or a p0_chain_free until the recording is freed.
using Keep = std::shared_ptr<void>;
void keep_for_recording(const Keep& k);   // the recording being made on the current stream, if any, holds k

// The per-process library context: one device, one current stream, one split-K workspace.
struct Ctx {
  int device = -1;
  hipStream_t own = nullptr;   // created by p0_open
  hipStream_t cur = nullptr;   // where ops are enqueued (own unless p0_set_stream)
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  // split-K workspace: partial sums of the K-slices of a call, and one arrival counter per (split, tile block).
  // Counters start at zero (cleared once by p0_open) and the last workgroup to arrive resets its counter, so every
  // call leaves them at zero again: no memset per call, which also keeps calls capturable into HIP graphs.
  float* part = nullptr;
  size_t part_floats = 0;
  unsigned* counters = nullptr;
  size_t n_counters = 0;
  // fp16 staging of GEMM activations that the MFMA kernel cannot stream as they are (bf16, the f32 prologues,
  // misaligned fp16): grown on demand, never inside a stream capture (ensure_xstage)
  void* xstage = nullptr;
  size_t xstage_bytes = 0;
  Keep xstage_keep;                 // owns xstage (freed once no recording holds it)
  bool recording = false;           // between p0_record_begin and p0_record_end
  std::vector<Keep> rec_keeps;      // what the recording being made holds
  int cu_count = 0;
  hipDeviceProp_t prop{};
};
Ctx& ctx();
int ensure_xstage(size_t bytes, const char* op);   // P0_OK, or an error (no room while the stream is being captured)
// per-file set-up at p0_open (kernel attributes; the no-allocation GEMM's scratch address)
int gemm_init();
int gemv_init();
int misc_init();

// Thread-local message of the last failure (p0_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline int fail_hip(hipError_t e, const char* what) {
  set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return P0_EHIP;
}
inline int require_open(const char* op) {
  if (ctx().device < 0) {
    set_error("%s: no device (p0_open was not called)", op);
    return P0_ENODEV;
  }
  return P0_OK;
}
// true between p0_chain_begin and p0_chain_end (gemv.hip): gemv / gemvM, copy, argmax / argmaxM, rowstats and normadd
// calls join a chain; every other op (the GEMM, the dequant, uploads) refuses to run meanwhile instead of running out of
// order
bool building_chain();
// ops that are not GEMVs join the chain being built (gemv.hip; the pipelined chain kernel runs them, chain_aux.hpp)
int chain_add_copy(const void* src, void* dst, int64_t words);
int chain_add_argmax(const float* mx, int64_t n, int64_t M, uint32_t* out);
int chain_add_rowstats(const float* x, int64_t ld, int64_t c0, int64_t rows, int64_t cols, int mode, float eps,
                       float* st, int64_t st_off);
int chain_add_normadd(const float* t, int64_t nsrc, int64_t ldp, const float* w, int64_t w_off, float* x, float* st,
                      int64_t st_off, int64_t D, int64_t M, float eps, float scale, int mode);
inline int refuse_in_chain(const char* op) {
  if (building_chain()) {
    set_error("%s: only gemv / gemvM, copy, argmax, rowstats and normadd calls join a chain (a chain is being built)", op);
    return P0_EINVAL;
  }
  return P0_OK;
}

#define P0_HIP(call, what)                         \
  do {                                             \
    hipError_t e_ = (call);                        \
    if (e_ != hipSuccess) return fail_hip(e_, what); \
  } while (0)

// Kernel launches report configuration errors through hipGetLastError; asynchronous faults surface at p0_done.
#define P0_LAUNCHED(what)                          \
  do {                                             \
    hipError_t e_ = hipGetLastError();             \
    if (e_ != hipSuccess) return fail_hip(e_, what); \
  } while (0)

}  // namespace p0
