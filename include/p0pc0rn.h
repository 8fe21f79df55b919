/*
 * p0pc0rn.h - C ABI of the MI355X (gfx950) int4 quantized-matmul library.
 *
 * This is the boundary the Node.js host (p0pc0rn_amd/js) binds through its N-API addon, and that Python binds
 * through ctypes. Every entry point takes plain pointers, sizes and enums; no torch or HIP types appear in the
 * signatures (streams are passed as opaque `void*`).
 *
 * The entry points replace the WebGPU dispatch underneath these reference functions (paths are relative to the
 * reference repository ArtistJoshHughes/p0pc0rn):
 *   p0_open / p0_close / p0_device_info  <- createGpu / Gpu.init / Gpu.describe   engine/core/gpu.js:18-78
 *   p0_buffer / p0_free                  <- Gpu.buffer / Gpu.free                 engine/core/gpu.js:81-95
 *   p0_upload / p0_read                  <- Gpu.upload / Gpu.read / readInto      engine/core/gpu.js:98-140
 *   p0_done                              <- Gpu.done                              engine/core/gpu.js:141-147
 *   p0_copy                              <- runner.copy                           engine/core/gpu.js:237-242
 *   p0_q4_gemv                           <- gemv(g, a)                            engine/llm/lops.js:108-141
 *   p0_q4_gemvM                          <- gemvM(g, a)                           engine/llm/lops_spec.js:159-191
 *   p0_q4_gemm                           <- gemm(gpu, a)                          engine/ops/gemm.js:255-322
 *   p0_q4_dequant                        <- the q4g32a.t64 unpacking of            engine/kcheck.js:22-38 (packQ4 deq),
 *                                           engine/ops/gemm.js:139-149 (fp16 tile) and engine/core/store.js:276-301
 *   p0_rowstats                          <- rowstats(gpu, a)                      engine/ops/misc.js:13-40
 *   p0_normadd                           <- normadd(g, a)                         engine/llm/lops.js:143-178
 *   p0_argmax / p0_argmaxM               <- argmax(g, a) / argmaxM(g, a)          engine/llm/lops.js:416-436,
 *                                                                                 engine/llm/lops_spec.js:327-348
 *   p0_upload_file                       <- PackStore.upload's shard streaming    engine/core/store.js:221-244
 *
 * Error behaviour: every function returns P0_OK (0) or a nonzero status. On failure, p0_last_error() returns the
 * message of the calling thread's last failure. Argument errors carry the reference's own text (for example
 * "gemv: N % 64" or "gemm: K must be a multiple of 32"), so a host shim can rethrow them as `new Error(msg)`
 * exactly where the reference throws. Argument validation runs before any device work, so it needs no GPU.
 *
 * Threading and streams: one library context per process, on the device given to p0_open. Ops are enqueued on the
 * library's current stream (p0_set_stream, default: a stream created by p0_open) and return immediately; p0_done
 * waits for them. The split-K workspace is shared by all ops of the context, so ops must not run concurrently on two
 * streams of one context.
 */
#ifndef P0PC0RN_H
#define P0PC0RN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------------------------------- */
enum {
  P0_OK = 0,
  P0_EINVAL = 1,   /* argument validation failed (the reference throws Error) */
  P0_EHIP = 2,     /* the HIP runtime reported an error */
  P0_ENODEV = 3,   /* no context (p0_open not called) or no gfx950 device */
  P0_ENOMEM = 4    /* device allocation failed */
};

/* ---- enums mirroring the reference's string options ------------------------------------------------------------ */
enum { P0_ENC_Q4G32A_T64 = 1, P0_ENC_Q8G64S_T64 = 2, P0_ENC_F16 = 3 };             /* a.w.enc */
enum { P0_PRO_RAW = 0, P0_PRO_RMS = 1, P0_PRO_SUM = 2, P0_PRO_PLEG = 3 };           /* gemv / gemvM a.pro */
enum { P0_EPI_STORE = 0, P0_EPI_GEGLU = 1, P0_EPI_SOFTCAP = 2 };                    /* gemv / gemvM a.epi */
enum { P0_XMODE_F16 = 0, P0_XMODE_LNMOD = 1, P0_XMODE_RMS = 2, P0_XMODE_BF16 = 3 }; /* gemm a.x.mode */
enum { P0_GEPI_F16 = 0, P0_GEPI_F32 = 1, P0_GEPI_RESADD = 2, P0_GEPI_SWIGLU = 3, P0_GEPI_BIAS = 4,
       P0_GEPI_HEADS = 5 };                                                         /* gemm a.epi */
enum { P0_ROPE_INTER = 0, P0_ROPE_HALF = 1 };                                       /* gemm a.heads.ropeMode */
enum { P0_ACT_SILU = 0, P0_ACT_GELU = 1 };                                          /* gemm a.act (swiglu) */

/* ---- device / buffers ------------------------------------------------------------------------------------------ */
const char* p0_last_error(void);
int p0_version(void);                          /* library ABI version (P0_ABI_VERSION) */
#define P0_ABI_VERSION 2

typedef struct {
  char name[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int device;
  int cu_count;
  int xcd_count;          /* 8 on MI355X (derived: cu_count / 32) */
  int64_t hbm_bytes;
  int64_t lds_bytes_per_cu;
  int clock_khz;
  int64_t workspace_bytes;
} p0_device_info_t;

int p0_open(int device);                       /* selects the device, checks gfx950, creates the stream + workspace */
int p0_close(void);
int p0_device_info(p0_device_info_t* out);
int p0_set_stream(void* stream);               /* hipStream_t as void*; NULL = the library's own stream */
void* p0_get_stream(void);

int p0_buffer(size_t bytes, void** out);       /* device allocation, size rounded up to 16 B (Gpu.buffer) */
int p0_free(void* buf);
int p0_upload(void* dst, size_t dst_off, const void* src, size_t bytes);   /* host -> device, ordered on the stream */
int p0_read(void* host_dst, const void* src, size_t src_off, size_t bytes); /* device -> host; waits for the stream */
int p0_fill(void* dst, size_t dst_off, uint32_t value, size_t words);       /* 32-bit pattern fill (NaN-fill checks) */
int p0_done(void);                             /* wait for every op enqueued on the stream */
/* device-to-device copy, ordered on the stream (runner.copy, engine/core/gpu.js:237-242): offsets and size multiples
 * of 4 (copyBufferToBuffer's rule); overlapping ranges are rejected */
int p0_copy(const void* src, size_t src_off, void* dst, size_t dst_off, size_t bytes);

/* Event timing on the current stream (for benchmarks): p0_timer_start records a start event, p0_timer_stop records a
 * stop event, waits for it and returns the elapsed milliseconds. */
int p0_timer_start(void);
int p0_timer_stop(float* ms);

/* ---- recorded op sequences: the decode-step recorder (engine/llm/drunner.js:1-8, 83-101 DecodeRunner) ------------ */
/* Between p0_record_begin and p0_record_end the ops called on this thread are recorded (HIP stream capture of the
 * current stream) instead of run; p0_replay enqueues the whole recorded sequence with one launch. The library's ops
 * clear nothing with memset and leave their split-K counters at zero, so a recording replays any number of times.
 * Buffers: the caller's buffers must outlive the recording. The library memory its kernels read (the GEMM's activation
 * staging workspace, the op table and state of a chain run inside it) is held by the recording: a later growth of the
 * workspace or a p0_chain_free leaves it in place until p0_record_free. A GEMM call that needs a larger staging
 * workspace than the current one is refused while recording (run it once before, or use p0_q4_gemm_noalloc).
 * p0_record_info gives the number of launches a replay makes (the DecodeRunner's dispatch count). */
int p0_record_begin(void);
int p0_record_end(void** rec_out);
int p0_replay(void* rec);
int p0_record_info(void* rec, int32_t* launches);
int p0_record_free(void* rec);

/* ---- q4g32a.t64 GEMV: y = x W^T for ONE row (engine/llm/lops.js:108-141) ---------------------------------------- */
/* Buffers are base pointers; offsets use the reference's units (w_off bytes, the rest in floats). */
typedef struct {
  const void* w;       /* a.w.buf */
  int64_t w_off;       /* a.w.off, bytes (multiple of 4; 16 on this build's fast path) */
  int32_t w_enc;       /* a.w.enc */
  int64_t w_rows;      /* a.w.rows */
  int64_t w_cols;      /* a.w.cols: groups per weight row = w_cols / 32 */
  const float* x;      /* a.x.buf */
  int64_t x_rowB;      /* a.x.rowB (floats) */
  int64_t N, K;        /* a.N (output rows; for geglu the gate rows), a.K */
  int64_t kPer;        /* a.kPer (0 = none) */
  int32_t pro, epi;    /* a.pro, a.epi */
  float* y;            /* a.y.buf */
  int64_t ldy;         /* a.ldy (0 = N) */
  const float* stat;   /* a.stat.buf (rms) */
  int64_t stat_off;    /* a.stat.off (floats) */
  const float* norm;   /* a.norm.buf (rms) */
  int64_t norm_off;    /* a.norm.off (floats) */
  int64_t src_n;       /* a.src.n (sum / pleg: number of producer partials) */
  int64_t src_ld;      /* a.src.ld (floats between partials) */
  const float* ev;     /* a.ev.buf (pleg) */
  int64_t ev_off;      /* a.ev.off (floats) */
  float* mx;           /* a.mx.buf (softcap: [N/64][2] max, bitcast index) */
  float cap;           /* a.cap (0 = 30) */
} p0_gemv_args_t;
int p0_q4_gemv(const p0_gemv_args_t* a, int32_t* nsplit_out);

/* ---- q4g32a.t64 GEMV-M: y[m] = x[m] W^T for M rows, weights read once (engine/llm/lops_spec.js:159-191) ---------- */
typedef struct {
  const void* w; int64_t w_off; int32_t w_enc; int64_t w_rows, w_cols;
  const float* x;      /* a.x.buf */
  int64_t x_ldx;       /* a.x.ldx (0 = K) */
  int64_t x_rowB;      /* a.x.rowB */
  int64_t M, N, K, kPer;
  int32_t pro, epi;    /* raw | rms | pleg ; store | geglu | softcap */
  float* y;
  int64_t y_ldy;       /* a.y.ldy (0 = M * ldm): floats between splits */
  int64_t y_ldm;       /* a.y.ldm (0 = N): floats between rows */
  const float* stat; int64_t stat_off, stat_ld;   /* rms: rstd of row m at stat[stat_off + m * stat_ld] (ld 0 = 2) */
  const float* norm; int64_t norm_off;
  int64_t src_n, src_ld;                          /* pleg partials (src_n 0 = 1) */
  const float* ev; int64_t ev_off, ev_ld;         /* pleg: ev row m at ev_off + m * ev_ld */
  float* mx;                                      /* softcap: [M][N/64][2] */
  float cap;
} p0_gemvm_args_t;
int p0_q4_gemvM(const p0_gemvm_args_t* a, int32_t* nsplit_out);

/* ---- q4g32a.t64 dequant-GEMM on MFMA: Y[m,n] = sum_k X'[m,k] * fl16(deq(W[n,k])) (engine/ops/gemm.js:255-322) --- */
typedef struct {
  const void* w; int64_t w_off; int32_t w_enc; int64_t w_rows, w_cols;
  const void* x;       /* a.x.buf */
  int64_t x_off;       /* a.x.off (bytes) */
  int64_t x_ld;        /* a.x.ld (elements; 0 = K) */
  int64_t x_k0;        /* a.x.k0 */
  int32_t x_mode;      /* a.x.mode: f16 | lnmod | rms (| bf16: this build's bf16 activations, converted to fp16) */
  int64_t M, N, K;
  int64_t wr0, wr1, wk0;   /* first weight row, swiglu 'up' first row, first weight k column */
  int32_t epi;
  void* y; int64_t y_off /* bytes */, y_ld /* elements, 0 = N */, y_n0;
  const float* ev; int64_t ev_off;            /* resadd gate / bias vector (floats) */
  const float* stats; int64_t stats_off;      /* lnmod / rms: (mean, rstd) pairs per row, off in rows */
  const float* pv; int64_t pv_off, pv_stride; /* lnmod: scale at pv_off, shift at pv_off + pv_stride (u32 wrap); rms: weight */
  const float* bv; int64_t bv_off, bv_up;     /* bias vector (resadd / swiglu: gate at bv_off, up at bv_off + bv_up) */
  int32_t act;         /* swiglu activation */
  int32_t store;       /* resadd: 1 = Y = gate * (acc + bias) instead of += */
  int32_t res;         /* bias: 1 = add the previous Y in place */
  /* heads (engine/ops/gemm.js:212-250, a.heads): every 128 output columns are one head; head h is a query head for
   * h < hq, a key head for h < hq + hkv, else a value head. Query and key heads are RMS-normalised over their 128 values
   * (eps), times the norm weights (ev[ev_off + c] for queries, ev[ev_off + 128 + c] for keys), then rotated by the
   * RoPE table rope[row][64][cos, sin] (row = heads_row_off + m): heads_rope P0_ROPE_INTER pairs columns (2p, 2p + 1)
   * with entry p, P0_ROPE_HALF pairs (d, d + 64) with entry d. Every head is written as fp16, head-major:
   * Y[((h * heads_ltot) + heads_row_off + m) * 128 + c] from byte y_off (y_ld and y_n0 are not used). */
  int64_t heads_ltot, heads_row_off;
  int32_t heads_hq, heads_hkv;
  float heads_eps;     /* 0 = 1e-6 */
  int32_t heads_rope;
  const float* rope;   /* the RoPE table (a.heads.rope.buf) */
} p0_gemm_args_t;
int p0_q4_gemm(const p0_gemm_args_t* a, double* flops_out);
/* p0_q4_gemm without any allocation. No counterpart in the reference: this is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same kernels and
 * results as p0_q4_gemm; the activation staging that bf16 / lnmod / rms / unaligned fp16 activations need goes to a
 * static device scratch of 32 MiB (M * K * 2 bytes at most, else P0_EINVAL), allocated with the library's code on each
 * GPU and held until the process ends. Every call on one GPU shares that scratch: calls that may overlap on one GPU
 * (two streams, two threads) race and must be ordered by the caller. Nothing in it needs to start at zero (each call
 * writes all it reads). */
int p0_q4_gemm_noalloc(const p0_gemm_args_t* a, double* flops_out);

/* ---- bit-exact dequant of whole q4g32a.t64 weights --------------------------------------------------------------- */
/* out32 (may be NULL): fl32(q * scale + min), row-major [N][K]; out16 (may be NULL): fl16 of that, the GEMM tile value. */
int p0_q4_dequant(const void* w, int64_t w_off, int64_t N, int64_t K, float* out32, uint16_t* out16);

/* ---- tuning knobs (the analogue of the reference's per-device kernel picks, engine/llm/lopsx.js:317-321) ---------- */
/* knob 0: waves a GEMV call aims for before it splits K (default 2048);
 * knob 1: output tiles from which a GEMV wave streams two tiles (default 1024);
 * knob 2: fewest q4 groups a wave streams when K is split (default 2);
 * knob 3: most waves sharing one tile slot's K range inside a workgroup (default 16, at most 16; 8 when M > 2);
 * knob 4: fewest x rows M from which a gemvM call outside a chain runs on the matrix cores (default 2, i.e. every
 *         M > 1; 17: never, the fp32 VALU kernel).
 * knob 5: K-slices per split of a q8g64s.t64 gemv (M = 1, splits of 1024-3072 k) across workgroups (default 0: planned,
 *         up to ~192 workgroups with at least 8 groups of 64 k a slice; a negative value restores the plan).
 * value <= 0 only queries (knob 5: value < 0 restores its plan). Returns the previous value, or -1 for an unknown
 * knob. */
int p0_gemv_tune(int knob, int value);

/* ---- GEMV chains: a decode step's GEMVs in ONE persistent launch (engine/llm/drunner.js:1-8, 83-101) ------------- */
/* Between p0_chain_begin and p0_chain_end, p0_q4_gemv / p0_q4_gemvM calls are validated and planned as usual but
 * appended to the chain instead of launched (all GEMV ops of a chain have the same M); p0_copy, p0_argmax /
 * p0_argmaxM, p0_rowstats and p0_normadd calls join the chain too (their results equal the standalone ops' bit for
 * bit), so a whole decode token, its argmax and result copy included, is one launch. Every other op (the GEMM, the
 * dequant, uploads) is refused while a chain is being built. p0_chain_run enqueues the whole chain as one kernel: the
 * pipelined kernel for M <= 5, the wide pipelined kernel for 6 - 16 rows (q4g32a.t64 ops with raw or rms prologues;
 * otherwise, where the rows use disjoint memory, i.e. no row of a buffer that one row group writes is touched by
 * another, one pipelined kernel per group of at most 5 rows, launched back to back): op i starts its arithmetic once
 * op i - 1 has written all of its outputs (so op i may read anything earlier ops wrote), and each workgroup streams op
 * i's first weights while it waits. Chains holding copy / argmax / rowstats / normadd or q8g64s.t64 ops run only on the
 * pipelined kernels (p0_chain_end refuses them otherwise). Buffers are bound at p0_chain_end; a chain runs any
 * number of times, also inside p0_record_begin / p0_record_end. Every wait is bounded: a wait that gives up (which
 * needs another kernel holding the GPU's CUs meanwhile) marks the chain, and p0_chain_status (which waits for the
 * stream) returns 1 once in *timed_out and resets the chain and the split-K counters; the results of that run are
 * invalid, and runs of the chain started before that call do nothing. Runs of one chain, or of chains sharing the
 * context's workspace, must not overlap (one stream). */
typedef struct {
  int32_t n_ops, m, workgroups, waves_per_workgroup;
  int64_t lds_bytes;
  int32_t mailboxes;   /* ops that take their input from the previous op's mailbox (p0_chain_tune knob 7) */
  int32_t staged;      /* M > 1: ops that take their x' staged by the previous op (p0_chain_tune knob 10) */
  int32_t passes;      /* launches per run: 1, or, for 6-16 rows as row-group passes, one per row group */
} p0_chain_info_t;
int p0_chain_begin(void);
int p0_chain_end(void** chain_out);
int p0_chain_run(void* chain);
int p0_chain_status(void* chain, int32_t* timed_out);
int p0_chain_info(void* chain, p0_chain_info_t* out);
int p0_chain_free(void* chain);
/* knob 0: waves per chain workgroup for M = 1 (8 or 16, default 16); knob 1: largest wave share in q4 groups before a
 * chain op splits K across workgroups (default 16); knob 2: polls before a chain wait gives up (default 2^22); knob 3:
 * 1 = every wait of later runs gives up at once (for tests of the timed-out path), 0 = normal; knob 4: 1 = staged ops
 * (each workgroup copies its share of an op's weights into LDS before it waits for the previous op; the default: M = 1
 * chains run on the pipelined kernel, whose loader waves stream every op's weights into an LDS ring ops ahead of the
 * arithmetic; other chains stage the ops whose share fits), 0 = every op streams its weights after the wait; knob 5:
 * loader waves of the pipelined kernel that stream (1..4, default 2); knob 6: LDS slots each loader keeps in flight in
 * M = 1 chains (1 or 2, default 2); knob 7: 1 = mailbox hand-offs in pipelined chains (the default: an op whose only
 * input is the previous op's output polls that output, tagged with the run, instead of the previous op's completion
 * flags), 0 = every op waits for the flags; knob 8: 1 = gemvM chains of M <= 5 rows also run on the pipelined kernel,
 * and chains of 6-16 rows as pipelined passes over row groups where their rows are independent (the default), 0 = on
 * the general chain kernel; knob 9: the fewest x rows for which a pipelined chain does its slot arithmetic on the
 * matrix cores (default 3: M = 2 runs faster on the fp32 VALU; 6 = never); knob 10: 1 = in pipelined M > 1 chains on
 * the matrix cores an op that reads one split of the previous op's output takes its x' as that op staged it (the
 * default), 0 = every op stages its own x' after its wait; knob 11: LDS slots each loader keeps in flight in chains of
 * M = 2-5 rows (1 or 2, default 1); knob 12: 1 = chains of 6-16 rows on the wide pipelined kernel, one pass (the
 * default), 0 = as row-group passes; knob 13: LDS slots each loader keeps in flight in the wide kernel (1 or 2, default
 * 2); knob 14: 1 = in the wide kernel a compute wave whose x' exceeded the producer's 2^8 fp16 staging in one op loads
 * the fp32 x' at once in the next (the default; the results are the same bit for bit), 0 = it tries the staging
 * first. Knobs 0-1 and 4-14 apply to chains begun afterwards, 2-3 to runs. value < 0 only queries (knobs 0-2 also ignore
 * 0); returns the previous value. */
int p0_chain_tune(int knob, int value);

/* ---- the GEMV's producer and consumers: row statistics, split-K sum + residual RMS, argmax over tile maxima ------- */
/* rowstats (engine/ops/misc.js:13-40): for each row r < rows of X (floats x[r * x_ld + x_c0 + c], c < cols, from byte
 * offset x_off), st[(st_off + r) * 2] = mean (0 for mode 1, rms) and st[(st_off + r) * 2 + 1] = 1 / sqrt(var + eps),
 * var = mean of (x - mean)^2. x_ld 0 = cols. The sums follow the reference's order: 256 strided partial sums, then a
 * halving tree. */
typedef struct {
  const void* x; int64_t x_off;   /* bytes */
  int64_t x_ld, x_c0;             /* floats */
  int64_t rows, cols;
  int32_t mode;                   /* 0 = LayerNorm (mean and variance), 1 = RMSNorm */
  float eps;
  float* st; int64_t st_off;      /* in rows: pairs (mean, rstd) */
} p0_rowstats_args_t;
int p0_rowstats(const p0_rowstats_args_t* a);

/* normadd (engine/llm/lops.js:143-178): for each row m < M of D floats, t = sum over the t_n split partials
 * t[j * t_ld + m D + i] (in j order); mode 0: x = (x + t / rms(t) * w[w_off + i]) * scale, rms(t) =
 * sqrt(mean(t^2) + eps); mode 1: x = t; then st[st_off + m] = 1 / sqrt(mean(x^2) + eps). The reference's defaults:
 * t_n 0 = 1, t_ld 0 = D M, M 0 = 1, eps 0 = 1e-6 (the caller passes scale; the reference's own default is 1). */
typedef struct {
  const float* t; int64_t t_n, t_ld;
  const float* w; int64_t w_off;  /* mode 0 only */
  float* x;                       /* [M][D], read and written */
  float* st; int64_t st_off;
  int64_t D, M;
  float eps, scale;
  int32_t mode;
} p0_normadd_args_t;
int p0_normadd(const p0_normadd_args_t* a);

/* argmax (engine/llm/lops.js:416-436): over the n pairs mx[2 i] = max, mx[2 i + 1] = bitcast(u32 index) that a
 * softcap GEMV writes per 64-row tile, out[0] = the index of the largest value (ties: the lowest index), out[1] = the
 * bits of that value; n = 0 leaves (0xFFFFFFFF, bits of -3.4e38). argmaxM (engine/llm/lops_spec.js:327-348): the same
 * for each of M rows of n pairs, out[2 m], out[2 m + 1]. out is device memory. */
int p0_argmax(const float* mx, int64_t n, uint32_t* out);
int p0_argmaxM(const float* mx, int64_t n, int64_t M, uint32_t* out);

/* ---- the pack reader's I/O (engine/core/store.js:221-244) ---------------------------------------------------------- */
/* bytes [offset, offset + bytes) of the file at path -> device memory dst + dst_off, streamed in 16 MB chunks through
 * two pinned host buffers (file reads overlap the host-to-device copies on the library's stream); returns when the
 * copies are done. The pack manifest (shards, tensors, encodings) is read by the host (p0pc0rn_amd/js/core/store.mjs). */
int p0_upload_file(const char* path, int64_t offset, int64_t bytes, void* dst, int64_t dst_off);

/* ---- synthetic weights on the device (the reference's GPU filler, engine/tune/autotune.js:73-87) ----------------- */
/* Symmetric BASELINE records: codes uniform in [0,16) (= q + 8 for q uniform in [-8, 8)), scale = fl16(|N(0, sigma)|),
 * min = -8 * scale; counter-based hash of (seed, index), so any sub-range is reproducible. */
int p0_fill_q4_sym(void* w, int64_t w_off, int64_t N, int64_t K, uint32_t seed, float sigma);
/* fp16 N(0,1)-shaped activations (hash-based Box-Muller), fp32 or fp16 output */
int p0_fill_randn(void* dst, int64_t off_bytes, int64_t n, uint32_t seed, float sigma, int32_t as_f16);
/* The dense fp16 matrix-core rate the chip sustains (no counterpart in the reference: a measurement probe for
 * bench.py, which reports it beside the spec-sheet peak). Enqueues one workgroup of 8 waves per CU, each wave running
 * `iters` rounds of 4 independent v_mfma_f32_32x32x16_f16 chains with no memory traffic; `sink` (one float per CU)
 * is written only on a value the sums never take. *flops_out = the flops enqueued; time it with p0_timer_*. */
int p0_probe_mfma(int64_t iters, float* sink, double* flops_out);
/* The HBM read rate the chip sustains (no counterpart in the reference: a measurement probe for bench.py, which reports
 * it beside the spec-sheet peak). Enqueues one pass of 16-byte loads over `bytes` (a positive multiple of 16) at `buf`,
 * 2048 workgroups of 256 threads in a grid-stride loop; `sink` (one word) is written only on a fold value the data
 * does not give. Time it with p0_timer_*. */
int p0_probe_read(const void* buf, int64_t bytes, uint32_t* sink);

#ifdef __cplusplus
}
#endif
#endif /* P0PC0RN_H */
