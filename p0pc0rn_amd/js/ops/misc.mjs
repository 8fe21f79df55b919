// misc.mjs - rowstats(gpu, a): per-row (mean, rstd) of LayerNorm / RMSNorm (engine/ops/misc.js:13-40), the stats slot
// the GEMV's rms prologue and the GEMM's lnmod / rms prologues read, on the MI355X library.
'use strict';
import { native } from '../native.mjs';
import { addr } from '../llm/lops.mjs';

/** x: {buf, off (bytes), ld (floats), c0}, rows, cols, mode 'ln'|'rms', eps, st: {buf, off (rows)}:
 *  ST[(off + r) * 2] = mean (0 for rms), ST[(off + r) * 2 + 1] = 1 / sqrt(var + eps) */
export function rowstats(gpu, a) {
  native().rowstats({
    x: addr(a.x.buf), x_off: a.x.off || 0, x_ld: a.x.ld || a.cols, x_c0: a.x.c0 || 0,
    rows: a.rows, cols: a.cols, mode: a.mode === 'rms' ? 1 : 0, eps: a.eps,
    st: addr(a.st.buf), st_off: a.st.off || 0,
  });
}
