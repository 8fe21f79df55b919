// index.mjs - the Node host's public surface: the device object, the three q4 ops and the GEMV's producer and
// consumers (rowstats, normadd, argmax, argmaxM), the tuned-GEMV pick surface (lopsx), and the pack reader (WeightStore),
// as the reference names them.
export { createGpu, Gpu, GpuError, view, f2h, h2f, toF16, fromF16, MB } from './core/gpu.mjs';
export { gemv, normadd, argmax, KCH } from './llm/lops.mjs';
export { gemvM, argmaxM } from './llm/lops_spec.mjs';
export { PICK, KX, setKX, KERNEL_VERSION, setPicks, picksNow, kxPick, okV5, directOkV5, u8ok, DIRECT_NEEDS, gemvV5, gemvMV5,
         v5code } from './llm/lopsx.mjs';
export { rowstats } from './ops/misc.mjs';
export { gemm, DEFAULT_TILE } from './ops/gemm.mjs';
export { DecodeRunner } from './llm/drunner.mjs';
export { WeightStore, PackStore } from './core/store.mjs';
