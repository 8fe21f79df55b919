// index.mjs - the Node host's public surface: the device object and the three q4 ops, as the reference names them.
export { createGpu, Gpu, GpuError, view, f2h, h2f, toF16, fromF16, MB } from './core/gpu.mjs';
export { gemv, KCH } from './llm/lops.mjs';
export { gemvM } from './llm/lops_spec.mjs';
export { gemm, DEFAULT_TILE } from './ops/gemm.mjs';
export { DecodeRunner } from './llm/drunner.mjs';
