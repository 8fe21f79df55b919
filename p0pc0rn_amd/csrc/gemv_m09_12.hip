// gemv_m09_12.hip - instantiates the GEMV and chain kernels for M = 9 .. 12 (one of four units compiled in
// parallel; the kernels themselves are in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace p0 {
template gemv_kernel_t pick_m<9>(int);
template chain_kernel_t pick_chain_m<9>(int);
template gemv_kernel_t pick_m<10>(int);
template chain_kernel_t pick_chain_m<10>(int);
template gemv_kernel_t pick_m<11>(int);
template chain_kernel_t pick_chain_m<11>(int);
template gemv_kernel_t pick_m<12>(int);
template chain_kernel_t pick_chain_m<12>(int);
}  // namespace p0
