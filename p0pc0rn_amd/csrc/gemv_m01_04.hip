// gemv_m01_04.hip - instantiates the GEMV and chain kernels for M = 1 .. 4 (one of four units compiled in
// parallel; the kernels themselves are in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace p0 {
template gemv_kernel_t pick_m<1>(int);
template chain_kernel_t pick_chain_m<1>(int);
template gemv_kernel_t pick_m<2>(int);
template chain_kernel_t pick_chain_m<2>(int);
template gemv_kernel_t pick_m<3>(int);
template chain_kernel_t pick_chain_m<3>(int);
template gemv_kernel_t pick_m<4>(int);
template chain_kernel_t pick_chain_m<4>(int);
}  // namespace p0
