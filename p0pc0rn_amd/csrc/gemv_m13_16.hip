// gemv_m13_16.hip - instantiates the GEMV and chain kernels for M = 13 .. 16 (one of four units compiled in
// parallel; the kernels themselves are in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace p0 {
template gemv_kernel_t pick_m<13>(int);
template chain_kernel_t pick_chain_m<13>(int);
template gemv_kernel_t pick_m<14>(int);
template chain_kernel_t pick_chain_m<14>(int);
template gemv_kernel_t pick_m<15>(int);
template chain_kernel_t pick_chain_m<15>(int);
template gemv_kernel_t pick_m<16>(int);
template chain_kernel_t pick_chain_m<16>(int);
}  // namespace p0
