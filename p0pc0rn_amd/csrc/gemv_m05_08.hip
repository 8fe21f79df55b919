// gemv_m05_08.hip - instantiates the GEMV and chain kernels for M = 5 .. 8 (one of four units compiled in
// parallel; the kernels themselves are in gemv_kernels.hpp).
#include "gemv_kernels.hpp"

namespace p0 {
template gemv_kernel_t pick_m<5>(int);
template chain_kernel_t pick_chain_m<5>(int);
template gemv_kernel_t pick_m<6>(int);
template chain_kernel_t pick_chain_m<6>(int);
template gemv_kernel_t pick_m<7>(int);
template chain_kernel_t pick_chain_m<7>(int);
template gemv_kernel_t pick_m<8>(int);
template chain_kernel_t pick_chain_m<8>(int);
}  // namespace p0
