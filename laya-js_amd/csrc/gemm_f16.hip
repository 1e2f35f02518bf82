// 16-bit weights: the MFMA GEMM kernels instantiated for these weight formats
// (the templates live in gemm_kernels.h).
#include "gemm_kernels.h"

namespace hb {

template void mfma_dtype<0, false, false>(int, bool, hipStream_t, int, unsigned, const uint16_t*, int64_t,
                                          const uint16_t*, QW, const uint16_t*, const uint16_t*, int64_t,
                                          uint16_t*, int64_t, int, int, int);

template void launch_qkv<false>(hipStream_t, int, unsigned, const uint16_t*, int64_t, const uint16_t*, uint16_t*, int,
                                int, int, QK);
template void launch_qkv<true>(hipStream_t, int, unsigned, const uint16_t*, int64_t, const uint16_t*, uint16_t*, int,
                               int, int, QK);

}  // namespace hb
