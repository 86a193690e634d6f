// The 64-bit-records forms (BIG = true) of the 256 x 256 DotGeneral cores, for
// operand slices of 2 GiB or more: their tiles' buffer descriptors take the bytes
// left in a slice of any size (gemm_bf16_dev.h, Ext64).  Kept out of k_gemm.hip
// so the two compile in parallel.
#include "gemm_kernels.h"

namespace ghip {

template hipError_t launch_bf16_4w<true, bf16_t, bf16_t>(GemmParams, bool, bool, hipStream_t);
template hipError_t launch_bf16_4w<true, bf16_t, float>(GemmParams, bool, bool, hipStream_t);
template hipError_t launch_bf16_4w<true, f16_t, f16_t>(GemmParams, bool, bool, hipStream_t);
template hipError_t launch_bf16_4w<true, f16_t, float>(GemmParams, bool, bool, hipStream_t);
template hipError_t launch_f32<256, 256, 2, 4, float, true>(GemmParams, bool, bool, hipStream_t);
template hipError_t launch_f32<256, 256, 2, 4, bf16_t, true>(GemmParams, bool, bool, hipStream_t);

}  // namespace ghip
