// Large-M 2:4 INT4 x FP16 GEMM: instantiation and launch of sm24_prefill_kernel.
#include "sm24_prefill.h"

namespace sm24 {

hipError_t launch_prefill(const GemmArgs& a, int rows, int chunks, bool grouped, hipStream_t stream) {
  const dim3 grid((a.N / (64 * chunks)) * ((a.M + rows - 1) / rows) * a.splits);
  constexpr int W = kPreChunks, NW = kPreNarrowChunks;
  if (chunks == NW) {  // 128-row tiles of 256 columns, 4 waves
    if (grouped) hipLaunchKernelGGL((sm24_prefill_kernel<true, 4, NW>), grid, dim3(64 * NW), 0, stream, a);
    else hipLaunchKernelGGL((sm24_prefill_kernel<false, 4, NW>), grid, dim3(64 * NW), 0, stream, a);
  } else if (rows == 64) {
    if (grouped) hipLaunchKernelGGL((sm24_prefill_kernel<true, 2, W>), grid, dim3(64 * W), 0, stream, a);
    else hipLaunchKernelGGL((sm24_prefill_kernel<false, 2, W>), grid, dim3(64 * W), 0, stream, a);
  } else {
    if (grouped) hipLaunchKernelGGL((sm24_prefill_kernel<true, 4, W>), grid, dim3(64 * W), 0, stream, a);
    else hipLaunchKernelGGL((sm24_prefill_kernel<false, 4, W>), grid, dim3(64 * W), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace sm24
