// Large-M 2:4 INT4 x FP16 GEMM: instantiation and launch of sm24_prefill_kernel.
#include "sm24_prefill.h"

namespace sm24 {

hipError_t launch_prefill(const GemmArgs& a, int rows, bool grouped, hipStream_t stream) {
  const dim3 grid((a.N / (64 * kPreChunks)) * ((a.M + rows - 1) / rows) * a.splits);
  if (rows == 64) {
    if (grouped) hipLaunchKernelGGL((sm24_prefill_kernel<true, 2>), grid, dim3(kPreThreads), 0, stream, a);
    else hipLaunchKernelGGL((sm24_prefill_kernel<false, 2>), grid, dim3(kPreThreads), 0, stream, a);
  } else {
    if (grouped) hipLaunchKernelGGL((sm24_prefill_kernel<true, 4>), grid, dim3(kPreThreads), 0, stream, a);
    else hipLaunchKernelGGL((sm24_prefill_kernel<false, 4>), grid, dim3(kPreThreads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace sm24
