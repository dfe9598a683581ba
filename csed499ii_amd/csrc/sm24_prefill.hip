// Large-M 2:4 INT4 x FP16 GEMM: instantiation and launch of sm24_prefill_kernel.
#include "sm24_prefill.h"

namespace sm24 {

hipError_t launch_prefill(const GemmArgs& a, bool grouped, hipStream_t stream) {
  const int tiles = (a.N / (64 * kPreChunks)) * ((a.M + kPreRows - 1) / kPreRows) * a.splits;
  if (grouped) hipLaunchKernelGGL(sm24_prefill_kernel<true>, dim3(tiles), dim3(kPreThreads), 0, stream, a);
  else hipLaunchKernelGGL(sm24_prefill_kernel<false>, dim3(tiles), dim3(kPreThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sm24
