// Instantiations and launcher of the dense large-M kernel (marlin_dense_prefill.h).
#include "marlin_dense_prefill.h"

namespace sm24 {

hipError_t launch_dense_prefill(const DensePreArgs& a, bool grouped, hipStream_t stream) {
  const int tiles = (a.N / kDpTileCols) * ((a.M + kDpRows - 1) / kDpRows) * a.splits;
  if (grouped) hipLaunchKernelGGL(marlin_dense_prefill_kernel<true>, dim3(tiles), dim3(kDpThreads), 0, stream, a);
  else hipLaunchKernelGGL(marlin_dense_prefill_kernel<false>, dim3(tiles), dim3(kDpThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sm24
