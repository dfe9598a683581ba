// Measurement aids of bench.py's floor workload (libmarlin_probe.so; not part of the
// GEMM library and with no counterpart in the reference).
//
//   marlin_probe_read   streams a byte range from device memory with 16-byte loads:
//                       the time one launch needs to move a decode call's weight
//                       bytes, at the rate the memory system gives a plain read.
//   marlin_probe_empty  an empty kernel on a given grid: the launch and dispatch cost
//                       of a call on that grid.
//   marlin_probe_mfma_32x32x16
//                       one v_mfma_f32_32x32x16_f16 whose operands and result are
//                       placed by the lane layout the dense large-M kernel assumes,
//                       so that a test can compare it with the plain product.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/marlin_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every thread reads 16-byte pieces i, i + stride, ... (consecutive threads read
// consecutive pieces), eight loads in flight per iteration, and XORs them.  The
// result is stored only when it equals a value that random data practically never
// gives, so the loads cannot be dropped and nearly nothing is written.
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                         uint32_t* __restrict__ sink) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 7 * stride < n16; i += 8 * stride) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < 8; u++) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9E3779B9u) sink[0] = x;
}

__global__ void probe_empty_kernel() {}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// One wave.  Lane l = 32 hk + i: A operand = row i, k 8 hk .. 8 hk + 7 of A (32 x 16,
// row-major); B operand = column i, the same k of B (16 x 32, row-major); result
// register r = D[8 (r / 4) + 4 hk + r % 4][i] of D (32 x 32, row-major).
__global__ __launch_bounds__(64) void probe_mfma_32x32x16_kernel(const _Float16* __restrict__ A,
                                                                 const _Float16* __restrict__ B,
                                                                 float* __restrict__ D) {
  const int l = threadIdx.x, i = l & 31, hk = l >> 5;
  half8_t a, b;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    a[e] = A[i * 16 + 8 * hk + e];
    b[e] = B[(8 * hk + e) * 32 + i];
  }
  f32x16 c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; r++) D[(8 * (r >> 2) + 4 * hk + (r & 3)) * 32 + i] = c[r];
}

}  // namespace

extern "C" {

int marlin_probe_read(const void* p, long long bytes, void* sink, int blocks, int dev, hipStream_t stream) {
  if (bytes < 0 || bytes % 16 != 0 || blocks <= 0) return 1;
  if (bytes == 0) return 0;
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_read_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const u32x4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int marlin_probe_empty(int blocks, int threads, int dev, hipStream_t stream) {
  if (blocks <= 0 || threads <= 0 || threads > 1024) return 1;
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_empty_kernel, dim3((unsigned)blocks), dim3((unsigned)threads), 0, stream);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int marlin_probe_mfma_32x32x16(const void* A, const void* B, void* D, int dev, hipStream_t stream) {
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_mfma_32x32x16_kernel, dim3(1), dim3(64), 0, stream, static_cast<const _Float16*>(A),
                     static_cast<const _Float16*>(B), static_cast<float*>(D));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"
