// Measurement aids of bench.py's floor workload (libmarlin_probe.so; not part of the
// GEMM library and with no counterpart in the reference).
//
//   marlin_probe_read   streams a byte range from device memory with 16-byte loads,
//                       in grid-stride order or a contiguous range per wave: the
//                       time one launch needs to move a decode call's weight bytes,
//                       at the rate the memory system gives a plain read.
//   marlin_probe_empty  an empty kernel on a given grid: the launch and dispatch cost
//                       of a call on that grid.
//   marlin_probe_mfma_32x32x16
//                       one v_mfma_f32_32x32x16_f16 whose operands and result are
//                       placed by the lane layout the dense large-M kernel assumes,
//                       so that a test can compare it with the plain product.
//   marlin_probe_smfmac_stream
//                       the MFMA-only ceiling of the large-M 2:4 kernel: on its grid
//                       and workgroup shape (8 waves, two per SIMD, 128 accumulator
//                       AGPRs per wave), every wave issues the 16
//                       v_smfmac_f32_32x32x32_f16 of a k-step per iteration from
//                       random fp16 operands held in registers, nothing else; wave 0
//                       of workgroup 0 also records the shader clock against the
//                       100 MHz real-time counter.
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

// Every wave reads its own contiguous range of the byte range (1 KiB per load
// instruction, 8 loads in flight), XORs it and stores as probe_read_kernel does.
__global__ __launch_bounds__(256) void probe_read_chunk_kernel(const u32x4* __restrict__ p, long long n16,
                                                               uint32_t* __restrict__ sink) {
  const long long waves = (long long)gridDim.x * 4;
  const long long wave = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const long long per = (n16 + waves - 1) / waves;  // pieces of one wave
  const long long b = wave * per, e = b + per < n16 ? b + per : n16;
  u32x4 acc = {0u, 0u, 0u, 0u};
  long long i = b + lane;
  for (; i + 7 * 64 < e; i += 8 * 64) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = p[i + u * 64];
#pragma unroll
    for (int u = 0; u < 8; u++) acc ^= v[u];
  }
  for (; i < e; i += 64) acc ^= p[i];
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

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half16_t __attribute__((ext_vector_type(16)));

// Random fp16 in [-1, 1) from a 32-bit hash (no NaN, infinity or subnormal).
__device__ inline _Float16 rnd_half(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return (_Float16)((float)(x >> 8) * (1.0f / 8388608.0f) - 1.0f);
}

template <int ABID>
__device__ __forceinline__ void stream_smfmac(f32x16& c, half8_t a, half16_t b, uint32_t idx) {
  if constexpr (ABID == 0)
    asm volatile("v_smfmac_f32_32x32x32_f16 %0, %1, %2, %3" : "+a"(c) : "v"(a), "v"(b), "v"(idx));
  else
    asm volatile("v_smfmac_f32_32x32x32_f16 %0, %1, %2, %3 abid:1" : "+a"(c) : "v"(a), "v"(b), "v"(idx));
}

// 8 waves; each keeps 8 accumulators of 16 AGPRs (as the 128-row tile: 4 row blocks x
// 2 column halves) and, per iteration, issues 16 smfmacs over them, rotating through
// 4 A operands, 4 B operands and both index halfwords (operands change from MFMA to
// MFMA, as in the GEMM).  Valid 2:4 indices (0 | 1 << 2 and 2 | 3 << 2 patterns).
// out[block * 8 + wave] receives a sum of the accumulators (keeps them live);
// clock[0..3] = shader clock and real-time counter at the start and end of wave 0 of
// workgroup 0.
__global__ __launch_bounds__(512, 1) void probe_smfmac_stream_kernel(int iters, float* __restrict__ out,
                                                                      unsigned long long* __restrict__ clock) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool rec = blockIdx.x == 0 && threadIdx.x == 0;
  unsigned long long c0 = 0, r0 = 0;
  if (rec) {
    c0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  const uint32_t seed = (blockIdx.x * 512u + threadIdx.x) * 131u;
  half8_t a[4];
  half16_t b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int e = 0; e < 8; e++) a[i][e] = rnd_half(seed + 16u * i + e);
#pragma unroll
    for (int e = 0; e < 16; e++) b[i][e] = rnd_half(seed + 1000u + 16u * i + e);
  }
  const uint32_t idx[2] = {0x4e4e4e4eu, 0xe4e4e4e4u};  // index nibbles (0,1) and (2,3)
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    acc[i] = (f32x16){};
    asm volatile("" : "+a"(acc[i]));
  }
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      if (r & 1) stream_smfmac<1>(acc[r & 7], a[r & 3], b[(r >> 2) & 3], idx[(r >> 3) & 1]);
      else stream_smfmac<0>(acc[r & 7], a[r & 3], b[(r >> 2) & 3], idx[(r >> 3) & 1]);
    }
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    f32x16 v = acc[i];
    asm volatile("" : "+v"(v));
#pragma unroll
    for (int e = 0; e < 16; e++) sum += v[e];
  }
  if (lane == 0) out[blockIdx.x * 8 + wave] = sum;
  if (rec) {
    clock[0] = c0;
    clock[1] = r0;
    clock[2] = __builtin_amdgcn_s_memtime();
    clock[3] = __builtin_amdgcn_s_memrealtime();
  }
}

}  // namespace

extern "C" {

int marlin_probe_read(const void* p, long long bytes, void* sink, int blocks, int dev, hipStream_t stream) {
  if (bytes < 0 || bytes % 16 != 0 || blocks == 0) return 1;
  if (bytes == 0) return 0;
  if (hipSetDevice(dev) != hipSuccess) return 3;
  // blocks > 0: grid-stride order; blocks < 0: -blocks workgroups, a contiguous range
  // per wave
  if (blocks > 0)
    hipLaunchKernelGGL(probe_read_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const u32x4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
  else
    hipLaunchKernelGGL(probe_read_chunk_kernel, dim3((unsigned)-blocks), dim3(256), 0, stream,
                       static_cast<const u32x4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int marlin_probe_empty(int blocks, int threads, int dev, hipStream_t stream) {
  if (blocks <= 0 || threads <= 0 || threads > 1024) return 1;
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_empty_kernel, dim3((unsigned)blocks), dim3((unsigned)threads), 0, stream);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int marlin_probe_smfmac_stream(int blocks, int iters, void* out, void* clock, int dev, hipStream_t stream) {
  if (blocks <= 0 || iters <= 0) return 1;
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_smfmac_stream_kernel, dim3((unsigned)blocks), dim3(512), 0, stream, iters,
                     static_cast<float*>(out), static_cast<unsigned long long*>(clock));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

int marlin_probe_mfma_32x32x16(const void* A, const void* B, void* D, int dev, hipStream_t stream) {
  if (hipSetDevice(dev) != hipSuccess) return 3;
  hipLaunchKernelGGL(probe_mfma_32x32x16_kernel, dim3(1), dim3(64), 0, stream, static_cast<const _Float16*>(A),
                     static_cast<const _Float16*>(B), static_cast<float*>(D));
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // extern "C"
