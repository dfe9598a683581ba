// Dense INT4 x FP16 GEMM on gfx950 (the reference's dense Marlin `mul`):
// C[M,N] = A[M,K] * W[K,N], W = (q - 8) * s with 4-bit codes q and fp16 scales.
//
// W is read in the dense Marlin pack() layout (reference
// kernel_experiments/sparse_marlin/src/marlin/__init__.py:78-99, 177-226):
//   * B  int32 [K/16][2N]: row r holds k-tile r (16 K).  Within a 64-column chunk c
//        (128 words) word w = 16*ci + 4*rq + jt holds, for the two columns
//        n = 64c + 16*jt + ci (bytes 0, 2) and n + 8 (bytes 1, 3), the codes of
//        k = 16r + {2rq, 2rq+8} (low / high nibble of byte 0 or 1) and
//        k = 16r + {2rq+1, 2rq+9} (low / high nibble of byte 2 or 3).
//   * s  fp16 [K/128][N] grouped: within 64 columns, slot 8i + j holds column i + 8j;
//        or [1][N] per column: within 32 columns, slot 8i + t holds column
//        2i + {0,1,8,9,16,17,24,25}[t] (applied to the fp16-rounded sum).
//
// The weight is the A operand of v_mfma_f32_16x16x32_f16 (rows = output columns),
// activations the B operand (columns = batch rows).  Lane (rho, h) = (l % 16, l / 16)
// of the MFMA for column tile jt holds column 64c + 16*jt + rho (ci = rho & 7, byte
// b = rho >> 3) and 8 k of k-tile kt = h >> 1 of the 32-deep k-step: k = 4(h&1) + 0..3
// (low nibbles of words rq = 2(h&1), 2(h&1)+1) and 8 + 4(h&1) + 0..3 (their high
// nibbles).  So one lane loads the two 16-byte word groups (ci, rq, jt = 0..3) and
// feeds the four column tiles of the chunk from them.
//
// Work decomposition (one launch): grid.x 64-column chunk, grid.y K split, grid.z
// batch tile of 16*BB rows; NW waves take contiguous ranges of the split's k-steps
// through a ring of U in-flight fragments and are reduced in LDS in a fixed order;
// with several splits the last workgroup to arrive at the tile's counter adds the
// splits' fp32 partials in split order (bit-identical from run to run).
//
// Reference: marlin_cuda_kernel.cu (Marlin at 90-605, host dispatch marlin_cuda at
// 655-736) and marlin_cuda.cpp:38-64 (the binding's checks).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "marlin_dense_prefill.h"
#include "sm24_device.h"
#include "sm24_host.h"
#include "../../include/marlin_hip.h"

namespace sm24 {

struct DenseArgs {
  const _Float16* A;
  const uint32_t* B;
  const _Float16* s;
  _Float16* C;
  const _Float16* zeros;  // >= 64 zero bytes (rows past M)
  int M, N, K;
  int splits;
  float* partial;      // [splits][M][N] when splits > 1
  uint32_t* counters;  // [gridDim.z][gridDim.x], zero between launches
};

template <int BB, bool GROUPED>
struct DenseFrag {
  u32x4 w0, w1;      // word groups (ci, rq0, jt = 0..3) and (ci, rq0 + 1, jt = 0..3)
  half8_t sc;        // grouped: scale slots 8*ci .. 8*ci + 7 (columns ci + 8j)
  half8_t act[BB];   // activation B operands
};

// The fields the prologue needs first come as leading scalar arguments, preloaded
// into SGPRs (this translation unit is built with -mllvm
// -amdgpu-kernarg-preload-count=14), ahead of the whole DenseArgs; the fp16
// pointers travel as void pointers, which keeps the kernel's name demangleable.
template <int BB, int NW, bool GROUPED>
__global__ __launch_bounds__(64 * NW) void marlin_dense_kernel(const void* A_, const uint32_t* B_, const void* s_,
                                                               const void* zeros_, int M_, int N_, int K_, int splits_,
                                                               DenseArgs a_) {
  DenseArgs a = a_;
  a.A = static_cast<const _Float16*>(A_);
  a.B = B_;
  a.s = static_cast<const _Float16*>(s_);
  a.zeros = static_cast<const _Float16*>(zeros_);
  a.M = M_;
  a.N = N_;
  a.K = K_;
  a.splits = splits_;
  constexpr int NT = 64 * NW;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int chunk = blockIdx.x, split = blockIdx.y, bt = blockIdx.z;
  const int N = a.N, K = a.K, M = a.M;
  const int nks = K >> 5;  // 32-deep k-steps
  int ks0 = 0, ks1 = nks;
  if (a.splits > 1) {  // uniform; nks * splits is small, so 32 bits are exact
    ks0 = (int)((unsigned)(nks * split) / (unsigned)a.splits);
    ks1 = (int)((unsigned)(nks * (split + 1)) / (unsigned)a.splits);
  }
  const int h = lane >> 4, rho = lane & 15;
  const int ci = rho & 7, b = rho >> 3;
  const int kt = h >> 1, rq0 = 2 * (h & 1);
  const uint32_t sh = 8u * (uint32_t)b;

  // k-step ks reads B rows 2ks + kt: words (ci, rq0, 0..3) and (ci, rq0 + 1, 0..3)
  const uint32_t* bw = a.B + 128 * (size_t)chunk + 16 * ci + 4 * rq0 + 2 * (size_t)N * kt;
  const size_t bstep = 4 * (size_t)N;  // words per k-step (two rows)
  const _Float16* sp = a.s + 64 * (size_t)chunk + 8 * ci;
  const int row0 = 16 * BB * bt + rho;
  const int koff = 16 * kt + 4 * (h & 1);

  auto fetch = [&](int ks, bool live, DenseFrag<BB, GROUPED>& f) {
    const uint32_t* p = bw + (size_t)ks * bstep;
    f.w0 = *reinterpret_cast<const u32x4*>(p);
    f.w1 = *reinterpret_cast<const u32x4*>(p + 4);
    if constexpr (GROUPED) f.sc = *reinterpret_cast<const half8_t*>(sp + (size_t)(ks >> 2) * N);
#pragma unroll
    for (int bb = 0; bb < BB; bb++) {
      // rows past M (and ring slots past the range) read the zero block: only the
      // address is selected, so the ring keeps a fixed shape
      const int m = row0 + 16 * bb;
      const _Float16* ap = (live && m < M) ? a.A + (size_t)m * K + 32 * ks + koff : a.zeros;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(ap);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(ap + 8);
      f.act[bb] = __builtin_bit_cast(half8_t, (u32x4){lo.x, lo.y, hi.x, hi.y});
    }
  };

  float4_t acc[BB][4];
#pragma unroll
  for (int bb = 0; bb < BB; bb++)
#pragma unroll
    for (int jt = 0; jt < 4; jt++) acc[bb][jt] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // Dequant constants held in VGPRs, so that mask-and-or is one v_and_or_b32.
  uint32_t kMask, kMaskHi, kMagic;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));
  const uint32_t ssh = 16u * (uint32_t)b;  // the lane's scale: half b of scale word jt
  auto compute = [&](const DenseFrag<BB, GROUPED>& f) {
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
      // column 16 jt + rho: byte b of words rq0 (k 4(h&1) + 0, 1 | 8 + ...) and rq0 + 1;
      // magic-exponent conversion as in dequant4 ({k, k+1 | k+8, k+9} of each word)
      const uint32_t x0 = f.w0[jt] >> sh, x1 = f.w1[jt] >> sh;
      const half2_t kz = {(_Float16)1032.0f, (_Float16)1032.0f};
      const half2_t k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
      const half2_t kzh = {(_Float16)-72.0f, (_Float16)-72.0f};
      const half2_t l0 = __builtin_bit_cast(half2_t, (x0 & kMask) | kMagic) - kz;
      const half2_t l1 = __builtin_bit_cast(half2_t, (x1 & kMask) | kMagic) - kz;
      const half2_t u0 = __builtin_bit_cast(half2_t, (x0 & kMaskHi) | kMagic) * k16 + kzh;
      const half2_t u1 = __builtin_bit_cast(half2_t, (x1 & kMaskHi) | kMagic) * k16 + kzh;
      half8_t aop = (half8_t){l0.x, l0.y, l1.x, l1.y, u0.x, u0.y, u1.x, u1.y};
      if constexpr (GROUPED) {
        // scale slot 2 jt + b: one shift of word jt (a variable element index would
        // compile to a select over all eight halves)
        const uint32_t sw = __builtin_bit_cast(u32x4, f.sc)[jt] >> ssh;
        const _Float16 sc = __builtin_bit_cast(half2_t, sw).x;
        aop = aop * (half8_t){sc, sc, sc, sc, sc, sc, sc, sc};
      }
#pragma unroll
      for (int bb = 0; bb < BB; bb++)
        acc[bb][jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, f.act[bb], acc[bb][jt], 0, 0, 0);
    }
  };

  // Each wave streams a contiguous share of the split's k-steps through a ring of U
  // fragments; slots past the end re-read the last k-step with zero activations.
  constexpr int U = BB == 1 ? 6 : 4;
  const int span = ks1 - ks0;
  const int r0 = ks0 + span * wave / NW;
  const int r1 = ks0 + span * (wave + 1) / NW;
  if (r1 > r0) {
    const int rlast = r1 - 1;
    DenseFrag<BB, GROUPED> ring[U];
#pragma unroll
    for (int i = 0; i < U; i++) {
      fetch(r0 + i < r1 ? r0 + i : rlast, r0 + i < r1, ring[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int base = r0; base < r1; base += U) {
#pragma unroll
      for (int i = 0; i < U; i++) {
        compute(ring[i]);
        __builtin_amdgcn_sched_barrier(0);
        const int rn = base + i + U;
        fetch(rn < r1 ? rn : rlast, rn < r1, ring[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ---- reduce the NW waves in LDS: red[wave][row][col], col = column in the chunk ----
  constexpr int RS = 65;  // padded row stride (floats)
  __shared__ float red[NW][16 * BB][RS];
#pragma unroll
  for (int bb = 0; bb < BB; bb++)
#pragma unroll
    for (int jt = 0; jt < 4; jt++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[wave][16 * bb + rho][16 * jt + 4 * h + i] = acc[bb][jt][i];
  __syncthreads();

  const int ntile = 16 * BB * 64;
  const int ncol0 = 64 * chunk;
  // per-column scale of chunk column nl (per-column quantization): slot 8 ((nl % 8) / 2)
  // + 2 (nl / 8) + nl % 2 of the 32-column half the column lies in
  auto col_scale = [&](int nl) -> _Float16 {
    const int c = nl & 31;
    return a.s[ncol0 + (nl & 32) + 8 * ((c & 7) >> 1) + 2 * (c >> 3) + (c & 1)];
  };
  if (a.splits == 1) {
    for (int e = threadIdx.x; e < ntile; e += NT) {
      const int ml = e >> 6, nl = e & 63;
      const int m = 16 * BB * bt + ml;
      if (m >= M) continue;
      float v = red[0][ml][nl];
#pragma unroll
      for (int w = 1; w < NW; w++) v += red[w][ml][nl];
      _Float16 o = (_Float16)v;
      if constexpr (!GROUPED) o = o * col_scale(nl);
      a.C[(size_t)m * N + ncol0 + nl] = o;
    }
    return;
  }

  // Split-K hand-off through the uncached scratch (device-scope atomic accesses): each
  // thread's partial stores complete before the workgroup barrier, the tile's counter
  // is bumped after it, and the last split to arrive adds all partials in split order,
  // writes C and resets the counter.
  for (int e = threadIdx.x; e < ntile; e += NT) {
    const int ml = e >> 6, nl = e & 63;
    const int m = 16 * BB * bt + ml;
    if (m >= M) continue;
    float v = red[0][ml][nl];
#pragma unroll
    for (int w = 1; w < NW; w++) v += red[w][ml][nl];
    __hip_atomic_store(a.partial + ((size_t)split * M + m) * N + ncol0 + nl, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  __shared__ uint32_t arrived;
  uint32_t* cnt = a.counters + bt * gridDim.x + chunk;
  if (threadIdx.x == 0) arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  __syncthreads();
  if (arrived != (uint32_t)a.splits) return;
  for (int e = threadIdx.x; e < ntile; e += NT) {
    const int ml = e >> 6, nl = e & 63;
    const int m = 16 * BB * bt + ml;
    if (m >= M) continue;
    const float* pp = a.partial + (size_t)m * N + ncol0 + nl;
    const size_t pstride = (size_t)M * N;
    float v = 0.f;
    int q = 0;
    for (; q + 4 <= a.splits; q += 4) {  // four loads in flight, summed in split order
      const float p0 = __hip_atomic_load(pp + (q + 0) * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float p1 = __hip_atomic_load(pp + (q + 1) * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float p2 = __hip_atomic_load(pp + (q + 2) * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float p3 = __hip_atomic_load(pp + (q + 3) * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v += p0;
      v += p1;
      v += p2;
      v += p3;
    }
    for (; q < a.splits; q++) v += __hip_atomic_load(pp + q * pstride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    _Float16 o = (_Float16)v;
    if constexpr (!GROUPED) o = o * col_scale(nl);
    a.C[(size_t)m * N + ncol0 + nl] = o;
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// The reference binding's and dispatch's shape rules (marlin_cuda.cpp:43-49,
// marlin_cuda_kernel.cu:660-683, 711-721): default tiles (thread_k, thread_n) =
// (128, 128) for at most 16 batch rows, else (64, 256); N % thread_n, K % thread_k
// and K % (groupsize / 16) (the reference's own test) or code 1; instantiated tiles
// (128, 128) for one 16-row block and (64, 256), with groupsize -1 or 128, or code 2.
int dense_validate(int prob_m, int prob_n, int prob_k, int groupsize, int thread_k, int thread_n) {
  if (thread_k == -1 || thread_n == -1) {
    if (prob_m <= 16) {
      thread_k = 128;
      thread_n = 128;
    } else {
      thread_k = 64;
      thread_n = 256;
    }
  }
  if (thread_k <= 0 || thread_n <= 0) return MARLIN_HIP_ERR_KERN_SHAPE;
  const int group_blocks = groupsize == -1 ? -1 : groupsize / 16;
  if (prob_n % thread_n != 0 || prob_k % thread_k != 0 || (group_blocks > 0 && prob_k % group_blocks != 0))
    return MARLIN_HIP_ERR_PROB_SHAPE;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return MARLIN_HIP_OK;
  const bool tile_ok = (thread_n == 128 && thread_k == 128 && prob_m <= 16) || (thread_n == 256 && thread_k == 64);
  if (!tile_ok || !(group_blocks == -1 || group_blocks == 8)) return MARLIN_HIP_ERR_KERN_SHAPE;
  return MARLIN_HIP_OK;
}

template <int BB, bool G>
hipError_t launch_dense_t(const DenseArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int NW = 4;
  hipLaunchKernelGGL((marlin_dense_kernel<BB, NW, G>), grid, dim3(64 * NW), 0, stream, a.A, a.B, a.s, a.zeros, a.M,
                     a.N, a.K, a.splits, a);
  return hipGetLastError();
}

// K splits, from forced splits 1-16 over the Llama-2-7B decode calls (MI355X): a
// split's hand-off costs microseconds, so tiles that already cover at least 3/4 of
// the CUs run unsplit (qkv, 192 chunks: 16.0 -> 13.8 us at M = 1 against three
// splits); fewer tiles split to about one workgroup per CU (o and down, 64 chunks:
// four splits, 9.9 -> 9.0 and 12.7 -> 12.2 us against eight); between one and two
// tiles per CU split in two, which balances the CUs (gate_up, 344 chunks: 20.7
// against 22.3 us unsplit).  Each wave keeps at least two k-steps; at most 16
// splits and one arrival counter per (chunk, batch tile).  MARLIN_HIP_DENSE_SPLITS
// forces the count.
int dense_splits(int chunks, int ztiles, int nks, int cus) {
  static const int forced = [] {
    const char* e = getenv("MARLIN_HIP_DENSE_SPLITS");
    const int x = e ? atoi(e) : 0;
    return x >= 1 && x <= 16 ? x : 0;
  }();
  const long long tiles = (long long)chunks * ztiles;
  int s = 1;
  if (forced) s = forced;
  else if (tiles >= cus) s = tiles < 2LL * cus ? 2 : 1;
  else if (4 * tiles < 3LL * cus) s = (int)((cus + tiles / 2) / tiles);
  const int smax = nks / 8 > 0 ? nks / 8 : 1;
  if (s > smax) s = smax;
  if (s > 16) s = 16;
  if (s < 1) s = 1;
  if ((size_t)tiles * sizeof(uint32_t) > kCounterBytes) s = 1;
  return s;
}

// Large-M path (marlin_dense_prefill_kernel): N a multiple of its 512-column tile, K of
// 128 (whole scale groups, an even number of 64-deep k-steps) and 32-bit operand
// offsets, from MARLIN_HIP_DENSE_PREFILL_MIN_M rows (default 65).
bool dense_prefill_fits(int M, int N, int K) {
  static const int forced_min_m = [] {
    const char* e = getenv("MARLIN_HIP_DENSE_PREFILL_MIN_M");
    const int x = e ? atoi(e) : 0;
    return x >= 1 ? x : 0;
  }();
  const int min_m = forced_min_m ? forced_min_m : 65;
  return M >= min_m && N % kDpTileCols == 0 && K % 128 == 0 && (long long)M * K < (1LL << 31) - 2048 &&
         (long long)K * N < (1LL << 33);
}

// K splits of the dense large-M kernel, by the 2:4 prefill planner's model: rounds of
// one workgroup per CU times the k-steps per split, plus the partial exchange (each
// split stores a 256 KiB fp32 tile), at ~1.3 us per 64-deep k-step of a tile (32
// MFMAs per wave) and ~2.5 TB/s for the exchange.  MARLIN_HIP_DENSE_PREFILL_SPLITS
// forces a count.
int dense_prefill_splits(int tiles, int nks, int cus) {
  static const int forced = [] {
    const char* e = getenv("MARLIN_HIP_DENSE_PREFILL_SPLITS");
    const int x = e ? atoi(e) : 0;
    return x >= 1 && x <= 16 ? x : 0;
  }();
  const int max_s = nks / 8;  // at least eight k-steps per split
  if (forced) return forced < max_s ? forced : (max_s > 0 ? max_s : 1);
  const double step_us = 1.3, exchange_bytes_per_us = 2.5e6;
  int best_s = 1;
  double best = 1e30;
  for (int s = 1; s <= 8 && s <= max_s; s++) {
    const long long rounds = ((long long)tiles * s + cus - 1) / cus;
    const double traffic = s > 1 ? 2.0 * tiles * s * (double)kDpSplitBytes : 0.0;
    const double cost = (double)rounds * step_us * nks / s + traffic / exchange_bytes_per_us;
    if (cost < 0.97 * best) {
      best = cost;
      best_s = s;
    }
  }
  if ((size_t)tiles * sizeof(uint32_t) > kCounterBytes) best_s = 1;
  return best_s;
}

int run_dense_prefill(const void* A, const void* B, void* C, const void* s, int M, int N, int K, bool grouped,
                      int dev, hipStream_t stream, int sms) {
  DensePreArgs p{};
  p.A = static_cast<const _Float16*>(A);
  p.B = static_cast<const uint32_t*>(B);
  p.s = static_cast<const _Float16*>(s);
  p.C = static_cast<_Float16*>(C);
  p.M = M;
  p.N = N;
  p.K = K;
  const int tiles = (N / kDpTileCols) * ((M + kDpRows - 1) / kDpRows);
  p.splits = dense_prefill_splits(tiles, K / 64, sms);
  if (p.splits > 1) {
    const int err = get_scratch(dev, stream, (size_t)tiles * p.splits * kDpSplitBytes, &p.counters, &p.partial);
    if (err != MARLIN_HIP_OK) return err;
    if (!p.counters) p.splits = 1;  // capturing, and this stream has no scratch yet
  }
  return launch_error(launch_dense_prefill(p, grouped, stream));
}

int run_dense(const void* A, const void* B, void* C, const void* s, int prob_m, int prob_n, int prob_k,
              int groupsize, int dev, hipStream_t stream, int thread_k, int thread_n, int sms) {
  int err = dense_validate(prob_m, prob_n, prob_k, groupsize, thread_k, thread_n);
  if (err != MARLIN_HIP_OK) return err;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return MARLIN_HIP_OK;
  const int M = prob_m, N = prob_n, K = prob_k;
  if (N % 64 != 0 || K % 128 != 0) {  // implied by the tiles above; the kernel's own units
    set_error("marlin_hip: dense N must be a multiple of 64 and K of 128");
    return MARLIN_HIP_ERR_PROB_SHAPE;
  }
  DeviceScope scope(dev);
  if (!scope.ok) return MARLIN_HIP_ERR_LAUNCH;
  if (sms <= 0) {
    if (hipDeviceGetAttribute(&sms, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || sms <= 0)
      sms = 256;
  }
  if (dense_prefill_fits(M, N, K)) return run_dense_prefill(A, B, C, s, M, N, K, groupsize != -1, dev, stream, sms);
  const int bb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int ztiles = (M + 16 * bb - 1) / (16 * bb);
  const int chunks = N / 64;
  DenseArgs a{};
  a.A = static_cast<const _Float16*>(A);
  a.B = static_cast<const uint32_t*>(B);
  a.s = static_cast<const _Float16*>(s);
  a.C = static_cast<_Float16*>(C);
  a.M = M;
  a.N = N;
  a.K = K;
  err = get_zeros(dev, stream, &a.zeros);
  if (err != MARLIN_HIP_OK) return err;
  a.splits = dense_splits(chunks, ztiles, K / 32, sms);
  if (a.splits > 1) {
    err = get_scratch(dev, stream, (size_t)a.splits * M * N * sizeof(float), &a.counters, &a.partial);
    if (err != MARLIN_HIP_OK) return err;
    if (!a.counters) a.splits = 1;  // capturing, and this stream has no scratch yet
  }
  const dim3 grid(chunks, a.splits, ztiles);
  const bool grouped = groupsize != -1;
  hipError_t e;
  if (bb == 1) e = grouped ? launch_dense_t<1, true>(a, grid, stream) : launch_dense_t<1, false>(a, grid, stream);
  else if (bb == 2) e = grouped ? launch_dense_t<2, true>(a, grid, stream) : launch_dense_t<2, false>(a, grid, stream);
  else e = grouped ? launch_dense_t<4, true>(a, grid, stream) : launch_dense_t<4, false>(a, grid, stream);
  return launch_error(e);
}

}  // namespace sm24

extern "C" int marlin_hip_mul(const void* A, const void* B, void* C, void* s, int prob_m, int prob_n, int prob_k,
                              void* workspace, int groupsize, int dev, hipStream_t stream, int thread_k,
                              int thread_n, int sms, int max_par) {
  (void)workspace;
  (void)max_par;
  return sm24::run_dense(A, B, C, s, prob_m, prob_n, prob_k, groupsize, dev, stream, thread_k, thread_n, sms);
}
