// 2:4-sparse INT4 x FP16 GEMM on gfx950: C[M,N] = A[M,K] * W[K,N].
//
// W is the Sparse-Marlin packed weight (values B, 2:4 metadata, fp16 scales) in the
// reference pack() layout; see sm24_device.h for the byte-level layout.  The weight
// is the sparse A operand of v_smfmac (MFMA rows = output columns), activations are
// the dense B operand (MFMA columns = batch rows).
//
// Work decomposition (one launch):
//   grid.x  64-column chunk of N (the unit of the packed layouts: 512 B of B,
//           256 B of metadata and 128 B of scales per k-block)
//   grid.y  K split: a contiguous range of 32-deep k-blocks
//   grid.z  batch tile of 16*BB rows
// Four waves per workgroup take interleaved k-blocks of the split; their fp32
// accumulators are reduced in LDS in a fixed order.  With more than one split,
// each workgroup stores its fp32 tile to scratch and the last one to arrive
// (agent-scope counter) sums the splits in split order and writes C.  The result
// is therefore bit-identical from run to run.
//
// Reference: kernel_experiments/sparse_marlin/src/marlin/marlin_cuda_kernel_nm.cu
// (Marlin_2_4 at 42-723, host dispatch marlin_cuda_2_4 at 751-830).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "sm24_device.h"
#include "../../include/marlin_hip.h"

namespace sm24 {

enum : int { VAL4 = 0, VAL3 = 1 };
enum : int { META4 = 0, META3 = 1 };

struct GemmArgs {
  const _Float16* A;
  const void* B;
  const void* meta;
  const _Float16* s;
  _Float16* C;
  int M, N, K;
  int splits;
  float* partial;  // [splits][M][N] when splits > 1
  uint32_t* counters;  // [gridDim.z][gridDim.x] tagged arrival counters
  uint32_t tag;        // launch tag, 1..2^24-1
};

// 4-bit nibble tables of the 3-bit metadata decoders (pair.cu:11 of the
// reference's decoder_dependency experiment): code c -> nibble (LUT >> 4c) & 15.
constexpr uint32_t lut_of(const int (&t)[8]) {
  uint32_t v = 0;
  for (int i = 0; i < 8; i++) v |= (uint32_t)t[i] << (4 * i);
  return v;
}
constexpr int kDecHigh[8] = {14, 13, 8, 13, 3, 4, 9, 12};
constexpr int kDecLow[8] = {12, 13, 14, 10, 8, 9, 4, 0};
constexpr uint32_t kLutHigh = lut_of(kDecHigh);
constexpr uint32_t kLutLow = lut_of(kDecLow);

template <int BB>
struct Frag {
  uint32_t w0, w1;   // packed words j = 2*jb, 2*jb+1 (nibble form)
  uint32_t idx;      // sparse-index bytes, byte (jj + 2*blk)
  half4_t sc;        // grouped scales {s(jj0,b0), s(jj0,b1), s(jj1,b0), s(jj1,b1)}
  half8_t act[BB];   // activation B operands
};

template <int BB, bool GROUPED, int VF, int MF>
__global__ __launch_bounds__(256) void sm24_gemm_kernel(GemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int chunk = blockIdx.x;
  const int split = blockIdx.y;
  const int bt = blockIdx.z;
  const int N = a.N, K = a.K, M = a.M;
  const int nkb = K >> 5;
  const int kb0 = (int)(((long long)nkb * split) / a.splits);
  const int kb1 = (int)(((long long)nkb * (split + 1)) / a.splits);

  const int h = lane >> 4;    // k-space lane group: dense groups h and h+4 of a k-block
  const int rho = lane & 15;  // A-operand row / B-operand column
  const int g = rho & 7;
  const int jb = rho >> 3;
  const uint32_t sh = 4u * (uint32_t)h;

  // Per-lane base pointers (k-block 0).
  const uint32_t* bw = static_cast<const uint32_t*>(a.B) + 128 * chunk + 16 * g + 4 * h + 2 * jb;
  const uint8_t* b3 = static_cast<const uint8_t*>(a.B) +
                      6 * (size_t)(64 * chunk + 8 * g + 2 * h + jb) - 2 * jb;
  const uint32_t* mw = static_cast<const uint32_t*>(a.meta) + 64 * chunk + 32 * jb + 4 * g;
  const uint32_t* m3 = static_cast<const uint32_t*>(a.meta) + 48 * chunk + 16 * (g >> 2) + 4 * (g & 3);
  const _Float16* sp = a.s + 64 * chunk + 8 * g + 4 * jb;
  const int row0 = 16 * BB * bt + rho;

  auto fetch = [&](int r, Frag<BB>& f) {
    if constexpr (VF == VAL4) {
      const u32x2 w = *reinterpret_cast<const u32x2*>(bw + (size_t)r * (2 * (size_t)N));
      f.w0 = w.x;
      f.w1 = w.y;
    } else {
      const u32x2 w = *reinterpret_cast<const u32x2_a4*>(b3 + (size_t)r * (6 * (size_t)N));
      const uint64_t v = ((uint64_t)w.y << 32 | w.x) >> (16 * jb);
      f.w0 = spread3((uint32_t)v & 0xFFFFFFu);
      f.w1 = spread3((uint32_t)(v >> 24) & 0xFFFFFFu);
    }
    if constexpr (MF == META4) {
      const u32x4 md = *reinterpret_cast<const u32x4*>(mw + (size_t)r * N);
      f.idx = idx_pair(md.x, md.y, sh) | (idx_pair(md.z, md.w, sh) << 8);
    } else {
      // 48-word group for (k-block r, chunk): words 0..15 / 16..31 / 32..47 hold
      // the 48-bit "first" and "second" code pairs of the 64 metadata words.
      const uint32_t* base = m3 + (size_t)r * (size_t)(3 * N / 4);
      const u32x4 X = *reinterpret_cast<const u32x4*>(base);
      const u32x4 Y = *reinterpret_cast<const u32x4*>(base + 16);
      const uint32_t lut = jb ? kLutLow : kLutHigh;
      uint32_t xs[4];
#pragma unroll
      for (int v = 0; v < 4; v++) {
        uint32_t c24;
        if ((g >> 2) == 0) {
          c24 = jb ? ((X[v] >> 24) | ((Y[v] & 0xFFFFu) << 8)) : (X[v] & 0xFFFFFFu);
        } else {
          c24 = jb ? ((Y[v] >> 8) & 0xFFFFFFu) : (((X[v] >> 16) | (Y[v] << 16)) & 0xFFFFFFu);
        }
        const uint32_t ca = (c24 >> (3 * h)) & 7u;
        const uint32_t cb = (c24 >> (3 * h + 12)) & 7u;
        xs[v] = ((lut >> (4 * ca)) & 15u) | (((lut >> (4 * cb)) & 15u) << 16);
      }
      f.idx = (xs[0] | (xs[1] << 4)) | ((xs[2] | (xs[3] << 4)) << 8);
    }
    if constexpr (GROUPED) {
      f.sc = *reinterpret_cast<const half4_t*>(sp + (size_t)(r >> 2) * N);
    }
#pragma unroll
    for (int bb = 0; bb < BB; bb++) {
      const int m = row0 + 16 * bb;
      if (m < M) {
        const _Float16* ap = a.A + (size_t)m * K + 32 * r + 4 * h;
        const half4_t lo = *reinterpret_cast<const half4_t*>(ap);
        const half4_t hi = *reinterpret_cast<const half4_t*>(ap + 16);
        f.act[bb] = (half8_t){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      } else {
        f.act[bb] = (half8_t){};
      }
    }
  };

  float4_t acc[BB][4];
#pragma unroll
  for (int bb = 0; bb < BB; bb++)
#pragma unroll
    for (int t = 0; t < 4; t++) acc[bb][t] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Frag<BB>& f) {
    half4_t a00, a01, a10, a11;  // (jj, blk)
    if constexpr (VF == VAL4) {
      a00 = dequant4(f.w0);
      a01 = dequant4(f.w0 >> 8);
      a10 = dequant4(f.w1);
      a11 = dequant4(f.w1 >> 8);
    } else {
      a00 = dequant3(f.w0);
      a01 = dequant3(f.w0 >> 8);
      a10 = dequant3(f.w1);
      a11 = dequant3(f.w1 >> 8);
    }
    if constexpr (GROUPED) {
      a00 = scale4(a00, f.sc.x);
      a01 = scale4(a01, f.sc.y);
      a10 = scale4(a10, f.sc.z);
      a11 = scale4(a11, f.sc.w);
    }
#pragma unroll
    for (int bb = 0; bb < BB; bb++) {
      acc[bb][0] = smfmac32<0>(a00, f.act[bb], acc[bb][0], f.idx);
      acc[bb][1] = smfmac32<1>(a10, f.act[bb], acc[bb][1], f.idx);
      acc[bb][2] = smfmac32<2>(a01, f.act[bb], acc[bb][2], f.idx);
      acc[bb][3] = smfmac32<3>(a11, f.act[bb], acc[bb][3], f.idx);
    }
  };

  int r = kb0 + wave;
  if (r < kb1) {
    Frag<BB> cur;
    fetch(r, cur);
    while (true) {
      const int rn = r + 4;
      Frag<BB> nxt;
      const bool more = rn < kb1;
      if (more) fetch(rn, nxt);
      compute(cur);
      if (!more) break;
      cur = nxt;
      r = rn;
    }
  }

  // ---- reduce the four waves in LDS: red[wave][row][col], col = n within chunk ----
  constexpr int RS = 65;  // padded row stride (floats)
  __shared__ float red[4][16 * BB][RS];
#pragma unroll
  for (int bb = 0; bb < BB; bb++) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int jj = t & 1, blk = t >> 1;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int rp = 4 * h + i;  // D row = A row index rho'
        const int n_local = 8 * (rp & 7) + 2 * (rp >> 3) + jj + 4 * blk;
        red[wave][16 * bb + rho][n_local] = acc[bb][t][i];
      }
    }
  }
  __syncthreads();

  const int ntile = 16 * BB * 64;
  const int ncol0 = 64 * chunk;
  if (a.splits == 1) {
    for (int e = threadIdx.x; e < ntile; e += 256) {
      const int ml = e >> 6, nl = e & 63;
      const int m = 16 * BB * bt + ml;
      if (m >= M) continue;
      const float v = red[0][ml][nl] + red[1][ml][nl] + red[2][ml][nl] + red[3][ml][nl];
      _Float16 o = (_Float16)v;
      if constexpr (!GROUPED) o = o * a.s[ncol0 + nl];
      a.C[(size_t)m * N + ncol0 + nl] = o;
    }
    return;
  }

  for (int e = threadIdx.x; e < ntile; e += 256) {
    const int ml = e >> 6, nl = e & 63;
    const int m = 16 * BB * bt + ml;
    if (m >= M) continue;
    const float v = red[0][ml][nl] + red[1][ml][nl] + red[2][ml][nl] + red[3][ml][nl];
    __hip_atomic_store(a.partial + ((size_t)split * M + m) * N + ncol0 + nl, v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __threadfence();
  __syncthreads();
  // Arrival counter of this (chunk, batch tile): bits 31..8 carry the launch's tag,
  // bits 7..0 the number of splits that have arrived.  A slot holding another tag
  // (a finished launch resets it to 0; anything else is stale) restarts at 1.
  __shared__ uint32_t arrived;
  uint32_t* cnt = a.counters + bt * gridDim.x + chunk;
  if (threadIdx.x == 0) {
    uint32_t old = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t nv;
    while (true) {
      nv = ((old >> 8) == a.tag) ? old + 1u : ((a.tag << 8) | 1u);
      if (__hip_atomic_compare_exchange_strong(cnt, &old, nv, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        break;
    }
    arrived = nv & 0xFFu;
  }
  __syncthreads();
  if (arrived != (uint32_t)a.splits) return;
  __threadfence();
  for (int e = threadIdx.x; e < ntile; e += 256) {
    const int ml = e >> 6, nl = e & 63;
    const int m = 16 * BB * bt + ml;
    if (m >= M) continue;
    float v = 0.f;
    for (int q = 0; q < a.splits; q++)
      v += __hip_atomic_load(a.partial + ((size_t)q * M + m) * N + ncol0 + nl, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    _Float16 o = (_Float16)v;
    if constexpr (!GROUPED) o = o * a.s[ncol0 + nl];
    a.C[(size_t)m * N + ncol0 + nl] = o;
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};

// Split-K scratch (arrival counters + fp32 partials), one per device and shared by
// every stream: calls that overlap in time on one device must not both split K.
// Buffers are never freed: a captured graph may still refer to an old one.
std::mutex g_scratch_mu;
std::map<int, Scratch> g_scratch;
std::map<int, uint32_t> g_tag;

constexpr size_t kCounterBytes = 64 * 1024;  // up to 16384 (chunk, batch-tile) counters

int get_scratch(int dev, hipStream_t stream, size_t partial_bytes, uint32_t** counters, float** partial,
                uint32_t* tag) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_scratch[dev];
  const size_t need = kCounterBytes + partial_bytes;
  if (s.bytes < need) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone) {
      set_error("marlin_hip: the split-K scratch would have to grow during stream capture; make one "
                "call of the same (or a larger) shape on this device before capturing");
      return MARLIN_HIP_ERR_LAUNCH;
    }
    size_t nb = need > 2 * s.bytes ? need : 2 * s.bytes;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, nb);
    if (e != hipSuccess) {
      set_error(std::string("marlin_hip: hipMalloc of scratch failed: ") + hipGetErrorString(e));
      return MARLIN_HIP_ERR_LAUNCH;
    }
    e = hipMemset(p, 0, kCounterBytes);
    if (e != hipSuccess) {
      set_error(std::string("marlin_hip: hipMemset of scratch failed: ") + hipGetErrorString(e));
      return MARLIN_HIP_ERR_LAUNCH;
    }
    s.ptr = p;
    s.bytes = nb;
  }
  uint32_t& t = g_tag[dev];
  t = (t % 0xFFFFFFu) + 1u;  // 1 .. 2^24-1; 0 marks a free counter
  *tag = t;
  *counters = static_cast<uint32_t*>(s.ptr);
  *partial = reinterpret_cast<float*>(static_cast<char*>(s.ptr) + kCounterBytes);
  return MARLIN_HIP_OK;
}

struct Plan {
  int bb;
  int splits;
  int ztiles;
};

Plan plan_for(int M, int N, int K, int cus) {
  Plan p;
  p.bb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.ztiles = (M + 16 * p.bb - 1) / (16 * p.bb);
  const int chunks = N / 64;
  const int nkb = K / 32;
  const long long tiles = (long long)chunks * p.ztiles;
  const long long target = 2LL * cus;
  int splits = (int)((target + tiles - 1) / tiles);
  const int max_splits = nkb / 4 > 0 ? nkb / 4 : 1;  // at least one k-block per wave
  if (splits > max_splits) splits = max_splits;
  if (splits > 32) splits = 32;
  if (splits < 1) splits = 1;
  p.splits = splits;
  return p;
}

template <int BB, bool GROUPED, int VF, int MF>
hipError_t launch_t(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((sm24_gemm_kernel<BB, GROUPED, VF, MF>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int VF, int MF>
hipError_t launch_v(const GemmArgs& a, int bb, bool grouped, dim3 grid, hipStream_t stream) {
  if (grouped) {
    if (bb == 1) return launch_t<1, true, VF, MF>(a, grid, stream);
    if (bb == 2) return launch_t<2, true, VF, MF>(a, grid, stream);
    return launch_t<4, true, VF, MF>(a, grid, stream);
  }
  if (bb == 1) return launch_t<1, false, VF, MF>(a, grid, stream);
  if (bb == 2) return launch_t<2, false, VF, MF>(a, grid, stream);
  return launch_t<4, false, VF, MF>(a, grid, stream);
}

// Shape/tile validation with the reference's rules and error codes
// (marlin_cuda_kernel_nm.cu:760-823).
int validate(int prob_m, int prob_n, int prob_k, int groupsize, int thread_k, int thread_m) {
  if (thread_k == -1 || thread_m == -1) {
    if (prob_n <= 16) {
      thread_k = 128;
      thread_m = 128;
    } else {
      thread_k = 64;
      thread_m = 256;
    }
  }
  if (thread_k <= 0 || thread_m <= 0) return MARLIN_HIP_ERR_KERN_SHAPE;
  const int group_blocks = groupsize == -1 ? -1 : groupsize / 16;
  if (prob_m % thread_m != 0 || prob_k % thread_k != 0 ||
      (group_blocks > 0 && (prob_k / 2) % group_blocks != 0))
    return MARLIN_HIP_ERR_PROB_SHAPE;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return MARLIN_HIP_OK;
  // The reference instantiates (thread_m, thread_k) = (128, 128) for one 16-row
  // batch block and (256, 64) for 1..4 blocks, with group_blocks in {-1, 4}.
  const bool tile_ok = (thread_m == 128 && thread_k == 128 && prob_n <= 16) ||
                       (thread_m == 256 && thread_k == 64);
  if (!tile_ok || !(group_blocks == -1 || group_blocks == 4)) return MARLIN_HIP_ERR_KERN_SHAPE;
  return MARLIN_HIP_OK;
}

int run(int vf, int mf, const void* A, const void* B, const void* meta, void* C, void* s, int prob_m,
        int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream, int thread_k, int thread_m,
        int sms) {
  int err = validate(prob_m, prob_n, prob_k, groupsize, thread_k, thread_m);
  if (err != MARLIN_HIP_OK) return err;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return MARLIN_HIP_OK;
  // The 64-column chunk and 32-deep k-block of the packed layouts (and 128-deep
  // scale groups) are this implementation's own granularity.
  if (prob_m % 64 != 0 || prob_k % 32 != 0 || (groupsize != -1 && prob_k % 128 != 0)) {
    set_error("marlin_hip: N must be a multiple of 64 and K of 32 (128 when grouped)");
    return MARLIN_HIP_ERR_PROB_SHAPE;
  }
  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) prev = -1;
  if (prev != dev && hipSetDevice(dev) != hipSuccess) {
    set_error("marlin_hip: hipSetDevice failed");
    return MARLIN_HIP_ERR_LAUNCH;
  }
  if (sms <= 0) {
    if (hipDeviceGetAttribute(&sms, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || sms <= 0)
      sms = 256;
  }
  const int M = prob_n, N = prob_m, K = prob_k;
  Plan plan = plan_for(M, N, K, sms);
  GemmArgs a;
  a.A = static_cast<const _Float16*>(A);
  a.B = B;
  a.meta = meta;
  a.s = static_cast<const _Float16*>(s);
  a.C = static_cast<_Float16*>(C);
  a.M = M;
  a.N = N;
  a.K = K;
  a.splits = plan.splits;
  a.partial = nullptr;
  a.counters = nullptr;
  a.tag = 0;
  const int chunks = N / 64;
  if (plan.splits > 1) {
    if ((size_t)chunks * plan.ztiles * sizeof(int) > kCounterBytes) {
      plan.splits = 1;
      a.splits = 1;
    } else {
      err = get_scratch(dev, stream, (size_t)plan.splits * M * N * sizeof(float), &a.counters, &a.partial,
                        &a.tag);
      if (err != MARLIN_HIP_OK) {
        if (prev >= 0 && prev != dev) (void)hipSetDevice(prev);
        return err;
      }
    }
  }
  dim3 grid(chunks, plan.splits, plan.ztiles);
  const bool grouped = groupsize != -1;
  hipError_t e;
  if (vf == VAL4 && mf == META4) e = launch_v<VAL4, META4>(a, plan.bb, grouped, grid, stream);
  else if (vf == VAL4) e = launch_v<VAL4, META3>(a, plan.bb, grouped, grid, stream);
  else e = launch_v<VAL3, META4>(a, plan.bb, grouped, grid, stream);
  if (prev >= 0 && prev != dev) (void)hipSetDevice(prev);
  if (e != hipSuccess) {
    set_error(std::string("marlin_hip: kernel launch failed: ") + hipGetErrorString(e));
    return MARLIN_HIP_ERR_LAUNCH;
  }
  return MARLIN_HIP_OK;
}

}  // namespace sm24

extern "C" {

int marlin_hip_mul_2_4(const void* A, const void* B, const void* meta, void* C, void* s, int prob_m,
                       int prob_n, int prob_k, void* workspace, int groupsize, int dev, hipStream_t stream,
                       int thread_k, int thread_m, int sms, int max_par) {
  (void)workspace;
  (void)max_par;
  return sm24::run(sm24::VAL4, sm24::META4, A, B, meta, C, s, prob_m, prob_n, prob_k, groupsize, dev, stream,
                   thread_k, thread_m, sms);
}

int marlin_hip_mul_2_4_meta3(const void* A, const void* B, const void* meta3, void* C, void* s, int prob_m,
                             int prob_n, int prob_k, void* workspace, int groupsize, int dev,
                             hipStream_t stream, int thread_k, int thread_m, int sms, int max_par) {
  (void)workspace;
  (void)max_par;
  return sm24::run(sm24::VAL4, sm24::META3, A, B, meta3, C, s, prob_m, prob_n, prob_k, groupsize, dev, stream,
                   thread_k, thread_m, sms);
}

int marlin_hip_mul_2_4_w3(const void* A, const void* B3, const void* meta, void* C, void* s, int prob_m,
                          int prob_n, int prob_k, void* workspace, int groupsize, int dev, hipStream_t stream,
                          int thread_k, int thread_m, int sms, int max_par) {
  (void)workspace;
  (void)max_par;
  return sm24::run(sm24::VAL3, sm24::META4, A, B3, meta, C, s, prob_m, prob_n, prob_k, groupsize, dev, stream,
                   thread_k, thread_m, sms);
}

const char* marlin_hip_last_error(void) { return sm24::g_last_error.c_str(); }

}  // extern "C"
