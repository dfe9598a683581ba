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
#include <stdlib.h>
#include <string.h>

#include <initializer_list>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "sm24_device.h"
#include "sm24_decode.h"
#include "sm24_host.h"
#include "sm24_native.h"
#include "../../include/marlin_hip.h"
#include "../../include/marlin_spans.h"

namespace sm24 {

// Raw operands of one k-block for one lane, as loaded (decoding happens at use, so
// that a deep ring of these stays in flight).
template <int BB, int VF, int MF>
struct Frag {
  u32x2 w;              // packed words j = 2*jb, 2*jb+1 (VAL3: the 8 bytes holding them)
  u32x4 m0;             // META4: units 16jb+2g, +1; META3: code words X
  u32x4 m1;             // META3 only: code words Y
  half4_t sc;           // grouped scales {s(jj0,b0), s(jj0,b1), s(jj1,b0), s(jj1,b1)}
  half8_t act[BB];      // activation B operands
};

template <int BB, int NW, bool GROUPED, int VF, int MF>
__global__ __launch_bounds__(64 * NW) void sm24_gemm_kernel(GemmArgs a) {
  constexpr int NT = 64 * NW;  // threads per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
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

  auto fetch = [&](int r, bool live, Frag<BB, VF, MF>& f) {
    if constexpr (VF == VAL4) {
      f.w = *reinterpret_cast<const u32x2*>(bw + (size_t)r * (2 * (size_t)N));
    } else {
      f.w = *reinterpret_cast<const u32x2_a4*>(b3 + (size_t)r * (6 * (size_t)N));
    }
    if constexpr (MF == META4) {
      f.m0 = *reinterpret_cast<const u32x4*>(mw + (size_t)r * N);
    } else {
      const uint32_t* base = m3 + (size_t)r * (size_t)(3 * N / 4);
      f.m0 = *reinterpret_cast<const u32x4*>(base);
      f.m1 = *reinterpret_cast<const u32x4*>(base + 16);
    }
    if constexpr (GROUPED) {
      f.sc = *reinterpret_cast<const half4_t*>(sp + (size_t)(r >> 2) * N);
    }
#pragma unroll
    for (int bb = 0; bb < BB; bb++) {
      // Rows past M (and slots past the range, live == false) read zeros from a
      // small zero-filled buffer: the load is unconditional, only its address is
      // selected, so the ring keeps a fixed shape.
      const int m = row0 + 16 * bb;
      const _Float16* ap =
          (live && m < M) ? a.A + (size_t)m * K + 32 * r + 4 * h : a.zeros;
      const u32x2 lo = *reinterpret_cast<const u32x2*>(ap);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(ap + 16);
      f.act[bb] = __builtin_bit_cast(half8_t, (u32x4){lo.x, lo.y, hi.x, hi.y});
    }
  };

  float4_t acc[BB][4];
#pragma unroll
  for (int bb = 0; bb < BB; bb++)
#pragma unroll
    for (int t = 0; t < 4; t++) acc[bb][t] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Frag<BB, VF, MF>& f) {
    uint32_t w0, w1, idx;
    if constexpr (VF == VAL4) {
      w0 = f.w.x;
      w1 = f.w.y;
    } else {
      const uint64_t v = ((uint64_t)f.w.y << 32 | f.w.x) >> (16 * jb);
      w0 = spread3((uint32_t)v & 0xFFFFFFu);
      w1 = spread3((uint32_t)(v >> 24) & 0xFFFFFFu);
    }
    if constexpr (MF == META4) {
      idx = idx_pair(f.m0.x, f.m0.y, sh) | (idx_pair(f.m0.z, f.m0.w, sh) << 8);
    } else {
      // 48-word group for (k-block, chunk): words 0..15 / 16..31 / 32..47 hold the
      // 48-bit "first" and "second" code pairs of the 64 metadata words.
      const uint32_t lut = jb ? kLutLow : kLutHigh;
      uint32_t xs[4];
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t X = f.m0[v], Y = f.m1[v];
        uint32_t c24;
        if ((g >> 2) == 0) {
          c24 = jb ? ((X >> 24) | ((Y & 0xFFFFu) << 8)) : (X & 0xFFFFFFu);
        } else {
          c24 = jb ? ((Y >> 8) & 0xFFFFFFu) : (((X >> 16) | (Y << 16)) & 0xFFFFFFu);
        }
        const uint32_t ca = (c24 >> (3 * h)) & 7u;
        const uint32_t cb = (c24 >> (3 * h + 12)) & 7u;
        xs[v] = ((lut >> (4 * ca)) & 15u) | (((lut >> (4 * cb)) & 15u) << 16);
      }
      idx = (xs[0] | (xs[1] << 4)) | ((xs[2] | (xs[3] << 4)) << 8);
    }
    half4_t a00, a01, a10, a11;  // (jj, blk)
    if constexpr (VF == VAL4) {
      a00 = dequant4(w0);
      a01 = dequant4(w0 >> 8);
      a10 = dequant4(w1);
      a11 = dequant4(w1 >> 8);
    } else {
      a00 = dequant3(w0);
      a01 = dequant3(w0 >> 8);
      a10 = dequant3(w1);
      a11 = dequant3(w1 >> 8);
    }
    if constexpr (GROUPED) {
      a00 = scale4(a00, f.sc.x);
      a01 = scale4(a01, f.sc.y);
      a10 = scale4(a10, f.sc.z);
      a11 = scale4(a11, f.sc.w);
    }
#pragma unroll
    for (int bb = 0; bb < BB; bb++) {
      acc[bb][0] = smfmac32<0>(a00, f.act[bb], acc[bb][0], idx);
      acc[bb][1] = smfmac32<1>(a10, f.act[bb], acc[bb][1], idx);
      acc[bb][2] = smfmac32<2>(a01, f.act[bb], acc[bb][2], idx);
      acc[bb][3] = smfmac32<3>(a11, f.act[bb], acc[bb][3], idx);
    }
  };

  // Each wave streams a contiguous quarter of the split's k-blocks through a ring of
  // U in-flight fragments: the load of k-block r+U is issued as soon as k-block r
  // has been consumed, so U k-blocks per wave are always on their way from HBM.
  // Slots past the end re-read the last k-block (a cache hit) with zero activations.
  constexpr int U = BB == 1 ? 8 : (BB == 2 ? 6 : 4);
  const int span = kb1 - kb0;
  const int r0 = kb0 + (int)(((long long)span * wave) / NW);
  const int r1 = kb0 + (int)(((long long)span * (wave + 1)) / NW);
  if (r1 > r0) {
    const int rlast = r1 - 1;
    Frag<BB, VF, MF> ring[U];
#pragma unroll
    for (int i = 0; i < U; i++) {  // prologue, issued in slot order
      fetch(r0 + i < r1 ? r0 + i : rlast, r0 + i < r1, ring[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int base = r0; base < r1; base += U) {
#pragma unroll
      for (int i = 0; i < U; i++) {
        // Scheduling barriers keep the decode of a fragment at its use: left free, the
        // scheduler pulls it up next to the load issued one ring-turn earlier and
        // the wave stalls on that load.
        compute(ring[i]);
        __builtin_amdgcn_sched_barrier(0);
        const int rn = base + i + U;
        fetch(rn < r1 ? rn : rlast, rn < r1, ring[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ---- reduce the NW waves in LDS: red[wave][row][col], col = n within chunk ----
  constexpr int RS = 65;  // padded row stride (floats)
  __shared__ float red[NW][16 * BB][RS];
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
    for (int e = threadIdx.x; e < ntile; e += NT) {
      const int ml = e >> 6, nl = e & 63;
      const int m = 16 * BB * bt + ml;
      if (m >= M) continue;
      float v = red[0][ml][nl];
#pragma unroll
      for (int w = 1; w < NW; w++) v += red[w][ml][nl];
      _Float16 o = (_Float16)v;
      if constexpr (!GROUPED) o = o * a.s[ncol0 + nl];
      a.C[(size_t)m * N + ncol0 + nl] = o;
    }
    return;
  }

  // Split-K hand-off.  The scratch lives in uncached device memory and every access
  // to it is a device-scope atomic, so partials and counters meet at the
  // device-coherent point without any L2-wide write-back or invalidate (which an
  // agent-scope fence would issue on every XCD).  Ordering: each thread waits for
  // its own partial stores to complete before the workgroup barrier; the counter is
  // bumped only after that barrier.
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
  // Arrival counter of this (chunk, batch tile); the last of the splits to arrive
  // reduces and resets it.  A single fetch-add per workgroup: no retry loop.
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
    if constexpr (!GROUPED) o = o * a.s[ncol0 + nl];
    a.C[(size_t)m * N + ncol0 + nl] = o;
  }
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string g_last_error;

// Buffer for the decode kernel's per-wave phase timestamps (marlin_hip_set_spans;
// recorded only by the measurement build).
uint64_t* g_spans = nullptr;

void set_error(const std::string& msg) { g_last_error = msg; }

struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};

// Split-K scratch (arrival counters + fp32 partials) and operand staging buffers,
// one per (device, stream): calls on different streams never share one, so they may
// overlap in time (the reference gets the same safety from one workspace per layer).
// Calls on one stream are ordered, so they may share theirs.  Buffers are never
// freed: a captured graph may still refer to an old one.
using StreamKey = std::pair<int, hipStream_t>;
std::mutex g_scratch_mu;
std::map<StreamKey, Scratch> g_scratch;
std::map<int, void*> g_zeros;

bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// The library's static device scratch: the zero block that the decode and general
// kernels read in place of activation rows that do not exist (rows past M, k-blocks
// past K).  Every device holds its own copy from module load until the process ends;
// no kernel writes it, so calls on any stream may share it.  It is all the scratch
// that marlin_hip_mul_2_4_noalloc needs, because that entry point never splits K.
constexpr size_t kScratchBytes = 256;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

__global__ void fill_zero_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of `scratch` on `dev` (the caller has made `dev` current).  Looked up
// once per device with hipGetSymbolAddress; the array's name itself is only a host
// stand-in.  The first lookup also clears the block with a fill kernel on `stream`
// (it is zero from module load; the fill is a guard that costs one launch per device
// and process), unless `stream` is being captured: a fill recorded into the caller's
// graph would run on every replay, and the block is already zero.
int get_zeros(int dev, hipStream_t stream, const _Float16** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void*& z = g_zeros[dev];
  if (!z) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error(std::string("marlin_hip: hipGetSymbolAddress of the static scratch failed: ") +
                hipGetErrorString(e));
      return MARLIN_HIP_ERR_LAUNCH;
    }
    if (!capturing(stream)) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(64), 0, stream, static_cast<uint32_t*>(p),
                         (int)(kScratchBytes / 4));
      const hipError_t le = hipGetLastError();
      if (le != hipSuccess) {
        set_error(std::string("marlin_hip: clearing the static scratch failed: ") + hipGetErrorString(le));
        return MARLIN_HIP_ERR_LAUNCH;
      }
    }
    z = p;
  }
  *out = static_cast<const _Float16*>(z);
  return MARLIN_HIP_OK;
}


// The split-K scratch of (dev, stream), grown to hold `partial_bytes` of partials.
// A buffer cannot be allocated while the stream is being captured into a graph: then,
// if the stream's scratch is too small, *counters and *partial come back null and
// the caller runs the call without splitting K (same result, one workgroup per tile;
// an eager call of the same shape on the capturing stream before the capture
// avoids that).
int get_scratch(int dev, hipStream_t stream, size_t partial_bytes, uint32_t** counters, float** partial) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_scratch[StreamKey(dev, stream)];
  const size_t need = kCounterBytes + partial_bytes;
  if (s.bytes < need) {
    if (capturing(stream)) {
      *counters = nullptr;
      *partial = nullptr;
      return MARLIN_HIP_OK;
    }
    size_t nb = need > 2 * s.bytes ? need : 2 * s.bytes;
    void* p = nullptr;
    // Uncached: split-K partials and counters are exchanged between workgroups that
    // run on different XCDs, whose L2 caches are not coherent with each other.
    // Never freed (see above), as uncached memory must not be recycled once read.
    hipError_t e = hipExtMallocWithFlags(&p, nb, hipDeviceMallocUncached);
    if (e != hipSuccess) {
      set_error(std::string("marlin_hip: uncached allocation of scratch failed: ") + hipGetErrorString(e));
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
  *counters = static_cast<uint32_t*>(s.ptr);
  *partial = reinterpret_cast<float*>(static_cast<char*>(s.ptr) + kCounterBytes);
  return MARLIN_HIP_OK;
}

// Staging buffer for operands expanded to the large-M kernel's 4-bit formats (3-bit
// values, 3-bit metadata, the lane-native layout above 16 rows), one per (device,
// stream).  Ordinary device memory (written and read by kernels of the same stream);
// grows, never freed.
std::map<StreamKey, Scratch> g_stage;

int get_stage(int dev, hipStream_t stream, size_t bytes, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_stage[StreamKey(dev, stream)];
  if (s.bytes < bytes) {
    if (capturing(stream)) {
      set_error("marlin_hip: the operand staging buffer of this stream would have to grow during stream "
                "capture; make one call of the same (or a larger) shape on the capturing stream before "
                "capturing");
      return MARLIN_HIP_ERR_LAUNCH;
    }
    const size_t nb = bytes > 2 * s.bytes ? bytes : 2 * s.bytes;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, nb);
    if (e != hipSuccess) {
      set_error(std::string("marlin_hip: allocation of the staging buffer failed: ") + hipGetErrorString(e));
      return MARLIN_HIP_ERR_LAUNCH;
    }
    s.ptr = p;
    s.bytes = nb;
  }
  *out = s.ptr;
  return MARLIN_HIP_OK;
}

// 3-bit value codes -> the 4-bit packed layout: 4-bit word w is the 24-bit field at
// bit 24w of the 3-bit stream, each code spread to a nibble and offset by 4 (zero
// point 4 -> 8), so (nibble - 8) * s equals (code - 4) * s.  One thread per 4 words
// (12 bytes in, 16 out).
__global__ __launch_bounds__(256) void w3_to_w4_kernel(const uint32_t* __restrict__ in, u32x4* __restrict__ out,
                                                       long long quads) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= quads) return;
  const uint32_t a0 = in[3 * i], a1 = in[3 * i + 1], a2 = in[3 * i + 2];
  u32x4 o;
  o.x = spread3(a0 & 0xFFFFFFu) + 0x44444444u;
  o.y = spread3(__builtin_amdgcn_alignbit(a1, a0, 24) & 0xFFFFFFu) + 0x44444444u;
  o.z = spread3(__builtin_amdgcn_alignbit(a2, a1, 16) & 0xFFFFFFu) + 0x44444444u;
  o.w = spread3(a2 >> 8) + 0x44444444u;
  out[i] = o;
}

// Tile height and K splits of the large-M kernel.  Its workgroups run one per CU, and
// the chip is power-limited at full occupancy: a 128-row k-step takes ~0.61 us with 64
// workgroups busy and ~1.03 us with all 256 CUs busy (MI355X, Llama-2-70B prefill
// shapes).  So a problem with few tiles runs on 64-row tiles (twice the tiles, each
// k-step 0.63 of a 128-row one at the same occupancy: half the MFMAs at twice the
// dequantization per MFMA) or split along K when K is long enough to pay for the
// hand-off: each split stores its fp32 partial (512 x rows floats) to uncached scratch
// and the last one reads them all back, ~5 TB/s for that exchange.  The estimate sums
// the rounds of workgroups over the CUs, each at the k-step time of its occupancy,
// plus the exchange; it reproduces the measured times of every prefill-sweep call to
// within ~5 % for both heights and 1-2 splits (forced by MARLIN_HIP_PREFILL_ROWS and
// MARLIN_HIP_PREFILL_SPLITS, read once).  `nosplit`: one split only.
// k-step of the narrow tile (4 waves, half the MFMAs of a 512x128 tile's k-step,
// one wave per SIMD) relative to a 512x128 tile's at the same occupancy, as the
// planner's model has it when the narrow tile is forced (fitted to forced plans of
// Llama-2-70B qkv and o at M = 512 and 1024, one box: 0.61-0.71, the higher at low
// occupancy).
constexpr double kPreNarrowStep = 0.66;
struct PrefillPlan {
  int rows;    // batch rows per tile: 128 or 64
  int splits;  // K splits
  int tiles;   // tiles (workgroups per split)
  int chunks;  // 64-column chunks per tile (= waves): 8, or 4 for the narrow 128-row tile
};
// k-step time (us) of a 128-row tile with a fraction x of the CUs busy (measured).
double prefill_step_us(double x) {
  static const double xs[] = {0.0, 0.25, 0.3125, 0.5, 0.625, 1.0};
  static const double us[] = {0.55, 0.61, 0.62, 0.70, 0.78, 1.03};
  if (x >= 1.0) return us[5];
  int i = 0;
  while (x > xs[i + 1]) i++;
  return us[i] + (us[i + 1] - us[i]) * (x - xs[i]) / (xs[i + 1] - xs[i]);
}
PrefillPlan prefill_plan(int M, int N, int K, int cus, bool nosplit) {
  static const int forced = [] {
    const char* e = getenv("MARLIN_HIP_PREFILL_SPLITS");
    const int x = e ? atoi(e) : 0;
    return x >= 1 && x <= 16 ? x : 0;
  }();
  static const int forced_rows = env_choice("MARLIN_HIP_PREFILL_ROWS", {64, 128}, 0);
  static const int forced_chunks = env_choice("MARLIN_HIP_PREFILL_CHUNKS", {kPreNarrowChunks, kPreChunks}, 0);
  const int nks = K / 64;
  const int max_s = nosplit ? 1 : (nks / 8 > 0 ? nks / 8 : 1);  // at least eight k-steps per split
  if (cus < 1) cus = 1;
  const double exchange_bytes_per_us = 5.0e6;
  PrefillPlan best{128, 1, (N / kPreTileCols) * ((M + 127) / 128), kPreChunks};
  double best_cost = 1e30;
  // Candidates: 512-column tiles of 128 or 64 rows (the narrow tile, 256 columns x
  // 128 rows of 4 waves, only when forced).  A k-step of a 64-row or narrow tile is
  // a fraction `hscale` of a 512x128 one at the same occupancy.
  struct Cand {
    int rows, chunks;
    double hscale;
  };
  const Cand cands[] = {{128, kPreChunks, 1.0}, {64, kPreChunks, 0.63}, {128, kPreNarrowChunks, kPreNarrowStep}};
  for (const Cand& c : cands) {
    if ((c.chunks == kPreNarrowChunks) != (forced_chunks == kPreNarrowChunks)) continue;
    if (forced_rows && c.rows != forced_rows) continue;
    if (forced_chunks && c.chunks != forced_chunks) continue;
    const int tiles = (N / (64 * c.chunks)) * ((M + c.rows - 1) / c.rows);
    if (forced && !nosplit) return PrefillPlan{c.rows, forced < max_s ? forced : max_s, tiles, c.chunks};
    for (int s = 1; s <= 8 && s <= max_s; s++) {
      const long long wgs = (long long)tiles * s, full = wgs / cus, tail = wgs - full * cus;
      double cost = ((double)full * prefill_step_us(1.0) + (tail ? prefill_step_us((double)tail / cus) : 0.0)) *
                    c.hscale * nks / s;
      if (s > 1) cost += 2.0 * tiles * s * (double)pre_split_bytes(c.rows, c.chunks) / exchange_bytes_per_us;
      if (cost < 0.98 * best_cost) {
        best_cost = cost;
        best = PrefillPlan{c.rows, s, tiles, c.chunks};
      }
    }
  }
  // A 64-row plan runs narrow tiles instead where they come to the same count (a
  // multiple of 128 rows, or the same ragged rounding): the same workgroups, MFMAs and
  // splits, but every dequantized weight fragment feeds four B fragments instead of
  // two.  Forced plans of Llama-2-70B (one box): qkv at M = 512 on 160 workgroups
  // 73.2 -> 66.1 us, o at M = 1024 on 256 89.0 -> 83.2, o at M = 512 in two splits
  // 58.5 -> 53.7.  MARLIN_HIP_PREFILL_CHUNKS = 8 keeps the 64-row tiles.
  if (best.rows == 64 && best.chunks == kPreChunks && forced_chunks != kPreChunks) {
    const int narrow = (N / (64 * kPreNarrowChunks)) * ((M + 127) / 128);
    if (narrow == best.tiles) best = PrefillPlan{128, best.splits, narrow, kPreNarrowChunks};
  }
  return best;
}

// A split plan needs one arrival counter per tile (at most 64-row tiles: the most).
bool prefill_counters_exceed(int N, int M) {
  return (size_t)(N / kPreTileCols) * ((M + 63) / 64) * sizeof(uint32_t) > kCounterBytes;
}

struct Plan {
  int bb;
  int splits;
  int ztiles;
};

// Workgroups per compute unit the planner aims for (MARLIN_HIP_WGS_PER_CU overrides;
// read once).
int wgs_per_cu() {
  static const int v = [] {
    const char* e = getenv("MARLIN_HIP_WGS_PER_CU");
    int x = e ? atoi(e) : 0;
    return x > 0 && x <= 64 ? x : 2;
  }();
  return v;
}

Plan plan_for(int M, int N, int K, int cus) {
  Plan p;
  p.bb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.ztiles = (M + 16 * p.bb - 1) / (16 * p.bb);
  const int chunks = N / 64;
  const int nkb = K / 32;
  const long long tiles = (long long)chunks * p.ztiles;
  const long long target = (long long)wgs_per_cu() * cus;
  int splits = (int)((target + tiles - 1) / tiles);
  const int max_splits = nkb / 8 > 0 ? nkb / 8 : 1;  // at least two k-blocks per wave
  if (splits > max_splits) splits = max_splits;
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  p.splits = splits;
  return p;
}

template <int BB, bool GROUPED, int VF, int MF>
hipError_t launch_t(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int NW = BB == 1 ? 8 : 4;  // waves per workgroup (LDS reduction buffer < 64 KiB)
  hipLaunchKernelGGL((sm24_gemm_kernel<BB, NW, GROUPED, VF, MF>), grid, dim3(64 * NW), 0, stream, a);
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

// Integer knob from the environment, read once per call site; `fallback` when unset
// or not one of `allowed`.
int env_choice(const char* name, std::initializer_list<int> allowed, int fallback) {
  const char* e = getenv(name);
  if (!e) return fallback;
  const int x = atoi(e);
  for (int v : allowed)
    if (v == x) return x;
  return fallback;
}

// Column-tile width, waves per workgroup and K splits of the decode kernel, from
// measured single-call times on MI355X (Llama-2-7B and -70B shapes, M in {1, 2, 4, 8,
// 16, 24, 32}, every forced choice of TC in {16, 32, 64}, NW in {4, 8} and splits in
// {1, 2, 4}, on one box).  Narrow N (fewer than CUs/2 64-column chunks) takes
// 16-column tiles for enough workgroups, until M grows: every tile re-reads all M
// activation rows over K, so from M = 5 (long K) or M > 16 64-column tiles split
// four ways along K keep the workgroup count while cutting that traffic (down
// 11008x4096 at M = 8: 9.13 -> 8.84 us; o 4096x4096 at M = 32: 8.46 -> 7.83 us).
// Wider N takes 64-column tiles from M = 8, below that 32-column tiles when N/32 is at
// least twice the CU count, else 16.  A split costs a hand-off through the uncached
// scratch (>= 2.5 us), so it is used only where measured to pay.  Long K (>= 8192):
// the widest N (Llama-2-70B gate_up) runs unsplit up to 8 rows (M = 4: 41.5 -> 38.5
// us against two splits) and splits in two beyond; N <= 10240 (qkv, down) splits K
// four ways (down at M = 1 two ways: 20.3 -> 19.4 us); Llama-2-70B o (N/16 = 2 per
// CU) keeps 32-column tiles unsplit up to M = 8 (8.55 -> 7.47 us at M = 1).  The 7B
// sweep (M in {1, 2, 4, 8, 16}) is within noise of the best forced choice per call.
// MARLIN_HIP_DECODE_TC / _WAVES / _SPLITS / _DEEP override.

bool decode_deep(int K, int splits);

// Whether ntiles 16-column tiles can run three to a workgroup of 12 waves: a multiple
// of 8 XCDs x 4 tiles per 64-column chunk x 3, in at most one workgroup per CU.
// MARLIN_HIP_DECODE_G = 1 keeps one tile per workgroup.
bool decode_g3_fits(int ntiles, int cus) {
  static const int forced_g = env_choice("MARLIN_HIP_DECODE_G", {1, 3}, 3);
  return forced_g == 3 && ntiles % 96 == 0 && cus > 0 && ntiles / 3 <= cus;
}

DecodeShape decode_shape(int M, int N, int K, int cus) {
  static const int forced_tc = env_choice("MARLIN_HIP_DECODE_TC", {16, 32, 64}, 0);
  static const int forced_nw = env_choice("MARLIN_HIP_DECODE_WAVES", {4, 8}, 0);
  static const int forced_splits = env_choice("MARLIN_HIP_DECODE_SPLITS", {1, 2, 3, 4}, 0);
  DecodeShape d;
  const bool wide32 = N / 32 >= 2 * cus;
  const bool narrow = 2 * (N / 64) < cus;
  const bool longk = K >= 8192;
  // 5-8 rows: the 8-row batch (activations through LDS, as for 2-4 rows) where it
  // measured faster than the 16-row one (M = 5 / 8, weights cold in HBM, one box:
  // 7B o 4096x4096 5.22 / 5.23 -> 4.94 / 5.09 us with 16-column tiles of 8 waves;
  // 7B gate_up 4096x22016 at M = 5 12.32 -> 11.45, but at M = 8 12.38 against 13.01,
  // so up to 6 rows; 70B gate_up 8192x57344 38.1 / 39.6 -> 36.1 / 37.6; 70B qkv
  // 8192x10240 11.7 / 12.3 -> 10.8 / 11.8).  The 16-row batch keeps 7B down and the
  // 70B o and down shapes, and takes 64-column tiles of 8 waves for 7B qkv
  // 4096x12288 (M = 5: 9.74 -> 7.56 us).
  const bool mid = M >= 5 && M <= 8 && decode_batch(8) == 8;
  if (mid && narrow && !longk && N / 16 >= cus) {
    d = {16, 8, 1};
    d.mb = 8;
  } else if (mid && wide32 && (longk || M <= 6)) {
    d = {longk ? 64 : 32, 4, 1};
    d.mb = 8;
  } else if (mid && longk && !wide32 && K < 16384 && N / 16 > 2 * cus) {
    d = {32, 8, 1};
    d.mb = 8;
  } else if (mid && !longk && !narrow && !wide32) {
    d = {64, 8, 1};
    d.mb = 16;
  } else if (narrow) {
    if (M > 16) d = {64, 4, 4};
    else if (longk && M > 4) d = {64, 8, 4};
    // 8 waves at 2-4 rows and for long K; 4 waves at one row and K < 8192 (7B o
    // 4096x4096 at M = 1: 4.15 -> 4.05 us, forced, one box, two runs each; at M = 2
    // 4.23 against 4.29, and 7B down at M = 1 6.23 against 6.99, stay on 8)
    else d = {16, (M <= 4 && (M > 1 || longk)) ? 8 : 4, 1};
  } else if (longk) {
    // long K at wide N (the Llama-2-70B shapes): unsplit tiles where N alone fills the
    // CUs (the widest N up to 8 rows), K splits of 64-column tiles otherwise; 32-column
    // tiles for few rows where N/16 fills one round of two per CU.  From forced choices
    // of TC x NW x S on the four Llama-2-70B shapes at M in {1, 2, 4, 8, 16} (one box):
    // down 28672x8192 at 2-4 rows two splits of 8-wave tiles (M = 2: 21.9 -> 19.9 us,
    // M = 4: 21.7 -> 20.5), at 5-8 rows four splits of 4-wave tiles (M = 8: 22.0 ->
    // 21.2); qkv 8192x10240 at 1-4 rows 32-column tiles (4 waves at M = 1, 8 above)
    // with the tail split (M = 1: 10.2 -> 10.1, M = 2: 10.9 -> 10.2, M = 4: 11.4 ->
    // 10.5); at 9-16 rows down two splits of
    // 8-wave tiles (24.5 -> 24.1), o 8192x8192 one round of 32-column tiles (9.75 ->
    // 9.25), qkv unsplit 8-wave 64-column tiles (13.5 -> 12.9).
    if (wide32) {
      if (M == 1) d = {32, 8, 1};
      else if (M <= 8) d = {64, M <= 4 ? 4 : 8, 1};
      else d = {64, 4, 2};
    } else if (M > 16) {
      d = {64, 4, 4};
    } else if (M > 8) {
      if (K >= 16384) d = {64, 8, 2};
      else if (cus > 0 && (N / 32) % cus == 0) d = {32, 8, 1};
      else d = {64, 8, 1};
    } else if (K >= 16384) {
      d = M <= 4 ? DecodeShape{64, 8, 2} : DecodeShape{64, 4, 4};
    } else if (N / 16 <= 2 * cus) {
      d = {32, 8, 1};
    } else {
      d = M == 1 ? DecodeShape{32, 4, 1} : M <= 4 ? DecodeShape{32, 8, 1} : DecodeShape{64, 4, 4};
    }
  } else if (M > 16) {
    d = {64, 4, N / 64 >= cus ? 2 : 1};
  } else if (M >= 8) {
    d = {64, wide32 ? 4 : 8, 1};
  } else if (wide32) {
    d = {32, 4, 1};
  } else {
    // 3-4 rows (the padded batch of 4) on 64-column tiles of 8 waves, as 5-8 rows,
    // where those tiles fill three quarters of the CUs: 7B qkv 4096x12288 at M = 4
    // 7.47 / 7.39 -> 7.14 us (forced sweep, one box); at 1-2 rows the 16-column tiles
    // stay faster (M = 2: 6.83 against 7.09 us).  Where the 16-column tiles run three
    // to a workgroup (below) they are faster at 3-4 rows too: 7B qkv at M = 4 6.89 ->
    // 6.55 us (A/B, same box, two runs each).
    d = M >= 3 && 4 * (N / 64) >= 3 * cus && !decode_g3_fits(N / 16, cus) ? DecodeShape{64, 8, 1}
                                                                         : DecodeShape{16, 4, 1};
  }
  if (mid && d.mb == 0) d.mb = 16;  // the rest keep the 16-row batch
  if (forced_tc) d.tc = forced_tc;
  if (forced_nw) d.nw = forced_nw;
  if (forced_splits) d.splits = forced_splits;
  // at most one split per stage, and a counter per column tile
  const int kpw = 64 / d.tc > 2 ? 64 / d.tc : 2;
  const int nst = (K / 32 + d.nw * kpw - 1) / (d.nw * kpw);
  if (d.splits > nst) d.splits = nst;
  // Tail split: with q whole rounds of tiles over the CUs and a tail of f <= CUs/2
  // tiles left over, the tail tiles are split S = min(4, CUs/f) ways, so that every
  // CU runs q whole tiles plus at most one piece instead of q + 1 whole tiles on f of
  // them (the pieces' hand-off overlaps the whole tiles).  7B gate_up 4096x22016 at
  // M = 8 and 16 (344 tiles on 256 CUs): 12.0 -> 11.0 and 13.7 -> 12.5 us; three
  // ways (264 pieces, more than the CUs) 13.0 and 13.7.  MARLIN_HIP_DECODE_TAIL
  // forces S (0: off).
  static const int forced_tail = env_choice("MARLIN_HIP_DECODE_TAIL", {0, 2, 3, 4}, -1);
  const int ntiles = N / d.tc;
  // A two-way split of every tile where the tiles leave such a tail: the tail split
  // alone balances the CUs with fewer hand-offs (Llama-2-70B gate_up at M = 16 / 32:
  // 49.3 -> 48.5 and 67.6 -> 65.2 us; 7B gate_up at M = 32: 18.6 -> 17.9 us).
  if (!forced_splits && forced_tail != 0 && d.splits == 2 && cus > 0 && ntiles > cus) {
    const int f = ntiles % cus;
    if (f > 0 && 2 * f <= cus) d.splits = 1;
  }
  if (d.splits == 1 && forced_tail != 0 && cus > 0 && ntiles > cus) {
    const int q = ntiles / cus, f = ntiles - q * cus;
    int st = forced_tail > 0 ? forced_tail : (2 * f <= cus && f > 0 ? cus / f : 1);
    if (st > 4) st = 4;
    if (st > nst) st = nst;
    if (st > 1 && f > 0) {
      d.tail_from = q * cus;
      d.splits = st;
    }
  }
  if ((size_t)ntiles * sizeof(uint32_t) > kCounterBytes) {
    d.splits = 1;
    d.tail_from = 0;
  }
  d.deep = decode_deep(K, d.tail_from > 0 ? 1 : d.splits);
  d.cus = cus;
  // Three 16-column tiles per workgroup of 12 waves where that makes one workgroup per
  // CU (unsplit, up to 4 rows, the tiles a multiple of 8 XCDs x 4 tiles per chunk x 3):
  // the workgroup copies its resident activation rows once instead of three times,
  // and no workgroup's copy queues behind another's weight stream on the CU.
  // MARLIN_HIP_DECODE_G = 1 keeps one tile per workgroup.
  if (d.tc == 16 && d.nw == 4 && d.splits == 1 && d.tail_from == 0 && !d.deep && decode_batch(M) <= 4 &&
      (d.mb == 0 || d.mb <= 4) && decode_g3_fits(ntiles, cus))
    d.g = 3;
  return d;
}

// Workgroups of a decode launch.
int decode_workgroups(int N, const DecodeShape& d) {
  const int ntiles = N / d.tc;
  if (d.g > 1) return ntiles / d.g;
  return d.tail_from > 0 ? d.tail_from + (ntiles - d.tail_from) * d.splits : ntiles * d.splits;
}

// Register ring depth: shallow (16 VGPRs: more resident workgroups) up to 16384 k per
// split, measured equal or faster at every Llama-2-7B and -70B decode call of the
// planner (K per split up to 11008: 7B down at M <= 4 runs 0.55-0.8 us faster than
// deep); deep (more stages in flight per wave) beyond.  MARLIN_HIP_DECODE_DEEP
// overrides.
bool decode_deep(int K, int splits) {
  static const int forced_deep = env_choice("MARLIN_HIP_DECODE_DEEP", {0, 1}, -1);
  return forced_deep >= 0 ? forced_deep == 1 : K / splits > 16384;
}

// The same decode shape without a K split (no split-K scratch available or wanted).
void decode_unsplit(DecodeShape& d, int K) {
  d.splits = 1;
  d.tail_from = 0;
  d.deep = decode_deep(K, 1);
}

// Padded batch of the decode kernel: 1, 4, 8 (activations staged through LDS), 16 or
// 32 (loaded straight into the MFMA operands: one or two 16-row blocks).  The tile
// table may raise 8 to 16 per shape.  MARLIN_HIP_DECODE_MB8=0 turns the 8-row batch
// off (read once).
int decode_batch(int M) {
  static const int mb8 = env_choice("MARLIN_HIP_DECODE_MB8", {0, 1}, 1);
  return M == 1 ? 1 : (M <= 4 ? 4 : (M <= 8 && mb8 ? 8 : (M <= 16 ? 16 : 32)));
}

hipError_t launch_decode(const GemmArgs& a, DecodeShape d, int vf, int mf, bool grouped, hipStream_t stream) {
  if (grouped) {
    if (d.tc == 64) return launch_decode_t<64, true>(a, d, vf, mf, stream);
    if (d.tc == 32) return launch_decode_t<32, true>(a, d, vf, mf, stream);
    return launch_decode_t<16, true>(a, d, vf, mf, stream);
  }
  if (d.tc == 64) return launch_decode_t<64, false>(a, d, vf, mf, stream);
  if (d.tc == 32) return launch_decode_t<32, false>(a, d, vf, mf, stream);
  return launch_decode_t<16, false>(a, d, vf, mf, stream);
}

// Large-M path (sm24_prefill_kernel): 4-bit values and metadata, N a multiple of its
// 512-column tile and K of its 64-deep k-step, from a batch threshold measured on
// MI355X against decode launches of <= 32 rows (Llama-2-7B and -70B shapes, M in
// 48..192, the planner's 64- or 128-row tiles): from M = 33 for the widest N (7B
// gate_up 4096x22016 at M = 48 / 64: 23.5 / 23.3 against 28.1 / 34.0 us) and for long
// K at N >= 10240 (70B qkv 8192x10240: 25.9 / 26.1 against 28.9 / 34.3 us); from
// M = 65 for N >= 4096 (M = 80 / 96: 7B qkv 23.0 / 22.8 against 28.4 / 31.7 us, 7B down
// 28.2 / 28.5 against 30.3 / 32.8, 70B o 27.9 / 27.5 against 36.1 / 39.7; at M = 48 /
// 64 the decode launches win for 7B o, down and qkv: 7B o 13.6 / 15.0 against 19.6 /
// 20.0 us); M >= 160 for narrower N.  MARLIN_HIP_PREFILL_MIN_M (>= 1) replaces the
// threshold.
int prefill_min_m(int N, int K) {
  // the widest N at long K already from 17 rows (70B gate_up 8192x57344 at M = 24 /
  // 32: 49.5 / 50.3 against 58.8 / 67.3 us; at M = 16 49.5 against 49.0)
  if (N >= 16384 && K >= 8192) return 17;
  if (N >= 16384 || (N >= 10240 && K >= 8192)) return kDecodeMaxM + 1;
  return N >= 4096 ? 65 : 160;
}
bool prefill_fits(int M, int N, int K, int vf, int mf) {
  static const int forced_min_m = [] {
    const char* e = getenv("MARLIN_HIP_PREFILL_MIN_M");
    const int x = e ? atoi(e) : 0;
    return x >= 1 ? x : 0;
  }();
  const int min_m = forced_min_m ? forced_min_m : prefill_min_m(N, K);
  return vf == VAL4 && mf == META4 && M >= min_m && N % kPreTileCols == 0 && K % 128 == 0 &&
         (long long)M * K < (1LL << 31) - 2048 && (long long)K * N < (1LL << 34);
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


enum : int { KERNEL_DECODE = 0, KERNEL_PREFILL = 1, KERNEL_GENERAL = 2, KERNEL_DECODE_DMA = 3 };

// The kernel a call on the reference layout runs (after 3-bit operands at large M are
// expanded to 4 bits): the decode kernel up to 32 rows, and below the large-M
// kernel's threshold up to 96 rows as consecutive launches of <= 32 rows (measured
// on the Llama-2-7B shapes: o at M = 64 17.8 against 28.8 us, down at M = 96 40.5
// against 49.7 us for the general kernel); the large-M kernel where it fits; the
// general kernel otherwise.
int kernel_for(int M, int N, int K) {
  if (prefill_fits(M, N, K, VAL4, META4)) return KERNEL_PREFILL;
  return M <= kDecodeChunkMaxM ? KERNEL_DECODE : KERNEL_GENERAL;
}

// What run() launches for a 4-bit call when nothing limits its scratch:
// out = {kernel (of the first launch), workgroups of the first launch, threads per
// workgroup, K splits of the first launch, launches}.
void describe(int M, int N, int K, int sms, bool noalloc, int out[5]) {
  const int kernel = kernel_for(M, N, K);
  out[0] = kernel;
  if (kernel == KERNEL_DECODE) {
    const int mc = M < kDecodeMaxM ? M : kDecodeMaxM;
    DecodeShape d = decode_shape(mc, N, K, sms);
    if (noalloc) decode_unsplit(d, K);
    // the 16- and 32-row batches run the LDS-DMA decode kernel
    if ((d.mb > decode_batch(mc) ? d.mb : decode_batch(mc)) >= 16) out[0] = KERNEL_DECODE_DMA;
    out[1] = decode_workgroups(N, d);
    out[2] = 64 * d.nw * d.g;
    out[3] = d.splits;
    out[4] = (M + kDecodeMaxM - 1) / kDecodeMaxM;
  } else if (kernel == KERNEL_PREFILL) {
    const PrefillPlan pp = prefill_plan(M, N, K, sms, noalloc || prefill_counters_exceed(N, M));
    out[1] = pp.tiles * pp.splits;
    out[2] = 64 * pp.chunks;
    out[3] = pp.splits;
    out[4] = 1;
  } else {
    Plan plan = plan_for(M, N, K, sms);
    if (noalloc || (size_t)(N / 64) * plan.ztiles * sizeof(int) > kCounterBytes) plan.splits = 1;
    out[1] = (N / 64) * plan.splits * plan.ztiles;
    out[2] = 64 * (plan.bb == 1 ? 8 : 4);
    out[3] = plan.splits;
    out[4] = 1;
  }
}

int launch_error(hipError_t e) {
  if (e == hipSuccess) return MARLIN_HIP_OK;
  set_error(std::string("marlin_hip: kernel launch failed: ") + hipGetErrorString(e));
  return MARLIN_HIP_ERR_LAUNCH;
}

// One GEMM call on the reference layout (or a 3-bit variant of it).  With `noalloc`
// the call allocates nothing: it never splits K (so it needs no partials or
// counters) and never stages operands (3-bit operands are refused), and its only
// scratch is the static zero block.
int run(int vf, int mf, const void* A, const void* B, const void* meta, void* C, void* s, int prob_m,
        int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream, int thread_k, int thread_m,
        int sms, bool noalloc = false) {
  int err = validate(prob_m, prob_n, prob_k, groupsize, thread_k, thread_m);
  if (err != MARLIN_HIP_OK) return err;
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) return MARLIN_HIP_OK;
  // The 64-column chunk and 32-deep k-block of the packed layouts (and 128-deep
  // scale groups) are this implementation's own granularity.
  if (prob_m % 64 != 0 || prob_k % 32 != 0 || (groupsize != -1 && prob_k % 128 != 0)) {
    set_error("marlin_hip: N must be a multiple of 64 and K of 32 (128 when grouped)");
    return MARLIN_HIP_ERR_PROB_SHAPE;
  }
  if (noalloc && (vf != VAL4 || mf != META4)) {
    set_error("marlin_hip: the no-allocation entry point takes 4-bit values and metadata only");
    return MARLIN_HIP_ERR_KERN_SHAPE;
  }
  DeviceScope scope(dev);
  if (!scope.ok) return MARLIN_HIP_ERR_LAUNCH;
  if (sms <= 0) {
    if (hipDeviceGetAttribute(&sms, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || sms <= 0)
      sms = 256;
  }
  const int M = prob_n, N = prob_m, K = prob_k;
  const _Float16* zeros = nullptr;
  err = get_zeros(dev, stream, &zeros);
  if (err != MARLIN_HIP_OK) return err;
  if (kernel_for(M, N, K) == KERNEL_DECODE) {
    for (int r0 = 0; r0 < M; r0 += kDecodeMaxM) {
      const int mc = M - r0 < kDecodeMaxM ? M - r0 : kDecodeMaxM;
      GemmArgs d{};
      d.A = static_cast<const _Float16*>(A) + (size_t)r0 * K;
      d.B = B;
      d.meta = meta;
      d.s = static_cast<const _Float16*>(s);
      d.C = static_cast<_Float16*>(C) + (size_t)r0 * N;
      d.zeros = zeros;
      d.spans = g_spans;
      d.M = mc;
      d.N = N;
      d.K = K;
      DecodeShape shape = decode_shape(mc, N, K, sms);
      if (noalloc) decode_unsplit(shape, K);
      if (shape.splits > 1) {
        const int rows = decode_batch(mc) > 16 ? decode_batch(mc) : 16;
        const size_t split_tiles = (size_t)(N / shape.tc - shape.tail_from);
        err = get_scratch(dev, stream, split_tiles * shape.splits * rows * shape.tc * sizeof(float), &d.counters,
                          &d.partial);
        if (err != MARLIN_HIP_OK) return err;
        if (!d.counters) decode_unsplit(shape, K);  // capturing, and this stream has no scratch yet
      }
      d.splits = shape.splits;
      d.tail_from = shape.tail_from;
      err = launch_error(launch_decode(d, shape, vf, mf, groupsize != -1, stream));
      if (err != MARLIN_HIP_OK) return err;
    }
    return MARLIN_HIP_OK;
  }
  if (prefill_fits(M, N, K, VAL4, META4) && (vf != VAL4 || mf != META4)) {
    // 3-bit values or metadata at large M: expand them into the 4-bit layouts on this
    // stream, then the large-M kernel reads the expanded copy.
    const size_t vbytes = vf == VAL3 ? (size_t)K * N / 4 : 0, mbytes = mf == META3 ? (size_t)K * N / 8 : 0;
    void* stage = nullptr;
    err = get_stage(dev, stream, vbytes + mbytes, &stage);
    if (err != MARLIN_HIP_OK) return err;
    if (vf == VAL3) {
      const long long quads = (long long)K * N / 64;
      hipLaunchKernelGGL(w3_to_w4_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                         static_cast<const uint32_t*>(B), static_cast<u32x4*>(stage), quads);
      B = stage;
    }
    if (mf == META3) {
      void* m4 = static_cast<char*>(stage) + vbytes;
      err = marlin_hip_meta3_unpack(meta, m4, (long long)K * N / 8 / 4 * 3 / 4, dev, stream);
      if (err != MARLIN_HIP_OK) return err;
      meta = m4;
    }
    vf = VAL4;
    mf = META4;
  }
  if (prefill_fits(M, N, K, vf, mf)) {
    GemmArgs p{};
    p.A = static_cast<const _Float16*>(A);
    p.B = B;
    p.meta = meta;
    p.s = static_cast<const _Float16*>(s);
    p.C = static_cast<_Float16*>(C);
    p.zeros = zeros;
    p.M = M;
    p.N = N;
    p.K = K;
    PrefillPlan pp = prefill_plan(M, N, K, sms, noalloc || prefill_counters_exceed(N, M));
    p.splits = pp.splits;
    if (p.splits > 1) {
      err = get_scratch(dev, stream, (size_t)pp.tiles * p.splits * pre_split_bytes(pp.rows, pp.chunks), &p.counters,
                        &p.partial);
      if (err != MARLIN_HIP_OK) return err;
      if (!p.counters) {  // no scratch: the best unsplit plan
        pp = prefill_plan(M, N, K, sms, true);
        p.splits = 1;
      }
    }
    return launch_error(launch_prefill(p, pp.rows, pp.chunks, groupsize != -1, stream));
  }
  Plan plan = plan_for(M, N, K, sms);
  const int chunks = N / 64;
  if (noalloc || (size_t)chunks * plan.ztiles * sizeof(int) > kCounterBytes) plan.splits = 1;
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(A);
  a.B = B;
  a.meta = meta;
  a.s = static_cast<const _Float16*>(s);
  a.C = static_cast<_Float16*>(C);
  a.zeros = zeros;
  a.M = M;
  a.N = N;
  a.K = K;
  if (plan.splits > 1) {
    err = get_scratch(dev, stream, (size_t)plan.splits * M * N * sizeof(float), &a.counters, &a.partial);
    if (err != MARLIN_HIP_OK) return err;
    if (!a.counters) plan.splits = 1;
  }
  a.splits = plan.splits;
  dim3 grid(chunks, plan.splits, plan.ztiles);
  const bool grouped = groupsize != -1;
  hipError_t e;
  if (vf == VAL4 && mf == META4) e = launch_v<VAL4, META4>(a, plan.bb, grouped, grid, stream);
  else if (vf == VAL4) e = launch_v<VAL4, META3>(a, plan.bb, grouped, grid, stream);
  else e = launch_v<VAL3, META4>(a, plan.bb, grouped, grid, stream);
  return launch_error(e);
}

// ---- lane-native layout (sm24_native.h): repack, unpack, GEMM ----

int check_native_shape(int N, int K, int groupsize) {
  if (N <= 0 || K <= 0 || N % 64 != 0 || K % 256 != 0 || !(groupsize == -1 || groupsize == 64)) {
    set_error("marlin_hip: the native layout needs N % 64 == 0, K % 256 == 0 and groupsize 64 (dense 128) or -1");
    return MARLIN_HIP_ERR_PROB_SHAPE;
  }
  return MARLIN_HIP_OK;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string("marlin_hip: ") + what + " launch failed: " + hipGetErrorString(e));
    return MARLIN_HIP_ERR_LAUNCH;
  }
  return MARLIN_HIP_OK;
}

int native_pack(const void* B, const void* meta, const void* s, void* W, void* X, void* S, int N, int K,
                int groupsize, int dev, hipStream_t stream) {
  int err = check_native_shape(N, K, groupsize);
  if (err != MARLIN_HIP_OK) return err;
  DeviceScope scope(dev);
  if (!scope.ok) return MARLIN_HIP_ERR_LAUNCH;
  const long long threads = (long long)(N / 16) * (K / 256) * 64;
  hipLaunchKernelGGL(native_pack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(B), static_cast<const uint16_t*>(meta),
                     static_cast<const _Float16*>(s), static_cast<u32x4*>(W), static_cast<u32x2*>(X),
                     static_cast<uint32_t*>(S), N, K, groupsize != -1 ? 1 : 0);
  err = launch_status("native pack");
  if (err == MARLIN_HIP_OK && groupsize == -1 &&
      hipMemcpyAsync(S, s, (size_t)N * 2, hipMemcpyDeviceToDevice, stream) != hipSuccess) {
    set_error("marlin_hip: copy of the per-column scales failed");
    err = MARLIN_HIP_ERR_LAUNCH;
  }
  return err;
}

int native_unpack(const void* W, const void* X, const void* S, void* B, void* meta, void* s, int N, int K,
                  int groupsize, int dev, hipStream_t stream) {
  int err = check_native_shape(N, K, groupsize);
  if (err != MARLIN_HIP_OK) return err;
  DeviceScope scope(dev);
  if (!scope.ok) return MARLIN_HIP_ERR_LAUNCH;
  const long long words = (long long)(K / 32) * 2 * N;
  hipLaunchKernelGGL(native_unpack_values_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(W), static_cast<uint32_t*>(B), N, K);
  const long long metas = (long long)N * (K / 16);
  hipLaunchKernelGGL(native_unpack_meta_kernel, dim3((unsigned)((metas + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const u32x2*>(X), static_cast<const uint32_t*>(S), static_cast<uint16_t*>(meta),
                     static_cast<_Float16*>(s), N, K, groupsize != -1 ? 1 : 0);
  err = launch_status("native unpack");
  if (err == MARLIN_HIP_OK && groupsize == -1 &&
      hipMemcpyAsync(s, S, (size_t)N * 2, hipMemcpyDeviceToDevice, stream) != hipSuccess) {
    set_error("marlin_hip: copy of the per-column scales failed");
    err = MARLIN_HIP_ERR_LAUNCH;
  }
  return err;
}

// Native kernel shapes, measured on MI355X (Llama-2-7B/70B shapes).  One row: one
// 16-column block per workgroup, a ring 4 quads deep, no split.  2-4 rows: two blocks
// per workgroup and a ring 2 quads deep where N/32 still gives a workgroup per CU
// (each read of the activation rows then serves 32 columns), else one block, 4 deep;
// K split in two at K >= 16384 (down-projection of Llama-2-70B at M = 4: 26.2 ->
// 21.1 us; splits cost the 70B gate_up 3-10 %).  5-16 rows (staged as 8 or 16): the
// activation rows dominate the L2 and LDS traffic, so the widest tile (4, 2 or 1
// blocks; ring 2 deep above one block) whose workgroups, with K split into pieces of
// at least 10 quads, cover 60 % of the CUs, split only when the tiles alone do not
// (a sweep of blocks x splits on the Llama-2 shapes: four blocks unsplit on 160-192
// workgroups beat two blocks or a split, 70B QKV at M = 16 14.0 against 16.8 us;
// split-K is a loss on short pieces: 7B O at M = 8 4.7 us unsplit, 8.1 us in 4).
// MARLIN_HIP_NATIVE_SPLITS forces the count and, at 5-16 rows, MARLIN_HIP_NATIVE_BLOCKS
// the blocks per workgroup (each read once).
struct NativeShape {
  int ncb, splits;
};

NativeShape native_shape(int MB, int N, int K, int cus) {
  static const int forced = env_choice("MARLIN_HIP_NATIVE_SPLITS", {1, 2, 3, 4, 5, 6, 7, 8}, 0);
  static const int forced_ncb = env_choice("MARLIN_HIP_NATIVE_BLOCKS", {1, 2, 4}, 0);
  const int nq = K / 256;
  NativeShape sh{1, 1};
  if (MB >= 8) {
    // the widest tile whose workgroups, with splits of >= 10 quads each, cover 60 %
    // of the CUs; split only below that (then up to one workgroup per CU)
    const int smax = nq / 10 < 1 ? 1 : (nq / 10 > 8 ? 8 : nq / 10);
    const int fill = (3 * cus + 4) / 5;
    for (int ncb = 4; ncb >= 1; ncb >>= 1) {
      const int tiles = N / (16 * ncb);
      if (tiles * smax >= fill || ncb == 1) {
        const int s = tiles >= fill ? 1 : (cus + tiles - 1) / tiles;
        sh = {ncb, s < smax ? s : smax};
        break;
      }
    }
  } else if (MB > 1) {
    sh = {N / 32 >= cus ? 2 : 1, K >= 16384 ? 2 : 1};
  }
  if (MB >= 8 && forced_ncb > 0) sh.ncb = forced_ncb;
  if (forced > 0) sh.splits = forced;
  sh.splits = sh.splits < nq ? sh.splits : nq;
  return sh;
}

template <int MB, int NCB, bool G>
void launch_native_t(const NativeArgs& a, size_t lds, hipStream_t stream) {
  constexpr int D = NCB == 1 ? 4 : 2;
  hipLaunchKernelGGL((sm24_native_decode_kernel<MB, NCB, 4, D, G>),
                     dim3((unsigned)(a.N / (16 * NCB)), (unsigned)a.splits), dim3(256), lds, stream, a.A, a.W, a.X,
                     a.S, a.s_col, a.M, a.N, a.K, a.splits, a);
}

int run_native(const void* A, const void* W, const void* X, void* C, const void* S, int N, int M, int K,
               int groupsize, int dev, hipStream_t stream, int sms) {
  int err = check_native_shape(N, K, groupsize);
  if (err != MARLIN_HIP_OK) return err;
  if (M < 0) return MARLIN_HIP_ERR_PROB_SHAPE;
  if (M == 0) return MARLIN_HIP_OK;
  DeviceScope scope(dev);
  if (!scope.ok) return MARLIN_HIP_ERR_LAUNCH;
  const bool grouped = groupsize != -1;
  if (M > 16) {
    // Larger batches: unpack to the reference layout in the staging buffer (on this
    // stream) and run the reference-layout kernels on it.
    const size_t vb = (size_t)K * N / 4, mb = (size_t)K * N / 8, sb = (size_t)(grouped ? K / 128 : 1) * N * 2;
    void* stage = nullptr;
    err = get_stage(dev, stream, vb + mb + sb, &stage);
    if (err != MARLIN_HIP_OK) return err;
    char* b = static_cast<char*>(stage);
    err = native_unpack(W, X, S, b, b + vb, b + vb + mb, N, K, groupsize, dev, stream);
    if (err != MARLIN_HIP_OK) return err;
    return run(VAL4, META4, A, b, b + vb, C, b + vb + mb, N, M, K, groupsize, dev, stream, -1, -1, sms);
  }
  NativeArgs a{};
  a.A = static_cast<const _Float16*>(A);
  a.W = static_cast<const u32x4*>(W);
  a.X = static_cast<const u32x2*>(X);
  a.S = static_cast<const uint32_t*>(S);
  a.s_col = static_cast<const _Float16*>(S);
  a.C = static_cast<_Float16*>(C);
  a.M = M;
  a.N = N;
  a.K = K;
  const int MB = M == 1 ? 1 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16));
  if (sms <= 0) {
    if (hipDeviceGetAttribute(&sms, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || sms <= 0)
      sms = 256;
  }
  const NativeShape sh = native_shape(MB, N, K, sms);
  const int ncb = sh.ncb;
  a.splits = sh.splits;
  if (a.splits > 1 && (size_t)(N / (16 * ncb)) * sizeof(uint32_t) > kCounterBytes) a.splits = 1;
  if (a.splits > 1) {
    err = get_scratch(dev, stream, (size_t)(N / 16) * a.splits * MB * 16 * sizeof(float), &a.counters, &a.partial);
    if (err != MARLIN_HIP_OK) return err;
    if (!a.counters) a.splits = 1;  // capturing, and this stream has no scratch yet
  }
  const size_t act = (size_t)4 * MB * 512;  // a staging slot per wave
  const size_t red = (size_t)4 * ncb * MB * 16 * sizeof(float);
  const size_t lds = act > red ? act : red;
  if (MB == 1) {
    if (grouped) launch_native_t<1, 1, true>(a, lds, stream);
    else launch_native_t<1, 1, false>(a, lds, stream);
  } else if (MB == 4 && ncb == 1) {
    if (grouped) launch_native_t<4, 1, true>(a, lds, stream);
    else launch_native_t<4, 1, false>(a, lds, stream);
  } else if (MB == 4) {
    if (grouped) launch_native_t<4, 2, true>(a, lds, stream);
    else launch_native_t<4, 2, false>(a, lds, stream);
  } else if (MB == 8 && ncb == 1) {
    if (grouped) launch_native_t<8, 1, true>(a, lds, stream);
    else launch_native_t<8, 1, false>(a, lds, stream);
  } else if (MB == 8 && ncb == 2) {
    if (grouped) launch_native_t<8, 2, true>(a, lds, stream);
    else launch_native_t<8, 2, false>(a, lds, stream);
  } else if (MB == 8) {
    if (grouped) launch_native_t<8, 4, true>(a, lds, stream);
    else launch_native_t<8, 4, false>(a, lds, stream);
  } else if (ncb == 1) {
    if (grouped) launch_native_t<16, 1, true>(a, lds, stream);
    else launch_native_t<16, 1, false>(a, lds, stream);
  } else if (ncb == 2) {
    if (grouped) launch_native_t<16, 2, true>(a, lds, stream);
    else launch_native_t<16, 2, false>(a, lds, stream);
  } else {
    if (grouped) launch_native_t<16, 4, true>(a, lds, stream);
    else launch_native_t<16, 4, false>(a, lds, stream);
  }
  return launch_status("native GEMM");
}

}  // namespace sm24

extern "C" {

int marlin_hip_native_pack(const void* B, const void* meta, const void* s, void* Bn, void* metan, void* sn,
                           int prob_m, int prob_k, int groupsize, int dev, hipStream_t stream) {
  return sm24::native_pack(B, meta, s, Bn, metan, sn, prob_m, prob_k, groupsize, dev, stream);
}

int marlin_hip_native_unpack(const void* Bn, const void* metan, const void* sn, void* B, void* meta, void* s,
                             int prob_m, int prob_k, int groupsize, int dev, hipStream_t stream) {
  return sm24::native_unpack(Bn, metan, sn, B, meta, s, prob_m, prob_k, groupsize, dev, stream);
}

int marlin_hip_mul_2_4_native(const void* A, const void* Bn, const void* metan, void* C, const void* sn,
                              int prob_m, int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream,
                              int sms) {
  return sm24::run_native(A, Bn, metan, C, sn, prob_m, prob_n, prob_k, groupsize, dev, stream, sms);
}

int marlin_hip_mul_2_4(const void* A, const void* B, const void* meta, void* C, void* s, int prob_m,
                       int prob_n, int prob_k, void* workspace, int groupsize, int dev, hipStream_t stream,
                       int thread_k, int thread_m, int sms, int max_par) {
  (void)workspace;
  (void)max_par;
  return sm24::run(sm24::VAL4, sm24::META4, A, B, meta, C, s, prob_m, prob_n, prob_k, groupsize, dev, stream,
                   thread_k, thread_m, sms);
}

int marlin_hip_plan(int prob_m, int prob_n, int prob_k, int groupsize, int thread_k, int thread_m, int sms,
                    int noalloc, int* out) {
  int err = sm24::validate(prob_m, prob_n, prob_k, groupsize, thread_k, thread_m);
  if (err != MARLIN_HIP_OK) return err;
  if (prob_m % 64 != 0 || prob_k % 32 != 0 || (groupsize != -1 && prob_k % 128 != 0)) {
    sm24::set_error("marlin_hip: N must be a multiple of 64 and K of 32 (128 when grouped)");
    return MARLIN_HIP_ERR_PROB_SHAPE;
  }
  if (prob_m == 0 || prob_n == 0 || prob_k == 0) {
    for (int i = 0; i < 5; i++) out[i] = 0;
    out[0] = -1;
    return MARLIN_HIP_OK;
  }
  sm24::describe(prob_n, prob_m, prob_k, sms > 0 ? sms : 256, noalloc != 0, out);
  return MARLIN_HIP_OK;
}

int marlin_hip_mul_2_4_noalloc(const void* A, const void* B, const void* meta, void* C, const void* s,
                               int prob_m, int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream,
                               int thread_k, int thread_m, int sms) {
  return sm24::run(sm24::VAL4, sm24::META4, A, B, meta, C, const_cast<void*>(s), prob_m, prob_n, prob_k,
                   groupsize, dev, stream, thread_k, thread_m, sms, /*noalloc=*/true);
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

int marlin_hip_set_spans(void* buf) {
  sm24::g_spans = static_cast<uint64_t*>(buf);
  return SM24_SPANS ? MARLIN_HIP_OK : MARLIN_HIP_ERR_KERN_SHAPE;
}

}  // extern "C"
