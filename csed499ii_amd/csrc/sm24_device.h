// Device-side building blocks of the 2:4 INT4 x FP16 GEMM for gfx950 (CDNA4).
//
// Operand layouts are the Sparse-Marlin pack() layouts (reference:
// kernel_experiments/sparse_marlin/src/marlin/__init__.py:331-388), consumed as they
// lie in HBM:
//   * B      int32 [K/32][2N]: nibble p of word (r, 128*c + 4*i + j) is the offset-8
//            code of compressed-K row 16r + ROW_t[p] (t = i%4) and output column
//            64c + 8*(i/4) + 4*BLK[p] + j, ROW_t = {2t,2t+8,2t,2t+8,2t+1,2t+9,2t+1,2t+9},
//            BLK = {0,0,1,1,0,0,1,1}.
//   * meta   int16, CUTLASS-reordered (reference _semi_structured_conversions.py:21-48):
//            for k-block r and 64-column chunk c the 256 bytes at int16 offset
//            2N*r + 128*c hold 32 units of 4 int16; unit q = 16*(j>>1) + 2*g + (j&1)
//            is {m(n,e0), m(n+4,e0), m(n,e1), m(n+4,e1)} for n = 64c + 8g + j, where
//            e selects the first/second 16 dense K of the k-block and nibble u of an
//            int16 is the 2:4 pattern (idx0 | idx1 << 2) of dense group u.
//   * s      fp16 [K/128][N] grouped (within 64 columns, packed slot 8a+b holds
//            column 8a + {0,4,1,5,2,6,3,7}[b]) or [1][N] per column (natural order).
//
// Sparse MFMA operand layout on gfx950, measured on the device (one-hot/random
// probes against a CPU model):
//   v_smfmac_f32_16x16x32_f16: A lane l: row l%16, 4 halves = 2 dense groups
//     (k-space groups 2*(l/16), 2*(l/16)+1), index byte ABID of the idx VGPR holds
//     (idx0 | idx1<<2) per group; B lane l: column l%16, k-space 8*(l/16)+[0,8);
//     D lane l: rows 4*(l/16)+[0,4), column l%16.
//   v_smfmac_f32_16x16x64_f16: A lane l: row l%16, 8 halves = k-space groups
//     4*(l/16)+[0,4), index half-word ABID; B lane l: column l%16, k-space
//     8*(l/16)+[0,8) then 32+8*(l/16)+[0,8); D as above.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sm24 {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half16_t __attribute__((ext_vector_type(16)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 8-byte load from an address that is only 4-byte aligned (3-bit value stream).
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Codes of one output column held in a packed word (after ">> 8" for the second
// column of the pair), as the four halves of a 16x16x32 A operand:
// {code(p0), code(p4), code(p1), code(p5)} - 8, exact in fp16.
// Magic-exponent conversion: (q & 0x000f000f) | 0x6400 is 1024 + code, and the
// high nibble pair is 1024 + 16*code, scaled by 1/16 and shifted by -72.
__device__ __forceinline__ half4_t dequant4(uint32_t q) {
  const uint32_t lo = (q & 0x000F000Fu) | 0x64006400u;
  const uint32_t hi = (q & 0x00F000F0u) | 0x64006400u;
  const half2_t l = __builtin_bit_cast(half2_t, lo) - (half2_t){(_Float16)1032.0f, (_Float16)1032.0f};
  const half2_t h = __builtin_bit_cast(half2_t, hi) * (half2_t){(_Float16)0.0625f, (_Float16)0.0625f} +
                    (half2_t){(_Float16)-72.0f, (_Float16)-72.0f};
  return (half4_t){l.x, l.y, h.x, h.y};
}

// Same for 3-bit codes (zero point 4) already spread to nibble positions.
__device__ __forceinline__ half4_t dequant3(uint32_t q) {
  const uint32_t lo = (q & 0x000F000Fu) | 0x64006400u;
  const uint32_t hi = (q & 0x00F000F0u) | 0x64006400u;
  const half2_t l = __builtin_bit_cast(half2_t, lo) - (half2_t){(_Float16)1028.0f, (_Float16)1028.0f};
  const half2_t h = __builtin_bit_cast(half2_t, hi) * (half2_t){(_Float16)0.0625f, (_Float16)0.0625f} +
                    (half2_t){(_Float16)-68.0f, (_Float16)-68.0f};
  return (half4_t){l.x, l.y, h.x, h.y};
}

// Spread 8 three-bit codes (bits 3i..3i+2 of a 24-bit field) to nibble i.
__device__ __forceinline__ uint32_t spread3(uint32_t x) {
  x = ((x & 0x00FFF000u) << 4) | (x & 0x00000FFFu);
  x = ((x & 0x0FC00FC0u) << 2) | (x & 0x003F003Fu);
  return ((x & 0x38383838u) << 1) | (x & 0x07070707u);
}

__device__ __forceinline__ half4_t scale4(half4_t a, _Float16 s) {
  return a * (half4_t){s, s, s, s};
}

// Sparse-index bytes for one unit pair: d0 = {m(n,e0) | m(n+4,e0) << 16},
// d1 = {m(n,e1) | m(n+4,e1) << 16}; sh = 4*h selects dense groups h and h+4.
// Result byte 0: index byte of column n, byte 2: of column n+4.
__device__ __forceinline__ uint32_t idx_pair(uint32_t d0, uint32_t d1, uint32_t sh) {
  const uint32_t x = (d0 >> sh) & 0x000F000Fu;
  const uint32_t y = (d1 >> sh) & 0x000F000Fu;
  return x | (y << 4);
}

enum : int { VAL4 = 0, VAL3 = 1 };
enum : int { META4 = 0, META3 = 1 };

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
// The same tables as bytes (entry c in byte c of the 8-byte pair lo | hi << 32), for
// a v_perm lookup of up to four codes at once.
constexpr uint32_t tab_of(const int (&t)[8], int half) {
  uint32_t v = 0;
  for (int i = 0; i < 4; i++) v |= (uint32_t)t[4 * half + i] << (8 * i);
  return v;
}
constexpr uint32_t kTabHighLo = tab_of(kDecHigh, 0), kTabHighHi = tab_of(kDecHigh, 1);
constexpr uint32_t kTabLowLo = tab_of(kDecLow, 0), kTabLowHi = tab_of(kDecLow, 1);

struct GemmArgs {
  const _Float16* A;
  const void* B;
  const void* meta;
  const _Float16* s;
  _Float16* C;
  const _Float16* zeros;  // >= 64 zero bytes (activation rows that do not exist)
  int M, N, K;
  int splits;
  int tail_from;   // decode: first split tile (0: every tile split when splits > 1)
  float* partial;  // [splits][M][N] when splits > 1
  uint32_t* counters;  // [gridDim.z][gridDim.x] arrival counters, zero between launches
  uint64_t* spans;     // per-wave timestamps (only read by a build with SM24_SPANS=1)
};

// The decode kernels take the fields their prologue needs first (14 dwords) as
// leading scalar arguments ahead of the whole GemmArgs: the translation units that
// instantiate them are built with -mllvm -amdgpu-kernarg-preload-count=14, so
// gfx950's dispatcher preloads those fields into SGPRs and the first address
// computation waits for no kernel-argument load.  (The fp16 pointers travel as void
// pointers: a _Float16 in a kernel's signature leaves its name undemangled in the
// profilers' traces.)
__device__ __forceinline__ GemmArgs with_lead(GemmArgs a, const void* B, const void* meta, const void* s,
                                              const void* A, const void* zeros, int M, int N, int K, int splits) {
  a.B = B;
  a.meta = meta;
  a.s = static_cast<const _Float16*>(s);
  a.A = static_cast<const _Float16*>(A);
  a.zeros = static_cast<const _Float16*>(zeros);
  a.M = M;
  a.N = N;
  a.K = K;
  a.splits = splits;
  return a;
}

// Per-wave phase timestamps of the decode kernel, compiled in only by the
// measurement build (SM24_SPANS=1, libmarlin_hip_spans.so): wave w of workgroup b
// writes kSpanWords 64-bit words at spans[(b * waves + w) * kSpanWords]: the 100 MHz
// real-time counter at entry (stamp 0), once the kernel arguments have arrived (1),
// once its load addresses are set up (2), once its first stages' loads are issued
// (3), after its last stage's MFMAs (4) and at exit (5); the shader clock at entry
// and exit; the hardware id of its compute unit; and the workgroup index.  Lane 0
// stores them with vector stores.
#ifndef SM24_SPANS
#define SM24_SPANS 0
#endif
constexpr int kSpanStamps = 6;
constexpr int kSpanWords = 12;
struct SpanStamps {
#if SM24_SPANS
  uint64_t t[kSpanStamps] = {};
  uint64_t c0 = 0;
#endif
  __device__ __forceinline__ void mark(int i) {
#if SM24_SPANS
    __builtin_amdgcn_sched_barrier(0);
    t[i] = __builtin_amdgcn_s_memrealtime();
    if (i == 0) c0 = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
#else
    (void)i;
#endif
  }
  // stamp 1: waits for a kernel argument first
  __device__ __forceinline__ void mark_args(int arg) {
#if SM24_SPANS
    asm volatile("" ::"s"(arg));
    mark(1);
#else
    (void)arg;
#endif
  }
  __device__ __forceinline__ void store(uint64_t* spans, int waves, int wave, int lane) {
#if SM24_SPANS
    mark(kSpanStamps - 1);
    const uint64_t c1 = __builtin_amdgcn_s_memtime();
    if (spans != nullptr && lane == 0) {
      uint64_t* o = spans + ((size_t)blockIdx.x * waves + wave) * kSpanWords;
      uint64_t v[kSpanWords] = {};
#pragma unroll
      for (int i = 0; i < kSpanStamps; i++) v[i] = t[i];
      v[6] = c0;
      v[7] = c1;
      v[8] = (uint64_t)__smid();
      v[9] = (uint64_t)blockIdx.x;
#pragma unroll
      for (int i = 0; i < kSpanWords; i++) __builtin_nontemporal_store(v[i], o + i);
    }
#else
    (void)spans, (void)waves, (void)wave, (void)lane;
#endif
  }
};

// Large-M kernel (sm24_prefill.hip): output columns per workgroup tile (N must be a
// multiple) and its launcher.
constexpr int kDecodeMaxM = 32;       // largest batch of one decode launch (two 16-row blocks)
constexpr int kDecodeChunkMaxM = 96;  // largest batch run as several decode launches
constexpr int kPreTileCols = 512;
constexpr int kPreThreads = 512;  // one wave per 64-column chunk of the tile
constexpr int kPreChunks = 8;        // 64-column chunks per tile = waves per workgroup
constexpr int kPreNarrowChunks = 4;  // the narrow tile: 256 columns (128 rows), 4 waves
// fp32 partial of one tile of `rows` (128 or 64) batch rows and `chunks` 64-column chunks
constexpr size_t pre_split_bytes(int rows, int chunks = 8) { return (size_t)64 * chunks * rows * sizeof(float); }
hipError_t launch_prefill(const GemmArgs& a, int rows, int chunks, bool grouped, hipStream_t stream);

template <int ABID>
__device__ __forceinline__ float4_t smfmac32(half4_t a, half8_t b, float4_t c, uint32_t idx) {
  return __builtin_amdgcn_smfmac_f32_16x16x32_f16(a, b, c, (int)idx, 0, ABID);
}

template <int ABID>
__device__ __forceinline__ float4_t smfmac64(half8_t a, half16_t b, float4_t c, uint32_t idx) {
  return __builtin_amdgcn_smfmac_f32_16x16x64_f16(a, b, c, (int)idx, 0, ABID);
}

// LDS-DMA (global_load_lds_*): every lane copies 16 (or 4) bytes from a global
// address to LDS byte address M0 + instruction offset + 16 (or 4) * lane; the
// instruction offset applies to both addresses.  Tracked by vmcnt, like any global
// load; the LDS address must be wave-uniform.  M0 is set in the same statement (one
// wait state before the first DMA reads it).

// Two DMAs of 16 bytes per lane into lds + 1024 u + 16 lane (u = 0, 1) from
// base + v[u] + 1024 u.
__device__ __forceinline__ void dma16x2(uint32_t lds, const uint32_t (&v)[2], const void* base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %3\n\t"
      "global_load_lds_dwordx4 %2, %3 offset:1024" ::"s"(lds),
      "v"(v[0]), "v"(v[1]), "s"(base)
      : "memory", "m0");
}
// As dma16x2 with one instruction: 16 bytes per lane from base + v into lds + 16 lane.
__device__ __forceinline__ void dma16x1(uint32_t lds, uint32_t v, const void* base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2" ::"s"(lds),
      "v"(v), "s"(base)
      : "memory", "m0");
}
// One wave's weight side of a k-step, into lds + [0, 1792): 16 bytes per lane from
// bw + vw (-> lds + 16 lane), 4 bytes per lane from bm + vm0 + 1024 (-> + 1024) and
// bm + vm1 + 1280 (-> + 1280), then 4 bytes per lane from bs + vs + 1536 (-> + 1536).
__device__ __forceinline__ void dma_chunk(uint32_t lds, uint32_t vw, const void* bw, uint32_t vm0, uint32_t vm1,
                                          const void* bm, uint32_t vs, const void* bs) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "global_load_lds_dword %3, %5 offset:1024\n\t"
      "global_load_lds_dword %4, %5 offset:1280\n\t"
      "global_load_lds_dword %6, %7 offset:1536" ::"s"(lds),
      "v"(vw), "s"(bw), "v"(vm0), "v"(vm1), "s"(bm), "v"(vs), "s"(bs)
      : "memory", "m0");
}
// As dma_chunk without the scales.
__device__ __forceinline__ void dma_chunk_nos(uint32_t lds, uint32_t vw, const void* bw, uint32_t vm0, uint32_t vm1,
                                              const void* bm) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "global_load_lds_dword %3, %5 offset:1024\n\t"
      "global_load_lds_dword %4, %5 offset:1280" ::"s"(lds),
      "v"(vw), "s"(bw), "v"(vm0), "v"(vm1), "s"(bm)
      : "memory", "m0");
}

// One DMA of 16 bytes per lane from the lane's own 64-bit address src into
// lds + 16 lane (lanes outside the exec mask copy nothing).
__device__ __forceinline__ void dma16(uint32_t lds, const void* src) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off" ::"s"(lds),
      "v"(src)
      : "memory", "m0");
}

// Waits until at most N vector-memory operations of this wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace sm24
