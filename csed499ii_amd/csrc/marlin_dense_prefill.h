// Prefill-sized (large M) dense INT4 x FP16 GEMM for gfx950 (the reference's dense
// Marlin `mul`, marlin_cuda_kernel.cu:655-736, at batch sizes where it is MFMA-bound).
//
// Workgroup tile: 512 output columns (8 chunks of 64) x 128 batch rows, 8 waves, two
// per SIMD; wave w owns chunk w for all 128 rows as 4 x 2 v_mfma_f32_32x32x16_f16
// accumulators (128 AGPRs).  K advances in steps of 64 (four 16-deep k-tiles); one
// k-step is 32 MFMAs per wave.
//
// Operand routes (all global reads are LDS-DMA; a ring of 4 k-steps, filled 3 steps
// ahead, one barrier per k-step):
//  * activations: 128 rows x 128 bytes per k-step, 16-byte pieces stored with the
//    logical slot XOR ((row >> 1) & 7) (the layout of the 2:4 prefill kernel), so the
//    two 8-byte B-operand reads of a lane are free of bank conflicts;
//  * packed codes: the raw dense Marlin words of the wave's chunk, 512 bytes per
//    k-tile (marlin/__init__.py:78-99): word 16 ci + 4 rq + jt holds columns
//    16 jt + ci (bytes 0, 2) and + 8 (bytes 1, 3), with k = 2 rq (low nibble of
//    byte 0 / 1), 2 rq + 8 (high), 2 rq + 1 (byte 2 / 3 low), 2 rq + 9 (high);
//  * grouped scales: the 256 bytes of the chunk pair (cw & ~1, cw | 1) of the step's
//    group (slot 8 i + j of a chunk holds column i + 8 j).
//
// MFMA roles.  The weight is the A operand (rows = output columns), the activations
// the B operand (columns = batch rows).  A lane l = 32 h + i of fragment (k-tile kt,
// half hf) holds output column 64 cw + 32 hf + i, i.e. ci = i & 7, byte half
// b = (i >> 3) & 1, jt = 2 hf + (i >> 4), and the 8 k of words rq = 2h and 2h + 1:
// low nibbles k = 4h .. 4h + 3, high nibbles k = 4h + 8 .. 4h + 11, in that order.
// B lane (row m, h) holds the same k of row m: the 8-byte units 4 kt + h and
// 4 kt + 2 + h of the row.  The result register r of lane l = 32 h + m is column
// 64 cw + 32 hf + 8 (r / 4) + 4 h + r % 4 of batch row m0 + 32 rg + m.
//
// Issue schedule.  Each k-tile is 8 regions (rg, hf), one MFMA each; beside them the
// next k-tile's two A fragments are dequantized in seven slices of at most four VALU
// instructions (regions 0-6: the operands are finished at least two instructions
// before the first MFMA that reads them), the next k-tile's B fragments are read three
// fragments ahead, the raw words two k-tiles ahead, and the DMAs of the step three
// ahead are issued in the step's first regions.
#pragma once
#include "sm24_device.h"

namespace sm24 {

struct DensePreArgs {
  const _Float16* A;
  const uint32_t* B;
  const _Float16* s;
  _Float16* C;
  int M, N, K;
  int splits;
  float* partial;      // [tiles][splits] x 256 KiB when splits > 1
  uint32_t* counters;  // one per tile, zero between launches
};

constexpr int kDpRows = 128;       // batch rows per tile
constexpr int kDpChunks = 8;       // 64-column chunks per tile = waves per workgroup
constexpr int kDpThreads = 64 * kDpChunks;
constexpr int kDpTileCols = 64 * kDpChunks;
constexpr int kDpRing = 4;                   // k-steps resident in LDS
constexpr int kDpActB = kDpRows * 128;       // activation bytes of one k-step
constexpr int kDpWgtW = 2048 + 256;          // per wave: codes of 4 k-tiles, scales
constexpr int kDpSlotB = kDpActB + kDpChunks * kDpWgtW;
constexpr int kDpLdsBytes = kDpRing * kDpSlotB;
constexpr size_t kDpSplitBytes = (size_t)kDpTileCols * kDpRows * sizeof(float);
static_assert(kDpLdsBytes <= 160 * 1024, "LDS");
static_assert(kDpWgtW % 256 == 0, "wave blocks keep the bank pattern");

typedef float f32x16 __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_f16 with the accumulator in AGPRs (inline assembly: for the
// builtin, hipcc moves 128 live accumulators between VGPRs and AGPRs around the
// MFMAs).  Outside the compiler's hazard tracking, so the kernel keeps the gfx950
// rules by construction: a VGPR operand written by VALU is read at least two
// instructions later, and the accumulators are read only after dp_mfma_drain.
__device__ __forceinline__ void dp_mfma(f32x16& c, half8_t a, half8_t b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

__device__ __forceinline__ void dp_mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// The weight side of one k-step for one wave: 16 bytes per lane from bw + v0 and
// bw + v1 + 1024 (-> lds + 16 lane, + 1024), and, grouped, 4 bytes per lane from
// bs + vs + 2048 (-> lds + 2048 + 4 lane).
__device__ __forceinline__ void dp_dma_w(uint32_t lds, uint32_t v0, uint32_t v1, const void* bw, uint32_t vs,
                                         const void* bs) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %3\n\t"
      "global_load_lds_dwordx4 %2, %3 offset:1024\n\t"
      "global_load_lds_dword %4, %5 offset:2048" ::"s"(lds),
      "v"(v0), "v"(v1), "s"(bw), "v"(vs), "s"(bs)
      : "memory", "m0");
}
__device__ __forceinline__ void dp_dma_w_nos(uint32_t lds, uint32_t v0, uint32_t v1, const void* bw) {
  asm volatile(
      "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %3\n\t"
      "global_load_lds_dwordx4 %2, %3 offset:1024" ::"s"(lds),
      "v"(v0), "v"(v1), "s"(bw)
      : "memory", "m0");
}

// Start of a k-step: this wave's DMAs except the last NDMA issued have landed, its
// LDS reads are complete; then the workgroup meets.
template <int NDMA>
__device__ __forceinline__ void dp_step_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(NDMA) : "memory");
}

template <int V>
struct DpC {
  static constexpr int value = V;
};

template <bool GROUPED>
__global__ __launch_bounds__(kDpThreads, 1) void marlin_dense_prefill_kernel(DensePreArgs a) {
  constexpr int MT = kDpRows, CT = kDpChunks;
  constexpr int NDMA = GROUPED ? 5 : 4;  // DMA instructions per wave and k-step
  __shared__ __attribute__((aligned(16))) uint8_t lds[kDpLdsBytes];
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const uint32_t lbase = (uint32_t)(size_t)(lds_u8*)lds;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // chunk of this wave
  const int M = a.M, N = a.N, K = a.K;
  const int nks = K >> 6;  // even: the host requires K % 128 == 0

  // ---- split-K: block b = z * T + tile; split z covers an even range of k-steps ----
  const int ntn = N / (64 * CT), ntm = (M + MT - 1) / MT;
  const int T = ntn * ntm;
  const int S = a.splits;
  int z = 0, tile = blockIdx.x, ks0 = 0, ks1 = nks;
  if (S > 1) {
    z = blockIdx.x / T;
    tile = blockIdx.x - z * T;
    ks0 = 2 * (int)(((long long)(nks >> 1) * z) / S);
    ks1 = 2 * (int)(((long long)(nks >> 1) * (z + 1)) / S);
  }
  // ---- tile order: each XCD (block b on XCD b % 8) works through a contiguous range
  // of tiles, row tiles fastest, so the workgroups on one XCD share a column tile's
  // codes in its L2 ----
  int t = tile;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int tn = t / ntm, tm = t - tn * ntm;
  const int c0 = tn * CT;
  const int m0 = tm * MT;
  const int cw = c0 + w;

  // ---- DMA sources: per-lane byte offsets from per-k-step bases ----
  // activations: instruction u of wave w fills pieces 64 (2w + u) + lane of the step's
  // 1024 16-byte pieces; piece P = row P >> 3, physical slot P & 7, holding logical
  // slot (P & 7) ^ ((row >> 1) & 7).  Rows past M repeat row M-1 (never stored).
  uint32_t act_v[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int p = 64 * (2 * w + u) + lane, row = p >> 3;
    const int ls = (p & 7) ^ ((row >> 1) & 7);
    const int m = m0 + row < M ? m0 + row : M - 1;
    act_v[u] = ((uint32_t)m * (uint32_t)K + 8 * ls) * 2 + 1024 * (1 - u);  // base lowered by 1024
  }
  // codes: instruction u copies k-tiles 2u + (lane >> 5), 16-byte piece lane & 31 of
  // the chunk's 512 bytes (k-tile rows are 8N bytes apart)
  const uint32_t rowB = 8 * (uint32_t)N;
  const uint32_t wv0 = (uint32_t)(lane >> 5) * rowB + 512 * (uint32_t)cw + 16 * (uint32_t)(lane & 31);
  const uint32_t wv1 = wv0 + 2 * rowB - 1024;
  // scales (4 bytes per lane) of the chunk pair (cw & ~1, cw | 1) (base lowered by 2048)
  const uint32_t sc_v = 128 * (uint32_t)(cw & ~1) + 4 * lane;

  const char* gA1 = reinterpret_cast<const char*>(a.A) - 1024;
  const char* gB = reinterpret_cast<const char*>(a.B);
  const char* gS1 = reinterpret_cast<const char*>(a.s) - 2048;
  const uint32_t strB = 4 * rowB, strS = 2 * (uint32_t)N;

  // DMA group g of local k-step s (clamped to the split's last) into ring slot q:
  // g = 0 this wave's share of the activation rows, g = 1 its chunk's codes (and the
  // scales of its chunk pair when grouped).  Step offsets are 32-bit: the host keeps
  // K N / 2 below 2^32.
  auto dma = [&](int s, int q, int g) {
    const uint32_t sc = (uint32_t)(ks0 + s < ks1 ? ks0 + s : ks1 - 1);
    const uint32_t slot = lbase + q * kDpSlotB;
    if (g == 0) {
      dma16x2(slot + 2048 * w, act_v, gA1 + 128 * sc);
    } else {
      const uint32_t l = slot + kDpActB + kDpWgtW * w;
      if constexpr (GROUPED)
        dp_dma_w(l, wv0, wv1, gB + sc * strB, sc_v, gS1 + (sc >> 1) * strS);
      else
        dp_dma_w_nos(l, wv0, wv1, gB + sc * strB);
    }
  };

  // ---- this lane's MFMA roles ----
  const int i = lane & 31, h = lane >> 5;
  const int ci = i & 7, bh = (i >> 3) & 1, ih = i >> 4;
  const int swz = (i >> 1) & 7;
  // B fragment (kt, rg): row 32 rg + i, 8-byte units 4 kt + h and 4 kt + 2 + h, i.e.
  // logical slots 2 kt and 2 kt + 1 at byte 8 h
  uint32_t b_off[4][2];
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int u = 0; u < 2; u++) b_off[kt][u] = i * 128 + 16 * ((2 * kt + u) ^ swz) + 8 * h;
  const uint32_t wblk = kDpActB + kDpWgtW * w;
  // codes of fragment (kt, hf): words (ci, 2h, jt) and (ci, 2h + 1, jt), jt = 2 hf + ih
  const uint32_t w_rd = wblk + 64 * ci + 32 * h + 4 * ih;
  // scale of column 32 hf + i of the chunk: slot 8 ci + 2 jt + bh
  const uint32_t s_rd = wblk + 2048 + 128 * (cw & 1) + 2 * (8 * ci + 2 * ih + bh);
  const uint32_t nsh = 8u * bh;

  uint32_t kMask, kMagic, kMaskHi;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));

  half8_t av[2][2];  // [k-tile parity][hf] dequantized weight fragments
  half8_t bv[4];     // B fragments, ring by fragment number 4 kt + rg
  f32x16 acc[4][2];  // [rg][hf]
#pragma unroll
  for (int rg = 0; rg < 4; rg++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      acc[rg][hf] = (f32x16){};
      asm volatile("" : "+a"(acc[rg][hf]));
    }

  auto read_b = [&](int q, int f) -> half8_t {
    const int kt = f >> 2, rg = f & 3;
    const uint8_t* base = lds + q * kDpSlotB + rg * 4096;
    const half4_t x0 = *reinterpret_cast<const half4_t*>(base + b_off[kt][0]);
    const half4_t x1 = *reinterpret_cast<const half4_t*>(base + b_off[kt][1]);
    return __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  // raw codes of k-tiles, two ahead: [k-tile parity][hf][word]
  uint32_t rw[2][2][2];
  auto read_raw = [&](int q, int kt, int par) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const uint8_t* p = lds + q * kDpSlotB + w_rd + 512 * kt + 8 * hf;
      rw[par][hf][0] = *reinterpret_cast<const uint32_t*>(p);
      rw[par][hf][1] = *reinterpret_cast<const uint32_t*>(p + 16);
    }
  };
  // [k-step parity][hf] the step's scales, broadcast; read one step ahead
  half2_t scv[2][2];
  auto read_scales = [&](int q, int par) {
    if constexpr (GROUPED) {
#pragma unroll
      for (int hf = 0; hf < 2; hf++) {
        const _Float16 v = *reinterpret_cast<const _Float16*>(lds + q * kDpSlotB + s_rd + 8 * hf);
        scv[par][hf] = (half2_t){v, v};
      }
    }
  };

  // ---- dequantization of the raw codes rw[rp] into av[ap], in seven slices of at
  // most four VALU instructions: words >> 8 bh -> magic-number halves 1024 + q (low
  // nibbles) or 1024 + 16 q (high) -> q - 8 -> times the scale ----
  uint32_t dx[2][4];
  half2_t dp[2][4];
  auto dq_slice = [&](int sl, int rp, int ap, int sp) {
    const half2_t k1032 = {(_Float16)1032.f, (_Float16)1032.f};
    const half2_t k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2_t km72 = {(_Float16)-72.f, (_Float16)-72.f};
    switch (sl) {
      case 0:
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
          dx[hf][0] = rw[rp][hf][0] >> nsh;
          dx[hf][1] = rw[rp][hf][1] >> nsh;
        }
        break;
      case 1:
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
          dx[hf][2] = (dx[hf][0] & kMaskHi) | kMagic;
          dx[hf][3] = (dx[hf][1] & kMaskHi) | kMagic;
        }
        break;
      case 2:
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
          dx[hf][0] = (dx[hf][0] & kMask) | kMagic;
          dx[hf][1] = (dx[hf][1] & kMask) | kMagic;
        }
        break;
      case 3:
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
          dp[hf][0] = __builtin_bit_cast(half2_t, dx[hf][0]) - k1032;
          dp[hf][1] = __builtin_bit_cast(half2_t, dx[hf][1]) - k1032;
        }
        break;
      case 4:
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
          dp[hf][2] = __builtin_bit_cast(half2_t, dx[hf][2]) * k16th + km72;
          dp[hf][3] = __builtin_bit_cast(half2_t, dx[hf][3]) * k16th + km72;
        }
        break;
      default: {  // 5: hf = 0, 6: hf = 1
        const int hf = sl - 5;
        if constexpr (GROUPED) {
#pragma unroll
          for (int e = 0; e < 4; e++) dp[hf][e] = dp[hf][e] * scv[sp][hf];
        }
        av[ap][hf] = (half8_t){dp[hf][0].x, dp[hf][0].y, dp[hf][1].x, dp[hf][1].y,
                               dp[hf][2].x, dp[hf][2].y, dp[hf][3].x, dp[hf][3].y};
        break;
      }
    }
  };

  // ---- k-step s in ring slot Q = s & 3 (slot QN: step s + 1, slot QD: step s + 3):
  //   barrier: this wave's DMAs of step s + 1 have landed, every wave has finished
  //   step s - 1 (its reads of slot QD);
  //   k-tile kt, region r = (rg, hf): MFMA (kt, rg, hf); at hf = 0 the read of B
  //   fragment f + 3 (f = 4 kt + rg; from step s + 1 past 15; its ring slot held
  //   fragment f - 1, used up by then); at r = 0 the raw codes
  //   of k-tile kt + 2 (from step s + 1 past 3) and, at kt = 2, the scales of step
  //   s + 1; at r < 7 slice r of dequantizing k-tile kt + 1 (with step s + 1's scales
  //   at kt = 3); at kt = 0, r = 1, 3 the DMA groups of step s + 3.
  // Steps past the last are skipped (uniform); the DMAs are clamped, so the vmcnt of
  // every barrier counts exactly the DMAs of one step. ----
  auto step = [&](int s, auto qc) {
    constexpr int Q = decltype(qc)::value, QN = (Q + 1) & 3, QD = (Q + 3) & 3, SP = Q & 1;
    dp_step_barrier<NDMA>();
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      const int P = kt & 1;
#pragma unroll
      for (int r = 0; r < 8; r++) {
        const int rg = r >> 1, hf = r & 1, f = 4 * kt + rg;
        dp_mfma(acc[rg][hf], av[P][hf], bv[f & 3]);
        __builtin_amdgcn_sched_barrier(0);  // the region's work follows its MFMA
        if (hf == 0) bv[(f + 3) & 3] = read_b(f + 3 < 16 ? Q : QN, (f + 3) & 15);
        if (r == 0) read_raw(kt + 2 < 4 ? Q : QN, (kt + 2) & 3, P);
        if (r == 0 && kt == 2) read_scales(QN, SP ^ 1);
        if (kt == 0 && (r == 1 || r == 3)) dma(s + 3, QD, r >> 1);
        if (r < 7) dq_slice(r, P ^ 1, P ^ 1, kt == 3 ? SP ^ 1 : SP);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // ---- prologue: DMAs of steps 0..2; step 0's scales, k-tile 0 dequantized, raw codes
  // of k-tile 1, the first three B fragments ----
#pragma unroll
  for (int s = 0; s < 3; s++)
#pragma unroll
    for (int g = 0; g < 2; g++) dma(s, s, g);
  dp_step_barrier<NDMA>();
  read_scales(0, 0);
  read_raw(0, 0, 1);
#pragma unroll
  for (int sl = 0; sl < 7; sl++) dq_slice(sl, 1, 0, 0);
  read_raw(0, 1, 1);
  bv[0] = read_b(0, 0);
  bv[1] = read_b(0, 1);
  bv[2] = read_b(0, 2);
  __builtin_amdgcn_sched_barrier(0);

  const int nls = ks1 - ks0;  // k-steps of this split (even)
  for (int s = 0; s < nls; s += 4) {
    step(s, DpC<0>{});
    step(s + 1, DpC<1>{});
    if (s + 2 < nls) {
      step(s + 2, DpC<2>{});
      step(s + 3, DpC<3>{});
    }
  }
  // DMAs of (clamped) steps past the last may still be landing in LDS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  dp_mfma_drain();
#pragma unroll
  for (int rg = 0; rg < 4; rg++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) asm volatile("" : "+a"(acc[rg][hf]));

  // ---- split-K hand-off: the partial tile goes to the uncached scratch in register
  // order ([tile][split][wave][rg][hf][q][lane] float4s, 256 KiB per tile and split);
  // the last split to arrive at the tile's counter reads all splits back and adds them
  // in split order (bit-identical from run to run, whichever split comes last),
  // writes C and resets the counter ----
  const float* const pbase = a.partial + ((size_t)tile * S) * 65536 + (size_t)w * 8192 + 4 * lane;
  if (S > 1) {
    float* const pmine = a.partial + ((size_t)tile * S + z) * 65536 + (size_t)w * 8192 + 4 * lane;
#pragma unroll
    for (int rg = 0; rg < 4; rg++) {
      if (m0 + 32 * rg >= M) break;  // 32-row blocks past M are never read back (uniform)
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int q = 0; q < 4; q++)
          *reinterpret_cast<float4_t*>(pmine + ((rg * 2 + hf) * 4 + q) * 256) =
              (float4_t){acc[rg][hf][4 * q], acc[rg][hf][4 * q + 1], acc[rg][hf][4 * q + 2], acc[rg][hf][4 * q + 3]};
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    __shared__ uint32_t arrived;
    if (tid == 0) arrived = __hip_atomic_fetch_add(a.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __syncthreads();
    if (arrived != (uint32_t)S) return;
    if (tid == 0) __hip_atomic_store(a.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- epilogue: register 4 q + e of acc[rg][hf] is column 64 cw + 32 hf + 8 q + 4 h
  // + e of batch row m0 + 32 rg + i: four consecutive columns per (rg, hf, q).  With
  // split-K the float4 (hf, q) is read back from every split, in split order, two
  // splits per batch of loads (16 loads in flight per lane). ----
#pragma unroll
  for (int rg = 0; rg < 4; rg++) {
    if (m0 + 32 * rg >= M) break;  // uniform: no rows of this block are stored
    float4_t v[2][4];
    if (S == 1) {
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int q = 0; q < 4; q++)
          v[hf][q] = (float4_t){acc[rg][hf][4 * q], acc[rg][hf][4 * q + 1], acc[rg][hf][4 * q + 2],
                                acc[rg][hf][4 * q + 3]};
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) v[k >> 2][k & 3] = (float4_t){0.f, 0.f, 0.f, 0.f};
      const float* p = pbase + rg * 8 * 256;
      for (int zz = 0; zz < S; zz += 2) {
        const bool two = zz + 1 < S;  // uniform
        float4_t t0[8], t1[8];
#pragma unroll
        for (int k = 0; k < 8; k++) t0[k] = *reinterpret_cast<const float4_t*>(p + k * 256 + (size_t)zz * 65536);
        if (two) {
#pragma unroll
          for (int k = 0; k < 8; k++)
            t1[k] = *reinterpret_cast<const float4_t*>(p + k * 256 + (size_t)(zz + 1) * 65536);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) v[k >> 2][k & 3] += t0[k];
        if (two) {
#pragma unroll
          for (int k = 0; k < 8; k++) v[k >> 2][k & 3] += t1[k];
        }
      }
    }
    const int m = m0 + 32 * rg + i;
    if (m < M) {
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int n = 64 * cw + 32 * hf + 8 * q + 4 * h;
          const float4_t x = v[hf][q];
          half4_t o = {(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
          if constexpr (!GROUPED) {
            // per-column scale of the fp16-rounded sum: within 32 columns, column c
            // sits at slot 8 ((c >> 1) & 3) + 2 ((c >> 3) & 3) + (c & 1)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int c = (n + e) & 31;
              o[e] = o[e] * a.s[((n + e) & ~31) + 8 * ((c >> 1) & 3) + 2 * ((c >> 3) & 3) + (c & 1)];
            }
          }
          *reinterpret_cast<half4_t*>(a.C + (size_t)m * N + n) = o;
        }
    }
  }
}

hipError_t launch_dense_prefill(const DensePreArgs& a, bool grouped, hipStream_t stream);

}  // namespace sm24
