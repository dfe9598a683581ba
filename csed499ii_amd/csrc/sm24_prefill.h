// Prefill-sized (large M) 2:4 INT4 x FP16 GEMM for gfx950, MFMA-bound.
//
// Workgroup tile: 512 output columns (8 chunks of 64) x 128 batch rows, 8 waves, two
// per SIMD; wave w owns chunk w (64 columns) for all 128 rows as 4 x 2
// v_smfmac_f32_32x32x32_f16 accumulators (128 AGPRs).  K advances in steps of 64 (two
// 32-deep k-blocks); one k-step is 16 MFMAs per wave.  A second instantiation
// (template argument RG = 2) runs 64-row tiles: 2 x 2 accumulators (64 AGPRs), 8
// MFMAs per k-step, for calls whose 128-row tiles would leave CUs idle.  A third
// (CT = 4 chunks) runs the narrow tile: 256 columns x 128 rows, 4 waves (one per
// SIMD, one workgroup per CU by its 92 KiB of LDS), the same per-wave work as the
// 512-column tile; it replaces 64-row tiles where it comes to the same number of
// workgroups, so that each dequantized weight fragment still feeds four B fragments.
//
// Why two waves per SIMD.  Measured on MI355X (random operands): a 32x32x32 smfmac
// takes ~35 cycles, and the VALU can issue ~4 instructions of 4 cycles beside it.
// With one wave per SIMD every other instruction (LDS read, LDS-DMA, SALU, wait) is
// issued in order by the same wave and adds ~3-10 cycles to its MFMA; with two waves
// the other wave's MFMA hides them, and a mix of 4 VALU + 1 ds_read_b128 + DMA per
// MFMA runs at ~37 cycles per MFMA instead of ~54.  Dequantization stays at ~3.4 VALU
// instructions per MFMA because each wave still covers all 128 rows of its columns
// (13 VALU per 8-value weight fragment, reused by 4 B fragments).
//
// Operand routes (all global reads are LDS-DMA: no staging registers, no staging
// VALU; a ring of 4 k-steps, filled 3 steps ahead, one barrier per k-step):
//  * activations: 128 rows x 128 bytes per k-step; 16-byte pieces stored with the
//    logical slot XOR ((row >> 1) & 7) so that the B-fragment reads are free of bank
//    conflicts; a B lane (row, h) reads the 32 contiguous bytes of k 16h..16h+15;
//  * packed values, metadata, scales: the raw global layout of each wave's own chunk
//    (512 + 256 bytes per k-block, 128 bytes of scales per group), read per lane.
//
// MFMA k order.  For a 32-deep k-block, A lane group h (lanes 32h..32h+31) holds MFMA
// groups 4h..4h+3 = real groups 2h, 2h+1, 2h+4, 2h+5, which makes:
//  * B lane group h's k-ranges (MFMA k 8h+[0,8) and 16+8h+[0,8)) the real k 16h..16h+15;
//  * the A values the nibbles of the packed words (g8, t = 2h, j) and (g8, 2h+1, j):
//    column half 0 (n) in bytes 0, 2 and half 1 (n+4) in bytes 1, 3 of each word;
//  * the index halfword of half hf = [byte h of m(n',e0), byte h of m(n',e1)] with
//    n' = n + 4hf, so one v_perm of the metadata unit gives both halves' indices
//    (selected by abid).
// A row rho (0..31) of fragment (chunk c, half hf) is output column
// 64c + 8*(rho >> 2) + 4*hf + (rho & 3).
#pragma once
#include "sm24_device.h"

namespace sm24 {

template <int V>
struct IntC {
  static constexpr int value = V;
};

typedef float f32x16 __attribute__((ext_vector_type(16)));

static_assert(64 * kPreChunks == kPreTileCols && kPreThreads == 64 * kPreChunks, "tile width");
constexpr int kPreRing = 4;                        // k-steps resident in LDS
// Weight side of one k-step, per wave (one chunk): packed values of both k-blocks
// (1 KiB), metadata of both k-blocks (2 x 256 B), scales of the chunk pair (256 B),
// contiguous so that one M0 value serves the wave's weight-side DMAs (instruction
// offsets 0/1024/1280/1536).
constexpr int kPreWgtW = 1792;
constexpr int kPreActOff = 0;
// LDS layout of a tile of RG 32-row blocks (128 or 64 batch rows): the activation
// ring (32 RG rows x 128 bytes per k-step), then the weight ring.
template <int RG, int CT = kPreChunks>
struct PreLds {
  static constexpr int act_b = 32 * RG * 128;  // activation bytes of one k-step
  static constexpr int wgt_b = CT * kPreWgtW;   // weight side of one k-step
  static constexpr int wgt_off = kPreActOff + kPreRing * act_b;
  static constexpr int bytes = wgt_off + kPreRing * wgt_b;
};
static_assert(kPreWgtW % 256 == 0, "wave blocks keep the bank pattern");
static_assert(PreLds<4>::bytes <= 160 * 1024 && PreLds<4, kPreNarrowChunks>::bytes <= 96 * 1024, "LDS");

// v_smfmac_f32_32x32x32_f16 with the accumulator in AGPRs; ABID selects the index
// halfword.  Written as inline assembly because, for the intrinsic, the compiler
// splits the accumulator registers between VGPRs and AGPRs and copies them around
// the MFMAs.  Assembly takes the MFMA out of the compiler's hazard tracking, so the
// kernel keeps the gfx950 rules by construction: an operand VGPR written by a VALU
// instruction is read at least two instructions later (operands come from LDS
// loads, which s_waitcnt covers, or were produced a k-step earlier), and the
// accumulators are read only after pre_mfma_drain.
template <int ABID>
__device__ __forceinline__ void pre_smfmac(f32x16& c, half8_t a, half16_t b, uint32_t idx) {
  if constexpr (ABID == 0)
    asm volatile("v_smfmac_f32_32x32x32_f16 %0, %1, %2, %3" : "+a"(c) : "v"(a), "v"(b), "v"(idx));
  else
    asm volatile("v_smfmac_f32_32x32x32_f16 %0, %1, %2, %3 abid:1" : "+a"(c) : "v"(a), "v"(b), "v"(idx));
}

// Wait states between the last MFMA and the first read of its result.
__device__ __forceinline__ void pre_mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Start of a k-step: this wave's DMAs except the last NDMA issued have landed, its
// LDS reads are complete; then the workgroup meets.
template <int NDMA>
__device__ __forceinline__ void pre_step_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(NDMA) : "memory");
}

// First dequantization slice of MFMA region r of a k-step with nr regions: the 14
// slices of the next step's two k-blocks run in regions 2..nr-1, one per region with
// 16 regions, with 8 three or two per region (k-block 0 in regions 2-4, 1 in 5-7).
constexpr int pre_slice0(int nr, int r) {
  return r <= 2 ? 0 : nr == 16 ? r - 2 : r == 3 ? 3 : r == 4 ? 5 : r == 5 ? 7 : r == 6 ? 10 : r == 7 ? 12 : 14;
}
static_assert(pre_slice0(16, 16) == 14 && pre_slice0(8, 8) == 14, "every slice once");

// RG: 32-row B fragments per wave, i.e. a tile of 32 RG batch rows.  RG = 4 is the
// tile described above; RG = 2 (64 rows) doubles the tiles of a call for batches whose
// 128-row tiles leave CUs idle, at twice the dequantization per MFMA (each weight
// fragment feeds two B fragments instead of four: ~6.5 VALU per MFMA).
template <bool GROUPED, int RG, int CT>
__global__ __launch_bounds__(64 * CT, 1) void sm24_prefill_kernel(GemmArgs a) {
  static_assert(RG == 4 || RG == 2, "128- or 64-row tiles");
  static_assert(CT == kPreChunks || (CT == kPreNarrowChunks && RG == 4), "512- or (128-row) 256-column tiles");
  constexpr int MT = 32 * RG;
  constexpr int NF = 2 * RG;               // B fragments per k-step (two k-blocks)
  constexpr int NR = 2 * NF;               // MFMA regions per k-step
  constexpr int ADMA = 4 * RG / CT;        // activation DMA instructions per wave and k-step
  constexpr int NDMA = ADMA + (GROUPED ? 4 : 3);  // DMA instructions per wave and k-step
  constexpr int kPreActB = PreLds<RG, CT>::act_b, kPreWgtOff = PreLds<RG, CT>::wgt_off;
  constexpr int kPreWgtB = PreLds<RG, CT>::wgt_b;
  constexpr int PSTRIDE = 2048 * CT * RG;  // floats of one (tile, split) partial
  __shared__ __attribute__((aligned(16))) uint8_t lds[PreLds<RG, CT>::bytes];
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const uint32_t lbase = (uint32_t)(size_t)(lds_u8*)lds;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // chunk of this wave
  const int M = a.M, N = a.N, K = a.K;
  const int nks = K >> 6;  // even: the host requires K % 128 == 0

  // ---- split-K: block b = z * T + tile; split z covers the k-steps [ks0, ks1), an even
  // number (>= 8: the host keeps splits <= nks / 8) ----
  const int ntn = N / (64 * CT), ntm = (M + MT - 1) / MT;
  const int T = ntn * ntm;
  const int S = a.splits;
  const int z = blockIdx.x / T;
  const int ks0 = 2 * (int)(((long long)(nks >> 1) * z) / S);
  const int ks1 = 2 * (int)(((long long)(nks >> 1) * (z + 1)) / S);

  // ---- tile order: each XCD (block b on XCD b % 8) works through a contiguous range
  // of tiles, in supertiles of GN column tiles x GM row tiles (rows fastest), so that
  // the workgroups resident on one XCD share weights and activations in its L2. ----
  const int tile = blockIdx.x - z * T;
  int t = tile;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int GM = ntm >= 8 ? 8 : ntm;
  const int GN = 32 / GM;
  int tn, tm;
  if (ntm % GM == 0 && ntn % GN == 0) {
    const int st = t / (GN * GM), r = t % (GN * GM);
    const int sm = ntm / GM;
    tn = (st / sm) * GN + r / GM;
    tm = (st % sm) * GM + r % GM;
  } else {
    tn = t / ntm;
    tm = t % ntm;
  }
  const int c0 = tn * CT;         // first chunk of the tile
  const int m0 = tm * MT;         // first batch row
  const int cw = c0 + w;          // chunk of this wave

  // ---- DMA sources: per-lane byte offsets from per-k-step bases ----
  // activations: instruction u of wave w fills pieces 64(ADMA w + u) + lane of the
  // step's 256 RG 16-byte pieces; piece P = row P >> 3, physical slot P & 7, which
  // holds the logical slot (P & 7) ^ ((row >> 1) & 7).  Rows past M repeat row M-1
  // (never stored); the host keeps 2 M K + 4096 below 2^32.
  uint32_t act_v[ADMA];
#pragma unroll
  for (int u = 0; u < ADMA; u++) {
    const int p = 64 * (ADMA * w + u) + lane, row = p >> 3;
    const int ls = (p & 7) ^ ((row >> 1) & 7);
    const int m = m0 + row < M ? m0 + row : M - 1;
    // + 1024 (1 - u % 2): instructions go in pairs, the second of a pair carries
    // offset 1024, the base is lowered by 1024
    act_v[u] = ((uint32_t)m * (uint32_t)K + 8 * ls) * 2 + 1024 * (1 - (u & 1));
  }
  // packed values: k-block lane >> 5 of chunk cw; LDS slot s = lane & 31 holds the
  // 16-byte piece 4 g8 + t (words (g8, t, 0..3)) with s = g8 + 8 (t >> 1) + 16 (t & 1),
  // so that the two words a lane reads, (g8, 2h) and (g8, 2h + 1), lie 16 slots apart
  // and the 32 lanes of each half-wave hit 32 distinct banks
  const int wsl = lane & 31;
  const uint32_t wv_v = (lane >> 5) * 8 * (uint32_t)N + 512 * (uint32_t)cw +
                        16 * (4 * (wsl & 7) + 2 * ((wsl >> 3) & 1) + (wsl >> 4));
  // metadata (4 bytes per lane) of k-block 0 of chunk cw (base lowered by 1024), and
  // of k-block 1 (4N bytes on; instruction offset 1280)
  const uint32_t mt_v0 = 256 * (uint32_t)cw + 4 * lane;
  const uint32_t mt_v1 = mt_v0 + 4 * (uint32_t)N - 256;
  // scales (4 bytes per lane) of the chunk pair (cw & ~1, cw | 1) (base lowered by 1536)
  const uint32_t sc_v = 128 * (uint32_t)(cw & ~1) + 4 * lane;

  const char* gA1 = reinterpret_cast<const char*>(a.A) - 1024;
  const char* gB = static_cast<const char*>(a.B);
  const char* gM1 = static_cast<const char*>(a.meta) - 1024;
  const char* gS1 = reinterpret_cast<const char*>(a.s) - 1536;
  const uint32_t strB = 16 * (uint32_t)N, strM = 8 * (uint32_t)N, strS = 2 * (uint32_t)N;

  // DMA group g of local k-step s (clamped to the split's last) into ring slot q:
  // g = 0 this wave's share of the step's activation rows (ADMA instructions), g = 1 the
  // weight side of its chunk (packed values, metadata of both k-blocks, and the
  // scales of its chunk pair when grouped).  Step offsets are 32-bit: the host keeps
  // K N / 4 below 2^32.
  auto dma = [&](int s, int q, int g) {
    const uint32_t sc = (uint32_t)(ks0 + s < ks1 ? ks0 + s : ks1 - 1);
    if (g == 0) {
      const uint32_t la = lbase + kPreActOff + q * kPreActB + 1024 * ADMA * w;
      if constexpr (ADMA == 1) {
        dma16x1(la, act_v[0], gA1 + 128 * sc);
      } else {
#pragma unroll
        for (int u = 0; u < ADMA; u += 2) {
          const uint32_t pair[2] = {act_v[u], act_v[u + 1]};
          dma16x2(la + 1024 * u, pair, gA1 + 128 * sc);
        }
      }
    } else {
      const uint32_t l = lbase + kPreWgtOff + q * kPreWgtB + kPreWgtW * w;
      if constexpr (GROUPED)
        dma_chunk(l, wv_v, gB + sc * strB, mt_v0, mt_v1, gM1 + sc * strM, sc_v, gS1 + (sc >> 1) * strS);
      else
        dma_chunk_nos(l, wv_v, gB + sc * strB, mt_v0, mt_v1, gM1 + sc * strM);
    }
  };

  // ---- this lane's MFMA roles ----
  const int rho = lane & 31, h = lane >> 5;
  const int g8 = rho >> 2, j = rho & 3;
  const int swz = (rho >> 1) & 7;
  // B fragment (kb, rg): row 32rg + rho, logical slots 4kb + 2h + {0, 1}
  uint32_t b_off[2][2];
#pragma unroll
  for (int kb = 0; kb < 2; kb++)
#pragma unroll
    for (int i = 0; i < 2; i++) b_off[kb][i] = kPreActOff + rho * 128 + 16 * ((4 * kb + 2 * h + i) ^ swz);
  const uint32_t wblk = kPreWgtOff + kPreWgtW * w;
  // packed words (kb, t = 2h) and (kb, 2h + 1) of column pair (8g8 + j, +4): slots
  // g8 + 8h and g8 + 8h + 16 (+ 256 bytes) of k-block kb's 512 bytes
  const uint32_t w_rd = wblk + 16 * (g8 + 8 * h) + 4 * j;
  // metadata unit of the column pair in k-block kb's 256 bytes
  const uint32_t m_rd = wblk + 1024 + 8 * (16 * (j >> 1) + 2 * g8 + (j & 1));
  // scales of columns 8g8 + j (+4): slots 8g8 + 2j, + 1 of this chunk's 128 bytes
  const uint32_t s_rd = wblk + 1536 + 128 * (cw & 1) + 16 * g8 + 4 * j;
  // index halfwords of both halves: [d0.b(h), d1.b(h), d0.b(2+h), d1.b(2+h)]
  const uint32_t isel = h ? 0x07030501u : 0x06020400u;

  uint32_t kMask, kMagic, kMaskHi;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));

  half8_t av[2][2][2];  // [parity][kb][hf] dequantized weight fragments
  uint32_t ix[2][2];    // [parity][kb] index halfwords (hf = abid)
  half16_t bv[4];       // B fragments, ring by fragment number kb*RG + rg
  f32x16 acc[RG][2];    // [rg][hf]
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      acc[rg][hf] = (f32x16){};
      asm volatile("" : "+a"(acc[rg][hf]));
    }

  auto read_b = [&](int q, int f) -> half16_t {
    const int kb = f / RG, rg = f % RG;
    const uint8_t* p0 = lds + b_off[kb][0] + q * kPreActB + rg * 4096;
    const uint8_t* p1 = lds + b_off[kb][1] + q * kPreActB + rg * 4096;
    const half8_t lo = *reinterpret_cast<const half8_t*>(p0);
    const half8_t hi = *reinterpret_cast<const half8_t*>(p1);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  };

  // raw operands of the next k-step's dequantization, per k-block
  uint32_t rw[2][2];  // packed words t = 2h, 2h + 1
  u32x2 rm[2];        // metadata unit
  uint32_t rs = 0;    // scales of columns (8g8 + j, + 4)
  auto read_raw = [&](int q, int kb) {
    const uint8_t* pw = lds + w_rd + q * kPreWgtB + 512 * kb;
    rw[kb][0] = *reinterpret_cast<const uint32_t*>(pw);
    rw[kb][1] = *reinterpret_cast<const uint32_t*>(pw + 256);
    rm[kb] = *reinterpret_cast<const u32x2*>(lds + m_rd + q * kPreWgtB + 256 * kb);
  };
  auto read_scales = [&](int q) {
    if constexpr (GROUPED) rs = *reinterpret_cast<const uint32_t*>(lds + s_rd + q * kPreWgtB);
  };

  // ---- dequantization of k-block kb into av[par][kb][hf], ix[par][kb], in seven
  // slices of at most four VALU instructions: word halves -> magic-number halves
  // 1024 + q (low nibbles) or 1024 + 16q (high nibbles) -> q - 8 -> times scale ----
  uint32_t dx[2][4];
  half2_t dp[2][4];
  auto dq_slice = [&](int kb, int sl, int par) {
    const half2_t k1032 = {(_Float16)1032.f, (_Float16)1032.f};
    const half2_t k16th = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2_t km72 = {(_Float16)-72.f, (_Float16)-72.f};
    const uint32_t w0 = rw[kb][0], w1 = rw[kb][1];
    const half2_t scv = __builtin_bit_cast(half2_t, rs);
    auto scl = [&](int hf, int i) {
      if constexpr (GROUPED) {
        const _Float16 sv = hf ? scv.y : scv.x;
        dp[hf][i] = dp[hf][i] * (half2_t){sv, sv};
      }
    };
    switch (sl) {
      case 0:
        dx[1][0] = w0 >> 8;  // (shifted words, turned into halves in the next slice)
        dx[1][1] = w1 >> 8;
        dx[0][0] = (w0 & kMask) | kMagic;
        dx[0][1] = (w1 & kMask) | kMagic;
        break;
      case 1:
        dx[0][2] = (w0 & kMaskHi) | kMagic;
        dx[0][3] = (w1 & kMaskHi) | kMagic;
        dx[1][2] = (dx[1][0] & kMaskHi) | kMagic;
        dx[1][3] = (dx[1][1] & kMaskHi) | kMagic;
        break;
      case 2:
        dx[1][0] = (dx[1][0] & kMask) | kMagic;
        dx[1][1] = (dx[1][1] & kMask) | kMagic;
        dp[0][0] = __builtin_bit_cast(half2_t, dx[0][0]) - k1032;
        dp[0][1] = __builtin_bit_cast(half2_t, dx[0][1]) - k1032;
        break;
      case 3:
        dp[0][2] = __builtin_bit_cast(half2_t, dx[0][2]) * k16th + km72;
        dp[0][3] = __builtin_bit_cast(half2_t, dx[0][3]) * k16th + km72;
        dp[1][0] = __builtin_bit_cast(half2_t, dx[1][0]) - k1032;
        dp[1][1] = __builtin_bit_cast(half2_t, dx[1][1]) - k1032;
        break;
      case 4:
        dp[1][2] = __builtin_bit_cast(half2_t, dx[1][2]) * k16th + km72;
        dp[1][3] = __builtin_bit_cast(half2_t, dx[1][3]) * k16th + km72;
        scl(0, 0);
        scl(0, 1);
        break;
      case 5:
        scl(0, 2);
        scl(0, 3);
        scl(1, 0);
        scl(1, 1);
        break;
      default:
        scl(1, 2);
        scl(1, 3);
        ix[par][kb] = __builtin_amdgcn_perm(rm[kb].y, rm[kb].x, isel);
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
          av[par][kb][hf] = (half8_t){dp[hf][0].x, dp[hf][0].y, dp[hf][1].x, dp[hf][1].y,
                                      dp[hf][2].x, dp[hf][2].y, dp[hf][3].x, dp[hf][3].y};
        break;
    }
  };

  // ---- k-step s in ring slot Q = s & 3 (slot Q+1: step s+1, slot Q+3: step s+3):
  //   barrier: this wave's DMAs of step s+1 have landed, every wave has finished step
  //   s-1 (its reads of slot Q+3);
  //   NR = 4 RG regions r = (kb, rg, hf), each one MFMA plus a share of: DMA group
  //   r >> 1 of step s+3 (r = 1, 3); at hf = 0 the read of B fragment f+3 (f = RG kb +
  //   rg; from step s+1 past NF-1; its ring slot held fragment f-1, used up by then);
  //   at r < 2 the raw words and metadata of step s+1, k-block r, and at r = 2 its
  //   scales; at r >= 2 the slices [pre_slice0(r), pre_slice0(r+1)) of dequantizing
  //   step s+1 (slice i: slice i % 7 of k-block i / 7).
  // Steps past the last are skipped (uniform); the DMAs are clamped, so the vmcnt of
  // every barrier counts exactly the DMAs of one step. ----
  auto step = [&](int s, auto qc) {
    constexpr int Q = decltype(qc)::value, P = Q & 1, QN = (Q + 1) & 3, QD = (Q + 3) & 3;
    pre_step_barrier<NDMA>();
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const int kb = r / (2 * RG), rg = (r >> 1) % RG, hf = r & 1, f = r >> 1;
      if (hf) pre_smfmac<1>(acc[rg][hf], av[P][kb][hf], bv[f & 3], ix[P][kb]);
      else pre_smfmac<0>(acc[rg][hf], av[P][kb][hf], bv[f & 3], ix[P][kb]);
      __builtin_amdgcn_sched_barrier(0);  // the region's work follows its MFMA
      if (hf == 0) bv[(f + 3) & 3] = read_b(f + 3 < NF ? Q : QN, (f + 3) % NF);
      if (r == 1 || r == 3) dma(s + 3, QD, r >> 1);
      if (r < 2) read_raw(QN, r);
      if (r == 2) read_scales(QN);
#pragma unroll
      for (int i = pre_slice0(NR, r); i < pre_slice0(NR, r + 1); i++) dq_slice(i / 7, i % 7, P ^ 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- prologue: DMAs of steps 0..2, then step 0's operands dequantized and its first
  // three B fragments read ----
#pragma unroll
  for (int s = 0; s < 3; s++)
#pragma unroll
    for (int g = 0; g < 2; g++) dma(s, s, g);
  pre_step_barrier<NDMA>();
#pragma unroll
  for (int kb = 0; kb < 2; kb++) read_raw(0, kb);
  read_scales(0);
#pragma unroll
  for (int kb = 0; kb < 2; kb++)
#pragma unroll
    for (int sl = 0; sl < 7; sl++) dq_slice(kb, sl, 0);
  bv[0] = read_b(0, 0);
  bv[1] = read_b(0, 1);
  bv[2] = read_b(0, 2);
  __builtin_amdgcn_sched_barrier(0);

  const int nls = ks1 - ks0;  // k-steps of this split (even)
  for (int s = 0; s < nls; s += 4) {
    step(s, IntC<0>{});
    step(s + 1, IntC<1>{});
    if (s + 2 < nls) {
      step(s + 2, IntC<2>{});
      step(s + 3, IntC<3>{});
    }
  }
  // DMAs of (clamped) steps past the last may still be landing in LDS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  pre_mfma_drain();
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int hf = 0; hf < 2; hf++) asm volatile("" : "+a"(acc[rg][hf]));

  // ---- split-K hand-off: the partial tile goes to uncached scratch in register order
  // ([tile][split][wave][rg][hf][i][lane] float4s, 64 RG KiB per tile and split); the
  // last split to arrive at the tile's counter reads all splits back and adds them in
  // split order (so the result is bit-identical from run to run, whichever split comes
  // last), writes C and resets the counter.  Each thread's stores complete before the
  // workgroup barrier; the counter is bumped after it. ----
  const float* const pbase = a.partial + ((size_t)tile * S) * PSTRIDE + (size_t)w * (2048 * RG) + 4 * lane;
  if (S > 1) {
    float* const pmine = a.partial + ((size_t)tile * S + z) * PSTRIDE + (size_t)w * (2048 * RG) + 4 * lane;
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
      if (m0 + 32 * rg >= M) break;  // 32-row blocks past M are never read back (uniform)
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          *reinterpret_cast<float4_t*>(pmine + ((rg * 2 + hf) * 4 + i) * 256) =
              (float4_t){acc[rg][hf][4 * i], acc[rg][hf][4 * i + 1], acc[rg][hf][4 * i + 2], acc[rg][hf][4 * i + 3]};
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
  // ---- epilogue: lane (rho, h) holds, for batch row m0 + 32rg + rho, the columns
  // 64cw + 16q + 8h + 4hf + i in register 4q + i of acc[rg][hf]: eight consecutive
  // columns per (rg, q).  With split-K the float4 (hf, q) of the sum is read back
  // from every split, in split order, two splits' 8 float4s per batch of loads: the
  // uncached reads are latency-bound, so each batch keeps 16 loads in flight. ----
#pragma unroll
  for (int rg = 0; rg < RG; rg++) {
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
        for (int k = 0; k < 8; k++) t0[k] = *reinterpret_cast<const float4_t*>(p + k * 256 + (size_t)zz * PSTRIDE);
        if (two) {
#pragma unroll
          for (int k = 0; k < 8; k++)
            t1[k] = *reinterpret_cast<const float4_t*>(p + k * 256 + (size_t)(zz + 1) * PSTRIDE);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) v[k >> 2][k & 3] += t0[k];
        if (two) {
#pragma unroll
          for (int k = 0; k < 8; k++) v[k >> 2][k & 3] += t1[k];
        }
      }
    }
    const int m = m0 + 32 * rg + rho;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int n = 64 * cw + 16 * q + 8 * h;
      const float4_t v0 = v[0][q], v1 = v[1][q];
      half8_t o = {(_Float16)v0.x, (_Float16)v0.y, (_Float16)v0.z, (_Float16)v0.w,
                   (_Float16)v1.x, (_Float16)v1.y, (_Float16)v1.z, (_Float16)v1.w};
      if constexpr (!GROUPED) o = o * *reinterpret_cast<const half8_t*>(a.s + n);
      if (m < M) *reinterpret_cast<half8_t*>(a.C + (size_t)m * N + n) = o;
    }
  }
}

}  // namespace sm24
