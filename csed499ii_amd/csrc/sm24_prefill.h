// Prefill-sized (large M) 2:4 INT4 x FP16 GEMM for gfx950, MFMA-bound.
//
// Workgroup tile: 512 output columns (8 chunks of 64) x 128 batch rows, 4 waves; wave
// w owns chunks 2w, 2w+1 (128 columns) for all 128 rows, so every wave holds
// 2 chunks x 4 fragments x 8 batch blocks of v_smfmac_f32_16x16x64_f16 accumulators
// (256 registers).  K advances in steps of 64 (two 32-deep k-blocks).
//
// Operand routes, chosen for the per-CU budgets measured on MI355X (LDS ~128 B/clk,
// ~16 cycles per 16-byte load instruction, 16 cycles per smfmac):
//  * activations: cooperative 16-byte loads -> registers -> LDS (two buffers), each
//    row stored in the MFMA's k order; every wave reads its 8 B fragments once per
//    k-step and uses each with 8 weight fragments;
//  * packed values: straight from global into registers, one 16-byte load per lane,
//    chunk and k-block (covering the lane's 4 fragments), two k-steps ahead;
//  * metadata: cooperative 8-byte loads of both k-blocks' units, transposed once per
//    column into the index halfword each lane needs (an LDS table of 4 KiB);
//  * scales: one 16-byte load per lane and chunk (the 4 fragments' scales).
//
// MFMA k order.  Within a 64-deep k-step, A lane group h holds MFMA groups 4h..4h+3
// = real groups (k-block 0, group h), (0, h+4), (1, h), (1, h+4): exactly the
// nibbles of the packed word (k-block, g8, t = h, j) for one column.  Activation
// rows are stored permuted the same way (real group (kb, g) at MFMA group
// g < 4 ? 4g + 2kb : 4(g-4) + 1 + 2kb), so a B lane's k-ranges [8h, 8h+8) and
// [32+8h, 32+8h+8) are 16 contiguous bytes each.
//
// Fragment f (0..3) of a chunk holds columns 8*g8 + 4*blk + f, row rho = 2*g8 + blk,
// so a lane's four fragments read four consecutive packed words (j = f).
#pragma once
#include "sm24_device.h"

namespace sm24 {

template <int V>
struct IntC {
  static constexpr int value = V;
};

constexpr int kPreRows = 128;   // batch rows per tile
constexpr int kPreChunks = 8;   // 64-column chunks per tile
static_assert(64 * kPreChunks == kPreTileCols, "tile width");
constexpr int kPreRS = 144;     // LDS bytes per activation row (128 + 16: conflict-free b128 reads)

// Real group (kb, g) of a 64-deep k-step -> MFMA group.
__device__ __forceinline__ int pre_mgroup(int kb, int g) { return g < 4 ? 4 * g + 2 * kb : 4 * (g - 4) + 1 + 2 * kb; }

// 4x4 nibble transpose of the metadata of one column pair.  x0, y0: k-block 0 words
// {m(n,e0) | m(n+4,e0) << 16}, {m(n,e1) | m(n+4,e1) << 16}; x1, y1: k-block 1.
// Returns, for column n (lo) and n+4 (hi), the index halfwords of lane groups h = 0..3:
// idx_h = m(kb0,e0)[h] | m(kb0,e1)[h] << 4 | m(kb1,e0)[h] << 8 | m(kb1,e1)[h] << 12.
__device__ __forceinline__ void pre_meta_transpose(uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1,
                                                   u32x2& lo, u32x2& hi) {
  // even / odd nibbles to separate bytes, then pair the e0/e1 nibbles of a byte
  const uint32_t ab_e = (x0 & 0x0F0F0F0Fu) | ((y0 & 0x0F0F0F0Fu) << 4);         // [h0, h2, h0', h2'] of kb0
  const uint32_t ab_o = ((x0 >> 4) & 0x0F0F0F0Fu) | (y0 & 0xF0F0F0F0u);         // [h1, h3, h1', h3'] of kb0
  const uint32_t cd_e = (x1 & 0x0F0F0F0Fu) | ((y1 & 0x0F0F0F0Fu) << 4);
  const uint32_t cd_o = ((x1 >> 4) & 0x0F0F0F0Fu) | (y1 & 0xF0F0F0F0u);
  // halfword h of column n = [ab byte, cd byte] with byte h/2 of the even (h even)
  // or odd (h odd) word; v_perm_b32 selector bytes: 0-3 = second operand, 4-7 = first.
  const uint32_t e = __builtin_amdgcn_perm(cd_e, ab_e, 0x05010400u);  // [ab_e.b0, cd_e.b0, ab_e.b1, cd_e.b1]
  const uint32_t o = __builtin_amdgcn_perm(cd_o, ab_o, 0x05010400u);
  const uint32_t e2 = __builtin_amdgcn_perm(cd_e, ab_e, 0x07030602u);  // bytes 2, 3: column n+4
  const uint32_t o2 = __builtin_amdgcn_perm(cd_o, ab_o, 0x07030602u);
  // words: [h0 | h1 << 16, h2 | h3 << 16]
  lo.x = __builtin_amdgcn_perm(o, e, 0x05040100u);
  lo.y = __builtin_amdgcn_perm(o, e, 0x07060302u);
  hi.x = __builtin_amdgcn_perm(o2, e2, 0x05040100u);
  hi.y = __builtin_amdgcn_perm(o2, e2, 0x07060302u);
}

template <bool GROUPED>
__global__ __launch_bounds__(256, 1) void sm24_prefill_kernel(GemmArgs a) {
  constexpr int MT = kPreRows, CT = kPreChunks, RS = kPreRS;
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][MT * RS];
  __shared__ __attribute__((aligned(16))) uint16_t lds_i[2][CT * 4 * 16 * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = a.M, N = a.N, K = a.K;
  const int nks = K >> 6;

  // ---- tile order: each XCD (block b on XCD b % 8) works through a contiguous range
  // of tiles, in supertiles of GN column tiles x GM row tiles (rows fastest), so that
  // the workgroups resident on one XCD share weights and activations in its L2. ----
  const int ntn = N / (64 * CT), ntm = (M + MT - 1) / MT;
  const int T = ntn * ntm;
  int t = blockIdx.x;
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
  const int c0 = tn * CT;  // first chunk of the tile
  const int m0 = tm * MT;  // first batch row

  // ---- cooperative activation pieces: p = tid + 256q -> row p>>3, 16-byte piece p&7 ----
  const _Float16* arow[4];
  uint32_t aoff0[4], aoff1[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int p = tid + 256 * q, r = p >> 3, u = p & 7;
    const int m = m0 + r < M ? m0 + r : M - 1;  // rows past M repeat row M-1 (never stored)
    arow[q] = a.A + (size_t)m * K + 8 * u;
    const int kb = u >> 2, g = 2 * (u & 3);
    aoff0[q] = r * RS + 8 * pre_mgroup(kb, g);
    aoff1[q] = r * RS + 8 * pre_mgroup(kb, g + 1);
  }
  // ---- cooperative metadata units: chunk tid>>5, unit tid&31 (both k-blocks) ----
  const int mq = tid & 31, mcc = tid >> 5;
  const uint8_t* mbase = static_cast<const uint8_t*>(a.meta) + 256 * (size_t)(c0 + mcc) + 8 * mq;
  const size_t mrow = 4 * (size_t)N;  // bytes per k-block row of metadata
  const int mj = 2 * (mq >> 4) + (mq & 1), mg8 = (mq >> 1) & 7;
  const uint32_t ioff = (((mcc * 4 + mj) * 16 + 2 * mg8) * 4) * 2;  // byte offset of [rho=2g8][h=0]

  // ---- this lane's MFMA roles ----
  const int rho = lane & 15, h = lane >> 4;
  const int g8 = rho >> 1, blk = rho & 1;
  const uint32_t vsh = 8u * blk;
  // packed values of chunk cl, k-block kb of k-step s: 16 bytes (words j = 0..3)
  const uint8_t* vbase = static_cast<const uint8_t*>(a.B) + 512 * (size_t)(c0 + 2 * wave) + 4 * (16 * g8 + 4 * h);
  const size_t vrow = 8 * (size_t)N;  // bytes per k-block row of values
  // scales of chunk cl: 16 bytes at slot 8*g8 (halves blk + 2f)
  const uint8_t* sbase = reinterpret_cast<const uint8_t*>(a.s) + 2 * (64 * (size_t)(c0 + 2 * wave) + 8 * g8);
  const size_t srow = 2 * (size_t)N;
  const uint32_t bofs = (uint32_t)rho * RS + 16 * h;                   // B fragment bf: + 16*bf*RS
  const uint32_t iofs = ((((2 * wave) * 4) * 16 + rho) * 4 + h) * 2;   // idx of chunk cl, fragment f: + (cl*4+f)*128

  uint32_t kMask, kMagic, kMaskHi;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));

  auto clampk = [&](int s) { return s < nks ? s : nks - 1; };
  u32x4 ast[4];          // activation staging (next k-step)
  u32x2 mst0, mst1;      // metadata staging (k-blocks 0 and 1)
  u32x4 vreg[2][2][2];   // [ring slot][chunk][k-block] packed values
  u32x4 sreg[2][2];      // [ring slot][chunk] scales
  auto load_stage = [&](int s) {
    const int sc = clampk(s);
#pragma unroll
    for (int q = 0; q < 4; q++) ast[q] = *reinterpret_cast<const u32x4*>(arow[q] + 64 * sc);
    mst0 = *reinterpret_cast<const u32x2*>(mbase + (size_t)(2 * sc) * mrow);
    mst1 = *reinterpret_cast<const u32x2*>(mbase + (size_t)(2 * sc + 1) * mrow);
  };
  auto load_weights = [&](int s, int slot) {
    const int sc = clampk(s);
#pragma unroll
    for (int cl = 0; cl < 2; cl++) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
        vreg[slot][cl][kb] = *reinterpret_cast<const u32x4*>(vbase + 512 * cl + (size_t)(2 * sc + kb) * vrow);
      if constexpr (GROUPED)
        sreg[slot][cl] = *reinterpret_cast<const u32x4*>(sbase + 128 * cl + (size_t)(sc >> 1) * srow);
    }
  };
  auto write_stage = [&](int buf) {
    uint8_t* la = lds_a[buf];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      *reinterpret_cast<u32x2*>(la + aoff0[q]) = (u32x2){ast[q].x, ast[q].y};
      *reinterpret_cast<u32x2*>(la + aoff1[q]) = (u32x2){ast[q].z, ast[q].w};
    }
    u32x2 lo, hi;
    pre_meta_transpose(mst0.x, mst0.y, mst1.x, mst1.y, lo, hi);
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint8_t*>(lds_i[buf]) + ioff) = (u32x4){lo.x, lo.y, hi.x, hi.y};
  };

  float4_t acc[2][4][8];
#pragma unroll
  for (int cl = 0; cl < 2; cl++)
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
      for (int bf = 0; bf < 8; bf++) acc[cl][f][bf] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // buf / slot are compile-time (the k-loop is unrolled by two): a runtime ring index
  // would turn every register access into indexed moves with full waits.  The eight
  // weight fragments are dequantized first (32 registers); the activation fragments
  // are then streamed from LDS, each used by all eight.
  auto compute = [&](auto par) {
    constexpr int buf = decltype(par)::value, slot = buf;
    const uint8_t* la = lds_a[buf];
    const uint8_t* li = reinterpret_cast<const uint8_t*>(lds_i[buf]);
    uint32_t idxs[2][4];
#pragma unroll
    for (int cl = 0; cl < 2; cl++)
#pragma unroll
      for (int f = 0; f < 4; f++) idxs[cl][f] = *reinterpret_cast<const uint16_t*>(li + iofs + (cl * 4 + f) * 128);
    half8_t av[2][4];
#pragma unroll
    for (int cl = 0; cl < 2; cl++) {
#pragma unroll
      for (int f = 0; f < 4; f++) {
        const uint32_t w0 = vreg[slot][cl][0][f] >> vsh;
        const uint32_t w1 = vreg[slot][cl][1][f] >> vsh;
        const half2_t p0 = __builtin_bit_cast(half2_t, (w0 & kMask) | kMagic) - (half2_t){(_Float16)1032.f, (_Float16)1032.f};
        const half2_t p1 = __builtin_bit_cast(half2_t, (w0 & kMaskHi) | kMagic) * (half2_t){(_Float16)0.0625f, (_Float16)0.0625f} +
                           (half2_t){(_Float16)-72.f, (_Float16)-72.f};
        const half2_t p2 = __builtin_bit_cast(half2_t, (w1 & kMask) | kMagic) - (half2_t){(_Float16)1032.f, (_Float16)1032.f};
        const half2_t p3 = __builtin_bit_cast(half2_t, (w1 & kMaskHi) | kMagic) * (half2_t){(_Float16)0.0625f, (_Float16)0.0625f} +
                           (half2_t){(_Float16)-72.f, (_Float16)-72.f};
        av[cl][f] = (half8_t){p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
        if constexpr (GROUPED) {
          const uint32_t sw = sreg[slot][cl][f] >> (16 * blk);
          const _Float16 sc = __builtin_bit_cast(half2_t, sw).x;
          av[cl][f] = av[cl][f] * (half8_t){sc, sc, sc, sc, sc, sc, sc, sc};
        }
      }
    }
#pragma unroll
    for (int bf = 0; bf < 8; bf++) {
      const half8_t lo = *reinterpret_cast<const half8_t*>(la + bofs + 16 * bf * RS);
      const half8_t hi = *reinterpret_cast<const half8_t*>(la + bofs + 16 * bf * RS + 64);
      const half16_t bv = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
#pragma unroll
      for (int cl = 0; cl < 2; cl++)
#pragma unroll
        for (int f = 0; f < 4; f++) acc[cl][f][bf] = smfmac64<0>(av[cl][f], bv, acc[cl][f][bf], idxs[cl][f]);
    }
  };

  // ---- pipeline: k-step s computes from LDS buffer / weight slot s & 1 while the
  // activations and metadata of s+1 are written to the other buffer and those of s+2
  // and the weights of s+2 are loaded.  Loads are unconditional (clamped to the last
  // k-step), so the compiler's waits stay exact; the loop is unrolled by two. ----
  auto step = [&](int s, auto par) {
    constexpr int P = decltype(par)::value;
    __syncthreads();
    if (s + 1 < nks) write_stage(P ^ 1);  // uniform
    load_stage(s + 2);
    if (s < nks) compute(par);            // uniform: false only after an odd k-step count
    load_weights(s + 2, P);
  };
  load_stage(0);
  load_weights(0, 0);
  load_weights(1, 1);
  write_stage(0);
  load_stage(1);
  for (int s = 0; s < nks; s += 2) {
    step(s, IntC<0>{});
    step(s + 1, IntC<1>{});
  }

  // ---- epilogue: lane (mcol = rho, h) holds rows 4h+i of every fragment, i.e. for
  // chunk cl and batch block bf the 16 columns 64c + 16h + [0, 16) (f fastest) of
  // batch row m0 + 16*bf + rho ----
#pragma unroll
  for (int cl = 0; cl < 2; cl++) {
    const int n = 64 * (c0 + 2 * wave + cl) + 16 * h;
    half8_t sc0 = {}, sc1 = {};
    if constexpr (!GROUPED) {
      sc0 = *reinterpret_cast<const half8_t*>(a.s + n);
      sc1 = *reinterpret_cast<const half8_t*>(a.s + n + 8);
    }
#pragma unroll
    for (int bf = 0; bf < 8; bf++) {
      const int m = m0 + 16 * bf + rho;
      half8_t o0, o1;
#pragma unroll
      for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int f = 0; f < 4; f++) {
          const int e = 4 * i + f;  // column n + e
          _Float16 v = (_Float16)acc[cl][f][bf][i];
          if constexpr (!GROUPED) v = v * (e < 8 ? sc0[e & 7] : sc1[e & 7]);
          if (e < 8) o0[e] = v;
          else o1[e - 8] = v;
        }
      }
      if (m < M) {
        _Float16* cp = a.C + (size_t)m * N + n;
        *reinterpret_cast<half8_t*>(cp) = o0;
        *reinterpret_cast<half8_t*>(cp + 8) = o1;
      }
    }
  }
}

}  // namespace sm24
