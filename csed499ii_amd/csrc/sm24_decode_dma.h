// Decode-sized 2:4 INT4 x FP16 GEMM for gfx950 at 16 and 32 padded batch rows (9-32
// rows per launch), fed by LDS-DMA.
//
// Work decomposition as the register-ring decode kernel (sm24_decode.h): one
// workgroup owns TC output columns (16, 32 or 64) over the whole K or over one K
// split; wave w of a stage of KS = NW * KPW k-blocks computes k-blocks
// [w * KPW, (w + 1) * KPW) for all the tile's columns, and the waves' partial sums
// are reduced in LDS at the end.
//
// Operand path.  Every stage of a wave lands in one of the wave's D LDS stage
// buffers through global_load_lds_dwordx4: the stage's P pieces of 16 bytes (packed
// values, metadata, the scales of the wave's one scale group and 4 pieces per batch
// row and k-block of activations, in the LDS order of sm24_decode_kernel's stage),
// 64 to an instruction, lane l of slot q moving piece 64 q + l.  Each lane keeps the
// 64-bit source of its piece in every slot, set up once at entry and advanced by one
// stage (one add) after each issue; the last slot's surplus lanes are masked off
// (EXEC) for its instruction.  Nothing is held in registers in flight, so the ring
// runs deeper than the register ring at 16 and 32 rows.  A stage that runs past K
// (the last stage of a K not a multiple of KS) moves the weight pieces of k-blocks
// past the last one back to the last one (rows that exist) and reads the zero block
// for their activation pieces, so that those k-blocks add nothing; stages past the
// split's end are not issued.
//
// Synchronisation.  A wave waits for its own DMAs with s_waitcnt vmcnt (they are
// counted like loads, in order), reads the stage's operands back from LDS, and
// refills the buffer D stages later; no workgroup barrier runs between stages.
// The LDS layout of a stage equals the register-ring kernel's, so the MFMA lane
// roles and the dequantisation are the same (see sm24_decode.h).
#pragma once
#include "sm24_decode.h"

namespace sm24 {

// 16 bytes per lane for lanes [0, n) from the lane's 64-bit address src into LDS at
// m0 + 16 * lane (global_load_lds_dwordx4); lanes >= n are masked off for the
// instruction only (the caller runs with every lane active: EXEC is all ones again
// afterwards).  `lds` is the wave-uniform LDS byte address.
template <int n>
__device__ __forceinline__ void dma_lanes_v(uint32_t lds, const void* src) {
  static_assert(n >= 1 && n <= 64, "one instruction moves at most 64 pieces");
  if constexpr (n == 64) {
    asm volatile(
        "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off" ::"s"(lds),
        "v"(src)
        : "memory", "m0");
  } else {
    constexpr uint32_t lo = n >= 32 ? 0xffffffffu : (uint32_t)((1ull << n) - 1);
    constexpr uint32_t hi = n <= 32 ? 0u : (uint32_t)((1ull << (n - 32)) - 1);
    asm volatile(
        "s_mov_b32 exec_lo, %2\n\t"
        "s_mov_b32 exec_hi, %3\n\t"
        "s_mov_b32 m0, %0\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b64 exec, -1" ::"s"(lds),
        "v"(src), "i"(lo), "i"(hi)
        : "memory", "m0");
  }
}

// Waits until at most min(k, KMAX) * L of the wave's vector memory operations are in
// flight (k uniform, >= 0): k stages of L instructions each.
template <int L, int KMAX>
__device__ __forceinline__ void wait_stages(int k) {
  static_assert(L * KMAX <= 63, "vmcnt counts to 63");
  if (k >= KMAX) {
    wait_vm<L * KMAX>();
    return;
  }
  switch (k) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<L * cmin(1, KMAX)>(); break;
    case 2: wait_vm<L * cmin(2, KMAX)>(); break;
    case 3: wait_vm<L * cmin(3, KMAX)>(); break;
    case 4: wait_vm<L * cmin(4, KMAX)>(); break;
    case 5: wait_vm<L * cmin(5, KMAX)>(); break;
    case 6: wait_vm<L * cmin(6, KMAX)>(); break;
    default: wait_vm<L * cmin(7, KMAX)>(); break;
  }
}

// Compile-time loop: f(IC<I>{}) for I in [I0, I1).
template <int I>
struct IC {
  static constexpr int value = I;
};
template <int I0, int I1, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < I1) {
    f(IC<I0>{});
    static_for<I0 + 1, I1>(f);
  }
}

template <int TC, int NW, int MB, bool GROUPED, int VF, int MF, bool DEEP>
__global__ __launch_bounds__(64 * NW) void sm24_decode_dma_kernel(const void* B_, const void* meta_, const void* s_,
                                                                  const void* A_, const void* zeros_, int M_, int N_,
                                                                  int K_, int splits_, GemmArgs a_) {
  const GemmArgs a = with_lead(a_, B_, meta_, s_, A_, zeros_, M_, N_, K_, splits_);
  constexpr int NCB = TC / 16;                           // 16-column MFMA blocks per tile
  constexpr int KPW = cmax(2, 64 / TC);                  // k-blocks per wave per stage (pairs)
  constexpr int KS = KPW * NW;                           // k-blocks per stage
  constexpr int BPK = VF == VAL4 ? TC / 2 : 3 * TC / 8;   // 16-byte value pieces per k-block
  constexpr int MPK = (MF == META3 && TC == 64) ? 12 : TC / 4;
  constexpr int SPG = TC / 8;                            // 16-byte scale pieces per scale group
  static_assert(MB == 16 || MB == 32, "16 or 32 padded batch rows: every operand lane is a batch row");
  constexpr int RB = MB > 16 ? MB / 16 : 1;              // 16-row batch blocks (MFMA B operands)
  constexpr int NB = KPW * BPK;
  constexpr int NM = KPW * MPK;
  constexpr int NSC = GROUPED ? SPG : 0;
  constexpr int NPA = KPW * 4 * MB;                      // activation pieces (4 per row and k-block)
  static_assert(NB <= 64 && NM <= 64, "values and metadata of a stage fit one instruction each");
  constexpr int MOFF = NB * 16, SOFF = MOFF + NM * 16, AOFF = SOFF + NSC * 16;
  constexpr int STAGE = AOFF + NPA * 16;                 // bytes of one wave's stage
  constexpr int P1 = NB + NM, P2 = P1 + NSC, P = P2 + NPA;  // pieces of a wave's stage
  constexpr int L = (P + 63) / 64;                       // DMA instructions (slots) per stage
  constexpr int LAST = P - 64 * (L - 1);                 // pieces of the last slot
  static_assert(KPW <= 4 && 4 % KPW == 0, "a wave's k-blocks lie in one scale group");
  static_assert(KS % 4 == 0, "scale groups of 4 k-blocks per stage");
  // Ring depth: stages in flight per wave.  Up to 4 while the workgroup's ring stays
  // within 32 KiB of LDS (more workgroups per CU where a stage is large: 16-row
  // 64-column tiles run two stages), up to 8 for DEEP (long K per split), and within
  // the 6-bit vmcnt.
  constexpr int D = cmax(2, cmin(DEEP ? 8 : 4, cmin((DEEP ? 64 : 32) * 1024 / (NW * STAGE), 60 / L)));
  constexpr int REDP = TC + 4;
  constexpr int REDB = NW * 16 * REDP * 4;
  constexpr int RING = NW * D * STAGE;
  constexpr int LDSB = RING > REDB ? RING : REDB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDSB];

  SpanStamps sp;  // phase timestamps (measurement build only)
  sp.mark(0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, K = a.K, M = a.M;
  sp.mark_args(N);
  const int nkb = K >> 5;
  // split-K range of this workgroup (as in sm24_decode_kernel)
  const int ntiles = N / TC;
  int S = 1;
  const int nst_all = (nkb + KS - 1) / KS;
  int z = 0, st0 = 0, nst = nst_all;
  int tile = blockIdx.x;
  int ptile = 0;
  if (a.splits > 1) {
    const int T0 = a.tail_from;
    if (T0 == 0) {
      S = a.splits;
      z = (int)((unsigned)blockIdx.x / (unsigned)ntiles);
      tile -= z * ntiles;
      ptile = tile;
    } else if ((int)blockIdx.x >= T0) {
      S = a.splits;
      const unsigned j = blockIdx.x - (unsigned)T0;
      ptile = (int)(j / (unsigned)S);
      z = (int)j - ptile * S;
      tile = T0 + ptile;
    }
    if (S > 1) {
      st0 = (int)((unsigned)(nst_all * z) / (unsigned)S);
      nst = (int)((unsigned)(nst_all * (z + 1)) / (unsigned)S) - st0;
    }
  }
  // XCD-aware tile order (see sm24_decode_kernel)
  constexpr int SUB = 64 / TC;
  if constexpr (SUB > 1) {
    if (ntiles % (8 * SUB) == 0) {
      const int x = tile & 7, jx = tile >> 3;
      tile = (8 * (jx / SUB) + x) * SUB + jx % SUB;
    }
  }
  const int n0 = tile * TC;
  const int chunk = n0 >> 6;
  const int g0 = (n0 & 63) >> 3;
  const int kw = wave * KPW;  // first k-block of this wave in a stage

  typedef __attribute__((address_space(3))) uint8_t lds_u8;

  // ---- per-lane source pointers: slot q of a stage carries pieces 64 q + lane ----
  // Piece pc of a wave's stage (values, then metadata, scales and activation pieces,
  // as the stage's LDS layout) lies at base_t + kk * row_t + col, where t is its
  // kind, kk its k-block within the wave's share (the scale group for scales) and
  // col its byte offset within that row; a stage later it lies inc_t = KS * row_t
  // further (KS / 4 scale rows).  Each lane keeps its slot's pointer for the next
  // stage to issue, advanced by one 64-bit add per stage.
  constexpr int bpc = VF == VAL4 ? 8 : 6;  // packed bytes per column and k-block
  const uint32_t rowV = bpc * (uint32_t)N, rowM = (MF == META4 ? 4u : 3u) * (uint32_t)N, rowS = 2u * (uint32_t)N;
  const int r00 = st0 * KS + kw;  // first k-block of the wave in stage 0 of the split
  const uint8_t* baseV = static_cast<const uint8_t*>(a.B) + (size_t)bpc * n0;
  const uint8_t* baseM = static_cast<const uint8_t*>(a.meta);
  if constexpr (MF == META4) baseM += 256 * (size_t)chunk + 16 * g0;
  else if constexpr (TC == 64) baseM += 192 * (size_t)chunk;
  else baseM += 192 * (size_t)chunk + 4 * (16 * (g0 >> 2) + ((4 * g0) & 15));
  const uint8_t* baseS = reinterpret_cast<const uint8_t*>(a.s) + 2 * (size_t)n0;
  const uint8_t* baseA = reinterpret_cast<const uint8_t*>(a.A);
  const uint8_t* zeros = reinterpret_cast<const uint8_t*>(a.zeros);
  const uint8_t* sptr[L];  // next stage's source of the lane's piece in slot q
  uint32_t sinc[L], srow[L], skk[L];
#pragma unroll
  for (int q = 0; q < L; q++) {
    const int pc = cmin(lane + 64 * q, P - 1);  // surplus lanes of the last slot are masked off
    uint32_t row, kk, col;
    const uint8_t* base;
    if (pc < NB) {
      kk = (uint32_t)(pc / BPK);
      col = 16u * (uint32_t)(pc % BPK);
      row = rowV;
      base = baseV + (size_t)r00 * rowV;
    } else if (pc < P1) {
      const int p1 = pc - NB, w = p1 % MPK;
      kk = (uint32_t)(p1 / MPK);
      if constexpr (MF == META4) col = 128u * (uint32_t)(w / (MPK / 2)) + 16u * (uint32_t)(w % (MPK / 2));
      else if constexpr (TC == 64) col = 16u * (uint32_t)w;
      else col = 64u * (uint32_t)(w / (TC / 8)) + 16u * (uint32_t)(w % (TC / 8));
      row = rowM;
      base = baseM + (size_t)r00 * rowM;
    } else if (pc < P2) {
      kk = 0;
      col = 16u * (uint32_t)(pc - P1);
      row = rowS;
      base = baseS + (size_t)(r00 >> 2) * rowS;
    } else {
      const int p3 = pc - P2, m = (p3 >> 2) % MB;
      kk = (uint32_t)(p3 / (4 * MB));
      col = 2u * (uint32_t)(m < M ? m : M - 1) * (uint32_t)K + 16u * (uint32_t)(p3 & 3);
      row = 64u;
      base = baseA + 64 * (size_t)r00;
    }
    sptr[q] = base + (kk * row + col);
    sinc[q] = pc >= P1 && pc < P2 ? (uint32_t)(KS / 4) * rowS : (uint32_t)KS * row;
    srow[q] = row;
    skk[q] = kk;
  }

  uint8_t* const wlds = lds + wave * (D * STAGE);  // this wave's D stage buffers
  const uint32_t wlds_addr = (uint32_t)(size_t)(lds_u8*)lds + (uint32_t)(wave * (D * STAGE));

  // DMAs of stage s (of this split) into stage buffer i: L instructions whatever the
  // stage.  A stage that runs past K moves the weight pieces of k-blocks past the last
  // one back to the last one (rows that exist) and reads the zero block for their
  // activation pieces, lane by lane.  Stages are issued in order, s = 0, 1, ...
  auto issue = [&](int i, int s) {
    const uint32_t lb = wlds_addr + (uint32_t)(i * STAGE);
    const int r0 = (st0 + s) * KS + kw;  // first k-block of the wave in this stage (uniform)
    if (__builtin_expect(r0 + KPW <= nkb, 1)) {
      static_for<0, L>([&](auto qi) {
        constexpr int q = decltype(qi)::value;
        dma_lanes_v<q == L - 1 ? LAST : 64>(lb + 1024 * q, sptr[q]);
      });
    } else {
      static_for<0, L>([&](auto qi) {
        constexpr int q = decltype(qi)::value;
        const int pc = cmin(lane + 64 * q, P - 1);
        const int over = pc >= P1 && pc < P2 ? (r0 >> 2) - ((nkb - 1) >> 2) : r0 + (int)skk[q] - (nkb - 1);
        const uint8_t* src = sptr[q];
        if (over > 0) src = pc >= P2 ? zeros : src - (size_t)over * srow[q];
        dma_lanes_v<q == L - 1 ? LAST : 64>(lb + 1024 * q, src);
      });
    }
#pragma unroll
    for (int q = 0; q < L; q++) sptr[q] += sinc[q];
  };

  sp.mark(2);
  // prologue: stages 0 .. D-1 of the split (those that exist)
#pragma unroll
  for (int i = 0; i < D; i++)
    if (i < nst) issue(i, i);  // uniform
  sp.mark(3);

  // ---- MFMA lane roles (as in sm24_decode_kernel) ----
  const int h = lane >> 4;
  const int rho = lane & 15;
  const int gl = rho >> 3, blk = (rho >> 2) & 1, j = rho & 3;
  const int jb = j >> 1, jj = j & 1;
  const int t0 = 2 * (h & 1);
  const int kh = h >> 1;
  const int au = kh | ((h & 1) << 1);
  const uint32_t nsh = 8u * blk;
  const uint32_t msel = (uint32_t)(2 * blk + (h & 1)) | ((uint32_t)(4 + 2 * blk + (h & 1)) << 8) | 0x0c0c0000u;
  const uint32_t m3pos = 3u * (4u * blk + 2u * (h & 1));
  const uint32_t m3s0 = (jb ? 24u : 0u) + m3pos, m3s1 = (jb ? 40u : 16u) + m3pos;
  const uint32_t m3tlo = jb ? kTabLowLo : kTabHighLo, m3thi = jb ? kTabLowHi : kTabHighHi;
  const int arow = rho;
  const uint32_t o_val = kh * (BPK * 16) + (VF == VAL4 ? 4 * (16 * gl + 4 * t0 + j) : 0);
  const int wi_lane = 16 * gl + 4 * t0 + j;
  const uint32_t o_meta = MOFF + kh * (MPK * 16) + jb * 2 * TC + 8 * (2 * gl + jj);
  const uint32_t o_mrow = MOFF + kh * (MPK * 16);
  const uint32_t o_scale = SOFF + 2 * (8 * gl + 2 * j + blk);
  const uint32_t o_act = AOFF + arow * 64 + 16 * au;
  uint32_t kMask, kMaskHi, kMagic;
  if constexpr (VF == VAL4) {
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
    asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));
  } else {
    asm volatile("v_mov_b32 %0, 0x00070007" : "=v"(kMask));
    asm volatile("v_mov_b32 %0, 0x00380038" : "=v"(kMaskHi));
  }
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));

  constexpr int KP = KPW / 2;
  float4_t acc[KP][NCB][RB];
#pragma unroll
  for (int q = 0; q < KP; q++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) acc[q][cb][rb] = (float4_t){0.f, 0.f, 0.f, 0.f};
  half8_t sact[RB][KPW];  // activation operands

  auto compute = [&](const uint8_t* st) {
    uint32_t xr[KP][NCB][2];
    uint32_t x3[KP][NCB][4];
    auto m3_which = [&](int cb) -> int { return TC == 64 ? (2 * cb + gl) >> 2 : g0 >> 2; };
    auto m3_shift = [&](int cb) -> uint32_t { return m3_which(cb) == 0 ? m3s0 : m3s1; };
    uint32_t m3y[KP][NCB][2], m3l[KP][NCB][2];
    u32x2 mr[KP][NCB];
    _Float16 sr[NCB];
    // every LDS operand of the stage first, then the dequantisation and MFMAs
#pragma unroll
    for (int q2 = 0; q2 < KP; q2++) {
#pragma unroll
      for (int rb = 0; rb < RB; rb++) {
        const uint8_t* ap = st + o_act + 16 * rb * 64;
        sact[rb][2 * q2] = *reinterpret_cast<const half8_t*>(ap + 2 * q2 * MB * 64);
        sact[rb][2 * q2 + 1] = *reinterpret_cast<const half8_t*>(ap + (2 * q2 + 1) * MB * 64);
      }
    }
#pragma unroll
    for (int q2 = 0; q2 < KP; q2++)
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        if constexpr (VF == VAL4) {
          const uint8_t* vp = st + o_val + 2 * q2 * (BPK * 16) + 128 * cb;
          xr[q2][cb][0] = *reinterpret_cast<const uint32_t*>(vp);
          xr[q2][cb][1] = *reinterpret_cast<const uint32_t*>(vp + 16);
        } else {
          const uint8_t* rowp = st + o_val + 2 * q2 * (BPK * 16);
          const int b0 = 3 * (wi_lane + 32 * cb), b1 = b0 + 12;
          const uint32_t* p0 = reinterpret_cast<const uint32_t*>(rowp + (b0 & ~3));
          const uint32_t* p1 = reinterpret_cast<const uint32_t*>(rowp + (b1 & ~3));
          x3[q2][cb][0] = p0[0];
          x3[q2][cb][1] = p0[1];
          x3[q2][cb][2] = p1[0];
          x3[q2][cb][3] = p1[1];
        }
        if constexpr (MF == META4) {
          mr[q2][cb] = *reinterpret_cast<const u32x2*>(st + o_meta + 2 * q2 * (MPK * 16) + 32 * cb);
        } else {
#pragma unroll
          for (int ehalf = 0; ehalf < 2; ehalf++) {
            const uint32_t* mrow = reinterpret_cast<const uint32_t*>(st + o_mrow + 2 * q2 * (MPK * 16));
            const int gt = 2 * cb + gl;
            int ix, iy;
            if constexpr (TC == 64) {
              ix = 16 * m3_which(cb) + ((4 * gt + 2 * jj + ehalf) & 15);
              iy = ix + 16;
            } else {
              ix = 4 * gt + 2 * jj + ehalf;
              iy = ix + TC / 2;
            }
            m3y[q2][cb][ehalf] = mrow[iy];
            m3l[q2][cb][ehalf] = mrow[m3_shift(cb) >= 32u ? iy : ix];
          }
        }
      }
    if constexpr (GROUPED) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) sr[cb] = *reinterpret_cast<const _Float16*>(st + o_scale + 32 * cb);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q2 = 0; q2 < KP; q2++) {
      half16_t act[RB];
#pragma unroll
      for (int rb = 0; rb < RB; rb++)
        act[rb] = __builtin_shufflevector(sact[rb][2 * q2], sact[rb][2 * q2 + 1], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10,
                                          11, 12, 13, 14, 15);
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        uint32_t lo0, lo1, hi0, hi1;
        if constexpr (VF == VAL4) {
          const uint32_t x0 = xr[q2][cb][0] >> nsh;
          const uint32_t x1 = xr[q2][cb][1] >> nsh;
          lo0 = (x0 & kMask) | kMagic;
          lo1 = (x1 & kMask) | kMagic;
          hi0 = (x0 & kMaskHi) | kMagic;
          hi1 = (x1 & kMaskHi) | kMagic;
        } else {
          const int b0 = 3 * (wi_lane + 32 * cb), b1 = b0 + 12;
          const uint32_t y0 = __builtin_amdgcn_alignbit(x3[q2][cb][1], x3[q2][cb][0], 8 * (b0 & 3) + 6 * blk);
          const uint32_t y1 = __builtin_amdgcn_alignbit(x3[q2][cb][3], x3[q2][cb][2], 8 * (b1 & 3) + 6 * blk);
          const uint32_t z0 = (y0 & 0x0000FFFFu) | ((y0 << 4) & 0xFFFF0000u);
          const uint32_t z1 = (y1 & 0x0000FFFFu) | ((y1 << 4) & 0xFFFF0000u);
          lo0 = (z0 & kMask) | kMagic;
          lo1 = (z1 & kMask) | kMagic;
          hi0 = (z0 & kMaskHi) | kMagic;
          hi1 = (z1 & kMaskHi) | kMagic;
        }
        constexpr float zp = VF == VAL4 ? 1032.0f : 1028.0f;
        constexpr float hs = VF == VAL4 ? 0.0625f : 0.125f;
        constexpr float zh = (zp - 1024.0f) + 1024.0f * hs;
        const half2_t kz = {(_Float16)zp, (_Float16)zp};
        const half2_t k16 = {(_Float16)hs, (_Float16)hs};
        const half2_t kzh = {(_Float16)-zh, (_Float16)-zh};
        const half2_t l0 = __builtin_bit_cast(half2_t, lo0) - kz;
        const half2_t l1 = __builtin_bit_cast(half2_t, lo1) - kz;
        const half2_t u0 = __builtin_bit_cast(half2_t, hi0) * k16 + kzh;
        const half2_t u1 = __builtin_bit_cast(half2_t, hi1) * k16 + kzh;
        half8_t aop = (half8_t){l0.x, l0.y, l1.x, l1.y, u0.x, u0.y, u1.x, u1.y};
        uint32_t idx;
        if constexpr (MF == META4) {
          const u32x2 unit = mr[q2][cb];
          idx = __builtin_amdgcn_perm(unit.y, unit.x, msel);
        } else {
          uint32_t v[2];
#pragma unroll
          for (int ehalf = 0; ehalf < 2; ehalf++)
            v[ehalf] = __builtin_amdgcn_alignbit(m3y[q2][cb][ehalf], m3l[q2][cb][ehalf], m3_shift(cb) & 31u);
          const uint32_t s2 = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u);
          const uint32_t sel = (s2 | (s2 << 13)) & 0x07070707u;
          const uint32_t nib = __builtin_amdgcn_perm(m3thi, m3tlo, sel);
          idx = (nib & 0x0f0fu) | ((nib >> 12) & 0xf0f0u);
        }
        if constexpr (GROUPED) {
          const _Float16 sc = sr[cb];
          aop = aop * (half8_t){sc, sc, sc, sc, sc, sc, sc, sc};
        }
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          acc[q2][cb][rb] = smfmac64<0>(aop, act[rb], acc[q2][cb][rb], idx);
          if constexpr (TC == 64) asm volatile("" : "+v"(acc[q2][cb][rb]));
        }
      }
    }
  };

  // ---- main loop: D stages per round, buffer i = stage % D ----
  // Rounds in which every stage refills its buffer (D stages later) run without
  // guards; the last (at most two) rounds check each stage.
  auto run_stage = [&](int i, int s, bool refill) {
    compute(wlds + i * STAGE);
    __builtin_amdgcn_sched_barrier(0);
    if (refill) {
      // the stage's LDS reads are complete before its buffer is refilled
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(i, s + D);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int base = 0;
  for (; base + 2 * D <= nst; base += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      wait_vm<L * (D - 1)>();
      run_stage(i, base + i, true);
    }
  }
  for (; base < nst; base += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      const int s = base + i;
      if (s < nst) {  // uniform
        wait_stages<L, D - 1>(nst - 1 - s);
        run_stage(i, s, s + D < nst);
      }
    }
  }
  sp.mark(4);

#pragma unroll
  for (int q = 1; q < KP; q++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) acc[0][cb][rb] += acc[q][cb][rb];

  // ---- reduction and store (as in sm24_decode_kernel) ----
  float* const red = reinterpret_cast<float*>(lds);
  const int r_out = tid / (TC / 4), c_out = 4 * (tid % (TC / 4));
  auto write_c = [&](int rb, float4_t v) {
    const int row = r_out + 16 * rb;
    if (row < M) {
      const int n = n0 + c_out;
      half4_t o;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o[i] = (_Float16)v[i];
        if constexpr (!GROUPED) o[i] = o[i] * a.s[n + i];
      }
      *reinterpret_cast<half4_t*>(a.C + (size_t)row * N + n) = o;
    }
  };
  auto partial_at = [&](int zz, int rb) -> float* {
    return a.partial + ((size_t)(ptile * S + zz) * RB + rb) * (16 * TC) + r_out * TC + c_out;
  };
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    __syncthreads();
    if (rho + 16 * rb < M) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++)
        *reinterpret_cast<float4_t*>(red + (wave * 16 + rho) * REDP + 16 * cb + 4 * h) = acc[0][cb][rb];
    }
    __syncthreads();
    if (tid < 4 * TC && r_out + 16 * rb < M) {
      float4_t v = *reinterpret_cast<const float4_t*>(red + r_out * REDP + c_out);
#pragma unroll
      for (int w = 1; w < NW; w++) v += *reinterpret_cast<const float4_t*>(red + (w * 16 + r_out) * REDP + c_out);
      if (S == 1) write_c(rb, v);
      else *reinterpret_cast<float4_t*>(partial_at(z, rb)) = v;
    }
  }
  if (S > 1) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    __shared__ uint32_t arrived;
    if (tid == 0) arrived = __hip_atomic_fetch_add(a.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __syncthreads();
    if (arrived != (uint32_t)S) {
      sp.store(a.spans, NW, wave, lane);
      return;
    }
    if (tid == 0) __hip_atomic_store(a.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 4 * TC && r_out < M) {
      float4_t v[RB];
      for (int z0 = 0; z0 < S; z0 += 4) {
        float4_t t[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (z0 + i < S) t[rb][i] = *reinterpret_cast<const float4_t*>(partial_at(z0 + i, rb));
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (z0 + i < S) v[rb] = z0 + i == 0 ? t[rb][0] : v[rb] + t[rb][i];
      }
#pragma unroll
      for (int rb = 0; rb < RB; rb++) write_c(rb, v[rb]);
    }
  }
  sp.store(a.spans, NW, wave, lane);
}

}  // namespace sm24
