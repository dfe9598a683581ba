// Decode-sized (M <= 16) 2:4 INT4 x FP16 GEMM for gfx950, no split-K.
//
// One workgroup owns a tile of TC output columns (TC = 16, 32 or 64, chosen so that
// the tiles cover the compute units) over the whole K, so the result never crosses
// workgroups: a cross-workgroup hand-off costs microseconds on this multi-XCD part,
// more than the whole weight stream of a 4096x4096 layer.
//
// The tile's packed weight is streamed in stages of KS k-blocks (KS * TC = 64 * NW
// column-k-blocks, 800 bytes of values + metadata + scales per wave).  Every thread owns one
// 16-byte piece of each stage (thread t: the t-th piece, same slot in every stage);
// a register ring keeps D stages in flight, i.e. D * 0.8 KiB per wave.  When a
// stage's pieces arrive they are written to one of two LDS buffers and, after a
// barrier, the four waves read their MFMA operands from LDS in the v_smfmac lane
// order (the 16-byte pieces are coalesced in HBM but hold 8 columns x 4 k-rows,
// while an MFMA row needs one column).
//
// Wave w computes k-blocks [w*KS/NW, (w+1)*KS/NW) of every stage for all 16-column
// blocks of the tile; activations (the dense B operand) come from L2, prefetched
// two or three stages ahead.  The four waves' accumulators are reduced in LDS.
#pragma once
#include "sm24_device.h"

namespace sm24 {

template <int TC, int NW, bool GROUPED, int VF, int MF>
__global__ __launch_bounds__(64 * NW) void sm24_decode_kernel(GemmArgs a) {
  constexpr int NT = 64 * NW;                           // threads
  constexpr int NCB = TC / 16;                          // 16-column MFMA blocks per tile
  constexpr int KPW = 64 / TC;                          // k-blocks per wave per stage
  constexpr int KS = KPW * NW;                          // k-blocks per stage (64*NW column-k-blocks)
  constexpr int BPK = VF == VAL4 ? TC / 2 : 3 * TC / 8;  // 16-byte value pieces per k-block
  // 16-byte metadata pieces per k-block: the tile's 4*TC bytes of 4-bit metadata, or
  // of the 3-bit code words (the whole 192-byte group when TC == 64).
  constexpr int MPK = (MF == META3 && TC == 64) ? 12 : TC / 4;
  constexpr int SPG = TC / 8;                           // 16-byte scale pieces per scale group
  constexpr int NB = KS * BPK;
  constexpr int NM = KS * MPK;
  constexpr int NSC = GROUPED ? (KS / 4) * SPG : 0;
  constexpr int NP = NB + NM + NSC;                     // pieces per stage (about 50 per wave)
  constexpr int BBYTES = NB * 16, MBYTES = NM * 16, SBYTES = NSC * 16;
  constexpr int DUMMY = BBYTES + MBYTES + SBYTES;       // threads without a piece write here
  constexpr int STAGE = DUMMY + (NT - NP) * 16;
  // Stages in flight D and activation ring ARS (prefetch distance ARS-1), sized so
  // that a wave never has more than 63 loads outstanding (the vmcnt limit):
  // D * (1 + KPW) <= 63.
  // With 16 waves (4 per SIMD) the register budget is 128: shallower rings.
  constexpr int D = NW == 16 ? (TC == 64 ? 12 : 8) : (TC == 16 ? 12 : 16);
  constexpr int ARS = (NW == 16 && TC == 16) ? 2 : 4;
  constexpr int AD = ARS - 1;
  static_assert(NP <= NT, "one piece per thread");

  __shared__ __attribute__((aligned(16))) uint8_t lds[2][STAGE];
  __shared__ float red[NW / 2][16][TC + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, K = a.K, M = a.M;
  const int nkb = K >> 5;
  const int ngroups = (nkb + 3) >> 2;
  const int nst = (nkb + KS - 1) / KS;
  const int n0 = blockIdx.x * TC;
  const int chunk = n0 >> 6;
  const int g0 = (n0 & 63) >> 3;

  // ---- this thread's piece: global byte offset = base + row * stride, row clamped ----
  const uint8_t* pbase;
  size_t pstride;
  int prow;      // k-block (or scale group) of the piece within a stage
  int pmaxrow;   // last valid k-block (or group)
  int pper;      // rows per stage (KS for k-blocks, KS/4 for groups)
  int plds;
  if (tid < NB) {
    const int kk = tid / BPK, w = tid % BPK;
    if constexpr (VF == VAL4) {
      pbase = static_cast<const uint8_t*>(a.B) + 8 * (size_t)n0 + 16 * w;
      pstride = 8 * (size_t)N;
    } else {
      pbase = static_cast<const uint8_t*>(a.B) + 6 * (size_t)n0 + 16 * w;
      pstride = 6 * (size_t)N;
    }
    prow = kk;
    pmaxrow = nkb - 1;
    pper = KS;
    plds = kk * BPK * 16 + 16 * w;
  } else if (tid < NB + NM) {
    const int q = tid - NB, kk = q / MPK, w = q % MPK;
    if constexpr (MF == META4) {
      // two parts (units of the first / second column pair j>>1), 2*TC bytes each
      const int jbp = w / (MPK / 2), wp = w % (MPK / 2);
      pbase = static_cast<const uint8_t*>(a.meta) + 256 * (size_t)chunk + 128 * jbp + 16 * g0 + 16 * wp;
      pstride = 4 * (size_t)N;
      plds = BBYTES + kk * MPK * 16 + jbp * 2 * TC + 16 * wp;
    } else if constexpr (TC == 64) {
      // the whole 48-word group of the chunk
      pbase = static_cast<const uint8_t*>(a.meta) + 192 * (size_t)chunk + 16 * w;
      pstride = 3 * (size_t)N;
      plds = BBYTES + kk * MPK * 16 + 16 * w;
    } else {
      // rows (which, which+1) of the group, TC/2 words each starting at word P0
      const int which = g0 >> 2, p0 = (4 * g0) & 15;
      const int row = w / (TC / 8), wp = w % (TC / 8);
      pbase = static_cast<const uint8_t*>(a.meta) + 192 * (size_t)chunk + 4 * (16 * (which + row) + p0) + 16 * wp;
      pstride = 3 * (size_t)N;
      plds = BBYTES + kk * MPK * 16 + row * 2 * TC + 16 * wp;
    }
    prow = kk;
    pmaxrow = nkb - 1;
    pper = KS;
  } else if (tid < NP) {
    const int q = tid - NB - NM, gl = q / SPG, w = q % SPG;
    pbase = reinterpret_cast<const uint8_t*>(a.s) + 2 * (size_t)n0 + 16 * w;
    pstride = 2 * (size_t)N;
    prow = gl;
    pmaxrow = ngroups - 1;
    pper = KS / 4;
    plds = BBYTES + MBYTES + gl * 2 * TC + 16 * w;
  } else {
    pbase = reinterpret_cast<const uint8_t*>(a.zeros);
    pstride = 0;
    prow = 0;
    pmaxrow = 0;
    pper = 0;
    plds = DUMMY + 16 * (tid - NP);
  }
  auto load_piece = [&](int s) -> u32x4 {
    int row = s * pper + prow;
    row = row < pmaxrow ? row : pmaxrow;
    return *reinterpret_cast<const u32x4*>(pbase + (size_t)row * pstride);
  };

  // ---- MFMA lane roles ----
  // Lane group h covers dense groups 2h and 2h+1 of a k-block (k-space = dense K, so
  // the activation operand is 16 contiguous bytes).  Group d of a column sits in word
  // t = d mod 4 of the packed layout, as its first (d < 4) or second (d >= 4) nibble
  // pair: lane group h reads words t0 = 2*(h&1) and t0+1 and takes nibble pair
  // p = 2*blk + (h>>1), i.e. nibbles p and p+4.
  const int h = lane >> 4;
  const int rho = lane & 15;   // A row = column n0 + 16*cb + rho; B column = batch row
  const int gl = rho >> 3, blk = (rho >> 2) & 1, j = rho & 3;
  const int jb = j >> 1, jj = j & 1;
  const int t0 = 2 * (h & 1);
  const int ehalf = h >> 1;                          // metadata int16: first/second 16 dense K
  const uint32_t nsh = 4u * (2u * blk + ehalf);      // nibble-pair shift in a value word
  const uint32_t msh = 8u * (h & 1);                 // index-byte shift in a metadata int16
  const int m_act = rho;
  const bool act_ok = m_act < M;

  auto load_act = [&](int s, half8_t* dst) {
#pragma unroll
    for (int q = 0; q < KPW; q++) {
      int kb = s * KS + wave * KPW + q;
      const bool live = act_ok && kb < nkb;
      const _Float16* ap = live ? a.A + (size_t)m_act * K + 32 * kb + 8 * h : a.zeros;
      dst[q] = *reinterpret_cast<const half8_t*>(ap);
    }
  };

  float4_t acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) acc[cb] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s, const uint8_t* st, const half8_t* act) {
#pragma unroll
    for (int q = 0; q < KPW; q++) {
      const int kk = wave * KPW + q;
      if (s * KS + kk >= nkb) break;  // wave-uniform
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        const int gt = 2 * cb + gl;
        const int wi0 = 16 * gt + 4 * t0 + j;  // words t0 and t0+1 of the tile's k-block row
        uint32_t w0, w1;
        if constexpr (VF == VAL4) {
          const uint8_t* rowp = st + kk * (BPK * 16);
          w0 = *reinterpret_cast<const uint32_t*>(rowp + 4 * wi0);
          w1 = *reinterpret_cast<const uint32_t*>(rowp + 4 * (wi0 + 4));
        } else {
          const uint8_t* rowp = st + kk * (BPK * 16);
          const int b0 = 3 * wi0, b1 = 3 * (wi0 + 4);
          const uint32_t* p0 = reinterpret_cast<const uint32_t*>(rowp + (b0 & ~3));
          const uint32_t* p1 = reinterpret_cast<const uint32_t*>(rowp + (b1 & ~3));
          w0 = spread3(__builtin_amdgcn_alignbit(p0[1], p0[0], 8 * (b0 & 3)) & 0xFFFFFFu);
          w1 = spread3(__builtin_amdgcn_alignbit(p1[1], p1[0], 8 * (b1 & 3)) & 0xFFFFFFu);
        }
        // values: nibble pairs of words t0, t0+1 -> {g_2h slot0, slot1, g_2h+1 slot0, slot1}
        const uint32_t x0 = ((w0 >> nsh) & 0x000F000Fu) | 0x64006400u;
        const uint32_t x1 = ((w1 >> nsh) & 0x000F000Fu) | 0x64006400u;
        constexpr float zp = VF == VAL4 ? 1032.0f : 1028.0f;  // 1024 + zero point
        const half2_t v0 = __builtin_bit_cast(half2_t, x0) - (half2_t){(_Float16)zp, (_Float16)zp};
        const half2_t v1 = __builtin_bit_cast(half2_t, x1) - (half2_t){(_Float16)zp, (_Float16)zp};
        half4_t aop = (half4_t){v0.x, v0.y, v1.x, v1.y};
        // metadata: int16 (blk, ehalf) of unit 16*jb + 2*gt + jj; byte h&1 holds the
        // nibbles of dense groups 2h and 2h+1
        uint32_t idx;
        if constexpr (MF == META4) {
          const uint16_t md = *reinterpret_cast<const uint16_t*>(
              st + BBYTES + kk * (MPK * 16) + jb * 2 * TC + 8 * (2 * gt + jj) + 2 * (blk + 2 * ehalf));
          idx = ((uint32_t)md >> msh) & 0xFFu;
        } else {
          // 3-bit code word of metadata word u = 32*jb + 4*g + 2*jj + ehalf: the low
          // (jb = 0) or high 24 bits of field "first" (g < 4) or "second" (g >= 4)
          // at position P = u mod 16, built from words (which, which+1).
          const uint32_t* mrow = reinterpret_cast<const uint32_t*>(st + BBYTES + kk * (MPK * 16));
          uint32_t X, Y;
          int which;
          if constexpr (TC == 64) {
            which = gt >> 2;
            const int P = (4 * gt + 2 * jj + ehalf) & 15;
            X = mrow[16 * which + P];
            Y = mrow[16 * (which + 1) + P];
          } else {
            which = g0 >> 2;
            const int pl = 4 * gt + 2 * jj + ehalf;
            X = mrow[pl];
            Y = mrow[TC / 2 + pl];
          }
          uint32_t c24;
          if (which == 0) c24 = jb ? ((X >> 24) | ((Y & 0xFFFFu) << 8)) : (X & 0xFFFFFFu);
          else c24 = jb ? ((Y >> 8) & 0xFFFFFFu) : (((X >> 16) | (Y << 16)) & 0xFFFFFFu);
          const uint32_t lut = jb ? kLutLow : kLutHigh;
          const uint32_t pos = 3u * (4u * blk + 2u * (h & 1));  // nibbles 2(h&1), +1 of int16 blk
          const uint32_t ca = (c24 >> pos) & 7u, cbv = (c24 >> (pos + 3u)) & 7u;
          idx = ((lut >> (4u * ca)) & 15u) | (((lut >> (4u * cbv)) & 15u) << 4);
        }
        if constexpr (GROUPED) {
          const _Float16 sc =
              *reinterpret_cast<const _Float16*>(st + BBYTES + MBYTES + (kk >> 2) * 2 * TC + 2 * (8 * gt + 2 * j + blk));
          aop = scale4(aop, sc);
        }
        acc[cb] = smfmac32<0>(aop, act[q], acc[cb], idx);
      }
    }
  };

  // ---- pipeline ----
  u32x4 wring[D];
  half8_t aring[ARS][KPW];
#pragma unroll
  for (int i = 0; i < D; i++) {
    wring[i] = load_piece(i);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < AD; i++) {
    load_act(i, aring[i]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int base = 0; base < nst; base += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      const int s = base + i;
      if (s >= nst) break;  // uniform
      *reinterpret_cast<u32x4*>(&lds[i & 1][plds]) = wring[i];
      wring[i] = load_piece(s + D);
      load_act(s + AD, aring[(i + AD) % ARS]);
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      compute(s, lds[i & 1], aring[i % ARS]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- reduce the NW waves pairwise in LDS (fixed order), wave 0 writes C ----
#pragma unroll
  for (int half = NW / 2; half >= 1; half >>= 1) {
    if (wave >= half && wave < 2 * half) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[wave - half][rho][16 * cb + 4 * h + i] = acc[cb][i];
    }
    __syncthreads();
    if (wave < half) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[cb][i] += red[wave][rho][16 * cb + 4 * h + i];
    }
    __syncthreads();
  }
  if (wave == 0 && rho < M) {
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int n = n0 + 16 * cb + 4 * h + i;
        _Float16 o = (_Float16)acc[cb][i];
        if constexpr (!GROUPED) o = o * a.s[n];
        a.C[(size_t)rho * N + n] = o;
      }
    }
  }
}

}  // namespace sm24
