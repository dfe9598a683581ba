// Decode-sized 2:4 INT4 x FP16 GEMM for gfx950 at 1, 4 and 8 padded batch rows (up to
// 8 rows per launch; 9-32 rows run sm24_decode_dma.h).
//
// One workgroup owns a tile of TC output columns (TC = 16, 32 or 64) over the whole
// K, or over one of a.splits contiguous ranges of its stages (split-K, of every tile
// or of the tiles past a.tail_from: the last split to arrive sums the ranges through
// the host's scratch).  Unsplit, the result never crosses workgroups: a
// cross-workgroup hand-off costs microseconds on this multi-XCD part, more than the
// whole weight stream of a 4096x4096 layer.
//
// Cost model (measured on MI355X): every 16-byte vector load instruction occupies a
// compute unit's address path for ~16 cycles whatever its lanes do (full, masked,
// duplicated or out of range alike), so the kernel issues as few load instructions
// as the bytes allow and fills every lane with a distinct useful 16-byte piece.
//
// A stage covers KS = NW * KPW k-blocks of the tile, KPW = max(2, 64 / TC) per wave.
// Each wave streams its own KPW k-blocks: their pieces - packed values, metadata,
// the scales of their one scale group and, unless resident, the activation rows - form a
// list of P 16-byte pieces; lane l loads pieces l, l + 64, ... (SL slots) of every
// stage, rows clamped to the operand, into a register ring D stages deep.  When a
// stage is due the wave writes its pieces to one of its two LDS buffers and reads its
// MFMA operands back: a wave's LDS operations complete in order, so no workgroup
// barrier runs between stages.  Batch rows past M read row M-1 (their outputs are not
// stored); k-blocks past K read zero activations, so the last stage needs no
// per-k-block branch.
//
// MFMA (v_smfmac_f32_16x16x64_f16, two k-blocks per instruction) lane roles: lane
// (rho, h) = (l % 16, l / 16) holds output column n = n0 + 16*cb + rho, i.e. word j =
// rho & 3 of column half blk = (rho >> 2) & 1 of 8-column group gl = rho >> 3, and
// the MFMA groups 4h..4h+3 = real groups t0, t0+1, t0+4, t0+5 (t0 = 2*(h&1)) of
// k-block h >> 1 of the pair.  Word t of a column holds groups t and t+4, so the
// lane's 8 values are all four nibbles of column half blk in words t0 and t0+1
// (bytes blk and blk+2): low nibbles give groups t0, t0+1, high nibbles t0+4, t0+5.
// Its index is byte h&1 of the column's two metadata int16s (groups 0-3 and 4-7),
// one v_perm of the 8-byte metadata unit.  Its activation operand is batch row rho,
// real dense K 4*(t0 + 4*(h>>1)) .. +7 of each k-block of the pair (the same 16-byte
// piece u = (h >> 1) | ((h & 1) << 1) of both k-block rows).  Wave w computes k-blocks
// [w*KPW, (w+1)*KPW) of every stage for all column blocks; the waves' partial sums
// are reduced in LDS at the end.
#pragma once
#include "sm24_device.h"

namespace sm24 {

constexpr int cmin(int a, int b) { return a < b ? a : b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }

// G: tiles per workgroup, each on its own NW waves, sharing the workgroup's resident
// activation rows (G = 3 for 16-column tiles, unsplit: one workgroup per CU where
// three tiles per CU would otherwise be three workgroups copying the same rows).
template <int TC, int NW, int MB, bool GROUPED, int VF, int MF, bool DEEP, bool RES, int G = 1>
__global__ __launch_bounds__(64 * NW * G) void sm24_decode_kernel(const void* B_, const void* meta_, const void* s_,
                                                              const void* A_, const void* zeros_, int M_, int N_,
                                                              int K_, int splits_, GemmArgs a_) {
  const GemmArgs a = with_lead(a_, B_, meta_, s_, A_, zeros_, M_, N_, K_, splits_);
  constexpr int NCB = TC / 16;                          // 16-column MFMA blocks per tile
  constexpr int KPW = cmax(2, 64 / TC);                 // k-blocks per wave per stage (pairs)
  constexpr int KS = KPW * NW;                          // k-blocks per stage
  constexpr int BPK = VF == VAL4 ? TC / 2 : 3 * TC / 8;  // 16-byte value pieces per k-block
  // 16-byte metadata pieces per k-block: the tile's 4*TC bytes of 4-bit metadata, or
  // of the 3-bit code words (the whole 192-byte group when TC == 64).
  constexpr int MPK = (MF == META3 && TC == 64) ? 12 : TC / 4;
  constexpr int SPG = TC / 8;                           // 16-byte scale pieces per scale group
  // Activations through LDS, either resident (RES: the workgroup's rows over its whole
  // k range, loaded once by LDS-DMA into the dynamic LDS) or with every stage's pieces.
  static_assert(MB == 1 || MB == 4 || MB == 8, "1, 4 or 8 padded batch rows");
  constexpr bool STAGED = !RES;                         // activations with the stage pieces
  constexpr int RB = 1;                                 // one 16-column MFMA B operand
  // Pieces of one wave's stage, in its LDS region in this order.
  constexpr int NB = KPW * BPK;
  constexpr int NM = KPW * MPK;
  constexpr int NSC = GROUPED ? SPG : 0;                // KPW <= 4 k-blocks: one scale group
  constexpr int NPA = STAGED ? KPW * 4 * MB : 0;        // activation pieces (4 per row and k-block)
  constexpr int P1 = NB + NM, P2 = P1 + NSC, P = P2 + NPA;
  constexpr int SL = (P + 63) / 64;                     // load slots per lane and stage
  constexpr int MOFF = NB * 16, SOFF = MOFF + NM * 16, AOFF = SOFF + NSC * 16;
  constexpr int STAGE = AOFF + NPA * 16;                // bytes of one wave's stage
  static_assert(KPW <= 4 && 4 % KPW == 0, "a wave's k-blocks lie in one scale group");
  // Ring depth: at most ~56 loads in flight per wave (vmcnt counts to 63) and a
  // register budget for the ring that keeps the kernel at <= 128 VGPRs (two
  // 8-wave or four 4-wave workgroups per CU).  Even, so that ring slot i always
  // uses LDS buffer i & 1 (consecutive stages must alternate buffers, also across
  // the wrap from slot D-1 to slot 0).
  constexpr int LPS = SL;
  // DEEP: a ring as deep as the budget allows (long K: more bytes in flight per
  // workgroup); otherwise 16 VGPRs, so that more workgroups are resident per CU.
  constexpr int RING_VGPRS = !DEEP ? 16 : 40;
  constexpr int D = cmax(2, cmin(16, cmin(56 / LPS, RING_VGPRS / (4 * LPS)))) & ~1;
  static_assert(D >= 2 && D % 2 == 0, "even ring depth");
  static_assert(KS % 4 == 0, "scale groups of 4 k-blocks per stage");

  // Two stage buffers per wave; after the last stage the same LDS holds every wave's
  // partial tile (16 rows x TC columns of fp32, rows padded to TC + 4) for the
  // reduction.
  constexpr int REDP = TC + 4;
  constexpr int REDB = NW * 16 * REDP * 4;
  static_assert(G == 1 || (G == 3 && TC == 16), "three 16-column tiles per workgroup, or one tile");
  constexpr int LDSB = 2 * NW * G * STAGE > G * REDB ? 2 * NW * G * STAGE : G * REDB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDSB];

  SpanStamps sp;  // phase timestamps (measurement build only)
  sp.mark(0);
  const int lane = threadIdx.x & 63;
  const int wall = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = G == 1 ? 0 : wall / NW;     // this wave's tile of the workgroup
  const int wave = G == 1 ? wall : wall % NW;  // its wave among that tile's NW
  const int tid = threadIdx.x - 64 * NW * grp;  // its thread among that tile's
  const int N = a.N, K = a.K, M = a.M;
  sp.mark_args(N);
  const int nkb = K >> 5;
  const int ngroups = (nkb + 3) >> 2;
  // Split-K: split z of a tile covers stages [st0, st0 + nst) (the host keeps splits
  // <= the stage count).  Every tile split (a.tail_from == 0): block b = z * ntiles +
  // tile.  Tail split (a.tail_from = T0 > 0): blocks b < T0 own the whole K of tile
  // b; the remaining ntiles - T0 tiles are split, block T0 + S * p + z running split
  // z of tile T0 + p, so that the few tiles past one per CU spread over all CUs
  // instead of doubling the load of some.  Without a split (the usual case) no
  // division runs: a 64-bit or even a 32-bit division is a long scalar chain that
  // every wave would pay before its first load.
  const int ntiles = N / TC;
  int S = 1;                          // splits of this workgroup's tile
  const int nst_all = (nkb + KS - 1) / KS;
  int z = 0, st0 = 0, nst = nst_all;  // split z covers stages [st0, st0 + nst)
  int tile = blockIdx.x;
  int ptile = 0;                      // index of the tile among the split tiles
  if (G == 1 && a.splits > 1) {  // uniform; nst_all * S is small, so 32 bits are exact
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
  // XCD-aware tile order.  Workgroups are dispatched round-robin over the 8 XCDs
  // (block b runs on XCD b % 8) and each XCD has its own L2.  The SUB = 64/TC tiles of
  // one 64-column chunk share 128-byte lines of metadata and scales (a tile's packed
  // values are whole lines), so they go to blocks b = 8*(SUB*q + s) + x, which all
  // sit on XCD x: each line is fetched from HBM once instead of once per tile.
  constexpr int SUB = 64 / TC;
  if constexpr (G > 1) {
    // block b = 8 j + x (on XCD x) runs tiles k = G j + grp of XCD x's share: chunk
    // 8 (k / SUB) + x, its tile k % SUB (the host launches ntiles / G blocks, unsplit,
    // with ntiles a multiple of 8 SUB G)
    const int x = blockIdx.x & 7, k = G * (blockIdx.x >> 3) + grp;
    tile = (8 * (k / SUB) + x) * SUB + k % SUB;
  } else if constexpr (SUB > 1) {
    if (ntiles % (8 * SUB) == 0) {
      const int x = tile & 7, jx = tile >> 3;
      tile = (8 * (jx / SUB) + x) * SUB + jx % SUB;
    }
  }
  const int n0 = tile * TC;
  const int chunk = n0 >> 6;
  const int g0 = (n0 & 63) >> 3;

  // ---- resident activations (RES): batch rows 0..M-1 of this split's k range, zero
  // past K, row m at byte m * RS of the dynamic LDS (RS = the range's bytes + 16, so
  // that the rows start on different banks); every wave copies every NW-th 1 KiB
  // chunk of each row by LDS-DMA, ahead of the weight ring's first loads ----
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
  const uint32_t span = (uint32_t)nst * (KS * 64);  // bytes of one row's k range
  const uint32_t RS = span + 16;
  if constexpr (RES) {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t act0 = (uint32_t)(size_t)(lds_u8*)dyn_lds;
    const int cpr = (int)((span + 1023) >> 10);
    const int k0 = st0 * KS * 32;
#pragma unroll
    for (int m = 0; m < MB; m++) {
      if (m < M) {  // uniform
        for (int jc = wall; jc < cpr; jc += NW * G) {
          const uint32_t b = (uint32_t)jc * 1024u + 16u * lane;
          if (b < span) {
            const int k = k0 + (int)(b >> 1);
            const _Float16* src = k < K ? a.A + (size_t)m * K + k : a.zeros;
            dma16(act0 + m * RS + (uint32_t)jc * 1024u, src);
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- per-slot piece state: bytes at base + min(s*per + row0, rmax) * stride ----
  const uint8_t* sbase[SL];
  uint32_t sstride[SL], srow0[SL], sper[SL], srmax[SL], slds[SL];
  bool szero[SL];  // activation piece: zero past the last k-block
  const int kw = wave * KPW;  // first k-block of this wave in a stage
#pragma unroll
  for (int q = 0; q < SL; q++) {
    const int pc = cmin(lane + q * 64, P - 1);  // surplus lanes repeat the last piece
    szero[q] = false;
    if (pc < NB) {
      const int kl = pc / BPK, w = pc % BPK;
      constexpr int bpc = VF == VAL4 ? 8 : 6;  // packed bytes per column and k-block
      sbase[q] = static_cast<const uint8_t*>(a.B) + bpc * (size_t)n0 + 16 * w;
      sstride[q] = bpc * (uint32_t)N;
      srow0[q] = kw + kl;
      sper[q] = KS;
      srmax[q] = nkb - 1;
      slds[q] = kl * BPK * 16 + 16 * w;
    } else if (pc < P1) {
      const int p = pc - NB, kk = p / MPK, w = p % MPK;  // kk: k-block of the wave's share
      const uint8_t* mb = static_cast<const uint8_t*>(a.meta);
      if constexpr (MF == META4) {
        // two parts (units of the column pairs j>>1 = 0, 1), 2*TC bytes each
        const int jbp = w / (MPK / 2), wp = w % (MPK / 2);
        sbase[q] = mb + 256 * (size_t)chunk + 128 * jbp + 16 * g0 + 16 * wp;
        sstride[q] = 4 * (uint32_t)N;
        slds[q] = MOFF + kk * MPK * 16 + jbp * 2 * TC + 16 * wp;
      } else if constexpr (TC == 64) {
        // the whole 48-word group of the chunk
        sbase[q] = mb + 192 * (size_t)chunk + 16 * w;
        sstride[q] = 3 * (uint32_t)N;
        slds[q] = MOFF + kk * MPK * 16 + 16 * w;
      } else {
        // rows (which, which+1) of the group, TC/2 words each starting at word p0
        const int which = g0 >> 2, p0 = (4 * g0) & 15;
        const int row = w / (TC / 8), wp = w % (TC / 8);
        sbase[q] = mb + 192 * (size_t)chunk + 4 * (16 * (which + row) + p0) + 16 * wp;
        sstride[q] = 3 * (uint32_t)N;
        slds[q] = MOFF + kk * MPK * 16 + row * 2 * TC + 16 * wp;
      }
      srow0[q] = kw + kk;
      sper[q] = KS;
      srmax[q] = nkb - 1;
    } else if (pc < P2) {
      const int p = pc - P1, gl = p / SPG, w = p % SPG;  // gl = 0: the wave's one group
      sbase[q] = reinterpret_cast<const uint8_t*>(a.s) + 2 * (size_t)n0 + 16 * w;
      sstride[q] = 2 * (uint32_t)N;
      srow0[q] = (kw >> 2) + gl;
      sper[q] = KS / 4;
      srmax[q] = ngroups - 1;
      slds[q] = SOFF + gl * 2 * TC + 16 * w;
    } else {
      const int p = pc - P2, kk = p / (4 * MB), m = (p >> 2) % MB, u = p & 3;
      const int mm = m < M ? m : M - 1;
      sbase[q] = reinterpret_cast<const uint8_t*>(a.A) + 2 * (size_t)mm * K + 16 * u;
      sstride[q] = 64;
      srow0[q] = kw + kk;
      sper[q] = KS;
      srmax[q] = nkb - 1;
      slds[q] = AOFF + (kk * MB + m) * 64 + 16 * u;
      szero[q] = true;
    }
  }
  // Every slot of every wave holds pieces (the last one repeats its final piece in
  // surplus lanes): loads are never under a branch, so the compiler's waits stay
  // exact.
  // Activation pieces past the last k-block read the zero buffer (an address select:
  // a select on the loaded value would wait for the load right away).
  const uint8_t* zeros = reinterpret_cast<const uint8_t*>(a.zeros);
  auto load_slot = [&](int q, int s) -> u32x4 {
    const uint32_t row = (uint32_t)(st0 + s) * sper[q] + srow0[q];
    const uint32_t r = row < srmax[q] ? row : srmax[q];
    const uint8_t* p = sbase[q] + (uint64_t)r * sstride[q];
    if (q * 64 + 64 > P2) {  // the slot may hold activation pieces
      if (szero[q] && row > srmax[q]) p = zeros;
    }
    return *reinterpret_cast<const u32x4*>(p);
  };

  // ---- MFMA lane roles ----
  const int h = lane >> 4;
  const int rho = lane & 15;   // A row = column n0 + 16*cb + rho; B column = batch row
  const int gl = rho >> 3, blk = (rho >> 2) & 1, j = rho & 3;
  const int jb = j >> 1, jj = j & 1;
  const int t0 = 2 * (h & 1);
  const int kh = h >> 1;                             // k-block of the pair
  const int au = kh | ((h & 1) << 1);                // activation piece of a k-block row
  const uint32_t nsh = 8u * blk;                     // byte shift: column half in a value word
  // metadata unit bytes -> index halfword: [byte h&1 of int16 blk, of int16 2 + blk]
  const uint32_t msel = (uint32_t)(2 * blk + (h & 1)) | ((uint32_t)(4 + 2 * blk + (h & 1)) << 8) | 0x0c0c0000u;
  // 3-bit metadata: bit position of the lane's two codes in its code word, the
  // 64-bit shifts that bring them to bit 0 (code word of field "first" / "second",
  // jb = 0 / 1 half), and its half's nibble table as 8 bytes
  const uint32_t m3pos = 3u * (4u * blk + 2u * (h & 1));
  const uint32_t m3s0 = (jb ? 24u : 0u) + m3pos, m3s1 = (jb ? 40u : 16u) + m3pos;
  const uint32_t m3tlo = jb ? kTabLowLo : kTabHighLo, m3thi = jb ? kTabLowHi : kTabHighHi;
  const int arow = rho & (MB - 1);                   // staged activation row (lanes rho < MB)

  // Per-lane LDS byte offsets of this wave's first k-block and column block; the
  // k-block pair (q2), column block (cb) and buffer parts are immediates.
  // (offsets within the wave's own stage region)
  const uint32_t o_val = kh * (BPK * 16) + (VF == VAL4 ? 4 * (16 * gl + 4 * t0 + j) : 0);
  const int wi_lane = 16 * gl + 4 * t0 + j;           // 3-bit values: word index without cb
  const uint32_t o_meta = MOFF + kh * (MPK * 16) + jb * 2 * TC + 8 * (2 * gl + jj);
  const uint32_t o_mrow = MOFF + kh * (MPK * 16);
  const uint32_t o_scale = SOFF + 2 * (8 * gl + 2 * j + blk);
  const uint32_t o_act = AOFF + arow * 64 + 16 * au;
  // Dequant constants held in VGPRs, so that mask-and-or is one v_and_or_b32.
  uint32_t kMask, kMaskHi, kMagic;
  if constexpr (VF == VAL4) {
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
    asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));
  } else {  // 3-bit codes at bits 0 / 16 and 3 / 19 of a half pair
    asm volatile("v_mov_b32 %0, 0x00070007" : "=v"(kMask));
    asm volatile("v_mov_b32 %0, 0x00380038" : "=v"(kMaskHi));
  }
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));

  // one accumulator per k-block pair of a wave's share (no MFMA dependency chains)
  constexpr int KP = KPW / 2;
  float4_t acc[KP][NCB][RB];
#pragma unroll
  for (int q = 0; q < KP; q++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) acc[q][cb][rb] = (float4_t){0.f, 0.f, 0.f, 0.f};

  half8_t sact[KPW];  // staged activation operands (lanes rho >= MB never reload)
#pragma unroll
  for (int q = 0; q < KPW; q++) sact[q] = (half8_t){};
  // resident row of the lane (rho < M), at the wave's first k-block of stage 0
  const uint32_t o_ract = (uint32_t)arow * RS + (uint32_t)kw * 64u + 16u * au;

  // st: the wave's stage buffer; aoff: byte offset of the stage in the resident rows
  auto compute = [&](const uint8_t* st, uint32_t aoff) {
    // Every LDS operand of the stage is read before the first is used (the larger
    // batches run one or two waves per SIMD, where a read per use exposes its whole
    // latency)
    uint32_t xr[KP][NCB][2];
    uint32_t x3[KP][NCB][4];  // 3-bit values: the two word pairs of the lane's fields
    // 3-bit metadata: the code word of metadata word u = 32*jb + 4*g + 2*jj + ehalf
    // is the low (jb = 0) or high 24 bits of field "first" (g < 4) or "second"
    // (g >= 4) at position P = u mod 16, in words (which, which+1); its two codes at
    // pos and pos + 3 are Y:X shifted by the sum S (m3_shift), as one alignbit of Y:X
    // (S < 32) or of Y:Y by S - 32 (only the low 6 bits are used).  m3_read returns
    // Y and the low word L of that alignbit.
    auto m3_which = [&](int cb) -> int { return TC == 64 ? (2 * cb + gl) >> 2 : g0 >> 2; };
    auto m3_shift = [&](int cb) -> uint32_t { return m3_which(cb) == 0 ? m3s0 : m3s1; };
    auto m3_read = [&](const uint8_t* stp, int q2, int cb, int ehalf, uint32_t& Y, uint32_t& L) {
      const uint32_t* mrow = reinterpret_cast<const uint32_t*>(stp + o_mrow + 2 * q2 * (MPK * 16));
      const int gt = 2 * cb + gl;
      int ix, iy;  // words X = mrow[ix], Y = mrow[iy]
      if constexpr (TC == 64) {
        ix = 16 * m3_which(cb) + ((4 * gt + 2 * jj + ehalf) & 15);
        iy = ix + 16;
      } else {
        ix = 4 * gt + 2 * jj + ehalf;
        iy = ix + TC / 2;
      }
      Y = mrow[iy];
      L = mrow[m3_shift(cb) >= 32u ? iy : ix];
    };
    uint32_t m3y[KP][NCB][2], m3l[KP][NCB][2];
    u32x2 mr[KP][NCB];
    _Float16 sr[NCB];
    {
#pragma unroll
      for (int q2 = 0; q2 < KP; q2++) {
        if constexpr (RES) {
          if (rho < M) {
            const uint8_t* ap = dyn_lds + o_ract + aoff + 2 * q2 * 64;
            sact[2 * q2] = *reinterpret_cast<const half8_t*>(ap);
            sact[2 * q2 + 1] = *reinterpret_cast<const half8_t*>(ap + 64);
          }
        } else if (rho < MB) {
          sact[2 * q2] = *reinterpret_cast<const half8_t*>(st + o_act + 2 * q2 * MB * 64);
          sact[2 * q2 + 1] = *reinterpret_cast<const half8_t*>(st + o_act + (2 * q2 + 1) * MB * 64);
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
            for (int ehalf = 0; ehalf < 2; ehalf++) m3_read(st, q2, cb, ehalf, m3y[q2][cb][ehalf], m3l[q2][cb][ehalf]);
          }
        }
      if constexpr (GROUPED) {
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) sr[cb] = *reinterpret_cast<const _Float16*>(st + o_scale + 32 * cb);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q2 = 0; q2 < KP; q2++) {
      // Only lanes of real batch rows read the staged row; the other lanes' MFMA
      // columns are never stored, so their operand keeps whatever the register held
      // (LDS reads are paid per active lane).
      half16_t act[RB];
      act[0] = __builtin_shufflevector(sact[2 * q2], sact[2 * q2 + 1], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14,
                                       15);
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        // values: bytes blk, blk+2 of words t0, t0+1; low nibbles -> groups t0, t0+1,
        // high nibbles (16x) -> groups t0+4, t0+5, each {slot 0, slot 1}; as halves
        // 1024 + q (lo) and 1024 + 16q (hi) by the magic-number trick
        uint32_t lo0, lo1, hi0, hi1;
        if constexpr (VF == VAL4) {
          // words t0 and t0+1 of the lane's k-block row
          const uint32_t x0 = xr[q2][cb][0] >> nsh;
          const uint32_t x1 = xr[q2][cb][1] >> nsh;
          lo0 = (x0 & kMask) | kMagic;
          lo1 = (x1 & kMask) | kMagic;
          hi0 = (x0 & kMaskHi) | kMagic;
          hi1 = (x1 & kMaskHi) | kMagic;
        } else {
          // 3-bit codes: word w is the 24-bit field at byte 3w of the row, nibble p at
          // bits 3p.  Shifted by 6 blk, the lane's four codes (nibbles 2blk, 2blk+1,
          // 4+2blk, 5+2blk) sit at bits 0, 3, 12, 15.
          const int b0 = 3 * (wi_lane + 32 * cb), b1 = b0 + 12;
          const uint32_t y0 = __builtin_amdgcn_alignbit(x3[q2][cb][1], x3[q2][cb][0], 8 * (b0 & 3) + 6 * blk);
          const uint32_t y1 = __builtin_amdgcn_alignbit(x3[q2][cb][3], x3[q2][cb][2], 8 * (b1 & 3) + 6 * blk);
          // One shift and one bit-field insert move the codes at bits 12 and 15 up to
          // 16 and 19, so that each half pair's codes sit 16 bits apart: masked and
          // or-ed with the magic exponent they are the halves 1024 + c (bits 0 / 16)
          // and 1024 + 8c (bits 3 / 19), both exact.
          const uint32_t z0 = (y0 & 0x0000FFFFu) | ((y0 << 4) & 0xFFFF0000u);
          const uint32_t z1 = (y1 & 0x0000FFFFu) | ((y1 << 4) & 0xFFFF0000u);
          lo0 = (z0 & kMask) | kMagic;
          lo1 = (z1 & kMask) | kMagic;
          hi0 = (z0 & kMaskHi) | kMagic;
          hi1 = (z1 & kMaskHi) | kMagic;
        }
        constexpr float zp = VF == VAL4 ? 1032.0f : 1028.0f;  // 1024 + zero point
        // the high pair is 1024 + 16 q (4-bit) or 1024 + 8 q (3-bit): times 1/16 (1/8)
        // less 64 (128) and the zero point, exact
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
        // metadata: byte h&1 of int16s blk (groups 0-3) and 2 + blk (groups 4-7) of
        // unit 16*jb + 2*gt + jj
        uint32_t idx;
        if constexpr (MF == META4) {
          const u32x2 unit = mr[q2][cb];
          idx = __builtin_amdgcn_perm(unit.y, unit.x, msel);
        } else {
          // 3-bit code word of metadata word u = 32*jb + 4*g + 2*jj + ehalf: the low
          // (jb = 0) or high 24 bits of field "first" (g < 4) or "second" (g >= 4)
          // at position P = u mod 16, in words (which, which+1).  The lane's two codes
          // of each ehalf go to selector bytes of one v_perm over the 8-byte nibble
          // table of its half (jb), which returns the four index nibbles as bytes,
          // then folded into the index halfword.
          uint32_t v[2];
#pragma unroll
          for (int ehalf = 0; ehalf < 2; ehalf++) {
            v[ehalf] = __builtin_amdgcn_alignbit(m3y[q2][cb][ehalf], m3l[q2][cb][ehalf], m3_shift(cb) & 31u);
          }
          // selector bytes {ca0, ca1, cb0, cb1} (code a / b of ehalf 0 / 1): the low
          // bytes of v[0], v[1] side by side, their b codes moved up by 13 bits
          const uint32_t s2 = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0400u);
          const uint32_t sel = (s2 | (s2 << 13)) & 0x07070707u;
          const uint32_t nib = __builtin_amdgcn_perm(m3thi, m3tlo, sel);  // the four nibbles as bytes
          idx = (nib & 0x0f0fu) | ((nib >> 12) & 0xf0f0u);                 // byte e: a | b << 4 of ehalf e
        }
        if constexpr (GROUPED) {
          const _Float16 sc = sr[cb];
          aop = aop * (half8_t){sc, sc, sc, sc, sc, sc, sc, sc};
        }
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
          acc[q2][cb][rb] = smfmac64<0>(aop, act[rb], acc[q2][cb][rb], idx);
          // 64-column tiles: keep each accumulator in one register set across the
          // unrolled stages (without this pin the register allocator alternates two
          // sets and copies every accumulator once per stage: 3 v_mov per MFMA)
          if constexpr (TC == 64) asm volatile("" : "+v"(acc[q2][cb][rb]));
        }
      }
    }
  };

  // ---- pipeline: ring of D stages ----
  // The prologue loads stages 0..D-1 and every full round of D stages loads the
  // stages D later, all unconditionally (stages past the end re-read the last rows:
  // the waits stay exact, which a conditional load would spoil).  The final round
  // issues no loads.
  sp.mark(2);
  u32x4 ring[D][SL];
#pragma unroll
  for (int i = 0; i < D; i++) {
#pragma unroll
    for (int q = 0; q < SL; q++)
      ring[i][q] = load_slot(q, i);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (RES) {
    // every wave's activation DMAs have landed: issued before the D * LPS ring loads,
    // they are older than every load still allowed in flight
    wait_vm<D * LPS>();
    __syncthreads();
  }
  sp.mark(3);
  uint8_t* const wlds = lds + wall * 2 * STAGE;  // this wave's two stage buffers
  auto stage = [&](int i, bool reload, int s) {
    uint8_t* st = wlds + (i & 1) * STAGE;
#pragma unroll
    for (int q = 0; q < SL; q++) {
      *reinterpret_cast<u32x4*>(st + slds[q]) = ring[i][q];
      if (reload) ring[i][q] = load_slot(q, s + D);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(st, (uint32_t)s * (KS * 64));
    __builtin_amdgcn_sched_barrier(0);
  };
  int base = 0;
  for (; base + D < nst; base += D) {
#pragma unroll
    for (int i = 0; i < D; i++) stage(i, true, base + i);
  }
#pragma unroll
  for (int i = 0; i < D; i++)
    if (base + i < nst) stage(i, false, base + i);  // uniform
  sp.mark(4);

#pragma unroll
  for (int q = 1; q < KP; q++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int rb = 0; rb < RB; rb++) acc[0][cb][rb] += acc[q][cb][rb];

  // ---- reduce the NW waves in LDS, one 16-row block at a time: every wave stores its
  // partial tile, then thread t < 4*TC adds the NW partials of 4 columns of one row in
  // wave order (fixed, so results are deterministic) and writes them (to C, or with
  // split-K to this split's fp32 partial in the uncached scratch) ----
  float* const red = reinterpret_cast<float*>(lds) + grp * (REDB / 4);  // this tile's
  const int r_out = tid / (TC / 4), c_out = 4 * (tid % (TC / 4));  // for tid < 4*TC
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
  // partial of (tile, split, rb): 16 x TC floats in row-major order
  auto partial_at = [&](int zz, int rb) -> float* {
    return a.partial + ((size_t)(ptile * S + zz) * RB + rb) * (16 * TC) + r_out * TC + c_out;
  };
#pragma unroll
  for (int rb = 0; rb < RB; rb++) {
    __syncthreads();  // the last stage's (or the previous block's) LDS reads are done
    // only the rows of real batch rows are stored, summed and written
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
  if (G == 1 && S > 1) {
    // hand-off: each thread's partial stores complete before the workgroup barrier;
    // the tile's counter is bumped after it; the last split to arrive adds all splits'
    // partials in split order (bit-identical whichever arrives last), writes C and
    // resets the counter
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    __shared__ uint32_t arrived;
    if (tid == 0) arrived = __hip_atomic_fetch_add(a.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __syncthreads();
    if (arrived != (uint32_t)S) {
      sp.store(a.spans, NW * G, wall, lane);
      return;
    }
    if (tid == 0) __hip_atomic_store(a.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 4 * TC && r_out < M) {
      // up to four splits' partials per batch of loads (the uncached reads are
      // latency-bound: one wait per batch, not per split)
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
  sp.store(a.spans, NW * G, wall, lane);
}

}  // namespace sm24
