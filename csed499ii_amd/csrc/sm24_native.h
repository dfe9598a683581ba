// Lane-native packed layout for decode, and its GEMM kernel (M <= 16).
//
// This layout is this library's own (an offline repack of the reference pack()
// layout, exactly invertible); the reference has no counterpart.  Per 16-column
// block c16 (columns n = 16 c16 + rho) and 256-deep quad q of dense K (k-pairs
// 4q + j, j = 0..3, 64 dense K each), lane l = 16 h + rho of the v_smfmac_f32_16x16x64_f16
// A operand owns:
//
//   W[(c16 * K/256 + q) * 64 + l]  u32x4: word j = the 8 compressed values of
//        column n, dense K 64(4q+j) + 16h .. +16 (4 groups of 4, 2 values each),
//        value e at nibble native_nibble(e) (the order in which the magic-number
//        dequantization of the word and of word >> 8 yields operand halves 0..7);
//   X[(c16 * K/256 + q) * 64 + l]  u32x2: halfword j = the logical 2:4 metadata
//        int16 of those 4 groups (the smfmac index set, selected by ABID = j & 1);
//   S[(c16 * K/256 + q) * 16 + rho] u32: fp16 scales of column n for groups 2q
//        (low half) and 2q+1 (high half), groupsize 128; with groupsize -1 the
//        N per-column scales in natural order instead.
//
// Bytes are those of the reference layout (values K*N/4, metadata K*N/8, scales
// K*N/64), but every operand word sits where its lane loads it: a wave reads 1 KiB
// of values, 512 B of metadata and 64 B of scales per quad with three coalesced
// loads straight into its registers, with no LDS staging and no per-stage barrier.
#pragma once
#include "sm24_device.h"

namespace sm24 {

// Nibble of a lane word that holds compressed value e of the lane.
__host__ __device__ constexpr int native_nibble(int e) { return (e & 1) * 4 + (e >> 1); }

struct NativeArgs {
  const _Float16* A;        // [M][K] activations
  const u32x4* W;           // lane-native values
  const u32x2* X;           // lane-native metadata
  const uint32_t* S;        // lane-native scales (groupsize 128)
  const _Float16* s_col;    // per-column scales (groupsize -1), natural order
  _Float16* C;              // [M][N]
  float* partial;           // split-K: [tiles][splits][NCB][MB][16] fp32
  uint32_t* counters;       // split-K: [tiles] arrival counters, zero between launches
  int M, N, K, splits;
};

// ---- repack kernels (reference layout <-> lane-native layout) ----

// Physical int16 index of logical metadata meta[n][c] (n < N, c < K/16) in the
// reference's reordered metadata (_semi_structured_conversions.py:21-48): the row
// swizzle inside 64-row groups, the 2x2 transpose, ColumnMajorInterleaved<2>.
__host__ __device__ inline size_t meta_phys_index(int n, int c, int N) {
  const int a = (n & 63) >> 3, b = (n & 7) >> 2, cb = (n & 3) >> 1, d = n & 1;
  const int r2 = (n >> 6) * 64 + 2 * d + b + 32 * cb + 4 * a;
  const int shift = ((r2 & 1) == 0 && (c & 1) == 1) ? 1 : (((r2 & 1) == 1 && (c & 1) == 0) ? -1 : 0);
  const int r3 = r2 + shift, c3 = c - shift;
  return (size_t)(c3 >> 1) * (size_t)N * 2 + (size_t)r3 * 2 + (c3 & 1);
}

// Position, within a 64-column chunk of the reference's packed scales, of column u
// (the inverse of scale_perm, __init__.py:262-265: slot 8a + b holds column
// 8a + [0,4,1,5,2,6,3,7][b]).
__host__ __device__ inline int scale_slot(int u) {
  const int b = u & 7;
  return (u & ~7) + ((b & 3) << 1) + (b >> 2);
}

// Word (row r, column w) and nibble p of the reference packed values holding
// compressed value kc of column n (__init__.py:359-386 with the permutation of
// _get_perms_2_4: nibble p of word 128c + 4i + j of row r is kc = 16r + ROW_t[p],
// n = 64c + 8(i/4) + 4 BLK[p] + j, t = i % 4).
__host__ __device__ inline void ref_value_pos(int kc, int n, int N, size_t* word, int* nib) {
  const int r = kc >> 4, v = kc & 15;
  const int t = (v & 7) >> 1, par = v & 1, hi8 = v >> 3;
  const int blk = (n >> 2) & 1, j = n & 3, g = (n & 63) >> 3, c = n >> 6;
  *word = (size_t)r * 2 * N + 128 * c + 4 * (4 * g + t) + j;
  *nib = 4 * par + 2 * blk + hi8;
}

// One thread per (c16, q, lane): the lane's 4 value words and 4 metadata halfwords;
// lanes rho of h == 0 also write the 16 scale words of (c16, q).
__global__ __launch_bounds__(256) void native_pack_kernel(const uint32_t* __restrict__ B,
                                                          const uint16_t* __restrict__ meta,
                                                          const _Float16* __restrict__ s, u32x4* __restrict__ W,
                                                          u32x2* __restrict__ X, uint32_t* __restrict__ S, int N,
                                                          int K, int grouped) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int nq = K >> 8;
  const long long total = (long long)(N >> 4) * nq * 64;
  if (t >= total) return;
  const int lane = (int)(t & 63);
  const long long bq = t >> 6;  // c16 * nq + q
  const int q = (int)(bq % nq), c16 = (int)(bq / nq);
  const int h = lane >> 4, rho = lane & 15;
  const int n = 16 * c16 + rho;
  u32x4 wv;
  uint32_t xh[4];
  for (int j = 0; j < 4; j++) {
    const int kp = 4 * q + j;
    uint32_t word = 0;
    for (int e = 0; e < 8; e++) {
      size_t wi;
      int p;
      ref_value_pos(32 * kp + 8 * h + e, n, N, &wi, &p);
      word |= ((B[wi] >> (4 * p)) & 15u) << (4 * native_nibble(e));
    }
    wv[j] = word;
    xh[j] = meta[meta_phys_index(n, 4 * kp + h, N)];
  }
  W[t] = wv;
  X[t] = (u32x2){xh[0] | (xh[1] << 16), xh[2] | (xh[3] << 16)};
  if (grouped && h == 0) {
    const size_t c0 = (size_t)(n & ~63) + scale_slot(n & 63);
    const uint16_t lo = __builtin_bit_cast(uint16_t, s[(size_t)(2 * q) * N + c0]);
    const uint16_t hi = __builtin_bit_cast(uint16_t, s[(size_t)(2 * q + 1) * N + c0]);
    S[bq * 16 + rho] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
}

// Inverse, values: one thread per reference word.
__global__ __launch_bounds__(256) void native_unpack_values_kernel(const uint32_t* __restrict__ W,
                                                                   uint32_t* __restrict__ B, int N, int K) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)(K >> 5) * 2 * N;
  if (t >= total) return;
  const int r = (int)(t / (2 * N)), w = (int)(t % (2 * N));
  const int c = w >> 7, i = (w & 127) >> 2, j = w & 3, g = i >> 2, ti = i & 3;
  const int nq = K >> 8;
  uint32_t word = 0;
  for (int p = 0; p < 8; p++) {
    const int off = 2 * ti + ((p & 4) ? 1 : 0) + ((p & 1) ? 8 : 0);  // ROW_t[p]
    const int kc = 16 * r + off;
    const int n = 64 * c + 8 * g + 4 * ((p >> 1) & 1) + j;
    const int kp = kc >> 5, h = (kc & 31) >> 3, e = kc & 7;
    const size_t lw = (((size_t)(n >> 4) * nq + (kp >> 2)) * 64 + 16 * h + (n & 15)) * 4 + (kp & 3);
    word |= ((W[lw] >> (4 * native_nibble(e))) & 15u) << (4 * p);
  }
  B[t] = word;
}

// Inverse, metadata and scales: one thread per logical metadata int16 (n, c); the
// threads of c < K/128 also write the packed scale of group c and column n.
__global__ __launch_bounds__(256) void native_unpack_meta_kernel(const u32x2* __restrict__ X,
                                                                 const uint32_t* __restrict__ S,
                                                                 uint16_t* __restrict__ meta,
                                                                 _Float16* __restrict__ s, int N, int K,
                                                                 int grouped) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int nc = K >> 4;
  const long long total = (long long)N * nc;
  if (t >= total) return;
  const int n = (int)(t / nc), c = (int)(t % nc);
  const int nq = K >> 8;
  const int kp = c >> 2, h = c & 3;
  const size_t lane_q = ((size_t)(n >> 4) * nq + (kp >> 2)) * 64 + 16 * h + (n & 15);
  const int j = kp & 3;
  const u32x2 xv = X[lane_q];
  meta[meta_phys_index(n, c, N)] = (uint16_t)((xv[j >> 1] >> (16 * (j & 1))) & 0xffffu);
  if (grouped && c < (K >> 7)) {
    const uint32_t sv = S[((size_t)(n >> 4) * nq + (c >> 1)) * 16 + (n & 15)];
    const uint16_t half = (uint16_t)((sv >> (16 * (c & 1))) & 0xffffu);
    s[(size_t)c * N + (n & ~63) + scale_slot(n & 63)] = __builtin_bit_cast(_Float16, half);
  }
}

// ---- GEMM over the lane-native layout, M <= MB (1, 4, 8 or 16) ----
//
// Workgroup: NCB 16-column blocks (a tile of 16 NCB columns) over the quads
// [q0, q1) of its K split; wave w takes quads q0 + w, q0 + w + NW, ... and streams
// them through a ring of D register slots (values, metadata and scales of one quad
// of every block, and the quad's MB activation rows), issued D quads ahead.  When a
// quad is due the wave writes its activation rows to its own LDS slot and reads them
// back in B-operand order (two 16-byte pieces per lane and k-pair, shared by the NCB
// blocks); one wave's LDS operations complete in order, so no barrier is needed and
// waves never wait on each other until the end.  Each quad is 4 smfmacs per block
// into 4 accumulators.  At the end the NW partial tiles are added in LDS in wave
// order (deterministic), and with split-K handed off as in the decode kernel.
// The fields the prologue needs first come as leading scalar arguments, preloaded
// into SGPRs (the translation unit is built with -mllvm
// -amdgpu-kernarg-preload-count=14), ahead of the whole NativeArgs; the fp16
// pointers travel as void pointers, which keeps the kernel's name demangleable.
template <int MB, int NCB, int NW, int D, bool GROUPED>
__global__ __launch_bounds__(64 * NW) void sm24_native_decode_kernel(const void* A_, const u32x4* W_, const u32x2* X_,
                                                                     const uint32_t* S_, const void* s_col_, int M_,
                                                                     int N_, int K_, int splits_, NativeArgs a_) {
  NativeArgs a = a_;
  a.A = static_cast<const _Float16*>(A_);
  a.W = W_;
  a.X = X_;
  a.S = S_;
  a.s_col = static_cast<const _Float16*>(s_col_);
  a.M = M_;
  a.N = N_;
  a.K = K_;
  a.splits = splits_;
  extern __shared__ __attribute__((aligned(16))) uint8_t nlds[];
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 4, rho = lane & 15;
  const int N = a.N, K = a.K, M = a.M, S = a.splits;
  const int nq = K >> 8;
  const int tile = blockIdx.x, z = blockIdx.y;  // grid (N / (16 NCB), splits)
  int q0 = 0, nqs = nq;                          // quads of this split (>= 1: the host keeps S <= nq)
  if (S > 1) {
    q0 = (int)((unsigned)(nq * z) / (unsigned)S);
    nqs = (int)((unsigned)(nq * (z + 1)) / (unsigned)S) - q0;
  }
  const int nr = (nqs - wave + NW - 1) / NW;  // quads of this wave (>= 0)

  // Ring slots: the quad of round r of this wave (clamped to the split's last):
  // values, metadata and scales of each block, and the quad's MB activation rows
  // (256 halves each), which the wave stages in its own LDS slot when the quad is
  // due (no workgroup barrier: only this wave reads it).
  constexpr int AP = MB * 32;                  // 16-byte activation pieces per quad
  constexpr int APL = (AP + 63) / 64;          // pieces per lane
  constexpr int SLOTB = MB * 512;              // LDS bytes of one staged quad
  u32x4 rw[D][NCB];
  u32x2 rx[D][NCB];
  uint32_t rs[D][NCB];
  u32x4 ra[D][APL];
  const size_t qbase = (size_t)tile * NCB * nq + q0;
  const u32x4* a4 = reinterpret_cast<const u32x4*>(a.A);
  // activation piece p of a quad: row p / 32 (clamped to M - 1), 16 bytes at 8 (p % 32)
  size_t arow_off[APL];
#pragma unroll
  for (int i = 0; i < APL; i++) {
    const int p = (lane + 64 * i) % AP;
    const int m = p >> 5;
    arow_off[i] = ((size_t)(m < M ? m : M - 1) * K + ((size_t)q0 << 8)) / 8 + (p & 31);
  }
  auto load = [&](int d, int r) {
    int ql = wave + r * NW;
    ql = ql < nqs ? ql : nqs - 1;
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      const size_t b = qbase + (size_t)cb * nq + ql;
      rw[d][cb] = a.W[b * 64 + lane];
      rx[d][cb] = a.X[b * 64 + lane];
      if constexpr (GROUPED) rs[d][cb] = a.S[b * 16 + rho];
    }
#pragma unroll
    for (int i = 0; i < APL; i++) ra[d][i] = a4[arow_off[i] + (size_t)ql * 32];
  };
#pragma unroll
  for (int d = 0; d < D; d++) load(d, d);

  uint32_t kMask, kMaskHi, kMagic;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(kMask));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(kMaskHi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kMagic));
  float4_t acc[4][NCB];
#pragma unroll
  for (int j = 0; j < 4; j++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) acc[j][cb] = (float4_t){0.f, 0.f, 0.f, 0.f};
  // the wave's staging slot; lanes of batch rows >= MB read row 0 (their columns are
  // never stored); rows >= M hold row M-1 (also never stored)
  uint8_t* const aslot = nlds + wave * SLOTB;
  const uint8_t* const arow = aslot + 2 * ((rho < MB ? rho : 0) * 256 + 8 * h);

  auto step = [&](int d, int r, bool reload) {
    // stage the quad's activation rows (each lane its pieces), then read them back in
    // operand order; LDS operations of one wave complete in order
#pragma unroll
    for (int i = 0; i < APL; i++)
      if (lane + 64 * i < AP) *reinterpret_cast<u32x4*>(aslot + 16 * (lane + 64 * i)) = ra[d][i];
    __builtin_amdgcn_wave_barrier();
    half16_t act[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      // B operand of lane (rho, h): dense K 8h..8h+7 and 32+8h..32+8h+7 of k-pair j
      const uint8_t* p = arow + 2 * (64 * j);
      const half8_t lo = *reinterpret_cast<const half8_t*>(p);
      const half8_t hi = *reinterpret_cast<const half8_t*>(p + 64);
      act[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
    }
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      const u32x4 wv = rw[d][cb];
      const u32x2 xv = rx[d][cb];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t w = wv[j], w8 = w >> 8;
        const uint32_t lo0 = (w & kMask) | kMagic, hi0 = (w & kMaskHi) | kMagic;
        const uint32_t lo1 = (w8 & kMask) | kMagic, hi1 = (w8 & kMaskHi) | kMagic;
        const half2_t kz = {(_Float16)1032.0f, (_Float16)1032.0f};
        const half2_t k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
        const half2_t kzh = {(_Float16)-72.0f, (_Float16)-72.0f};
        const half2_t l0 = __builtin_bit_cast(half2_t, lo0) - kz;
        const half2_t l1 = __builtin_bit_cast(half2_t, lo1) - kz;
        const half2_t u0 = __builtin_bit_cast(half2_t, hi0) * k16 + kzh;
        const half2_t u1 = __builtin_bit_cast(half2_t, hi1) * k16 + kzh;
        half8_t aop = (half8_t){l0.x, l0.y, u0.x, u0.y, l1.x, l1.y, u1.x, u1.y};
        if constexpr (GROUPED) {
          const half2_t sc2 = __builtin_bit_cast(half2_t, rs[d][cb]);
          const _Float16 sc = sc2[j >> 1];
          aop = aop * (half8_t){sc, sc, sc, sc, sc, sc, sc, sc};
        }
        if (j & 1) acc[j][cb] = smfmac64<1>(aop, act[j], acc[j][cb], xv[j >> 1]);
        else acc[j][cb] = smfmac64<0>(aop, act[j], acc[j][cb], xv[j >> 1]);
        asm volatile("" : "+v"(acc[j][cb]));
      }
    }
    __builtin_amdgcn_wave_barrier();  // the slot's reads are issued before the next quad's writes
    if (reload) load(d, r + D);
  };
  int base = 0;
  for (; base + D < nr; base += D) {
#pragma unroll
    for (int d = 0; d < D; d++) step(d, base + d, true);
  }
#pragma unroll
  for (int d = 0; d < D; d++)
    if (base + d < nr) step(d, base + d, false);  // uniform

  // ---- reduction: lane (rho, h) holds batch row rho, columns 4h..4h+3 of each block ----
  constexpr int TV = NCB * MB * 16;  // outputs of the tile: (block, row, column)
  __syncthreads();                   // every wave is done with the activation rows
  float* red = reinterpret_cast<float*>(nlds);
  if (rho < MB) {
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      const float4_t v = (acc[0][cb] + acc[1][cb]) + (acc[2][cb] + acc[3][cb]);
      *reinterpret_cast<float4_t*>(red + wave * TV + (cb * MB + rho) * 16 + 4 * h) = v;
    }
  }
  __syncthreads();
  // thread tid owns the outputs o = tid + NT i of the tile (block o / (16 MB), batch
  // row (o / 16) % MB, column o % 16)
  constexpr int OPT = (TV + NT - 1) / NT;
  auto write_c = [&](int o, float v) {
    const int m_out = (o >> 4) % MB;
    const int n_out = 16 * (tile * NCB + o / (MB * 16)) + (o & 15);
    if (m_out < M) {
      _Float16 r = (_Float16)v;
      if constexpr (!GROUPED) r = r * a.s_col[n_out];
      a.C[(size_t)m_out * N + n_out] = r;
    }
  };
  float* const pbase = a.partial + (size_t)tile * S * TV;
#pragma unroll
  for (int i = 0; i < OPT; i++) {
    const int o = tid + NT * i;
    if (o < TV) {
      float v = red[o];
#pragma unroll
      for (int w = 1; w < NW; w++) v += red[w * TV + o];
      if (S == 1) write_c(o, v);
      else pbase[(size_t)z * TV + o] = v;
    }
  }
  if (S > 1) {
    // hand-off: the stores complete before the barrier, the tile's counter is bumped
    // after it, and the last split to arrive adds the splits' partials in split order
    // (bit-identical whichever arrives last), writes C and resets the counter
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    __shared__ uint32_t arrived;
    if (tid == 0)
      arrived = __hip_atomic_fetch_add(a.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    __syncthreads();
    if (arrived != (uint32_t)S) return;
    if (tid == 0) __hip_atomic_store(a.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int j = 0; j < OPT; j++) {
      const int o = tid + NT * j;
      if (o < TV) {
        float v = 0.f;
        for (int z0 = 0; z0 < S; z0 += 4) {
          float t[4];
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (z0 + i < S) t[i] = pbase[(size_t)(z0 + i) * TV + o];
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (z0 + i < S) v = z0 + i == 0 ? t[0] : v + t[i];
        }
        write_c(o, v);
      }
    }
  }
}

}  // namespace sm24
