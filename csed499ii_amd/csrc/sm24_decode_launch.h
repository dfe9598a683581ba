// Launchers of the decode kernels (sm24_decode.h for 1, 4 and 8 padded rows,
// sm24_decode_dma.h for 16 and 32), instantiated per tile width in sm24_decode_16.hip,
// sm24_decode_32.hip and sm24_decode_64.hip so that the library's translation units
// compile in parallel; sm24_gemm.hip's launch_decode dispatches to them.
#pragma once
#include "sm24_decode.h"
#include "sm24_decode_dma.h"
#include "sm24_host.h"

namespace sm24 {

// Static LDS bytes of a kernel (cached per instantiation by the caller).
inline size_t static_lds(const void* fn) {
  hipFuncAttributes attr{};
  return hipFuncGetAttributes(&attr, fn) == hipSuccess ? attr.sharedSizeBytes : SIZE_MAX;
}

// Batches of up to 4 rows keep their activation rows resident in LDS (one copy per
// workgroup, loaded once: every stage's loads are weight pieces only) when a
// workgroup runs at least 8 stages and the rows of its k range fit beside the
// kernel's static LDS in 64 KiB, or in the CU's whole 160 KiB where the grid has at
// most one workgroup per CU; otherwise each stage carries its activation pieces.
// Measured on the Llama-2-7B shapes at M in {1, 2, 4}: 0.03-0.47 us faster per call
// from 8 stages up (gate_up at M = 2: 10.09 -> 9.62 us), 0.07-0.23 us slower for o
// 4096x4096 (4 stages of 32 k-blocks: the copy and its barrier are not amortised).
// Beyond 64 KiB at one workgroup per CU: 7B down 11008x4096 at M = 2 / 4 (90 KiB of
// rows) 7.01 -> 6.72 / 7.55 -> 7.18 us, Llama-2-70B o 8192x8192 (66 KiB) 8.63 ->
// 7.47 / 8.64 -> 7.75 us; at two per CU (70B down, 57 KiB of rows each) it was
// slower (20.05 -> 20.60 us at M = 4), so that case keeps the rows per stage.
// MARLIN_HIP_DECODE_RES=0 turns it off.
constexpr size_t kDecodeLdsMax = 64 * 1024;
constexpr size_t kCuLds = 160 * 1024;  // LDS of one gfx950 compute unit
template <int TC, int NW, int MB, bool GROUPED, int VF, int MF, bool DEEP, int G = 1>
void launch_decode_v(const GemmArgs& a, int cus, hipStream_t stream) {
  const int ntiles = a.N / TC;
  const dim3 grid(G > 1 ? ntiles / G
                        : a.tail_from > 0 ? a.tail_from + (ntiles - a.tail_from) * a.splits : ntiles * a.splits);
  const dim3 block(64 * NW * G);
  if constexpr (MB >= 16) {
    // 16 and 32 padded rows: the LDS-DMA kernel (sm24_decode_dma.h).  Its activation
    // pieces travel with each stage into LDS; against the register-ring kernel with
    // direct activation operands (same tile table, same box): Llama-2-7B at M = 16 qkv
    // 8.37 -> 7.71, o 6.54 -> 5.88, gate_up 12.21 -> 11.35, down 9.30 -> 8.71 us.
    hipLaunchKernelGGL((sm24_decode_dma_kernel<TC, NW, MB, GROUPED, VF, MF, DEEP>), grid, block, 0, stream,
                       a.B, a.meta, a.s, a.A, a.zeros, a.M, a.N, a.K, a.splits, a);
  } else {
    static const int forced_res = env_choice("MARLIN_HIP_DECODE_RES", {0, 1}, 1);
    constexpr int ks = NW * (64 / TC > 2 ? 64 / TC : 2);
    const int nst_all = (a.K / 32 + ks - 1) / ks;
    const int nst_max = a.tail_from > 0 ? nst_all : (nst_all + a.splits - 1) / a.splits;
    const size_t dyn = (size_t)MB * ((size_t)nst_max * ks * 64 + 16);
    static const size_t stat =
        static_lds(reinterpret_cast<const void*>(&sm24_decode_kernel<TC, NW, MB, GROUPED, VF, MF, DEEP, true, G>));
    const bool fits = stat <= kCuLds && dyn <= kCuLds - stat &&
                      (stat + dyn <= kDecodeLdsMax || (cus > 0 && grid.x <= (unsigned)cus));
    if (forced_res == 1 && nst_max >= 8 && fits) {
      hipLaunchKernelGGL((sm24_decode_kernel<TC, NW, MB, GROUPED, VF, MF, DEEP, true, G>), grid, block, dyn, stream,
                         a.B, a.meta, a.s, a.A, a.zeros, a.M, a.N, a.K, a.splits, a);
      return;
    }
    hipLaunchKernelGGL((sm24_decode_kernel<TC, NW, MB, GROUPED, VF, MF, DEEP, false, G>), grid, block, 0, stream,
                       a.B, a.meta, a.s, a.A, a.zeros, a.M, a.N, a.K, a.splits, a);
  }
}

template <int TC, int NW, int MB, bool GROUPED>
void launch_decode_mb(const GemmArgs& a, bool deep, int vf, int mf, int cus, hipStream_t stream) {
  if (vf == VAL3) {
    if (deep) launch_decode_v<TC, NW, MB, GROUPED, VAL3, META4, true>(a, cus, stream);
    else launch_decode_v<TC, NW, MB, GROUPED, VAL3, META4, false>(a, cus, stream);
  } else if (mf == META3) {
    if (deep) launch_decode_v<TC, NW, MB, GROUPED, VAL4, META3, true>(a, cus, stream);
    else launch_decode_v<TC, NW, MB, GROUPED, VAL4, META3, false>(a, cus, stream);
  } else {
    if (deep) launch_decode_v<TC, NW, MB, GROUPED, VAL4, META4, true>(a, cus, stream);
    else launch_decode_v<TC, NW, MB, GROUPED, VAL4, META4, false>(a, cus, stream);
  }
}

template <int TC, int NW, bool GROUPED>
void launch_decode_nw(const GemmArgs& a, int mb, bool deep, int vf, int mf, int cus, hipStream_t stream) {
  if (mb == 1) launch_decode_mb<TC, NW, 1, GROUPED>(a, deep, vf, mf, cus, stream);
  else if (mb == 4) launch_decode_mb<TC, NW, 4, GROUPED>(a, deep, vf, mf, cus, stream);
  else if (mb == 8) launch_decode_mb<TC, NW, 8, GROUPED>(a, deep, vf, mf, cus, stream);
  else if (mb == 16) launch_decode_mb<TC, NW, 16, GROUPED>(a, deep, vf, mf, cus, stream);
  else launch_decode_mb<TC, NW, 32, GROUPED>(a, deep, vf, mf, cus, stream);
}

// Three 16-column tiles of 4 waves per workgroup, 1 or 4 padded rows.
template <bool GROUPED, int VF, int MF>
void launch_decode_g3(const GemmArgs& a, int mb, int cus, hipStream_t stream) {
  if (mb == 1) launch_decode_v<16, 4, 1, GROUPED, VF, MF, false, 3>(a, cus, stream);
  else launch_decode_v<16, 4, 4, GROUPED, VF, MF, false, 3>(a, cus, stream);
}

template <int TC, bool GROUPED>
hipError_t launch_decode_t(const GemmArgs& a, const DecodeShape& d, int vf, int mf, hipStream_t stream) {
  const int mb = d.mb >= decode_batch(a.M) ? d.mb : decode_batch(a.M);
  if constexpr (TC == 16) {
    // three tiles per workgroup (decode_shape sets g = 3 only for these shapes)
    if (d.g == 3 && d.nw == 4 && !d.deep && (mb == 1 || mb == 4)) {
      if (vf == VAL3) launch_decode_g3<GROUPED, VAL3, META4>(a, mb, d.cus, stream);
      else if (mf == META3) launch_decode_g3<GROUPED, VAL4, META3>(a, mb, d.cus, stream);
      else launch_decode_g3<GROUPED, VAL4, META4>(a, mb, d.cus, stream);
      return hipGetLastError();
    }
  }
  if (d.nw == 4) launch_decode_nw<TC, 4, GROUPED>(a, mb, d.deep, vf, mf, d.cus, stream);
  else launch_decode_nw<TC, 8, GROUPED>(a, mb, d.deep, vf, mf, d.cus, stream);
  return hipGetLastError();
}

// One tile width's launchers (both scale modes) per translation unit.
#define SM24_DECODE_INSTANTIATE(TC)                                                                   \
  template hipError_t launch_decode_t<TC, true>(const GemmArgs&, const DecodeShape&, int, int, hipStream_t); \
  template hipError_t launch_decode_t<TC, false>(const GemmArgs&, const DecodeShape&, int, int, hipStream_t);

}  // namespace sm24
