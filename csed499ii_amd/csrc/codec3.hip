// 3-bit codecs of the 2:4 path on gfx950.
//
// (1) 2:4 metadata, 4 -> 3 bits per dense group.  Only 6 of the 16 nibbles are valid
//     2:4 patterns, so every nibble is re-coded as a 3-bit index.  Each group of 64
//     metadata words (the 256 bytes of one 64-column chunk and one 32-deep k-block)
//     becomes 48 words: for p < 16,
//        first  = enc_hi(a[p])    | enc_lo(a[p+32]) << 24    (48 bits)
//        second = enc_hi(a[p+16]) | enc_lo(a[p+48]) << 24
//        out[p] = first[31:0], out[16+p] = first[47:32] | second[15:0] << 16,
//        out[32+p] = second[47:16]
//     Reference: kernel_experiments/sparse_marlin/metadata_decode/codec.cu:7-41 (layout
//     and tables), decoder_dependency/pair.cu:11 (decode tables).
// (2) 3-bit code stream expansion: 128 codes (48 bytes, code i at bit 3i) -> 128
//     nibbles (64 bytes) with dec(x) = {4,4,9,8,E,E,D,C}[x].
//     Reference: kernel_experiments/3bit_encoding/experiment.cu:12-40.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/marlin_hip.h"

namespace sm24 {
void set_error(const std::string& msg);
}

namespace codec3 {

// nibble -> 3-bit code, 8 = not a 2:4 pattern; packed 4 bits per nibble value.
constexpr uint64_t enc_lut(const int (&t)[16]) {
  uint64_t v = 0;
  for (int i = 0; i < 16; i++) v |= (uint64_t)t[i] << (4 * i);
  return v;
}
//                              0  1  2  3  4  5  6  7  8  9 10 11 12 13 14 15
constexpr int kEncHigh[16] = {8, 8, 8, 8, 5, 8, 8, 8, 2, 6, 8, 8, 7, 1, 0, 8};
constexpr int kEncLow[16] = {8, 8, 8, 8, 6, 8, 8, 8, 4, 5, 8, 8, 0, 1, 2, 8};
constexpr uint64_t kEncHighLut = enc_lut(kEncHigh);
constexpr uint64_t kEncLowLut = enc_lut(kEncLow);

constexpr uint32_t dec_lut(const int (&t)[8]) {
  uint32_t v = 0;
  for (int i = 0; i < 8; i++) v |= (uint32_t)t[i] << (4 * i);
  return v;
}
constexpr int kDecHigh[8] = {14, 13, 8, 13, 3, 4, 9, 12};
constexpr int kDecLow[8] = {12, 13, 14, 10, 8, 9, 4, 0};
constexpr uint32_t kDecHighLut = dec_lut(kDecHigh);
constexpr uint32_t kDecLowLut = dec_lut(kDecLow);

__device__ __forceinline__ uint32_t encode_word(uint32_t x, uint64_t lut, uint32_t& bad) {
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    uint32_t c = (uint32_t)(lut >> (4 * ((x >> (4 * i)) & 15u))) & 15u;
    bad += c >> 3;
    out |= (c & 7u) << (3 * i);
  }
  return out;
}

__device__ __forceinline__ uint32_t decode_word(uint32_t c24, uint32_t lut) {
  uint32_t out = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) out |= ((lut >> (4 * ((c24 >> (3 * i)) & 7u))) & 15u) << (4 * i);
  return out;
}

// One thread per (group, p), p < 16.
__global__ __launch_bounds__(256) void meta3_pack_kernel(const uint32_t* __restrict__ in,
                                                         uint32_t* __restrict__ out, long long pairs,
                                                         uint32_t* __restrict__ errors) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs) return;
  const long long grp = idx >> 4;
  const int p = (int)(idx & 15);
  const uint32_t* a = in + grp * 64;
  uint32_t bad = 0;
  const uint64_t first = (uint64_t)encode_word(a[p], kEncHighLut, bad) |
                         ((uint64_t)encode_word(a[p + 32], kEncLowLut, bad) << 24);
  const uint64_t second = (uint64_t)encode_word(a[p + 16], kEncHighLut, bad) |
                          ((uint64_t)encode_word(a[p + 48], kEncLowLut, bad) << 24);
  uint32_t* o = out + grp * 48;
  o[p] = (uint32_t)first;
  o[16 + p] = (uint32_t)(first >> 32) | (uint32_t)(second << 16);
  o[32 + p] = (uint32_t)(second >> 16);
  if (bad) __hip_atomic_fetch_add(errors, bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void meta3_unpack_kernel(const uint32_t* __restrict__ in,
                                                           uint32_t* __restrict__ out, long long pairs) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= pairs) return;
  const long long grp = idx >> 4;
  const int p = (int)(idx & 15);
  const uint32_t* i = in + grp * 48;
  const uint64_t w0 = i[p], w1 = i[16 + p], w2 = i[32 + p];
  const uint64_t first = w0 | ((w1 & 0xFFFFu) << 32);
  const uint64_t second = (w1 >> 16) | (w2 << 16);
  uint32_t* o = out + grp * 64;
  o[p] = decode_word((uint32_t)first & 0xFFFFFFu, kDecHighLut);
  o[p + 32] = decode_word((uint32_t)(first >> 24) & 0xFFFFFFu, kDecLowLut);
  o[p + 16] = decode_word((uint32_t)second & 0xFFFFFFu, kDecHighLut);
  o[p + 48] = decode_word((uint32_t)(second >> 24) & 0xFFFFFFu, kDecLowLut);
}

// Spread 8 three-bit codes of a 24-bit field to nibbles, then apply
// dec(x) = 3 ^ (x | (7 + (x >> 1))) to all nibbles at once (x >> 1 <= 3, so
// 7 + (x >> 1) <= 10 never carries into the next nibble).
__device__ __forceinline__ uint32_t expand8(uint32_t x) {
  x = ((x & 0x00FFF000u) << 4) | (x & 0x00000FFFu);
  x = ((x & 0x0FC00FC0u) << 2) | (x & 0x003F003Fu);
  x = ((x & 0x38383838u) << 1) | (x & 0x07070707u);
  return (x | (((x >> 1) & 0x33333333u) + 0x77777777u)) ^ 0x33333333u;
}

// One thread per output word: 16 threads per 128-code group.
__global__ __launch_bounds__(256) void expand3_kernel(const uint32_t* __restrict__ in,
                                                      uint32_t* __restrict__ out, long long words) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= words) return;
  const long long grp = idx >> 4;
  const int t = (int)(idx & 15);
  const uint32_t* w = in + grp * 12;
  const int bit = 24 * t;
  const int k = bit >> 5;
  const int k1 = k + 1 < 12 ? k + 1 : 11;
  const uint32_t x = __builtin_amdgcn_alignbit(w[k1], w[k], bit & 31) & 0xFFFFFFu;
  out[idx] = expand8(x);
}

int launch_check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    sm24::set_error(std::string("marlin_hip: ") + what + " launch failed: " + hipGetErrorString(e));
    return MARLIN_HIP_ERR_LAUNCH;
  }
  return MARLIN_HIP_OK;
}

struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

}  // namespace codec3

extern "C" {

int marlin_hip_meta3_pack(const void* meta, void* out, long long n_int16, void* errors, int dev,
                          hipStream_t stream) {
  if (n_int16 < 0 || n_int16 % 128 != 0) return MARLIN_HIP_ERR_PROB_SHAPE;
  if (n_int16 == 0) return MARLIN_HIP_OK;
  codec3::DeviceGuard guard(dev);
  if (!guard.ok) return MARLIN_HIP_ERR_LAUNCH;
  const long long pairs = n_int16 / 128 * 16;
  const long long blocks = (pairs + 255) / 256;
  hipLaunchKernelGGL(codec3::meta3_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(meta), static_cast<uint32_t*>(out), pairs,
                     static_cast<uint32_t*>(errors));
  return codec3::launch_check("meta3_pack");
}

int marlin_hip_meta3_unpack(const void* packed, void* out, long long n_words, int dev, hipStream_t stream) {
  if (n_words < 0 || n_words % 48 != 0) return MARLIN_HIP_ERR_PROB_SHAPE;
  if (n_words == 0) return MARLIN_HIP_OK;
  codec3::DeviceGuard guard(dev);
  if (!guard.ok) return MARLIN_HIP_ERR_LAUNCH;
  const long long pairs = n_words / 48 * 16;
  const long long blocks = (pairs + 255) / 256;
  hipLaunchKernelGGL(codec3::meta3_unpack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(packed), static_cast<uint32_t*>(out), pairs);
  return codec3::launch_check("meta3_unpack");
}

int marlin_hip_expand3(const void* in, void* out, long long n_groups, int dev, hipStream_t stream) {
  if (n_groups < 0) return MARLIN_HIP_ERR_PROB_SHAPE;
  if (n_groups == 0) return MARLIN_HIP_OK;
  codec3::DeviceGuard guard(dev);
  if (!guard.ok) return MARLIN_HIP_ERR_LAUNCH;
  const long long words = n_groups * 16;
  const long long blocks = (words + 255) / 256;
  hipLaunchKernelGGL(codec3::expand3_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(in), static_cast<uint32_t*>(out), words);
  return codec3::launch_check("expand3");
}

}  // extern "C"
