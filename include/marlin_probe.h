/* C ABI of libmarlin_probe.so: measurement aids of bench.py's floor and mfma_floor
 * workloads and a lane-layout check of one MFMA instruction for the tests.  Not
 * part of the GEMM library and with no counterpart in the reference.  Return codes:
 * 0 ok, 1 bad argument, 3 HIP failure. */
#ifndef MARLIN_PROBE_H
#define MARLIN_PROBE_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read `bytes` (a multiple of 16) from device pointer `p` with 16-byte loads on
 * |blocks| workgroups of 256 threads, in grid-stride order (blocks > 0) or with a
 * contiguous range per wave (blocks < 0); `sink` is a device uint32 that is written only
 * in the (practically impossible) case that the XOR of all words is 0x9E3779B9. */
int marlin_probe_read(const void* p, long long bytes, void* sink, int blocks, int dev, hipStream_t stream);

/* An empty kernel on `blocks` workgroups of `threads` threads. */
int marlin_probe_empty(int blocks, int threads, int dev, hipStream_t stream);

/* The MFMA-only ceiling of the large-M 2:4 kernel: `blocks` workgroups of 512
 * threads (8 waves, 128 accumulator AGPRs each), every wave issuing `iters` x 16
 * v_smfmac_f32_32x32x32_f16 from random fp16 register operands.  `out` is a device
 * float array of blocks * 8 (a checksum per wave); `clock` is a device uint64 array
 * of 4: shader clock and 100 MHz real-time counter at the start and end of wave 0 of
 * workgroup 0. */
int marlin_probe_smfmac_stream(int blocks, int iters, void* out, void* clock, int dev, hipStream_t stream);

/* One v_mfma_f32_32x32x16_f16 on one wave with the operand and result lane layout
 * the dense large-M kernel assumes: A 32 x 16 and B 16 x 32 fp16, D 32 x 32 fp32,
 * all row-major device arrays.  D equals A @ B when the assumption holds. */
int marlin_probe_mfma_32x32x16(const void* A, const void* B, void* D, int dev, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MARLIN_PROBE_H */
