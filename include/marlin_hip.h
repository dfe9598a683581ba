/* C ABI of the MI355X (gfx950) Sparse-Marlin 2:4 INT4 x FP16 GEMM library
 * (libmarlin_hip.so).  Plain pointers and sizes only; every tensor is caller-owned
 * device memory on device `dev`, and every call is asynchronous on `stream`.
 *
 * Naming follows the reference: prob_m = N (output features), prob_n = batch rows
 * M, prob_k = K; groupsize is in COMPRESSED-K units (64 for a dense group of 128,
 * -1 for one scale per output column).
 *
 * Return codes mirror the reference dispatch (marlin_cuda_kernel_nm.cu:748-749):
 *   0 ok, 1 problem shape incompatible with the tile, 2 no kernel for the tile or
 *   group size, and 3 (new) a HIP launch or scratch-allocation failure, described
 *   by marlin_hip_last_error().
 *
 * Buffer sizes are the caller's contract (they cannot be checked through plain
 * pointers): A M*K halves, B K*N/16 int32, meta K*N/16 int16, C M*N halves,
 * s (K/128 or 1)*N halves.
 *
 * The planner may split K (decode calls at wide N or long K, decode calls whose
 * column tiles leave a tail of at most half the compute units past whole rounds,
 * where only the tail tiles are split, large-M calls with few column tiles,
 * lane-native calls at 5-16 rows whose tiles cover too few compute units, and at
 * 2-4 rows when K >= 16384).  The split-K scratch (fp32 partials and
 * arrival counters) is uncached device memory that the library allocates per
 * (device, stream), grows on demand and never frees; the operand staging buffer of
 * the 3-bit variants at large M and of the lane-native layout above 16 rows is kept
 * the same way.  Calls on different streams therefore never share a buffer and may
 * overlap in time; calls on one stream are ordered.  `workspace` is not used (the
 * reference keeps its split-K locks there, common/mem.h:111-142).
 * The counters are zeroed at allocation and each is returned to zero by the last
 * workgroup that arrives on it, so no buffer needs to be zeroed by the caller.
 * During stream capture nothing can be allocated: a call whose stream has no large
 * enough scratch yet then runs without splitting K (same result within the GEMM
 * tolerance, a different summation order), and one that needs a larger staging
 * buffer fails with code 3; an eager call of the same shape on the capturing stream
 * before the capture sizes both.
 * A captured call keeps the scratch of the stream it was captured on, whatever
 * stream the graph is later replayed on.  So replays of graphs captured on one
 * stream (torch.cuda.graph() without stream= captures every graph on one default
 * capture stream) share that stream's scratch with each other and with eager calls
 * on it: they must not overlap in time.  Graphs captured on distinct streams may be
 * replayed concurrently.
 */
#ifndef MARLIN_HIP_H
#define MARLIN_HIP_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MARLIN_HIP_OK = 0,
  MARLIN_HIP_ERR_PROB_SHAPE = 1,
  MARLIN_HIP_ERR_KERN_SHAPE = 2,
  MARLIN_HIP_ERR_LAUNCH = 3
};

/* C[M,N] = A[M,K] * W[K,N], W in the Sparse-Marlin pack() layout.
 * Replaces marlin::marlin_cuda_2_4 (kernel_experiments/sparse_marlin/src/marlin/
 * marlin_cuda_kernel_nm.cu:751-755), same parameter order and meaning.
 * `workspace` and `max_par` are accepted for signature compatibility; this library
 * keeps its own scratch per (device, stream), so the caller's workspace is neither
 * read nor written.  thread_k/thread_m are validated exactly as the reference does
 * (the kernel and tile are then chosen by this library's planner). */
int marlin_hip_mul_2_4(const void* A, const void* B, const void* meta, void* C, void* s,
                       int prob_m, int prob_n, int prob_k, void* workspace, int groupsize,
                       int dev, hipStream_t stream, int thread_k, int thread_m, int sms,
                       int max_par);

/* marlin_hip_mul_2_4 without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory at call time (code under HIP
 * graph capture on a stream that has no scratch yet, serving loops and harnesses
 * that forbid hipMalloc).  It never splits K and never stages operands, so the only
 * scratch its kernels use is the library's static 256-byte zero block (a
 * `__device__` array that every device holds from module load to process end); no
 * problem size needs more, and shapes are refused only by marlin_hip_mul_2_4's
 * rules.  Same arguments and return codes as marlin_hip_mul_2_4 without workspace
 * and max_par.  The zero block is read-only, so overlapping calls on one device do
 * not race on it. */
int marlin_hip_mul_2_4_noalloc(const void* A, const void* B, const void* meta, void* C, const void* s,
                               int prob_m, int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream,
                               int thread_k, int thread_m, int sms);

/* The launch plan of a marlin_hip_mul_2_4 call (noalloc = 0) or of a
 * marlin_hip_mul_2_4_noalloc call (noalloc = 1), computed on the host without a GPU:
 * out[0] kernel of the first launch (0 decode at 1-8 padded rows, 3 decode at 16 or
 * 32 padded rows (the LDS-DMA kernel), 1 large-M, 2 general; -1 for an empty problem),
 * out[1] workgroups of the first launch, out[2] threads per workgroup, out[3] K
 * splits of the first launch (> 1: the call uses its stream's split-K scratch),
 * out[4] launches.  sms <= 0 plans for 256 compute units.  Returns the codes of
 * marlin_hip_mul_2_4's shape checks.  No counterpart in the reference (its host
 * dispatch, marlin_cuda_kernel_nm.cu:763-806, is not exposed); it lets a caller see
 * which calls split K and lets a benchmark launch an empty kernel on the same grid. */
int marlin_hip_plan(int prob_m, int prob_n, int prob_k, int groupsize, int thread_k, int thread_m, int sms,
                    int noalloc, int* out);

/* Dense INT4 x FP16 GEMM, C[M,N] = A[M,K] * W[K,N], W in the dense Marlin pack()
 * layout (B int32 [K/16][2N], s fp16 [K/128][N] or [1][N]).  Replaces
 * marlin::marlin_cuda (kernel_experiments/sparse_marlin/src/marlin/
 * marlin_cuda_kernel.cu:655-658), same parameter order and meaning: unlike
 * marlin_hip_mul_2_4, prob_m = M (batch rows), prob_n = N, and groupsize is in dense
 * K units (128 or -1).  Codes and tile rules as the reference (thread_k, thread_n) =
 * (128, 128) for M <= 16 or (64, 256); workspace and max_par are accepted for
 * signature compatibility and not used (split-K scratch as above). */
int marlin_hip_mul(const void* A, const void* B, void* C, void* s, int prob_m, int prob_n, int prob_k,
                   void* workspace, int groupsize, int dev, hipStream_t stream, int thread_k, int thread_n,
                   int sms, int max_par);

/* Same GEMM with 3-bit-compressed metadata (48 uint32 per 64-word group) as
 * produced by marlin_hip_meta3_pack.  Replaces the generated
 * decode_fetch::marlin_cuda_2_4 (kernel_experiments/sparse_marlin/metadata_decode/
 * setup.py:13-44, bound at setup.py:36-44). */
int marlin_hip_mul_2_4_meta3(const void* A, const void* B, const void* meta3, void* C, void* s,
                             int prob_m, int prob_n, int prob_k, void* workspace, int groupsize,
                             int dev, hipStream_t stream, int thread_k, int thread_m, int sms,
                             int max_par);

/* Same GEMM with 3-bit nonzero values: B3 is the code stream of the 4-bit layout
 * re-packed at 3 bits per code (code of nibble p of word w at bit 3*(8w+p), the
 * kernel_experiments/3bit_encoding bit layout), codes offset by 4.  The reference
 * has no implementation of 3-bit values (its 3-bit work encodes metadata); this
 * entry point serves the benchmark config that asks for them (3-bit values). */
int marlin_hip_mul_2_4_w3(const void* A, const void* B3, const void* meta, void* C, void* s,
                          int prob_m, int prob_n, int prob_k, void* workspace, int groupsize,
                          int dev, hipStream_t stream, int thread_k, int thread_m, int sms,
                          int max_par);

/* 4-bit 2:4 metadata (n_int16 int16, multiple of 128) -> 3-bit codes
 * (n_int16*3/8 uint32).  `errors` is a device uint32 counter that is incremented
 * once per nibble that is not a valid 2:4 pattern (the caller zeroes it).
 * Replaces pack_metadata (kernel_experiments/sparse_marlin/metadata_decode/
 * codec.cu:18-24, 30-35). */
int marlin_hip_meta3_pack(const void* meta, void* out, long long n_int16, void* errors,
                          int dev, hipStream_t stream);

/* Inverse of marlin_hip_meta3_pack: n_words uint32 (multiple of 48) -> n_words*8/3
 * int16.  Replaces unpack_metadata (codec.cu:25-29, 36-41). */
int marlin_hip_meta3_unpack(const void* packed, void* out, long long n_words, int dev,
                            hipStream_t stream);

/* Expand n_groups groups of 128 three-bit codes (48 bytes each, code i at bit 3i)
 * into 128 nibbles (64 bytes each) with dec(x) = {4,4,9,8,E,E,D,C}[x].
 * Replaces expansion<9> (kernel_experiments/3bit_encoding/experiment.cu:36-40). */
int marlin_hip_expand3(const void* in, void* out, long long n_groups, int dev,
                       hipStream_t stream);

/* Lane-native decode layout: an offline repack of the pack() layout (B, meta, s)
 * into per-lane operand order for the MI355X decode kernel, exactly invertible.
 * No counterpart in the reference; it is the "offline repack to a native format"
 * that the pack() layout's in-kernel remapping invites.  Sizes equal the reference
 * layout's: Bn K*N/16 uint32 (K*N/4 bytes), metan K*N/16 uint16, sn K/128*N halves
 * (groupsize 64) or N halves (groupsize -1).  Needs N % 64 == 0 and K % 256 == 0.
 * Layout: csed499ii_amd/csrc/sm24_native.h. */
int marlin_hip_native_pack(const void* B, const void* meta, const void* s, void* Bn, void* metan, void* sn,
                           int prob_m, int prob_k, int groupsize, int dev, hipStream_t stream);

/* Exact inverse of marlin_hip_native_pack. */
int marlin_hip_native_unpack(const void* Bn, const void* metan, const void* sn, void* B, void* meta, void* s,
                             int prob_m, int prob_k, int groupsize, int dev, hipStream_t stream);

/* C[M,N] = A[M,K] * W[K,N] with W in the lane-native layout (same arguments as
 * marlin_hip_mul_2_4 where they exist; automatic tiles only).  M <= 16 runs the
 * native decode kernel (split along K at 2-4 rows when K >= 16384, and at 5-16 rows
 * when the column tiles alone cover under 60 % of the compute units, through the
 * stream's split-K scratch); larger M unpacks the weight into the stream's staging
 * buffer and runs the reference-layout kernels.
 * No counterpart in the reference (see marlin_hip_native_pack). */
int marlin_hip_mul_2_4_native(const void* A, const void* Bn, const void* metan, void* C, const void* sn,
                              int prob_m, int prob_n, int prob_k, int groupsize, int dev, hipStream_t stream,
                              int sms);

/* Message describing the last MARLIN_HIP_ERR_* of the calling thread. */
const char* marlin_hip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MARLIN_HIP_H */
