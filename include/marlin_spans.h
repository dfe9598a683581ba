/* Measurement hook of libmarlin_hip.so: per-wave phase timestamps of the decode
 * kernel (bench.py --workload spans).  No counterpart in the reference.
 *
 * The kernels record stamps only in the measurement build of the library
 * (libmarlin_hip_spans.so, compiled with SM24_SPANS=1 by csed499ii_amd/build.py);
 * the product build exports the same symbol and records nothing. */
#ifndef MARLIN_SPANS_H
#define MARLIN_SPANS_H

#ifdef __cplusplus
extern "C" {
#endif

/* Device buffer for the stamps of the decode launches made from now on (null: none).
 * Every wave w of workgroup b of a launch writes 12 uint64 words at
 * buf[(b * waves + w) * 12]: the real-time counter (100 MHz) at entry, once the
 * kernel arguments have arrived, once its load addresses are set up, once its
 * first stages' loads are issued, after its last stage and at exit (words 0-5);
 * the shader clock at entry and exit (6, 7); its hardware compute-unit id (8); its
 * workgroup index (9); words 10-11 are zero.  The buffer must hold every
 * wave of the launch (marlin_hip_plan gives workgroups and threads per workgroup).
 * Returns 0 in the measurement build, 2 in the product build (no stamps). */
int marlin_hip_set_spans(void* buf);

#ifdef __cplusplus
}
#endif

#endif /* MARLIN_SPANS_H */
