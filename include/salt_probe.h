/*
 * libsalt_probe.so -- measurement probes used by bench.py for the roofline (no
 * counterpart in the reference, and not part of the forward path).
 */
#ifndef SALT_PROBE_H
#define SALT_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SALT_PROBE_READ_B32 0
#define SALT_PROBE_READ_B64 1
#define SALT_PROBE_READ_B128 2
#define SALT_PROBE_WRITE_B32 3

/* LDS bandwidth of the current device: `blocks` work-groups of 256 threads, each with a
 * 32 KB LDS buffer, make `iters` x 16 conflict-free accesses per thread of the given kind.
 * One warm-up launch, then one timed launch (HIP events on the null stream); *seconds is
 * the timed launch's duration and *bytes the bytes it moved through LDS.
 * Returns 0, -1 on invalid arguments, -2 on a HIP error. */
int32_t salt_probe_lds(int32_t kind, int32_t blocks, int32_t iters, double* seconds,
                       double* bytes);

#ifdef __cplusplus
}
#endif
#endif
