/*
 * bsparse_timeline — the per-workgroup timeline of the instrumented build
 * (libbsparse_timeline.so), the measurement half of the profiling harness.
 *
 * The reference decomposes its kernels' cost with profiling variants of its
 * operators, registered beside the plain ones (HostCodeRegistryProfiling,
 * block_spmm/inc/host_code.hpp:195-222; block_sddmm/PROFILING_PLAN.md) and
 * timed per core with Tracy zones.  Here the decomposition comes from time
 * stamps instead: libbsparse_timeline.so is built from the same sources as
 * libbsparse.so with BSP_TIMELINE defined, exports every function of
 * bsparse.h with the same behaviour and results, and in addition has wave 0
 * of every workgroup of the persistent SpMM, sweep SpMM and one-shot SDDMM
 * kernels record the 100 MHz wall clock (s_memrealtime) at fixed points of
 * its work into an LDS log, flushed to a caller's buffer when the workgroup
 * ends.  Nothing is skipped: the instrumented launch does all of the work of
 * the plain one (the log costs a scalar clock read per stamp and one 512-byte
 * store per workgroup).
 *
 * Stamp slots per workgroup (BSP_TIMELINE_SLOTS, 0 = not reached):
 *   0   the workgroup starts (first instruction of wave 0)
 *   1   the first operands have landed (the first barrier is passed)
 *   2.. persistent SpMM: the end of each unit with entries, in stream order
 *       (slot 2 + u for unit u < 60 of the workgroup's list); sweep SpMM:
 *       entries 0 .. k+1 multiplied, every 8th entry (slot 2 + k/8 for
 *       k % 8 == 0, k/8 < 60); one-shot SDDMM: slot 2 = products done
 *   63  wave 0 has issued its last store (the end of its work)
 * A workgroup that ends without work (an idle one-shot SDDMM workgroup)
 * leaves its slots untouched: clear the buffer before a launch.
 */
#ifndef BSPARSE_TIMELINE_H
#define BSPARSE_TIMELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSP_TIMELINE_SLOTS 64

/* Attaches a device buffer of `capacity` workgroups x BSP_TIMELINE_SLOTS
 * uint64 stamps on `device` (NULL detaches).  Launches from then on write the
 * stamps of workgroups below `capacity` (workgroup g at g*64 .. g*64+63) and
 * zero the slots they do not reach.  Calls that overlap on the device share
 * the buffer.  Returns a bsp_status. */
int bsp_timeline_attach(void* buffer, int64_t capacity, int device);

/* Frequency of the stamps' clock in kHz (hipDeviceAttributeWallClockRate). */
int bsp_timeline_clock_khz(int device, int* khz);

#ifdef __cplusplus
}
#endif

#endif /* BSPARSE_TIMELINE_H */
