/*
 * bsparse_timeline — the profiling harness of the instrumented build
 * (libbsparse_timeline.so): per-workgroup time stamps, and switches that
 * leave parts of a launch's work out.
 *
 * The reference decomposes its kernels' cost with profiling variants of its
 * operators, registered beside the plain ones (HostCodeRegistryProfiling,
 * block_spmm/inc/host_code.hpp:195-222: the _no_a_read, _no_b_read,
 * _no_compute and _no_write wrappers of :86-153; block_sddmm/inc/
 * host_code.hpp:71-153: _no_b_read, _no_c_read, _no_d_read, _no_compute,
 * _no_write) and timed per core with Tracy zones.  libbsparse_timeline.so is
 * built from the same sources as libbsparse.so with BSP_TIMELINE defined and
 * exports every function of bsparse.h with the same behaviour and results,
 * plus:
 *   - time stamps: wave 0 of every workgroup of the persistent SpMM, sweep
 *     SpMM and one-shot SDDMM kernels records the 100 MHz wall clock
 *     (s_memrealtime) at fixed points of its work: the persistent and sweep
 *     SpMM store each stamp to the caller's buffer at once (their wave 0
 *     waits for none of its own memory operations, and their LDS has no byte
 *     to spare); the one-shot SDDMM keeps its four stamps in registers and
 *     writes them when the workgroup ends (a scalar clock read per stamp, one
 *     store of 8 bytes per stamp);
 *   - skip switches (bsp_timeline_skip), off by default: with none set a
 *     launch does all of the work of the plain library's, bit for bit.
 *
 * Stamp slots per workgroup (BSP_TIMELINE_SLOTS, 0 = not reached):
 *   0   the workgroup starts (first instruction of wave 0)
 *   1   the first operands have landed (the first barrier is passed)
 *   2.. persistent SpMM: the end of each unit with entries, in stream order
 *       (slot 2 + u for unit u < 60 of the workgroup's list); sweep SpMM:
 *       entries 0 .. k+1 multiplied, every 8th entry (slot 2 + k/8 for
 *       k % 8 == 0, k/8 < 60); one-shot SDDMM: slot 2 = products done
 *   63  wave 0 has issued its last store (the end of its work)
 * Slots a workgroup does not reach keep what the buffer held (the
 * persistent SpMM writes only the slots it reaches; an idle one-shot SDDMM
 * workgroup writes none): clear the buffer before each launch.
 */
#ifndef BSPARSE_TIMELINE_H
#define BSPARSE_TIMELINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSP_TIMELINE_SLOTS 64

/* Skip switches (bit flags).  Sparse operand = A of SpMM, the mask values of
 * SDDMM (the reference's SDDMM "b"); dense = B of SpMM, X of SDDMM ("c");
 * dense2 = Y of SDDMM ("d").
 *   BSP_SKIP_*_READ: the operand's loads are not issued where the waves that
 *     issue them wait for nothing else (persistent SpMM with single stripes:
 *     its A and B loader waves; one-shot SDDMM: its one wait is for all
 *     loads); where a wave's waits count the loads of two operands together
 *     (the persistent SpMM with stripe pairs for A, the sweep SpMM, the
 *     256-column row-group SpMM) every load of the operand reads where the
 *     workgroup's first entry reads it instead -- an L2 hit after the
 *     first, on a line of its own per workgroup -- so that the operand
 *     moves no HBM or Infinity-Cache bytes while its requests and bytes
 *     into LDS stay; with both operands of such a kernel left out, no load
 *     is issued at all;
 *   BSP_SKIP_COMPUTE: no matrix-core products (the operands are still read
 *     from LDS; the accumulators stay zero);
 *   BSP_SKIP_WRITE: no stores of the output.
 * A skipped part leaves the output wrong: the switches are for timing. */
#define BSP_SKIP_SPARSE_READ 1
#define BSP_SKIP_DENSE_READ 2
#define BSP_SKIP_DENSE2_READ 4
#define BSP_SKIP_COMPUTE 8
#define BSP_SKIP_WRITE 16

/* Attaches a device buffer of `capacity` workgroups x BSP_TIMELINE_SLOTS
 * uint64 stamps on `device` (NULL detaches).  Launches from then on write the
 * stamps of workgroups below `capacity` (workgroup g at g*64 .. g*64+63).
 * Calls that overlap on the device share the buffer.  Returns a bsp_status. */
int bsp_timeline_attach(void* buffer, int64_t capacity, int device);

/* Frequency of the stamps' clock in kHz (hipDeviceAttributeWallClockRate). */
int bsp_timeline_clock_khz(int device, int* khz);

/* Leaves the work named by `flags` (BSP_SKIP_*, 0 = none) out of every SpMM
 * and SDDMM launch of this process from now on, on every device.  A launch
 * whose kernel has no switches (per-item SpMM kernels other than the
 * 256-column row-group one, the attention pair, the SDDMM ring kernel)
 * returns BSP_ERR_UNSUPPORTED while flags are set.  Not for concurrent use
 * with launches on other host threads.  Returns a bsp_status. */
int bsp_timeline_skip(int flags);

#ifdef __cplusplus
}
#endif

#endif /* BSPARSE_TIMELINE_H */
