/*
 * bsparse — block-sparse SpMM and SDDMM on MI355X (gfx950), C ABI.
 *
 * This is the boundary below the host-side operator entry points of
 * salmanra/Tenstorrent-WH-BlockSpMM (paths relative to that repository):
 *
 *   SpMM   C = A * B      A: BSR (bf16 R x C blocks), B: dense bf16, C: dense
 *          replaces HostCodeFunctionPtr, block_spmm/inc/host_code.hpp:165-177
 *          (bsr_spmm_multicore_load_balanced_new_DM / _snf / _snfin0_cdain1,
 *          :35-82)
 *   SDDMM  A = mask (.) (X * Y)  output only at the mask's nonzero blocks
 *          replaces SDDMMHostCodeFunctionPtr,
 *          block_sddmm/inc/host_code.hpp:104-115
 *          (bsr_sddmm_multicore_naive / _CDA, :43-69)
 *   SpGEMM C = A * B      A, B, C: BSR; a device path for the CPU routine
 *          bsr_matrix<T>::spgemm, sparse_common/bsr_matrix.hpp:741-810
 *
 * Data layout is the reference's untilized host layout: dense matrices are
 * row-major, BSR blocks are R x C row-major in CSR order with int32 indptr
 * (block-row pointers) and indices (block-column indices)
 * (sparse_common/bsr_matrix.hpp:202-213).  The reference's device path takes
 * 32x32-tilized buffers (block_spmm/src/test_block_spmm.cpp:77-78); that is a
 * Tenstorrent artefact and is not part of this ABI.
 *
 * Errors: every function returns a bsp_status; nothing throws across the ABI.
 * The reference aborts on malformed input (TT_ASSERT/TT_FATAL); here the same
 * conditions return BSP_ERR_BAD_STRUCTURE / BSP_ERR_INVALID_ARGUMENT and set a
 * thread-local message readable with bsp_last_error().
 *
 * Two levels:
 *   - plan + device pointers + stream (bsp_*_plan_create, bsp_spmm,
 *     bsp_sddmm): the structure is analysed once on the host and uploaded;
 *     each call is stream-ordered and asynchronous.  A plan is immutable after
 *     creation and may be used from several host threads, but calls that use
 *     the same plan must not overlap on the device (a plan owns one scratch
 *     area for split rows); order them on one stream.
 *   - host buffers, blocking (bsp_host_spmm, bsp_host_sddmm): the shape of the
 *     reference's operator entry points: allocate, upload, launch, download,
 *     synchronise, all in one call (the reference ends every call with
 *     Finish(cq), block_spmm/inc/host_code/bsr_spmm_multicore_snfin0_cdain1.cpp:840).
 *
 * Supported: R, C, M (=H), K (=W), N multiples of 32; bf16 inputs; fp32
 * accumulation; fp32 or bf16 output.  Duplicate and unsorted column indices
 * inside a block row are accepted and summed, as the reference's golden does.
 */
#ifndef BSPARSE_H
#define BSPARSE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BSP_ABI_VERSION 6

typedef enum bsp_status {
    BSP_OK = 0,
    BSP_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, misaligned pointer */
    BSP_ERR_BAD_STRUCTURE = 2,    /* malformed BSR (indptr/indices/shape) */
    BSP_ERR_UNSUPPORTED = 3,      /* valid input this build does not handle */
    BSP_ERR_DEVICE = 4,           /* HIP runtime error or no device */
    BSP_ERR_OUT_OF_MEMORY = 5
} bsp_status;

typedef enum bsp_dtype {
    BSP_DTYPE_F32 = 0,
    BSP_DTYPE_BF16 = 1
} bsp_dtype;

typedef enum bsp_layout {
    BSP_ROW_MAJOR = 0, /* element (r, c) at ptr[r * ld + c] */
    BSP_COL_MAJOR = 1  /* element (r, c) at ptr[c * ld + r] */
} bsp_layout;

/* BSR structure on the host (the index arrays of bsr_matrix<T>,
 * sparse_common/bsr_matrix.hpp:205-213: H, W, R, C, nblocks, indptr, indices). */
typedef struct bsp_bsr_desc {
    int64_t H;              /* rows (elements) */
    int64_t W;              /* columns (elements) */
    int64_t R;              /* block rows */
    int64_t C;              /* block columns */
    int64_t nblocks;        /* number of stored blocks */
    const int32_t* indptr;  /* H/R + 1 entries, indptr[0] == 0, non-decreasing,
                               indptr[H/R] == nblocks */
    const int32_t* indices; /* nblocks entries, each in [0, W/C) */
} bsp_bsr_desc;

typedef struct bsp_plan bsp_plan;

/* Schedule summary of a plan (for tests and the bench report). */
typedef struct bsp_plan_info {
    int32_t kind;        /* 1 = SpMM, 2 = SDDMM, 3 = fused attention pair,
                            4 = SpGEMM */
    int32_t tile_n;      /* SpMM: output columns per workgroup */
    int32_t n_tiles;     /* SpMM: N / tile_n */
    int32_t n_items;     /* work items (row pieces / mask-row chunks /
                            SpGEMM output 32x32 sub-blocks) */
    int32_t n_entries;   /* 32x32 sub-block products listed in the schedule */
    int32_t n_split_rows;/* SpMM: rows cut into several pieces */
    int32_t n_slots;     /* SpMM: partial-result slots used by split rows */
    int32_t grid;        /* workgroups per launch */
    int32_t max_item_entries;
    int32_t stages;      /* SpMM, SpGEMM: depth of the LDS ring (entries in
                            flight + 1); SDDMM: 1 = one-shot kernel, 0 = looped */
    int32_t group;       /* SpMM: 32-row stripes of one block row per workgroup
                            (1; or 2, 4, 8 for blocks of R >= 64) */
    int32_t waves;       /* SpMM: waves per workgroup (fixed at plan creation) */
    int64_t workspace_bytes; /* device scratch owned by the plan */
    int32_t persistent;  /* SpMM: 0 = one work item per workgroup; 1 or 2 =
                            persistent kernel with that many pipelines per
                            workgroup (each pipeline streams a list of stripe x
                            tile units; n_items counts the units, stages is the
                            B ring depth); 3 = sweep kernel (one workgroup per
                            compute unit holding up to 16 units at once, see
                            bsp_spmm_sweep_schedule) */
    int32_t a_stages;    /* SpMM persistent: depth of the A ring */
    int32_t step_entries;/* SpMM: entries per ring step, i.e. per workgroup
                            barrier (1, or 2 for the persistent kernel's
                            paired steps); 0 for other kinds */
    int32_t stripes_per_unit; /* SpMM: 32-row stripes per persistent unit (2:
                            stripe pairs that share one B slice per shared
                            block column; n_items then counts pair x tile
                            units); 1 otherwise; 0 for other kinds */
    int32_t units_rotated; /* SpMM persistent: 1 when each unit's entries start
                            at its column group's share of the block columns
                            (the default; BSP_SPMM_ROTATE=0 at plan creation
                            keeps them in CSR order), 0 otherwise */
} bsp_plan_info;

/* ---- library ------------------------------------------------------------- */
int bsp_abi_version(void);
const char* bsp_status_string(int status);
/* Message of the last failing call on this host thread ("" if none). */
const char* bsp_last_error(void);

/* Structural check of a BSR description; host only, no device needed.
 * The reference asserts the same shape rules in its constructors
 * (sparse_common/bsr_matrix.hpp:246-252, :609-616). */
int bsp_validate_bsr(const bsp_bsr_desc* desc);

/* ---- SpMM: C[M x N] = A[M x K] (BSR) * B[K x N] ------------------------------
 * Plan: analyses A's structure for a given N, b_layout and output dtype on
 * `device` (HIP device ordinal) and uploads the schedule.  Replaces the host
 * analysis each reference factory repeats per call (row folding, core
 * assignment and load balancing,
 * block_spmm/inc/host_code/bsr_spmm_multicore_load_balanced_new_DM.cpp:50-61,
 * :339-393). */
int bsp_spmm_plan_create(bsp_plan** plan, const bsp_bsr_desc* a, int64_t N,
                         int b_layout, int out_dtype, int device);

/* Launch on `stream` (a hipStream_t; NULL = the device's null stream).
 * a_vals: device, nblocks*R*C bf16 (16-byte aligned).
 * b:      device, bf16, K x N in b_layout with leading dimension ldb
 *         (16-byte aligned, ldb a multiple of 8 and below 2^26).
 * c:      device, M x N row-major with leading dimension ldc, fp32 or bf16 as
 *         planned; every element is written (block rows without nonzeros get
 *         zeros, which the reference obtains by zeroing the output first,
 *         block_spmm/src/test_block_spmm.cpp:67-69). */
int bsp_spmm(const bsp_plan* plan, const uint16_t* a_vals, const uint16_t* b, int64_t ldb,
             void* c, int64_t ldc, void* stream);

/* ---- SDDMM: out = mask (.) (X[M x K] * Y[K x N]) at mask's blocks ----------
 * The output has the mask's structure (indptr/indices copied, as
 * sparse_common/bsr_matrix.hpp:824-825); only its values are produced, in
 * block order, each block R x C row-major.  mask_vals multiply elementwise
 * (a true Hadamard product, :849-851). */
int bsp_sddmm_plan_create(bsp_plan** plan, const bsp_bsr_desc* mask, int64_t K,
                          int y_layout, int out_dtype, int device);

/* x: device bf16 M x K row-major, leading dimension ldx.
 * y: device bf16 K x N in y_layout (BSP_COL_MAJOR = Y^T stored row-major,
 *    e.g. the key matrix of Q*K^T), leading dimension ldy.
 * mask_vals: device, nblocks*R*C bf16.  out_vals: device, nblocks*R*C. */
int bsp_sddmm(const bsp_plan* plan, const uint16_t* mask_vals, const uint16_t* x, int64_t ldx,
              const uint16_t* y, int64_t ldy, void* out_vals, void* stream);

/* ---- fused block-sparse attention pair: O = S * V,
 *      S = bf16(mask (.) (Q * K^T)) at the mask's blocks -------------------
 * The reference has no fused operator; this is the pair of its two operators
 * on one structure: SDDMMHostCodeFunctionPtr (block_sddmm/inc/host_code.hpp
 * :104-115) with c = Q and d = K^T, its output cast to bf16 (the reference's
 * output type), then HostCodeFunctionPtr (block_spmm/inc/host_code.hpp
 * :165-177) with a = S and b = V.  S stays on the compute unit.  The result
 * equals bsp_sddmm (y_layout BSP_COL_MAJOR with y = K, bf16 output) followed
 * by bsp_spmm (a_vals = S, b = V) up to the fp32 summation order of O.
 * mask: queries x keys (H x W), R and C multiples of 32; head_dim 32, 64 or
 * 128. */
int bsp_attention_plan_create(bsp_plan** plan, const bsp_bsr_desc* mask, int64_t head_dim,
                              int out_dtype, int device);

/* mask_vals: device, nblocks*R*C bf16.  q: queries x head_dim, k and v:
 * keys x head_dim, all bf16 row-major (16-byte aligned, leading dimensions
 * multiples of 8, ldk and ldv below 2^26).  out: queries x head_dim row-major, fp32 or bf16 as
 * planned; every element is written. */
int bsp_attention(const bsp_plan* plan, const uint16_t* mask_vals, const uint16_t* q, int64_t ldq,
                  const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, void* out,
                  int64_t ldo, void* stream);

/* ---- SpGEMM: C = A * B, A and B BSR, C BSR -----------------------------------
 * The reference has this product only as a CPU routine (bsr_matrix<T>::spgemm,
 * sparse_common/bsr_matrix.hpp:741-810, which the tests' golden uses); there is
 * no device operator to replace.  Same contract: A is H x W in R x C blocks,
 * B is W x N in C x BC blocks (A.W == B.H and A.C == B.R, as :742-743
 * assert); C is H x N in R x BC blocks.  C(i, j) is stored iff some stored
 * A(i, k) meets some stored B(k, j) -- decided by the structures, not the
 * values -- with each block row's columns ascending (:786-801).  Duplicate
 * blocks contribute once per stored copy.  R, C and BC multiples of 32.
 *
 * Symbolic phase, host only (no device): C's structure.  Call with NULL
 * indptr/indices to get *nblocks, then with indptr[H/R + 1] and
 * indices[*nblocks]. */
int bsp_spgemm_symbolic(const bsp_bsr_desc* a, const bsp_bsr_desc* b, int64_t* nblocks,
                        int32_t* indptr, int32_t* indices);

/* Plan: the symbolic phase plus the per-sub-block product lists, uploaded to
 * `device`.  bsp_spgemm_structure copies the plan's C structure (same two-call
 * rule as bsp_spgemm_symbolic). */
int bsp_spgemm_plan_create(bsp_plan** plan, const bsp_bsr_desc* a, const bsp_bsr_desc* b,
                           int out_dtype, int device);
int bsp_spgemm_structure(const bsp_plan* plan, int64_t* nblocks, int32_t* indptr,
                         int32_t* indices);

/* Numeric phase on `stream`.  a_vals: device, A.nblocks*R*C bf16; b_vals:
 * device, B.nblocks*C*BC bf16; out_vals: device, nblocks*R*BC, fp32 or bf16
 * as planned, every value written.  All three 16-byte aligned. */
int bsp_spgemm(const bsp_plan* plan, const uint16_t* a_vals, const uint16_t* b_vals, void* out_vals,
               void* stream);

int bsp_plan_info_get(const bsp_plan* plan, bsp_plan_info* info);
int bsp_plan_destroy(bsp_plan* plan);

/* ---- host-only schedule queries (no device needed) --------------------------
 * Compute the schedule a plan would upload, for `num_cus` compute units, so it
 * can be inspected without a GPU.  Call once with NULL arrays to get the sizes
 * in *info, then again with arrays of those sizes.
 * SpMM:  items  n_items x 6 int32 {sub_row, e_begin, e_end, slot, base, npieces}
 *                (slot = -1 for a whole row; else the row is split into
 *                npieces pieces whose partials use slots base..base+npieces-1)
 *        ent_row n_entries int32  first row of B read by the entry
 *        ent_off n_entries int64  element offset of the 32x32 A sub-block
 *        wgmap  grid int32        item * n_tiles + tile, or -1 (idle slot)
 * SDDMM: items  n_items x 6 int32 {x_row0, e_begin, e_end, 0, 0, 0}
 *        ent_row n_entries int32  first column of Y read by the entry
 *        ent_off n_entries int64  element offset of the 32x32 output sub-block
 *        wgmap  grid int32        item index, or -1 */
int bsp_spmm_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, bsp_plan_info* info,
                      int32_t* items, int32_t* ent_row, int64_t* ent_off, int32_t* wgmap);
int bsp_sddmm_schedule(const bsp_bsr_desc* mask, int64_t K, int num_cus, bsp_plan_info* info,
                       int32_t* items, int32_t* ent_row, int64_t* ent_off, int32_t* wgmap);

/* SpMM sweep schedule (the sweep kernel a plan takes for large 32x32-block
 * structures: one workgroup per compute unit holding up to 16 units -- 32-row
 * stripe x 128 columns -- whose entries are merged by block column).  No
 * counterpart in the reference: its load balancing is
 * block_spmm/inc/host_code/bsr_spmm_multicore_load_balanced_new_DM.cpp
 * :339-393, this is the MI355X schedule that replaces it for such shapes.
 * col_groups: 0 = the plan's choice, else 1, 2, 4 or 8.  Sizes in *info:
 * grid workgroups, n_slots sweep records, n_entries entries, group = column
 * groups taken.
 *   wgs     grid x 4 int32   {first entry, entries, first sweep, sweeps}
 *   sweeps  n_slots x 33 int32 {entries, stripe of slots 0-15 (-1: unused),
 *                               first column of slots 0-15}
 *   bw      n_entries int64  first row of B | first column << 32 | slot << 56
 *                            | skip << 60 (a skip entry pads a sweep to an
 *                            even count and is not multiplied) | last << 61
 *                            (the last entry of its unit in stream order)
 *   aw      n_entries uint32 element offset of the 32x32 A sub-block / 32 */
int bsp_spmm_sweep_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, int col_groups,
                            bsp_plan_info* info, int32_t* wgs, int32_t* sweeps, int64_t* bw,
                            uint32_t* aw);

/* ---- host-buffer, blocking entry points ------------------------------------
 * bsp_host_spmm: the HostCodeFunctionPtr shape (block_spmm/inc/host_code.hpp
 * :165-177) with host arrays: a_vals (nblocks*R*C bf16), b (K x N row-major
 * bf16), out (M x N row-major, fp32 or bf16).  The reference's bcast_batch and
 * B arguments are always false / 1 at its call sites
 * (block_spmm/src/test_block_spmm.cpp:80) and are not carried. */
int bsp_host_spmm(const bsp_bsr_desc* a, const uint16_t* a_vals, const uint16_t* b, int64_t N,
                  void* out, int out_dtype, int device);

/* bsp_host_sddmm: the SDDMMHostCodeFunctionPtr shape
 * (block_sddmm/inc/host_code.hpp:104-115) with host arrays: x (M x K), y
 * (K x N), both row-major bf16; out_vals receives nblocks*R*C values. */
int bsp_host_sddmm(const bsp_bsr_desc* mask, const uint16_t* mask_vals, const uint16_t* x,
                   const uint16_t* y, int64_t K, void* out_vals, int out_dtype, int device);

/* bsp_host_spgemm: bsr_matrix<T>::spgemm (sparse_common/bsr_matrix.hpp
 * :741-810) with host arrays and the device doing the products: a_vals
 * (A.nblocks*R*C bf16), b_vals (B.nblocks*C*BC bf16).  The caller sizes the
 * output from bsp_spgemm_symbolic: out_indptr[H/R + 1], out_indices[nblocks],
 * out_vals[nblocks*R*BC] (fp32 or bf16). */
int bsp_host_spgemm(const bsp_bsr_desc* a, const uint16_t* a_vals, const bsp_bsr_desc* b,
                    const uint16_t* b_vals, int32_t* out_indptr, int32_t* out_indices,
                    void* out_vals, int out_dtype, int device);

/* ---- SpMM without device allocation ------------------------------------------
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (serving loops that must not touch the allocator,
 * harnesses that forbid hipMalloc).  C = A * B on the persistent SpMM kernel
 * (the 32-row stripe kernel a plan takes for 32x32 blocks), without a plan:
 * the schedule is built on the host and staged in a static device array of
 * BSP_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on
 * until the process ends.  It calls no hipMalloc or hipFree.
 *   Result: bit-identical to bsp_spmm with a plan that takes the persistent
 *   kernel with single stripes (a plan's stripe pairs give the same bits).  A
 *   plan that takes another kernel -- the row-group kernels some R >= 64
 *   structures take, or a schedule changed by environment overrides at plan
 *   creation -- may sum in another order; both stay within the oracle's
 *   tolerance.
 *   Synchronisation: the call copies the schedule on `stream` and then WAITS
 *   ON THE HOST for `stream` (all of its earlier work and that copy) before
 *   launching asynchronously.  It is therefore not asynchronous in the host's
 *   sense, and it cannot be recorded into a HIP graph: on a stream under
 *   capture it returns BSP_ERR_UNSUPPORTED without touching the stream.
 *   Sharing: calls on one GPU share the array, which keeps the last call's
 *   contents; two calls that overlap on one GPU race (order them on one
 *   stream, and let a launch finish before the next call from another
 *   stream).
 *   Errors: the structure is validated first (as bsp_validate_bsr);
 *   a schedule above the limit, N not a multiple of 128, or R, C not
 *   multiples of 32 return BSP_ERR_UNSUPPORTED; no device, or a failed
 *   compute-unit count query, BSP_ERR_DEVICE.
 * a: host BSR structure; a_vals, b, c: device pointers as for bsp_spmm. */
#define BSP_NOALLOC_SCRATCH_BYTES (16 << 20)
int bsp_spmm_noalloc(const bsp_bsr_desc* a, const uint16_t* a_vals, const uint16_t* b, int64_t N,
                     int64_t ldb, void* c, int64_t ldc, int out_dtype, int device, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BSPARSE_H */
