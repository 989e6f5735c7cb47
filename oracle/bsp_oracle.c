/*
 * ORACLE — test infrastructure, not product code.
 *
 * A plain-C restatement of the CPU golden that salmanra/Tenstorrent-WH-BlockSpMM
 * checks its block-sparse SpMM / SDDMM device paths against, and its BSR x BSR
 * SpGEMM golden (a CPU routine with no device path in the reference).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this file's
 * library, and only as the checker (or, in bench.py, as the timed CPU baseline).
 * The product path (libbsparse.so) never links, loads or calls it.
 *
 * Every function names the reference lines it follows.  Paths are relative to
 * the reference checkout.  The reference's golden lives in member templates of
 * bsr_matrix<T> (header-only C++) that include tt-metal headers; those are not
 * present here, so the reference cannot be compiled and this restatement is the
 * oracle.  How each function is pinned (closed forms, brute force, planted
 * mistakes) is listed next to it; tests/test_oracle.py holds the checks.
 *
 * Data conventions (the reference's own, untilized):
 *   - BSR: indptr[nbrows+1], indices[nblocks] (block-column index), values
 *     nblocks*R*C, each block R x C row-major, blocks in CSR order
 *     (sparse_common/bsr_matrix.hpp:202-213).
 *   - dense: row-major H x W, data[i*W + j] (sparse_common/bsr_matrix.hpp:39-46).
 *   - bf16 values are passed as raw uint16_t bit patterns.
 *
 * Mutations: the `mutation` argument plants one deliberate mistake (0 = none).
 * The tests use them to show that each pinning check fails on a plausible bug.
 * Product code never passes a non-zero mutation.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_TILE 32 /* TILE_SIZE, sparse_common/bsr_matrix.hpp:22 */

/* ---- bf16 <-> fp32 -------------------------------------------------------
 * Round-to-nearest-even from fp32, NaN kept quiet.  The reference uses
 * tt-metal's bfloat16(float) constructor (sparse_common/bsr_matrix.hpp:120-126,
 * :682-688), whose source is not in the reference tree; RNE is the IEEE default
 * and what torch.bfloat16 uses.  Pinned by tests against torch's conversion on
 * every special class (ties, subnormals, inf, NaN). */
uint16_t orc_bf16_from_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_bf16_from_f32_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(in[i]);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

static int orc_threads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

int orc_have_openmp(void) {
#ifdef _OPENMP
    return 1;
#else
    return 0;
#endif
}

/* ---- SpMM golden ----------------------------------------------------------
 * Follows bsr_matrix<T>::omp_spmm_bf16, block_spmm/inc/bsr_matrix.hpp:954-1000
 * (same arithmetic as spmm_bfloat16 :737-781 and sparse_common copy :909-955):
 *   for block row i, for 32-row tile r, for 32-col tile p of B:
 *     fp32 output_tile[32x32] = 0
 *     for each nonzero idx of row i in CSR order (j = indices[idx]):
 *       for each 32-wide tile c of the block's C columns:
 *         for rr, pp: sum = sum_{cc in tile} float(a)*float(b) (fp32, in order);
 *                     output_tile[rr][pp] += sum
 *     store output_tile
 * The reference stores T(output_tile) (bf16); this function stores the fp32
 * tile (the "fp32 golden" the tolerance is stated against) and the bf16 result
 * is orc_bf16_from_f32 of it.  Block rows with no nonzeros are written as
 * zeros: the reference leaves them untouched in a caller-zeroed output
 * (block_spmm/src/test_block_spmm.cpp:67-69), which is the same result.
 * Duplicate and unsorted column indices are summed in CSR order, as the
 * reference does.
 * `threads` > 1 applies the reference's intended `#pragma omp parallel for` over
 * block rows (:959); 1 reproduces how the reference actually runs (serial).
 * Pinned by: test_1_block_id / _uniform / _arange closed forms
 * (block_spmm/inc/test_suite.hpp:1862-1925), brute force against to_dense +
 * a float64 GEMM, empty rows, duplicate columns, linearity.
 * Mutations: 1 transposed B access, 2 drop the last nonzero of each row,
 *            3 subtract instead of add, 4 column index off by one block. */
int orc_spmm_bf16(const int32_t* indptr, const int32_t* indices, const uint16_t* a_vals,
                  int64_t nbrows, int64_t R, int64_t C, const uint16_t* b, int64_t K,
                  int64_t N, float* out, int threads, int mutation) {
    if (!indptr || !out || R <= 0 || C <= 0 || N <= 0 || nbrows < 0) return 1;
    const int64_t nbcols = K / C;
    int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) if (nt > 1)
    for (int64_t i = 0; i < nbrows; ++i) {
        float tile[ORC_TILE * ORC_TILE];
        int64_t lo = indptr[i], hi = indptr[i + 1];
        if (mutation == 2 && hi > lo) hi -= 1;
        for (int64_t r = 0; r < R; r += ORC_TILE) {
            for (int64_t p = 0; p < N; p += ORC_TILE) {
                memset(tile, 0, sizeof(tile));
                for (int64_t idx = lo; idx < hi; ++idx) {
                    int64_t j = indices[idx];
                    if (mutation == 4) j = (j + 1) % (nbcols > 0 ? nbcols : 1);
                    const uint16_t* ablk = a_vals + idx * R * C;
                    const uint16_t* bpan = b + j * C * N;
                    for (int64_t c = 0; c < C; c += ORC_TILE) {
                        int64_t rr_end = r + ORC_TILE < R ? r + ORC_TILE : R;
                        int64_t pp_end = p + ORC_TILE < N ? p + ORC_TILE : N;
                        int64_t cc_end = c + ORC_TILE < C ? c + ORC_TILE : C;
                        for (int64_t rr = r; rr < rr_end; ++rr) {
                            for (int64_t pp = p; pp < pp_end; ++pp) {
                                float sum = 0.0f;
                                for (int64_t cc = c; cc < cc_end; ++cc) {
                                    float av = orc_bf16_to_f32(ablk[rr * C + cc]);
                                    float bv;
                                    if (mutation == 1) {
                                        /* transposed operand: element (k, n) of the
                                           K x N array read at n*K + k (in bounds). */
                                        bv = orc_bf16_to_f32(b[pp * K + j * C + cc]);
                                    } else {
                                        bv = orc_bf16_to_f32(bpan[cc * N + pp]);
                                    }
                                    sum += av * bv;
                                }
                                if (mutation == 3)
                                    tile[(rr - r) * ORC_TILE + pp - p] -= sum;
                                else
                                    tile[(rr - r) * ORC_TILE + pp - p] += sum;
                            }
                        }
                    }
                }
                int64_t rr_end = r + ORC_TILE < R ? r + ORC_TILE : R;
                int64_t pp_end = p + ORC_TILE < N ? p + ORC_TILE : N;
                for (int64_t rr = r; rr < rr_end; ++rr)
                    for (int64_t pp = p; pp < pp_end; ++pp)
                        out[(i * R + rr) * N + pp] = tile[(rr - r) * ORC_TILE + pp - p];
            }
        }
    }
    return 0;
}

/* ---- SDDMM golden ---------------------------------------------------------
 * Follows bsr_matrix<T>::sddmm, sparse_common/bsr_matrix.hpp:816-857 (SpMM-side
 * copy block_spmm/inc/bsr_matrix.hpp:861-902):
 *   out(i,j)[r][c] = float(mask(i,j)[r][c]) * sum_{k<K} float(X[iR+r][k]) *
 *                    float(Y[k][jC+c]), the dot product summed in k order in
 *   fp32; the output copies the mask's indptr/indices (:824-825) and stores
 *   T(mask_val * dot) in block order.
 * Here the fp32 value mask_val*dot is stored; bf16 = orc_bf16_from_f32 of it.
 * The output structure is the mask's structure, so only values are produced.
 * `y_colmajor` != 0 reads Y from a row-major N x K array (i.e. Y^T stored
 * row-major, as K in Q*K^T), element (k, n) at y[n*K + k]; this is a layout
 * option of this build, the arithmetic is unchanged.
 * Pinned by: the UNIFORM/ARANGE closed forms of block_sddmm/inc/test_suite.hpp
 * :27-110 (out = sum_k bf16(row*K + k)), identity mask (:57-62), full mask ==
 * dense GEMM blocks (:45-52), brute force against float64.
 * Mutations: 1 ignore mask values, 2 transposed Y access, 3 drop the last k,
 *            4 read the mask block of the next block. */
int orc_sddmm(const int32_t* indptr, const int32_t* indices, const uint16_t* mask_vals,
              int64_t nbrows, int64_t R, int64_t C, const uint16_t* x, int64_t K,
              const uint16_t* y, int64_t N, int y_colmajor, float* out_vals, int threads,
              int mutation) {
    if (!indptr || R <= 0 || C <= 0 || K < 0 || nbrows < 0) return 1;
    int64_t nblocks = indptr[nbrows];
    int nt = orc_threads(threads);
    int64_t kend = (mutation == 3 && K > 0) ? K - 1 : K;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1) if (nt > 1)
    for (int64_t i = 0; i < nbrows; ++i) {
        for (int64_t blk = indptr[i]; blk < indptr[i + 1]; ++blk) {
            int64_t j = indices[blk];
            int64_t mblk = blk;
            if (mutation == 4) mblk = (blk + 1) % (nblocks > 0 ? nblocks : 1);
            const uint16_t* mb = mask_vals + mblk * R * C;
            for (int64_t r = 0; r < R; ++r) {
                for (int64_t c = 0; c < C; ++c) {
                    float dot = 0.0f;
                    int64_t row = i * R + r, col = j * C + c;
                    for (int64_t k = 0; k < kend; ++k) {
                        float xv = orc_bf16_to_f32(x[row * K + k]);
                        float yv;
                        int colmajor = y_colmajor;
                        if (mutation == 2) colmajor = !colmajor;
                        if (colmajor) {
                            int64_t idx = col * K + k;
                            if (mutation == 2) idx %= (K * N > 0 ? K * N : 1);
                            yv = orc_bf16_to_f32(y[idx]);
                        } else {
                            int64_t idx = k * N + col;
                            if (mutation == 2) idx %= (K * N > 0 ? K * N : 1);
                            yv = orc_bf16_to_f32(y[idx]);
                        }
                        dot += xv * yv;
                    }
                    float mval = mutation == 1 ? 1.0f : orc_bf16_to_f32(mb[r * C + c]);
                    out_vals[blk * R * C + r * C + c] = mval * dot;
                }
            }
        }
    }
    return 0;
}

/* ---- SpGEMM: BSR x BSR -> BSR ------------------------------------------------
 * Follows bsr_matrix<T>::spgemm, sparse_common/bsr_matrix.hpp:741-810.  A is
 * nbrows x (W/C) blocks of R x C, B has blocks of C x BC (A's C is B's R) in
 * b_nbc block columns.  Output block (i, j) is present iff some A(i, k) and
 * B(k, j) are stored blocks (decided by the structure, not the values); the
 * output lists each block row's columns in ascending order (the reference
 * builds it by scanning j).  For every pair, in A's CSR order then B's CSR
 * order, each element gets the C-term fp32 dot product (c ascending) added to
 * its fp32 accumulator; the accumulator is returned (the reference stores
 * T(acc)).  Duplicate columns in A or B contribute once per stored block.
 * Two calls: with out_indices == NULL it fills out_indptr and *nblocks_out;
 * then with arrays of that size it fills indices and values (nblocks*R*BC).
 * Pinned by: the block-pattern boolean product, the dense float64 product of
 * to_dense(A) and to_dense(B), identity B, brute force on tiny inputs.
 * Mutations: 1 transposed B block access, 2 skip the last A block of each row,
 *            3 output column + 1, 4 skip the c = 0 term. */
int orc_spgemm(const int32_t* a_indptr, const int32_t* a_indices, const uint16_t* a_vals,
               int64_t nbrows, int64_t R, int64_t C, const int32_t* b_indptr,
               const int32_t* b_indices, const uint16_t* b_vals, int64_t BC, int64_t b_nbc,
               int32_t* out_indptr, int32_t* out_indices, float* out_vals, int64_t* nblocks_out,
               int mutation) {
    if (!a_indptr || !b_indptr || !out_indptr || !nblocks_out || R <= 0 || C <= 0 || BC <= 0 ||
        b_nbc < 0 || nbrows < 0)
        return 1;
    const int64_t blk = R * BC;
    unsigned char* present = (unsigned char*)calloc((size_t)(b_nbc > 0 ? b_nbc : 1), 1);
    float* acc = NULL;
    if (out_indices) {
        acc = (float*)calloc((size_t)(b_nbc > 0 ? b_nbc : 1) * (size_t)blk, sizeof(float));
        if (!acc) {
            free(present);
            return 2;
        }
    }
    if (!present) {
        free(acc);
        return 2;
    }
    int64_t nout = 0;
    out_indptr[0] = 0;
    for (int64_t i = 0; i < nbrows; ++i) {
        int64_t a_end = a_indptr[i + 1];
        if (mutation == 2 && a_end > a_indptr[i]) a_end -= 1;
        for (int64_t ai = a_indptr[i]; ai < a_end; ++ai) {
            const int64_t k = a_indices[ai];
            const uint16_t* ab = a_vals ? a_vals + ai * R * C : NULL;
            for (int64_t bi = b_indptr[k]; bi < b_indptr[k + 1]; ++bi) {
                const int64_t j = b_indices[bi];
                present[j] = 1;
                if (!acc) continue;
                const uint16_t* bb = b_vals + bi * C * BC;
                float* o = acc + j * blk;
                for (int64_t r = 0; r < R; ++r)
                    for (int64_t p = 0; p < BC; ++p) {
                        float sum = 0.0f;
                        for (int64_t c = (mutation == 4 ? 1 : 0); c < C; ++c) {
                            const int64_t bidx = mutation == 1 ? (p * C + c) % (C * BC) : c * BC + p;
                            sum += orc_bf16_to_f32(ab[r * C + c]) * orc_bf16_to_f32(bb[bidx]);
                        }
                        o[r * BC + p] += sum;
                    }
            }
        }
        for (int64_t j = 0; j < b_nbc; ++j) {
            if (!present[j]) continue;
            if (out_indices) {
                out_indices[nout] = (int32_t)(mutation == 3 ? (j + 1) % b_nbc : j);
                memcpy(out_vals + nout * blk, acc + j * blk, (size_t)blk * sizeof(float));
                memset(acc + j * blk, 0, (size_t)blk * sizeof(float));
            }
            present[j] = 0;
            ++nout;
        }
        out_indptr[i + 1] = (int32_t)nout;
    }
    *nblocks_out = nout;
    free(present);
    free(acc);
    return 0;
}

/* ---- to_dense -------------------------------------------------------------
 * Follows bsr_matrix<T>::to_dense, sparse_common/bsr_matrix.hpp:1056-1070:
 * zero-filled H x W, each block assigned (not added) at its position, in CSR
 * order, so with duplicate columns the later block wins. */
int orc_bsr_to_dense(const int32_t* indptr, const int32_t* indices, const uint16_t* vals,
                     int64_t nbrows, int64_t R, int64_t C, int64_t W, uint16_t* out) {
    if (!indptr || !out) return 1;
    memset(out, 0, (size_t)(nbrows * R * W) * sizeof(uint16_t));
    for (int64_t i = 0; i < nbrows; ++i)
        for (int64_t idx = indptr[i]; idx < indptr[i + 1]; ++idx) {
            int64_t j = indices[idx];
            for (int64_t r = 0; r < R; ++r)
                for (int64_t c = 0; c < C; ++c)
                    out[(i * R + r) * W + j * C + c] = vals[idx * R * C + r * C + c];
        }
    return 0;
}

/* ---- dense GEMM with fp32 accumulation ------------------------------------
 * Follows dense_matrix<T>::gemm_bfloat16, sparse_common/bsr_matrix.hpp:158-171:
 * out[i][j] = sum_k float(a[i][k]) * float(b[k][j]) in k order; the fp32 sum is
 * stored (the reference stores T(sum)). */
int orc_gemm_bf16(const uint16_t* a, const uint16_t* b, int64_t H, int64_t Kd, int64_t W,
                  float* out) {
    if (!a || !b || !out) return 1;
    for (int64_t i = 0; i < H; ++i)
        for (int64_t j = 0; j < W; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < Kd; ++k)
                sum += orc_bf16_to_f32(a[i * Kd + k]) * orc_bf16_to_f32(b[k * W + j]);
            out[i * W + j] = sum;
        }
    return 0;
}

/* ---- Pearson correlation ---------------------------------------------------
 * Follows check_bfloat16_vector_pcc, sparse_common/bmm_op.hpp:79-113: float
 * means, then float covariance and variances (each divided by n), then
 * cov / (sqrt(var_x) * sqrt(var_y)).  The reference takes bf16 vectors; this
 * takes fp32 (pass bf16 values widened exactly to compare bf16 outputs). */
float orc_pcc(const float* xa, const float* ya, int64_t n) {
    float xm = 0.0f, ym = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        xm += xa[i];
        ym += ya[i];
    }
    xm /= (float)n;
    ym /= (float)n;
    float cov = 0.0f, xs = 0.0f, ys = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float xd = xa[i] - xm, yd = ya[i] - ym;
        cov += xd * yd;
        xs += xd * xd;
        ys += yd * yd;
    }
    cov /= (float)n;
    xs /= (float)n;
    ys /= (float)n;
    return cov / (sqrtf(xs) * sqrtf(ys));
}
