// Kernel argument blocks and launchers shared by the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "bsp_schedule.hpp"

namespace bsp {

// Work the instrumented build (libbsparse_timeline.so) can leave out of a
// launch, for cost decompositions (the values of BSP_SKIP_* in
// bsparse_timeline.h).  Sparse = A of SpMM, the mask values of SDDMM; dense
// = B of SpMM, X of SDDMM; dense2 = Y of SDDMM.
constexpr int kSkipSparseRead = 1;
constexpr int kSkipDenseRead = 2;
constexpr int kSkipDense2Read = 4;
constexpr int kSkipCompute = 8;
constexpr int kSkipWrite = 16;

struct SpmmArgs {
    const uint16_t* a;        // A block values (bf16), nblocks*R*C
    const uint16_t* b;        // B (bf16), row-major K x N, leading dim ldb
    void* c;                  // C (fp32 or bf16), row-major M x N, leading dim ldc
    const SpmmWg* wgs;        // one record per workgroup (row == -1: idle)
    const int64_t* ents;      // per entry: first row of B (low 32 bits) | A offset / 32 (high)
    const SpmmSplit* splits;  // split rows (row, first slot, pieces), for the reduce kernel
    float* ws;                // partial results of split-row pieces
    int64_t ldb;
    int64_t ldc;
    int32_t lda;              // row stride inside an A block (= C)
    int32_t n_tiles;
    int32_t N;                // columns of B and C (the last tile may be partial)
    int32_t skips;            // work the instrumented build leaves out (kSkip*; 0 in libbsparse.so)
};

// Persistent SpMM (spmm_stream_kernel): each workgroup streams the entries of
// its units (stripe or stripe pair x tile) through one ring.
struct SpmmStreamArgs {
    const uint16_t* a;             // A block values (bf16)
    const uint16_t* b;             // B (bf16), row-major K x N, leading dim ldb
    void* c;                       // C (fp32 or bf16), row-major M x N, leading dim ldc
    const SpmmStreamHead* heads;   // one per workgroup (per pipeline)
    const SpmmStreamUnit* units;   // unit records (padded)
    const int64_t* bw;             // per stream entry: first row of B | first column << 32 (padded)
    const uint32_t* aw;            // per stream entry: A sub-block offset / 32 (padded; one stripe)
    const uint64_t* apw;           // stripe pairs: per stream entry, both stripes' A offsets / 32 (padded)
    int64_t ldb;
    int64_t ldc;
    int32_t lda;                   // row stride inside an A block (= C)
    int32_t N;
    int32_t skips;                 // work the instrumented build leaves out (kSkip*; 0 in libbsparse.so)
    int32_t pad;
};

// Sweep SpMM (spmm_sweep_kernel): one workgroup per compute unit holds a
// sweep's units (up to 16) and streams their entries merged by first row of B.
struct SpmmSweepArgs {
    const uint16_t* a;             // A block values (bf16)
    const uint16_t* b;             // B (bf16), row-major K x N, leading dim ldb
    void* c;                       // C (fp32 or bf16), row-major M x N, leading dim ldc
    const SpmmSweepHead* heads;    // one per workgroup
    const SpmmSweepRec* sweeps;    // sweep records (padded)
    const int64_t* bw;             // per entry: first row of B | first column << 32 | slot << 56 (padded)
    const uint32_t* aw;            // per entry: A sub-block offset / 32 (padded)
    int64_t ldb;
    int64_t ldc;
    int32_t lda;                   // row stride inside an A block (= C)
    int32_t N;
    int32_t skips;                 // work the instrumented build leaves out (kSkip*; 0 in libbsparse.so)
    int32_t pad;
};

// The sweep kernel: rings of 16 stages (A 2 KB and B 8 KB each: all 160 KB
// of a compute unit's LDS), eight MFMA waves, an A loader and two B loaders.
constexpr int kSweepStages = 16;
constexpr int kSweepWaves = 11;

hipError_t launch_spmm_sweep(const SpmmSweepArgs& a, bool out_bf16, int grid, hipStream_t stream);

// Whether an SpMM plan takes the sweep kernel: 32x32-multiple blocks, N a
// multiple of 128, at least 8 units (stripe x 128 columns) per compute unit
// and a B of at least 8 MB (below that the whole of B stays in the L2s and
// the persistent kernel's two workgroups per compute unit do better).
// BSP_SPMM_SWEEP=0 turns it off, 2 takes it whenever the shape allows.
bool choose_spmm_sweep(const bsp_bsr_desc* a, int64_t N, int cus);

// Compiled persistent SpMM variants: tile width, B ring depth, A ring depth,
// B loader waves, pipelines per workgroup, entries per ring step, stripes per
// unit.  A pipeline has 4 MFMA waves (each 32*tile/128 columns), the B loader
// waves and one A loader wave, and LDS of 64*tile*SB + 2 KB*SA*stripes (+ 8
// bytes*SA of A words with stripe pairs); two pipelines add a 16 KB
// (32 KB at tile 256) exchange buffer.  With two entries per step (one
// pipeline, even ring depths of at most 16) the workgroup passes one barrier
// per pair of entries; stripe pairs need two entries per step.
#define BSP_SPMM_STREAM_VARIANTS(X) \
    X(128, 8, 8, 2, 1, 2, 1)        \
    X(128, 14, 16, 4, 1, 2, 1)      \
    X(128, 8, 8, 2, 1, 2, 2)        \
    X(128, 6, 12, 2, 1, 2, 1)       \
    X(128, 6, 12, 2, 1, 1, 1)       \
    X(128, 6, 12, 4, 1, 1, 1)       \
    X(128, 4, 16, 4, 1, 1, 1)       \
    X(128, 8, 16, 8, 1, 1, 1)       \
    X(256, 4, 16, 4, 1, 1, 1)       \
    X(256, 5, 16, 8, 1, 1, 1)       \
    X(256, 6, 8, 8, 1, 1, 1)        \
    X(128, 6, 12, 2, 2, 1, 1)       \
    X(128, 5, 12, 2, 2, 1, 1)

struct SpmmStreamVariant {
    int tile_n;
    int sb;
    int sa;
    int nbw;
    int pipes = 1;
    int eps = 1;  // entries per ring step
    int sr = 1;   // stripes per unit (2: stripe pairs)
};

// The default (uniform rows), the skewed-row and the stripe-pair choices of
// choose_spmm_stream.
constexpr SpmmStreamVariant kSpmmStreamDefault{128, 8, 8, 2, 1, 2, 1};
constexpr SpmmStreamVariant kSpmmStreamSkewed{128, 14, 16, 4, 1, 2, 1};
constexpr SpmmStreamVariant kSpmmStreamPairs{128, 8, 8, 2, 1, 2, 2};

inline bool spmm_stream_variant_supported(const SpmmStreamVariant& v) {
#define BSP_SPMM_STREAM_MATCH(TN, SB, SA, NB, PP, EPS, SR)                                           \
    if (v.tile_n == TN && v.sb == SB && v.sa == SA && v.nbw == NB && v.pipes == PP && v.eps == EPS && \
        v.sr == SR)                                                                                  \
        return true;
    BSP_SPMM_STREAM_VARIANTS(BSP_SPMM_STREAM_MATCH)
#undef BSP_SPMM_STREAM_MATCH
    return false;
}

inline int spmm_stream_lds_bytes(const SpmmStreamVariant& v) {
    return v.pipes * (64 * v.tile_n * v.sb + 2048 * v.sa * v.sr + (v.sr > 1 ? 8 * v.sa : 0)) +
           (v.pipes > 1 ? 4 * (v.tile_n / 128) * 16 * 64 * 4 : 0);
}

hipError_t launch_spmm_stream(const SpmmStreamArgs& a, const SpmmStreamVariant& v, bool out_bf16, int grid,
                              hipStream_t stream);

// Whether an SpMM plan on A (R x C blocks) and N output columns runs the
// persistent kernel, with which variant and workgroups per compute unit
// (bsp_capi.cpp; environment overrides are read here, at plan creation).
bool choose_spmm_stream(const bsp_bsr_desc* a, int64_t N, int cus, SpmmStreamVariant* sv, int* wpc);
// Sets the calling thread's last-error message (bsp_last_error) and returns status.
int record_error(int status, const std::string& msg);

// Fused attention pair: the SpMM arguments with the mask as A (a = mask
// values), V as B (b, ldb) and O as C (c, ldc), N = head dimension; plus Q and K.
struct AttentionArgs {
    SpmmArgs s;
    const uint16_t* q;        // Q (bf16), row-major queries x d, leading dim ldq
    const uint16_t* k;        // K (bf16), row-major keys x d, leading dim ldk
    int64_t ldq;
    int64_t ldk;
};

struct SddmmArgs {
    const uint16_t* mask;     // mask block values (bf16), nblocks*R*C
    const uint16_t* x;        // X (bf16), row-major M x K, leading dim ldx
    const uint16_t* y;        // Y (bf16), K x N row-major or N x K row-major (col-major Y)
    void* out;                // output block values (fp32 or bf16), nblocks*R*C
    const SddmmItem* wgs;     // one record per workgroup (empty range: idle)
    const int32_t* ent_col;   // first column of Y per entry
    const int64_t* ent_off;   // element offset of the output sub-block per entry
    int64_t ldx;
    int64_t ldy;
    int32_t ldo;              // row stride inside an output / mask block (= C)
    int32_t K;
    int32_t one_shot;         // 1: sddmm_shot_kernel (chosen at plan creation)
    int32_t skips;            // work the instrumented build leaves out (kSkip*; 0 in libbsparse.so)
};

// The one-shot SDDMM kernel takes K of 32, 64, 128 or 256 and items of at
// most four entries (one per wave).
inline bool sddmm_shot_supported(int64_t K, int max_item_entries) {
    return (K == 32 || K == 64 || K == 128 || K == 256) && max_item_entries <= 4;
}

struct SpgemmArgs {
    const uint16_t* a;          // A block values (bf16), R x C blocks
    const uint16_t* b;          // B block values (bf16), C x BC blocks
    void* out;                  // C block values (fp32 or bf16), R x BC blocks
    const SpgemmTask* tasks;    // one per 32x32 output sub-block
    const uint64_t* terms;      // per product: A offset / 32 (low 32 bits) | B offset / 32 (high)
    const SpgemmRun* runs;      // grid * 4 wave runs
    int32_t lda;                // row stride inside an A block (= C)
    int32_t ldb;                // row stride inside a B block (= BC)
    int32_t ldo;                // row stride inside an output block (= BC)
    int32_t wg_per_xcd;         // workgroups per XCD (grid / kNumXcd)
};

// Floats of partial-result scratch per (slot, tile): a 32 x tile_n block.
inline int64_t spmm_partial_floats(int tile_n) { return (int64_t)tile_n * 32; }

// Compiled SpMM kernel variants: workgroup tile width (4 waves of 32 or 64
// columns), ring depth (entries in flight + 1) and row group (32-row stripes
// of one block row per workgroup; groups take 128-column tiles, or 256 in the
// wide group kernel).  LDS per workgroup = (2 KB * group + 64 * tile_n bytes)
// * stages, except that the wide kernel fetching A in entry pairs (C a
// multiple of 64) keeps 2 * (stages / 2 + 1) A slots: group 8 with three
// stages takes 112 KB, not 96.  Two workgroups share a compute unit while
// that is at most 80 KB (the wide kernel: groups of 2 and 4 with three stages).
#define BSP_SPMM_VARIANTS(X) \
    X(128, 4, 1)             \
    X(128, 6, 1)             \
    X(128, 8, 1)             \
    X(256, 3, 1)             \
    X(256, 4, 1)             \
    X(128, 6, 2)             \
    X(256, 3, 2)             \
    X(128, 4, 4)             \
    X(128, 5, 4)             \
    X(256, 3, 4)             \
    X(128, 3, 8)             \
    X(128, 4, 8)             \
    X(256, 3, 8)             \
    X(256, 4, 8)

struct SpmmVariant {
    int tile_n;
    int stages;
    int group;
    int waves = 4;  // 256-column row groups: 8 (default) or 4 waves per workgroup
};

inline bool spmm_variant_supported(const SpmmVariant& v) {
#define BSP_SPMM_MATCH(TN, S, G) \
    if (v.tile_n == TN && v.stages == S && v.group == G) return true;
    BSP_SPMM_VARIANTS(BSP_SPMM_MATCH)
#undef BSP_SPMM_MATCH
    return false;
}

// Default ring depth for a tile width and row group.
inline SpmmVariant spmm_default_variant(int tile_n, int group) {
    switch (group) {
        case 2: return tile_n >= 256 ? SpmmVariant{256, 3, 2, 8} : SpmmVariant{128, 6, 2};
        case 4: return tile_n >= 256 ? SpmmVariant{256, 3, 4, 8} : SpmmVariant{128, 4, 4};
        case 8: return tile_n >= 256 ? SpmmVariant{256, 4, 8, 8} : SpmmVariant{128, 3, 8};
        default: return tile_n >= 256 ? SpmmVariant{256, 4, 1} : SpmmVariant{128, 6, 1};
    }
}

// Launches the SpMM kernel and, when the plan has split rows, the reduce kernel.
hipError_t launch_spmm(const SpmmArgs& a, const SpmmVariant& v, bool out_bf16, int grid, int n_split,
                       hipStream_t stream);
// Head dimensions of the fused attention kernel (one 128-column tile).
inline bool attention_head_dim_supported(int64_t d) { return d == 32 || d == 64 || d == 128; }
constexpr int kAttentionTileN = 128;
constexpr int kAttentionStages = 4;

// Launches the fused attention kernel and, for split rows, the reduce kernel.
hipError_t launch_attention(const AttentionArgs& a, int head_dim, bool out_bf16, int grid, int n_split,
                            hipStream_t stream);

hipError_t launch_sddmm(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid,
                        hipStream_t stream);

// Ring depths of the SpGEMM kernel (products in flight + 1 per wave; LDS per
// workgroup = 16 KB * stages) and the default.
inline bool spgemm_stages_supported(int s) { return s == 2 || s == 3 || s == 4; }
constexpr int kSpgemmStages = 3;
hipError_t launch_spgemm(const SpgemmArgs& a, int stages, bool out_bf16, int grid, hipStream_t stream);

}  // namespace bsp
