// Kernel argument blocks and launchers shared by the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsp_schedule.hpp"

namespace bsp {

struct SpmmArgs {
    const uint16_t* a;        // A block values (bf16), nblocks*R*C
    const uint16_t* b;        // B (bf16), row-major K x N, leading dim ldb
    void* c;                  // C (fp32 or bf16), row-major M x N, leading dim ldc
    const SpmmItem* items;
    const int32_t* ent_row;   // first row of B per entry
    const int64_t* ent_off;   // element offset of the A sub-block per entry
    const int32_t* wgmap;     // workgroup -> item * n_tiles + tile, or -1
    float* ws;                // partial results of split rows
    int32_t* cnt;             // arrival counters of split rows (zero between launches)
    int64_t ldb;
    int64_t ldc;
    int32_t lda;              // row stride inside an A block (= C)
    int32_t n_tiles;
};

struct SddmmArgs {
    const uint16_t* mask;     // mask block values (bf16), nblocks*R*C
    const uint16_t* x;        // X (bf16), row-major M x K, leading dim ldx
    const uint16_t* y;        // Y (bf16), K x N row-major or N x K row-major (col-major Y)
    void* out;                // output block values (fp32 or bf16), nblocks*R*C
    const SddmmItem* items;
    const int32_t* ent_col;   // first column of Y per entry
    const int64_t* ent_off;   // element offset of the output sub-block per entry
    const int32_t* wgmap;     // workgroup -> item, or -1
    int64_t ldx;
    int64_t ldy;
    int32_t ldo;              // row stride inside an output / mask block (= C)
    int32_t K;
};

// Number of floats of partial-result scratch per (slot, tile) for a tile width.
inline int64_t spmm_partial_floats(int tile_n) {
    // NTW*16 accumulators per lane, NW*64 lanes; NW*NTW*32 == tile_n.
    return (int64_t)tile_n * 32;
}

hipError_t launch_spmm(const SpmmArgs& a, int tile_n, bool out_bf16, int grid, hipStream_t stream);
hipError_t launch_sddmm(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid,
                        hipStream_t stream);

}  // namespace bsp
