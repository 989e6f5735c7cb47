// HIP kernels for block-sparse SpMM and SDDMM on gfx950 (MI355X).
//
// Every product is cut into 32x32 sub-blocks and issued as
// v_mfma_f32_32x32x16_bf16 (bf16 operands, fp32 accumulation), two per
// 32-deep block.  Lane layout of that instruction (64 lanes, q = lane / 32):
//   A operand: lane holds A[lane % 32][16*s + 8*q + 0..7]  (s = k-step)
//   B operand: lane holds B[16*s + 8*q + 0..7][lane % 32]
//   result:    acc[4*i + j] is C[8*i + 4*q + j][lane % 32]
// Both operands must therefore be contiguous along k in each lane.  A blocks
// and X rows already are; a row-major dense operand (B of SpMM, Y of SDDMM) is
// contiguous along n instead, so it is staged through LDS as k-pairs: dword
// (p, n) holds (B[2p][n], B[2p+1][n]), and a lane gathers its 8 k-values with
// four dword reads.
//
// Reference semantics followed: block_spmm/inc/bsr_matrix.hpp:954-1000 (SpMM),
// sparse_common/bsr_matrix.hpp:816-857 (SDDMM).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "bsp_kernels.hpp"

namespace bsp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Packs rows k (r0) and k+1 (r1), 8 columns each, into 8 k-pair dwords in
// column order.
__device__ __forceinline__ void pack_pairs(const u32x4& r0, const u32x4& r1, u32x4& lo,
                                           u32x4& hi) {
    lo.x = (r0.x & 0xffffu) | (r1.x << 16);
    lo.y = (r0.x >> 16) | (r1.x & 0xffff0000u);
    lo.z = (r0.y & 0xffffu) | (r1.y << 16);
    lo.w = (r0.y >> 16) | (r1.y & 0xffff0000u);
    hi.x = (r0.z & 0xffffu) | (r1.z << 16);
    hi.y = (r0.z >> 16) | (r1.z & 0xffff0000u);
    hi.z = (r0.w & 0xffffu) | (r1.w << 16);
    hi.w = (r0.w >> 16) | (r1.w & 0xffff0000u);
}

// ---------------------------------------------------------------------------
// SpMM.  Workgroup = one work item (a run of one 32-row stripe's sub-block
// products) x one tile of TN output columns; NW waves, each owning NTW 32-col
// MFMA tiles.  Per entry: the 32x32 A sub-block and the 32 x TN slice of B are
// loaded (16-byte, coalesced) into registers one entry ahead, then written to
// a double-buffered LDS stage; one barrier per entry.
template <int NW, int NTW, bool OUT_BF16>
__global__ __launch_bounds__(NW * 64) void spmm_kernel(SpmmArgs p) {
    constexpr int NT = NW * 64;
    constexpr int TN = NW * NTW * 32;
    constexpr int A_LD = 40;      // bf16 per LDS row of A (32 + 8 pad)
    constexpr int B_LD = TN + 8;  // dwords per LDS k-pair row of B
    constexpr int ACH = (128 + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][32 * A_LD];
    __shared__ __attribute__((aligned(16))) uint32_t sB[2][16 * B_LD];
    __shared__ int s_last;

    const int wg = p.wgmap[blockIdx.x];
    if (wg < 0) return;
    const int item_id = wg / p.n_tiles;
    const int tile = wg - item_id * p.n_tiles;
    const SpmmItem it = p.items[item_id];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, q = lane >> 5;
    const int n0 = tile * TN;

    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    u32x4 ra[ACH];
    u32x4 rb0[NTW], rb1[NTW];

    auto gload = [&](int e) {
        const int32_t brow = p.ent_row[e];
        const uint16_t* ablk = p.a + p.ent_off[e];
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + i * NT;
            if (c < 128)
                ra[i] = *(const u32x4*)(ablk + (int64_t)(c >> 2) * p.lda + (c & 3) * 8);
        }
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int qq = tid + i * NT;
            const int pr = qq / (TN / 8), c8 = (qq % (TN / 8)) * 8;
            const uint16_t* src = p.b + (int64_t)(brow + 2 * pr) * p.ldb + n0 + c8;
            rb0[i] = *(const u32x4*)src;
            rb1[i] = *(const u32x4*)(src + p.ldb);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; ++i) {
            const int c = tid + i * NT;
            if (c < 128) *(u32x4*)&sA[buf][(c >> 2) * A_LD + (c & 3) * 8] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
            const int qq = tid + i * NT;
            const int pr = qq / (TN / 8), c8 = (qq % (TN / 8)) * 8;
            u32x4 lo, hi;
            pack_pairs(rb0[i], rb1[i], lo, hi);
            *(u32x4*)&sB[buf][pr * B_LD + c8] = lo;
            *(u32x4*)&sB[buf][pr * B_LD + c8 + 4] = hi;
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const u32x4 av = *(const u32x4*)&sA[buf][l32 * A_LD + 16 * s + 8 * q];
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                const uint32_t* bp = &sB[buf][(8 * s + 4 * q) * B_LD + wave * (NTW * 32) + nt * 32 + l32];
                u32x4 bv;
                bv.x = bp[0];
                bv.y = bp[B_LD];
                bv.z = bp[2 * B_LD];
                bv.w = bp[3 * B_LD];
                acc[nt] = mfma32(av, bv, acc[nt]);
            }
        }
    };

    const int e_begin = it.e_begin, e_end = it.e_end;
    if (e_begin < e_end) gload(e_begin);
    for (int e = e_begin; e < e_end; ++e) {
        const int buf = (e - e_begin) & 1;
        lstore(buf);
        if (e + 1 < e_end) gload(e + 1);
        __syncthreads();
        compute(buf);
    }

    if (it.slot >= 0) {
        // Piece of a split row: publish the partial, and let the last piece to
        // arrive add all partials in piece order (deterministic) and store.
        constexpr int PER = NTW * 16 * NT;  // floats per (slot, tile)
        float* mine = p.ws + ((int64_t)it.slot * p.n_tiles + tile) * PER;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[(nt * 16 + v) * NT + tid] = acc[nt][v];
        __threadfence();
        __syncthreads();
        int32_t* counter = p.cnt + (int64_t)it.base * p.n_tiles + tile;
        if (tid == 0) {
            const int prev = atomicAdd(counter, 1);
            s_last = (prev == it.npieces - 1);
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[nt][v] = 0.0f;
        for (int pc = 0; pc < it.npieces; ++pc) {
            const float* src = p.ws + ((int64_t)(it.base + pc) * p.n_tiles + tile) * PER;
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[nt][v] += src[(nt * 16 + v) * NT + tid];
        }
        if (tid == 0) *counter = 0;  // ready for the next launch
    }

    const int64_t r0 = (int64_t)it.row * 32;
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
        const int64_t col = n0 + wave * (NTW * 32) + nt * 32 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t row = r0 + 8 * (v >> 2) + 4 * q + (v & 3);
            if (OUT_BF16)
                ((uint16_t*)p.c)[row * p.ldc + col] = f32_to_bf16_rne(acc[nt][v]);
            else
                ((float*)p.c)[row * p.ldc + col] = acc[nt][v];
        }
    }
}

// ---------------------------------------------------------------------------
// SDDMM.  Workgroup = one work item (up to `chunk` output sub-blocks sharing
// the same 32 rows of X); its four waves take the item's entries round-robin
// and each computes one 32x32 output sub-block at a time over the full K,
// then applies the mask values and stores.  X rows are read straight into
// A-operand registers (contiguous along k).  Y in BSP_COL_MAJOR (Y^T row-major,
// e.g. K of Q*K^T) is read the same way; row-major Y goes through a
// wave-private LDS k-pair stage.
template <bool Y_COLMAJOR, bool OUT_BF16>
__global__ __launch_bounds__(256) void sddmm_kernel(SddmmArgs p) {
    constexpr int Y_LD = 40;  // dwords per LDS k-pair row (32 + 8 pad)
    __shared__ __attribute__((aligned(16))) uint32_t sY[4][16 * Y_LD];

    const int wg = p.wgmap[blockIdx.x];
    if (wg < 0) return;
    const SddmmItem it = p.items[wg];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, q = lane >> 5;
    const uint16_t* xlane = p.x + (int64_t)(it.x_row0 + l32) * p.ldx + 8 * q;
    uint32_t* sw = sY[wave];
    const int pr = lane >> 2, c8 = (lane & 3) * 8;  // row-major Y staging role

    for (int e = it.e_begin + wave; e < it.e_end; e += 4) {
        const int32_t ycol = p.ent_col[e];
        const int64_t off = p.ent_off[e];
        f32x16 acc;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = 0.0f;

        if (Y_COLMAJOR) {
            const uint16_t* ylane = p.y + (int64_t)(ycol + l32) * p.ldy + 8 * q;
            for (int k0 = 0; k0 < p.K; k0 += 32) {
                const u32x4 a0 = *(const u32x4*)(xlane + k0);
                const u32x4 a1 = *(const u32x4*)(xlane + k0 + 16);
                const u32x4 b0 = *(const u32x4*)(ylane + k0);
                const u32x4 b1 = *(const u32x4*)(ylane + k0 + 16);
                acc = mfma32(a0, b0, acc);
                acc = mfma32(a1, b1, acc);
            }
        } else {
            const uint16_t* ysrc = p.y + (int64_t)(2 * pr) * p.ldy + ycol + c8;
            for (int k0 = 0; k0 < p.K; k0 += 32) {
                const u32x4 a0 = *(const u32x4*)(xlane + k0);
                const u32x4 a1 = *(const u32x4*)(xlane + k0 + 16);
                const u32x4 y0 = *(const u32x4*)(ysrc + (int64_t)k0 * p.ldy);
                const u32x4 y1 = *(const u32x4*)(ysrc + (int64_t)(k0 + 1) * p.ldy);
                u32x4 lo, hi;
                pack_pairs(y0, y1, lo, hi);
                // The previous k-step's reads of this wave-private stage were
                // issued before these writes; LDS serves one wave in order.
                *(u32x4*)&sw[pr * Y_LD + c8] = lo;
                *(u32x4*)&sw[pr * Y_LD + c8 + 4] = hi;
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const uint32_t* bp = &sw[(8 * s + 4 * q) * Y_LD + l32];
                    u32x4 bv;
                    bv.x = bp[0];
                    bv.y = bp[Y_LD];
                    bv.z = bp[2 * Y_LD];
                    bv.w = bp[3 * Y_LD];
                    acc = mfma32(s == 0 ? a0 : a1, bv, acc);
                }
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
        }

#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t idx = off + (int64_t)(8 * (v >> 2) + 4 * q + (v & 3)) * p.ldo + l32;
            const float val = acc[v] * bf16_to_f32(p.mask[idx]);
            if (OUT_BF16)
                ((uint16_t*)p.out)[idx] = f32_to_bf16_rne(val);
            else
                ((float*)p.out)[idx] = val;
        }
    }
}

// ---------------------------------------------------------------------------
hipError_t launch_spmm(const SpmmArgs& a, int tile_n, bool out_bf16, int grid,
                       hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
#define BSP_SPMM_CASE(TN, NW, NTW)                                                        \
    case TN:                                                                              \
        if (out_bf16)                                                                     \
            hipLaunchKernelGGL((spmm_kernel<NW, NTW, true>), dim3(grid), dim3(NW * 64), 0, \
                               stream, a);                                                \
        else                                                                              \
            hipLaunchKernelGGL((spmm_kernel<NW, NTW, false>), dim3(grid), dim3(NW * 64), 0, \
                               stream, a);                                                \
        break;
    switch (tile_n) {
        BSP_SPMM_CASE(256, 4, 2)
        BSP_SPMM_CASE(128, 4, 1)
        BSP_SPMM_CASE(64, 2, 1)
        BSP_SPMM_CASE(32, 1, 1)
        default:
            return hipErrorInvalidValue;
    }
#undef BSP_SPMM_CASE
    return hipGetLastError();
}

hipError_t launch_sddmm(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid,
                        hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    if (y_colmajor) {
        if (out_bf16)
            hipLaunchKernelGGL((sddmm_kernel<true, true>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((sddmm_kernel<true, false>), dim3(grid), dim3(256), 0, stream, a);
    } else {
        if (out_bf16)
            hipLaunchKernelGGL((sddmm_kernel<false, true>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((sddmm_kernel<false, false>), dim3(grid), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace bsp
