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
// contiguous along n instead.  SpMM stages B in LDS as it lies in memory and
// reads it with the LDS transpose read (ds_read_b64_tr_b16); SDDMM re-packs
// row-major Y into k-pairs in LDS (dword (p, n) holds (Y[2p][n], Y[2p+1][n]))
// and a lane gathers its 8 k-values with four dword reads.
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

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// Reads plan data (written before the launch, never by a kernel) through the
// constant address space so that it is fetched with scalar loads.
template <typename T>
__device__ __forceinline__ T load_const(const T* ptr) {
    static_assert(sizeof(T) % 4 == 0, "plan records are whole dwords");
    const __attribute__((address_space(4))) uint32_t* src =
        (const __attribute__((address_space(4))) uint32_t*)(uintptr_t)ptr;
    uint32_t w[sizeof(T) / 4];
#pragma unroll
    for (unsigned i = 0; i < sizeof(T) / 4; ++i) w[i] = src[i];
    T out;
    __builtin_memcpy(&out, w, sizeof(T));
    return out;
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
// products) x one tile of TN = 128*NTW output columns; 4 waves, each owning
// NTW 32-column MFMA tiles.
//
// Data movement is an S-stage ring in LDS filled by direct global->LDS loads
// (global_load_lds_dwordx4, no register staging), so S-1 entries are in flight
// per workgroup while one is multiplied; one barrier per entry.  The operands
// of the next entry are read into registers while the current one is
// multiplied.  Stage s holds (in an A array and a B array)
//   - the entry's 32x32 A sub-block (2 KB, shared by the four waves) as four
//     512-byte segments, segment w = rows 8w..8w+7, its 16-byte chunk
//     8*j + r%8 = A[8w + r%8][8*j .. 8*j+7].  Wave w loads segment w from 512
//     contiguous bytes (a 32x32 block), and the A operand of k-step s for lane
//     (r, q) is the chunk 8*(2s+q) + r%8 of segment r/8: each 8-lane group of
//     the ds_read_b128 reads 128 contiguous bytes;
//   - the 32 x TN slice of row-major B (64*TN bytes), row k at k*2*TN bytes,
//     its 16-byte chunk c stored at slot c ^ 4*(k % 4) (spreads the rows one
//     transpose read touches over the LDS banks).
// The B operand (8 consecutive k at one column) is read with two
// ds_read_b64_tr_b16: in each 16-lane group, source lane 4*j + m addresses
// row k0+j, columns n+4m..n+4m+3, and output lane i receives rows k0..k0+3 of
// column n+i.
namespace spmm_detail {

constexpr int kA_BYTES = 2048;

// Direct global->LDS load of 16 bytes per lane: lane L's bytes land at
// lds_wave_base + 16*L (lds_wave_base is wave-uniform).  Issued as inline asm
// so that the compiler does not track it: its own bookkeeping would otherwise
// wait for every outstanding load before each LDS read or barrier, which
// serialises the ring.  Completion is awaited explicitly with wait_vmcnt.
// Nothing else in these kernels uses M0.
__device__ __forceinline__ void gl_lds16(const void* g, uint32_t lds_wave_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_wave_base);
    __asm__ volatile(
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %0, off"
        :
        : "v"(g), "s"(lds)
        : "memory");
}

// Workgroup barrier without a memory fence (a fence would wait for all
// outstanding loads); the empty asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void barrier_no_fence() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] bits 3:0, expcnt bits 6:4, lgkmcnt bits 11:8, vmcnt[5:4] bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 0x3) << 14));
    __asm__ volatile("" ::: "memory");
}

// Waits until at most PER*n vector loads of this wave are outstanding, n <= NMAX.
template <int PER, int NMAX>
__device__ __forceinline__ void wait_stages(int n) {
    if constexpr (NMAX >= 0) {
        if (n >= NMAX) {
            wait_vmcnt<PER * NMAX>();
            return;
        }
        wait_stages<PER, NMAX - 1>(n);
    }
}

__device__ __forceinline__ u32x4 ld_tr_b16(const uint8_t* lds) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(__attribute__((address_space(3))) uint8_t*)lds);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 w = __builtin_bit_cast(u32x2, v);
    return u32x4{w.x, w.y, 0u, 0u};
}

}  // namespace spmm_detail

// Stores the accumulators of one 32 x TN tile (columns past N skipped).
template <int NTW, bool OUT_BF16>
__device__ __forceinline__ void spmm_store_tile(const SpmmArgs& p, const f32x16 (&acc)[NTW], int64_t row0,
                                                int n0, int wave, int l32, int q) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
        const int64_t col = n0 + wave * (NTW * 32) + nt * 32 + l32;
        if (col >= p.N) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t row = row0 + 8 * (v >> 2) + 4 * q + (v & 3);
            if (OUT_BF16)
                ((uint16_t*)p.c)[row * p.ldc + col] = f32_to_bf16_rne(acc[nt][v]);
            else
                ((float*)p.c)[row * p.ldc + col] = acc[nt][v];
        }
    }
}

template <int NTW, int S, bool OUT_BF16>
__global__ __launch_bounds__(256) void spmm_kernel(SpmmArgs p) {
    using namespace spmm_detail;
    constexpr int TN = 128 * NTW;
    constexpr int ROW_BYTES = 2 * TN;
    constexpr int B_BYTES = 32 * ROW_BYTES;
    constexpr int BI = B_BYTES / 1024 / 4;  // B wave-instructions per wave per step (= 2*NTW)
    constexpr int PER = BI + 1;              // loads per wave per step (B + a half-wave of A)
    constexpr int B_RING = S * kA_BYTES;     // A ring first, then the B ring
    static_assert(PER * (S - 2) < 64, "vmcnt budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[S * (kA_BYTES + B_BYTES)];

    const SpmmWg it = load_const(p.wgs + blockIdx.x);
    if (it.row < 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const int l32 = lane & 31, q = lane >> 5;
    const int n0 = it.tile * TN;
    const uint32_t lds0 = lds_address(smem);

    // Loads of one entry, per wave: lanes 0-31 fetch A segment `wave` (lane
    // 8*j + i loads A[8*wave + i][8*j .. +7]) and BI wave-wide 1 KB pieces of
    // the swizzled B slice.
    const int a_goff = (8 * wave + (lane & 7)) * p.lda + 8 * ((lane & 31) >> 3);
    const uint32_t a_lds = lds0 + wave * 512;
    const uint32_t b_lds = lds0 + B_RING + wave * BI * 1024;
    int64_t b_goff[BI];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
        const int byte = (wave * BI + j) * 1024 + lane * 16;
        const int r = byte / ROW_BYTES;
        const int slot = (byte % ROW_BYTES) / 16;
        // Columns past N (a partial last tile) read a valid chunk; they are not stored.
        const int col = min(n0 + 8 * (slot ^ (4 * (r & 3))), p.N - 8);
        b_goff[j] = (int64_t)r * p.ldb + col;
    }

    // Entry words: low 32 bits = first row of B, high 32 bits = A offset / 32.
    const int e0 = it.e_begin, n = it.e_end - it.e_begin;
    const uint32_t* words = (const uint32_t*)(p.ents + e0);
    // Issues the PER loads of one entry into ring stage `stage`.
    auto issue = [&](int e, int stage) {
        const uint32_t bw = load_const(words + 2 * e);
        const uint32_t aw = load_const(words + 2 * e + 1);
        if (lane < 32) gl_lds16(p.a + (int64_t)aw * 32 + a_goff, a_lds + stage * kA_BYTES);
        const uint16_t* bpan = p.b + (int64_t)bw * p.ldb;
#pragma unroll
        for (int j = 0; j < BI; ++j) gl_lds16(bpan + b_goff[j], b_lds + stage * B_BYTES + j * 1024);
    };

    // Per-lane LDS offsets of the operand reads (ring-stage relative).
    const int a_rd = (l32 >> 3) * 512 + (8 * q + (l32 & 7)) * 16;  // + s * 256
    int b_rd[2][2][NTW];         // [k-step][half][tile]
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                const int g = lane >> 4;
                const int r = 16 * s2 + 8 * (g >> 1) + 4 * h + ((lane & 15) >> 2);
                const int col = wave * (NTW * 32) + nt * 32 + 16 * (g & 1) + 4 * (lane & 3);
                const int c = col >> 3;
                b_rd[s2][h][nt] = r * ROW_BYTES + 16 * (c ^ (4 * (r & 3))) + 2 * (col & 7);
            }

    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    // Operands of one entry in registers: A of both k-steps and the B
    // operands of every tile.  The LDS reads of entry k+1 are issued right
    // after entry k's MFMAs, so their latency overlaps the MFMAs, the wait for
    // the next stage and the barrier.
    struct Operands {
        u32x4 a[2];
        u32x4 b[2][NTW];
    };
    auto read_operands = [&](int stage, Operands& o) {
        const uint8_t* as = smem + stage * kA_BYTES;
        const uint8_t* bs = smem + B_RING + stage * B_BYTES;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            o.a[s2] = *(const u32x4*)(as + s2 * 256 + a_rd);
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
                const u32x4 lo = ld_tr_b16(bs + b_rd[s2][0][nt]);
                const u32x4 hi = ld_tr_b16(bs + b_rd[s2][1][nt]);
                o.b[s2][nt] = u32x4{lo.x, lo.y, hi.x, hi.y};
            }
        }
    };
    auto multiply = [&](const Operands& o) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) acc[nt] = mfma32(o.a[s2], o.b[s2][nt], acc[nt]);
    };

    // Entry e lives in ring stage e % S.  Entries 0..S-2 are issued first;
    // entry S-1 goes into the still unused last stage once entry 0 has landed.
    // Iteration k multiplies entry k from registers, waits for entry k+1 to
    // land (the loads issued after it are those of entries k+2..k+S-1), and
    // after the barrier (every wave holds entry k's operands in registers, so
    // stage k % S is free) issues entry k+S into stage k % S and reads entry
    // k+1's operands.
#pragma unroll
    for (int e = 0; e < S - 1; ++e)
        if (e < n) issue(e, e);
    Operands cur;
    if (n > 0) {
        wait_stages<PER, S - 2>(n - 1);  // entry 0 landed
        barrier_no_fence();
        if (S - 1 < n) issue(S - 1, S - 1);
        read_operands(0, cur);
    }
    int k = 0;
    int stage = 0;  // stage of entry k
    for (; k < n - S + 1; ++k) {
        multiply(cur);
        // Entry k's operand reads must be complete before the barrier frees
        // its stage (the compiler would otherwise wait only at their first
        // use, which it may schedule after the barrier and the next issue).
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_vmcnt<PER * (S - 2)>();  // entry k+1 landed
        barrier_no_fence();
        if (k + S < n) issue(k + S, stage);
        stage = stage == S - 1 ? 0 : stage + 1;
        read_operands(stage, cur);
    }
    // Tail: every entry is issued; fewer are in flight.
    for (; k < n; ++k) {
        multiply(cur);
        if (k + 1 < n) {
            wait_stages<PER, S - 2>(n - 2 - k);  // entry k+1 landed
            barrier_no_fence();
            stage = stage == S - 1 ? 0 : stage + 1;
            read_operands(stage, cur);
        }
    }

    if (it.slot >= 0) {
        // Piece of a split row: the partial goes to scratch; spmm_reduce_kernel
        // adds the pieces in order after this launch.
        constexpr int PF = NTW * 16 * 256;
        float* mine = p.ws + ((int64_t)it.slot * p.n_tiles + it.tile) * PF;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[(nt * 16 + v) * 256 + tid] = acc[nt][v];
        return;
    }
    spmm_store_tile<NTW, OUT_BF16>(p, acc, (int64_t)it.row * 32, n0, wave, l32, q);
}

// Adds the partials of each split row in piece order (deterministic) and
// stores the 32 x TN tile: one workgroup per (split row, tile).
template <int NTW, bool OUT_BF16>
__global__ __launch_bounds__(256) void spmm_reduce_kernel(SpmmArgs p) {
    constexpr int PF = NTW * 16 * 256;
    const int tile = blockIdx.x % p.n_tiles;
    const SpmmSplit sp = load_const(p.splits + blockIdx.x / p.n_tiles);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    f32x16 acc[NTW];
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[nt][v] = 0.0f;
    for (int pc = 0; pc < sp.npieces; ++pc) {
        const float* src = p.ws + ((int64_t)(sp.base + pc) * p.n_tiles + tile) * PF;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[nt][v] += src[(nt * 16 + v) * 256 + tid];
    }
    spmm_store_tile<NTW, OUT_BF16>(p, acc, (int64_t)sp.row * 32, tile * 128 * NTW, wave, lane & 31, lane >> 5);
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

    const SddmmItem it = p.wgs[blockIdx.x];
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
template <int NTW, int S>
static void launch_spmm_t(const SpmmArgs& a, bool out_bf16, int grid, int n_split, hipStream_t stream) {
    if (out_bf16)
        hipLaunchKernelGGL((spmm_kernel<NTW, S, true>), dim3(grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((spmm_kernel<NTW, S, false>), dim3(grid), dim3(256), 0, stream, a);
    if (n_split > 0) {
        const int g = n_split * a.n_tiles;
        if (out_bf16)
            hipLaunchKernelGGL((spmm_reduce_kernel<NTW, true>), dim3(g), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((spmm_reduce_kernel<NTW, false>), dim3(g), dim3(256), 0, stream, a);
    }
}

hipError_t launch_spmm(const SpmmArgs& a, const SpmmVariant& v, bool out_bf16, int grid, int n_split,
                       hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    if (!spmm_variant_supported(v)) return hipErrorInvalidValue;
#define BSP_SPMM_CASE(TN, S)                                              \
    if (v.tile_n == TN && v.stages == S) {                               \
        launch_spmm_t<TN / 128, S>(a, out_bf16, grid, n_split, stream);  \
        return hipGetLastError();                                        \
    }
    BSP_SPMM_VARIANTS(BSP_SPMM_CASE)
#undef BSP_SPMM_CASE
    return hipErrorInvalidValue;
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
