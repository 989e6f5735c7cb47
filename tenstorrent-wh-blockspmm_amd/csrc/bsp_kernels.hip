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
// contiguous along n instead: both kernels stage it in LDS as it lies in
// memory and read it with the LDS transpose read (ds_read_b64_tr_b16).
//
// Reference semantics followed: block_spmm/inc/bsr_matrix.hpp:954-1000 (SpMM),
// sparse_common/bsr_matrix.hpp:816-857 (SDDMM).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>

#include "bsp_kernels.hpp"
#ifdef BSP_TIMELINE
#include "bsparse_timeline.h"
#endif

namespace bsp {

// ---------------------------------------------------------------------------
// Per-workgroup timeline (the instrumented build, BSP_TIMELINE; the slots are
// listed in bsparse_timeline.h).  Wave 0 of a workgroup takes the stamps.
#ifdef BSP_TIMELINE
__device__ uint64_t* g_timeline_buf = nullptr;
__device__ int64_t g_timeline_cap = 0;

// Slots 0, 1, 2 and 63 held in registers and written when wave 0 ends, for a
// kernel whose wave 0 waits for all of its loads at once and whose LDS is
// sized to an exact occupancy (the one-shot SDDMM: two workgroups of 80 KB per
// compute unit, which a log in LDS would halve).
struct TimelineRegs {
    uint64_t t0 = 0, t1 = 0, t2 = 0;  // (scalars: a lane-indexed array would go to scratch)
    __device__ __forceinline__ TimelineRegs() { t0 = wall_clock64(); }
    __device__ __forceinline__ void mark(int i) {
        if (i == 1) t1 = wall_clock64();
        if (i == 2) t2 = wall_clock64();
    }
    __device__ __forceinline__ void flush() {
        const uint64_t end = wall_clock64();
        uint64_t* buf = g_timeline_buf;
        const int l = threadIdx.x;
        const uint64_t v = l == 0 ? t0 : l == 1 ? t1 : l == 2 ? t2 : l == BSP_TIMELINE_SLOTS - 1 ? end : 0;
        if (l < BSP_TIMELINE_SLOTS && buf && (int64_t)blockIdx.x < g_timeline_cap)
            buf[(int64_t)blockIdx.x * BSP_TIMELINE_SLOTS + l] = v;
    }
};
// Stamps stored straight to the attached buffer by lane 0 of wave 0, for a
// kernel whose wave 0 waits for none of its own vector-memory operations
// (the persistent and sweep SpMM, where wave 0 is an MFMA wave: it issues
// stores and no loads, and waits only for its LDS reads; a stamp store in a
// loader wave's queue would stretch the waits that count its loads) and whose
// LDS has no bytes to spare (two 80 KB workgroups per compute unit, or one of
// 160 KB).  Slots a workgroup does not reach keep what the buffer held.
struct TimelineGlobal {
    uint64_t* row = nullptr;
    __device__ __forceinline__ TimelineGlobal() {
        uint64_t* buf = g_timeline_buf;
        if (buf && (int64_t)blockIdx.x < g_timeline_cap) row = buf + (int64_t)blockIdx.x * BSP_TIMELINE_SLOTS;
        mark(0);
    }
    __device__ __forceinline__ void mark(int i) {
        if (row && threadIdx.x == 0 && i >= 0 && i < BSP_TIMELINE_SLOTS) row[i] = wall_clock64();
    }
    __device__ __forceinline__ void flush() { mark(BSP_TIMELINE_SLOTS - 1); }
};
#define BSP_TL_DECL_REGS() TimelineRegs bsp_tl
#define BSP_TL_DECL_GLOBAL() TimelineGlobal bsp_tl
#define BSP_TL_MARK(i) bsp_tl.mark(i)
#define BSP_TL_FLUSH() bsp_tl.flush()
// Whether the launch leaves out a part of the work (kSkip* bit of the
// kernel arguments, a wave-uniform scalar).
#define BSP_SKIP(p, bit) (((p).skips & (bit)) != 0)
#else
#define BSP_TL_DECL_REGS() ((void)0)
#define BSP_TL_DECL_GLOBAL() ((void)0)
#define BSP_TL_MARK(i) ((void)0)
#define BSP_TL_FLUSH() ((void)0)
#define BSP_SKIP(p, bit) false
#endif

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with round-to-nearest-even: gfx950's v_cvt_pk_bf16_f32, which
// converts two values per instruction.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two values to packed bf16 (lo in bits 0-15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: lane l holds A[l%16][8*(l/16) .. +7] and
// B[8*(l/16) .. +7][l%16]; result element v of lane l is D[4*(l/16) + v][l%16].
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
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
//     8*(j ^ (w % 2)) + r%8 = A[8w + r%8][8*j .. 8*j+7] (a_load_offset,
//     a_read_offset).  Wave w loads segment w from 512 contiguous bytes (a
//     32x32 block), and the A operand of k-step s for lane (r, q) is chunk
//     2s+q of row r: each 8-lane group of the ds_read_b128 reads 128
//     contiguous bytes, and the XOR puts rows r and r+8 (same chunk) 128
//     bytes apart, so that each 16-lane quarter covers all 64 banks of the
//     LDS (without it, the segments 512 bytes apart hit the same 32 banks);
//   - the 32 x TN slice of row-major B (64*TN bytes), row k at k*2*TN bytes,
//     its 16-byte chunk c stored at slot c ^ 4*(k % 4) (spreads the rows one
//     transpose read touches over the LDS banks).
// The B operand (8 consecutive k at one column) is read with two
// ds_read_b64_tr_b16: in each 16-lane group, source lane 4*j + m addresses
// row k0+j, columns n+4m..n+4m+3, and output lane i receives rows k0..k0+3 of
// column n+i.
namespace spmm_detail {

constexpr int kA_BYTES = 2048;

// Element offset, from the sub-block's first element, of what lane `lane`
// of a 512-byte segment load fetches for segment g (rows 8g..8g+7) of a 32x32
// A sub-block with row stride lda: it lands at slot lane % 32 = 8*c' + r of
// the segment, holding row 8g + r, chunk c' ^ (g % 2).
__device__ __forceinline__ int a_load_offset(int g, int lane, int lda) {
    return (8 * g + (lane & 7)) * lda + 8 * (((lane & 31) >> 3) ^ (g & 1));
}
// Byte offset in the sub-block of lane (l32, q)'s A operand of k-step 0 (chunk
// q of row l32); k-step s adds 256 bytes (chunk 2s + q: (2s + q) ^ b = 2s + (q ^ b)).
__device__ __forceinline__ int a_read_offset(int l32, int q) {
    const int g = l32 >> 3;
    return g * 512 + (8 * (q ^ (g & 1)) + (l32 & 7)) * 16;
}

// Row layout of a 32x32 A sub-block (the persistent kernel): row r at 64 r,
// its 16-byte chunk c at slot c ^ ((r >> 2) & 3).  Load j (1 KB, rows
// 16j .. 16j+15): lane L fills slot L % 4 of row 16j + L / 4, so each four
// lanes fetch one row's 64 contiguous bytes.  Element offset of what lane L
// fetches in load j:
__device__ __forceinline__ int a_row_load_offset(int j, int lane, int lda) {
    const int r = 16 * j + (lane >> 2);
    return r * lda + 8 * ((lane & 3) ^ ((r >> 2) & 3));
}
// Byte offset of lane (l32, q)'s A operand of k-step s (chunk 2s + q of row
// l32).  A 16-lane quarter reads one chunk of 16 consecutive rows: their
// offsets modulo 256 bytes are 64 (r % 4) + 16 (chunk ^ ((r >> 2) & 3)), all
// sixteen distinct, so the quarter covers the 64 banks once.
__device__ __forceinline__ int a_row_read_offset(int l32, int q, int s) {
    return 64 * l32 + 16 * ((2 * s + q) ^ ((l32 >> 2) & 3));
}

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

// The same load with a wave-uniform 64-bit base in SGPRs and a per-lane
// 32-bit byte offset (the global saddr form): half the address data of the
// 64-bit form, and the per-lane offset stays loop-invariant, so issuing a
// product's loads needs no vector address arithmetic.
__device__ __forceinline__ void gl_lds16_s(uint32_t voff_bytes, const void* sbase, uint32_t lds_wave_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_wave_base);
    __asm__ volatile(
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff_bytes), "s"(sbase), "s"(lds)
        : "memory");
}

// The same with M0 = lds_base + IMM: one scalar add sets the LDS destination
// (gl_lds16_s takes an add and a move).  The loader waves of the persistent
// kernels issue several of these per entry, and a compute unit issues one
// scalar instruction per cycle across all of its waves.
template <int IMM>
__device__ __forceinline__ void gl_lds16_si(uint32_t voff_bytes, const void* sbase, uint32_t lds_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_base);
    if constexpr (IMM == 0) {
        __asm__ volatile(
            "s_mov_b32 m0, %2\n\t"
            "global_load_lds_dwordx4 %0, %1"
            :
            : "v"(voff_bytes), "s"(sbase), "s"(lds)
            : "memory");
    } else {
        __asm__ volatile(
            "s_add_u32 m0, %2, %3\n\t"
            "global_load_lds_dwordx4 %0, %1"
            :
            : "v"(voff_bytes), "s"(sbase), "s"(lds), "n"(IMM)
            : "memory", "scc");
    }
}

// The same with 4 bytes per lane (lane i's dword lands at M0 + 4i).
__device__ __forceinline__ void gl_lds4_s(uint32_t voff_bytes, const void* sbase, uint32_t lds_wave_base) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_wave_base);
    __asm__ volatile(
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dword %0, %1"
        :
        : "v"(voff_bytes), "s"(sbase), "s"(lds)
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

// Waits until this wave's LDS accesses (and scalar loads) have completed.
// The builtin, not inline asm: the compiler's own wait insertion then knows
// that the LDS reads before it have returned, and adds no waits of its own
// before later uses of the registers they wrote (with the asm form it kept
// them pending and made the products of a step wait for the reads of the
// next).
__device__ __forceinline__ void wait_lgkm0() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __asm__ volatile("" ::: "memory");
}

// Waits until at most PER*n + EXTRA vector loads of this wave are
// outstanding, n <= NMAX.
template <int PER, int NMAX, int EXTRA = 0>
__device__ __forceinline__ void wait_stages(int n) {
    if constexpr (NMAX >= 0) {
        if (n >= NMAX) {
            wait_vmcnt<PER * NMAX + EXTRA>();
            return;
        }
        wait_stages<PER, NMAX - 1, EXTRA>(n);
    }
}

// A pointer the compiler may hold in VGPRs made wave-uniform (SGPRs), for the
// saddr operand of gl_lds16_s / gl_lds4_s, which must be an SGPR pair.  Only
// for pointers that are uniform by construction (derived from plan words or
// kernel arguments), where the compiler's divergence analysis loses that.
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* ptr) {
    const uint64_t v = (uint64_t)(uintptr_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
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

// Output stores are non-temporal (global stores with nt: streamed through the
// L2 without displacing the operands it holds, completing at the L2).  The
// output is written once and never read by the kernel.  Against write-through
// stores (sc1: a store that completes only when it has left the L2), measured
// in one process on one MI355X, graph replay of the persistent SpMM kernel
// with cold operands: 4096^2 x 512 fp32 C at 1% 5.50 -> 3.88 us, 5%
// 6.29 -> 5.97 us, 25% 14.40 -> 14.10 us; the skewed 16384^2 x 1024 workload
// 43.3 -> 39.7 us; the attention SDDMM 6.93 -> 6.55 us; the group kernels and
// the fused attention kernel within 1%.  A wave that waits on vmcnt for loads
// issued after its stores (the SpGEMM ring) would also wait for write-through
// stores to leave the L2 (SpGEMM 8192^2 fp32: 108 us with them, 28 us with
// non-temporal stores).
template <typename T>
__device__ __forceinline__ void store_out(T* p, T v) {
    __builtin_nontemporal_store(v, p);
}

// Stores one 32x32 MFMA result at rows row0.., column col (this lane's
// column; skipped past N).
template <bool OUT_BF16>
__device__ __forceinline__ void store_tile32(const SpmmArgs& p, const f32x16& acc, int64_t row0, int64_t col,
                                             int q) {
    if (col >= p.N) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int64_t row = row0 + 8 * (v >> 2) + 4 * q + (v & 3);
        if (OUT_BF16)
            store_out(&((uint16_t*)p.c)[row * p.ldc + col], f32_to_bf16_rne(acc[v]));
        else
            store_out(&((float*)p.c)[row * p.ldc + col], acc[v]);
    }
}

// Stores the accumulators of one 32 x TN tile (wave w holds columns
// w*NTW*32 ..).
template <int NTW, bool OUT_BF16>
__device__ __forceinline__ void spmm_store_tile(const SpmmArgs& p, const f32x16 (&acc)[NTW], int64_t row0,
                                                int n0, int wave, int l32, int q) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt)
        store_tile32<OUT_BF16>(p, acc[nt], row0, n0 + wave * (NTW * 32) + nt * 32 + l32, q);
}

namespace spmm_detail {

// Runs the LDS ring of an SpMM-shaped kernel over n entries.  Entry e lives
// in ring stage e % S; issue(e, stage) issues its PER loads per wave,
// read(stage, ops) issues the LDS reads of its operands into registers,
// multiply(ops) accumulates.  Entries 0..S-2 are issued first; entry S-1
// goes into the still unused last stage once entry 0 has landed.  Step k
// (entry k+1 exists): wait for this wave's reads of entry k, wait for entry
// k+1 to land (the loads issued after it are those of entries k+2..k+S-1),
// barrier (every wave has entry k's operands, so stage k % S is free, and
// entry k+1 is visible), issue entry k+S into stage k % S, issue the reads of
// entry k+1, then multiply entry k: the MFMAs cover the reads' latency.  The
// loop is unrolled by two so the two operand sets keep their registers.
// With OVERLAP = false (one operand set, for kernels whose accumulators leave
// no registers for a second) entry k is multiplied before the barrier and
// entry k+1's reads follow it.  landed() runs once entry 0 (and every load
// issued before it) has landed and is visible to all waves.  With MIX (and
// OVERLAP), entry k+1's reads and entry k's products form one scheduling
// region.  With XCHG (and OVERLAP), read() may leave LDS data that the other
// waves' multiply() of the same entry reads: a barrier then also follows
// landed() (whose LDS reads complete first) and precedes a multiply() that no
// ring step separates from its entry's read().
template <int S, int PER, bool OVERLAP, class Ops, bool MIX = false, bool XCHG = false, class Issue, class Read,
          class Multiply, class Landed>
__device__ __forceinline__ void run_ring(int n, Issue&& issue, Read&& read, Multiply&& multiply,
                                         Landed&& landed) {
    static_assert(PER * (S - 2) < 64, "vmcnt budget");
    if (n <= 0) return;
#pragma unroll
    for (int e = 0; e < S - 1; ++e)
        if (e < n) issue(e, e);
    Ops o0;
    wait_stages<PER, S - 2>(n - 1);  // entry 0 landed
    barrier_no_fence();
    landed();
    auto xchg = [] {
        if constexpr (XCHG) {
            spmm_detail::wait_lgkm0();
            barrier_no_fence();
        }
    };
    xchg();
    if (S - 1 < n) issue(S - 1, S - 1);
    read(0, o0);
    int stage = 0;  // stage of entry k
    // Waits for entry k+1 and frees stage k % S (entry k's reads are this
    // wave's; the compiler would otherwise wait for them only at their first
    // use, after the barrier and the next issue).
    auto sync = [&](int k) {
        spmm_detail::wait_lgkm0();
        if (k <= n - S)
            wait_vmcnt<PER * (S - 2)>();         // entry k+1 landed
        else
            wait_stages<PER, S - 2>(n - 2 - k);  // the same, fewer in flight
        barrier_no_fence();
        if (k + S < n) issue(k + S, stage);
        stage = stage == S - 1 ? 0 : stage + 1;
    };
    // The same step while entry k+S exists: a fixed wait and an unconditional
    // issue, so the steady state carries no branches for the ring's tail
    // (scalar instructions are the per-entry cost of this loop).
    auto sync_full = [&](int k) {
        spmm_detail::wait_lgkm0();
        wait_vmcnt<PER * (S - 2)>();
        barrier_no_fence();
        issue(k + S, stage);
        stage = stage == S - 1 ? 0 : stage + 1;
    };
    int k = 0;
    // The scheduler would otherwise hoist the MFMAs above the LDS reads they
    // do not depend on; the reads must be in flight while the MFMAs run.
    auto fence_sched = [] { __builtin_amdgcn_sched_barrier(0); };
    if constexpr (OVERLAP) {
        auto fence_rm = [&] {
            if constexpr (!MIX) fence_sched();
        };
        Ops o1;
        for (; k + S + 1 < n; k += 2) {
            sync_full(k);
            read(stage, o1);
            fence_rm();
            multiply(o0);
            fence_sched();
            sync_full(k + 1);
            read(stage, o0);
            fence_rm();
            multiply(o1);
            fence_sched();
        }
        for (; k + 2 < n; k += 2) {
            sync(k);
            read(stage, o1);
            fence_rm();
            multiply(o0);
            fence_sched();
            sync(k + 1);
            read(stage, o0);
            fence_rm();
            multiply(o1);
            fence_sched();
        }
        if (k + 1 < n) {
            sync(k);
            read(stage, o1);
            fence_rm();
            multiply(o0);
            xchg();
            multiply(o1);
        } else {
            xchg();
            multiply(o0);
        }
    } else {
        for (; k + S < n; ++k) {
            multiply(o0);
            sync_full(k);
            read(stage, o0);
        }
        for (; k + 1 < n; ++k) {
            multiply(o0);
            sync(k);
            read(stage, o0);
        }
        multiply(o0);
    }
}

// The ring of run_ring (one operand set) with each entry's operands and
// products in two halves (the two 16-deep k-steps).  Step k:
//   1. half 0's products of entry k, interleaved with the LDS reads of entry
//      k's half 1 (into the registers half 1 released in the previous step);
//   2. sync: the reads complete, entry k+1 landed, barrier (stage k % S is
//      then free), entry k+S issued;
//   3. half 1's products of entry k, interleaved with the reads of entry
//      k+1's half 0.
// The reads go two after each of the first PAIRS/2 products (PAIRS products
// per half), so that the last of them lands before the next part's first
// product needs it, and no phase of a step is reads alone: the two waves of
// a SIMD, in step with each other through the barrier, would otherwise both
// read while the matrix core idles, then both multiply.  (256x256 blocks:
// reads before the products 281-290 us, one read per product 270-277, two
// per product over the first half 265-273.)  An entry issues PER loads per wave, an even entry EXTRA more (a
// load shared by an entry pair goes with its first entry).  read(k, stage,
// o, h) reads half h of entry k (in stage `stage`).
template <int S, int PER, int EXTRA, int PAIRS, class Ops, class Issue, class Read, class Multiply, class Landed>
__device__ __forceinline__ void run_ring_halves(int n, Issue&& issue, Read&& read, Multiply&& multiply,
                                                Landed&& landed) {
    // Loads issued for entries j+1 .. last (the even ones carry EXTRA more).
    auto after = [](int j, int last) { return (last - j) * PER + EXTRA * ((last >> 1) - (j >> 1)); };
    constexpr int MAXW = PER * (S - 2) + EXTRA * ((S - 1) / 2);
    static_assert(MAXW < 64, "vmcnt budget");
    if (n <= 0) return;
#pragma unroll
    for (int e = 0; e < S - 1; ++e)
        if (e < n) issue(e, e);
    Ops o;
    wait_stages<1, MAXW>(after(0, min(S - 2, n - 1)));  // entry 0 landed
    barrier_no_fence();
    landed();
    if (S - 1 < n) issue(S - 1, S - 1);
    read(0, 0, o, 0);
    int stage = 0;
    auto fence_sched = [] { __builtin_amdgcn_sched_barrier(0); };
    auto interleave = [] {
#pragma unroll
        for (int i = 0; i < PAIRS / 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two LDS reads
        }
        __builtin_amdgcn_sched_group_barrier(0x008, PAIRS - PAIRS / 2, 0);
    };
    auto step = [&](int k, bool full) {
        multiply(o, 0);
        read(k, stage, o, 1);
        interleave();
        fence_sched();
        spmm_detail::wait_lgkm0();
        // Entry k+1 landed: at most the loads of the entries after it are outstanding.
        if constexpr (EXTRA == 0 || S % 2 == 0) {
            if (full || k <= n - S)
                wait_vmcnt<PER * (S - 2) + EXTRA * ((S - 2) / 2)>();
            else
                wait_stages<1, MAXW>(after(k + 1, n - 1));
        } else {
            wait_stages<1, MAXW>(after(k + 1, min(k + S - 1, n - 1)));
        }
        barrier_no_fence();
        if (full || k + S < n) issue(k + S, stage);
        stage = stage == S - 1 ? 0 : stage + 1;
        multiply(o, 1);
        read(k + 1, stage, o, 0);
        interleave();
        fence_sched();
    };
    int k = 0;
    for (; k + S < n; ++k) step(k, true);
    for (; k + 1 < n; ++k) step(k, false);
    multiply(o, 0);
    read(k, stage, o, 1);
    interleave();
    fence_sched();
    multiply(o, 1);
}

// The entry words of a work item held in lanes: lane j has word 64c + j of
// the current chunk c (first row of B in the low 32 bits, A offset / 32 in
// the high).  They are loaded, and waited for, before the ring starts; an
// item of more than 64 entries reloads at each chunk boundary (inside the
// issue that crosses it) and waits there.  A scalar load per entry would put
// the scalar cache's latency on every step of the ring.
struct EntryWords {
    const int64_t* ents;
    int n;
    uint32_t lo = 0, hi = 0;
    __device__ __forceinline__ EntryWords(const int64_t* e, int n_, int lane) : ents(e), n(n_) { fetch(0, lane); }
    __device__ __forceinline__ void fetch(int base, int lane) {
        if (base + lane < n) {
            const int64_t w = ents[base + lane];
            lo = (uint32_t)w;
            hi = (uint32_t)((uint64_t)w >> 32);
        }
        __asm__ volatile("" : "+v"(lo), "+v"(hi));
    }
    // Words of entry e (e increasing from call to call).
    __device__ __forceinline__ void get(int e, int lane, uint32_t& b_word, uint32_t& a_word) {
        if ((e & 63) == 0 && e > 0) fetch(e, lane);
        b_word = __builtin_amdgcn_readlane(lo, e & 63);
        a_word = __builtin_amdgcn_readlane(hi, e & 63);
    }
};

// The 32 x TN slice of row-major B (rows brow..brow+31, columns n0..) in LDS:
// row k at k*2*TN bytes, its 16-byte chunk c at slot c ^ 4*(k % 4).  Each of
// the NW waves loads BI = 64 * TN / 1024 / NW pieces of 1 KB.
template <int NTW, int NW = 4>
struct BSlice {
    static constexpr int TN = 128 * NTW;
    static constexpr int ROW_BYTES = 2 * TN;
    static constexpr int BYTES = 32 * ROW_BYTES;
    static constexpr int BI = BYTES / 1024 / NW;
    uint32_t voff[BI];  // byte offsets of this lane's chunks from the slice's first row
                        // (32 rows of B span less than 4 GB: ldb < 2^26, checked by the host)

    __device__ __forceinline__ BSlice(int wave, int lane, int n0, int N, int64_t ldb) {
#pragma unroll
        for (int j = 0; j < BI; ++j) {
            const int byte = (wave * BI + j) * 1024 + lane * 16;
            const int r = byte / ROW_BYTES;
            const int slot = (byte % ROW_BYTES) / 16;
            // Columns past N (a partial last tile) read a valid chunk; they are not stored.
            const int col = min(n0 + 8 * (slot ^ (4 * (r & 3))), N - 8);
            voff[j] = (uint32_t)(2 * ((int64_t)r * ldb + col));
        }
    }
    __device__ __forceinline__ void issue(const uint16_t* b, int64_t ldb, uint32_t brow, uint32_t lds_wave) const {
        const uint16_t* bpan = b + (int64_t)brow * ldb;
#pragma unroll
        for (int j = 0; j < BI; ++j) gl_lds16_s(voff[j], bpan, lds_wave + j * 1024);
    }
};

// B operands of NT 32-column tiles (from column col0 of a TN-wide slice) by
// transpose reads.  The rows read for k-step s2, lane half q, 4-row group h
// are 16*s2 + 8*q + 4*h (the MFMA's own order) or, with permuted, 16*s2 +
// 8*h + 4*q (the order in which a 32x32 MFMA result holds its rows, for an A
// operand built from a result).
template <int TN, int NT>
struct BReads {
    int rd[2][2][NT];  // LDS offsets [k-step][4-row group][tile]

    __device__ __forceinline__ BReads(int lane, int col0, bool permuted) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int g = lane >> 4;
                    const int r = 16 * s2 + (permuted ? 8 * h + 4 * (g >> 1) : 8 * (g >> 1) + 4 * h) +
                                  ((lane & 15) >> 2);
                    const int col = col0 + nt * 32 + 16 * (g & 1) + 4 * (lane & 3);
                    const int c = col >> 3;
                    rd[s2][h][nt] = r * (2 * TN) + 16 * (c ^ (4 * (r & 3))) + 2 * (col & 7);
                }
    }
    __device__ __forceinline__ void read(const uint8_t* bs, u32x4 (&o)[2][NT]) const {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) read_half(bs, o, s2);
    }
    // The operands of k-step s2 only.
    __device__ __forceinline__ void read_half(const uint8_t* bs, u32x4 (&o)[2][NT], int s2) const {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const u32x4 lo = ld_tr_b16(bs + rd[s2][0][nt]);
            const u32x4 hi = ld_tr_b16(bs + rd[s2][1][nt]);
            o[s2][nt] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
    }
};

}  // namespace spmm_detail

// Ends a work item: a piece of a split row leaves its partial in scratch
// (spmm_reduce_kernel adds the pieces in order after this launch); a whole
// row stores its tile.
template <int NTW, bool OUT_BF16>
__device__ __forceinline__ void spmm_finish(const SpmmArgs& p, const SpmmWg& it, const f32x16 (&acc)[NTW], int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    if (it.slot >= 0) {
        constexpr int PF = NTW * 16 * 256;
        float* mine = p.ws + ((int64_t)it.slot * p.n_tiles + it.tile) * PF;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[(nt * 16 + v) * 256 + tid] = acc[nt][v];
        return;
    }
    spmm_store_tile<NTW, OUT_BF16>(p, acc, (int64_t)it.row * 32, it.tile * 128 * NTW, wave, lane & 31, lane >> 5);
}

template <int NTW, int S, bool OUT_BF16>
__global__ __launch_bounds__(256) void spmm_kernel(SpmmArgs p) {
    using namespace spmm_detail;
    using Slice = BSlice<NTW>;
    constexpr int PER = Slice::BI + 1;          // loads per wave per entry (B + a half-wave of A)
    constexpr int B_RING = S * kA_BYTES;         // A ring first, then the B ring
    __shared__ __attribute__((aligned(1024))) uint8_t smem[S * (kA_BYTES + Slice::BYTES)];

    const SpmmWg it = load_const(p.wgs + blockIdx.x);
    if (it.row < 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
    const int l32 = lane & 31, q = lane >> 5;
    const uint32_t lds0 = lds_address(smem);
    const Slice bsl(wave, lane, it.tile * Slice::TN, p.N, p.ldb);
    const BReads<Slice::TN, NTW> brd(lane, wave * NTW * 32, false);

    // Loads of one entry, per wave: lanes 0-31 fetch A segment `wave` (lane
    // 8*j + i loads A[8*wave + i][8*j .. +7]) and the wave's pieces of the B slice.
    const uint32_t a_voff = 2 * a_load_offset(wave, lane, p.lda);
    const uint32_t a_lds = lds0 + wave * 512;
    const uint32_t b_lds = lds0 + B_RING + wave * Slice::BI * 1024;
    // Entry words: low 32 bits = first row of B, high 32 bits = A offset / 32.
    EntryWords words(p.ents + it.e_begin, it.e_end - it.e_begin, lane);
    auto issue = [&](int e, int stage) {
        uint32_t bw, aw;
        words.get(e, lane, bw, aw);
        if (lane < 32) gl_lds16_s(a_voff, p.a + (int64_t)aw * 32, a_lds + stage * kA_BYTES);
        bsl.issue(p.b, p.ldb, bw, b_lds + stage * Slice::BYTES);
    };

    const int a_rd = a_read_offset(l32, q);  // + s * 256
    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    struct Operands {
        u32x4 a[2];
        u32x4 b[2][NTW];
    };
    run_ring<S, PER, true, Operands>(
        it.e_end - it.e_begin, issue,
        [&](int stage, Operands& o) {
            const uint8_t* as = smem + stage * kA_BYTES;
            o.a[0] = *(const u32x4*)(as + a_rd);
            o.a[1] = *(const u32x4*)(as + 256 + a_rd);
            brd.read(smem + B_RING + stage * Slice::BYTES, o.b);
        },
        [&](const Operands& o) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) acc[nt] = mfma32(o.a[s2], o.b[s2][nt], acc[nt]);
        },
        [] {});
    spmm_finish<NTW, OUT_BF16>(p, it, acc, tid);
}

// ---------------------------------------------------------------------------
// SpMM over row groups: a workgroup takes RW (2, 4 or 8) consecutive 32-row
// stripes of one block row (R >= 64) and one 128-column tile, so each entry's
// B panel is loaded once and multiplied by the RW stripes' A sub-blocks
// (which share the block row's column pattern).  The four waves form a WR x
// WC grid: wave (wr, wc) holds SR = RW/WR stripes x NT = 4/WC 32-column
// tiles.  A ring stage holds the entry's RW A sub-blocks (each in the layout
// of the single-stripe kernel, sub-block s at s*2 KB) and the B slice; the
// ring, B slice and epilogue are the single-stripe kernel's.
// Two waves per SIMD (two workgroups per compute unit): the register budget
// that keeps the 8-stripe accumulators of a wave (128 values) without spills.
template <int RW, int S, bool OUT_BF16>
__global__ __launch_bounds__(256, 2) void spmm_group_kernel(SpmmArgs p) {
    using namespace spmm_detail;
    using Slice = BSlice<1>;
    constexpr int WR = RW < 4 ? RW : 4;
    constexpr int WC = 4 / WR;
    constexpr int SR = RW / WR;
    constexpr int NT = 4 / WC;
    constexpr int A_BYTES = RW * kA_BYTES;
    constexpr int AI = RW / 2;  // A load instructions per wave (two 512-byte segments each)
    constexpr int PER = AI + Slice::BI;
    constexpr int B_RING = S * A_BYTES;
    static_assert(RW == 2 || RW == 4 || RW == 8, "row group");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[S * (A_BYTES + Slice::BYTES)];

    const SpmmWg it = load_const(p.wgs + blockIdx.x);
    if (it.row < 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, q = lane >> 5;
    const int wr = wave / WC, wc = wave % WC;
    const uint32_t lds0 = lds_address(smem);
    const Slice bsl(wave, lane, it.tile * Slice::TN, p.N, p.ldb);
    const BReads<Slice::TN, NT> brd(lane, wc * NT * 32, false);

    // A of one entry: 4*RW segments of 512 bytes (sub-block L/4, rows
    // 8*(L%4) .. +7); segment L lands at L*512, and wave w's load j covers
    // segments 2*(w*AI + j) and 2*(w*AI + j) + 1.
    uint32_t a_voff[AI];  // byte offsets from the group's first A sub-block
#pragma unroll
    for (int j = 0; j < AI; ++j) {
        const int L = 2 * (wave * AI + j) + (lane >> 5);
        a_voff[j] = 2 * ((L >> 2) * 32 * p.lda + a_load_offset(L & 3, lane, p.lda));
    }
    const uint32_t a_lds = lds0 + wave * AI * 1024;
    const uint32_t b_lds = lds0 + B_RING + wave * Slice::BI * 1024;
    // Entry words: first row of B | A offset of the group's first stripe / 32.
    EntryWords words(p.ents + it.e_begin, it.e_end - it.e_begin, lane);
    auto issue = [&](int e, int stage) {
        uint32_t bw, aw;
        words.get(e, lane, bw, aw);
        const uint16_t* ablk = p.a + (int64_t)aw * 32;
#pragma unroll
        for (int j = 0; j < AI; ++j) gl_lds16_s(a_voff[j], ablk, a_lds + stage * A_BYTES + j * 1024);
        bsl.issue(p.b, p.ldb, bw, b_lds + stage * Slice::BYTES);
    };

    const int a_rd = a_read_offset(l32, q);  // + s * 256 + sub-block * 2 KB
    f32x16 acc[SR][NT];
#pragma unroll
    for (int i = 0; i < SR; ++i)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][nt][v] = 0.0f;

    struct Operands {
        u32x4 a[SR][2];
        u32x4 b[2][NT];
    };
    run_ring<S, PER, (RW < 8), Operands>(
        it.e_end - it.e_begin, issue,
        [&](int stage, Operands& o) {
            const uint8_t* as = smem + stage * A_BYTES;
#pragma unroll
            for (int i = 0; i < SR; ++i) {
                o.a[i][0] = *(const u32x4*)(as + (wr * SR + i) * kA_BYTES + a_rd);
                o.a[i][1] = *(const u32x4*)(as + (wr * SR + i) * kA_BYTES + 256 + a_rd);
            }
            brd.read(smem + B_RING + stage * Slice::BYTES, o.b);
        },
        [&](const Operands& o) {
#pragma unroll
            for (int i = 0; i < SR; ++i)
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[i][nt] = mfma32(o.a[i][s2], o.b[s2][nt], acc[i][nt]);
        },
        [] {});

#pragma unroll
    for (int i = 0; i < SR; ++i) {
        const int st = wr * SR + i;  // stripe within the group
        if (it.slot >= 0) {
            // Piece of a split group: stripe st's partial goes to its own slot
            // in the single-stripe layout (tile c's column l at c*64 + l).
            const int slot = it.base + st * it.npieces + (it.slot - it.base);
            float* mine = p.ws + ((int64_t)slot * p.n_tiles + it.tile) * (16 * 256);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) mine[v * 256 + (wc * NT + nt) * 64 + lane] = acc[i][nt][v];
        } else {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                store_tile32<OUT_BF16>(p, acc[i][nt], (int64_t)(it.row + st) * 32,
                                       (int64_t)it.tile * Slice::TN + (wc * NT + nt) * 32 + l32, q);
        }
    }
}

// ---------------------------------------------------------------------------
// SpMM over RW-stripe row groups (RW = 2, 4 or 8: R = 64, 128 or 256) with a
// 256-column tile: a workgroup owns a 32*RW x 256 output tile, one workgroup
// per compute unit (two for RW = 2 and 4, on a 3-stage ring: 64 and 80 KB
// of LDS), with a deep ring (S stages of RW x 2 KB of A and 16 KB of B).  NW = 8 waves (two per SIMD) in a 2 x 4 grid each hold RW/2 stripes x 2
// 32-column tiles (128 accumulators per lane at RW = 8); NW = 4 waves (one
// per SIMD) in a 2 x 2 grid hold RW/2 x 4 (256 accumulators at RW = 8, the
// whole register file shared with the AGPRs), which reads fewer LDS bytes
// per product but leaves no second wave to hide a wave's waits behind:
// eight waves measure 6% faster.  Either way one operand set per wave, read
// in halves under the other half's products (run_ring_halves).  Ring, B
// slice and entry words are the single-stripe kernel's; split pieces leave
// their partials in the 256-column single-stripe layout (tile t's column l
// at the slot's ((t % 2) * 16 + v) * 256 + (t / 2) * 64 + l), which
// spmm_reduce_kernel<2> adds.
template <int RW, int S, bool OUT_BF16, int NW, bool PAIR>
__global__ __launch_bounds__(64 * NW, RW <= 4 && S == 3 ? 2 : 1) void spmm_group_wide_kernel(SpmmArgs p) {
    using namespace spmm_detail;
    static_assert(NW == 4 || NW == 8, "waves");
    static_assert(RW == 2 || RW == 4 || RW == 8, "row group");
    using Slice = BSlice<2, NW>;
    constexpr int SR = RW / 2;   // stripes per wave
    constexpr int WC = NW / 2;   // wave grid 2 x WC
    constexpr int NT = 8 / WC;   // 32-column tiles per wave
    constexpr int A_BYTES = RW * kA_BYTES;  // A of one entry (RW sub-blocks)
    constexpr int A_KB = A_BYTES / 1024;    // its 1 KB loads
    // Without pairs and with fewer loads than waves (RW = 2, eight waves),
    // each wave loads one 512-byte segment with lanes 0-31.
    constexpr bool HALF = !PAIR && A_KB < NW;
    constexpr int NP = S / 2 + 1;           // pair slots (the pairs of entries k .. k+S-1, and one being filled)
    constexpr int A_RING = PAIR ? NP * 2 * A_BYTES : S * A_BYTES;
    // A loads per wave and issue (an even entry's, for a pair).
    constexpr int AL = PAIR ? 2 * A_KB / NW : (HALF ? 1 : A_KB / NW);
    static_assert(AL >= 1 && (PAIR ? AL * NW == 2 * A_KB : (HALF ? NW == 4 * RW : AL * NW == A_KB)), "A loads");
    constexpr int PER = PAIR ? Slice::BI : AL + Slice::BI;
    constexpr int EXTRA = PAIR ? AL : 0;
    constexpr int B_RING = A_RING;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[A_RING + S * Slice::BYTES];

    const SpmmWg it = load_const(p.wgs + blockIdx.x);
    if (it.row < 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, q = lane >> 5;
    const int wr = wave / WC, wc = wave % WC;
    const uint32_t lds0 = lds_address(smem);
    const Slice bsl(wave, lane, it.tile * Slice::TN, p.N, p.ldb);
    const BReads<Slice::TN, NT> brd(lane, wc * NT * 32, false);

    // A without pairs: of one entry, 4*RW segments of 512 bytes (sub-block
    // L/4, rows 8*(L%4) .. +7); segment L lands at L*512, and wave w's load j
    // covers segments 2*(w*AL + j) and 2*(w*AL + j) + 1 (HALF: segment w).
    // A with pairs (C a multiple of 64: entries 2m and 2m+1 of an item are the
    // two 32-column halves of the same 64 columns of one block): an even
    // entry fetches both, 32*RW rows of 128 bytes, so that every request is a
    // whole 128-byte line (a 64-byte half-line request costs the L1 as much
    // as a whole line: a DMA-only copy of the loop on 256x256 blocks took
    // 189 us without pairs, 161 us with).  Load I (0 .. 4*RW-1) holds rows
    // 8I .. 8I+7 of the group, row r of them at I*1024 + (r%8)*128 with its
    // 16-byte chunk c at position c ^ ((r%8)/2 + 4*(I%2)): each 16-lane
    // quarter of a read then covers every bank.  Pair m sits in slot m % NP.
    uint32_t a_voff[AL];
#pragma unroll
    for (int j = 0; j < AL; ++j) {
        if constexpr (PAIR) {
            const int I = wave * AL + j, r = lane >> 3;
            const int c = (lane & 7) ^ ((r >> 1) | ((I & 1) << 2));
            a_voff[j] = 2 * ((8 * I + r) * p.lda + 8 * c);
        } else {
            const int L = HALF ? wave : 2 * (wave * AL + j) + (lane >> 5);
            a_voff[j] = 2 * ((L >> 2) * 32 * p.lda + a_load_offset(L & 3, lane, p.lda));
        }
    }
    const uint32_t a_lds = lds0 + wave * (HALF ? 512 : AL * 1024);
    const uint32_t b_lds = lds0 + B_RING + wave * Slice::BI * 1024;
    EntryWords words(p.ents + it.e_begin, it.e_end - it.e_begin, lane);
    // (An operand left out by the instrumented build is read, for every
    // entry, where the item's first entry reads it -- an L2 hit after the
    // first, a different line per workgroup: the waits count both operands'
    // loads, so the loads stay.)
    uint32_t bw_first = 0, aw_first = 0;
    if (BSP_SKIP(p, kSkipSparseRead | kSkipDenseRead)) words.get(0, lane, bw_first, aw_first);
    auto issue = [&](int e, int stage) {
        uint32_t bw, aw;
        words.get(e, lane, bw, aw);
        // Both operands left out: no loads at all (the waits then pass at once).
        if (BSP_SKIP(p, kSkipSparseRead) && BSP_SKIP(p, kSkipDenseRead)) return;
        if (BSP_SKIP(p, kSkipSparseRead)) aw = aw_first;
        if (BSP_SKIP(p, kSkipDenseRead)) bw = bw_first;
        const uint16_t* ablk = p.a + (int64_t)aw * 32;
        if constexpr (PAIR) {
            if ((e & 1) == 0) {
                const uint32_t slot = a_lds + ((e >> 1) % NP) * (2 * A_BYTES);
#pragma unroll
                for (int j = 0; j < AL; ++j) gl_lds16_s(a_voff[j], ablk, slot + j * 1024);
            }
        } else {
#pragma unroll
            for (int j = 0; j < AL; ++j)
                if (!HALF || lane < 32) gl_lds16_s(a_voff[j], ablk, a_lds + stage * A_BYTES + j * 1024);
        }
        bsl.issue(p.b, p.ldb, bw, b_lds + stage * Slice::BYTES);
    };

    const int a_rd = a_read_offset(l32, q);  // + s * 256 + sub-block * 2 KB
    // With pairs, lane (l32, q)'s A operand of k-step s of the pair's half
    // ph: row l32 of the stripe (load 4*stripe + l32/8, row r = l32%8),
    // chunk 4*ph + 2*s + q, at position chunk ^ (r/2 + 4*((l32/8)%2)); half
    // ph = 1 flips bit 2 of the position (byte offset bit 6).
    int a_rdp[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        const int r = l32 & 7;
        const int c = (2 * s2 + q) ^ ((r >> 1) | (((l32 >> 3) & 1) << 2));
        a_rdp[s2] = (l32 >> 3) * 1024 + r * 128 + c * 16;
    }
    f32x16 acc[SR][NT];
#pragma unroll
    for (int i = 0; i < SR; ++i)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][nt][v] = 0.0f;

    struct Operands {
        u32x4 a[SR][2];
        u32x4 b[2][NT];
    };
    auto read_half = [&](int k, int stage, Operands& o, int h) {
        if constexpr (PAIR) {
            const uint8_t* as = smem + ((k >> 1) % NP) * (2 * A_BYTES);
            const int off = a_rdp[h] ^ ((k & 1) << 6);
#pragma unroll
            for (int i = 0; i < SR; ++i) o.a[i][h] = *(const u32x4*)(as + (wr * SR + i) * 4096 + off);
        } else {
            const uint8_t* as = smem + stage * A_BYTES;
#pragma unroll
            for (int i = 0; i < SR; ++i) o.a[i][h] = *(const u32x4*)(as + (wr * SR + i) * kA_BYTES + 256 * h + a_rd);
        }
        brd.read_half(smem + B_RING + stage * Slice::BYTES, o.b, h);
    };
    auto mul_half = [&](const Operands& o, int h) {
        if (BSP_SKIP(p, kSkipCompute)) return;
#pragma unroll
        for (int i = 0; i < SR; ++i)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) acc[i][nt] = mfma32(o.a[i][h], o.b[h][nt], acc[i][nt]);
    };
    run_ring_halves<S, PER, EXTRA, SR * NT, Operands>(it.e_end - it.e_begin, issue, read_half, mul_half, [] {});

    if (BSP_SKIP(p, kSkipWrite)) return;
#pragma unroll
    for (int i = 0; i < SR; ++i) {
        const int st = wr * SR + i;  // stripe within the group
        if (it.slot >= 0) {
            const int slot = it.base + st * it.npieces + (it.slot - it.base);
            float* mine = p.ws + ((int64_t)slot * p.n_tiles + it.tile) * (2 * 16 * 256);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int t = wc * NT + nt;  // 32-column tile within the 256
#pragma unroll
                for (int v = 0; v < 16; ++v) mine[((t & 1) * 16 + v) * 256 + (t >> 1) * 64 + lane] = acc[i][nt][v];
            }
        } else {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                store_tile32<OUT_BF16>(p, acc[i][nt], (int64_t)(it.row + st) * 32,
                                       (int64_t)it.tile * Slice::TN + (wc * NT + nt) * 32 + l32, q);
        }
    }
}

// ---------------------------------------------------------------------------
// Persistent SpMM with specialised waves.  A workgroup owns a list of units
// (one 32-row stripe x one tile of TN = 128*NTW columns) and streams the
// entries of all of them, back to back, through two LDS rings: an A ring of SA
// stages (2 KB each) and a B ring of SB stages (the 32 x TN slice of B).
//   - waves 0-3 (MFMA waves) read the operands from LDS, multiply, and store
//     each unit's tile when its last entry is done; they issue no loads, so
//     their stores never sit in front of a load in a wave's queue;
//   - waves 4 .. 4+NBW-1 (B loaders) issue the B slice of each entry;
//   - wave 4+NBW (A loader) issues the entry's A sub-block.
// With stripe pairs (SR = 2) a unit is two stripes that share block columns
// and an entry is one block column of their union: one B slice serves both
// stripes.  The A stage holds both stripes' sub-blocks, waves 0-3 work for the
// first stripe and waves 4-7 for the second (the loaders follow them), and a
// wave whose stripe has no block in the entry's column skips its products.
// A sub-blocks mostly miss to HBM while B slices mostly hit in L2.  A wave's
// loads return in order, so an A miss at the head of a wave's queue holds back
// the B hits behind it: with the two in separate waves, a 2 MB L2-resident
// stream mixed with 1/5 (1/9) of its bytes from HBM measured 19.2 (21.3) TB/s
// against 15.8 (15.6) with every wave loading both (same byte counts).
// The ring never drains between units, so a unit's store and the next unit's
// first loads overlap, and only the first entry of the whole stream waits
// for a cold fetch.
// Step k (one barrier X_k): loaders wait until entry k has landed, barrier,
// then refill the stage of entry k-1 with entry k+S-1; the MFMA waves read
// entry k's operands (into the set not in use) and multiply entry k-1, then
// wait for their LDS reads (the stage of entry k is refilled after X_{k+1}).
// Every wave executes the same n barriers.  With two entries per step the
// same holds per pair: ceil(n/2) barriers, the stages of entries k-2 and k-1
// refilled after step k (stream_loader2).
namespace spmm_detail {

// The B slice pieces (1 KB each) of B loader wave wb: piece p = wb*BI + j of
// the 32 x TN slice in the layout of BSlice; the byte offsets are relative to
// (first row, first column) of the slice, which the entry word supplies.
template <int TN, int NBW>
struct BSliceLoader {
    static constexpr int ROW_BYTES = 2 * TN;
    static constexpr int BYTES = 32 * ROW_BYTES;
    static constexpr int BI = BYTES / 1024 / NBW;
    static_assert(BI * NBW * 1024 == BYTES, "B pieces per loader wave");
    uint32_t voff[BI];
    __device__ __forceinline__ BSliceLoader(int wb, int lane, int64_t ldb) {
#pragma unroll
        for (int j = 0; j < BI; ++j) {
            const int byte = (wb * BI + j) * 1024 + lane * 16;
            const int r = byte / ROW_BYTES;
            const int slot = (byte % ROW_BYTES) / 16;
            voff[j] = (uint32_t)(2 * ((int64_t)r * ldb + 8 * (slot ^ (4 * (r & 3)))));
        }
    }
    // Issues pieces J .. BI-1 of the slice at bpan into LDS at dst + 1 KB per piece.
    template <int J = 0>
    __device__ __forceinline__ void issue(const uint16_t* bpan, uint32_t dst) const {
        if constexpr (J < BI) {
            gl_lds16_si<J * 1024>(voff[J], bpan, dst);
            issue<J + 1>(bpan, dst);
        }
    }
};

// First element of an entry's B slice: row (low 32 bits of the word) times
// ldb plus the column (bits 32 .. 32+CB-1).  ldb < 2^26 (checked by the host),
// so the product is one 32 x 32-bit multiply with a 64-bit result.
template <int CB = 32>
__device__ __forceinline__ const uint16_t* b_slice(const uint16_t* b, int64_t ldb, int64_t w) {
    const uint32_t col = CB == 32 ? (uint32_t)((uint64_t)w >> 32) : (uint32_t)((uint64_t)w >> 32) & ((1u << CB) - 1u);
    return b + ((uint64_t)(uint32_t)w * (uint32_t)ldb + col);
}

// One loader wave's side of the ring: issue(e, word) issues entry e's loads
// (P per wave) into stage e % S; the wave takes part in the n barriers.  The
// entry words come from plan memory through scalar loads, eight at a time and
// two chunks ahead of use (a scalar-cache miss on the step that needs the
// word would otherwise stall the issue on every eighth entry).  The first two
// chunks come from the workgroup's head (`head`, loaded with its record), the
// rest from the stream (`words`).  The word arrays are padded past every
// stream's end, so the chunks ahead need no bounds test.
template <int S, int P, typename WT, class Issue>
__device__ __forceinline__ void stream_loader(int n, const WT* head, const WT* words, Issue&& issue) {
    static_assert(P * (S - 2) < 64, "vmcnt budget");
    static_assert(S - 1 <= 16 && kHeadWords == 16, "the prologue takes its words from the head's two chunks");
    struct W8 {
        WT w[8];
    };
    const W8* hc = (const W8*)head;
    const W8* ch = (const W8*)words;
    {
        const W8 c0 = load_const(hc), c1 = load_const(hc + 1);
#pragma unroll
        for (int e = 0; e < S - 1; ++e)
            if (e < n) issue(e, e < 8 ? c0.w[e] : c1.w[e - 8]);
    }
    // Steps 8m .. 8m+7 issue entries 8m+S-1 .. 8m+S+6: chunks m+OFF and m+OFF+1.
    constexpr int OFF = (S - 1) / 8, R0 = (S - 1) % 8;
    W8 ca = load_const((OFF < 2 ? hc : ch) + OFF), cb = load_const((OFF + 1 < 2 ? hc : ch) + OFF + 1);
    for (int k0 = 0; k0 < n; k0 += 8) {
        const W8 cc = load_const(ch + k0 / 8 + OFF + 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = k0 + j;
            if (k >= n) break;
            if (k + S - 1 < n) {
                wait_vmcnt<P * (S - 2)>();  // entry k landed (entries k+1 .. k+S-2 may be in flight)
                barrier_no_fence();
                issue(k + S - 1, R0 + j < 8 ? ca.w[R0 + j] : cb.w[R0 + j - 8]);
            } else {
                wait_stages<P, S - 2>(n - 1 - k);
                barrier_no_fence();
            }
        }
        ca = cb;
        cb = cc;
    }
}

// The same with two entries per step (S even): step k (k = 0, 2, 4, ...)
// waits until entries k and k+1 have landed, passes one barrier, then refills
// the stages of entries k-2 and k-1 (read by the MFMA waves during step k-2)
// with entries k+S-2 and k+S-1.  The prologue fills all S stages; ceil(n/2)
// barriers in all.
template <int S, int P, typename WT, class Issue>
__device__ __forceinline__ void stream_loader2(int n, const WT* head, const WT* words, Issue&& issue) {
    static_assert(S % 2 == 0 && S >= 4, "two entries per step need an even ring of at least 4 stages");
    static_assert(S <= 16 && kHeadWords == 16, "the prologue takes its words from the head's two chunks");
    static_assert(P * (S - 2) < 64, "vmcnt budget");
    struct W8 {
        WT w[8];
    };
    const W8* hc = (const W8*)head;
    const W8* ch = (const W8*)words;
    {
        const W8 c0 = load_const(hc), c1 = load_const(hc + 1);
#pragma unroll
        for (int e = 0; e < S; ++e)
            if (e < n) issue(e, e < 8 ? c0.w[e] : c1.w[e - 8]);
    }
    if (n <= 0) return;
    wait_stages<P, S - 2>(max(0, min(S, n) - 2));  // entries 0 and 1 landed
    barrier_no_fence();
    // Steps s0+2 .. s0+8 issue entries s0+S .. s0+S+7: positions R0 .. R0+7 of
    // chunks s0/8+OFF and s0/8+OFF+1 (R0 even, so a pair never straddles them).
    constexpr int OFF = S / 8, R0 = S % 8;
    W8 ca = load_const((OFF < 2 ? hc : ch) + OFF), cb = load_const((OFF + 1 < 2 ? hc : ch) + OFF + 1);
    for (int s0 = 0; s0 + 2 < n; s0 += 8) {
        const W8 cc = load_const(ch + s0 / 8 + OFF + 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = s0 + 2 + 2 * i;  // the step's first entry
            if (k >= n) break;
            const int e = k + S - 2, r = R0 + 2 * i;
            if (e + 1 < n) {
                wait_vmcnt<P * (S - 4)>();  // entries k, k+1 landed (k+2 .. k+S-3 may be in flight)
                barrier_no_fence();
                issue(e, r < 8 ? ca.w[r] : cb.w[r - 8]);
                issue(e + 1, r + 1 < 8 ? ca.w[r + 1] : cb.w[r + 1 - 8]);
            } else {
                wait_stages<P, S - 4>(max(0, min(n, e) - (k + 2)));
                barrier_no_fence();
                if (e < n) issue(e, r < 8 ? ca.w[r] : cb.w[r - 8]);
            }
        }
        ca = cb;
        cb = cc;
    }
}

}  // namespace spmm_detail

// With PIPES = 2, one workgroup holds two such pipelines (each with its own
// rings, MFMA waves and loaders) that share the per-entry barrier and split
// their compute unit's entry stream in half: the unit that straddles the
// half is accumulated by both, the second pipeline leaves its part in an LDS
// exchange buffer (unit flag 1) and the first adds it before storing (flag 2)
// after one last barrier.  Two independent workgroups per compute unit hold
// one unit each, and the one with the longer row finishes alone at the rate
// of a single workgroup's loaders; the halves end together.
// With EPS = 2 (one pipeline) every step covers two entries: one barrier per
// pair, the MFMA waves reading both entries of a step into one register set
// while multiplying the previous pair from the other (stream_loader2).
template <int NTW, int SB, int SA, int NBW, int PIPES, bool OUT_BF16, int EPS, int SR>
__global__ __launch_bounds__(64 * (4 * SR + 1 + NBW) * PIPES) void spmm_stream_kernel(SpmmStreamArgs p) {
    using namespace spmm_detail;
    static_assert(EPS == 1 || (EPS == 2 && PIPES == 1), "two entries per step with one pipeline");
    static_assert(SR == 1 || (SR == 2 && EPS == 2), "stripe pairs run two entries per step");
    constexpr int TN = 128 * NTW;
    using Loader = BSliceLoader<TN, NBW>;
    constexpr int A_STAGE = SR * kA_BYTES;  // one A sub-block per stripe of the unit
    constexpr int A_RING = SA * A_STAGE;
    // Stripe pairs: the entry's 8-byte A word per A stage (a half equal to
    // kNoBlock: that stripe has no block in the entry's column), after the
    // rings.
    constexpr int FLAGS = A_RING + SB * Loader::BYTES;
    constexpr int PIPE_LDS = FLAGS + (SR > 1 ? 8 * SA : 0);
    constexpr int MW = 4 * SR;                                   // MFMA waves: four per stripe of a unit
    constexpr int WPP = MW + 1 + NBW;                            // waves per pipeline
    constexpr int XCHG = PIPES > 1 ? 4 * NTW * 16 * 64 * 4 : 0;  // fp32 tile of the shared unit
    static_assert(PIPES == 1 || PIPES == 2, "pipelines");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[PIPES * PIPE_LDS + XCHG];
    BSP_TL_DECL_GLOBAL();

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pipe = PIPES > 1 ? wave_id / WPP : 0;
    const int wave = wave_id - pipe * WPP;  // role within the pipeline
    const SpmmStreamHead* head = p.heads + blockIdx.x * PIPES + pipe;
    const SpmmStreamWg wg = load_const(&head->wg);
    const int n = wg.n;
    // Barriers every wave takes: the longer pipeline's steps (+1 to close the exchange).
    int steps = n;
    if constexpr (PIPES > 1) {
        const SpmmStreamWg w0 = load_const(&p.heads[blockIdx.x * PIPES].wg);
        const SpmmStreamWg w1 = load_const(&p.heads[blockIdx.x * PIPES + 1].wg);
        steps = max(w0.n, w1.n);
    }
    uint8_t* psmem = smem + pipe * PIPE_LDS;
    float* xchg = (float*)(smem + PIPES * PIPE_LDS);
    const uint32_t lds0 = lds_address(psmem);
    auto idle_steps = [&] {
        for (int k = n; k < steps; ++k) barrier_no_fence();
        if constexpr (PIPES > 1) barrier_no_fence();
    };

    if (wave == MW + NBW) {
        // A loader: load j (1 KB) covers rows 16j .. 16j+15 of the 32x32
        // sub-block, in the row layout of a_row_load_offset.
        uint32_t a_voff[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) a_voff[j] = 2 * a_row_load_offset(j, lane, p.lda);
        if constexpr (SR == 2) {
            // Stripe pairs: both halves of the stage; a half whose stripe has no
            // block here gets two 16-byte loads by lane 0 (from the other
            // half's sub-block, into its own stale slot), so that every entry
            // issues the same five loads and the vmcnt waits keep their counts.
            // The fifth brings the entry's A word into the stage's word slot
            // (lanes 0 and 1, 4 bytes each) through the same DMA path, so the
            // loader's wait for the entry covers it too.
            const void* words = p.apw + wg.w_begin;
            // (A left out by the instrumented build: every entry's loads read
            // the A sub-blocks of the workgroup's first entry, an L2 hit after
            // the first, so that the wave's five loads per entry stay.)
            uint64_t apw_first = 0;
            if (BSP_SKIP(p, kSkipSparseRead)) apw_first = load_const(&head->apw[0]);
            auto issue_pair = [&](int e, uint64_t w) {
                const uint32_t st = (uint32_t)(e % SA);
                const uint64_t wa = BSP_SKIP(p, kSkipSparseRead) ? apw_first : w;
                const uint32_t w0 = (uint32_t)wa, w1 = (uint32_t)(wa >> 32);
                const uint32_t any = w0 != kNoBlock ? w0 : w1;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t wh = h == 0 ? w0 : w1;
                    const bool here = wh != kNoBlock;
                    const uint16_t* ablk = p.a + (int64_t)(here ? wh : any) * 32;
                    const uint32_t dst = lds0 + st * A_STAGE + h * kA_BYTES;
                    if (here || lane == 0) {
                        gl_lds16_s(a_voff[0], ablk, dst);
                        gl_lds16_s(a_voff[1], ablk, dst + 1024);
                    }
                }
                if (lane < 2) gl_lds4_s((uint32_t)e * 8 + lane * 4, words, lds0 + FLAGS + st * 8);
            };
            stream_loader2<SA, 5>(n, head->apw, p.apw + wg.w_begin, issue_pair);
            idle_steps();
            return;
        }
        auto issue_a = [&](int e, uint32_t w) {
            if (BSP_SKIP(p, kSkipSparseRead)) return;  // left out: the wave's waits pass at once
            const uint16_t* ablk = p.a + (uint64_t)w * 32;
            const uint32_t dst = lds0 + (uint32_t)(e % SA) * A_STAGE;
            gl_lds16_si<0>(a_voff[0], ablk, dst);
            gl_lds16_si<1024>(a_voff[1], ablk, dst);
        };
        if constexpr (EPS == 2)
            stream_loader2<SA, 2>(n, head->aw, p.aw + wg.w_begin, issue_a);
        else
            stream_loader<SA, 2>(n, head->aw, p.aw + wg.w_begin, issue_a);
        idle_steps();
        return;
    }
    if (wave >= MW) {
        const int wb = wave - MW;
        const Loader ld(wb, lane, p.ldb);
        const uint32_t b_lds = lds0 + A_RING + wb * Loader::BI * 1024;
        auto issue_b = [&](int e, int64_t w) {
            if (BSP_SKIP(p, kSkipDenseRead)) return;  // left out: the wave's waits pass at once
            ld.issue(b_slice(p.b, p.ldb, w), b_lds + (uint32_t)(e % SB) * Loader::BYTES);
        };
        if constexpr (EPS == 2)
            stream_loader2<SB, Loader::BI>(n, head->bw, p.bw + wg.w_begin, issue_b);
        else
            stream_loader<SB, Loader::BI>(n, head->bw, p.bw + wg.w_begin, issue_b);
        idle_steps();
        return;
    }

    // MFMA waves: wave w owns stripe w/4 of the unit (the first stripe, or
    // with stripe pairs the second) and columns (w%4)*NTW*32 .. of its tile.
    const int l32 = lane & 31, q = lane >> 5;
    const int half = wave >> 2, wc = wave & 3;
    const BReads<TN, NTW> brd(lane, wc * NTW * 32, false);
    const int a_rd0 = a_row_read_offset(l32, q, 0) + half * kA_BYTES;
    const int a_rd1 = a_row_read_offset(l32, q, 1) + half * kA_BYTES;
    f32x16 acc[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    // Unit walk: `cur` is the unit being accumulated, `left` its entries not
    // yet multiplied, `nxt` the record after it, loaded ahead.  Units with no
    // entries are stored as zeros on the way.  (The unit array is padded: the
    // records ahead are valid reads even past the last unit.)
    const SpmmStreamUnit* units = p.units + wg.u_begin;
    int u = 0;
    SpmmStreamUnit cur = load_const(&head->u[0]);  // = units[0], units[1]
    SpmmStreamUnit nxt = load_const(&head->u[1]);
    SpmmStreamUnit held{};  // the shared unit, stored after the exchange (flag 2)
    bool holding = false;
    // Stores this wave's part of the unit's tile (with stripe pairs, of its
    // stripe; the second stripe of an odd one out is -1).
    auto store_unit = [&](const SpmmStreamUnit& un) {
        if (BSP_SKIP(p, kSkipWrite)) return;
        const int32_t stripe = half == 0 ? un.row : un.aux;
        if (SR > 1 && stripe < 0) return;
        const int64_t row0 = (int64_t)stripe * 32;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const int64_t col = un.n0 + wc * (NTW * 32) + nt * 32 + l32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = row0 + 8 * (v >> 2) + 4 * q + (v & 3);
                if (OUT_BF16)
                    store_out(&((uint16_t*)p.c)[row * p.ldc + col], f32_to_bf16_rne(acc[nt][v]));
                else
                    store_out(&((float*)p.c)[row * p.ldc + col], acc[nt][v]);
            }
        }
    };
    auto xchg_at = [&](int nt, int v) { return xchg + ((wave * NTW + nt) * 16 + v) * 64 + lane; };
    auto zero_acc = [&] {
#pragma unroll
        for (int i = 0; i < NTW; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;
    };
    // Ends unit `cur`: store it, or (two pipelines) leave it in the exchange
    // buffer, or hold it for the exchange.
    auto finish_cur = [&] {
        BSP_TL_MARK(2 + min(u, 60));
        if (PIPES > 1 && cur.aux == 1) {
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) *xchg_at(nt, v) = acc[nt][v];
            zero_acc();
        } else if (PIPES > 1 && cur.aux == 2) {
            held = cur;
            holding = true;
        } else {
            store_unit(cur);
            zero_acc();
        }
    };
    // Moves to the next unit with entries, storing (zero) tiles of empty ones.
    auto next_unit = [&] {
        ++u;
        while (u < wg.n_units) {
            cur = nxt;
            nxt = load_const(units + u + 1);
            if (cur.count > 0) return cur.count;
            store_unit(cur);
            ++u;
        }
        return 0;
    };
    int left = 0;
    if (wg.n_units > 0) {
        if (cur.count > 0) {
            left = cur.count;
        } else {
            store_unit(cur);
            left = next_unit();
        }
    }

    struct Operands {
        u32x4 a[2];
        u32x4 b[2][NTW];
        uint32_t w;  // stripe pairs: this wave's stripe's half of the entry's A word
    };
    auto read = [&](int k, Operands& o) {
        const uint8_t* as = psmem + (k % SA) * A_STAGE;
        o.a[0] = *(const u32x4*)(as + a_rd0);
        o.a[1] = *(const u32x4*)(as + a_rd1);
        if constexpr (SR > 1) o.w = *(const uint32_t*)(psmem + FLAGS + (k % SA) * 8 + half * 4);
        brd.read(psmem + A_RING + (k % SB) * Loader::BYTES, o.b);
    };
    auto multiply = [&](const Operands& o) {
        // With stripe pairs, a wave whose stripe has no block in the entry's
        // column skips its products (the word was read in an earlier step).
        if (!BSP_SKIP(p, kSkipCompute) && (SR == 1 || __builtin_amdgcn_readfirstlane(o.w) != kNoBlock)) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt) acc[nt] = mfma32(o.a[s2], o.b[s2][nt], acc[nt]);
        }
        if (--left == 0) {
            finish_cur();
            left = next_unit();
        }
    };
    auto fence_sched = [] { __builtin_amdgcn_sched_barrier(0); };
    auto lds_done = [] { wait_lgkm0(); };
    if constexpr (EPS == 2) {
        struct Pair {
            Operands e0, e1;
        };
        Pair pa, pb;
        if (n > 0) {
            barrier_no_fence();  // step 0
            BSP_TL_MARK(1);
            read(0, pa.e0);
            if (1 < n) read(1, pa.e1);
            lds_done();
        }
        // Step k: read entries k and k+1 into `in`, multiply entries k-2 and
        // k-1 (both exist, as k < n) from `out`.
        auto step2 = [&](int k, Pair& in, Pair& out) {
            barrier_no_fence();
            read(k, in.e0);
            if (k + 1 < n) read(k + 1, in.e1);
            fence_sched();
            multiply(out.e0);
            multiply(out.e1);
            fence_sched();
            lds_done();
        };
        int k = 2;
        for (; k + 2 < n; k += 4) {
            step2(k, pb, pa);
            step2(k + 2, pa, pb);
        }
        if (k < n) {
            step2(k, pb, pa);
            multiply(pb.e0);
            if (k + 1 < n) multiply(pb.e1);
        } else if (n > 0) {
            multiply(pa.e0);  // entries k-2 and, if it exists, k-1
            if (k - 1 < n) multiply(pa.e1);
        }
        if (wave_id == 0) BSP_TL_FLUSH();
        return;
    }
    Operands o0, o1;
    int k = 0;
    if (n > 0) {
        barrier_no_fence();  // X_0
        BSP_TL_MARK(1);
        read(0, o0);
        lds_done();
        k = 1;
    }
    // Steps k (odd) and k+1: reads into o1 then o0.
    for (; k + 1 < n; k += 2) {
        barrier_no_fence();
        read(k, o1);
        fence_sched();
        multiply(o0);
        fence_sched();
        lds_done();
        barrier_no_fence();
        read(k + 1, o0);
        fence_sched();
        multiply(o1);
        fence_sched();
        lds_done();
    }
    if (k < n) {
        barrier_no_fence();
        read(k, o1);
        fence_sched();
        multiply(o0);
        lds_done();
        multiply(o1);
    } else if (n > 0) {
        multiply(o0);
    }
    if constexpr (PIPES > 1) {
        lds_done();  // exchange writes complete before the closing barrier
        for (int s = n; s < steps; ++s) barrier_no_fence();
        barrier_no_fence();
        if (holding) {
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[nt][v] += *xchg_at(nt, v);
            store_unit(held);
        }
    }
    if (wave_id == 0) BSP_TL_FLUSH();
}

// ---------------------------------------------------------------------------
// Sweep SpMM: one workgroup per compute unit holds the accumulators of every
// unit of a sweep (up to 16 units of one 32-row stripe x 128 columns) and
// streams their entries merged in ascending first row of B, so that all
// workgroups of an XCD walk K together: a 32-row slice of B is fetched from
// HBM by the first unit that needs it and served from the XCD's L2 to the
// others shortly after, where a unit-by-unit walk spreads a slice's uses over
// the whole launch and the A and C streams evict it in between.
//   - waves 0-7 (MFMA waves), two groups of four: group g owns slots
//     8g .. 8g+7 and wave 4g + w columns 32w .. 32w+31 of each of them, 8 x 16
//     fp32 accumulator registers per lane; they issue no loads;
//   - wave 8 (A loader) and waves 9 .. 8+NBW (B loaders) run the persistent
//     kernel's ring (stream_loader2: two entries per barrier, entry words by
//     scalar loads two chunks ahead) over the workgroup's merged stream;
//   - the MFMA waves read the same stream's B words by scalar loads (a
//     step's two, one step ahead, in the scalar cache after the loaders'
//     reads): the slot (bits 56-58 within the group) picks the accumulator,
//     the skip bit (60) marks a padding entry (loaded, never multiplied);
//   - right after the products of a unit's last entry (the last bit of its
//     word, bit 61) the waves of its group store their columns of its tile,
//     so that the output streams out while the walk goes on instead of in
//     one burst at its end; units without entries are stored as zeros when
//     their sweep opens, and the accumulators are cleared between sweeps.
// A step reads and multiplies this group's entries among its two one after
// the other, into one operand set (the 128 accumulators leave no registers
// for a second); the plan gives the two groups alternate units, longest
// first, so that their entry counts are alike.
template <int SB, int SA, int NBW, bool OUT_BF16>
__global__ __launch_bounds__(64 * (8 + 1 + NBW), 1) void spmm_sweep_kernel(SpmmSweepArgs p) {
    using namespace spmm_detail;
    static_assert(SB % 2 == 0 && SA % 2 == 0 && SB <= 16 && SA <= 16, "two entries per step");
    constexpr int TN = kSweepTile;
    using Loader = BSliceLoader<TN, NBW>;
    constexpr int A_RING = SA * kA_BYTES;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[A_RING + SB * Loader::BYTES];
    BSP_TL_DECL_GLOBAL();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const SpmmSweepHead* head = p.heads + blockIdx.x;
    const SpmmSweepWg wg = load_const(&head->wg);
    const int n = wg.n;
    const uint32_t lds0 = lds_address(smem);

    if (wave == 8) {
        // A loader: load j (1 KB) covers rows 16j .. 16j+15 of the sub-block
        // (the row layout of a_row_load_offset).
        uint32_t a_voff[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) a_voff[j] = 2 * a_row_load_offset(j, lane, p.lda);
        auto issue_a = [&](int e, uint32_t w) {
            if (BSP_SKIP(p, kSkipSparseRead)) return;  // left out: the wave's waits pass at once
            const uint16_t* ablk = p.a + (uint64_t)w * 32;
            const uint32_t dst = lds0 + (uint32_t)(e % SA) * kA_BYTES;
            gl_lds16_si<0>(a_voff[0], ablk, dst);
            gl_lds16_si<1024>(a_voff[1], ablk, dst);
        };
        stream_loader2<SA, 2>(n, head->aw, p.aw + wg.w_begin, issue_a);
        return;
    }
    if (wave > 8) {
        const int wb = wave - 9;
        const Loader ld(wb, lane, p.ldb);
        const uint32_t b_lds = lds0 + A_RING + wb * Loader::BI * 1024;
        auto issue_b = [&](int e, int64_t w) {
            if (BSP_SKIP(p, kSkipDenseRead)) return;  // left out: the wave's waits pass at once
            ld.issue(b_slice<24>(p.b, p.ldb, w), b_lds + (uint32_t)(e % SB) * Loader::BYTES);
        };
        stream_loader2<SB, Loader::BI>(n, head->bw, p.bw + wg.w_begin, issue_b);
        return;
    }

    // ---- MFMA waves.
    const int l32 = lane & 31, q = lane >> 5;
    const int group = wave >> 2, wc = wave & 3;
    const BReads<TN, 1> brd(lane, wc * 32, false);
    const int a_rd0 = a_row_read_offset(l32, q, 0);
    const int a_rd1 = a_row_read_offset(l32, q, 1);
    // (The lambdas are forced inline: one left out of line would take acc by
    // address and move it to scratch memory.)
    f32x16 acc[8];
    auto zero_acc = [&] () __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
    };
    zero_acc();
    const SpmmSweepRec* sweeps = p.sweeps + wg.s_begin;
    int sw = 0, left = 0;
    SpmmSweepHalf h{};  // this group's units in the open sweep
    // Stores this wave's columns of a unit's tile (t: its accumulator, or zeros).
    auto store_tile = [&](const f32x16& t, int32_t stripe, int32_t n0) __attribute__((always_inline)) {
        const int64_t row0 = (int64_t)stripe * 32;
        const int64_t col = n0 + wc * 32 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t row = row0 + 8 * (v >> 2) + 4 * q + (v & 3);
            if (OUT_BF16)
                store_out(&((uint16_t*)p.c)[row * p.ldc + col], f32_to_bf16_rne(t[v]));
            else
                store_out(&((float*)p.c)[row * p.ldc + col], t[v]);
        }
    };
    // Stores the tile of the unit in `slot` after its last entry's products.
    auto store_slot = [&](int slot) __attribute__((always_inline)) {
        if (BSP_SKIP(p, kSkipWrite)) return;
        // Wait states between the products (asm, unseen by the compiler's
        // hazard checks; twelve at the end of their block) and the reads of
        // their result: more than a 16-pass product's 18.
        __asm__ volatile("s_nop 7\n\ts_nop 7" ::: "memory");
        switch (slot) {
#define BSP_SWEEP_STORE(J) \
            case J: store_tile(acc[J], h.row[J], h.n0[J]); break;
            BSP_SWEEP_STORE(0) BSP_SWEEP_STORE(1) BSP_SWEEP_STORE(2) BSP_SWEEP_STORE(3)
            BSP_SWEEP_STORE(4) BSP_SWEEP_STORE(5) BSP_SWEEP_STORE(6) BSP_SWEEP_STORE(7)
#undef BSP_SWEEP_STORE
            default: break;
        }
    };
    // Opens the next sweep with entries: its units' records, and zero tiles
    // for its units without entries (all of them in a sweep of none).
    struct Head4 {
        int32_t count, empty, pad[2];
    };
    auto open = [&] () __attribute__((always_inline)) {
        while (sw < wg.n_sweeps) {
            const Head4 r = load_const((const Head4*)&sweeps[sw]);
            h = load_const(&sweeps[sw].half[group]);
            const int empty = (r.empty >> (8 * group)) & 0xff;
            if (empty != 0 && !BSP_SKIP(p, kSkipWrite)) {
                const f32x16 zero = {};
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if ((empty >> j) & 1) store_tile(zero, h.row[j], h.n0[j]);
            }
            if (r.count > 0) {
                left = r.count;
                return;
            }
            ++sw;
        }
        left = 0;
    };
    open();

    struct Ops {
        u32x4 a[2];
        u32x4 b[2][1];
    };
    auto read = [&](int k, Ops& o) __attribute__((always_inline)) {
        const uint8_t* as = smem + (k % SA) * kA_BYTES;
        o.a[0] = *(const u32x4*)(as + a_rd0);
        o.a[1] = *(const u32x4*)(as + a_rd1);
        brd.read(smem + A_RING + (k % SB) * Loader::BYTES, o.b);
    };
    // The products of one entry on the accumulator of its slot, as a single
    // asm block that holds the dispatch (a three-level tree on the slot's
    // bits) and takes all eight accumulators as in-out operands.  Any dispatch
    // the compiler sees -- a switch, or a chain of ifs, on builtin or asm
    // products -- leaves it a join where each accumulator is either updated
    // or not, and it resolves those joins by copying accumulators between two
    // register sets.  Here every acc[j] keeps one register, updated in place
    // (the accumulate form: destination = source C).  The compiler's hazard
    // checks do not see into the block: the products need two wait states
    // after a vector ALU write of source C (the zeroing after a sweep: s_nop 1
    // at the block's start), none between products on one accumulator (source
    // C exactly overlapping the previous destination), and the stores that
    // read the results are preceded by explicit wait states (store_sweep).
    // The block ends with twelve wait states, so that the next LDS read into
    // the same operand registers never overwrites a source the products may
    // still be reading.
    auto multiply = [&](const Ops& o, int slot) __attribute__((always_inline)) {
        if (BSP_SKIP(p, kSkipCompute)) return;
        __asm__ volatile(
            "s_nop 1\n\t"
            "s_bitcmp1_b32 %12, 2\n\ts_cbranch_scc1 .Lsw4567_%=\n\t"
            "s_bitcmp1_b32 %12, 1\n\ts_cbranch_scc1 .Lsw23_%=\n\t"
            "s_bitcmp1_b32 %12, 0\n\ts_cbranch_scc1 .Lsw1_%=\n\t"
            "s_branch .Lsw0_%=\n"
            ".Lsw23_%=:\n\t"
            "s_bitcmp1_b32 %12, 0\n\ts_cbranch_scc1 .Lsw3_%=\n\t"
            "s_branch .Lsw2_%=\n"
            ".Lsw4567_%=:\n\t"
            "s_bitcmp1_b32 %12, 1\n\ts_cbranch_scc1 .Lsw67_%=\n\t"
            "s_bitcmp1_b32 %12, 0\n\ts_cbranch_scc1 .Lsw5_%=\n\t"
            "s_branch .Lsw4_%=\n"
            ".Lsw67_%=:\n\t"
            "s_bitcmp1_b32 %12, 0\n\ts_cbranch_scc1 .Lsw7_%=\n\t"
            "s_branch .Lsw6_%=\n"
#define BSP_SWEEP_CASE(J)                                              \
            ".Lsw" #J "_%=:\n\t"                                      \
            "v_mfma_f32_32x32x16_bf16 %" #J ", %8, %10, %" #J "\n\t"   \
            "v_mfma_f32_32x32x16_bf16 %" #J ", %9, %11, %" #J "\n\t"   \
            "s_branch .Lswd_%=\n"
            BSP_SWEEP_CASE(0) BSP_SWEEP_CASE(1) BSP_SWEEP_CASE(2) BSP_SWEEP_CASE(3)
            BSP_SWEEP_CASE(4) BSP_SWEEP_CASE(5) BSP_SWEEP_CASE(6) BSP_SWEEP_CASE(7)
#undef BSP_SWEEP_CASE
            ".Lswd_%=:\n\t"
            "s_nop 7\n\ts_nop 3"
            : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]),
              "+v"(acc[6]), "+v"(acc[7])
            : "v"(o.a[0]), "v"(o.a[1]), "v"(o.b[0][0]), "v"(o.b[1][0]), "s"(slot)
            : "scc");
    };
    auto lds_done = [] { wait_lgkm0(); };
    // Step k (k = 0, 2, 4, ...; the loaders' barrier for entries k and k+1):
    // read and multiply this group's entries among k and k+1.
    // This group's entry among a step's two: its slot, or -1.
    // (w: the high half of the entry's word, which holds the slot code and
    // the last bit.)
    auto mine = [&](uint32_t w) __attribute__((always_inline)) {
        const uint32_t code = (w >> (kSweepSlotShift - 32)) & 31u;
        return (code & 16u) == 0 && (int)(code >> 3) == group ? (int)(code & 7u) : -1;
    };
    constexpr uint32_t kLastHi = (uint32_t)((uint64_t)kSweepLast >> 32);
    auto step = [&](int k, uint32_t w0, uint32_t w1) __attribute__((always_inline)) {
        barrier_no_fence();
        const int s0 = mine(w0), s1 = mine(w1);
        Ops o;
        if (s0 >= 0) {
            read(k, o);
            lds_done();
            multiply(o, s0);
            if (w0 & kLastHi) store_slot(s0);  // the unit's last entry
        }
        if (s1 >= 0) {
            read(k + 1, o);
            lds_done();
            multiply(o, s1);
            if (w1 & kLastHi) store_slot(s1);
        }
        left -= 2;
        if (left == 0) {
            zero_acc();
            ++sw;
            open();
        }
    };
    // The high halves of the stream's B words, a step's two by scalar loads
    // one step ahead, waited for with the step's LDS reads (the arrays are
    // padded past every stream's end).  Only the high halves: with whole
    // words, the compiler reused the registers of the unused low halves
    // while their load was in flight, and so waited for the load at once,
    // at the top of every step.
    const uint32_t* wh = (const uint32_t*)(p.bw + wg.w_begin) + 1;
    uint32_t c0 = load_const(wh), c1 = load_const(wh + 2);
    wait_lgkm0();
    for (int k = 0; k < n; k += 2) {
        const uint32_t n0 = load_const(wh + 2 * k + 4), n1 = load_const(wh + 2 * k + 6);
        step(k, c0, c1);
        if (k == 0) BSP_TL_MARK(1);
        if ((k & 7) == 0 && k < 8 * 60) BSP_TL_MARK(2 + (k >> 3));
        c0 = n0;
        c1 = n1;
    }
    if (wave == 0) BSP_TL_FLUSH();
}

// ---------------------------------------------------------------------------
// Block-sparse attention pair, fused: O = S * V with S = bf16(mask (.) (Q*K^T))
// at the mask's blocks, S never leaving the compute unit.  Same schedule and
// ring as the SpMM (the mask plays A, V plays B, one 128-column tile); each
// ring stage also carries the entry's 32 x DK block of K.  Each wave computes
// one 16 x 16 quadrant of the entry's S^T = K_blk * Q^T from LDS (its 16
// queries of Q^T stay in registers), applies the mask, rounds to bf16 and
// writes the quadrant to an S buffer in LDS; after the next ring barrier
// every wave reads the whole 32 x 32 S from there as the A operand of
// O += S * V.  Numerically the same as bsp_sddmm (column-major Y = K, bf16
// output) followed by bsp_spmm with the same structure, up to the fp32
// summation order of Q K^T.
template <int DK, int S, bool OUT_BF16>
__global__ __launch_bounds__(256) void attention_kernel(AttentionArgs pa) {
    using namespace spmm_detail;
    using Slice = BSlice<1>;
    const SpmmArgs& p = pa.s;
    constexpr int K_BYTES = 64 * DK;              // 32 keys x DK bf16
    constexpr int K_LANES = DK >= 64 ? 64 : 32;    // lanes per K load instruction
    constexpr int KI = K_BYTES / 4 / (16 * K_LANES);  // K load instructions per wave
    constexpr int PER = 1 + KI + Slice::BI;
    constexpr int K_RING = S * kA_BYTES;
    constexpr int B_RING = K_RING + S * K_BYTES;
    constexpr int Q_AREA = B_RING + S * Slice::BYTES;
    static_assert(KI >= 1 && DK % 32 == 0 && DK <= 128, "head dimension");
    // The Q area holds Q, then (Q in registers) the two 2 KB S buffers.
    __shared__ __attribute__((aligned(1024))) uint8_t smem[Q_AREA + (K_BYTES > 4096 ? K_BYTES : 4096)];

    const SpmmWg it = load_const(p.wgs + blockIdx.x);
    if (it.row < 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, q = lane >> 5;
    const uint32_t lds0 = lds_address(smem);
    const Slice bsl(wave, lane, 0, p.N, p.ldb);
    const BReads<Slice::TN, 1> brd(lane, wave * 32, false);

    // K blocks and the stripe's Q rows in LDS as 16-byte chunks (c, row r) at
    // (32c + r) * 16, so that the operand of step s of row l32 (chunk 2s + q)
    // is one conflict-free ds_read_b128.  Wave w loads chunks [w*DK, (w+1)*DK).
    uint32_t k_voff[KI];  // byte offsets from the block's first key row
    int64_t q_goff[KI];
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        const int ci = wave * DK + j * K_LANES + (lane & (K_LANES - 1));
        k_voff[j] = (uint32_t)(2 * ((int64_t)(ci & 31) * pa.ldk + 8 * (ci >> 5)));
        q_goff[j] = (int64_t)(ci & 31) * pa.ldq + 8 * (ci >> 5);
    }
    const int n = it.e_end - it.e_begin;
    // Q of the stripe goes through the same DMA path ahead of the ring, so it
    // has landed once entry 0 has; its operands are then read from LDS (plain
    // global loads here would be waited for inside the loop by the compiler,
    // which cannot see that they completed, draining the ring every entry).
    if (n > 0) {
        const uint16_t* qrow = pa.q + (int64_t)it.row * 32 * pa.ldq;
#pragma unroll
        for (int j = 0; j < KI; ++j)
            if (lane < K_LANES) gl_lds16(qrow + q_goff[j], lds0 + Q_AREA + wave * DK * 16 + j * K_LANES * 16);
    }
    // S = mask (.) Q K^T of an entry is computed in four 16 x 16 quadrants,
    // one per wave: wave w takes keys ka = 16*(w%2) .. +15 and queries
    // qb = 16*(w/2) .. +15, S^T quadrant = K[ka..][:] * Q[qb..][:]^T in DK/32
    // 16x16x32 products.  Lane l holds Q[qb + l%16][32t + 8*(l/16) .. +7]
    // for each 32-deep step t (the B operand).
    const int ka = 16 * (wave & 1), qb = 16 * (wave >> 1);
    const int l16 = lane & 15, g4 = lane >> 4;
    u32x4 qv[DK / 32];
    const uint32_t a_voff = 2 * ((8 * wave + (lane & 7)) * p.lda + 8 * ((lane & 31) >> 3));
    const uint32_t a_lds = lds0 + wave * 512;
    const uint32_t k_lds = lds0 + K_RING + wave * DK * 16;
    const uint32_t b_lds = lds0 + B_RING + wave * Slice::BI * 1024;
    EntryWords words(p.ents + it.e_begin, n, lane);
    auto issue = [&](int e, int stage) {
        uint32_t bw, aw;  // first key of the block, mask block offset / 32
        words.get(e, lane, bw, aw);
        if (lane < 32) gl_lds16_s(a_voff, p.a + (int64_t)aw * 32, a_lds + stage * kA_BYTES);
        const uint16_t* kblk = pa.k + (int64_t)bw * pa.ldk;
#pragma unroll
        for (int j = 0; j < KI; ++j)
            if (lane < K_LANES) gl_lds16_s(k_voff[j], kblk, k_lds + stage * K_BYTES + j * K_LANES * 16);
        bsl.issue(p.b, p.ldb, bw, b_lds + stage * Slice::BYTES);
    };

    // The quadrant's mask values of lane l: query qb + l%16, keys ka + 4*(l/16)
    // .. +3, 8 bytes of the mask's row.  The mask is loaded without the SpMM A
    // layout's chunk XOR: segment g, chunk j of row r at (8j + r%8) * 16.
    const int mq = qb + l16, mkey = ka + 4 * g4;
    const int m_rd = (mq >> 3) * 512 + (8 * (mkey >> 3) + (mq & 7)) * 16 + 2 * (mkey & 7);
    // S of an entry in LDS (two buffers in the Q area, free once Q is in
    // registers), bf16 row-major by query, 64 bytes a row, 16-byte chunk c of
    // row r at position c ^ (r/4 % 4): each 16-lane quarter of the O
    // operand read, and each half-wave of the quadrant write, covers every bank.
    auto s_pos = [](int r, int key) { return r * 64 + 16 * ((key >> 3) ^ ((r >> 2) & 3)) + 2 * (key & 7); };
    const int s_wr = s_pos(mq, mkey);
    const int s_rd0 = s_pos(l32, 8 * q), s_rd1 = s_pos(l32, 16 + 8 * q);
    f32x16 acc[1];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][v] = 0.0f;

    // Operands of one entry kept in registers: V's rows (its S is in LDS).
    struct Operands {
        u32x4 b[2][1];
    };
    int e_read = 0, e_mul = 0;  // entries read / multiplied so far (S buffer = entry % 2)
    run_ring<S, PER, true, Operands, true, true>(
        n, issue,
        [&](int stage, Operands& o) {
            const uint8_t* ks = smem + K_RING + stage * K_BYTES;
            f32x4 sq = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < DK / 32; ++t)
                sq = mfma16(*(const u32x4*)(ks + (32 * (4 * t + g4) + ka + l16) * 16), qv[t], sq);
            const uint64_t mw = *(const uint64_t*)(smem + stage * kA_BYTES + m_rd);
            const uint32_t m0 = (uint32_t)mw, m1 = (uint32_t)(mw >> 32);
            // sq[v] = S^T[ka + 4*(l/16) + v][qb + l%16]: keys mkey + v of query mq.
            const uint32_t lo = pack_bf16x2(sq[0] * __uint_as_float(m0 << 16), sq[1] * __uint_as_float(m0 & 0xffff0000u));
            const uint32_t hi = pack_bf16x2(sq[2] * __uint_as_float(m1 << 16), sq[3] * __uint_as_float(m1 & 0xffff0000u));
            *(uint64_t*)(smem + Q_AREA + (e_read & 1) * 2048 + s_wr) = (uint64_t)lo | ((uint64_t)hi << 32);
            ++e_read;
            brd.read(smem + B_RING + stage * Slice::BYTES, o.b);
        },
        [&](const Operands& o) {
            const uint8_t* sx = smem + Q_AREA + (e_mul & 1) * 2048;
            ++e_mul;
            acc[0] = mfma32(*(const u32x4*)(sx + s_rd0), o.b[0][0], acc[0]);
            acc[0] = mfma32(*(const u32x4*)(sx + s_rd1), o.b[1][0], acc[0]);
        },
        [&] {
#pragma unroll
            for (int t = 0; t < DK / 32; ++t)
                qv[t] = *(const u32x4*)(smem + Q_AREA + (32 * (4 * t + g4) + qb + l16) * 16);
        });
    spmm_finish<1, OUT_BF16>(p, it, acc, tid);
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
    // Pieces are added in order; the loads of up to four pieces are issued
    // together so their round trips overlap.
    constexpr int AHEAD = NTW == 1 ? 4 : 2;
    int pc = 0;
    for (; pc + AHEAD <= sp.npieces; pc += AHEAD) {
        float v4[AHEAD][NTW * 16];
#pragma unroll
        for (int j = 0; j < AHEAD; ++j) {
            const float* src = p.ws + ((int64_t)(sp.base + pc + j) * p.n_tiles + tile) * PF;
#pragma unroll
            for (int i = 0; i < NTW * 16; ++i) v4[j][i] = src[i * 256 + tid];
        }
#pragma unroll
        for (int j = 0; j < AHEAD; ++j)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[nt][v] += v4[j][nt * 16 + v];
    }
    for (; pc < sp.npieces; ++pc) {
        const float* src = p.ws + ((int64_t)(sp.base + pc) * p.n_tiles + tile) * PF;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[nt][v] += src[(nt * 16 + v) * 256 + tid];
    }
    spmm_store_tile<NTW, OUT_BF16>(p, acc, (int64_t)sp.row * 32, tile * 128 * NTW, wave, lane & 31, lane >> 5);
}

// ---------------------------------------------------------------------------
// SDDMM.  Workgroup = one work item: a run of output sub-blocks (entries) of
// one 32-row stripe, taken one entry at a time by all four waves, each over a
// quarter of K: wave w takes the k-steps (32 deep) w, w+4, w+8, ...  The
// partial 32x32 sums meet in LDS; wave w then adds the four partials of rows
// 8w..8w+7, applies the mask values there and stores them.
//
// Operands go straight from global memory into MFMA registers: X rows and the
// rows of Y^T (Y in BSP_COL_MAJOR, e.g. the key matrix of Q*K^T) are
// contiguous along k.  Row-major Y is loaded as it lies (16 rows x 64 bytes
// per instruction) into a wave-private LDS tile and read back with the LDS
// transpose read, as in the SpMM kernel.  Each wave issues the loads of its
// next entry before it multiplies the current one; when a wave's k-steps fit
// in one register chunk (K <= 256) its X operands are loaded once per item.
namespace sddmm_detail {

constexpr int kKW = 2;  // k-steps per register chunk and wave

// One unit of a wave's stream: up to kKW k-steps of one entry.  With X_KEEP
// (K <= 256: every wave's k-steps fit one chunk) the X operands are loaded
// once per item and the chunk carries only Y.
template <bool X_KEEP>
struct Chunk {
    u32x4 b[kKW][2];   // Y operands (k-step j, half s), or raw row-major Y rows (i = 0, 1)
    u32x4 a[kKW][2];   // X operands
    uint32_t m[4];     // mask values (bf16 bits) of this wave's 4 rows, first chunk only
};
template <>
struct Chunk<true> {
    u32x4 b[kKW][2];
    uint32_t m[4];
};

}  // namespace sddmm_detail

template <bool Y_COLMAJOR, bool OUT_BF16, bool X_KEEP>
__global__ __launch_bounds__(256) void sddmm_kernel(SddmmArgs p) {
    using namespace sddmm_detail;
    __shared__ __attribute__((aligned(16))) float red[4][16 * 64];  // partial sums of one entry
    __shared__ __attribute__((aligned(16))) uint8_t ytile[Y_COLMAJOR ? 1 : 4][2048];

    const SddmmItem it = load_const(p.wgs + blockIdx.x);
    const int n_e = it.e_end - it.e_begin;
    if (n_e <= 0) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, q = lane >> 5;
    const int KT = p.K >> 5;
    const int nks = KT > wave ? (KT - wave + 3) >> 2 : 0;  // k-steps of this wave
    // Chunks per entry and the unit count are the same for every wave (wave 0
    // has the most k-steps), so all waves meet at the same barriers.
    const int nks0 = (KT + 3) >> 2;
    const int nch = X_KEEP ? 1 : (nks0 + kKW - 1) / kKW;
    const int UW = n_e * nch;  // units (entry, chunk)

    // The item's entry words, one entry per lane (an item holds at most 64
    // entries), fetched once; entry eu's words are read back with readlane.
    int32_t lane_col = 0;
    int64_t lane_off = 0;
    if (lane < n_e) {
        lane_col = p.ent_col[it.e_begin + lane];
        lane_off = p.ent_off[it.e_begin + lane];
    }
    auto entry_col = [&](int eu) { return __builtin_amdgcn_readlane(lane_col, eu); };
    auto entry_off = [&](int eu) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)lane_off, eu);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)lane_off >> 32), eu);
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };

    const uint16_t* xlane = p.x + (int64_t)(it.x_row0 + l32) * p.ldx + 8 * q;
    auto load_x = [&](int c, u32x4 (&a)[kKW][2]) {
#pragma unroll
        for (int j = 0; j < kKW; ++j) {
            const int kj = c * kKW + j;
            if (kj < nks) {
                const int k0 = (wave + 4 * kj) * 32;
                a[j][0] = *(const u32x4*)(xlane + k0);
                a[j][1] = *(const u32x4*)(xlane + k0 + 16);
            }
        }
    };
    auto load = [&](int u, Chunk<X_KEEP>& ch) {
        const int eu = X_KEEP ? u : u / nch, c = u - eu * nch;
        const int32_t ycol = entry_col(eu);
        if constexpr (!X_KEEP) load_x(c, ch.a);
#pragma unroll
        for (int j = 0; j < kKW; ++j) {
            const int kj = c * kKW + j;
            if (kj < nks) {
                const int k0 = (wave + 4 * kj) * 32;
                if (Y_COLMAJOR) {
                    const uint16_t* yl = p.y + (int64_t)(ycol + l32) * p.ldy + k0 + 8 * q;
                    ch.b[j][0] = *(const u32x4*)yl;
                    ch.b[j][1] = *(const u32x4*)(yl + 16);
                } else {
                    const uint16_t* yl = p.y + (int64_t)(k0 + (lane >> 2)) * p.ldy + ycol + 8 * (lane & 3);
                    ch.b[j][0] = *(const u32x4*)yl;
                    ch.b[j][1] = *(const u32x4*)(yl + 16 * p.ldy);
                }
            }
        }
        if (c == 0) {
            const uint16_t* ml = p.mask + entry_off(eu) + (int64_t)(8 * wave + 4 * q) * p.ldo + l32;
#pragma unroll
            for (int j = 0; j < 4; ++j) ch.m[j] = ml[j * p.ldo];
        }
    };

    // Row-major Y: LDS offsets of the transpose reads for k-step half s and
    // 4-row group h (16-lane group g reads rows 16s + 8(g/2) + 4h .. +3 of
    // columns 16(g%2) + i).
    int ytr[2][2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int g = lane >> 4, ll = lane & 15;
            const int row = 16 * s2 + 8 * (g >> 1) + 4 * h + (ll >> 2);
            const int col = 16 * (g & 1) + 4 * (ll & 3);
            ytr[s2][h] = row * 64 + col * 2;
        }

    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    u32x4 xa[kKW][2];
    if constexpr (X_KEEP) load_x(0, xa);
    uint32_t mcur[4] = {0u, 0u, 0u, 0u};

    auto compute = [&](int u, Chunk<X_KEEP>& ch) {
        const int eu = X_KEEP ? u : u / nch, c = u - eu * nch;
        if (c == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) mcur[j] = ch.m[j];
        }
#pragma unroll
        for (int j = 0; j < kKW; ++j) {
            const int kj = c * kKW + j;
            if (kj < nks) {
                u32x4 a0, a1;
                if constexpr (X_KEEP) {
                    a0 = xa[j][0];
                    a1 = xa[j][1];
                } else {
                    a0 = ch.a[j][0];
                    a1 = ch.a[j][1];
                }
                u32x4 b0, b1;
                if (Y_COLMAJOR) {
                    b0 = ch.b[j][0];
                    b1 = ch.b[j][1];
                } else {
                    // Rows 16i + lane/4, 16-byte chunk lane%4: 64-byte rows.
                    // One tile per wave: the LDS serves a wave's accesses in
                    // order, so the next k-step's writes follow these reads.
                    uint8_t* yt = ytile[wave];
                    *(u32x4*)(yt + lane * 16) = ch.b[j][0];
                    *(u32x4*)(yt + 1024 + lane * 16) = ch.b[j][1];
                    const u32x4 l0 = spmm_detail::ld_tr_b16(yt + ytr[0][0]);
                    const u32x4 h0 = spmm_detail::ld_tr_b16(yt + ytr[0][1]);
                    const u32x4 l1 = spmm_detail::ld_tr_b16(yt + ytr[1][0]);
                    const u32x4 h1 = spmm_detail::ld_tr_b16(yt + ytr[1][1]);
                    b0 = u32x4{l0.x, l0.y, h0.x, h0.y};
                    b1 = u32x4{l1.x, l1.y, h1.x, h1.y};
                }
                acc = mfma32(a0, b0, acc);
                acc = mfma32(a1, b1, acc);
            }
        }
        if (c == nch - 1) {
            // Entry done: meet the other waves' partials, finish rows 8w..8w+7.
            // The first barrier keeps this entry's writes behind every wave's
            // reads of the previous entry; the waits before each barrier make
            // the LDS accesses complete without a fence (a fence would also
            // wait for the next unit's loads, which stay in flight).
            spmm_detail::wait_lgkm0();
            spmm_detail::barrier_no_fence();
            float* mine = red[wave];
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[v * 64 + lane] = acc[v];
            spmm_detail::wait_lgkm0();
            spmm_detail::barrier_no_fence();
            const int64_t off = entry_off(eu);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int v = 4 * wave + j;
                float sum = 0.0f;
#pragma unroll
                for (int w2 = 0; w2 < 4; ++w2) sum += red[w2][v * 64 + lane];
                const float val = sum * bf16_to_f32((uint16_t)mcur[j]);
                const int64_t idx = off + (int64_t)(8 * wave + 4 * q + j) * p.ldo + l32;
                if (OUT_BF16)
                    store_out(&((uint16_t*)p.out)[idx], f32_to_bf16_rne(val));
                else
                    store_out(&((float*)p.out)[idx], val);
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
        }
    };

    // Unit u+1's loads are issued before unit u is multiplied; unrolled by
    // two so that the two chunks keep their registers (a copy would wait for
    // the loads).
    Chunk<X_KEEP> c0, c1;
    load(0, c0);
    for (int u = 0; u < UW; u += 2) {
        if (u + 1 < UW) load(u + 1, c1);
        compute(u, c0);
        if (u + 1 < UW) {
            if (u + 2 < UW) load(u + 2, c0);
            compute(u + 1, c1);
        }
    }
}

// ---------------------------------------------------------------------------
// SDDMM for K <= 256 in one shot.  A workgroup takes an item of up to four
// output sub-blocks of one 32-row stripe, one per wave.  All its operands go
// global->LDS at once: the X stripe (32 x K, shared, loaded by all waves) and
// each wave's Y panel (K x 32, or 32 x K rows of Y^T).  One wait for the
// wave's own loads and one barrier (for the other waves' parts of X), then
// each wave runs its whole K-deep 32x32 product, multiplies by the mask
// block and stores it.  No loop-carried loads, so nothing the compiler waits
// for; LDS = 320 * K bytes, two workgroups per compute unit at K = 256.
// MASK16 (mask values 16-byte aligned): the wave fetches its 32x32 mask
// sub-block row-wise, two 16-byte loads per lane in flight with the operands
// (sixteen 2-byte loads per lane cost 1.4 us of 8.7 at the 10% workload);
// after the products it stages them in its own Y panel, free by then, and
// reads them back in the accumulator's layout with the transpose read.
//   X (and Y^T) rows: 2K bytes, 16-byte chunk c of row r at slot
//   c ^ (r % min(K/8, 16)) (conflict-free row reads);
//   row-major Y panel: 64-byte rows, read with the transpose read.
namespace sddmm_shot {
template <int K>
struct Layout {
    static constexpr int NC = K / 8;                 // 16-byte chunks per row
    static constexpr int SW = NC < 16 ? NC : 16;     // swizzle period
    static constexpr int RP = 2 * K;                 // row pitch (bytes)
    static constexpr int PANEL = 64 * K;             // 32 x K or K x 32 bf16
    static constexpr int XI = PANEL / 1024;          // 1 KB loads per panel
    static constexpr int LDS = 5 * PANEL;            // X + four Y panels
};
}  // namespace sddmm_shot

template <int K, bool Y_COLMAJOR, bool OUT_BF16, bool MASK16>
__global__ __launch_bounds__(256, 2) void sddmm_shot_kernel(SddmmArgs p) {
    using namespace spmm_detail;
    using L = sddmm_shot::Layout<K>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[L::LDS];
    BSP_TL_DECL_REGS();
    const SddmmItem it = load_const(p.wgs + blockIdx.x);
    if (it.e_end <= it.e_begin) return;  // idle workgroup (uniform)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, q = lane >> 5;
    const int e = it.e_begin + wave;
    const bool has = e < it.e_end;  // uniform per wave
    const uint32_t lds0 = lds_address(smem);
    const uint32_t ylds = lds0 + (1 + wave) * L::PANEL;

    // Mask values: (MASK16) 16-byte chunks c = lane, lane + 64 of the
    // row-major 32x32 sub-block (row c / 4, columns 8 * (c % 4) ..), issued
    // first so their fetch overlaps the operands' issue (nothing uses them
    // before the products); otherwise this lane's 16 outputs, after the
    // operands.
    int64_t off = 0;
    uint32_t mk[16];
    u32x4 mraw[2];
    if (has) off = load_const(p.ent_off + e);
    // (A read left out by the instrumented build is not issued: every wait
    // here is for all of the workgroup's loads.)
    if constexpr (MASK16) {
        if (has && !BSP_SKIP(p, kSkipSparseRead)) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = lane + 64 * h;
                mraw[h] = *(const u32x4*)(p.mask + off + (int64_t)(c >> 2) * p.ldo + 8 * (c & 3));
            }
        } else {
            mraw[0] = mraw[1] = u32x4{0u, 0u, 0u, 0u};
        }
    }

    // A 32-row panel (X stripe, or 32 rows of Y^T) into LDS, load t of it:
    // slot 64t + lane holds row (64t + lane) / NC, chunk c ^ (row % SW).
    auto rows_panel = [&](const uint16_t* base, int64_t ld, int t, uint32_t dst) {
        const int slot = 64 * t + lane;
        const int r = slot / L::NC;
        const int c = (slot % L::NC) ^ (r % L::SW);
        gl_lds16(base + (int64_t)r * ld + 8 * c, dst + 1024 * t);
    };
#pragma unroll
    for (int j = 0; j < (L::XI + 3) / 4; ++j) {
        const int t = wave + 4 * j;
        if (t < L::XI && !BSP_SKIP(p, kSkipDenseRead)) rows_panel(p.x + (int64_t)it.x_row0 * p.ldx, p.ldx, t, lds0);
    }
    if (has && !BSP_SKIP(p, kSkipDense2Read)) {
        const int32_t col = load_const(p.ent_col + e);
        if (Y_COLMAJOR) {
#pragma unroll
            for (int t = 0; t < L::XI; ++t) rows_panel(p.y + (int64_t)col * p.ldy, p.ldy, t, ylds);
        } else {
            // K rows of 64 bytes: slot 64t + lane holds row slot / 4, chunk slot % 4.
#pragma unroll
            for (int t = 0; t < L::XI; ++t) {
                const int slot = 64 * t + lane;
                gl_lds16(p.y + (int64_t)(slot >> 2) * p.ldy + col + 8 * (slot & 3), ylds + 1024 * t);
            }
        }
    }
    if constexpr (!MASK16) {
        if (has && !BSP_SKIP(p, kSkipSparseRead)) {
#pragma unroll
            for (int v = 0; v < 16; ++v)
                mk[v] = p.mask[off + (int64_t)(8 * (v >> 2) + 4 * q + (v & 3)) * p.ldo + l32];
        } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) mk[v] = 0u;
        }
    }
    wait_vmcnt<0>();
    barrier_no_fence();
    BSP_TL_MARK(1);
    if (!has) return;

    const uint8_t* xs = smem;
    const uint8_t* ys = smem + (1 + wave) * L::PANEL;
    // Row reads: row l32, logical chunk 4*ks + 2*s2 + q.
    auto row_read = [&](const uint8_t* panel, int ch) {
        return *(const u32x4*)(panel + l32 * L::RP + 16 * (ch ^ (l32 % L::SW)));
    };
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int ch = 4 * ks + 2 * s2 + q;
            const u32x4 a = row_read(xs, ch);
            u32x4 b;
            if (Y_COLMAJOR) {
                b = row_read(ys, ch);
            } else {
                const int g = lane >> 4;
                const int r = 32 * ks + 16 * s2 + 8 * q + ((lane & 15) >> 2);
                const int cb = 2 * (16 * (g & 1) + 4 * (lane & 3));
                const u32x4 lo = ld_tr_b16(ys + r * 64 + cb);
                const u32x4 hi = ld_tr_b16(ys + (r + 4) * 64 + cb);
                b = u32x4{lo.x, lo.y, hi.x, hi.y};
            }
            if (!BSP_SKIP(p, kSkipCompute)) acc = mfma32(a, b, acc);
        }
    BSP_TL_MARK(2);
    if constexpr (MASK16) {
        // The products have consumed this wave's Y panel: stage the mask
        // sub-block there (row-major, 64-byte rows) and read back rows
        // 8i + 4q .. +3 of column l32 (the accumulator's values 4i .. 4i+3).
        uint8_t* mt = smem + (1 + wave) * L::PANEL;
        *(u32x4*)(mt + 16 * lane) = mraw[0];
        *(u32x4*)(mt + 16 * (lane + 64)) = mraw[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 8 * i + 4 * q + ((lane & 15) >> 2);
            const int col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            const u32x4 r = ld_tr_b16(mt + row * 64 + 2 * col);
            mk[4 * i + 0] = r.x & 0xffffu;
            mk[4 * i + 1] = r.x >> 16;
            mk[4 * i + 2] = r.y & 0xffffu;
            mk[4 * i + 3] = r.y >> 16;
        }
    }
    if (!BSP_SKIP(p, kSkipWrite)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float val = acc[v] * bf16_to_f32((uint16_t)mk[v]);
            const int64_t idx = off + (int64_t)(8 * (v >> 2) + 4 * q + (v & 3)) * p.ldo + l32;
            if (OUT_BF16)
                store_out(&((uint16_t*)p.out)[idx], f32_to_bf16_rne(val));
            else
                store_out(&((float*)p.out)[idx], val);
        }
    }
    if (wave == 0) BSP_TL_FLUSH();
}

// ---------------------------------------------------------------------------
// SpGEMM numeric phase, C = A * B with A, B and C in BSR (C's structure and
// the product lists come from the plan).  The unit of output is a 32x32
// sub-block (a task) with its run of products; a wave takes a contiguous
// run of tasks (at most 64) and streams all their products through one
// wave-private ring of S LDS stages (2 KB of A, then 2 KB of B, loaded
// global->LDS), so the ring stays full across sub-block boundaries.  At the
// last product of a task the wave stores the sub-block and clears its
// accumulators.  Waves never wait for each other (no barriers).  Run slot
// (x * wg_per_xcd + j) * 4 + wave belongs to workgroup j * 8 + x, which runs
// on XCD x; the plan puts there the runs of one region of the output (a
// band of block rows crossed with a band of block columns), so the XCD's L2
// holds the A and B blocks the region shares.
namespace spgemm_detail {
constexpr int kStage = kSpgemmStageBytes;  // A sub-block (2 KB) + B sub-block (2 KB)
constexpr int kPer = 4;                    // global->LDS loads per wave per product
constexpr int kWords = 128;                // product words held in registers (two per lane)
}  // namespace spgemm_detail

template <int S, bool OUT_BF16>
__global__ __launch_bounds__(256) void spgemm_kernel(SpgemmArgs p) {
    using namespace spmm_detail;
    using namespace spgemm_detail;
    static_assert(kPer * (S - 1) < 64, "vmcnt budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * S * kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int xcd = blockIdx.x % kNumXcd, slot = blockIdx.x / kNumXcd;
    const int id = (xcd * p.wg_per_xcd + slot) * 4 + wave;
    const SpgemmRun run = load_const(p.runs + id);
    const int32_t t0 = run.t0, t1 = run.t1, p0 = run.p0;
    if (t0 >= t1) return;
    const int n = run.p1 - p0;  // products of the run (>= 1 per task)
    const int l32 = lane & 31, q = lane >> 5;
    const uint32_t lds_w = lds_address(smem) + wave * S * kStage;
    const uint8_t* smem_w = smem + wave * S * kStage;

    // Lane j holds task t0 + j (output offset, end of its products relative
    // to the run) and product words kWords * c + 64 * h + j of the current
    // chunk c, h = 0, 1.  All are loaded, and waited for, before the ring
    // starts; a run of more than kWords products reloads the words in the
    // (rare) issue that crosses a chunk and waits for them there.  No load is
    // then pending anywhere in the loop (the compiler would otherwise wait
    // for every outstanding load, the ring included, before a use).
    uint32_t off_lo = 0, off_hi = 0;
    int32_t t_end = 0;
    if (t0 + lane < t1) {
        const SpgemmTask tk = p.tasks[t0 + lane];
        off_lo = (uint32_t)tk.out_off;
        off_hi = (uint32_t)(tk.out_off >> 32);
        t_end = tk.t_end - p0;
    }
    const uint64_t* terms = p.terms + p0;
    uint32_t w_lo0 = 0, w_hi0 = 0, w_lo1 = 0, w_hi1 = 0;
    auto fetch_words = [&](int base) {
        if (base + lane < n) {
            const uint64_t w = terms[base + lane];
            w_lo0 = (uint32_t)w;
            w_hi0 = (uint32_t)(w >> 32);
        }
        if (base + 64 + lane < n) {
            const uint64_t w = terms[base + 64 + lane];
            w_lo1 = (uint32_t)w;
            w_hi1 = (uint32_t)(w >> 32);
        }
        __asm__ volatile("" : "+v"(w_lo0), "+v"(w_hi0), "+v"(w_lo1), "+v"(w_hi1));
    };
    fetch_words(0);
    __asm__ volatile("" : "+v"(off_lo), "+v"(off_hi), "+v"(t_end));

    // Loads of one product (two 1 KB instructions each for A and B):
    //   A: instruction h, lane L loads segment g = 2h + L/32: row 8g + L%8,
    //      16-byte chunk ((L%32)/8) ^ (g%2) into byte 1024h + 16L (the SpMM
    //      sub-block layout, a_load_offset / a_read_offset).
    //   B: instruction h, lane L loads row 16h + L/4, chunk L%4 into byte
    //      1024h + 16L: plain row-major rows of 64 bytes.
    int64_t a_goff0, a_goff1, b_goff0, b_goff1;
    a_goff0 = spmm_detail::a_load_offset(lane >> 5, lane, p.lda);
    a_goff1 = spmm_detail::a_load_offset(2 + (lane >> 5), lane, p.lda);
    b_goff0 = (int64_t)(lane >> 2) * p.ldb + 8 * (lane & 3);
    b_goff1 = b_goff0 + (int64_t)16 * p.ldb;
    auto issue = [&](int e, int stage) {
        if ((e & (kWords - 1)) == 0 && e > 0) fetch_words(e);
        const bool h = (e & 64) != 0;
        const uint32_t aw = __builtin_amdgcn_readlane(h ? w_lo1 : w_lo0, e & 63);
        const uint32_t bw = __builtin_amdgcn_readlane(h ? w_hi1 : w_hi0, e & 63);
        const uint16_t* ab = p.a + (int64_t)aw * 32;
        const uint16_t* bb = p.b + (int64_t)bw * 32;
        const uint32_t st = lds_w + stage * kStage;
        gl_lds16(ab + a_goff0, st);
        gl_lds16(ab + a_goff1, st + 1024);
        gl_lds16(bb + b_goff0, st + 2048);
        gl_lds16(bb + b_goff1, st + 3072);
    };
    // Operand reads: A row l32, chunk 2*s + q; B column l32 by transpose
    // reads of rows 16*s + 8*q + 4*h + (lane%16)/4, columns 16*(lane/16 % 2)
    // + 4*(lane%4) (the second k-step adds 16 rows = 1 KB).
    const int a_rd = spmm_detail::a_read_offset(l32, q);  // + 256 * s
    const int b_rd = 2048 + (8 * ((lane >> 4) >> 1) + ((lane & 15) >> 2)) * 64 +
                     2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3));  // + 256 * h + 1024 * s

#pragma unroll
    for (int e = 0; e < S - 1; ++e)
        if (e < n) issue(e, e);
    int stage = 0;  // stage of product k
    int k = 0;      // next product of the run
    const int ntask = t1 - t0;
    for (int ct = 0; ct < ntask; ++ct) {
        const int kend = __builtin_amdgcn_readlane(t_end, ct);
        f32x16 acc;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
        for (; k < kend; ++k) {
            // Product k+S-1 goes into the stage product k-1 used: this wave's
            // reads of it are complete once lgkmcnt is 0 (no scalar loads are
            // in flight here, so the wait covers only those reads).
            if (k + S - 1 < n) {
                spmm_detail::wait_lgkm0();
                issue(k + S - 1, stage == 0 ? S - 1 : stage - 1);
            }
            // Product k landed (stores in flight only make this wait longer:
            // loads complete in order, so the count still covers product k).
            wait_stages<kPer, S - 1>(min(S - 1, n - 1 - k));
            const uint8_t* st = smem_w + stage * kStage;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const u32x4 av = *(const u32x4*)(st + a_rd + 256 * s2);
                const u32x4 lo = ld_tr_b16(st + b_rd + 1024 * s2);
                const u32x4 hi = ld_tr_b16(st + b_rd + 1024 * s2 + 256);
                acc = mfma32(av, u32x4{lo.x, lo.y, hi.x, hi.y}, acc);
            }
            stage = stage == S - 1 ? 0 : stage + 1;
        }
        // Store through the stage the task's last product used (free until
        // the next issue, whose lgkmcnt wait covers these LDS accesses): the
        // sub-block goes to LDS row-major, then out in 16-byte pieces, whole
        // rows per group of lanes.
        const int64_t off = (int64_t)(((uint64_t)__builtin_amdgcn_readlane(off_hi, ct) << 32) |
                                      __builtin_amdgcn_readlane(off_lo, ct));
        uint8_t* tile = (uint8_t*)smem_w + (stage == 0 ? S - 1 : stage - 1) * kStage;
        constexpr int ESZ = OUT_BF16 ? 2 : 4;
        constexpr int ROW = 32 * ESZ;          // bytes per tile row
        constexpr int PIECES = 32 * ROW / 16;  // 16-byte pieces of the tile
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = 8 * (v >> 2) + 4 * q + (v & 3);
            if (OUT_BF16)
                *(uint16_t*)(tile + r * ROW + 2 * l32) = f32_to_bf16_rne(acc[v]);
            else
                *(float*)(tile + r * ROW + 4 * l32) = acc[v];
        }
#pragma unroll
        for (int i = 0; i < PIECES / 64; ++i) {
            const int c = 64 * i + lane;
            const u32x4 val = *(const u32x4*)(tile + 16 * c);
            const int r = c / (ROW / 16), col = (c % (ROW / 16)) * (16 / ESZ);
            const int64_t idx = off + (int64_t)r * p.ldo + col;
            store_out((u32x4*)((uint8_t*)p.out + idx * ESZ), val);
        }
    }
}

// ---------------------------------------------------------------------------
template <int NTW, int S, int G>
static void launch_spmm_t(const SpmmArgs& a, bool out_bf16, int grid, int n_split, int waves, hipStream_t stream) {
    if constexpr (G == 1) {
        if (out_bf16)
            hipLaunchKernelGGL((spmm_kernel<NTW, S, true>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((spmm_kernel<NTW, S, false>), dim3(grid), dim3(256), 0, stream, a);
    } else if constexpr (NTW == 2) {
        // Eight waves (two per SIMD, 32*RW/2 x 64 outputs each), or four as the
        // plan fixed (not at RW = 8: four waves of 256 accumulators each spill
        // there); A fetched in entry pairs when C is a multiple of 64 (the plan
        // then starts every item at an even entry of its block).
        constexpr bool four_ok = G != 8;
        const bool four = four_ok && waves == 4;
        const bool pair = a.lda % 64 == 0;
#define BSP_WIDE(NW_, PAIR_)                                                                                  \
    do {                                                                                                      \
        if (out_bf16)                                                                                         \
            hipLaunchKernelGGL((spmm_group_wide_kernel<G, S, true, NW_, PAIR_>), dim3(grid), dim3(64 * NW_), 0, \
                               stream, a);                                                                    \
        else                                                                                                  \
            hipLaunchKernelGGL((spmm_group_wide_kernel<G, S, false, NW_, PAIR_>), dim3(grid), dim3(64 * NW_), 0, \
                               stream, a);                                                                    \
    } while (0)
        bool launched = false;
        if constexpr (four_ok) {
            if (four) {
                if (pair) BSP_WIDE(4, true);
                else BSP_WIDE(4, false);
                launched = true;
            }
        }
        if (!launched) {
            if (pair) BSP_WIDE(8, true);
            else BSP_WIDE(8, false);
        }
#undef BSP_WIDE
    } else {
        if (out_bf16)
            hipLaunchKernelGGL((spmm_group_kernel<G, S, true>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((spmm_group_kernel<G, S, false>), dim3(grid), dim3(256), 0, stream, a);
    }
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
#define BSP_SPMM_CASE(TN, S, G)                                                   \
    if (v.tile_n == TN && v.stages == S && v.group == G) {                       \
        launch_spmm_t<TN / 128, S, G>(a, out_bf16, grid, n_split, v.waves, stream); \
        return hipGetLastError();                                                \
    }
    BSP_SPMM_VARIANTS(BSP_SPMM_CASE)
#undef BSP_SPMM_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_spmm_stream(const SpmmStreamArgs& a, const SpmmStreamVariant& v, bool out_bf16, int grid,
                              hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
#define BSP_STREAM_CASE(TN, SB, SA, NB, PP, EPS, SR)                                                              \
    if (v.tile_n == TN && v.sb == SB && v.sa == SA && v.nbw == NB && v.pipes == PP && v.eps == EPS &&            \
        v.sr == SR) {                                                                                            \
        if (out_bf16)                                                                                            \
            hipLaunchKernelGGL((spmm_stream_kernel<TN / 128, SB, SA, NB, PP, true, EPS, SR>), dim3(grid),          \
                               dim3(64 * (4 * SR + 1 + NB) * PP), 0, stream, a);                                 \
        else                                                                                                     \
            hipLaunchKernelGGL((spmm_stream_kernel<TN / 128, SB, SA, NB, PP, false, EPS, SR>), dim3(grid),         \
                               dim3(64 * (4 * SR + 1 + NB) * PP), 0, stream, a);                                 \
        return hipGetLastError();                                                                                \
    }
    BSP_SPMM_STREAM_VARIANTS(BSP_STREAM_CASE)
#undef BSP_STREAM_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_spmm_sweep(const SpmmSweepArgs& a, bool out_bf16, int grid, hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    constexpr int NBW = kSweepWaves - 9;
    if (out_bf16)
        hipLaunchKernelGGL((spmm_sweep_kernel<kSweepStages, kSweepStages, NBW, true>), dim3(grid),
                           dim3(64 * kSweepWaves), 0, stream, a);
    else
        hipLaunchKernelGGL((spmm_sweep_kernel<kSweepStages, kSweepStages, NBW, false>), dim3(grid),
                           dim3(64 * kSweepWaves), 0, stream, a);
    return hipGetLastError();
}

template <int DK>
static void launch_attention_t(const AttentionArgs& a, bool out_bf16, int grid, int n_split, hipStream_t stream) {
    if (out_bf16)
        hipLaunchKernelGGL((attention_kernel<DK, kAttentionStages, true>), dim3(grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((attention_kernel<DK, kAttentionStages, false>), dim3(grid), dim3(256), 0, stream, a);
    if (n_split > 0) {
        const int g = n_split * a.s.n_tiles;
        if (out_bf16)
            hipLaunchKernelGGL((spmm_reduce_kernel<1, true>), dim3(g), dim3(256), 0, stream, a.s);
        else
            hipLaunchKernelGGL((spmm_reduce_kernel<1, false>), dim3(g), dim3(256), 0, stream, a.s);
    }
}

hipError_t launch_attention(const AttentionArgs& a, int head_dim, bool out_bf16, int grid, int n_split,
                            hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    switch (head_dim) {
        case 32: launch_attention_t<32>(a, out_bf16, grid, n_split, stream); break;
        case 64: launch_attention_t<64>(a, out_bf16, grid, n_split, stream); break;
        case 128: launch_attention_t<128>(a, out_bf16, grid, n_split, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool Y_COLMAJOR, bool OUT_BF16>
static void launch_sddmm_t(const SddmmArgs& a, int grid, hipStream_t stream) {
    // X operands stay in registers when every wave has at most two k-steps.
    if (a.K <= 4 * 32 * sddmm_detail::kKW)
        hipLaunchKernelGGL((sddmm_kernel<Y_COLMAJOR, OUT_BF16, true>), dim3(grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((sddmm_kernel<Y_COLMAJOR, OUT_BF16, false>), dim3(grid), dim3(256), 0, stream, a);
}

template <int K, bool MASK16>
static void launch_sddmm_shot_m(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid, hipStream_t stream) {
    if (y_colmajor) {
        if (out_bf16)
            hipLaunchKernelGGL((sddmm_shot_kernel<K, true, true, MASK16>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((sddmm_shot_kernel<K, true, false, MASK16>), dim3(grid), dim3(256), 0, stream, a);
    } else {
        if (out_bf16)
            hipLaunchKernelGGL((sddmm_shot_kernel<K, false, true, MASK16>), dim3(grid), dim3(256), 0, stream, a);
        else
            hipLaunchKernelGGL((sddmm_shot_kernel<K, false, false, MASK16>), dim3(grid), dim3(256), 0, stream, a);
    }
}

template <int K>
static void launch_sddmm_shot(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid, hipStream_t stream) {
    if (((uintptr_t)a.mask & 15u) == 0)
        launch_sddmm_shot_m<K, true>(a, y_colmajor, out_bf16, grid, stream);
    else
        launch_sddmm_shot_m<K, false>(a, y_colmajor, out_bf16, grid, stream);
}

hipError_t launch_sddmm(const SddmmArgs& a, bool y_colmajor, bool out_bf16, int grid,
                        hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    if (a.one_shot) {
        switch (a.K) {
            case 32: launch_sddmm_shot<32>(a, y_colmajor, out_bf16, grid, stream); break;
            case 64: launch_sddmm_shot<64>(a, y_colmajor, out_bf16, grid, stream); break;
            case 128: launch_sddmm_shot<128>(a, y_colmajor, out_bf16, grid, stream); break;
            default: launch_sddmm_shot<256>(a, y_colmajor, out_bf16, grid, stream); break;
        }
        return hipGetLastError();
    }
    if (y_colmajor) {
        if (out_bf16)
            launch_sddmm_t<true, true>(a, grid, stream);
        else
            launch_sddmm_t<true, false>(a, grid, stream);
    } else {
        if (out_bf16)
            launch_sddmm_t<false, true>(a, grid, stream);
        else
            launch_sddmm_t<false, false>(a, grid, stream);
    }
    return hipGetLastError();
}

template <int S>
static void launch_spgemm_t(const SpgemmArgs& a, bool out_bf16, int grid, hipStream_t stream) {
    if (out_bf16)
        hipLaunchKernelGGL((spgemm_kernel<S, true>), dim3(grid), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((spgemm_kernel<S, false>), dim3(grid), dim3(256), 0, stream, a);
}

hipError_t launch_spgemm(const SpgemmArgs& a, int stages, bool out_bf16, int grid, hipStream_t stream) {
    if (grid <= 0) return hipSuccess;
    switch (stages) {
        case 2: launch_spgemm_t<2>(a, out_bf16, grid, stream); break;
        case 3: launch_spgemm_t<3>(a, out_bf16, grid, stream); break;
        case 4: launch_spgemm_t<4>(a, out_bf16, grid, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace bsp

#ifdef BSP_TIMELINE
extern "C" int bsp_timeline_attach(void* buffer, int64_t capacity, int device) {
    if (capacity < 0 || (buffer == nullptr) != (capacity == 0)) return BSP_ERR_INVALID_ARGUMENT;
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != device) e = hipSetDevice(device);
    uint64_t* ptr = (uint64_t*)buffer;
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(bsp::g_timeline_buf), &ptr, sizeof(ptr));
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(bsp::g_timeline_cap), &capacity, sizeof(capacity));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    return e == hipSuccess ? BSP_OK : BSP_ERR_DEVICE;
}

extern "C" int bsp_timeline_clock_khz(int device, int* khz) {
    if (!khz) return BSP_ERR_INVALID_ARGUMENT;
    return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, device) == hipSuccess ? BSP_OK : BSP_ERR_DEVICE;
}
#endif
