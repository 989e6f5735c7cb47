// bsp_spmm_noalloc: SpMM without any device allocation, for callers that
// cannot allocate (serving loops that must not touch the allocator, harnesses
// that forbid hipMalloc).  It runs the persistent SpMM kernel of bsp_spmm with
// the kernel's schedule -- the per-workgroup head records, unit records and
// entry words that a plan uploads into memory it allocates -- staged instead in
// `scratch`, a file-scope device array of BSP_NOALLOC_SCRATCH_BYTES that every
// GPU the library runs on holds from module load to the end of the process.
//
// Set-up: the first call on a device takes the array's device address with
// that device current (hipGetSymbolAddress) and keeps it per device; host code
// passes that address, never the array's name, to the copy and the kernel.
// Each call validates the structure, builds the schedule on the host, copies
// it into the array on the caller's stream and waits for that copy (so the
// host staging buffer can be reused), then launches asynchronously.  The wait
// blocks the host on the caller's stream, so the call cannot be recorded into
// a HIP graph: on a stream under capture it returns BSP_ERR_UNSUPPORTED
// before touching the stream.  Nothing in the array needs to start
// at zero: every byte the kernel reads is written by the call's own copy.
// Calls on one GPU share the array and keep the last call's contents, so two
// calls that overlap on one GPU (different streams, or a launch still running
// when the next call's copy lands) race.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "bsp_kernels.hpp"
#include "bsp_schedule.hpp"
#include "bsparse.h"

namespace {

__device__ __align__(256) unsigned char scratch[BSP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned char* g_scratch[kMaxDevices] = {};

// The scratch array's address on `device` (taken once, with the device current).
int scratch_on(int device, unsigned char** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        int prev = -1;
        hipError_t e = hipGetDevice(&prev);
        if (e == hipSuccess && prev != device) e = hipSetDevice(device);
        void* ptr = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
        if (e != hipSuccess || !ptr)
            return bsp::record_error(BSP_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") +
                                                         hipGetErrorString(e));
        g_scratch[device] = (unsigned char*)ptr;
    }
    *out = g_scratch[device];
    return BSP_OK;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

template <typename T>
size_t put(std::vector<unsigned char>& buf, size_t off, const std::vector<T>& v) {
    if (!v.empty()) std::memcpy(buf.data() + off, v.data(), v.size() * sizeof(T));
    return align256(off + v.size() * sizeof(T));
}

}  // namespace

extern "C" int bsp_spmm_noalloc(const bsp_bsr_desc* a, const uint16_t* a_vals, const uint16_t* b, int64_t N,
                                int64_t ldb, void* c, int64_t ldc, int out_dtype, int device, void* stream) {
    if (!a) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "null BSR descriptor");
    {
        // The structure first: the variant choice and the schedule builder
        // below index host arrays by indptr and indices.
        std::string vmsg;
        const int vst = bsp::validate_bsr(a, vmsg);
        if (vst != BSP_OK) return bsp::record_error(vst, vmsg);
    }
    if (N <= 0) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "N must be positive");
    if (a->C % 32 != 0 || a->R % 32 != 0)
        return bsp::record_error(BSP_ERR_UNSUPPORTED, "R and C must be multiples of 32");
    if (out_dtype != BSP_DTYPE_F32 && out_dtype != BSP_DTYPE_BF16)
        return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "out_dtype must be BSP_DTYPE_F32 or BSP_DTYPE_BF16");
    if (!b || !c || (a->nblocks > 0 && !a_vals)) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "null device pointer");
    if (ldb < N || ldc < N) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "ldb and ldc must be >= N");
    if (ldb % 8 != 0) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "ldb must be a multiple of 8");
    if (ldb >= (int64_t(1) << 26)) return bsp::record_error(BSP_ERR_UNSUPPORTED, "ldb must be below 2^26");
    if (((uintptr_t)b & 15u) || (a_vals && ((uintptr_t)a_vals & 15u)))
        return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "A values and B must be 16-byte aligned");
    if ((uintptr_t)c % (out_dtype == BSP_DTYPE_BF16 ? 2 : 4))
        return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "C is misaligned");
    if (device < 0 || device >= kMaxDevices) return bsp::record_error(BSP_ERR_INVALID_ARGUMENT, "device out of range");
    if (N % 128 != 0)
        return bsp::record_error(BSP_ERR_UNSUPPORTED, "bsp_spmm_noalloc needs N a multiple of 128 (the persistent "
                                                      "kernel's tile); use a plan for other N");
    {
        // A lower bound of the schedule, checked before any device query: its
        // entry words alone (an int64 B word and a uint32 A word per 32x32
        // sub-block product and column tile), at the widest tile (256).
        const int64_t min_bytes = 12 * a->nblocks * (a->R / 32) * (a->C / 32) * (N / 256);
        if (min_bytes > (int64_t)BSP_NOALLOC_SCRATCH_BYTES)
            return bsp::record_error(BSP_ERR_UNSUPPORTED,
                                     "the schedule needs at least " + std::to_string((long long)min_bytes) +
                                         " bytes, above the " + std::to_string((long long)BSP_NOALLOC_SCRATCH_BYTES) +
                                         " bytes of the no-allocation scratch; use a plan");
    }

    // The device: present, not capturing on `stream` (the copy below waits on
    // the host), and its compute-unit count, for which the schedule is built.
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0 || device >= count)
        return bsp::record_error(BSP_ERR_DEVICE, "no HIP device " + std::to_string(device));
    int cus = 0;
    hipError_t qe = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (qe != hipSuccess || cus <= 0)
        return bsp::record_error(BSP_ERR_DEVICE, std::string("compute-unit count of device ") + std::to_string(device) +
                                                     ": " + hipGetErrorString(qe));
    {
        int prev = -1;
        hipError_t ce = hipGetDevice(&prev);
        if (ce == hipSuccess && prev != device) ce = hipSetDevice(device);
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (ce == hipSuccess) ce = hipStreamIsCapturing((hipStream_t)stream, &cap);
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
        if (ce != hipSuccess)
            return bsp::record_error(BSP_ERR_DEVICE, std::string("hipStreamIsCapturing: ") + hipGetErrorString(ce));
        if (cap != hipStreamCaptureStatusNone)
            return bsp::record_error(BSP_ERR_UNSUPPORTED, "bsp_spmm_noalloc waits for its schedule copy on the host and "
                                                          "cannot be captured in a HIP graph; use a plan (bsp_spmm)");
    }
    // The schedule, built on the host as a plan builds it (same variant
    // choice, but one pipeline per workgroup and one stripe per unit: a plan
    // that would take stripe pairs runs the default variant here, with the
    // same per-stripe summation order).  Blocks of R >= 64, which a plan may
    // run on the row-group kernels, run the persistent kernel here.
    bsp::SpmmStreamVariant sv = bsp::kSpmmStreamDefault;
    int wpc = 2;
    if (!bsp::choose_spmm_stream(a, N, cus, &sv, &wpc) || sv.pipes != 1 || sv.sr != 1) {
        sv = bsp::kSpmmStreamDefault;
        wpc = 2;
    }
    bsp::SpmmStream ss;
    std::string msg;
    int st = bsp::build_spmm_stream(a, N, cus, sv.tile_n, wpc, ss, msg, 0, 1);
    if (st != BSP_OK) return bsp::record_error(st, msg);
    const size_t o_units = align256(ss.heads.size() * sizeof(bsp::SpmmStreamHead));
    const size_t o_bw = align256(o_units + ss.units.size() * sizeof(bsp::SpmmStreamUnit));
    const size_t o_aw = align256(o_bw + ss.bw.size() * sizeof(int64_t));
    const size_t total = align256(o_aw + ss.aw.size() * sizeof(uint32_t));
    if (total > (size_t)BSP_NOALLOC_SCRATCH_BYTES)
        return bsp::record_error(BSP_ERR_UNSUPPORTED,
                                 "the schedule needs " + std::to_string(total) + " bytes, above the " +
                                     std::to_string((long long)BSP_NOALLOC_SCRATCH_BYTES) +
                                     " bytes of the no-allocation scratch; use a plan");

    unsigned char* base = nullptr;
    st = scratch_on(device, &base);
    if (st != BSP_OK) return st;
    // Host staging of the schedule in the scratch array's layout.
    std::vector<unsigned char> host(total);
    put(host, 0, ss.heads);
    put(host, o_units, ss.units);
    put(host, o_bw, ss.bw);
    put(host, o_aw, ss.aw);

    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != device) e = hipSetDevice(device);
    if (e == hipSuccess) e = hipMemcpyAsync(base, host.data(), total, hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    if (e == hipSuccess) {
        bsp::SpmmStreamArgs args{};
        args.a = a_vals;
        args.b = b;
        args.c = c;
        args.heads = (const bsp::SpmmStreamHead*)base;
        args.units = (const bsp::SpmmStreamUnit*)(base + o_units);
        args.bw = (const int64_t*)(base + o_bw);
        args.aw = (const uint32_t*)(base + o_aw);
        args.ldb = ldb;
        args.ldc = ldc;
        args.lda = (int32_t)a->C;
        args.N = (int32_t)N;
        e = bsp::launch_spmm_stream(args, sv, out_dtype == BSP_DTYPE_BF16, (int)ss.wgs.size(), (hipStream_t)stream);
    }
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return bsp::record_error(BSP_ERR_DEVICE, std::string("bsp_spmm_noalloc: ") + hipGetErrorString(e));
    return BSP_OK;
}
