// C ABI of libbsparse: plans, launches and the blocking host-buffer entry
// points.  See include/bsparse.h for the contract of each function.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "bsp_kernels.hpp"
#include "bsp_schedule.hpp"
#include "bsparse.h"
#ifdef BSP_TIMELINE
#include "bsparse_timeline.h"
static_assert(BSP_SKIP_SPARSE_READ == bsp::kSkipSparseRead && BSP_SKIP_DENSE_READ == bsp::kSkipDenseRead &&
                  BSP_SKIP_DENSE2_READ == bsp::kSkipDense2Read && BSP_SKIP_COMPUTE == bsp::kSkipCompute &&
                  BSP_SKIP_WRITE == bsp::kSkipWrite,
              "skip flags of bsparse_timeline.h and the kernels");
#endif

struct bsp_plan {
    int kind = 0;  // 1 SpMM, 2 SDDMM, 3 fused attention pair, 4 SpGEMM
    int device = 0;
    int out_dtype = BSP_DTYPE_F32;
    int layout = BSP_ROW_MAJOR;
    int64_t M = 0, K = 0, N = 0, R = 0, C = 0, nblocks = 0;
    bsp_plan_info info{};
    void* d_wgs = nullptr;  // per-workgroup records (SpmmWg / SddmmItem)
    int32_t* d_ent_row = nullptr;   // SDDMM: first column of Y per entry
    int64_t* d_ent_off = nullptr;   // SDDMM: output offset per entry; SpMM: packed entries
    bsp::SpmmSplit* d_splits = nullptr;
    float* d_ws = nullptr;
    // SpGEMM: B's block count and width, C's structure, product lists.
    int64_t b_nblocks = 0, BC = 0;
    std::vector<int32_t> out_indptr, out_indices;
    uint64_t* d_terms = nullptr;
    bsp::SpgemmRun* d_runs = nullptr;  // wave runs
    int32_t wg_per_xcd = 0;
    int32_t sddmm_one_shot = 0;  // SDDMM: the one-shot kernel runs this plan
    // SpMM persistent kernel: variant, unit records and A words (the B words
    // go in d_ent_off, the workgroup heads in d_wgs; d_apw with stripe pairs).
    bsp::SpmmStreamVariant stream_variant{};
    bsp::SpmmStreamUnit* d_units = nullptr;
    uint32_t* d_aw = nullptr;
    uint64_t* d_apw = nullptr;
    // SpMM sweep kernel (info.persistent == 3): sweep records (heads in
    // d_wgs, B words in d_ent_off, A words in d_aw).
    bsp::SpmmSweepRec* d_sweeps = nullptr;
};

namespace {

thread_local std::string g_last_error;

// Work left out of every launch from now on (the instrumented build's
// bsp_timeline_skip; always 0 in libbsparse.so).
#ifdef BSP_TIMELINE
std::atomic<int> g_skips{0};
int launch_skips() { return g_skips.load(std::memory_order_relaxed); }
#else
constexpr int launch_skips() { return 0; }
#endif

int fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return fail(e == hipErrorOutOfMemory ? BSP_ERR_OUT_OF_MEMORY : BSP_ERR_DEVICE, m);
}

// Makes `device` current for the lifetime of the guard.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int device) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != device) err = hipSetDevice(device);
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

template <typename T>
hipError_t upload(T** dst, const std::vector<T>& src) {
    size_t bytes = std::max<size_t>(1, src.size()) * sizeof(T);
    hipError_t e = hipMalloc((void**)dst, bytes);
    if (e != hipSuccess) return e;
    if (!src.empty()) e = hipMemcpy(*dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice);
    return e;
}

void free_plan_buffers(bsp_plan* p) {
    if (p->d_wgs) (void)hipFree(p->d_wgs);
    if (p->d_ent_row) (void)hipFree(p->d_ent_row);
    if (p->d_ent_off) (void)hipFree(p->d_ent_off);
    if (p->d_splits) (void)hipFree(p->d_splits);
    if (p->d_ws) (void)hipFree(p->d_ws);
    if (p->d_terms) (void)hipFree(p->d_terms);
    if (p->d_runs) (void)hipFree(p->d_runs);
    if (p->d_units) (void)hipFree(p->d_units);
    if (p->d_aw) (void)hipFree(p->d_aw);
    if (p->d_apw) (void)hipFree(p->d_apw);
    if (p->d_sweeps) (void)hipFree(p->d_sweeps);
    p->d_sweeps = nullptr;
    p->d_units = nullptr;
    p->d_aw = nullptr;
    p->d_apw = nullptr;
    p->d_terms = nullptr;
    p->d_runs = nullptr;
    p->d_wgs = nullptr;
    p->d_ent_row = nullptr;
    p->d_ent_off = nullptr;
    p->d_splits = nullptr;
    p->d_ws = nullptr;
}

int device_cus(int device, int* cus) {
    int n = 0;
    hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(CU count)");
    *cus = n > 0 ? n : 256;
    return BSP_OK;
}

int check_device(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) return fail(BSP_ERR_DEVICE, "no HIP device available");
    if (device < 0 || device >= count)
        return fail(BSP_ERR_INVALID_ARGUMENT, "device " + std::to_string(device) + " out of range");
    return BSP_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The kernels address one 32-row panel of a dense operand with 32-bit byte
// offsets from the panel's first row: 32 rows must span less than 4 GB.
constexpr int64_t kMaxLeadingDim = int64_t(1) << 26;

void fill_info_spmm(const bsp::SpmmSchedule& s, bsp_plan_info* info) {
    std::memset(info, 0, sizeof(*info));
    info->kind = 1;
    info->tile_n = s.tile_n;
    info->n_tiles = s.n_tiles;
    info->n_items = (int32_t)s.items.size();
    info->n_entries = (int32_t)s.ent_row.size();
    info->n_split_rows = s.n_split_rows;
    info->n_slots = s.n_slots;
    info->grid = (int32_t)s.wgmap.size();
    info->max_item_entries = s.max_item_entries;
    // Ring depth: the default for the tile width and row group, or a
    // supported override (BSP_SPMM_STAGES) for experiments.
    bsp::SpmmVariant v = bsp::spmm_default_variant(s.tile_n, s.group);
    if (const char* e = std::getenv("BSP_SPMM_STAGES")) {
        const bsp::SpmmVariant w{s.tile_n, std::atoi(e), s.group};
        if (bsp::spmm_variant_supported(w)) v = w;
    }
    info->stages = v.stages;
    info->step_entries = 1;
    info->stripes_per_unit = 1;
    info->group = s.group;
    // Row groups on 256-column tiles run eight waves (two per SIMD) unless
    // BSP_SPMM_WIDE_WAVES=4 asks for four (groups of 2 or 4 stripes only: four
    // waves holding 8 stripes spill); read here, once, so that a plan
    // launches the same kernel every time (a captured graph included).
    info->waves = 4;
    if (s.group > 1 && s.tile_n == 256) {
        const char* ww = std::getenv("BSP_SPMM_WIDE_WAVES");
        info->waves = (ww && std::atoi(ww) == 4 && s.group != 8) ? 4 : 8;
    }
    info->workspace_bytes =
        (int64_t)s.n_slots * s.n_tiles * bsp::spmm_partial_floats(s.tile_n) * (int64_t)sizeof(float);
}

void fill_info_sddmm(const bsp::SddmmSchedule& s, bsp_plan_info* info) {
    std::memset(info, 0, sizeof(*info));
    info->kind = 2;
    info->n_items = (int32_t)s.items.size();
    info->n_entries = (int32_t)s.ent_col.size();
    info->grid = (int32_t)s.wgmap.size();
    info->max_item_entries = s.max_item_entries;
}

}  // namespace

extern "C" {

int bsp_abi_version(void) { return BSP_ABI_VERSION; }

const char* bsp_status_string(int status) {
    switch (status) {
        case BSP_OK: return "ok";
        case BSP_ERR_INVALID_ARGUMENT: return "invalid argument";
        case BSP_ERR_BAD_STRUCTURE: return "malformed BSR structure";
        case BSP_ERR_UNSUPPORTED: return "unsupported";
        case BSP_ERR_DEVICE: return "device error";
        case BSP_ERR_OUT_OF_MEMORY: return "out of memory";
        default: return "unknown status";
    }
}

const char* bsp_last_error(void) { return g_last_error.c_str(); }

int bsp_validate_bsr(const bsp_bsr_desc* desc) {
    std::string msg;
    int st = bsp::validate_bsr(desc, msg);
    if (st != BSP_OK) return fail(st, msg);
    return BSP_OK;
}

int bsp_spmm_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, bsp_plan_info* info,
                      int32_t* items, int32_t* ent_row, int64_t* ent_off, int32_t* wgmap) {
    if (!info) return fail(BSP_ERR_INVALID_ARGUMENT, "info is null");
    bsp::SpmmSchedule s;
    std::string msg;
    int st = bsp::build_spmm_schedule(a, N, num_cus, s, msg);
    if (st != BSP_OK) return fail(st, msg);
    fill_info_spmm(s, info);
    if (items)
        for (size_t i = 0; i < s.items.size(); ++i) {
            const bsp::SpmmItem& t = s.items[i];
            int32_t* o = items + 6 * i;
            o[0] = t.row; o[1] = t.e_begin; o[2] = t.e_end; o[3] = t.slot; o[4] = t.base; o[5] = t.npieces;
        }
    if (ent_row && !s.ent_row.empty()) std::memcpy(ent_row, s.ent_row.data(), s.ent_row.size() * 4);
    if (ent_off && !s.ent_off.empty()) std::memcpy(ent_off, s.ent_off.data(), s.ent_off.size() * 8);
    if (wgmap && !s.wgmap.empty()) std::memcpy(wgmap, s.wgmap.data(), s.wgmap.size() * 4);
    return BSP_OK;
}

int bsp_spmm_sweep_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, int col_groups, bsp_plan_info* info,
                            int32_t* wgs, int32_t* sweeps, int64_t* bw, uint32_t* aw) {
    if (!info) return fail(BSP_ERR_INVALID_ARGUMENT, "info is null");
    bsp::SpmmSweep s;
    std::string msg;
    int st = bsp::build_spmm_sweep(a, N, num_cus, s, msg, col_groups);
    if (st != BSP_OK) return fail(st, msg);
    std::memset(info, 0, sizeof(*info));
    info->kind = 1;
    info->tile_n = bsp::kSweepTile;
    info->n_tiles = s.n_tiles;
    info->n_items = (int32_t)s.n_units;
    info->n_entries = (int32_t)s.n_entries;
    info->grid = (int32_t)s.wgs.size();
    info->max_item_entries = s.max_wg_entries;
    info->n_slots = (int32_t)(s.sweeps.size() - bsp::kStreamPad);
    info->stages = bsp::kSweepStages;
    info->group = s.col_groups;
    info->waves = bsp::kSweepWaves;
    info->persistent = 3;
    info->a_stages = bsp::kSweepStages;
    info->step_entries = 2;
    info->stripes_per_unit = 1;
    info->units_rotated = s.rotated;
    if (wgs)
        for (size_t g = 0; g < s.wgs.size(); ++g) {
            const bsp::SpmmSweepWg& w = s.wgs[g];
            int32_t* o = wgs + 4 * g;
            o[0] = w.w_begin; o[1] = w.n; o[2] = w.s_begin; o[3] = w.n_sweeps;
        }
    if (sweeps)
        for (int32_t r = 0; r < info->n_slots; ++r) {
            const bsp::SpmmSweepRec& rec = s.sweeps[(size_t)r];
            int32_t* o = sweeps + 33 * r;
            o[0] = rec.count;
            for (int j = 0; j < 16; ++j) {
                o[1 + j] = rec.half[j / 8].row[j % 8];
                o[17 + j] = rec.half[j / 8].n0[j % 8];
            }
        }
    if (bw && s.n_entries) std::memcpy(bw, s.bw.data(), (size_t)s.n_entries * 8);
    if (aw && s.n_entries) std::memcpy(aw, s.aw.data(), (size_t)s.n_entries * 4);
    return BSP_OK;
}

int bsp_sddmm_schedule(const bsp_bsr_desc* m, int64_t K, int num_cus, bsp_plan_info* info,
                       int32_t* items, int32_t* ent_row, int64_t* ent_off, int32_t* wgmap) {
    if (!info) return fail(BSP_ERR_INVALID_ARGUMENT, "info is null");
    bsp::SddmmSchedule s;
    std::string msg;
    int st = bsp::build_sddmm_schedule(m, K, num_cus, s, msg);
    if (st != BSP_OK) return fail(st, msg);
    fill_info_sddmm(s, info);
    if (items)
        for (size_t i = 0; i < s.items.size(); ++i) {
            const bsp::SddmmItem& t = s.items[i];
            int32_t* o = items + 6 * i;
            o[0] = t.x_row0; o[1] = t.e_begin; o[2] = t.e_end; o[3] = 0; o[4] = 0; o[5] = 0;
        }
    if (ent_row && !s.ent_col.empty()) std::memcpy(ent_row, s.ent_col.data(), s.ent_col.size() * 4);
    if (ent_off && !s.ent_off.empty()) std::memcpy(ent_off, s.ent_off.data(), s.ent_off.size() * 8);
    if (wgmap && !s.wgmap.empty()) std::memcpy(wgmap, s.wgmap.data(), s.wgmap.size() * 4);
    return BSP_OK;
}

}  // extern "C"

namespace {

int64_t env_int(const char* name, int64_t dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    long long x = std::strtoll(v, &end, 10);
    return (end && *end == 0) ? (int64_t)x : dflt;
}

}  // namespace

namespace bsp {

// Whether an SpMM plan takes the sweep kernel (see bsp_kernels.hpp).  It is
// taken only when asked for (BSP_SPMM_SWEEP=2: whenever the shape allows; 1:
// for 32x32 blocks, a structure the persistent kernel would run as single
// stripes, at least 8 units per compute unit and B of at least 8 MB).  It
// cuts the skewed 16384^2 x 1024 workload's HBM-side reads from 189 to 111 MB
// but runs it in 69-88 us against the persistent kernel's 37, so no plan
// takes it by default.
bool choose_spmm_sweep(const bsp_bsr_desc* a, int64_t N, int cus) {
    const int64_t mode = env_int("BSP_SPMM_SWEEP", 0);
    if (mode == 0) return false;
    if (a->R % bsp::kSub || a->C % bsp::kSub || N <= 0 || N % bsp::kSweepTile || N >= bsp::kSweepMaxN) return false;
    if (a->nblocks * a->R * a->C / bsp::kSub > UINT32_MAX) return false;
    if (mode == 2) return true;
    if (std::getenv("BSP_SPMM_STREAM_VARIANT")) return false;  // a persistent variant was asked for
    if (a->R != bsp::kSub || a->C != bsp::kSub) return false;
    const int64_t units = (a->H / bsp::kSub) * (N / bsp::kSweepTile);
    if (units < 8 * (int64_t)cus || a->W * N * 2 < (int64_t(8) << 20)) return false;
    bsp::SpmmStreamVariant sv{};
    int wpc = 1;
    if (!choose_spmm_stream(a, N, cus, &sv, &wpc)) return false;
    return sv.sr == 1;
}

// Whether an SpMM plan runs the persistent kernel, and which variant.  It
// takes blocks whose stripes do not form row groups (row groups share each B
// panel among the stripes of a block row, which the per-item group kernels
// exploit) and N a multiple of 128.  BSP_SPMM_STREAM=0 turns it off;
// BSP_SPMM_STREAM_VARIANT="tile,sb,sa,nbw[,pipes[,entries per step]]" picks
// another compiled variant and BSP_SPMM_STREAM_WPC the workgroups per compute
// unit (all read here, at plan creation).  A two-pipeline variant runs one
// workgroup per compute unit.
bool choose_spmm_stream(const bsp_bsr_desc* a, int64_t N, int cus, SpmmStreamVariant* sv, int* wpc) {
    if (env_int("BSP_SPMM_STREAM", 1) == 0) return false;
    if (N % 128 != 0) return false;
    const int64_t group = env_int("BSP_SPMM_GROUP", bsp::spmm_choose_group(a->R, a->H, N, cus));
    if (group > 1 && (a->R / bsp::kSub) % group == 0) return false;
    bsp::SpmmStreamVariant v = bsp::kSpmmStreamDefault;
    // Stripe pairs (32x32 blocks): one workgroup per compute unit streams a
    // pair's union of block columns, an 8 KB B slice per entry with one or two
    // 2 KB A blocks, where single stripes stream 10 KB per block.  Estimated
    // per compute unit: single = 10 KB x max(blocks x tiles / CUs, longest
    // row); pairs = 1.2 x (8 + 2 x blocks / union entries) KB x max(union
    // entries x tiles / CUs, largest union), the 1.2 being what one workgroup
    // per compute unit costs.  Pairs are taken when they come out cheaper.
    // The estimate orders every measured structure (4096^2 x 512, pairs :
    // single us): identical rows of 51 blocks 14.3-14.9 : 18.3-19.4; banded
    // rows of 4 / 16 / 32 / 64 blocks 5.5 / 8.7-9.1 / 12.0-12.2 / 19.9-20.4 :
    // 5.8-6.1 / 9.6 / 14.4-14.6 / 23.1-25.0; identical pairs of rows of 20-60
    // blocks 15.7-15.8 : 15.5-15.7 (the largest union sets the end);
    // uniform-random 25% / 50% 16.4-16.7 / 23.7-23.9 : 13.1-13.4 / 21.5-22.8.
    // BSP_SPMM_PAIRS=0 turns them off, 2 takes them whenever the structure
    // allows.
    // (The pairing's overlap table is quadratic in the block rows: at most
    // 1024 of them, and only when the pairs could fill the compute units.)
    const int64_t pairs_mode = env_int("BSP_SPMM_PAIRS", 1);
    bool pairs_ok = false;
    const int64_t pair_units = (a->H / bsp::kSub + 1) / 2 * (N / 128);
    if (pairs_mode > 0 && N % 128 == 0 && (pairs_mode == 2 || pair_units >= (int64_t)cus)) {
        std::vector<std::pair<int32_t, int32_t>> pl;
        int64_t shared = 0, max_union = 0;
        if (bsp::spmm_stripe_pairs(a, bsp::kPairMaxRows, pl, &shared, &max_union)) {
            const double tiles = (double)(N / 128), nb = (double)a->nblocks;
            const double uni = nb - (double)shared;  // union entries over all pairs
            int64_t longest = 0;
            for (int64_t i = 0; i < a->H / bsp::kSub; ++i)
                longest = std::max<int64_t>(longest, a->indptr[i + 1] - a->indptr[i]);
            const double single = 10.0 * std::max(nb * tiles / cus, (double)longest);
            const double paired =
                uni > 0 ? 1.2 * (8.0 + 2.0 * nb / uni) * std::max(uni * tiles / cus, (double)max_union) : single;
            pairs_ok = pairs_mode == 2 || paired < single;
        }
    }
    const char* forced = std::getenv("BSP_SPMM_STREAM_VARIANT");
    if (forced) {
        bsp::SpmmStreamVariant w{};
        const int got = std::sscanf(forced, "%d,%d,%d,%d,%d,%d,%d", &w.tile_n, &w.sb, &w.sa, &w.nbw, &w.pipes, &w.eps,
                                    &w.sr);
        if (got < 5) w.pipes = 1;
        if (got < 6) w.eps = 1;
        if (got < 7) w.sr = 1;
        if (got >= 4 && bsp::spmm_stream_variant_supported(w) && N % w.tile_n == 0 && (w.sr == 1 || pairs_ok)) v = w;
    }
    int w = -1;
    if (!forced && pairs_ok) {
        v = bsp::kSpmmStreamPairs;
        w = 1;
    }
    // Many units per workgroup with some longer than a workgroup's share (a
    // skewed row distribution): one workgroup per compute unit with four B
    // loaders and deep rings streams the compute unit's units back to back,
    // where two workgroups would leave one of them running alone behind its
    // longest unit.  (Zipf(1.2) 16384^2 x 1024: 40.6-41.0 us with two
    // workgroups, 37.7-38.2 with this variant; with one unit per workgroup,
    // as at uniform 1-50%, two workgroups stay faster: 25% 14.2 against 16.0
    // us.)
    if (!forced && !pairs_ok && a->R == bsp::kSub) {
        const int64_t n_tiles = N / 128, stripes = a->H / bsp::kSub;
        int64_t longest = 0;
        for (int64_t i = 0; i < a->H / a->R; ++i) longest = std::max<int64_t>(longest, a->indptr[i + 1] - a->indptr[i]);
        longest *= a->C / bsp::kSub;
        const int64_t total = a->nblocks * (a->C / bsp::kSub) * n_tiles;
        const int64_t wgs = 2 * (int64_t)cus;
        if (stripes * n_tiles >= 4 * wgs && longest * wgs > total) {
            v = bsp::kSpmmStreamSkewed;
            w = 1;
        }
    }
    const int lds = bsp::spmm_stream_lds_bytes(v);
    if (w < 0) w = v.pipes > 1 ? 1 : std::max(1, std::min(2, bsp::kLdsBytesPerCu / lds));
    if (v.pipes == 1 && v.sr == 1) w = (int)env_int("BSP_SPMM_STREAM_WPC", w);
    if (v.sr == 2) w = 1;  // one unit (a stripe pair) per compute unit
    if (w < 1 || w * lds > bsp::kLdsBytesPerCu) w = 1;
    *sv = v;
    *wpc = w;
    return true;
}

int record_error(int status, const std::string& msg) { return fail(status, msg); }

}  // namespace bsp

namespace {

// Plan of the persistent SpMM kernel: per-workgroup unit lists and entry
// streams, uploaded once.
int make_spmm_stream_plan(bsp_plan** out, const bsp_bsr_desc* a, int64_t N, int out_dtype, int device, int cus,
                          const bsp::SpmmStreamVariant& sv, int wpc) {
    std::string msg;
    bsp::SpmmStream ss;
    const int cg = (int)env_int("BSP_SPMM_XCD_COLS", 0);
    int st = bsp::build_spmm_stream(a, N, cus, sv.tile_n, wpc, ss, msg, cg, sv.pipes, sv.sr == 2);
    if (st != BSP_OK) return fail(st, msg);
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp_plan* p = new bsp_plan();
    p->kind = 1;
    p->device = device;
    p->out_dtype = out_dtype;
    p->layout = BSP_ROW_MAJOR;
    p->M = a->H;
    p->K = a->W;
    p->N = N;
    p->R = a->R;
    p->C = a->C;
    p->nblocks = a->nblocks;
    p->stream_variant = sv;
    bsp_plan_info& in = p->info;
    std::memset(&in, 0, sizeof(in));
    in.kind = 1;
    in.tile_n = ss.tile_n;
    in.n_tiles = ss.n_tiles;
    in.n_items = (int32_t)(ss.units.size() - bsp::kStreamPad);
    in.n_entries = (int32_t)ss.n_entries;
    in.grid = (int32_t)(ss.wgs.size() / sv.pipes);
    in.max_item_entries = ss.max_wg_entries;
    in.stages = sv.sb;
    in.group = 1;
    in.waves = (4 * sv.sr + 1 + sv.nbw) * sv.pipes;
    in.persistent = sv.pipes;
    in.a_stages = sv.sa;
    in.step_entries = sv.eps;
    in.stripes_per_unit = sv.sr;
    in.units_rotated = ss.rotated;
    hipError_t e = upload((bsp::SpmmStreamHead**)&p->d_wgs, ss.heads);
    if (e == hipSuccess) e = upload(&p->d_units, ss.units);
    if (e == hipSuccess) e = upload(&p->d_ent_off, ss.bw);
    if (e == hipSuccess) e = ss.pairs ? upload(&p->d_apw, ss.apw) : upload(&p->d_aw, ss.aw);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_plan_buffers(p);
        delete p;
        return hip_fail(e, "SpMM plan upload");
    }
    *out = p;
    return BSP_OK;
}

// Plan of the sweep SpMM kernel: per-workgroup sweeps of up to 16 units and
// their entries merged by first row of B.
int make_spmm_sweep_plan(bsp_plan** out, const bsp_bsr_desc* a, int64_t N, int out_dtype, int device, int cus) {
    std::string msg;
    bsp::SpmmSweep sw;
    const int cg = (int)env_int("BSP_SPMM_XCD_COLS", 0);
    int st = bsp::build_spmm_sweep(a, N, cus, sw, msg, cg);
    if (st != BSP_OK) return fail(st, msg);
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp_plan* p = new bsp_plan();
    p->kind = 1;
    p->device = device;
    p->out_dtype = out_dtype;
    p->layout = BSP_ROW_MAJOR;
    p->M = a->H;
    p->K = a->W;
    p->N = N;
    p->R = a->R;
    p->C = a->C;
    p->nblocks = a->nblocks;
    bsp_plan_info& in = p->info;
    std::memset(&in, 0, sizeof(in));
    in.kind = 1;
    in.tile_n = bsp::kSweepTile;
    in.n_tiles = sw.n_tiles;
    in.n_items = (int32_t)sw.n_units;
    in.n_entries = (int32_t)sw.n_entries;
    in.grid = (int32_t)sw.wgs.size();
    in.max_item_entries = sw.max_wg_entries;
    in.stages = bsp::kSweepStages;
    in.group = 1;
    in.waves = bsp::kSweepWaves;
    in.persistent = 3;
    in.a_stages = bsp::kSweepStages;
    in.step_entries = 2;
    in.stripes_per_unit = 1;
    in.units_rotated = sw.rotated;
    hipError_t e = upload((bsp::SpmmSweepHead**)&p->d_wgs, sw.heads);
    if (e == hipSuccess) e = upload(&p->d_sweeps, sw.sweeps);
    if (e == hipSuccess) e = upload(&p->d_ent_off, sw.bw);
    if (e == hipSuccess) e = upload(&p->d_aw, sw.aw);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_plan_buffers(p);
        delete p;
        return hip_fail(e, "SpMM plan upload");
    }
    *out = p;
    return BSP_OK;
}

// Plan of an SpMM-shaped launch (SpMM, or the fused attention pair with the
// mask as A and N = head dimension): schedule, upload, split-row scratch.
int make_spmm_plan(bsp_plan** out, int kind, const bsp_bsr_desc* a, int64_t N, int out_dtype, int device,
                   int force_tile_n) {
    std::string msg;
    int st = bsp::validate_bsr(a, msg);
    if (st != BSP_OK) return fail(st, msg);
    st = check_device(device);
    if (st != BSP_OK) return st;
    int cus = 256;
    st = device_cus(device, &cus);
    if (st != BSP_OK) return st;
    if (kind == 1) {
        if (bsp::choose_spmm_sweep(a, N, cus)) return make_spmm_sweep_plan(out, a, N, out_dtype, device, cus);
        bsp::SpmmStreamVariant sv{};
        int wpc = 1;
        if (bsp::choose_spmm_stream(a, N, cus, &sv, &wpc)) return make_spmm_stream_plan(out, a, N, out_dtype, device, cus, sv, wpc);
    }
    bsp::SpmmSchedule s;
    st = bsp::build_spmm_schedule(a, N, cus, s, msg, force_tile_n, kind == 3 ? 1 : 0);
    if (st != BSP_OK) return fail(st, msg);

    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp_plan* p = new bsp_plan();
    p->kind = kind;
    p->device = device;
    p->out_dtype = out_dtype;
    p->layout = BSP_ROW_MAJOR;
    p->M = a->H;
    p->K = a->W;
    p->N = N;
    p->R = a->R;
    p->C = a->C;
    p->nblocks = a->nblocks;
    fill_info_spmm(s, &p->info);
    if (kind == 3) {
        p->info.kind = 3;
        p->info.stages = bsp::kAttentionStages;
    }
    hipError_t e = upload((bsp::SpmmWg**)&p->d_wgs, bsp::spmm_wg_records(s));
    if (e == hipSuccess) e = upload(&p->d_ent_off, bsp::spmm_packed_entries(s));
    if (e == hipSuccess) e = upload(&p->d_splits, bsp::spmm_splits(s));
    if (e == hipSuccess && s.n_slots > 0) {
        const size_t nf = (size_t)s.n_slots * s.n_tiles * bsp::spmm_partial_floats(s.tile_n);
        e = hipMalloc((void**)&p->d_ws, nf * sizeof(float));
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_plan_buffers(p);
        delete p;
        return hip_fail(e, kind == 3 ? "attention plan upload" : "SpMM plan upload");
    }
    *out = p;
    return BSP_OK;
}

// Kernel arguments of an SpMM-shaped plan.
bsp::SpmmArgs spmm_args(const bsp_plan* p, const uint16_t* a_vals, const uint16_t* b, int64_t ldb, void* c,
                        int64_t ldc) {
    bsp::SpmmArgs args{};
    args.a = a_vals;
    args.b = b;
    args.c = c;
    args.wgs = (const bsp::SpmmWg*)p->d_wgs;
    args.ents = p->d_ent_off;
    args.splits = p->d_splits;
    args.ws = p->d_ws;
    args.ldb = ldb;
    args.ldc = ldc;
    args.lda = (int32_t)p->C;
    args.n_tiles = p->info.n_tiles;
    args.N = (int32_t)p->N;
    args.skips = launch_skips();
    return args;
}

}  // namespace

extern "C" {

int bsp_spmm_plan_create(bsp_plan** out, const bsp_bsr_desc* a, int64_t N, int b_layout,
                         int out_dtype, int device) {
    if (!out) return fail(BSP_ERR_INVALID_ARGUMENT, "plan output pointer is null");
    *out = nullptr;
    if (out_dtype != BSP_DTYPE_F32 && out_dtype != BSP_DTYPE_BF16)
        return fail(BSP_ERR_INVALID_ARGUMENT, "out_dtype must be BSP_DTYPE_F32 or BSP_DTYPE_BF16");
    if (b_layout != BSP_ROW_MAJOR && b_layout != BSP_COL_MAJOR)
        return fail(BSP_ERR_INVALID_ARGUMENT, "b_layout must be BSP_ROW_MAJOR or BSP_COL_MAJOR");
    if (b_layout != BSP_ROW_MAJOR)
        return fail(BSP_ERR_UNSUPPORTED, "SpMM takes B row-major (the reference's layout)");
    return make_spmm_plan(out, 1, a, N, out_dtype, device, 0);
}

int bsp_spmm(const bsp_plan* p, const uint16_t* a_vals, const uint16_t* b, int64_t ldb, void* c,
             int64_t ldc, void* stream) {
    if (!p || p->kind != 1) return fail(BSP_ERR_INVALID_ARGUMENT, "not an SpMM plan");
    if (!b || !c || (p->nblocks > 0 && !a_vals))
        return fail(BSP_ERR_INVALID_ARGUMENT, "null device pointer");
    if (ldb < p->N || ldc < p->N) return fail(BSP_ERR_INVALID_ARGUMENT, "ldb and ldc must be >= N");
    if (ldb % 8 != 0) return fail(BSP_ERR_INVALID_ARGUMENT, "ldb must be a multiple of 8");
    if (ldb >= kMaxLeadingDim) return fail(BSP_ERR_UNSUPPORTED, "ldb must be below 2^26");
    if (!aligned16(b) || (a_vals && !aligned16(a_vals)))
        return fail(BSP_ERR_INVALID_ARGUMENT, "A values and B must be 16-byte aligned");
    const size_t esz = p->out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    if (((uintptr_t)c % esz) != 0) return fail(BSP_ERR_INVALID_ARGUMENT, "C is misaligned");
    DeviceGuard g(p->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    const bsp::SpmmArgs args = spmm_args(p, a_vals, b, ldb, c, ldc);
    // Work can be left out (the instrumented build) of the persistent, sweep
    // and 256-column row-group kernels only.
    if (args.skips != 0 && !p->info.persistent && !(p->info.group > 1 && p->info.tile_n == 256))
        return fail(BSP_ERR_UNSUPPORTED, "this plan's kernel has no switches to leave work out");
    hipError_t e;
    if (p->info.persistent == 3) {
        bsp::SpmmSweepArgs sa{};
        sa.a = a_vals;
        sa.b = b;
        sa.c = c;
        sa.heads = (const bsp::SpmmSweepHead*)p->d_wgs;
        sa.sweeps = p->d_sweeps;
        sa.bw = p->d_ent_off;
        sa.aw = p->d_aw;
        sa.ldb = ldb;
        sa.ldc = ldc;
        sa.lda = (int32_t)p->C;
        sa.N = (int32_t)p->N;
        sa.skips = args.skips;
        e = bsp::launch_spmm_sweep(sa, p->out_dtype == BSP_DTYPE_BF16, p->info.grid, (hipStream_t)stream);
    } else if (p->info.persistent) {
        bsp::SpmmStreamArgs sa{};
        sa.a = a_vals;
        sa.b = b;
        sa.c = c;
        sa.heads = (const bsp::SpmmStreamHead*)p->d_wgs;
        sa.units = p->d_units;
        sa.bw = p->d_ent_off;
        sa.aw = p->d_aw;
        sa.apw = p->d_apw;
        sa.ldb = ldb;
        sa.ldc = ldc;
        sa.lda = (int32_t)p->C;
        sa.N = (int32_t)p->N;
        sa.skips = args.skips;
        e = bsp::launch_spmm_stream(sa, p->stream_variant, p->out_dtype == BSP_DTYPE_BF16, p->info.grid,
                                    (hipStream_t)stream);
    } else {
        const bsp::SpmmVariant v{p->info.tile_n, p->info.stages, p->info.group, p->info.waves};
        e = bsp::launch_spmm(args, v, p->out_dtype == BSP_DTYPE_BF16, p->info.grid, p->info.n_split_rows,
                             (hipStream_t)stream);
    }
    if (e != hipSuccess) return hip_fail(e, "SpMM launch");
    return BSP_OK;
}

int bsp_attention_plan_create(bsp_plan** out, const bsp_bsr_desc* mask, int64_t head_dim, int out_dtype,
                              int device) {
    if (!out) return fail(BSP_ERR_INVALID_ARGUMENT, "plan output pointer is null");
    *out = nullptr;
    if (out_dtype != BSP_DTYPE_F32 && out_dtype != BSP_DTYPE_BF16)
        return fail(BSP_ERR_INVALID_ARGUMENT, "out_dtype must be BSP_DTYPE_F32 or BSP_DTYPE_BF16");
    if (!bsp::attention_head_dim_supported(head_dim))
        return fail(BSP_ERR_UNSUPPORTED, "head_dim must be 32, 64 or 128");
    return make_spmm_plan(out, 3, mask, head_dim, out_dtype, device, bsp::kAttentionTileN);
}

int bsp_attention(const bsp_plan* p, const uint16_t* mask_vals, const uint16_t* q, int64_t ldq,
                  const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, void* out, int64_t ldo,
                  void* stream) {
    if (!p || p->kind != 3) return fail(BSP_ERR_INVALID_ARGUMENT, "not an attention plan");
    if (!q || !k || !v || !out || (p->nblocks > 0 && !mask_vals))
        return fail(BSP_ERR_INVALID_ARGUMENT, "null device pointer");
    const int64_t d = p->N;
    if (ldq < d || ldk < d || ldv < d || ldo < d)
        return fail(BSP_ERR_INVALID_ARGUMENT, "leading dimensions must be >= head_dim");
    if (ldq % 8 || ldk % 8 || ldv % 8)
        return fail(BSP_ERR_INVALID_ARGUMENT, "ldq, ldk and ldv must be multiples of 8");
    if (ldk >= kMaxLeadingDim || ldv >= kMaxLeadingDim)
        return fail(BSP_ERR_UNSUPPORTED, "ldk and ldv must be below 2^26");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (mask_vals && !aligned16(mask_vals)))
        return fail(BSP_ERR_INVALID_ARGUMENT, "mask values, Q, K and V must be 16-byte aligned");
    const size_t esz = p->out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    if (((uintptr_t)out % esz) != 0) return fail(BSP_ERR_INVALID_ARGUMENT, "output is misaligned");
    DeviceGuard g(p->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp::AttentionArgs args{};
    args.s = spmm_args(p, mask_vals, v, ldv, out, ldo);
    if (args.s.skips != 0) return fail(BSP_ERR_UNSUPPORTED, "the attention kernel has no switches to leave work out");
    args.q = q;
    args.k = k;
    args.ldq = ldq;
    args.ldk = ldk;
    hipError_t e = bsp::launch_attention(args, (int)d, p->out_dtype == BSP_DTYPE_BF16, p->info.grid,
                                         p->info.n_split_rows, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "attention launch");
    return BSP_OK;
}

int bsp_sddmm_plan_create(bsp_plan** out, const bsp_bsr_desc* mask, int64_t K, int y_layout,
                          int out_dtype, int device) {
    if (!out) return fail(BSP_ERR_INVALID_ARGUMENT, "plan output pointer is null");
    *out = nullptr;
    if (out_dtype != BSP_DTYPE_F32 && out_dtype != BSP_DTYPE_BF16)
        return fail(BSP_ERR_INVALID_ARGUMENT, "out_dtype must be BSP_DTYPE_F32 or BSP_DTYPE_BF16");
    if (y_layout != BSP_ROW_MAJOR && y_layout != BSP_COL_MAJOR)
        return fail(BSP_ERR_INVALID_ARGUMENT, "y_layout must be BSP_ROW_MAJOR or BSP_COL_MAJOR");
    std::string msg;
    int st = bsp::validate_bsr(mask, msg);
    if (st != BSP_OK) return fail(st, msg);
    st = check_device(device);
    if (st != BSP_OK) return st;
    int cus = 256;
    st = device_cus(device, &cus);
    if (st != BSP_OK) return st;
    bsp::SddmmSchedule s;
    st = bsp::build_sddmm_schedule(mask, K, cus, s, msg);
    if (st != BSP_OK) return fail(st, msg);

    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp_plan* p = new bsp_plan();
    p->kind = 2;
    p->device = device;
    p->out_dtype = out_dtype;
    p->layout = y_layout;
    p->M = mask->H;
    p->N = mask->W;
    p->K = K;
    p->R = mask->R;
    p->C = mask->C;
    p->nblocks = mask->nblocks;
    fill_info_sddmm(s, &p->info);
    // BSP_SDDMM_LOOP selects the looped kernel for every K (for comparison).
    p->sddmm_one_shot = bsp::sddmm_shot_supported(K, s.max_item_entries) && !std::getenv("BSP_SDDMM_LOOP");
    p->info.stages = p->sddmm_one_shot ? 1 : 0;
    hipError_t e = upload((bsp::SddmmItem**)&p->d_wgs, bsp::sddmm_wg_records(s));
    if (e == hipSuccess) e = upload(&p->d_ent_row, s.ent_col);
    if (e == hipSuccess) e = upload(&p->d_ent_off, s.ent_off);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_plan_buffers(p);
        delete p;
        return hip_fail(e, "SDDMM plan upload");
    }
    *out = p;
    return BSP_OK;
}

int bsp_sddmm(const bsp_plan* p, const uint16_t* mask_vals, const uint16_t* x, int64_t ldx,
              const uint16_t* y, int64_t ldy, void* out_vals, void* stream) {
    if (!p || p->kind != 2) return fail(BSP_ERR_INVALID_ARGUMENT, "not an SDDMM plan");
    if (p->nblocks == 0) return BSP_OK;
    if (!mask_vals || !x || !y || !out_vals) return fail(BSP_ERR_INVALID_ARGUMENT, "null device pointer");
    if (ldx < p->K) return fail(BSP_ERR_INVALID_ARGUMENT, "ldx must be >= K");
    if (p->layout == BSP_ROW_MAJOR ? ldy < p->N : ldy < p->K)
        return fail(BSP_ERR_INVALID_ARGUMENT, "ldy too small for Y's layout");
    if (ldx % 8 != 0 || ldy % 8 != 0)
        return fail(BSP_ERR_INVALID_ARGUMENT, "ldx and ldy must be multiples of 8");
    if (!aligned16(x) || !aligned16(y))
        return fail(BSP_ERR_INVALID_ARGUMENT, "X and Y must be 16-byte aligned");
    const size_t esz = p->out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    if (((uintptr_t)out_vals % esz) != 0 || ((uintptr_t)mask_vals % 2) != 0)
        return fail(BSP_ERR_INVALID_ARGUMENT, "output or mask values misaligned");
    DeviceGuard g(p->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp::SddmmArgs args{};
    args.mask = mask_vals;
    args.x = x;
    args.y = y;
    args.out = out_vals;
    args.wgs = (const bsp::SddmmItem*)p->d_wgs;
    args.ent_col = p->d_ent_row;
    args.ent_off = p->d_ent_off;
    args.ldx = ldx;
    args.ldy = ldy;
    args.ldo = (int32_t)p->C;
    args.K = (int32_t)p->K;
    args.one_shot = p->sddmm_one_shot;
    args.skips = launch_skips();
    if (args.skips != 0 && !args.one_shot)
        return fail(BSP_ERR_UNSUPPORTED, "this plan's kernel has no switches to leave work out");
    hipError_t e = bsp::launch_sddmm(args, p->layout == BSP_COL_MAJOR,
                                     p->out_dtype == BSP_DTYPE_BF16, p->info.grid,
                                     (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "SDDMM launch");
    return BSP_OK;
}

int bsp_spgemm_symbolic(const bsp_bsr_desc* a, const bsp_bsr_desc* b, int64_t* nblocks, int32_t* indptr,
                        int32_t* indices) {
    if (!nblocks) return fail(BSP_ERR_INVALID_ARGUMENT, "nblocks is null");
    std::vector<int32_t> ip, ix;
    std::string msg;
    int st = bsp::spgemm_symbolic(a, b, ip, ix, msg);
    if (st != BSP_OK) return fail(st, msg);
    *nblocks = (int64_t)ix.size();
    if (indptr) std::memcpy(indptr, ip.data(), ip.size() * sizeof(int32_t));
    if (indices && !ix.empty()) std::memcpy(indices, ix.data(), ix.size() * sizeof(int32_t));
    return BSP_OK;
}

int bsp_spgemm_plan_create(bsp_plan** out, const bsp_bsr_desc* a, const bsp_bsr_desc* b, int out_dtype,
                           int device) {
    if (!out) return fail(BSP_ERR_INVALID_ARGUMENT, "plan output pointer is null");
    *out = nullptr;
    if (out_dtype != BSP_DTYPE_F32 && out_dtype != BSP_DTYPE_BF16)
        return fail(BSP_ERR_INVALID_ARGUMENT, "out_dtype must be BSP_DTYPE_F32 or BSP_DTYPE_BF16");
    // Argument and structure errors first (no device needed), then the device.
    std::vector<int32_t> ip, ix;
    std::string msg;
    int st = bsp::spgemm_symbolic(a, b, ip, ix, msg);
    if (st != BSP_OK) return fail(st, msg);
    st = check_device(device);
    if (st != BSP_OK) return st;
    int cus = 256;
    st = device_cus(device, &cus);
    if (st != BSP_OK) return st;
    int stages = bsp::kSpgemmStages;
    if (const char* e = std::getenv("BSP_SPGEMM_STAGES"))
        if (bsp::spgemm_stages_supported(std::atoi(e))) stages = std::atoi(e);
    // Two runs per resident wave: the second round's start overlaps the
    // first round's tail (8192^2, 5% x 5%: 29.4 -> 28.2 us fp32).
    int rounds = 2;
    if (const char* e = std::getenv("BSP_SPGEMM_ROUNDS")) rounds = std::atoi(e);
    bsp::SpgemmSchedule s;
    st = bsp::build_spgemm_schedule(a, b, cus, stages, rounds, s, msg);
    if (st != BSP_OK) return fail(st, msg);

    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp_plan* p = new bsp_plan();
    p->kind = 4;
    p->device = device;
    p->out_dtype = out_dtype;
    p->M = a->H;
    p->K = a->W;
    p->N = b->W;
    p->R = a->R;
    p->C = a->C;
    p->BC = b->C;
    p->nblocks = a->nblocks;
    p->b_nblocks = b->nblocks;
    p->out_indptr = std::move(s.indptr);
    p->out_indices = std::move(s.indices);
    bsp_plan_info& info = p->info;
    info.kind = 4;
    info.tile_n = bsp::kSub;
    info.n_tiles = 1;
    info.n_items = (int32_t)s.tasks.size();
    info.n_entries = (int32_t)s.terms.size();
    info.grid = s.grid;
    info.max_item_entries = s.max_task_terms;
    info.stages = stages;
    info.group = 1;
    p->wg_per_xcd = s.wg_per_xcd;
    hipError_t e = upload((bsp::SpgemmTask**)&p->d_wgs, s.tasks);
    if (e == hipSuccess) e = upload(&p->d_terms, s.terms);
    if (e == hipSuccess) e = upload(&p->d_runs, s.runs);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_plan_buffers(p);
        delete p;
        return hip_fail(e, "SpGEMM plan upload");
    }
    *out = p;
    return BSP_OK;
}

int bsp_spgemm_structure(const bsp_plan* p, int64_t* nblocks, int32_t* indptr, int32_t* indices) {
    if (!p || p->kind != 4) return fail(BSP_ERR_INVALID_ARGUMENT, "not an SpGEMM plan");
    if (!nblocks) return fail(BSP_ERR_INVALID_ARGUMENT, "nblocks is null");
    *nblocks = (int64_t)p->out_indices.size();
    if (indptr) std::memcpy(indptr, p->out_indptr.data(), p->out_indptr.size() * sizeof(int32_t));
    if (indices && !p->out_indices.empty())
        std::memcpy(indices, p->out_indices.data(), p->out_indices.size() * sizeof(int32_t));
    return BSP_OK;
}

int bsp_spgemm(const bsp_plan* p, const uint16_t* a_vals, const uint16_t* b_vals, void* out_vals, void* stream) {
    if (!p || p->kind != 4) return fail(BSP_ERR_INVALID_ARGUMENT, "not an SpGEMM plan");
    if (p->out_indices.empty()) return BSP_OK;
    if (!a_vals || !b_vals || !out_vals) return fail(BSP_ERR_INVALID_ARGUMENT, "null device pointer");
    if (!aligned16(a_vals) || !aligned16(b_vals) || !aligned16(out_vals))
        return fail(BSP_ERR_INVALID_ARGUMENT, "A, B and output values must be 16-byte aligned");
    DeviceGuard g(p->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    bsp::SpgemmArgs args{};
    args.a = a_vals;
    args.b = b_vals;
    args.out = out_vals;
    args.tasks = (const bsp::SpgemmTask*)p->d_wgs;
    args.terms = p->d_terms;
    args.runs = p->d_runs;
    args.lda = (int32_t)p->C;
    args.ldb = (int32_t)p->BC;
    args.ldo = (int32_t)p->BC;
    args.wg_per_xcd = p->wg_per_xcd;
    hipError_t e = bsp::launch_spgemm(args, p->info.stages, p->out_dtype == BSP_DTYPE_BF16, p->info.grid,
                                      (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "SpGEMM launch");
    return BSP_OK;
}

int bsp_plan_info_get(const bsp_plan* p, bsp_plan_info* info) {
    if (!p || !info) return fail(BSP_ERR_INVALID_ARGUMENT, "null plan or info");
    *info = p->info;
    return BSP_OK;
}

int bsp_plan_destroy(bsp_plan* p) {
    if (!p) return BSP_OK;
    DeviceGuard g(p->device);
    free_plan_buffers(p);
    delete p;
    return BSP_OK;
}

int bsp_host_spmm(const bsp_bsr_desc* a, const uint16_t* a_vals, const uint16_t* b, int64_t N,
                  void* out, int out_dtype, int device) {
    if (!b || !out || (a && a->nblocks > 0 && !a_vals))
        return fail(BSP_ERR_INVALID_ARGUMENT, "null host pointer");
    bsp_plan* p = nullptr;
    int st = bsp_spmm_plan_create(&p, a, N, BSP_ROW_MAJOR, out_dtype, device);
    if (st != BSP_OK) return st;
    DeviceGuard g(device);
    const size_t esz = out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    const size_t a_bytes = std::max<size_t>(16, (size_t)a->nblocks * a->R * a->C * 2);
    const size_t b_bytes = (size_t)a->W * N * 2;
    const size_t c_bytes = (size_t)a->H * N * esz;
    uint16_t *da = nullptr, *db = nullptr;
    void* dc = nullptr;
    hipError_t e = hipMalloc((void**)&da, a_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&db, b_bytes);
    if (e == hipSuccess) e = hipMalloc(&dc, c_bytes);
    if (e == hipSuccess && a->nblocks > 0)
        e = hipMemcpy(da, a_vals, (size_t)a->nblocks * a->R * a->C * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b, b_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        st = bsp_spmm(p, da, db, N, dc, N, nullptr);
        if (st == BSP_OK) {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipMemcpy(out, dc, c_bytes, hipMemcpyDeviceToHost);
        }
    }
    if (da) (void)hipFree(da);
    if (db) (void)hipFree(db);
    if (dc) (void)hipFree(dc);
    bsp_plan_destroy(p);
    if (st != BSP_OK) return st;
    if (e != hipSuccess) return hip_fail(e, "bsp_host_spmm");
    return BSP_OK;
}

int bsp_host_sddmm(const bsp_bsr_desc* mask, const uint16_t* mask_vals, const uint16_t* x,
                   const uint16_t* y, int64_t K, void* out_vals, int out_dtype, int device) {
    if (!x || !y || (mask && mask->nblocks > 0 && (!mask_vals || !out_vals)))
        return fail(BSP_ERR_INVALID_ARGUMENT, "null host pointer");
    bsp_plan* p = nullptr;
    int st = bsp_sddmm_plan_create(&p, mask, K, BSP_ROW_MAJOR, out_dtype, device);
    if (st != BSP_OK) return st;
    if (mask->nblocks == 0) {
        bsp_plan_destroy(p);
        return BSP_OK;
    }
    DeviceGuard g(device);
    const size_t esz = out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    const size_t nv = (size_t)mask->nblocks * mask->R * mask->C;
    const size_t x_bytes = (size_t)mask->H * K * 2;
    const size_t y_bytes = (size_t)K * mask->W * 2;
    uint16_t *dm = nullptr, *dx = nullptr, *dy = nullptr;
    void* dout = nullptr;
    hipError_t e = hipMalloc((void**)&dm, nv * 2);
    if (e == hipSuccess) e = hipMalloc((void**)&dx, x_bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&dy, y_bytes);
    if (e == hipSuccess) e = hipMalloc(&dout, nv * esz);
    if (e == hipSuccess) e = hipMemcpy(dm, mask_vals, nv * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dx, x, x_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dy, y, y_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        st = bsp_sddmm(p, dm, dx, K, dy, mask->W, dout, nullptr);
        if (st == BSP_OK) {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipMemcpy(out_vals, dout, nv * esz, hipMemcpyDeviceToHost);
        }
    }
    if (dm) (void)hipFree(dm);
    if (dx) (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (dout) (void)hipFree(dout);
    bsp_plan_destroy(p);
    if (st != BSP_OK) return st;
    if (e != hipSuccess) return hip_fail(e, "bsp_host_sddmm");
    return BSP_OK;
}

int bsp_host_spgemm(const bsp_bsr_desc* a, const uint16_t* a_vals, const bsp_bsr_desc* b,
                    const uint16_t* b_vals, int32_t* out_indptr, int32_t* out_indices, void* out_vals,
                    int out_dtype, int device) {
    if (!out_indptr || (a && a->nblocks > 0 && !a_vals) || (b && b->nblocks > 0 && !b_vals))
        return fail(BSP_ERR_INVALID_ARGUMENT, "null host pointer");
    bsp_plan* p = nullptr;
    int st = bsp_spgemm_plan_create(&p, a, b, out_dtype, device);
    if (st != BSP_OK) return st;
    int64_t nb = 0;
    bsp_spgemm_structure(p, &nb, out_indptr, nullptr);
    if (nb == 0) {
        bsp_plan_destroy(p);
        return BSP_OK;
    }
    if (!out_indices || !out_vals) {
        bsp_plan_destroy(p);
        return fail(BSP_ERR_INVALID_ARGUMENT, "null host pointer");
    }
    bsp_spgemm_structure(p, &nb, out_indptr, out_indices);
    DeviceGuard g(device);
    const size_t esz = out_dtype == BSP_DTYPE_BF16 ? 2 : 4;
    const size_t a_n = (size_t)a->nblocks * a->R * a->C, b_n = (size_t)b->nblocks * b->R * b->C;
    const size_t o_n = (size_t)nb * a->R * b->C;
    uint16_t *da = nullptr, *db = nullptr;
    void* dout = nullptr;
    hipError_t e = hipMalloc((void**)&da, a_n * 2);
    if (e == hipSuccess) e = hipMalloc((void**)&db, b_n * 2);
    if (e == hipSuccess) e = hipMalloc(&dout, o_n * esz);
    if (e == hipSuccess) e = hipMemcpy(da, a_vals, a_n * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(db, b_vals, b_n * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        st = bsp_spgemm(p, da, db, dout, nullptr);
        if (st == BSP_OK) {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = hipMemcpy(out_vals, dout, o_n * esz, hipMemcpyDeviceToHost);
        }
    }
    if (da) (void)hipFree(da);
    if (db) (void)hipFree(db);
    if (dout) (void)hipFree(dout);
    bsp_plan_destroy(p);
    if (st != BSP_OK) return st;
    if (e != hipSuccess) return hip_fail(e, "bsp_host_spgemm");
    return BSP_OK;
}

}  // extern "C"

#ifdef BSP_TIMELINE
extern "C" int bsp_timeline_skip(int flags) {
    const int all = BSP_SKIP_SPARSE_READ | BSP_SKIP_DENSE_READ | BSP_SKIP_DENSE2_READ | BSP_SKIP_COMPUTE | BSP_SKIP_WRITE;
    if (flags & ~all) return fail(BSP_ERR_INVALID_ARGUMENT, "unknown skip flags");
    g_skips.store(flags, std::memory_order_relaxed);
    return BSP_OK;
}
#endif
