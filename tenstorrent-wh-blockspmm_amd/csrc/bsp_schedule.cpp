// Host-side schedule construction for the SpMM and SDDMM kernels.
//
// Replaces the reference's per-call host analysis: folding of empty block
// rows and serpentine assignment of rows to Tensix core rows
// (block_spmm/inc/host_code/bsr_spmm_multicore_load_balanced_new_DM.cpp:50-61,
// :339-393), and the SDDMM flat block split / first-fit packing
// (block_sddmm/inc/host_code/bsr_sddmm_multicore_naive.cpp:154-166, :267-310;
// bsr_sddmm_multicore_CDA.cpp:95-187).  Here the unit of work is a run of
// 32x32 sub-block products of one 32-row output stripe; rows longer than a
// limit derived from the nnz prefix are cut into pieces, and the pieces are
// spread over the GPU's XCDs longest-first.
#include "bsp_schedule.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <numeric>
#include <queue>

namespace bsp {

namespace {

int64_t env_int(const char* name, int64_t dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    long long x = std::strtoll(v, &end, 10);
    return (end && *end == 0) ? (int64_t)x : dflt;
}

// Load balancing of the SpMM schedules (BSP_SPMM_BALANCE, read when a
// schedule is built): 1 (default) = the nnz-cost split of long rows and the
// longest-first placement; 0 = neither: rows whole and work in its natural
// order, in contiguous ranges -- the counterpart of the reference's operators
// without load balancing (bsr_spmm_multicore_load_balanced_new_DM_no_lb and
// its SnF / CDA siblings, block_spmm/inc/host_code.hpp:113-124, :158-161,
// which deal contiguous row ranges to cores,
// bsr_spmm_multicore_load_balanced_new_DM.cpp:339-344).
bool load_balance() { return env_int("BSP_SPMM_BALANCE", 1) != 0; }

}  // namespace

int validate_bsr(const bsp_bsr_desc* d, std::string& msg) {
    if (!d) {
        msg = "null BSR descriptor";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    if (d->R <= 0 || d->C <= 0 || d->H <= 0 || d->W <= 0) {
        msg = "H, W, R, C must be positive";
        return BSP_ERR_BAD_STRUCTURE;
    }
    if (d->H % d->R != 0 || d->W % d->C != 0) {
        msg = "H must be a multiple of R and W a multiple of C";
        return BSP_ERR_BAD_STRUCTURE;
    }
    if (d->nblocks < 0 || d->nblocks * d->R * d->C > d->H * d->W) {
        msg = "nblocks must satisfy 0 <= nblocks*R*C <= H*W";
        return BSP_ERR_BAD_STRUCTURE;
    }
    if (d->H / d->R > INT32_MAX - 1 || d->nblocks > INT32_MAX) {
        msg = "structure too large for int32 indices";
        return BSP_ERR_UNSUPPORTED;
    }
    if (!d->indptr) {
        msg = "indptr is null";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    if (d->nblocks > 0 && !d->indices) {
        msg = "indices is null";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    const int64_t nbr = d->H / d->R, nbc = d->W / d->C;
    if (d->indptr[0] != 0) {
        msg = "indptr[0] must be 0";
        return BSP_ERR_BAD_STRUCTURE;
    }
    for (int64_t i = 0; i < nbr; ++i) {
        if (d->indptr[i + 1] < d->indptr[i]) {
            msg = "indptr must be non-decreasing (row " + std::to_string(i) + ")";
            return BSP_ERR_BAD_STRUCTURE;
        }
    }
    if ((int64_t)d->indptr[nbr] != d->nblocks) {
        msg = "indptr[H/R] = " + std::to_string(d->indptr[nbr]) + " but nblocks = " +
              std::to_string(d->nblocks);
        return BSP_ERR_BAD_STRUCTURE;
    }
    for (int64_t e = 0; e < d->nblocks; ++e) {
        if (d->indices[e] < 0 || d->indices[e] >= nbc) {
            msg = "indices[" + std::to_string(e) + "] = " + std::to_string(d->indices[e]) +
                  " outside [0, W/C = " + std::to_string(nbc) + ")";
            return BSP_ERR_BAD_STRUCTURE;
        }
    }
    return BSP_OK;
}

std::vector<int32_t> xcd_lpt_map(const std::vector<int64_t>& unit_cost, int width) {
    const int64_t nunits = (int64_t)unit_cost.size();
    std::vector<int32_t> order(nunits);
    std::iota(order.begin(), order.end(), 0);
    // Longest first; ties by index so the map is deterministic.
    std::stable_sort(order.begin(), order.end(),
                     [&](int32_t a, int32_t b) { return unit_cost[a] > unit_cost[b]; });
    std::vector<std::vector<int32_t>> bins(kNumXcd);
    using Load = std::pair<int64_t, int>;  // (load, xcd)
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int x = 0; x < kNumXcd; ++x) heap.push({0, x});
    for (int32_t u : order) {
        Load l = heap.top();
        heap.pop();
        for (int t = 0; t < width; ++t) bins[l.second].push_back(u * width + t);
        heap.push({l.first + unit_cost[u] * width, l.second});
    }
    size_t maxlen = 0;
    for (auto& b : bins) maxlen = std::max(maxlen, b.size());
    std::vector<int32_t> map(maxlen * kNumXcd, -1);
    for (int x = 0; x < kNumXcd; ++x)
        for (size_t j = 0; j < bins[x].size(); ++j) map[j * kNumXcd + x] = bins[x][j];
    return map;
}

void pair_rounds(std::vector<int32_t>& bin, int cus_per_xcd) {
    const int64_t len = (int64_t)bin.size();
    if (cus_per_xcd <= 0 || len <= cus_per_xcd || len > 2 * (int64_t)cus_per_xcd) return;
    std::reverse(bin.begin() + cus_per_xcd, bin.end());
}

std::vector<int32_t> xcd_tile_map(const std::vector<int64_t>& item_cost, int n_tiles, int col_groups,
                                  int cus_per_xcd, bool row_bands) {
    if (col_groups < 1 || kNumXcd % col_groups != 0 || n_tiles % col_groups != 0) col_groups = 1;
    const int row_groups = kNumXcd / col_groups;
    const int64_t nitems = (int64_t)item_cost.size();
    std::vector<int32_t> order(nitems);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(),
                     [&](int32_t a, int32_t b) { return item_cost[a] > item_cost[b]; });
    std::vector<std::vector<int32_t>> rows(row_groups);
    if (row_bands) {
        // Contiguous runs of items (rows in order), equal in count (the
        // workgroups an XCD must hold at once).
        for (int64_t u = 0; u < nitems; ++u) rows[u * row_groups / std::max<int64_t>(1, nitems)].push_back((int32_t)u);
        for (auto& r : rows)
            std::stable_sort(r.begin(), r.end(), [&](int32_t a, int32_t b) { return item_cost[a] > item_cost[b]; });
    } else {
        using Load = std::pair<int64_t, int>;
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
        for (int g = 0; g < row_groups; ++g) heap.push({0, g});
        for (int32_t u : order) {
            Load l = heap.top();
            heap.pop();
            rows[l.second].push_back(u);
            heap.push({l.first + item_cost[u], l.second});
        }
    }
    const int tpg = n_tiles / col_groups;
    std::vector<std::vector<int32_t>> bins(kNumXcd);
    for (int rg = 0; rg < row_groups; ++rg)
        for (int cg = 0; cg < col_groups; ++cg) {
            auto& b = bins[rg * col_groups + cg];
            for (int32_t u : rows[rg])
                for (int t = cg * tpg; t < (cg + 1) * tpg; ++t) b.push_back(u * n_tiles + t);
            pair_rounds(b, cus_per_xcd);
        }
    size_t maxlen = 0;
    for (auto& b : bins) maxlen = std::max(maxlen, b.size());
    std::vector<int32_t> map(maxlen * kNumXcd, -1);
    for (int x = 0; x < kNumXcd; ++x)
        for (size_t j = 0; j < bins[x].size(); ++j) map[j * kNumXcd + x] = bins[x][j];
    return map;
}

std::vector<SpmmWg> spmm_wg_records(const SpmmSchedule& s) {
    std::vector<SpmmWg> out(s.wgmap.size());
    for (size_t g = 0; g < s.wgmap.size(); ++g) {
        const int32_t u = s.wgmap[g];
        if (u < 0) {
            out[g] = {-1, 0, 0, -1, -1, 0, 0, 0};
            continue;
        }
        const SpmmItem& it = s.items[u / s.n_tiles];
        out[g] = {it.row, it.e_begin, it.e_end, it.slot, it.base, it.npieces, u % s.n_tiles, 0};
    }
    return out;
}

std::vector<int64_t> spmm_packed_entries(const SpmmSchedule& s) {
    std::vector<int64_t> out(s.ent_row.size());
    for (size_t e = 0; e < out.size(); ++e)
        out[e] = (int64_t)(uint32_t)s.ent_row[e] | ((s.ent_off[e] / kSub) << 32);
    return out;
}

std::vector<SpmmSplit> spmm_splits(const SpmmSchedule& s) {
    std::vector<SpmmSplit> out;
    for (const SpmmItem& it : s.items)
        if (it.slot >= 0 && it.slot == it.base)
            for (int32_t st = 0; st < s.group; ++st)
                out.push_back({it.row + st, it.base + st * it.npieces, it.npieces, 0});
    return out;
}

int spmm_choose_group(int64_t R, int64_t H, int64_t N, int num_cus) {
    const int64_t rs = R / kSub, nsr = H / kSub, tiles = (N + 127) / 128;
    for (int g : {8, 4, 2})
        if (rs % g == 0 && (nsr / g) * tiles >= 2 * (int64_t)num_cus) return g;
    return 1;
}

std::vector<SddmmItem> sddmm_wg_records(const SddmmSchedule& s) {
    std::vector<SddmmItem> out(s.wgmap.size());
    for (size_t g = 0; g < s.wgmap.size(); ++g) {
        const int32_t u = s.wgmap[g];
        out[g] = u < 0 ? SddmmItem{0, 0, 0, 0} : s.items[u];
    }
    return out;
}

int build_spmm_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, SpmmSchedule& s,
                        std::string& msg, int force_tile_n, int group) {
    int st = validate_bsr(a, msg);
    if (st != BSP_OK) return st;
    if (N <= 0) {
        msg = "N must be positive";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    if (a->R % kSub || a->C % kSub || N % kSub || N > INT32_MAX / 2) {
        msg = "R, C and N must be multiples of 32";
        return BSP_ERR_UNSUPPORTED;
    }
    if (num_cus <= 0) num_cus = 256;
    const int64_t RS = a->R / kSub, CS = a->C / kSub;
    const int64_t nbr = a->H / a->R;
    const int64_t nsr = a->H / kSub;
    const int64_t total = a->nblocks * RS * CS;
    if (total > INT32_MAX || a->W > INT32_MAX || nsr > INT32_MAX) {
        msg = "problem too large for int32 schedule fields";
        return BSP_ERR_UNSUPPORTED;
    }

    // Row groups: stripes of one block row that share every B panel.
    if (group <= 0) group = (int)env_int("BSP_SPMM_GROUP", spmm_choose_group(a->R, a->H, N, num_cus));
    if (group != 1 && group != 2 && group != 4 && group != 8) group = 1;
    if (RS % group != 0) group = 1;
    s.group = group;
    // Row groups take 256-column tiles (the wide group kernel: two workgroups
    // per compute unit for groups of 2 and 4 with a three-stage ring, else
    // one) when N is a multiple of 256 and the groups' tiles
    // still fill every compute unit, else 128-column tiles.
    // (BSP_SPMM_WIDE_GROUP: 0 never, 2 whenever N allows it.)
    if (group > 1) {
        const int64_t wide_tiles = N % 256 == 0 ? (nsr / group) * (N / 256) : 0;
        const int64_t wide = env_int("BSP_SPMM_WIDE_GROUP", 1);
        force_tile_n = (wide_tiles > 0 && (wide == 2 || (wide == 1 && wide_tiles >= num_cus))) ? 256 : 128;
    }

    // Workgroup width: 128 columns (four waves of 32); 256 (four waves of 64)
    // only when N is a multiple of 256 and rows alone give two workgroups per
    // compute unit, and unless only the narrower tile's column groups bring
    // each XCD's slice of B within its 4 MB L2 (skewed 16384^2 x 1024:
    // 46.6 -> 44.6 us).  The last tile of a row may be partial.
    int64_t tn = force_tile_n ? force_tile_n : env_int("BSP_SPMM_TILE_N", 0);
    if (tn != 0 && tn != 128 && tn != 256) tn = 0;
    if (tn == 0) {
        tn = (N % 256 == 0 && nsr * (N / 256) >= 2 * (int64_t)num_cus) ? 256 : 128;
        const int64_t bb = a->W * N * 2;
        constexpr int64_t kL2 = int64_t(4) << 20;
        if (tn == 256 && bb / std::min<int64_t>(kNumXcd, N / 256) > kL2 &&
            bb / std::min<int64_t>(kNumXcd, N / 128) <= kL2)
            tn = 128;
    }
    s.tile_n = (int32_t)tn;
    s.n_tiles = (int32_t)((N + tn - 1) / tn);

    // Split limit: a piece holds at most L entries.  L is the larger of twice
    // the mean length of non-empty rows (uniform rows stay whole) and one
    // compute unit's fair share of the total (a longer row would alone
    // outlast the rest), and at least 32.  A split row costs a partial round
    // trip and a second launch, which a row shorter than the fair share does
    // not repay: the skewed 16384^2 Zipf(1.2) workload (rows of at most 101
    // entries, fair share 164) ran 8-11% faster with its rows whole than
    // with its 12 longest halved at half the fair share (two boxes:
    // 42.2-43.4 -> 37.7-38.2 us, 44.4-44.9 -> 40.8-41.4 us).
    // (In units of group entries: one entry of a group serves `group` stripes.)
    const int64_t gtotal = total / group;
    int64_t nonempty = 0;
    for (int64_t i = 0; i < nbr; ++i) nonempty += (a->indptr[i + 1] > a->indptr[i]) ? RS / group : 0;
    const int64_t mean = nonempty ? (gtotal + nonempty - 1) / nonempty : 0;
    const int64_t fair = (gtotal * s.n_tiles + num_cus - 1) / num_cus;
    int64_t L = std::max<int64_t>({32, 2 * mean, fair});
    if (!load_balance()) L = INT32_MAX;  // rows whole
    L = env_int("BSP_SPMM_SPLIT", L);
    if (L < 1) L = 1;
    if (a->C % 64 == 0 && L < 2) L = 2;  // pieces hold whole entry pairs (below)
    s.split_limit = (int32_t)L;

    s.items.clear();
    s.ent_row.clear();
    s.ent_off.clear();
    s.ent_row.reserve(total);
    s.ent_off.reserve(total);
    s.n_slots = 0;
    s.n_split_rows = 0;
    s.max_item_entries = 0;
    std::vector<int64_t> cost;
    for (int64_t sr = 0; sr < nsr; sr += group) {
        const int64_t i = sr / RS, sub = sr % RS;
        const int32_t e0 = (int32_t)s.ent_row.size();
        for (int64_t blk = a->indptr[i]; blk < a->indptr[i + 1]; ++blk) {
            for (int64_t t = 0; t < CS; ++t) {
                s.ent_row.push_back((int32_t)((int64_t)a->indices[blk] * a->C + kSub * t));
                s.ent_off.push_back(blk * a->R * a->C + kSub * sub * a->C + kSub * t);
            }
        }
        const int32_t e1 = (int32_t)s.ent_row.size();
        const int64_t cnt = e1 - e0;
        // Cost model: one unit per 32x32 product (per stripe of the group)
        // plus a fixed share for the output store (split pieces add a
        // partial round trip).
        if (cnt <= L) {
            s.items.push_back({(int32_t)sr, e0, e1, -1, -1, 0});
            cost.push_back((cnt + 2) * group);
            s.max_item_entries = std::max<int32_t>(s.max_item_entries, (int32_t)cnt);
        } else {
            // Pieces start at an even entry of the block when C is a multiple
            // of 64 (a row's count is then even): the kernels may fetch A for
            // the two 32-column halves of 64 columns together.
            const int64_t unit = (a->C % 64 == 0) ? 2 : 1;
            const int64_t cu = cnt / unit, lu = std::max<int64_t>(1, L / unit);
            const int64_t np = (cu + lu - 1) / lu;
            const int32_t base = s.n_slots;
            s.n_slots += (int32_t)(np * group);
            s.n_split_rows += group;
            for (int64_t p = 0; p < np; ++p) {
                const int32_t b0 = e0 + (int32_t)(unit * (cu * p / np));
                const int32_t b1 = e0 + (int32_t)(unit * (cu * (p + 1) / np));
                s.items.push_back({(int32_t)sr, b0, b1, base + (int32_t)p, base, (int32_t)np});
                cost.push_back(((b1 - b0) + 4) * group);
                s.max_item_entries = std::max<int32_t>(s.max_item_entries, b1 - b0);
            }
        }
    }
    if ((int64_t)s.items.size() * s.n_tiles > INT32_MAX / 2) {
        msg = "too many work items";
        return BSP_ERR_UNSUPPORTED;
    }
    // With C a multiple of 64 every item must start at an even 32-column
    // step of its block: a kernel then fetches A for entries 2m and 2m+1 as
    // one 64-column span, which for an odd start would reach past the row.
    if (a->C % 64 == 0)
        for (const SpmmItem& it : s.items)
            if (it.e_end > it.e_begin && (s.ent_off[it.e_begin] % a->C) / kSub % 2 != 0) {
                msg = "internal: work item starts at an odd 32-column step";
                return BSP_ERR_UNSUPPORTED;
            }
    // Column groups of the XCD map: the fewest (1, 2, 4, 8) that bring one
    // XCD's slice of B to at most 2 MiB, limited by the tile count.
    int64_t cg = 1;
    const int64_t b_bytes = a->W * N * 2;
    while (cg < kNumXcd && b_bytes / cg > (2 << 20) && s.n_tiles % (cg * 2) == 0) cg *= 2;
    cg = env_int("BSP_SPMM_XCD_COLS", cg);
    if (cg < 1 || kNumXcd % cg != 0 || s.n_tiles % cg != 0) cg = 1;
    s.xcd_col_groups = (int32_t)cg;
    // Heavy-with-light pairing on a compute unit pays once rows carry a few
    // entries each (at about one entry per row the store dominates and the
    // plain longest-first order measured faster).
    const int pair_cus = (int)env_int("BSP_SPMM_PAIR_CUS", mean >= 4 ? num_cus / kNumXcd : 0);
    if (!load_balance()) {
        // Natural order: workgroup g takes item g / n_tiles, tile g % n_tiles.
        s.wgmap.resize(s.items.size() * (size_t)s.n_tiles);
        std::iota(s.wgmap.begin(), s.wgmap.end(), 0);
        return BSP_OK;
    }
    s.wgmap = xcd_tile_map(cost, s.n_tiles, (int)cg, pair_cus, false);
    // Rows in contiguous bands per XCD instead (a banded structure, whose
    // nearby rows read nearby rows of B): kept when the busiest XCD then
    // reads fewer distinct 32-row panels of B (per tile) and carries at most
    // 10% more work than under the longest-first map.  (Banded attention
    // mask, O = S*V: 6.9 -> 6.6 us; a uniform structure keeps the
    // longest-first map.)
    if (kNumXcd / cg > 1) {
        const std::vector<int32_t> banded = xcd_tile_map(cost, s.n_tiles, (int)cg, pair_cus, true);
        auto busiest = [&](const std::vector<int32_t>& map) {
            int64_t worst = 0;
            std::vector<int32_t> seen;
            for (int x = 0; x < kNumXcd; ++x) {
                seen.clear();
                for (size_t j = x; j < map.size(); j += kNumXcd) {
                    const int32_t u = map[j];
                    if (u < 0) continue;
                    const SpmmItem& it = s.items[u / s.n_tiles];
                    for (int32_t e = it.e_begin; e < it.e_end; ++e)
                        seen.push_back((s.ent_row[e] / kSub) * s.n_tiles + u % s.n_tiles);
                }
                std::sort(seen.begin(), seen.end());
                worst = std::max<int64_t>(worst, std::unique(seen.begin(), seen.end()) - seen.begin());
            }
            return worst;
        };
        auto heaviest = [&](const std::vector<int32_t>& map) {
            int64_t worst = 0;
            for (int x = 0; x < kNumXcd; ++x) {
                int64_t c = 0;
                for (size_t j = x; j < map.size(); j += kNumXcd)
                    if (map[j] >= 0) c += cost[map[j] / s.n_tiles];
                worst = std::max(worst, c);
            }
            return worst;
        };
        const int64_t force = env_int("BSP_SPMM_ROW_BANDS", -1);
        const bool fewer = busiest(banded) < busiest(s.wgmap);
        const bool balanced = heaviest(banded) * 10 <= heaviest(s.wgmap) * 11;  // within 10%
        if (force == 1 || (force != 0 && fewer && balanced)) s.wgmap = banded;
    }
    return BSP_OK;
}

bool spmm_stripe_pairs(const bsp_bsr_desc* a, int64_t max_rows, std::vector<std::pair<int32_t, int32_t>>& pairs,
                       int64_t* shared, int64_t* max_union) {
    pairs.clear();
    if (shared) *shared = 0;
    if (max_union) *max_union = 0;
    if (!a || a->R != kSub || a->C != kSub || a->H % kSub || a->W % kSub) return false;
    const int64_t nbr = a->H / kSub, nbc = a->W / kSub;
    if (nbr < 2 || nbr > max_rows) return false;
    for (int64_t i = 0; i < nbr; ++i)
        for (int64_t k = a->indptr[i] + 1; k < a->indptr[i + 1]; ++k)
            if (a->indices[k] <= a->indices[k - 1]) return false;  // columns must increase strictly
    // Shared block columns of every two block rows, through the rows of each
    // column; give up when that costs too much host time.
    std::vector<std::vector<int32_t>> rows_of(nbc);
    for (int64_t i = 0; i < nbr; ++i)
        for (int64_t k = a->indptr[i]; k < a->indptr[i + 1]; ++k) rows_of[a->indices[k]].push_back((int32_t)i);
    int64_t work = 0;
    for (const auto& r : rows_of) work += (int64_t)r.size() * (int64_t)r.size();
    if (work > (int64_t)1 << 26) return false;
    std::vector<int32_t> ov((size_t)(nbr * nbr), 0);
    for (const auto& r : rows_of)
        for (size_t x = 0; x < r.size(); ++x)
            for (size_t y = x + 1; y < r.size(); ++y) ++ov[(size_t)r[x] * nbr + r[y]];
    struct Cand {
        int32_t n, i, j;
    };
    std::vector<Cand> cand;
    for (int64_t i = 0; i < nbr; ++i)
        for (int64_t j = i + 1; j < nbr; ++j)
            if (ov[(size_t)i * nbr + j] > 0) cand.push_back({ov[(size_t)i * nbr + j], (int32_t)i, (int32_t)j});
    std::stable_sort(cand.begin(), cand.end(), [](const Cand& x, const Cand& y) { return x.n > y.n; });
    std::vector<char> used(nbr, 0);
    int64_t sh = 0;
    for (const Cand& c : cand)
        if (!used[c.i] && !used[c.j]) {
            used[c.i] = used[c.j] = 1;
            pairs.push_back({c.i, c.j});
            sh += c.n;
        }
    int32_t left = -1;
    for (int64_t i = 0; i < nbr; ++i) {
        if (used[i]) continue;
        if (left < 0) {
            left = (int32_t)i;
        } else {
            pairs.push_back({left, (int32_t)i});
            left = -1;
        }
    }
    if (left >= 0) pairs.push_back({left, -1});
    std::sort(pairs.begin(), pairs.end());
    int64_t mu = 0;
    for (const auto& [i, j] : pairs) {
        const int64_t ni = a->indptr[i + 1] - a->indptr[i];
        const int64_t nj = j >= 0 ? a->indptr[j + 1] - a->indptr[j] : 0;
        const int64_t o = j >= 0 ? ov[(size_t)std::min(i, j) * nbr + std::max(i, j)] : 0;
        mu = std::max(mu, ni + nj - o);
    }
    // Leftover pairs share no columns (any two unpaired rows that did were a candidate).
    if (shared) *shared = sh;
    if (max_union) *max_union = mu;
    return true;
}

int build_spmm_stream(const bsp_bsr_desc* a, int64_t N, int num_cus, int tile_n, int wg_per_cu, SpmmStream& s,
                      std::string& msg, int col_groups, int pipes, bool pairs) {
    int st = validate_bsr(a, msg);
    if (st != BSP_OK) return st;
    if (tile_n != 128 && tile_n != 256) {
        msg = "stream tile must be 128 or 256 columns";
        return BSP_ERR_UNSUPPORTED;
    }
    if (N <= 0 || N % tile_n != 0 || N > INT32_MAX / 2) {
        msg = "N must be a positive multiple of the stream tile";
        return BSP_ERR_UNSUPPORTED;
    }
    if (a->R % kSub || a->C % kSub) {
        msg = "R and C must be multiples of 32";
        return BSP_ERR_UNSUPPORTED;
    }
    if (num_cus <= 0) num_cus = 256;
    if (wg_per_cu < 1) wg_per_cu = 1;
    if (pipes != 1 && pipes != 2) {
        msg = "pipelines per workgroup must be 1 or 2";
        return BSP_ERR_UNSUPPORTED;
    }
    if (pipes == 2) wg_per_cu = 1;
    std::vector<std::pair<int32_t, int32_t>> pair_list;
    if (pairs) {
        if (pipes != 1 || !spmm_stripe_pairs(a, kPairMaxRows, pair_list, nullptr)) {
            msg = "stripe pairs need one pipeline, 32x32 blocks, strictly increasing block columns and at most "
                  "1024 block rows";
            return BSP_ERR_UNSUPPORTED;
        }
    }
    const int64_t RS = a->R / kSub, CS = a->C / kSub;
    // The scheduled rows: stripes, or stripe pairs (row = the pair's index).
    const int64_t nsr = pairs ? (int64_t)pair_list.size() : a->H / kSub;
    const int64_t n_tiles = N / tile_n;
    const int64_t per_stripe_total = a->nblocks * CS;  // entries summed over one stripe of every block row
    if (per_stripe_total * RS * n_tiles > INT32_MAX - kStreamPad || nsr > INT32_MAX || a->W > INT32_MAX ||
        a->nblocks * a->R * a->C / kSub > UINT32_MAX) {
        msg = "problem too large for the stream schedule";
        return BSP_ERR_UNSUPPORTED;
    }
    s = SpmmStream{};
    s.tile_n = tile_n;
    s.n_tiles = (int32_t)n_tiles;
    s.wg_per_cu = wg_per_cu;
    s.pairs = pairs ? 1 : 0;

    // Column groups: the fewest (1, 2, 4, 8) that bring one XCD's slice of B
    // to at most 2 MiB, limited by the tile count (or as asked).
    int64_t cg = 1;
    const int64_t b_bytes = a->W * N * 2;
    while (cg < kNumXcd && b_bytes / cg > (2 << 20) && n_tiles % (cg * 2) == 0) cg *= 2;
    if (col_groups > 0) cg = col_groups;
    if (cg < 1 || kNumXcd % cg != 0 || n_tiles % cg != 0) cg = 1;
    s.col_groups = (int32_t)cg;
    const int64_t rg_count = kNumXcd / cg, tpg = n_tiles / cg;
    const bool rotate = pipes == 1 && env_int("BSP_SPMM_ROTATE", 1) != 0;
    s.rotated = rotate ? 1 : 0;

    // Stripe entry counts; a unit costs its entries plus the store.  (A
    // cost fitted to per-unit times measured on the skewed workload,
    // 0.1114 c + 0.3324 sqrt(c) us, which long units' faster streaming
    // suggested, measured 0.5-1.5 us slower there: the spread of the
    // workgroups' busy times comes from the memory system more than from
    // the units' sizes.)
    constexpr int64_t kStoreCost = 2;
    // A pair's entries: the union of its two block rows' columns, merged in
    // column order (each row's own blocks keep their CSR order); emit(col,
    // blk0, blk1) with -1 for a row without a block in that column.
    auto merge = [&](int32_t r0, int32_t r1, auto&& emit_one) {
        int64_t k0 = a->indptr[r0], k1 = r1 >= 0 ? a->indptr[r1] : 0;
        const int64_t e0 = a->indptr[r0 + 1], e1 = r1 >= 0 ? a->indptr[r1 + 1] : 0;
        while (k0 < e0 || k1 < e1) {
            const int32_t c0 = k0 < e0 ? a->indices[k0] : INT32_MAX, c1 = k1 < e1 ? a->indices[k1] : INT32_MAX;
            if (c0 == c1) {
                emit_one(c0, k0++, k1++);
            } else if (c0 < c1) {
                emit_one(c0, k0++, (int64_t)-1);
            } else {
                emit_one(c1, (int64_t)-1, k1++);
            }
        }
    };
    std::vector<int64_t> cnt(nsr);
    for (int64_t sr = 0; sr < nsr; ++sr) {
        if (pairs) {
            int64_t n = 0;
            merge(pair_list[sr].first, pair_list[sr].second, [&](int32_t, int64_t, int64_t) { ++n; });
            cnt[sr] = n;
        } else {
            const int64_t i = sr / RS;
            cnt[sr] = (int64_t)(a->indptr[i + 1] - a->indptr[i]) * CS;
        }
    }
    // Stripes onto row groups, longest first onto the least-loaded group
    // (without load balancing: contiguous ranges in stripe order).
    const bool balance = load_balance();
    std::vector<int32_t> order(nsr);
    std::iota(order.begin(), order.end(), 0);
    if (balance)
        std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) { return cnt[x] > cnt[y]; });
    std::vector<std::vector<int32_t>> rows(rg_count);
    using Load = std::pair<int64_t, int>;
    if (balance) {
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
        for (int g = 0; g < rg_count; ++g) heap.push({0, g});
        for (int32_t sr : order) {
            Load l = heap.top();
            heap.pop();
            rows[l.second].push_back(sr);
            heap.push({l.first + cnt[sr] + kStoreCost, l.second});
        }
    } else {
        for (int64_t i = 0; i < nsr; ++i) rows[i * rg_count / nsr].push_back((int32_t)i);
    }
    // Inside each XCD: units longest first onto the least-loaded compute
    // unit, then each compute unit's units longest first onto the
    // least-loaded of its workgroups.  The two workgroups of a compute unit
    // share its load path, so the balance that matters first is per compute
    // unit.  An XCD's dispatcher gives its j-th workgroup to compute unit
    // j % C (C = compute units per XCD): workgroup c of compute unit u is the
    // XCD's workgroup u + c*C.
    const int cus_per_xcd = std::max(1, num_cus / kNumXcd);
    const int bins = cus_per_xcd * wg_per_cu;
    std::vector<std::vector<SpmmStreamUnit>> wg_units((size_t)bins * kNumXcd);
    auto lpt = [balance](const std::vector<SpmmStreamUnit>& us, int nb, std::vector<std::vector<SpmmStreamUnit>>& out) {
        out.assign(nb, {});
        if (!balance) {  // contiguous ranges in order
            for (size_t i = 0; i < us.size(); ++i) out[i * nb / us.size()].push_back(us[i]);
            return;
        }
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
        for (int b = 0; b < nb; ++b) heap.push({0, b});
        for (const SpmmStreamUnit& u : us) {  // longest first
            Load l = heap.top();
            heap.pop();
            out[l.second].push_back(u);
            heap.push({l.first + u.count + kStoreCost, l.second});
        }
    };
    for (int64_t rg = 0; rg < rg_count; ++rg)
        for (int64_t c = 0; c < cg; ++c) {
            const int x = (int)(rg * cg + c);
            std::vector<SpmmStreamUnit> us;
            for (int32_t sr : rows[rg])  // rows[rg] is longest first
                for (int64_t t = c * tpg; t < (c + 1) * tpg; ++t) {
                    if (pairs)
                        us.push_back({pair_list[sr].first, (int32_t)(t * tile_n), (int32_t)cnt[sr],
                                      pair_list[sr].second});
                    else
                        us.push_back({sr, (int32_t)(t * tile_n), (int32_t)cnt[sr], 0});
                }
            std::vector<std::vector<SpmmStreamUnit>> per_cu, per_wg;
            lpt(us, cus_per_xcd, per_cu);
            for (int cu = 0; cu < cus_per_xcd; ++cu) {
                lpt(per_cu[cu], wg_per_cu, per_wg);
                for (int w = 0; w < wg_per_cu; ++w)
                    wg_units[(size_t)(cu + w * cus_per_xcd) * kNumXcd + x] = std::move(per_wg[w]);
            }
        }
    // A part of a unit: entries [e0, e1) of the stripe's list (in the
    // reference's order: blocks in CSR order, then the 32-column steps).
    struct Part {
        SpmmStreamUnit u;
        int32_t e0, e1;
    };
    // Two pipelines: the compute unit's units, empty ones first, then longest
    // first, concatenated and cut at ceil(total / 2).
    auto halves = [&](const std::vector<SpmmStreamUnit>& us, std::vector<Part>& p0, std::vector<Part>& p1) {
        std::vector<SpmmStreamUnit> order(us);
        std::stable_sort(order.begin(), order.end(),
                         [](const SpmmStreamUnit& x, const SpmmStreamUnit& y) { return (x.count > 0) < (y.count > 0); });
        int64_t total = 0;
        for (const SpmmStreamUnit& u : order) total += u.count;
        const int64_t cut = (total + 1) / 2;
        int64_t pos = 0;
        for (const SpmmStreamUnit& u : order) {
            const int64_t b = pos, e = pos + u.count;
            if (e <= cut) {
                p0.push_back({u, 0, u.count});
            } else if (b >= cut) {
                p1.push_back({u, 0, u.count});
            } else {  // straddles the cut
                SpmmStreamUnit a0 = u, a1 = u;
                a0.count = (int32_t)(cut - b);
                a0.aux = 2;
                a1.count = (int32_t)(e - cut);
                a1.aux = 1;
                p0.push_back({a0, 0, a0.count});
                p1.insert(p1.begin(), {a1, a0.count, u.count});
            }
            pos = e;
        }
    };
    // Each unit of column group c > 0 starts at its first block column at or
    // past c/cg of A's block columns and wraps around
    // (spmm_stream_rotation_column); returns the offset of that entry among
    // the unit's entries at `first`.
    auto rotation = [&](size_t first, int32_t n0) -> int64_t {
        if (!rotate) return 0;
        const int64_t kcol = spmm_stream_rotation_column(a->W / a->C, (n0 / tile_n) / tpg, cg);
        const int64_t len = (int64_t)(s.bw.size() - first);
        int64_t off = 0;
        while (off < len && (int64_t)((uint32_t)s.bw[first + off] / a->C) < kcol) ++off;
        return off == len ? 0 : off;
    };
    auto emit = [&](const std::vector<Part>& parts) {
        SpmmStreamWg w{};
        w.w_begin = (int32_t)s.bw.size();
        w.u_begin = (int32_t)s.units.size();
        w.n_units = (int32_t)parts.size();
        for (const Part& pt : parts) {
            s.units.push_back(pt.u);
            if (pairs) {
                const size_t first = s.bw.size();
                merge(pt.u.row, pt.u.aux, [&](int32_t col, int64_t k0, int64_t k1) {
                    const uint64_t w0 = k0 >= 0 ? (uint64_t)(k0 * a->R * a->C / kSub) : kNoBlock;
                    const uint64_t w1 = k1 >= 0 ? (uint64_t)(k1 * a->R * a->C / kSub) : kNoBlock;
                    s.bw.push_back((int64_t)col * a->C | ((int64_t)pt.u.n0 << 32));
                    s.apw.push_back(w0 | w1 << 32);
                });
                const int64_t off = rotation(first, pt.u.n0);
                std::rotate(s.bw.begin() + first, s.bw.begin() + first + off, s.bw.end());
                std::rotate(s.apw.begin() + first, s.apw.begin() + first + off, s.apw.end());
                continue;
            }
            const int64_t i = pt.u.row / RS, sub = pt.u.row % RS;
            const size_t first = s.bw.size();
            int64_t e = 0;
            for (int64_t blk = a->indptr[i]; blk < a->indptr[i + 1]; ++blk)
                for (int64_t t = 0; t < CS; ++t, ++e) {
                    if (e < pt.e0 || e >= pt.e1) continue;
                    const int64_t brow = (int64_t)a->indices[blk] * a->C + kSub * t;
                    s.bw.push_back(brow | ((int64_t)pt.u.n0 << 32));
                    s.aw.push_back((uint32_t)((blk * a->R * a->C + kSub * sub * a->C + kSub * t) / kSub));
                }
            const int64_t off = rotation(first, pt.u.n0);
            std::rotate(s.bw.begin() + first, s.bw.begin() + first + off, s.bw.end());
            std::rotate(s.aw.begin() + first, s.aw.begin() + first + off, s.aw.end());
        }
        w.n = (int32_t)(s.bw.size() - w.w_begin);
        s.max_wg_entries = std::max(s.max_wg_entries, w.n);
        s.wgs.push_back(w);
    };
    // Streams, workgroup by workgroup (workgroup g = bin * kNumXcd + xcd);
    // with two pipelines, records 2g and 2g+1.
    for (size_t g = 0; g < wg_units.size(); ++g) {
        if (pipes == 1) {
            std::vector<Part> parts;
            for (const SpmmStreamUnit& u : wg_units[g]) parts.push_back({u, 0, u.count});
            emit(parts);
        } else {
            std::vector<Part> p0, p1;
            halves(wg_units[g], p0, p1);
            emit(p0);
            emit(p1);
        }
    }
    s.n_entries = (int64_t)s.bw.size();
    s.bw.resize(s.bw.size() + kStreamPad, 0);
    if (pairs)
        s.apw.resize(s.apw.size() + kStreamPad, 0);
    else
        s.aw.resize(s.aw.size() + kStreamPad, 0);
    s.units.resize(s.units.size() + kStreamPad, SpmmStreamUnit{0, 0, 0, 0});
    s.heads.assign(s.wgs.size(), SpmmStreamHead{});
    for (size_t g = 0; g < s.wgs.size(); ++g) {
        SpmmStreamHead& h = s.heads[g];
        const SpmmStreamWg& w = s.wgs[g];
        h.wg = w;
        for (int j = 0; j < 2; ++j) h.u[j] = s.units[(size_t)w.u_begin + j];
        for (int j = 0; j < kHeadWords; ++j) {
            h.bw[j] = s.bw[(size_t)w.w_begin + j];
            if (pairs)
                h.apw[j] = s.apw[(size_t)w.w_begin + j];
            else
                h.aw[j] = s.aw[(size_t)w.w_begin + j];
        }
    }
    return BSP_OK;
}

namespace {

// Entries (32x32 sub-block products) of each 32-row stripe.
std::vector<int64_t> stripe_entries(const bsp_bsr_desc* a) {
    const int64_t RS = a->R / kSub, CS = a->C / kSub, nsr = a->H / kSub;
    std::vector<int64_t> cnt(nsr);
    for (int64_t sr = 0; sr < nsr; ++sr) {
        const int64_t i = sr / RS;
        cnt[sr] = (int64_t)(a->indptr[i + 1] - a->indptr[i]) * CS;
    }
    return cnt;
}

// Stripes onto `groups` row groups, longest first onto the least-loaded
// (load: entries plus a store); each group's list longest first.
std::vector<std::vector<int32_t>> stripe_row_groups(const std::vector<int64_t>& cnt, int64_t groups) {
    constexpr int64_t kStoreCost = 2;
    std::vector<int32_t> order(cnt.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) { return cnt[x] > cnt[y]; });
    std::vector<std::vector<int32_t>> rows(groups);
    using Load = std::pair<int64_t, int64_t>;
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int64_t g = 0; g < groups; ++g) heap.push({0, g});
    for (int32_t sr : order) {
        Load l = heap.top();
        heap.pop();
        rows[l.second].push_back(sr);
        heap.push({l.first + cnt[sr] + kStoreCost, l.second});
    }
    return rows;
}

}  // namespace

int64_t spmm_sweep_read_estimate(const bsp_bsr_desc* a, int64_t N, int col_groups) {
    if (col_groups < 1 || kNumXcd % col_groups) return INT64_MAX;
    const std::vector<int64_t> cnt = stripe_entries(a);
    const auto rows = stripe_row_groups(cnt, kNumXcd / col_groups);
    const int64_t RS = a->R / kSub, nbc = a->W / a->C;
    std::vector<int32_t> seen(nbc, -1);
    int64_t b_bytes = 0;
    for (size_t g = 0; g < rows.size(); ++g) {
        int64_t distinct = 0;
        for (int32_t sr : rows[g]) {
            const int64_t i = sr / RS;
            for (int64_t blk = a->indptr[i]; blk < a->indptr[i + 1]; ++blk)
                if (seen[a->indices[blk]] != (int32_t)g) {
                    seen[a->indices[blk]] = (int32_t)g;
                    ++distinct;
                }
        }
        b_bytes += distinct * a->C * N * 2;
    }
    return col_groups * a->nblocks * a->R * a->C * 2 + b_bytes;
}

int build_spmm_sweep(const bsp_bsr_desc* a, int64_t N, int num_cus, SpmmSweep& s, std::string& msg,
                     int col_groups) {
    int st = validate_bsr(a, msg);
    if (st != BSP_OK) return st;
    if (a->R % kSub || a->C % kSub) {
        msg = "R and C must be multiples of 32";
        return BSP_ERR_UNSUPPORTED;
    }
    if (N <= 0 || N % kSweepTile != 0 || N >= kSweepMaxN) {
        msg = "the sweep kernel needs N a positive multiple of 128 below 2^24";
        return BSP_ERR_UNSUPPORTED;
    }
    const int64_t RS = a->R / kSub, CS = a->C / kSub, nsr = a->H / kSub;
    if (a->nblocks * a->R * a->C / kSub > UINT32_MAX || a->nblocks * RS * CS * (N / kSweepTile) > INT32_MAX - kStreamPad ||
        a->W > INT32_MAX) {
        msg = "problem too large for the sweep schedule";
        return BSP_ERR_UNSUPPORTED;
    }
    if (num_cus <= 0) num_cus = 256;
    const int64_t n_tiles = N / kSweepTile;
    int64_t cg = col_groups;
    if (cg <= 0) {
        int64_t best = INT64_MAX;
        for (int64_t c = 1; c <= kNumXcd; c *= 2) {
            if (n_tiles % c) continue;
            const int64_t est = spmm_sweep_read_estimate(a, N, (int)c);
            if (est < best) {
                best = est;
                cg = c;
            }
        }
    }
    if (cg < 1 || kNumXcd % cg || n_tiles % cg) cg = 1;
    const std::vector<int64_t> cnt = stripe_entries(a);
    const bool balance = load_balance();
    std::vector<std::vector<int32_t>> rows;
    if (balance) {
        rows = stripe_row_groups(cnt, kNumXcd / cg);
    } else {  // contiguous ranges in stripe order
        rows.assign(kNumXcd / cg, {});
        for (int64_t i = 0; i < nsr; ++i) rows[i * (kNumXcd / cg) / nsr].push_back((int32_t)i);
    }
    const int64_t tpg = n_tiles / cg;
    const int cus_per_xcd = std::max(1, num_cus / kNumXcd);
    const bool rotate = env_int("BSP_SWEEP_ROTATE", 0) != 0;
    constexpr int64_t kStoreCost = 2;

    s = SpmmSweep{};
    s.n_tiles = (int32_t)n_tiles;
    s.col_groups = (int32_t)cg;
    s.rotated = rotate ? 1 : 0;
    s.wgs.assign((size_t)cus_per_xcd * kNumXcd, SpmmSweepWg{});
    struct Unit {
        int32_t row, n0;
        int64_t count;
    };
    struct Entry {
        int64_t brow;
        uint32_t aw;
        int32_t slot;
        int32_t n0;
    };
    for (int64_t r = 0; r < kNumXcd / cg; ++r)
        for (int64_t c = 0; c < cg; ++c) {
            const int x = (int)(r * cg + c);
            std::vector<Unit> us;
            for (int32_t sr : rows[r])  // longest first
                for (int64_t t = c * tpg; t < (c + 1) * tpg; ++t) us.push_back({sr, (int32_t)(t * kSweepTile), cnt[sr]});
            // Units onto the XCD's workgroups, longest first onto the
            // least-loaded one that has a free slot.
            const int64_t n_sw = std::max<int64_t>(1, ((int64_t)us.size() + (int64_t)cus_per_xcd * kSweepSlots - 1) /
                                                          ((int64_t)cus_per_xcd * kSweepSlots));
            const int64_t cap = n_sw * kSweepSlots;
            std::vector<std::vector<Unit>> per(cus_per_xcd);
            using Load = std::pair<int64_t, int>;
            if (balance) {
                std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
                for (int w = 0; w < cus_per_xcd; ++w) heap.push({0, w});
                for (const Unit& u : us) {
                    Load l = heap.top();
                    heap.pop();
                    per[l.second].push_back(u);
                    if ((int64_t)per[l.second].size() < cap) heap.push({l.first + u.count + kStoreCost, l.second});
                }
            } else if (!us.empty()) {  // contiguous ranges in order (at most cap each)
                for (size_t i = 0; i < us.size(); ++i) per[i * cus_per_xcd / us.size()].push_back(us[i]);
            }
            // Each workgroup's units into n_sw sweeps (unit i -> sweep i % n_sw,
            // longest first), its entries merged by first row of B.
            const int64_t stagger = env_int("BSP_SWEEP_STAGGER", 0);
            for (int w = 0; w < cus_per_xcd; ++w) {
                const int64_t kcol = ((rotate ? spmm_stream_rotation_column(a->W / a->C, c, cg) : 0) + stagger * w) %
                                     (a->W / a->C) * a->C;
                SpmmSweepWg& rec = s.wgs[(size_t)w * kNumXcd + x];
                rec.w_begin = (int32_t)s.bw.size();
                rec.s_begin = (int32_t)s.sweeps.size();
                const std::vector<Unit>& mine = per[w];
                for (int64_t sw = 0; sw < n_sw; ++sw) {
                    SpmmSweepRec sr{};
                    for (int g = 0; g < 2; ++g)
                        for (int j = 0; j < 8; ++j) {
                            sr.half[g].row[j] = -1;
                            sr.half[g].n0[j] = 0;
                        }
                    // The sweep's k-th unit (longest first) takes slot
                    // (k % 2) * 8 + k / 2, so that the two MFMA wave groups
                    // (slots 0-7 and 8-15) get alternate units and similar
                    // entry counts.
                    std::vector<Entry> es[2];
                    uint32_t used = 0;
                    int k = 0;
                    for (size_t ui = (size_t)sw; ui < mine.size(); ui += (size_t)n_sw, ++k) {
                        const Unit& u = mine[ui];
                        const int slot = (k % 2) * 8 + k / 2;
                        used |= 1u << slot;
                        sr.half[slot / 8].row[slot % 8] = u.row;
                        sr.half[slot / 8].n0[slot % 8] = u.n0;
                        const int64_t i = u.row / RS, sub = u.row % RS;
                        for (int64_t blk = a->indptr[i]; blk < a->indptr[i + 1]; ++blk)
                            for (int64_t t = 0; t < CS; ++t)
                                es[slot / 8].push_back({(int64_t)a->indices[blk] * a->C + kSub * t,
                                                        (uint32_t)((blk * a->R * a->C + kSub * sub * a->C + kSub * t) / kSub),
                                                        slot, u.n0});
                    }
                    if (k == 0) continue;  // no units left for this sweep
                    // The sweep's entries merged by first row of B (rotated to
                    // start at kcol); each unit's last entry in stream order
                    // carries the last bit (the kernel stores the unit's tile
                    // after it); units with no entries are marked in the
                    // record's empty mask.
                    std::vector<Entry> e = es[0];
                    e.insert(e.end(), es[1].begin(), es[1].end());
                    std::stable_sort(e.begin(), e.end(), [](const Entry& p, const Entry& q) { return p.brow < q.brow; });
                    if (kcol > 0) {
                        size_t off = 0;
                        while (off < e.size() && e[off].brow < kcol) ++off;
                        if (off == e.size()) off = 0;
                        std::rotate(e.begin(), e.begin() + off, e.end());
                    }
                    uint32_t has = 0;
                    std::vector<uint8_t> last(e.size(), 0);
                    for (size_t i = e.size(); i-- > 0;)
                        if (!(has & (1u << e[i].slot))) {
                            has |= 1u << e[i].slot;
                            last[i] = 1;
                        }
                    for (size_t i = 0; i < e.size(); ++i) {
                        s.bw.push_back(e[i].brow | ((int64_t)e[i].n0 << 32) | ((int64_t)e[i].slot << kSweepSlotShift) |
                                       (last[i] ? kSweepLast : 0));
                        s.aw.push_back(e[i].aw);
                    }
                    if (e.size() % 2) {  // pad to an even count
                        s.bw.push_back((s.bw.back() | kSweepSkip) & ~kSweepLast);
                        s.aw.push_back(s.aw.back());
                    }
                    sr.count = (int32_t)(e.size() + e.size() % 2);
                    sr.empty = (int32_t)(used & ~has);
                    s.sweeps.push_back(sr);
                    ++rec.n_sweeps;
                }
                rec.n = (int32_t)(s.bw.size() - rec.w_begin);
                s.max_wg_entries = std::max(s.max_wg_entries, rec.n);
                s.max_sweeps = std::max(s.max_sweeps, rec.n_sweeps);
                s.n_units += (int64_t)mine.size();
            }
        }
    s.n_entries = (int64_t)s.bw.size();
    s.bw.resize(s.bw.size() + kStreamPad, 0);
    s.aw.resize(s.aw.size() + kStreamPad, 0);
    SpmmSweepRec zero{};
    s.sweeps.resize(s.sweeps.size() + kStreamPad, zero);
    s.heads.assign(s.wgs.size(), SpmmSweepHead{});
    for (size_t g = 0; g < s.wgs.size(); ++g) {
        SpmmSweepHead& h = s.heads[g];
        h.wg = s.wgs[g];
        for (int j = 0; j < kHeadWords; ++j) {
            h.bw[j] = s.bw[(size_t)h.wg.w_begin + j];
            h.aw[j] = s.aw[(size_t)h.wg.w_begin + j];
        }
    }
    return BSP_OK;
}

int build_sddmm_schedule(const bsp_bsr_desc* m, int64_t K, int num_cus, SddmmSchedule& s,
                         std::string& msg) {
    int st = validate_bsr(m, msg);
    if (st != BSP_OK) return st;
    if (K <= 0) {
        msg = "K must be positive";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    if (m->R % kSub || m->C % kSub || K % kSub) {
        msg = "R, C and K must be multiples of 32";
        return BSP_ERR_UNSUPPORTED;
    }
    if (num_cus <= 0) num_cus = 256;
    const int64_t RS = m->R / kSub, CS = m->C / kSub;
    const int64_t nsr = m->H / kSub;
    const int64_t total = m->nblocks * RS * CS;
    if (total > INT32_MAX || m->W > INT32_MAX || m->H > INT32_MAX) {
        msg = "problem too large for int32 schedule fields";
        return BSP_ERR_UNSUPPORTED;
    }
    // Entries per item (all four waves work on each entry in turn): about two
    // workgroups per compute unit, at most 4 (measured best for 1600-2700
    // entries on 256 compute units).
    int64_t q = (total + 2 * num_cus - 1) / (2 * (int64_t)num_cus);
    q = std::min<int64_t>(4, std::max<int64_t>(1, q));
    q = env_int("BSP_SDDMM_CHUNK", q);
    q = std::min<int64_t>(64, std::max<int64_t>(1, q));  // the kernel holds an item's entries in one wave
    s.chunk = (int32_t)q;

    // Items and the workgroup map for `bands` contiguous bands of mask
    // columns: XCD x = row_group * bands + band runs the items of its row
    // group's stripes that fall in its band (one band: items longest first
    // over all XCDs).  An item is a run of at most q entries of one stripe
    // and one band.
    const int64_t ncol32 = m->W / kSub;
    auto build = [&](int64_t bands, bool by_items, SddmmSchedule& o) {
        o.chunk = (int32_t)q;
        o.items.clear();
        o.ent_col.clear();
        o.ent_off.clear();
        o.ent_col.reserve(total);
        o.ent_off.reserve(total);
        o.max_item_entries = 0;
        std::vector<int64_t> cost;
        std::vector<int32_t> item_band, item_stripe;
        std::vector<int64_t> stripe_cost(nsr, 0);
        std::vector<std::pair<int32_t, int64_t>> ents;
        for (int64_t sr = 0; sr < nsr; ++sr) {
            const int64_t i = sr / RS, sub = sr % RS;
            ents.clear();
            for (int64_t blk = m->indptr[i]; blk < m->indptr[i + 1]; ++blk)
                for (int64_t t = 0; t < CS; ++t)
                    ents.push_back({(int32_t)((int64_t)m->indices[blk] * m->C + kSub * t),
                                    blk * m->R * m->C + kSub * sub * m->C + kSub * t});
            for (int64_t band = 0; band < bands; ++band) {
                const int32_t e0 = (int32_t)o.ent_col.size();
                for (const auto& [col, off] : ents)
                    if ((col / kSub) * bands / ncol32 == band) {
                        o.ent_col.push_back(col);
                        o.ent_off.push_back(off);
                    }
                const int32_t e1 = (int32_t)o.ent_col.size();
                for (int32_t b = e0; b < e1; b += (int32_t)q) {
                    const int32_t b1 = std::min<int32_t>(e1, b + (int32_t)q);
                    o.items.push_back({(int32_t)(sr * kSub), b, b1, 0});
                    cost.push_back((b1 - b) + 1);
                    item_band.push_back((int32_t)band);
                    item_stripe.push_back((int32_t)sr);
                    stripe_cost[sr] += (b1 - b) + 1;
                    o.max_item_entries = std::max<int32_t>(o.max_item_entries, b1 - b);
                }
            }
        }
        if (bands == 1) {
            o.wgmap = xcd_lpt_map(cost, 1);
            return;
        }
        // Stripes onto the 8 / bands row groups: longest first onto the
        // least-loaded group (by_items false), or, so that every XCD's item
        // count stays within one round of workgroups, most items first onto
        // the group whose fullest XCD would hold the fewest items afterwards
        // (by_items true; a stripe adds items to one XCD per band).
        const int rgs = (int)(kNumXcd / bands);
        std::vector<int32_t> order(nsr);
        std::iota(order.begin(), order.end(), 0);
        std::vector<int32_t> stripe_rg(nsr, 0);
        if (!by_items) {
            std::stable_sort(order.begin(), order.end(),
                             [&](int32_t x, int32_t y) { return stripe_cost[x] > stripe_cost[y]; });
            std::vector<int64_t> load(rgs, 0);
            for (int32_t sr : order) {
                const int g = (int)(std::min_element(load.begin(), load.end()) - load.begin());
                stripe_rg[sr] = g;
                load[g] += stripe_cost[sr];
            }
        } else {
            std::vector<int64_t> n_items(nsr * bands, 0);  // items of stripe sr in band b
            for (size_t u = 0; u < o.items.size(); ++u) ++n_items[(int64_t)item_stripe[u] * bands + item_band[u]];
            std::vector<int64_t> tot(nsr, 0), most(nsr, 0);
            for (int64_t sr = 0; sr < nsr; ++sr)
                for (int64_t b = 0; b < bands; ++b) {
                    tot[sr] += n_items[sr * bands + b];
                    most[sr] = std::max(most[sr], n_items[sr * bands + b]);
                }
            std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) {
                return tot[x] != tot[y] ? tot[x] > tot[y] : most[x] > most[y];
            });
            std::vector<int64_t> load(rgs * bands, 0);
            for (int32_t sr : order) {
                int best = 0;
                int64_t best_max = INT64_MAX, best_sum = INT64_MAX;
                for (int g = 0; g < rgs; ++g) {
                    int64_t mx = 0, sum = 0;
                    for (int64_t b = 0; b < bands; ++b) {
                        const int64_t v = load[g * bands + b] + n_items[sr * bands + b];
                        mx = std::max(mx, v);
                        sum += v;
                    }
                    if (mx < best_max || (mx == best_max && sum < best_sum)) best = g, best_max = mx, best_sum = sum;
                }
                stripe_rg[sr] = best;
                for (int64_t b = 0; b < bands; ++b) load[best * bands + b] += n_items[sr * bands + b];
            }
        }
        std::vector<std::vector<int32_t>> bins(kNumXcd);
        for (size_t u = 0; u < o.items.size(); ++u)
            bins[stripe_rg[item_stripe[u]] * bands + item_band[u]].push_back((int32_t)u);
        size_t maxlen = 0;
        for (auto& b : bins) {
            std::stable_sort(b.begin(), b.end(), [&](int32_t x, int32_t y) { return cost[x] > cost[y]; });
            maxlen = std::max(maxlen, b.size());
        }
        o.wgmap.assign(maxlen * kNumXcd, -1);
        for (int x = 0; x < kNumXcd; ++x)
            for (size_t j = 0; j < bins[x].size(); ++j) o.wgmap[j * kNumXcd + x] = bins[x][j];
    };
    // The band count: the fewest rounds of resident workgroups (the one-shot
    // kernel fits 160 KB / (320 K) per compute unit), then the least data the
    // busiest XCD's L2 must fetch (its distinct X stripes and Y column blocks,
    // 64 K bytes each).  A banded mask (rows that reach nearby columns only)
    // gains; a uniform one mostly does not.
    const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(8, (160 * 1024) / (320 * K)));
    const int64_t slots = per_cu * num_cus;
    int64_t best_bands = 1, best_rounds = 0, best_bytes = 0;
    bool best_by_items = false;
    const int64_t forced = env_int("BSP_SDDMM_XCD_COLS", 0);
    for (int64_t cand = 0; cand < 5; ++cand) {
        const int64_t bands = cand == 0 ? 1 : (cand + 1) / 2 * 2;  // 1, 2, 2, 4, 4
        const bool by_items = cand > 0 && cand % 2 == 0;
        if (forced && bands != forced) continue;
        if (bands > 1 && ncol32 < 2 * bands) continue;
        SddmmSchedule t;
        build(bands, by_items, t);
        const int64_t rounds = ((int64_t)t.wgmap.size() + slots - 1) / slots;
        int64_t worst = 0;
        for (int x = 0; x < kNumXcd; ++x) {
            std::vector<char> xs(nsr, 0), ys(ncol32, 0);
            int64_t n = 0;
            for (size_t j = x; j < t.wgmap.size(); j += kNumXcd) {
                const int32_t u = t.wgmap[j];
                if (u < 0) continue;
                const SddmmItem& it = t.items[u];
                if (!xs[it.x_row0 / kSub]) xs[it.x_row0 / kSub] = 1, ++n;
                for (int32_t e = it.e_begin; e < it.e_end; ++e)
                    if (!ys[t.ent_col[e] / kSub]) ys[t.ent_col[e] / kSub] = 1, ++n;
            }
            worst = std::max(worst, n * 64 * K);
        }
        if (best_rounds == 0 || rounds < best_rounds || (rounds == best_rounds && worst < best_bytes)) {
            best_bands = bands;
            best_by_items = by_items;
            best_rounds = rounds;
            best_bytes = worst;
        }
    }
    build(best_bands, best_by_items, s);
    return BSP_OK;
}

namespace {

int check_spgemm_operands(const bsp_bsr_desc* a, const bsp_bsr_desc* b, std::string& msg) {
    int st = validate_bsr(a, msg);
    if (st != BSP_OK) {
        msg = "A: " + msg;
        return st;
    }
    st = validate_bsr(b, msg);
    if (st != BSP_OK) {
        msg = "B: " + msg;
        return st;
    }
    // The golden asserts these (sparse_common/bsr_matrix.hpp:742-743).
    if (a->W != b->H || a->C != b->R) {
        msg = "A's columns and block width must equal B's rows and block height";
        return BSP_ERR_INVALID_ARGUMENT;
    }
    if (a->R % kSub || a->C % kSub || b->C % kSub) {
        msg = "block sizes must be multiples of 32";
        return BSP_ERR_UNSUPPORTED;
    }
    return BSP_OK;
}

// Walks block row i of C: calls emit(j, pairs) for each output column j in
// ascending order with the (A block, B block) pairs of C(i, j) in the
// golden's order.  mark/cnt/pos are nbc-sized scratch (mark starts at -1).
template <class Emit>
void spgemm_row(const bsp_bsr_desc* a, const bsp_bsr_desc* b, int64_t i, std::vector<int64_t>& mark,
                std::vector<int32_t>& cnt, std::vector<int64_t>& pos, std::vector<int32_t>& cols,
                std::vector<std::pair<int32_t, int32_t>>& pairs, bool want_pairs, Emit&& emit) {
    cols.clear();
    int64_t npairs = 0;
    for (int64_t ai = a->indptr[i]; ai < a->indptr[i + 1]; ++ai) {
        const int64_t k = a->indices[ai];
        for (int64_t bi = b->indptr[k]; bi < b->indptr[k + 1]; ++bi) {
            const int32_t j = b->indices[bi];
            if (mark[j] != i) {
                mark[j] = i;
                cnt[j] = 0;
                cols.push_back(j);
            }
            ++cnt[j];
            ++npairs;
        }
    }
    std::sort(cols.begin(), cols.end());
    if (want_pairs) {
        int64_t run = 0;
        for (int32_t j : cols) {
            pos[j] = run;
            run += cnt[j];
        }
        pairs.resize(npairs);
        for (int64_t ai = a->indptr[i]; ai < a->indptr[i + 1]; ++ai) {
            const int64_t k = a->indices[ai];
            for (int64_t bi = b->indptr[k]; bi < b->indptr[k + 1]; ++bi)
                pairs[pos[b->indices[bi]]++] = {(int32_t)ai, (int32_t)bi};
        }
    }
    int64_t start = 0;
    for (int32_t j : cols) {
        emit(j, want_pairs ? pairs.data() + start : nullptr, cnt[j]);
        start += cnt[j];
    }
}

}  // namespace

int spgemm_symbolic(const bsp_bsr_desc* a, const bsp_bsr_desc* b, std::vector<int32_t>& indptr,
                    std::vector<int32_t>& indices, std::string& msg) {
    int st = check_spgemm_operands(a, b, msg);
    if (st != BSP_OK) return st;
    const int64_t nbr = a->H / a->R, nbc = b->W / b->C;
    std::vector<int64_t> mark(nbc, -1), pos;
    std::vector<int32_t> cnt(nbc), cols;
    std::vector<std::pair<int32_t, int32_t>> pairs;
    indptr.assign(nbr + 1, 0);
    indices.clear();
    for (int64_t i = 0; i < nbr; ++i) {
        spgemm_row(a, b, i, mark, cnt, pos, cols, pairs, false,
                   [&](int32_t j, const std::pair<int32_t, int32_t>*, int32_t) { indices.push_back(j); });
        if ((int64_t)indices.size() > INT32_MAX) {
            msg = "output has more than 2^31 - 1 blocks";
            return BSP_ERR_UNSUPPORTED;
        }
        indptr[i + 1] = (int32_t)indices.size();
    }
    return BSP_OK;
}

int build_spgemm_schedule(const bsp_bsr_desc* a, const bsp_bsr_desc* b, int num_cus, int stages, int rounds,
                          SpgemmSchedule& s, std::string& msg) {
    int st = check_spgemm_operands(a, b, msg);
    if (st != BSP_OK) return st;
    const int64_t R = a->R, C = a->C, BC = b->C;
    // Sub-block offsets are kept / 32 in 32 bits.
    if (a->nblocks * R * C / kSub > (int64_t)UINT32_MAX || b->nblocks * C * BC / kSub > (int64_t)UINT32_MAX) {
        msg = "A or B has more than 2^37 values";
        return BSP_ERR_UNSUPPORTED;
    }
    const int64_t nbr = a->H / R, nbc = b->W / BC;
    const int64_t RS = R / kSub, CS = C / kSub, PS = BC / kSub;
    std::vector<int64_t> mark(nbc, -1), pos(nbc);
    std::vector<int32_t> cnt(nbc), cols;
    std::vector<std::pair<int32_t, int32_t>> pairs;
    s = SpgemmSchedule{};
    s.indptr.assign(nbr + 1, 0);
    std::vector<int32_t> task_row, task_col;  // output block row / column of each task
    bool too_big = false;
    for (int64_t i = 0; i < nbr && !too_big; ++i) {
        spgemm_row(a, b, i, mark, cnt, pos, cols, pairs, true,
                   [&](int32_t j, const std::pair<int32_t, int32_t>* pr, int32_t np) {
                       const int64_t ob = (int64_t)s.indices.size();
                       s.indices.push_back(j);
                       if ((int64_t)s.terms.size() + (int64_t)np * CS * RS * PS > INT32_MAX) {
                           too_big = true;
                           return;
                       }
                       for (int64_t ra = 0; ra < RS; ++ra)
                           for (int64_t pb = 0; pb < PS; ++pb) {
                               SpgemmTask t{};
                               t.out_off = ob * R * BC + ra * kSub * BC + pb * kSub;
                               t.t_begin = (int32_t)s.terms.size();
                               for (int32_t n = 0; n < np; ++n)
                                   for (int64_t cs = 0; cs < CS; ++cs) {
                                       const uint64_t ao = (uint64_t)pr[n].first * R * C + ra * kSub * C + cs * kSub;
                                       const uint64_t bo =
                                           (uint64_t)pr[n].second * C * BC + cs * kSub * BC + pb * kSub;
                                       s.terms.push_back(ao / kSub | (bo / kSub) << 32);
                                   }
                               t.t_end = (int32_t)s.terms.size();
                               s.max_task_terms = std::max(s.max_task_terms, t.t_end - t.t_begin);
                               s.tasks.push_back(t);
                               task_row.push_back((int32_t)i);
                               task_col.push_back(j);
                           }
                   });
        if ((int64_t)s.indices.size() > INT32_MAX) too_big = true;
        s.indptr[i + 1] = (int32_t)s.indices.size();
    }
    if (too_big || (int64_t)s.tasks.size() > INT32_MAX) {
        msg = "product too large for int32 schedule fields";
        return BSP_ERR_UNSUPPORTED;
    }
    s.nblocks = (int64_t)s.indices.size();
    const int64_t ntask = (int64_t)s.tasks.size();
    if (num_cus <= 0) num_cus = 256;
    auto cost = [&](const SpgemmTask& t) -> int64_t { return (t.t_end - t.t_begin) + 2; };
    int64_t total = 0;
    for (const SpgemmTask& t : s.tasks) total += cost(t);

    // XCD regions: the output block rows are cut into RG groups of about
    // equal cost and, inside each row group, the output block columns into
    // CG = 8 / RG groups; region x = rg * CG + cg runs on XCD x.  An XCD then
    // reads the A blocks of its rows that meet its columns and the B blocks
    // of its columns that meet its rows: about CG * |A| + RG * |B| in all
    // (a split by rows alone reads B into every XCD's L2).  RG minimises
    // that sum; BSP_SPGEMM_XCD_ROWS overrides it.
    const int64_t bytes_a = a->nblocks * R * C, bytes_b = b->nblocks * C * BC;
    int RG = 8;
    for (int g : {4, 2, 1})
        if ((kNumXcd / g) * bytes_a + g * bytes_b < (kNumXcd / RG) * bytes_a + RG * bytes_b) RG = g;
    const int64_t rg_env = env_int("BSP_SPGEMM_XCD_ROWS", 0);
    if (rg_env == 1 || rg_env == 2 || rg_env == 4 || rg_env == 8) RG = (int)rg_env;
    const int CG = kNumXcd / RG;
    std::vector<int64_t> row_cost(nbr, 0);
    for (int64_t t = 0; t < ntask; ++t) row_cost[task_row[t]] += cost(s.tasks[t]);
    std::vector<int32_t> row_group(nbr);
    {
        int64_t run = 0;
        for (int64_t r = 0; r < nbr; ++r) {
            row_group[r] = (int32_t)std::min<int64_t>(RG - 1, total ? run * RG / total : 0);
            run += row_cost[r];
        }
    }
    std::vector<int64_t> col_cost((size_t)RG * nbc, 0), group_total(RG, 0);
    for (int64_t t = 0; t < ntask; ++t) {
        const int g = row_group[task_row[t]];
        col_cost[(size_t)g * nbc + task_col[t]] += cost(s.tasks[t]);
        group_total[g] += cost(s.tasks[t]);
    }
    std::vector<int32_t> col_group((size_t)RG * nbc);
    for (int g = 0; g < RG; ++g) {
        int64_t run = 0;
        for (int64_t c = 0; c < nbc; ++c) {
            col_group[(size_t)g * nbc + c] =
                (int32_t)std::min<int64_t>(CG - 1, group_total[g] ? run * CG / group_total[g] : 0);
            run += col_cost[(size_t)g * nbc + c];
        }
    }
    // Tasks (and their products) reordered by region, output order inside one.
    std::vector<int32_t> region(ntask);
    std::vector<int64_t> region_cost(kNumXcd, 0);
    std::vector<int32_t> region_count(kNumXcd + 1, 0);
    for (int64_t t = 0; t < ntask; ++t) {
        const int g = row_group[task_row[t]];
        region[t] = g * CG + col_group[(size_t)g * nbc + task_col[t]];
        region_cost[region[t]] += cost(s.tasks[t]);
        ++region_count[region[t] + 1];
    }
    for (int x = 0; x < kNumXcd; ++x) region_count[x + 1] += region_count[x];
    {
        std::vector<int32_t> next(region_count.begin(), region_count.end() - 1);
        std::vector<SpgemmTask> tasks(ntask);
        std::vector<uint64_t> terms;
        terms.reserve(s.terms.size());
        std::vector<int32_t> order(ntask);
        for (int64_t t = 0; t < ntask; ++t) order[next[region[t]]++] = (int32_t)t;
        for (int64_t u = 0; u < ntask; ++u) {
            const SpgemmTask& o = s.tasks[order[u]];
            tasks[u].out_off = o.out_off;
            tasks[u].t_begin = (int32_t)terms.size();
            terms.insert(terms.end(), s.terms.begin() + o.t_begin, s.terms.begin() + o.t_end);
            tasks[u].t_end = (int32_t)terms.size();
        }
        s.tasks.swap(tasks);
        s.terms.swap(terms);
    }

    // Wave runs: contiguous task ranges of one region of about equal cost
    // (products, plus the store counted as two products), `rounds` times as
    // many in all as waves fit the GPU, each at most kSpgemmRunTasks tasks;
    // a region's share follows its cost.  Run slot (x * wg_per_xcd + j) * 4
    // + wave belongs to a workgroup on XCD x and holds region x's runs.
    rounds = std::min(16, std::max(1, rounds));
    const int64_t nw = std::max<int64_t>(
        1, std::min<int64_t>(ntask, (int64_t)rounds * num_cus * spgemm_waves_per_cu(stages)));
    std::vector<std::vector<SpgemmRun>> region_runs(kNumXcd);
    for (int x = 0; x < kNumXcd; ++x) {
        const int64_t t_lo = region_count[x], t_hi = region_count[x + 1];
        if (t_lo == t_hi) continue;
        const int64_t want = std::max<int64_t>(1, total ? (nw * region_cost[x] + total - 1) / total : 1);
        const int64_t target = std::max<int64_t>(1, (region_cost[x] + want - 1) / want);
        int64_t acc = 0, begin = t_lo;
        for (int64_t t = t_lo; t < t_hi; ++t) {
            acc += cost(s.tasks[t]);
            if (acc >= target || t + 1 - begin == kSpgemmRunTasks || t + 1 == t_hi) {
                region_runs[x].push_back({(int32_t)begin, (int32_t)(t + 1), s.tasks[begin].t_begin, s.tasks[t].t_end});
                acc = 0;
                begin = t + 1;
            }
        }
    }
    int64_t per = 1;
    s.pieces = 0;
    for (int x = 0; x < kNumXcd; ++x) {
        per = std::max<int64_t>(per, ((int64_t)region_runs[x].size() + 3) / 4);
        s.pieces += (int32_t)region_runs[x].size();
    }
    s.wg_per_xcd = (int32_t)per;
    s.grid = (int32_t)(per * kNumXcd);
    const int32_t pend = ntask ? s.tasks.back().t_end : 0;
    s.runs.assign((size_t)s.grid * 4, SpgemmRun{(int32_t)ntask, (int32_t)ntask, pend, pend});
    for (int x = 0; x < kNumXcd; ++x)
        std::copy(region_runs[x].begin(), region_runs[x].end(), s.runs.begin() + (size_t)x * per * 4);
    return BSP_OK;
}

}  // namespace bsp
