// Host scheduler checks (tenstorrent-wh-blockspmm_amd/csrc/bsp_schedule.cpp),
// built with g++ from the scheduler's source alone: no device and no HIP.
//
// For SpMM, SDDMM and SpGEMM plans over generated structures (uniform,
// skewed, duplicate columns, empty rows, large and non-square blocks) it
// checks that the work lists the kernels walk are exact: every product of the
// reference's loops (block_spmm/inc/bsr_matrix.hpp:954-1000,
// sparse_common/bsr_matrix.hpp:816-857 and :741-810) appears once, in the
// reference's order within a row, with the right operand offsets; that the
// workgroup maps hold every unit once on the XCD its column group names; and
// that a compute unit's two workgroups pair a heavy row with a light one.
//
//   test_schedule          exit status 0 when every check passes
#include <algorithm>
#include <cstring>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "bsp_schedule.hpp"

using namespace bsp;

namespace {

int g_fail = 0;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        ++g_fail;
        if (g_fail < 40) std::printf("  FAIL: %s\n", what.c_str());
    }
}

struct Bsr {
    int64_t H, W, R, C;
    std::vector<int32_t> indptr, indices;
    bsp_bsr_desc desc() const {
        return {H, W, R, C, (int64_t)indices.size(), indptr.data(), indices.data()};
    }
};

// Uniform distinct positions, columns ascending per row.
Bsr uniform(int64_t H, int64_t W, int64_t R, int64_t C, int64_t nnzb, uint32_t seed) {
    std::mt19937 rng(seed);
    const int64_t nbr = H / R, nbc = W / C;
    std::vector<int64_t> all(nbr * nbc);
    for (int64_t i = 0; i < (int64_t)all.size(); ++i) all[i] = i;
    std::shuffle(all.begin(), all.end(), rng);
    all.resize(nnzb);
    std::sort(all.begin(), all.end());
    Bsr b{H, W, R, C, std::vector<int32_t>(nbr + 1, 0), {}};
    for (int64_t f : all) {
        ++b.indptr[f / nbc + 1];
        b.indices.push_back((int32_t)(f % nbc));
    }
    for (int64_t i = 0; i < nbr; ++i) b.indptr[i + 1] += b.indptr[i];
    return b;
}

// Rows drawn with a cubic skew; columns random with repeats (duplicates and
// unsorted columns, as the reference's FILL_COL produces).
Bsr skewed(int64_t H, int64_t W, int64_t R, int64_t C, int64_t nnzb, uint32_t seed) {
    std::mt19937 rng(seed);
    std::uniform_real_distribution<double> u(0.0, 1.0);
    const int64_t nbr = H / R, nbc = W / C;
    std::vector<std::vector<int32_t>> rows(nbr);
    for (int64_t k = 0; k < nnzb; ++k) {
        const double x = u(rng);
        rows[std::min<int64_t>(nbr - 1, (int64_t)(nbr * x * x * x))].push_back((int32_t)(rng() % nbc));
    }
    Bsr b{H, W, R, C, std::vector<int32_t>(nbr + 1, 0), {}};
    for (int64_t i = 0; i < nbr; ++i) {
        b.indptr[i + 1] = b.indptr[i] + (int32_t)rows[i].size();
        b.indices.insert(b.indices.end(), rows[i].begin(), rows[i].end());
    }
    return b;
}

// Causal block bands at offsets 0..-(bands-1) plus `extra` random blocks
// below the band (the fused attention pair's mask shape), columns ascending.
Bsr banded(int64_t n, int64_t blk, int bands, int extra, uint32_t seed) {
    std::mt19937 rng(seed);
    const int64_t nb = n / blk;
    std::vector<std::set<int32_t>> rows(nb);
    for (int64_t i = 0; i < nb; ++i)
        for (int d = 0; d < bands && i - d >= 0; ++d) rows[i].insert((int32_t)(i - d));
    for (int k = 0; k < extra; ++k) {
        const int64_t i = rng() % nb;
        if (i > bands) rows[i].insert((int32_t)(rng() % (i - bands)));
    }
    Bsr b{n, n, blk, blk, std::vector<int32_t>(nb + 1, 0), {}};
    for (int64_t i = 0; i < nb; ++i) {
        b.indptr[i + 1] = b.indptr[i] + (int32_t)rows[i].size();
        b.indices.insert(b.indices.end(), rows[i].begin(), rows[i].end());
    }
    return b;
}

void check_spmm(const Bsr& a, int64_t N, int cus, const std::string& name) {
    SpmmSchedule s;
    std::string msg;
    const bsp_bsr_desc d = a.desc();
    const int st = build_spmm_schedule(&d, N, cus, s, msg);
    expect(st == BSP_OK, name + ": build " + msg);
    if (st != BSP_OK) return;
    const int64_t RS = a.R / kSub, CS = a.C / kSub, G = s.group;
    expect(G >= 1 && RS % G == 0, name + ": group divides R/32");
    // Entries: per group of stripes, the blocks of the row in CSR order and
    // their 32-column steps; B row and A sub-block offset of each.
    std::vector<int32_t> want_row;
    std::vector<int64_t> want_off;
    std::vector<int64_t> stripe_begin;
    for (int64_t sr = 0; sr < a.H / kSub; sr += G) {
        stripe_begin.push_back((int64_t)want_row.size());
        const int64_t i = sr / RS, sub = sr % RS;
        for (int64_t blk = a.indptr[i]; blk < a.indptr[i + 1]; ++blk)
            for (int64_t t = 0; t < CS; ++t) {
                want_row.push_back((int32_t)(a.indices[blk] * a.C + kSub * t));
                want_off.push_back(blk * a.R * a.C + kSub * sub * a.C + kSub * t);
            }
    }
    stripe_begin.push_back((int64_t)want_row.size());
    expect(s.ent_row == want_row, name + ": entry B rows");
    expect(s.ent_off == want_off, name + ": entry A offsets");
    const std::vector<int64_t> packed = spmm_packed_entries(s);
    bool pk = packed.size() == want_row.size();
    for (size_t e = 0; pk && e < packed.size(); ++e)
        pk = (uint32_t)packed[e] == (uint32_t)want_row[e] && (packed[e] >> 32) == want_off[e] / kSub;
    expect(pk, name + ": packed entries");
    // Items partition each stripe group's entries in order; split pieces
    // stay within the split limit and own consecutive slots.
    std::map<int32_t, std::vector<const SpmmItem*>> by_row;
    for (const SpmmItem& it : s.items) by_row[it.row].push_back(&it);
    int64_t covered = 0;
    for (auto& [row, its] : by_row) {
        expect(row % G == 0, name + ": item row aligned to the group");
        const int64_t gi = row / G;
        int64_t at = stripe_begin[gi];
        for (size_t k = 0; k < its.size(); ++k) {
            expect(its[k]->e_begin == at, name + ": items contiguous");
            if (a.C % 64 == 0)
                expect((its[k]->e_begin - stripe_begin[gi]) % 2 == 0, name + ": items start at an even entry (A pairs)");
            at = its[k]->e_end;
            covered += its[k]->e_end - its[k]->e_begin;
            if (its.size() > 1) {
                expect(its[k]->slot == its[0]->base + (int32_t)k, name + ": piece slots consecutive");
                expect(its[k]->npieces == (int32_t)its.size(), name + ": piece count");
                expect(its[k]->e_end - its[k]->e_begin <= s.split_limit, name + ": piece within the limit");
            } else {
                expect(its[k]->slot == -1, name + ": whole row has no slot");
            }
        }
        expect(at == stripe_begin[gi + 1], name + ": items end at the stripe group's end");
    }
    expect(covered == (int64_t)want_row.size(), name + ": items cover every entry once");
    // Workgroup map: every (item, tile) once; the tile's column group names
    // the XCD's column group; all tiles of a column group of one item share
    // an XCD.
    const int64_t nunits = (int64_t)s.items.size() * s.n_tiles;
    expect(s.wgmap.size() % kNumXcd == 0, name + ": grid multiple of 8");
    std::vector<int> seen(nunits, 0);
    std::vector<int> xcd_of(nunits, -1);
    const int cg = s.xcd_col_groups, tpg = s.n_tiles / cg;
    for (size_t g = 0; g < s.wgmap.size(); ++g) {
        const int32_t u = s.wgmap[g];
        if (u < 0) continue;
        expect(u < nunits, name + ": unit in range");
        if (u >= nunits) continue;
        ++seen[u];
        xcd_of[u] = (int)(g % kNumXcd);
        expect((int)(g % kNumXcd) % cg == (u % s.n_tiles) / tpg, name + ": tile on its column group's XCD");
    }
    bool once = true;
    for (int64_t u = 0; u < nunits; ++u) once = once && seen[u] == 1;
    expect(once, name + ": every unit mapped once");
    for (size_t it = 0; it < s.items.size(); ++it)
        for (int t = 1; t < s.n_tiles; ++t)
            if (t / tpg == (t - 1) / tpg)
                expect(xcd_of[it * s.n_tiles + t] == xcd_of[it * s.n_tiles + t - 1], name + ": item's tiles share an XCD");
    const std::vector<SpmmWg> recs = spmm_wg_records(s);
    bool rec_ok = recs.size() == s.wgmap.size();
    for (size_t g = 0; rec_ok && g < recs.size(); ++g) {
        const int32_t u = s.wgmap[g];
        if (u < 0) {
            rec_ok = recs[g].row == -1;
            continue;
        }
        const SpmmItem& it = s.items[u / s.n_tiles];
        rec_ok = recs[g].row == it.row && recs[g].e_begin == it.e_begin && recs[g].e_end == it.e_end &&
                 recs[g].slot == it.slot && recs[g].tile == u % s.n_tiles;
    }
    expect(rec_ok, name + ": workgroup records follow the map");
    const std::vector<SpmmSplit> splits = spmm_splits(s);
    expect((int64_t)splits.size() == s.n_split_rows, name + ": one split record per split stripe");
    std::printf("%-34s items %5zu tiles %d grid %5zu split rows %3d group %d\n", name.c_str(), s.items.size(),
                s.n_tiles, s.wgmap.size(), s.n_split_rows, s.group);
}

// The pairing of a compute unit's two workgroups: on a longest-first XCD
// list of C < len <= 2C units, the first round (slots j < C) stays longest
// first and the second round runs shortest first, so slot j's partner at
// j + C is the (len - 1 - j)-th longest.
void check_pairing() {
    std::vector<int32_t> bin(48);
    for (int i = 0; i < 48; ++i) bin[i] = i;
    pair_rounds(bin, 32);
    bool ok = true;
    for (int j = 0; j < 32; ++j) ok = ok && bin[j] == j;
    for (int j = 0; j < 16; ++j) ok = ok && bin[32 + j] == 47 - j;
    expect(ok, "pair_rounds: second round reversed");
    std::vector<int32_t> one(32), three(65);
    for (int i = 0; i < 32; ++i) one[i] = i;
    for (int i = 0; i < 65; ++i) three[i] = i;
    std::vector<int32_t> one0 = one, three0 = three;
    pair_rounds(one, 32);
    pair_rounds(three, 32);
    expect(one == one0 && three == three0, "pair_rounds: one round or more than two left alone");
    // Through the map: 64 items of distinct costs on one column group give
    // each XCD 8 items x 4 tiles = 32 units for 4 compute units per XCD,
    // outside the window; 16 units (4 items x 4 tiles) against 8 units per
    // XCD are paired: per XCD, unit costs fall over the first 8 slots and
    // rise over the next 8.
    std::vector<int64_t> cost(32);
    for (int i = 0; i < 32; ++i) cost[i] = 1000 - 7 * i;
    const std::vector<int32_t> map = xcd_tile_map(cost, 4, 1, 8);
    bool shape = map.size() == 16 * kNumXcd;
    for (int x = 0; shape && x < kNumXcd; ++x) {
        std::vector<int64_t> c;
        for (int j = 0; j < 16; ++j) c.push_back(cost[map[j * kNumXcd + x] / 4]);
        for (int j = 1; j < 8; ++j) shape = shape && c[j] <= c[j - 1];
        for (int j = 9; j < 16; ++j) shape = shape && c[j] >= c[j - 1];
        // partners: the heaviest with the lightest
        shape = shape && c[0] == *std::max_element(c.begin(), c.end()) &&
                c[8] == *std::min_element(c.begin(), c.end());
    }
    expect(shape, "xcd_tile_map: heavy units paired with light ones");
    std::printf("%-34s %s\n", "pairing", "checked");
}

void check_sddmm(const Bsr& m, int64_t K, int cus, const std::string& name) {
    SddmmSchedule s;
    std::string msg;
    const bsp_bsr_desc d = m.desc();
    const int st = build_sddmm_schedule(&d, K, cus, s, msg);
    expect(st == BSP_OK, name + ": build " + msg);
    if (st != BSP_OK) return;
    const int64_t RS = m.R / kSub, CS = m.C / kSub;
    std::vector<int32_t> want_col;
    std::vector<int64_t> want_off, want_x;
    for (int64_t sr = 0; sr < m.H / kSub; ++sr) {
        const int64_t i = sr / RS, sub = sr % RS;
        for (int64_t blk = m.indptr[i]; blk < m.indptr[i + 1]; ++blk)
            for (int64_t t = 0; t < CS; ++t) {
                want_col.push_back((int32_t)(m.indices[blk] * m.C + kSub * t));
                want_off.push_back(blk * m.R * m.C + kSub * sub * m.C + kSub * t);
                want_x.push_back(sr * kSub);
            }
    }
    // Within a stripe the entries may be grouped by column band (the map's
    // XCD split); across the list, each (X rows, Y column, output offset)
    // triple appears once.
    std::vector<std::tuple<int64_t, int32_t, int64_t>> want_t, got_t;
    for (size_t e = 0; e < want_col.size(); ++e) want_t.emplace_back(want_x[e], want_col[e], want_off[e]);
    bool sizes = s.ent_col.size() == want_col.size() && s.ent_off.size() == want_off.size();
    expect(sizes, name + ": entry count");
    if (!sizes) return;
    std::vector<int64_t> ent_x(s.ent_col.size(), -1);
    for (const SddmmItem& it : s.items)
        for (int32_t e = it.e_begin; e < it.e_end && e < (int32_t)ent_x.size(); ++e) ent_x[e] = it.x_row0;
    for (size_t e = 0; e < s.ent_col.size(); ++e) got_t.emplace_back(ent_x[e], s.ent_col[e], s.ent_off[e]);
    std::sort(want_t.begin(), want_t.end());
    std::sort(got_t.begin(), got_t.end());
    expect(want_t == got_t, name + ": entries (X rows, Y column, output offset) once each");
    // Every output sub-block once (the offsets are distinct and tile the
    // output values).
    std::set<int64_t> offs(want_off.begin(), want_off.end());
    expect((int64_t)offs.size() == (int64_t)want_off.size() &&
               (int64_t)want_off.size() == (int64_t)m.indices.size() * RS * CS,
           name + ": sub-blocks distinct");
    int64_t at = 0;
    bool items_ok = true;
    for (const SddmmItem& it : s.items) {
        items_ok = items_ok && it.e_begin == at && it.e_end > it.e_begin && it.e_end - it.e_begin <= s.chunk &&
                   it.x_row0 % kSub == 0 && it.x_row0 < m.H;
        at = it.e_end;
    }
    expect(items_ok && at == (int64_t)want_col.size(), name + ": items partition the entries");
    // An entry's output sub-block lies in its item's X rows: the block row
    // of ent_off is x_row0's.
    bool rows_ok = true;
    for (const SddmmItem& it : s.items)
        for (int32_t e = it.e_begin; e < it.e_end; ++e) {
            const int64_t blk = s.ent_off[e] / (m.R * m.C);
            const int64_t sub = (s.ent_off[e] % (m.R * m.C)) / (kSub * m.C);
            int64_t row = 0;
            while (row + 1 < (int64_t)m.indptr.size() && m.indptr[row + 1] <= blk) ++row;
            rows_ok = rows_ok && row * m.R + sub * kSub == it.x_row0;
        }
    expect(rows_ok, name + ": each entry in its item's stripe");
    std::vector<int> seen(s.items.size(), 0);
    for (int32_t u : s.wgmap)
        if (u >= 0 && u < (int32_t)s.items.size()) ++seen[u];
    expect(std::all_of(seen.begin(), seen.end(), [](int v) { return v == 1; }) && s.wgmap.size() % kNumXcd == 0,
           name + ": every item mapped once");
    std::printf("%-34s items %5zu chunk %d grid %5zu\n", name.c_str(), s.items.size(), s.chunk, s.wgmap.size());
}

void check_spgemm(const Bsr& a, const Bsr& b, int cus, const std::string& name) {
    SpgemmSchedule s;
    std::string msg;
    const bsp_bsr_desc da = a.desc(), db = b.desc();
    const int st = build_spgemm_schedule(&da, &db, cus, 3, 2, s, msg);
    expect(st == BSP_OK, name + ": build " + msg);
    if (st != BSP_OK) return;
    const int64_t R = a.R, C = a.C, BC = b.C, RS = R / kSub, CS = C / kSub, PS = BC / kSub;
    // Brute force: per output block row, the columns reached and the
    // (A block, B block) pairs in A's then B's CSR order.
    std::vector<int32_t> indptr{0}, indices;
    std::vector<uint64_t> terms;
    std::vector<SpgemmTask> tasks;
    for (int64_t i = 0; i < a.H / R; ++i) {
        std::map<int32_t, std::vector<std::pair<int32_t, int32_t>>> row;
        for (int32_t ai = a.indptr[i]; ai < a.indptr[i + 1]; ++ai) {
            const int32_t k = a.indices[ai];
            for (int32_t bi = b.indptr[k]; bi < b.indptr[k + 1]; ++bi) row[b.indices[bi]].push_back({ai, bi});
        }
        for (auto& [j, pairs] : row) {
            const int64_t ob = (int64_t)indices.size();
            indices.push_back(j);
            for (int64_t ra = 0; ra < RS; ++ra)
                for (int64_t pb = 0; pb < PS; ++pb) {
                    SpgemmTask t{ob * R * BC + ra * kSub * BC + pb * kSub, (int32_t)terms.size(), 0};
                    for (auto& [ai, bi] : pairs)
                        for (int64_t cs = 0; cs < CS; ++cs) {
                            const uint64_t ao = (uint64_t)ai * R * C + ra * kSub * C + cs * kSub;
                            const uint64_t bo = (uint64_t)bi * C * BC + cs * kSub * BC + pb * kSub;
                            terms.push_back(ao / kSub | (bo / kSub) << 32);
                        }
                    t.t_end = (int32_t)terms.size();
                    tasks.push_back(t);
                }
        }
        indptr.push_back((int32_t)indices.size());
    }
    expect(s.indptr == indptr && s.indices == indices, name + ": output structure");
    // The schedule orders tasks by XCD region; each output sub-block must
    // still be one task holding its products in the golden's order.
    std::map<int64_t, std::vector<uint64_t>> want, got;
    for (const SpgemmTask& t : tasks) want[t.out_off].assign(terms.begin() + t.t_begin, terms.begin() + t.t_end);
    bool tk = s.tasks.size() == tasks.size() && s.terms.size() == terms.size();
    for (const SpgemmTask& t : s.tasks) {
        tk = tk && t.t_begin <= t.t_end && t.t_end <= (int32_t)s.terms.size() && !got.count(t.out_off);
        if (tk) got[t.out_off].assign(s.terms.begin() + t.t_begin, s.terms.begin() + t.t_end);
    }
    expect(tk && got == want, name + ": each sub-block's products, in order");
    // Wave runs: grid * 4 slots, each task in exactly one run, the run's
    // products those of its tasks.
    expect(s.grid % kNumXcd == 0 && (int64_t)s.runs.size() == (int64_t)s.grid * 4, name + ": run slots");
    std::vector<int> seen(s.tasks.size(), 0);
    bool runs_ok = true;
    for (const SpgemmRun& r : s.runs) {
        if (r.t0 == r.t1) continue;
        runs_ok = runs_ok && r.t0 < r.t1 && r.t1 <= (int32_t)s.tasks.size() && r.t1 - r.t0 <= kSpgemmRunTasks &&
                  r.p0 == s.tasks[r.t0].t_begin && r.p1 == s.tasks[r.t1 - 1].t_end;
        for (int32_t t = r.t0; runs_ok && t < r.t1; ++t) ++seen[t];
    }
    expect(runs_ok && std::all_of(seen.begin(), seen.end(), [](int v) { return v == 1; }),
           name + ": runs cover every task once");
    std::printf("%-34s out blocks %5lld tasks %6zu products %7zu grid %d\n", name.c_str(), (long long)s.nblocks,
                s.tasks.size(), s.terms.size(), s.grid);
}

// Persistent SpMM schedule: every (stripe, tile) unit appears once, on the
// XCD whose column group holds its tile; each unit's stream entries are the
// stripe's products in the reference's order (blocks in CSR order, then the
// 32-column steps of a block) with the right B row, column and A offset; the
// workgroup streams are contiguous and their lengths add up.  With two
// pipelines, a compute unit's two streams differ by at most one entry, and a
// unit cut between them is the first pipeline's last unit (flag 2) and the
// second's first (flag 1), the two parts covering its entries once, in order.
void check_spmm_stream(const Bsr& a, int64_t N, int cus, int tile_n, int wpc, const std::string& name, int pipes = 1) {
    SpmmStream s;
    std::string msg;
    const bsp_bsr_desc d = a.desc();
    const int st = build_spmm_stream(&d, N, cus, tile_n, wpc, s, msg, 0, pipes);
    expect(st == BSP_OK, name + ": build (" + msg + ")");
    if (st != BSP_OK) return;
    const int64_t RS = a.R / kSub, CS = a.C / kSub, nsr = a.H / kSub, n_tiles = N / tile_n;
    const int64_t grid = (int64_t)(cus / kNumXcd) * (pipes == 2 ? 1 : wpc) * kNumXcd;
    const char* rot_env = std::getenv("BSP_SPMM_ROTATE");
    expect(s.rotated == (pipes == 1 && !(rot_env && std::atoi(rot_env) == 0) ? 1 : 0),
           name + ": units rotated with one pipeline unless BSP_SPMM_ROTATE=0");
    expect((int64_t)s.wgs.size() == grid * pipes && s.heads.size() == s.wgs.size(), name + ": grid");
    std::vector<int> seen(nsr * n_tiles, 0);  // entries seen per unit (as a count of parts' coverage)
    std::vector<int64_t> covered(nsr * n_tiles, 0);
    int64_t w = 0, u = 0;
    const int64_t tpg = n_tiles / s.col_groups;
    for (size_t r = 0; r < s.wgs.size(); ++r) {
        const SpmmStreamWg& wg = s.wgs[r];
        const int64_t g = (int64_t)r / pipes, pipe = (int64_t)r % pipes;
        expect(wg.w_begin == w && wg.u_begin == u, name + ": contiguous streams");
        int64_t e = wg.w_begin, total = 0;
        for (int32_t j = 0; j < wg.n_units; ++j) {
            const SpmmStreamUnit& un = s.units[wg.u_begin + j];
            const int64_t tile = un.n0 / tile_n;
            expect(un.n0 % tile_n == 0 && tile < n_tiles && un.row < nsr, name + ": unit fields");
            expect(tile / tpg == (int64_t)((g % kNumXcd) % s.col_groups), name + ": unit on its column group's XCD");
            const int64_t i = un.row / RS, sub = un.row % RS;
            const int64_t full = (a.indptr[i + 1] - a.indptr[i]) * CS;
            int64_t e0 = 0, e1 = full;
            if (un.aux == 0) {
                expect(un.count == full, name + ": unit count");
                ++seen[un.row * n_tiles + tile];
            } else {
                expect(pipes == 2, name + ": flags only with two pipelines");
                expect(un.aux == 2 ? (pipe == 0 && j == wg.n_units - 1) : (pipe == 1 && j == 0),
                       name + ": cut unit is the first pipeline's last and the second's first");
                if (un.aux == 2) {
                    e1 = un.count;
                } else {
                    e0 = full - un.count;
                    ++seen[un.row * n_tiles + tile];
                }
            }
            covered[un.row * n_tiles + tile] += e1 - e0;
            std::vector<std::pair<int64_t, int64_t>> want;  // (B row, A offset) in CSR order
            int64_t idx = 0;
            for (int64_t blk = a.indptr[i]; blk < a.indptr[i + 1]; ++blk)
                for (int64_t t = 0; t < CS; ++t, ++idx)
                    if (idx >= e0 && idx < e1)
                        want.push_back({(int64_t)a.indices[blk] * a.C + kSub * t,
                                        blk * a.R * a.C + kSub * sub * a.C + kSub * t});
            if (s.rotated) {  // start at the first block column of the unit's rotation, wrapping around
                expect(pipes == 1, name + ": rotation with one pipeline only");
                const int64_t kcol = spmm_stream_rotation_column(a.W / a.C, tile / tpg, s.col_groups);
                size_t off = 0;
                while (off < want.size() && want[off].first / a.C < kcol) ++off;
                if (off == want.size()) off = 0;
                std::rotate(want.begin(), want.begin() + off, want.end());
            }
            for (const auto& wb : want) {
                expect((s.bw[e] & 0xffffffffLL) == wb.first && (s.bw[e] >> 32) == un.n0, name + ": B word");
                expect((int64_t)s.aw[e] * kSub == wb.second, name + ": A word");
                ++e;
            }
            total += un.count;
        }
        expect(total == wg.n && e == wg.w_begin + wg.n, name + ": stream length");
        // The head repeats the record, the first two unit records and the
        // first kHeadWords words of both streams (past the stream's end: the
        // arrays' padding or the next stream's words, as the kernel would
        // have read them from the arrays).
        const SpmmStreamHead& h = s.heads[r];
        expect(std::memcmp(&h.wg, &wg, sizeof wg) == 0, name + ": head record");
        for (int j = 0; j < 2; ++j)
            expect(std::memcmp(&h.u[j], &s.units[wg.u_begin + j], sizeof(SpmmStreamUnit)) == 0, name + ": head units");
        for (int j = 0; j < kHeadWords; ++j)
            expect(h.bw[j] == s.bw[wg.w_begin + j] && h.aw[j] == s.aw[wg.w_begin + j], name + ": head words");
        if (pipes == 2 && pipe == 1)
            expect(s.wgs[r - 1].n - wg.n == 0 || s.wgs[r - 1].n - wg.n == 1, name + ": halves within one entry");
        w += wg.n;
        u += wg.n_units;
    }
    expect(std::all_of(seen.begin(), seen.end(), [](int v) { return v == 1; }), name + ": every unit once");
    bool cov = true;
    for (int64_t sr = 0; sr < nsr; ++sr)
        for (int64_t t = 0; t < n_tiles; ++t) {
            const int64_t i = sr / RS;
            cov = cov && covered[sr * n_tiles + t] == (a.indptr[i + 1] - a.indptr[i]) * CS;
        }
    expect(cov, name + ": every entry of every unit once");
    expect(w == s.n_entries && (int64_t)s.bw.size() == w + kStreamPad && (int64_t)s.aw.size() == w + kStreamPad &&
               (int64_t)s.units.size() == u + kStreamPad,
           name + ": padding");
    std::printf("%-34s units %6lld entries %8lld grid %lld cg %d max wg %d\n", name.c_str(), (long long)u,
                (long long)s.n_entries, (long long)grid, s.col_groups, s.max_wg_entries);
}

}  // namespace

// Persistent SpMM with stripe pairs: the pairs cover every block row once
// (one odd row alone at most); every (pair, tile) unit appears once, on its
// column group's XCD; along a unit's entries the columns increase strictly,
// each entry holds a block of at least one of the two rows, a column that both
// rows hold is one entry with both, and each row's blocks appear once, in
// CSR order, with the right B row and A offset.  The heads repeat the records
// and the first words of the B and pair streams.
void check_spmm_stream_pairs(const Bsr& a, int64_t N, int cus, const std::string& name) {
    SpmmStream s;
    std::string msg;
    const bsp_bsr_desc d = a.desc();
    const int st = build_spmm_stream(&d, N, cus, 128, 1, s, msg, 0, 1, true);
    expect(st == BSP_OK, name + ": build (" + msg + ")");
    if (st != BSP_OK) return;
    expect(s.pairs == 1 && s.aw.empty(), name + ": pair streams");
    const int64_t nsr = a.H / kSub, n_tiles = N / 128, tpg = n_tiles / s.col_groups;
    std::vector<int> seen(nsr * n_tiles, 0);
    int64_t w = 0, u = 0;
    for (size_t g = 0; g < s.wgs.size(); ++g) {
        const SpmmStreamWg& wg = s.wgs[g];
        expect(wg.w_begin == w && wg.u_begin == u, name + ": contiguous streams");
        int64_t e = wg.w_begin;
        for (int32_t j = 0; j < wg.n_units; ++j) {
            const SpmmStreamUnit& un = s.units[wg.u_begin + j];
            const int64_t tile = un.n0 / 128;
            expect(un.row >= 0 && un.row < nsr && un.aux < nsr && un.aux != un.row && tile < n_tiles,
                   name + ": unit fields");
            expect(tile / tpg == (int64_t)((g % kNumXcd) % s.col_groups), name + ": unit on its column group's XCD");
            ++seen[un.row * n_tiles + tile];
            if (un.aux >= 0) ++seen[un.aux * n_tiles + tile];
            // The union in column order: one entry per column either row holds,
            // with each row's block there (or none), rotated like a single
            // stripe's unit.
            std::map<int32_t, std::pair<uint32_t, uint32_t>> uni;
            for (int h = 0; h < 2; ++h) {
                const int32_t row = h == 0 ? un.row : un.aux;
                if (row < 0) continue;
                for (int64_t blk = a.indptr[row]; blk < a.indptr[row + 1]; ++blk) {
                    auto it = uni.emplace(a.indices[blk], std::make_pair(kNoBlock, kNoBlock)).first;
                    (h == 0 ? it->second.first : it->second.second) = (uint32_t)(blk * a.R * a.C / kSub);
                }
            }
            std::vector<std::pair<int32_t, std::pair<uint32_t, uint32_t>>> want(uni.begin(), uni.end());
            if (s.rotated) {
                const int64_t kcol = spmm_stream_rotation_column(a.W / a.C, tile / tpg, s.col_groups);
                size_t off = 0;
                while (off < want.size() && want[off].first < kcol) ++off;
                if (off == want.size()) off = 0;
                std::rotate(want.begin(), want.begin() + off, want.end());
            }
            bool ok = un.count == (int32_t)want.size();
            for (size_t c = 0; ok && c < want.size(); ++c, ++e) {
                const auto& wt = want[c];
                ok = (s.bw[e] >> 32) == un.n0 && (s.bw[e] & 0xffffffffLL) == (int64_t)wt.first * a.C &&
                     s.apw[e] == ((uint64_t)wt.second.first | (uint64_t)wt.second.second << 32);
            }
            if (!ok) e = wg.w_begin + wg.n;  // keep the stream-length check meaningful after a mismatch
            expect(ok, name + ": pair entries (union, each row in CSR order, words)");
        }
        expect(e == wg.w_begin + wg.n, name + ": stream length");
        const SpmmStreamHead& h = s.heads[g];
        expect(std::memcmp(&h.wg, &wg, sizeof wg) == 0, name + ": head record");
        for (int j = 0; j < kHeadWords; ++j)
            expect(h.bw[j] == s.bw[wg.w_begin + j] && h.apw[j] == s.apw[wg.w_begin + j], name + ": head words");
        w += wg.n;
        u += wg.n_units;
    }
    expect(std::all_of(seen.begin(), seen.end(), [](int v) { return v == 1; }), name + ": every stripe's tile once");
    expect((int64_t)s.bw.size() == w + kStreamPad && (int64_t)s.apw.size() == w + kStreamPad, name + ": padding");
    int64_t shared = 0, max_union = -1;
    std::vector<std::pair<int32_t, int32_t>> pl;
    expect(spmm_stripe_pairs(&d, kPairMaxRows, pl, &shared, &max_union), name + ": pairs");
    int64_t singles = 0, largest = 0;
    for (const auto& pr : pl) {
        singles += pr.second < 0;
        std::vector<int32_t> cols(a.indices.begin() + a.indptr[pr.first], a.indices.begin() + a.indptr[pr.first + 1]);
        if (pr.second >= 0)
            cols.insert(cols.end(), a.indices.begin() + a.indptr[pr.second], a.indices.begin() + a.indptr[pr.second + 1]);
        std::sort(cols.begin(), cols.end());
        largest = std::max<int64_t>(largest, std::unique(cols.begin(), cols.end()) - cols.begin());
    }
    expect(max_union == largest, name + ": largest union of block columns");
    expect(singles == nsr % 2 && (int64_t)pl.size() == (nsr + 1) / 2, name + ": pairs cover the rows");
    expect(w == (a.indptr[nsr] - shared) * n_tiles, name + ": entries = blocks - shared columns, per tile");
    std::printf("%-34s pairs %5zu shared %6lld entries %8lld grid %zu\n", name.c_str(), pl.size(), (long long)shared,
                (long long)w, s.wgs.size());
}

int main() {
    const int cus = 256;
    check_pairing();
    check_spmm(uniform(4096, 4096, 32, 32, 4096, 1), 512, cus, "spmm 4096^2 25% N=512");
    check_spmm(uniform(4096, 4096, 32, 32, 819, 2), 512, cus, "spmm 4096^2 5% N=512");
    check_spmm(uniform(4096, 4096, 32, 32, 164, 3), 512, cus, "spmm 4096^2 1% N=512");
    check_spmm(uniform(4096, 4096, 32, 32, 4096, 4), 160, cus, "spmm partial tile N=160");
    check_spmm(skewed(16384, 16384, 32, 32, 5243, 5), 1024, cus, "spmm skewed, duplicates");
    check_spmm(uniform(8192, 8192, 256, 256, 256, 6), 8192, cus, "spmm 256x256 blocks (row groups)");
    check_spmm(uniform(2048, 1024, 64, 128, 60, 7), 256, cus, "spmm 64x128 blocks");
    for (const char* lim : {"1", "3", "6"}) {
        setenv("BSP_SPMM_SPLIT", lim, 1);
        check_spmm(uniform(2048, 2048, 256, 256, 40, 8), 512, cus, std::string("spmm 256x256 split ") + lim);
        check_spmm(uniform(2048, 1024, 64, 128, 60, 7), 256, cus, std::string("spmm 64x128 split ") + lim);
        unsetenv("BSP_SPMM_SPLIT");
    }
    check_spmm(skewed(1024, 2048, 128, 64, 40, 8), 96, cus, "spmm 128x64 blocks, skewed");
    check_spmm(uniform(1024, 1024, 32, 32, 0, 9), 256, cus, "spmm empty");
    check_spmm(banded(8192, 32, 8, 655, 19), 128, cus, "spmm banded 8192^2 (row bands)");
    check_spmm_stream(uniform(4096, 4096, 32, 32, 4096, 1), 512, cus, 128, 2, "stream 4096^2 25% tile 128");
    check_spmm_stream(uniform(4096, 4096, 32, 32, 4096, 1), 512, cus, 256, 1, "stream 4096^2 25% tile 256");
    check_spmm_stream(uniform(4096, 4096, 32, 32, 164, 3), 512, cus, 128, 2, "stream 4096^2 1%");
    check_spmm_stream(skewed(16384, 16384, 32, 32, 5243, 5), 1024, cus, 128, 2, "stream skewed, duplicates");
    check_spmm_stream(uniform(2048, 1024, 64, 128, 60, 7), 256, cus, 256, 1, "stream 64x128 blocks");
    check_spmm_stream(uniform(4096, 4096, 32, 64, 1500, 11), 512, cus, 128, 2, "stream 32x64 blocks, 2 col groups");
    check_spmm_stream(uniform(4096, 4096, 32, 128, 700, 12), 512, cus, 128, 2, "stream 32x128 blocks, 2 col groups");
    check_spmm_stream(skewed(4096, 4096, 32, 32, 3000, 13), 512, cus, 128, 2, "stream unsorted+dups, 2 col groups");
    check_spmm_stream(uniform(1024, 1024, 32, 32, 0, 9), 256, cus, 128, 1, "stream empty");
    check_spmm_stream(uniform(1024, 1024, 32, 32, 30, 9), 128, 8, 128, 2, "stream 8 CUs");
    check_spmm_stream(uniform(4096, 4096, 32, 32, 4096, 1), 512, cus, 128, 1, "stream 25% two pipelines", 2);
    check_spmm_stream(skewed(16384, 16384, 32, 32, 5243, 5), 1024, cus, 128, 1, "stream skewed two pipelines", 2);
    check_spmm_stream(uniform(4096, 4096, 32, 32, 164, 3), 512, cus, 128, 1, "stream 1% two pipelines", 2);
    check_spmm_stream(uniform(1024, 1024, 32, 32, 0, 9), 256, cus, 128, 1, "stream empty two pipelines", 2);
    check_spmm_stream(uniform(1024, 1024, 32, 32, 30, 9), 128, 8, 128, 1, "stream 8 CUs two pipelines", 2);
    check_spmm_stream_pairs(uniform(4096, 4096, 32, 32, 4096, 1), 512, cus, "pairs 4096^2 25%");
    check_spmm_stream_pairs(uniform(4096, 4096, 32, 32, 8192, 2), 512, cus, "pairs 4096^2 50%");
    check_spmm_stream_pairs(uniform(4064, 4096, 32, 32, 2000, 4), 256, cus, "pairs odd stripe count");
    check_spmm_stream_pairs(uniform(4096, 4096, 32, 32, 164, 3), 512, cus, "pairs 1%, empty stripes");
    check_spmm_stream_pairs(uniform(1024, 1024, 32, 32, 0, 9), 256, cus, "pairs empty");
    check_spmm_stream_pairs(uniform(32768, 4096, 32, 32, 2000, 6), 1024, cus, "pairs many units per workgroup");
    check_spmm_stream_pairs(uniform(1024, 1024, 32, 32, 30, 9), 128, 8, "pairs 8 CUs");
    check_sddmm(uniform(4096, 4096, 32, 32, 1638, 10), 256, cus, "sddmm 4096^2 10% K=256");
    check_sddmm(skewed(2048, 2048, 64, 32, 300, 11), 128, cus, "sddmm 64x32 blocks, skewed");
    check_sddmm(uniform(1024, 1024, 128, 128, 20, 12), 64, cus, "sddmm 128x128 blocks");
    check_sddmm(banded(8192, 32, 8, 655, 20), 128, cus, "sddmm banded 8192^2 (column bands)");
    check_spgemm(uniform(2048, 2048, 32, 32, 300, 13), uniform(2048, 2048, 32, 32, 300, 14), cus,
                 "spgemm 2048^2 7% x 7%");
    check_spgemm(skewed(1024, 512, 64, 32, 80, 15), uniform(512, 768, 32, 96, 30, 16), cus,
                 "spgemm 64x32 x 32x96, duplicates");
    check_spgemm(uniform(512, 512, 128, 128, 6, 17), uniform(512, 256, 128, 64, 5, 18), cus,
                 "spgemm 128x128 x 128x64");
    std::printf("%s (%d failed checks)\n", g_fail ? "FAIL" : "PASS", g_fail);
    return g_fail ? 1 : 0;
}
