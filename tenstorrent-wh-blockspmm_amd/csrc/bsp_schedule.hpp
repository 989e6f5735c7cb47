// Host-side analysis of a BSR structure into the work lists the HIP kernels
// walk.  Pure C++ (no HIP), so it runs and is tested without a device.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "bsparse.h"

namespace bsp {

// Width of the sub-block every kernel works in: R x C blocks are cut into
// (R/32) x (C/32) sub-blocks of 32 x 32 (the reference's TILE_SIZE,
// sparse_common/bsr_matrix.hpp:22).
constexpr int kSub = 32;
// MI355X has 8 XCDs; workgroups are handed to XCDs round-robin by workgroup id.
constexpr int kNumXcd = 8;

// One unit of SpMM work: a contiguous range of a sub-row's entries.
struct SpmmItem {
    int32_t row;      // sub-row (32 output rows)
    int32_t e_begin;  // entries [e_begin, e_end) of the entry arrays
    int32_t e_end;
    int32_t slot;     // -1: whole row; else partial-result slot of this piece
    int32_t base;     // first slot of the row's pieces (also its counter index)
    int32_t npieces;  // pieces the row is split into (0 for a whole row)
};
static_assert(sizeof(SpmmItem) == 24, "SpmmItem layout is shared with the kernels");

// What one SpMM workgroup reads first: its item and N tile (idle slots of the
// XCD map have row == -1).
struct SpmmWg {
    int32_t row;
    int32_t e_begin;
    int32_t e_end;
    int32_t slot;
    int32_t base;
    int32_t npieces;
    int32_t tile;
    int32_t pad;
};
static_assert(sizeof(SpmmWg) == 32, "SpmmWg layout is shared with the kernels");

// One split row: its sub-row, first partial slot and number of pieces.
struct SpmmSplit {
    int32_t row;
    int32_t base;
    int32_t npieces;
    int32_t pad;
};
static_assert(sizeof(SpmmSplit) == 16, "SpmmSplit layout is shared with the kernels");

struct SpmmSchedule {
    int32_t tile_n = 0;
    int32_t n_tiles = 0;
    int32_t group = 1;        // 32-row stripes per item (rows of one block row sharing B)
    int32_t split_limit = 0;  // max entries per piece
    int32_t n_slots = 0;
    int32_t n_split_rows = 0;
    int32_t max_item_entries = 0;
    int32_t xcd_col_groups = 1;  // column groups of the XCD map
    std::vector<SpmmItem> items;
    std::vector<int32_t> ent_row;  // first row of B for the entry
    std::vector<int64_t> ent_off;  // element offset of the 32x32 A sub-block (of the item's
                                   // first stripe; stripe s of a group adds 32*s*C)
    std::vector<int32_t> wgmap;    // workgroup id -> item * n_tiles + tile, or -1
};

// Per-workgroup records in launch order (items expanded through wgmap).
std::vector<SpmmWg> spmm_wg_records(const SpmmSchedule& s);

// ---- persistent SpMM (spmm_stream_kernel) -----------------------------------
// A unit is one 32-row stripe (or, with stripe pairs, two stripes that share
// block columns) times one tile of tile_n output columns.  Each workgroup of
// the persistent grid owns a list of units and streams their entries (32x32
// sub-block products; with pairs, one B slice and the A sub-blocks of either
// or both stripes) back to back through one LDS ring, so the ring never
// drains between units and a unit's store overlaps the next unit's loads.
struct SpmmStreamWg {
    int32_t w_begin;  // first word of this workgroup's entry stream
    int32_t n;        // entries in the stream (sum of its units' counts)
    int32_t u_begin;  // first unit record
    int32_t n_units;
};
static_assert(sizeof(SpmmStreamWg) == 16, "SpmmStreamWg layout is shared with the kernels");

struct SpmmStreamUnit {
    int32_t row;    // stripe (32 output rows)
    int32_t n0;     // first output column
    int32_t count;  // entries (0: the stripe has no nonzeros; its tile is stored as zeros)
    int32_t aux;    // one stripe: 0 = store the tile; two pipelines: 1 = this part
                    // goes to the exchange buffer, 2 = add the exchange buffer,
                    // then store.  Stripe pairs: the second stripe (-1: none)
};
static_assert(sizeof(SpmmStreamUnit) == 16, "SpmmStreamUnit layout is shared with the kernels");

// Trailing words and units past the last workgroup's stream: the kernels
// prefetch a few records ahead without a bounds test.
constexpr int kStreamPad = 64;

// What a workgroup reads first, in 384 contiguous bytes of its own: its
// record, its first two unit records and the first kHeadWords words of each
// of its entry streams (copies of the arrays' records and words, which the
// arrays keep as well; apw is zero without stripe pairs).  The kernel loads
// them all at once from an address that depends only on the workgroup id, so
// the first entry's loads follow one round trip to memory instead of two
// dependent ones (record, then words).
constexpr int kHeadWords = 16;
struct SpmmStreamHead {
    SpmmStreamWg wg;
    SpmmStreamUnit u[2];
    int32_t pad[4];
    int64_t bw[kHeadWords];
    uint32_t aw[kHeadWords];
    uint64_t apw[kHeadWords];
};
static_assert(sizeof(SpmmStreamHead) == 384, "SpmmStreamHead layout is shared with the kernels");

// An absent A sub-block in a stripe pair's entry word (either half).
constexpr uint32_t kNoBlock = 0xffffffffu;
static_assert(kStreamPad >= kHeadWords && kStreamPad >= 2, "heads copy words and units from the padded arrays");

struct SpmmStream {
    int32_t tile_n = 0;
    int32_t n_tiles = 0;
    int32_t wg_per_cu = 1;
    int32_t col_groups = 1;        // column groups of the XCD map
    int32_t pairs = 0;             // 1: units are stripe pairs (apw holds the A words)
    int32_t rotated = 0;           // 1: units start at spmm_stream_rotation_column (one pipeline)
    int32_t max_wg_entries = 0;    // longest workgroup stream
    int64_t n_entries = 0;         // sum over units (entries x tiles)
    std::vector<SpmmStreamWg> wgs;        // one per workgroup; workgroup g runs on XCD g % kNumXcd
    std::vector<SpmmStreamHead> heads;    // one per record of wgs, what the kernel reads first
    std::vector<SpmmStreamUnit> units;    // + kStreamPad zero records
    std::vector<int64_t> bw;              // per stream entry: first row of B | first column << 32 (+ pad)
    std::vector<uint32_t> aw;             // per stream entry: A sub-block element offset / 32 (+ pad);
                                          // empty with stripe pairs
    std::vector<uint64_t> apw;            // stripe pairs, per stream entry: the two stripes' A offsets
                                          // / 32 (low: the unit's row, high: its aux), kNoBlock where a
                                          // stripe has no block in the entry's column (+ pad)
};

// Stripe pairs for the persistent SpMM (32x32 blocks with strictly increasing
// columns in every block row): pairs of block rows, chosen greedily by the
// number of block columns they share (most first, ties by lower indices),
// leftovers paired in index order and an odd one alone (second = -1).
// Returns false (and no pairs) if the structure does not qualify or the
// problem is larger than max_rows block rows.  shared = block columns the
// pairs share in all (the B slices the pairs save per tile); max_union = the
// largest pair's union of block columns (its entries per tile).
bool spmm_stripe_pairs(const bsp_bsr_desc* a, int64_t max_rows, std::vector<std::pair<int32_t, int32_t>>& pairs,
                       int64_t* shared, int64_t* max_union = nullptr);
// The most block rows a pairing considers (its overlap table is quadratic).
constexpr int64_t kPairMaxRows = 1024;

// Persistent schedule for 32-row stripes (any R, C multiples of 32) and
// tiles of tile_n (128 or 256) columns, N a multiple of tile_n, wg_per_cu
// workgroups per compute unit.  Units are spread over the XCDs in a 2-D split
// (column groups of tiles, row groups of stripes, as xcd_tile_map) and, inside
// an XCD, longest first onto the least-loaded workgroup.  Cost of a unit:
// entries + store_cost.
// pipes = 2: one workgroup per compute unit with two pipelines; the compute
// unit's units (longest first) are concatenated and cut in half, the unit
// that straddles the cut going to both pipelines (flag 2 on the first's part,
// flag 1 on the second's).  wgs then holds two records per workgroup.
// pairs = true (pipes 1, 32x32 blocks): units are the stripe pairs of
// spmm_stripe_pairs; a pair's entries are the union of its two stripes'
// block columns, in column order (each stripe's own entries keep their CSR
// order), and its cost is the union's size.  With one pipeline, every unit's
// entries (a stripe's in CSR order, a pair's union) are then rotated to start
// at spmm_stream_rotation_column (above).
// Rotation of a unit's entries (one pipeline; BSP_SPMM_ROTATE=0 turns it
// off): a unit of column group g starts at its first entry whose block column
// is at least spmm_stream_rotation_column(block columns of A, g, col_groups)
// and wraps around to its first entry (no rotation when there is none).  The
// column groups then sweep the block columns 1/col_groups apart, the units
// of one column group (which read the same rows of B) still together; in CSR
// order every workgroup opens on the lowest block columns at once.  Only the
// summation order of a unit changes (a stripe pair rotates at the same column
// as its two stripes, so pairs stay bit-identical to single stripes).
// (4096^2 x 512, f32 C, graph replay: 25% 13.2-13.4 -> 12.3-12.4 us, 50%
// 21.8-22.3 -> 20.8-21.6 us, 1%, 5% and the skewed workload unchanged.)
inline int64_t spmm_stream_rotation_column(int64_t block_cols, int64_t group, int64_t col_groups) {
    return col_groups > 1 ? group * block_cols / col_groups : 0;
}

int build_spmm_stream(const bsp_bsr_desc* a, int64_t N, int num_cus, int tile_n, int wg_per_cu,
                      SpmmStream& s, std::string& msg, int col_groups = 0, int pipes = 1, bool pairs = false);
// Entries packed for the kernel: first row of B | (A offset / 32) << 32.
std::vector<int64_t> spmm_packed_entries(const SpmmSchedule& s);
// The split stripes in slot order (a split group contributes each of its
// stripes: stripe s of a group piece p uses slot base + s * npieces + p).
std::vector<SpmmSplit> spmm_splits(const SpmmSchedule& s);

// ---- sweep SpMM (spmm_sweep_kernel) ------------------------------------------
// One workgroup per compute unit holds the accumulators of up to
// kSweepSlots units (32-row stripe x 128-column tile) at once -- a sweep --
// and streams the entries of all of them merged in ascending first row of B
// (block column), so that every workgroup of an XCD walks K in step with the
// others and each 32-row slice of B is read from HBM once per XCD and reused
// from the L2 by every unit that needs it, instead of being evicted between
// uses by the A and C streams that pass through the same L2.  Slots 8g .. 8g+7
// belong to wave group g (waves 4g .. 4g+3, each 32 columns of the tile).
constexpr int kSweepSlots = 16;
constexpr int kSweepTile = 128;

struct SpmmSweepWg {
    int32_t w_begin;   // first word of this workgroup's entry stream
    int32_t n;         // entries in the stream (all sweeps)
    int32_t s_begin;   // first sweep record
    int32_t n_sweeps;
};
static_assert(sizeof(SpmmSweepWg) == 16, "SpmmSweepWg layout is shared with the kernels");

// The units of one wave group in a sweep: stripe (-1: slot unused) and first
// output column of each of its eight slots.
struct SpmmSweepHalf {
    int32_t row[8];
    int32_t n0[8];
};
struct SpmmSweepRec {
    int32_t count;     // entries of the sweep (0: its units are empty stripes, stored as zeros)
    int32_t empty;     // bit j: the unit of slot j has no entries (its tile is stored as zeros)
    int32_t pad[2];
    SpmmSweepHalf half[2];
};
static_assert(sizeof(SpmmSweepRec) == 144, "SpmmSweepRec layout is shared with the kernels");

// What a workgroup reads first: its record and the first kHeadWords words
// of its streams (copies; the arrays keep them too).
struct SpmmSweepHead {
    SpmmSweepWg wg;
    int32_t pad[12];
    int64_t bw[kHeadWords];
    uint32_t aw[kHeadWords];
    uint32_t pad2[16];
};
static_assert(sizeof(SpmmSweepHead) == 320, "SpmmSweepHead layout is shared with the kernels");

// B word of a sweep entry: first row of B (bits 0-31) | first output column
// (bits 32-55) | slot (bits 56-59) | skip (bit 60) | last (bit 61: the last
// entry of its unit in stream order).  Every sweep has an even number of
// entries: an odd one is padded with a skip entry (a copy of its last entry's
// words with the skip bit and without the last bit, loaded and not
// multiplied).
constexpr int kSweepSlotShift = 56;
constexpr int64_t kSweepSkip = int64_t(1) << 60;
constexpr int64_t kSweepLast = int64_t(1) << 61;
constexpr int64_t kSweepMaxN = int64_t(1) << 24;

struct SpmmSweep {
    int32_t n_tiles = 0;
    int32_t col_groups = 1;      // column groups of the XCD map
    int32_t max_sweeps = 0;      // most sweeps of any workgroup
    int32_t max_wg_entries = 0;  // longest workgroup stream
    int32_t rotated = 0;         // 1: each XCD's sweeps start at its column group's share of K
    int64_t n_entries = 0;
    int64_t n_units = 0;
    std::vector<SpmmSweepWg> wgs;      // one per workgroup (= compute unit); workgroup g on XCD g % kNumXcd
    std::vector<SpmmSweepHead> heads;  // one per workgroup
    std::vector<SpmmSweepRec> sweeps;  // (+ kStreamPad zero records)
    std::vector<int64_t> bw;           // per entry (+ pad)
    std::vector<uint32_t> aw;          // per entry: A sub-block element offset / 32 (+ pad)
};

// Estimated HBM-side reads (bytes) of a sweep plan with col_groups column
// groups: A read once per column group, and each row group's touched 32-row
// slices of B read once per XCD.
int64_t spmm_sweep_read_estimate(const bsp_bsr_desc* a, int64_t N, int col_groups);

// Builds the sweep schedule for num_cus compute units (one workgroup each).
// col_groups = 0 picks the count (1, 2, 4, 8 dividing the tile count) of
// least estimated reads.  R and C multiples of 32, N a multiple of 128 below
// 2^24.
int build_spmm_sweep(const bsp_bsr_desc* a, int64_t N, int num_cus, SpmmSweep& s, std::string& msg,
                     int col_groups = 0);

// One unit of SDDMM work: a run of output sub-blocks that share 32 rows of X.
struct SddmmItem {
    int32_t x_row0;
    int32_t e_begin;
    int32_t e_end;
    int32_t pad;
};
static_assert(sizeof(SddmmItem) == 16, "SddmmItem layout is shared with the kernels");

struct SddmmSchedule {
    int32_t chunk = 0;  // max entries per item
    int32_t max_item_entries = 0;
    std::vector<SddmmItem> items;
    std::vector<int32_t> ent_col;  // first column of Y for the entry
    std::vector<int64_t> ent_off;  // element offset of the 32x32 output sub-block
    std::vector<int32_t> wgmap;    // workgroup id -> item, or -1
};

// Per-workgroup items in launch order; idle slots get an empty range.
std::vector<SddmmItem> sddmm_wg_records(const SddmmSchedule& s);

// One SpGEMM wave task: a 32x32 output sub-block and its run of products.
struct SpgemmTask {
    int64_t out_off;  // element offset of the sub-block in the output values
    int32_t t_begin;  // products [t_begin, t_end) of the term array
    int32_t t_end;
};
static_assert(sizeof(SpgemmTask) == 16, "SpgemmTask layout is shared with the kernels");

// One SpGEMM wave run: tasks [t0, t1) and their products [p0, p1) (the
// products of consecutive tasks are contiguous); t0 == t1 for an idle slot.
struct SpgemmRun {
    int32_t t0;
    int32_t t1;
    int32_t p0;
    int32_t p1;
};
static_assert(sizeof(SpgemmRun) == 16, "SpgemmRun layout is shared with the kernels");

// SpGEMM C = A * B with A, B and C in BSR.  The symbolic phase: C's structure
// (block (i, j) present iff some stored A(i, k) meets some stored B(k, j),
// columns ascending per row, as bsr_matrix<T>::spgemm builds it,
// sparse_common/bsr_matrix.hpp:741-810) and, per 32x32 output sub-block, its
// products in the golden's order (A's CSR order, then B's, then the inner
// 32-column steps of the shared dimension).
struct SpgemmSchedule {
    int64_t nblocks = 0;             // output blocks
    std::vector<int32_t> indptr;     // output block-row pointers (H/R + 1)
    std::vector<int32_t> indices;    // output block columns (nblocks)
    std::vector<SpgemmTask> tasks;   // one per output sub-block, in output order
    std::vector<uint64_t> terms;     // A sub-block offset / 32 | (B sub-block offset / 32) << 32
    std::vector<SpgemmRun> runs;     // grid * 4 wave slots
    int32_t max_task_terms = 0;
    int32_t pieces = 0;              // non-empty wave runs
    int32_t grid = 0;                // workgroups, a multiple of kNumXcd
    int32_t wg_per_xcd = 0;
};

// SpGEMM wave runs: contiguous task ranges of about equal cost, at most
// kSpgemmRunTasks tasks each, `rounds` runs per resident wave (compute units
// x waves that fit a compute unit's LDS at `stages` ring stages).
constexpr int kSpgemmRunTasks = 64;
constexpr int kSpgemmStageBytes = 4096;
constexpr int kLdsBytesPerCu = 160 * 1024;
inline int spgemm_waves_per_cu(int stages) { return 4 * (kLdsBytesPerCu / (4 * stages * kSpgemmStageBytes)); }

// Output structure only (no product lists).
int spgemm_symbolic(const bsp_bsr_desc* a, const bsp_bsr_desc* b, std::vector<int32_t>& indptr,
                    std::vector<int32_t>& indices, std::string& msg);
// Structure, product lists and the wave runs for `num_cus` compute units and
// a ring of `stages` stages.
int build_spgemm_schedule(const bsp_bsr_desc* a, const bsp_bsr_desc* b, int num_cus, int stages, int rounds,
                          SpgemmSchedule& s, std::string& msg);

// Structural checks of sparse_common/bsr_matrix.hpp:246-252 / :610-616 plus
// the CSR invariants the golden relies on implicitly.  On failure returns a
// bsp_status and fills `msg`.
int validate_bsr(const bsp_bsr_desc* d, std::string& msg);

// force_tile_n: a fixed workgroup width (the fused attention kernel's one
// 128-column tile) instead of the automatic choice.  group: stripes per item
// (1, or 2, 4, 8 dividing R/32, with a 128-column tile); 0 chooses.
int build_spmm_schedule(const bsp_bsr_desc* a, int64_t N, int num_cus, SpmmSchedule& out,
                        std::string& msg, int force_tile_n = 0, int group = 0);

// Row-group size for R x C blocks: the largest of 8, 4, 2 that divides R/32
// and still gives two workgroups per compute unit, else 1.
int spmm_choose_group(int64_t R, int64_t H, int64_t N, int num_cus);
int build_sddmm_schedule(const bsp_bsr_desc* mask, int64_t K, int num_cus, SddmmSchedule& out,
                         std::string& msg);

// SpMM workgroup map over the XCDs in a 2-D split: the N tiles are cut into
// `col_groups` contiguous groups and the items into kNumXcd / col_groups row
// groups balanced by cost (longest first onto the least-loaded group); XCD
// x = row_group * col_groups + col_group runs that row group's items on that
// column group's tiles, longest first.  Each XCD then reads only its column
// slice of B, which stays in its L2.  Returns item * n_tiles + tile per
// workgroup id (workgroup g runs on XCD g % kNumXcd), -1 for idle slots.
// When an XCD's list fills between one and two workgroups per compute unit,
// its second round is reversed (pair_rounds).  row_bands: the row groups are
// contiguous runs of items (rows in order) of about equal cost instead.
std::vector<int32_t> xcd_tile_map(const std::vector<int64_t>& item_cost, int n_tiles, int col_groups,
                                  int cus_per_xcd, bool row_bands = false);

// The XCD's dispatcher gives its j-th workgroup to compute unit j % C (C =
// compute units per XCD) while every workgroup is resident, so workgroups j
// and j + C share a unit.  On a longest-first list of C < len <= 2C entries,
// reversing the second round pairs the heaviest with the lightest, which
// evens out the work per compute unit (the two share its load path).
void pair_rounds(std::vector<int32_t>& bin, int cus_per_xcd);

// Spreads weighted units over the XCDs (longest first onto the least-loaded
// XCD), then lays them out so that workgroup id g runs on XCD g % kNumXcd in
// each XCD's longest-first order.  Unit u expands to `width` consecutive
// workgroups (the N tiles of one SpMM item stay on one XCD, so the A blocks
// they share are read into one L2).  Returns the workgroup map; -1 = idle.
std::vector<int32_t> xcd_lpt_map(const std::vector<int64_t>& unit_cost, int width);

}  // namespace bsp
