// Host-side matrix types with the reference's API surface.
//
// Mirrors sparse_common/bsr_matrix.hpp of salmanra/Tenstorrent-WH-BlockSpMM:
// dense_matrix<T> (:39-196) and bsr_matrix<T> (:202-1126) keep their public
// field names (data/H/W; indptr/indices/data/H/W/nblocks/R/C), their layouts
// (row-major dense, R x C row-major blocks in CSR order) and the constructors
// the test registries use (content types RAND/UNIFORM/ARANGE/ID, fill types
// FILL_ROW/COL/DIAG/TRIL/MULTI_DIAG/TRIU, random positions, custom arrays).
// Differences, on purpose:
//   - RAND is U[-1, 1] from a seeded generator (the reference uses unseeded
//     rand() scaled to about +-5e5 and clock-seeded positions,
//     sparse_common/bsr_matrix.hpp:23-24, :55, :646-647);
//   - FILL_COL produces a valid column pattern (the reference's loop emits
//     duplicate columns once nblocks > H/R, :291-317);
//   - the CPU golden methods (spmm_bfloat16, omp_spmm_bf16, sddmm, ...) are
//     not here: the product computes on the GPU, and the golden lives with
//     the test oracle.
#pragma once

#include <algorithm>
#include <cassert>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <numeric>
#include <random>
#include <stdexcept>
#include <utility>
#include <vector>

namespace bsp_host {

// bf16 storage type (tt-metal's bfloat16 in the reference): 16-bit pattern,
// round-to-nearest-even from float.
struct bfloat16 {
    uint16_t bits = 0;
    bfloat16() = default;
    bfloat16(float f) {  // NOLINT: implicit like the reference's type
        uint32_t u;
        std::memcpy(&u, &f, 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            bits = (uint16_t)((u >> 16) | 0x40u);
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);
            bits = (uint16_t)(u >> 16);
        }
    }
    static bfloat16 from_bits(uint16_t b) {
        bfloat16 r;
        r.bits = b;
        return r;
    }
    float to_float() const {
        uint32_t u = (uint32_t)bits << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
    bool operator==(const bfloat16& o) const { return bits == o.bits; }
};
static_assert(sizeof(bfloat16) == 2, "bfloat16 must be 2 bytes");

enum content_type { RAND, UNIFORM, ARANGE, ID };

#define BSP_FILL_ROW 1
#define BSP_FILL_COL 2
#define BSP_FILL_DIAG 3
#define BSP_FILL_TRIL 4
#define BSP_FILL_MULTI_DIAG 5
#define BSP_FILL_TRIU 6

// Seeded source of RAND content (one per process; reseed for reproducibility).
inline std::mt19937_64& content_rng() {
    static std::mt19937_64 g(0x5EED0000ull);
    return g;
}
inline void seed_content(uint64_t s) { content_rng().seed(s); }
inline float rand_unit() {  // U[-1, 1): 24 random bits
    return (float)((int64_t)(content_rng()() >> 40) - (1 << 23)) / (float)(1 << 23);
}

template <typename T>
inline T from_float(float f) {
    return T(f);
}

template <typename T>
class dense_matrix {
public:
    std::vector<T> data;
    size_t H = 0;
    size_t W = 0;

    dense_matrix() = default;
    dense_matrix(size_t rows, size_t cols) : data(rows * cols, from_float<T>(0.0f)), H(rows), W(cols) {}
    dense_matrix(size_t rows, size_t cols, T val) : data(rows * cols, val), H(rows), W(cols) {}
    dense_matrix(size_t rows, size_t cols, content_type content) : data(rows * cols), H(rows), W(cols) {
        for (size_t k = 0; k < data.size(); ++k) {
            switch (content) {
                case RAND: data[k] = from_float<T>(rand_unit()); break;
                case UNIFORM: data[k] = from_float<T>(1.0f); break;
                case ID: data[k] = from_float<T>((k / W) == (k % W) ? 1.0f : 0.0f); break;
                case ARANGE: data[k] = from_float<T>((float)k); break;
            }
        }
    }
    dense_matrix(const std::vector<T>& d, size_t rows, size_t cols) : data(d), H(rows), W(cols) {
        if (d.size() != rows * cols) throw std::invalid_argument("dense_matrix: size mismatch");
    }

    dense_matrix<bfloat16> bfloat16_cast() const {
        std::vector<bfloat16> out(data.size());
        for (size_t i = 0; i < data.size(); ++i) out[i] = bfloat16(to_f(data[i]));
        return dense_matrix<bfloat16>(out, H, W);
    }

    // all_close_bfloat16 (sparse_common/bsr_matrix.hpp:184-195): absolute tolerance.
    bool all_close_bfloat16(const dense_matrix<bfloat16>& other, float tol = 1) const {
        if (H != other.H || W != other.W) return false;
        for (size_t i = 0; i < data.size(); ++i)
            if (std::fabs(to_f(data[i]) - other.data[i].to_float()) > tol) return false;
        return true;
    }

    void pretty_print(std::ostream& os = std::cout) const {
        os << "Dense Matrix:\nSize (H x W): " << H << " x " << W << std::endl;
    }

    static float to_f(const bfloat16& v) { return v.to_float(); }
    static float to_f(float v) { return v; }
};

template <typename T>
class bsr_matrix {
public:
    std::vector<int> indptr;
    std::vector<int> indices;
    std::vector<T> data;
    size_t H = 0;
    size_t W = 0;
    size_t nblocks = 0;
    size_t R = 0;
    size_t C = 0;

    bsr_matrix() = default;

    // Custom arrays (sparse_common/bsr_matrix.hpp:593-617).
    bsr_matrix(std::vector<T> d, std::vector<int> ip, std::vector<int> ix, size_t rows, size_t cols,
               size_t block_rows, size_t block_cols, size_t num_blocks)
        : indptr(std::move(ip)), indices(std::move(ix)), data(std::move(d)), H(rows), W(cols),
          nblocks(num_blocks), R(block_rows), C(block_cols) {
        check_shape();
    }

    // Fill-type constructor (:244-408; FILL_TRIU from the SpMM-side copy).
    bsr_matrix(size_t rows, size_t cols, size_t block_rows, size_t block_cols, size_t num_blocks,
               int fill_type, content_type content = RAND)
        : H(rows), W(cols), nblocks(num_blocks), R(block_rows), C(block_cols) {
        check_shape();
        const size_t bh = H / R, bw = W / C;
        std::vector<std::pair<size_t, size_t>> pos;
        switch (fill_type) {
            case BSP_FILL_ROW:
                for (size_t f = 0; f < std::min(nblocks, bh * bw); ++f) pos.emplace_back(f / bw, f % bw);
                break;
            case BSP_FILL_COL:
                for (size_t f = 0; f < std::min(nblocks, bh * bw); ++f) pos.emplace_back(f % bh, f / bh);
                break;
            case BSP_FILL_DIAG:
                if (nblocks > std::min(bh, bw)) throw std::invalid_argument("FILL_DIAG: too many blocks");
                for (size_t i = 0; i < nblocks; ++i) pos.emplace_back(i, i);
                break;
            case BSP_FILL_TRIL:
            case BSP_FILL_TRIU:
                if (bh != bw) throw std::invalid_argument("FILL_TRIL/TRIU need a square block grid");
                for (size_t i = 0; i < bh; ++i)
                    for (size_t j = 0; j < bw; ++j)
                        if (fill_type == BSP_FILL_TRIL ? j <= i : j >= i) pos.emplace_back(i, j);
                break;
            case BSP_FILL_MULTI_DIAG:
                pos = multi_diag_positions(bh, bw, nblocks);
                break;
            default:
                throw std::invalid_argument("invalid fill type");
        }
        std::stable_sort(pos.begin(), pos.end(),
                         [](const auto& a, const auto& b) { return a.first < b.first; });
        build(pos, content);
    }

    // Uniform-random distinct positions (:619-679), seeded.
    bsr_matrix(size_t rows, size_t cols, size_t block_rows, size_t block_cols, size_t num_blocks,
               content_type content, uint64_t seed)
        : H(rows), W(cols), nblocks(num_blocks), R(block_rows), C(block_cols) {
        check_shape();
        const size_t bh = H / R, bw = W / C;
        std::vector<size_t> slots(bh * bw);
        std::iota(slots.begin(), slots.end(), 0);
        std::mt19937_64 g(seed);
        for (size_t i = 0; i < nblocks; ++i) {  // partial Fisher-Yates
            std::uniform_int_distribution<size_t> d(i, slots.size() - 1);
            std::swap(slots[i], slots[d(g)]);
        }
        std::sort(slots.begin(), slots.begin() + nblocks);
        std::vector<std::pair<size_t, size_t>> pos;
        for (size_t i = 0; i < nblocks; ++i) pos.emplace_back(slots[i] / bw, slots[i] % bw);
        build(pos, content);
    }

    // multi_diag_positions (:215-240): diagonals 0, +1, -1, +2, -2, ... then sorted.
    static std::vector<std::pair<size_t, size_t>> multi_diag_positions(size_t bh, size_t bw, size_t n) {
        std::vector<std::pair<size_t, size_t>> pos;
        for (long d = 0; pos.size() < n;) {
            if (d >= 0) {
                for (size_t i = 0; i < bh && i + (size_t)d < bw && pos.size() < n; ++i)
                    pos.emplace_back(i, i + (size_t)d);
            } else {
                const size_t ad = (size_t)(-d);
                for (size_t j = 0; j < bw && j + ad < bh && pos.size() < n; ++j) pos.emplace_back(j + ad, j);
            }
            d = d <= 0 ? -d + 1 : -d;
            if ((size_t)std::labs(d) >= std::max(bh, bw)) break;
        }
        std::sort(pos.begin(), pos.end());
        return pos;
    }

    bsr_matrix<bfloat16> bfloat16_cast() const {
        std::vector<bfloat16> out(data.size());
        for (size_t i = 0; i < data.size(); ++i) out[i] = bfloat16(dense_matrix<T>::to_f(data[i]));
        return bsr_matrix<bfloat16>(out, indptr, indices, H, W, R, C, nblocks);
    }

    // to_dense (:1056-1070): later duplicates overwrite earlier ones.
    dense_matrix<T> to_dense() const {
        dense_matrix<T> out(H, W);
        for (size_t i = 0; i + 1 < indptr.size(); ++i)
            for (int idx = indptr[i]; idx < indptr[i + 1]; ++idx) {
                const size_t j = (size_t)indices[idx];
                for (size_t r = 0; r < R; ++r)
                    for (size_t c = 0; c < C; ++c)
                        out.data[(i * R + r) * W + j * C + c] = data[(size_t)idx * R * C + r * C + c];
            }
        return out;
    }

    void pretty_print(std::ostream& os = std::cout) const {
        os << "BSR Matrix:\nSize (H x W): " << H << " x " << W << "\nBlock Size (R x C): " << R << " x "
           << C << "\nNumber of blocks: " << nblocks << std::endl;
    }

private:
    void check_shape() const {
        if (R == 0 || C == 0 || H % R || W % C || H < R || W < C || H * W < nblocks * R * C)
            throw std::invalid_argument("bsr_matrix: invalid shape");
    }

    void build(const std::vector<std::pair<size_t, size_t>>& pos, content_type content) {
        const size_t bh = H / R;
        nblocks = pos.size();
        indptr.assign(bh + 1, 0);
        indices.clear();
        data.clear();
        data.reserve(nblocks * R * C);
        for (const auto& p : pos) {
            indptr[p.first + 1]++;
            indices.push_back((int)p.second);
            for (size_t k = 0; k < R * C; ++k) {
                switch (content) {
                    case RAND: data.push_back(from_float<T>(rand_unit())); break;
                    case UNIFORM: data.push_back(from_float<T>(1.0f)); break;
                    case ID: data.push_back(from_float<T>((k / C) == (k % C) ? 1.0f : 0.0f)); break;
                    case ARANGE: data.push_back(from_float<T>((float)k)); break;
                }
            }
        }
        for (size_t i = 1; i < indptr.size(); ++i) indptr[i] += indptr[i - 1];
    }
};

}  // namespace bsp_host
