// SpGEMM test driver: bsr_matrix<T>::spgemm (sparse_common/bsr_matrix.hpp
// :741-810) on pairs of the reference's generated patterns (FILL_* and the
// random constructor), run through the host mirror's
// bsr_spgemm_host_code::bsr_spgemm_mi355x.
//
//   test_spgemm <case|-1 for all> <0 = device | -1 = CPU-only>
//
// CPU-only mode checks the symbolic phase without a device: the structure
// bsp_spgemm_symbolic returns equals the oracle's (oracle/bsp_oracle.c
// orc_spgemm) bit for bit.  Device mode requires the same structure from the
// device result, PCC > 0.99, and every value within
// 1e-2*sqrt(K_e/32)*max(1,|g|) of the fp32 golden (K_e = block pairs of the
// output block times C), with the bf16 output compared after rounding.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <tuple>
#include <vector>

#include "bsparse.h"
#include "host_code.hpp"

extern "C" {
int orc_spgemm(const int32_t*, const int32_t*, const uint16_t*, int64_t, int64_t, int64_t, const int32_t*,
               const int32_t*, const uint16_t*, int64_t, int64_t, int32_t*, int32_t*, float*, int64_t*, int);
float orc_pcc(const float*, const float*, int64_t);
}

using namespace bsp_host;
using Case = std::tuple<bsr_matrix<bfloat16>, bsr_matrix<bfloat16>, std::string>;

namespace {

Case fill(size_t H, size_t K, size_t N, size_t R, size_t C, size_t BC, size_t na, int fa, size_t nb, int fb,
          content_type content, const std::string& name) {
    bsr_matrix<float> a(H, K, R, C, na, fa, content);
    bsr_matrix<float> b(K, N, C, BC, nb, fb, content);
    return {a.bfloat16_cast(), b.bfloat16_cast(), name};
}

Case rand_pair(size_t H, size_t K, size_t N, size_t R, size_t C, size_t BC, size_t na, size_t nb, uint64_t seed,
               const std::string& name) {
    bsr_matrix<float> a(H, K, R, C, na, RAND, seed);
    bsr_matrix<float> b(K, N, C, BC, nb, RAND, seed + 1);
    return {a.bfloat16_cast(), b.bfloat16_cast(), name};
}

std::vector<std::function<Case()>> registry() {
    std::vector<std::function<Case()>> r;
    r.push_back([] { return fill(32, 32, 32, 32, 32, 32, 1, BSP_FILL_ROW, 1, BSP_FILL_ROW, UNIFORM, "single_block"); });
    r.push_back([] { return fill(128, 128, 128, 32, 32, 32, 4, BSP_FILL_DIAG, 4, BSP_FILL_DIAG, RAND, "diag_x_diag"); });
    r.push_back([] { return fill(128, 128, 128, 32, 32, 32, 16, BSP_FILL_ROW, 4, BSP_FILL_DIAG, ID, "full_x_identity"); });
    r.push_back([] { return fill(256, 256, 256, 32, 32, 32, 36, BSP_FILL_TRIL, 36, BSP_FILL_TRIL, RAND, "tril_x_tril"); });
    r.push_back([] { return fill(256, 256, 256, 32, 32, 32, 20, BSP_FILL_MULTI_DIAG, 20, BSP_FILL_COL, RAND, "multidiag_x_col"); });
    r.push_back([] { return fill(256, 128, 256, 64, 32, 64, 8, BSP_FILL_ROW, 8, BSP_FILL_ROW, RAND, "row_x_row_R64C32BC64"); });
    r.push_back([] { return rand_pair(512, 512, 512, 32, 32, 32, 40, 40, 21, "random_R32"); });
    r.push_back([] { return rand_pair(1024, 1024, 1024, 64, 64, 64, 60, 60, 23, "random_R64"); });
    r.push_back([] { return rand_pair(1024, 512, 768, 128, 64, 96, 12, 14, 25, "random_R128C64BC96"); });
    r.push_back([] { return rand_pair(2048, 2048, 2048, 32, 32, 32, 410, 410, 27, "random_2048_10pct"); });
    return r;
}

struct Golden {
    std::vector<int32_t> indptr, indices;
    std::vector<float> vals;
};

Golden golden(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b) {
    Golden g;
    g.indptr.assign(a.H / a.R + 1, 0);
    int64_t n = 0;
    orc_spgemm(a.indptr.data(), a.indices.data(), reinterpret_cast<const uint16_t*>(a.data.data()), a.H / a.R,
               a.R, a.C, b.indptr.data(), b.indices.data(), reinterpret_cast<const uint16_t*>(b.data.data()), b.C,
               b.W / b.C, g.indptr.data(), nullptr, nullptr, &n, 0);
    g.indices.assign(std::max<int64_t>(n, 1), 0);
    g.vals.assign(std::max<int64_t>(n, 1) * a.R * b.C, 0.0f);
    orc_spgemm(a.indptr.data(), a.indices.data(), reinterpret_cast<const uint16_t*>(a.data.data()), a.H / a.R,
               a.R, a.C, b.indptr.data(), b.indices.data(), reinterpret_cast<const uint16_t*>(b.data.data()), b.C,
               b.W / b.C, g.indptr.data(), g.indices.data(), g.vals.data(), &n, 0);
    g.indices.resize(n);
    g.vals.resize((size_t)n * a.R * b.C);
    return g;
}

bool cpu_structure_check(const Case& cs) {
    const auto& [a, b, name] = cs;
    const Golden g = golden(a, b);
    bsp_bsr_desc da{(int64_t)a.H, (int64_t)a.W, (int64_t)a.R, (int64_t)a.C, (int64_t)a.nblocks, a.indptr.data(),
                    a.indices.data()};
    bsp_bsr_desc db{(int64_t)b.H, (int64_t)b.W, (int64_t)b.R, (int64_t)b.C, (int64_t)b.nblocks, b.indptr.data(),
                    b.indices.data()};
    int64_t n = 0;
    if (bsp_spgemm_symbolic(&da, &db, &n, nullptr, nullptr) != BSP_OK) return false;
    std::vector<int32_t> ip(a.H / a.R + 1), ix(std::max<int64_t>(n, 1));
    if (bsp_spgemm_symbolic(&da, &db, &n, ip.data(), ix.data()) != BSP_OK) return false;
    ix.resize(n);
    return ip == g.indptr && ix == g.indices;
}

int run_device(Case& cs, float* pcc_out, double* worst_out) {
    auto& [a, b, name] = cs;
    const Golden g = golden(a, b);
    Device* dev = CreateDevice(0);
    bsr_matrix<bfloat16> out = bsr_spgemm_host_code::bsr_spgemm_mi355x(a, b, dev);
    CloseDevice(dev);
    if (out.H != a.H || out.W != b.W || out.R != a.R || out.C != b.C || out.indptr != g.indptr ||
        out.indices != g.indices || out.data.size() != g.vals.size()) {
        std::printf("  structure mismatch\n");
        return 1;
    }
    // Pairs per output block: the reduction length of its values is pairs * C.
    std::vector<int32_t> pairs(out.nblocks, 0);
    for (size_t i = 0; i + 1 < a.indptr.size(); ++i)
        for (int ai = a.indptr[i]; ai < a.indptr[i + 1]; ++ai) {
            const int k = a.indices[ai];
            for (int bi = b.indptr[k]; bi < b.indptr[k + 1]; ++bi)
                for (int ob = out.indptr[i]; ob < out.indptr[i + 1]; ++ob)
                    if (out.indices[ob] == b.indices[bi]) ++pairs[ob];
        }
    const size_t blk = a.R * b.C;
    std::vector<float> gb(g.vals.size()), ob(g.vals.size());
    double worst = 0.0;
    bool finite = true;
    for (size_t v = 0; v < g.vals.size(); ++v) {
        gb[v] = bfloat16(g.vals[v]).to_float();
        ob[v] = out.data[v].to_float();
        if (!std::isfinite(ob[v])) finite = false;
        const double ke = std::max(32.0, (double)pairs[v / blk] * a.C);
        const double bound = 1e-2 * std::sqrt(ke / 32.0) * std::max(1.0, (double)std::fabs(g.vals[v]));
        worst = std::max(worst, std::fabs((double)ob[v] - g.vals[v]) / bound);
    }
    const float pcc = gb.empty() ? 1.0f : orc_pcc(gb.data(), ob.data(), (int64_t)gb.size());
    *pcc_out = pcc;
    *worst_out = worst;
    const bool degenerate = !std::isfinite(pcc);
    return (finite && worst <= 1.0 && (degenerate || pcc > 0.99f)) ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
    auto reg = registry();
    const int which = argc > 1 ? std::atoi(argv[1]) : -1;
    const int mode = argc > 2 ? std::atoi(argv[2]) : 0;
    int passed = 0, failed = 0;
    for (size_t i = 0; i < reg.size(); ++i) {
        if (which >= 0 && (size_t)which != i) continue;
        seed_content(0x5EED2000ull + i);
        Case cs = reg[i]();
        const std::string& name = std::get<2>(cs);
        int rc;
        if (mode < 0) {
            rc = cpu_structure_check(cs) ? 0 : 1;
            std::printf("%-28s %s (A %zu, B %zu blocks)\n", name.c_str(), rc ? "FAIL" : "PASS", std::get<0>(cs).nblocks,
                        std::get<1>(cs).nblocks);
        } else {
            float pcc = 0;
            double worst = 0;
            rc = run_device(cs, &pcc, &worst);
            std::printf("%-28s %s (PCC=%.6f, max|err|/bound=%.4f)\n", name.c_str(), rc ? "FAIL" : "PASS", pcc, worst);
        }
        std::fflush(stdout);
        (rc ? failed : passed)++;
    }
    std::printf("Mode: %s\nPassed: %d / %d\n", mode < 0 ? "CPU-only" : "bsr_spgemm_mi355x", passed, passed + failed);
    if (failed) std::printf("Failed: %d\n", failed);
    return passed + failed == 0 ? 2 : (failed ? 1 : 0);
}
