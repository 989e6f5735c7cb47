// SDDMM test driver in the shape of the reference's test_sddmm
// (block_sddmm/src/test_sddmm.cpp): the registry of block_sddmm/inc/
// test_suite.hpp:176-198 run through an operator entry point of the
// SDDMMHostCodeFunctionPtr shape.
//
//   test_sddmm <case|-1 for all> <host_code|-1 for CPU-only>
//
// CPU-only mode (host_code = -1, test_sddmm.cpp:159-194 of the reference)
// checks structure without a device: the mask validates and the SDDMM
// schedule lists every output sub-block exactly once.  Device mode requires
// the output structure to equal the mask's bit for bit
// (indptr/indices/nblocks/H/W/R/C), PCC > 0.99 as the reference
// (test_sddmm.cpp:256), and every value within 1e-2*sqrt(K/32)*max(1,|g|) of
// the fp32 golden (the oracle, oracle/bsp_oracle.c).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "bsparse.h"
#include "host_code.hpp"

extern "C" {
int orc_sddmm(const int32_t*, const int32_t*, const uint16_t*, int64_t, int64_t, int64_t, const uint16_t*,
              int64_t, const uint16_t*, int64_t, int, float*, int, int);
float orc_pcc(const float*, const float*, int64_t);
}

using namespace bsp_host;
using Case = std::tuple<bsr_matrix<bfloat16>, dense_matrix<bfloat16>, dense_matrix<bfloat16>, std::string>;

namespace {

std::string sfx(size_t R, size_t C) { return "_R" + std::to_string(R) + "C" + std::to_string(C); }

Case mk(size_t H, size_t W, size_t R, size_t C, size_t nb, int fill, content_type mc, size_t K,
        const std::string& name) {
    bsr_matrix<float> mask(H, W, R, C, nb, fill, mc);
    dense_matrix<float> c(H, K, ARANGE);
    dense_matrix<float> d(K, W, UNIFORM);
    return {mask.bfloat16_cast(), c.bfloat16_cast(), d.bfloat16_cast(), name};
}

std::vector<std::function<Case()>> registry() {
    std::vector<std::function<Case()>> r;
    auto add_block = [&](size_t R, size_t C) {
        r.push_back([=] { return mk(R, C, R, C, 1, BSP_FILL_ROW, UNIFORM, 2 * C, "single_block" + sfx(R, C)); });
        r.push_back([=] { return mk(4 * R, 4 * C, R, C, 4, BSP_FILL_DIAG, UNIFORM, 2 * C, "diagonal_mask" + sfx(R, C)); });
        r.push_back([=] { return mk(2 * R, 2 * C, R, C, 4, BSP_FILL_ROW, UNIFORM, C, "full_mask" + sfx(R, C)); });
        r.push_back([=] { return mk(4 * R, 4 * C, R, C, 4, BSP_FILL_DIAG, ID, 2 * C, "identity_mask" + sfx(R, C)); });
        r.push_back([=] { return mk(8 * R, 4 * C, R, C, 8, BSP_FILL_ROW, UNIFORM, 2 * C, "nonsquare" + sfx(R, C)); });
    };
    add_block(32, 32);
    r.push_back([] {
        bsr_matrix<float> mask(256, 256, 32, 32, 16, UNIFORM, 11);
        dense_matrix<float> c(256, 128, ARANGE), d(128, 256, UNIFORM);
        return Case{mask.bfloat16_cast(), c.bfloat16_cast(), d.bfloat16_cast(), "random_sparse_mask_R32C32"};
    });
    r.push_back([] {
        bsr_matrix<float> mask(512, 512, 32, 32, 26, UNIFORM, 12);
        dense_matrix<float> c(512, 256, ARANGE), d(256, 512, UNIFORM);
        return Case{mask.bfloat16_cast(), c.bfloat16_cast(), d.bfloat16_cast(), "large_random_R32C32"};
    });
    add_block(64, 64);
    r.push_back([] { return mk(256, 256, 128, 128, 4, BSP_FILL_ROW, UNIFORM, 128, "full_mask_R128C128"); });
    r.push_back([] { return mk(512, 512, 256, 256, 4, BSP_FILL_ROW, UNIFORM, 256, "full_mask_R256C256"); });
    r.push_back([] {
        return mk(1024, 1024, 256, 256, 4, BSP_FILL_DIAG, UNIFORM, 256, "diagonal_mask_shortk_R256C256");
    });
    r.push_back([] { return mk(2048, 1024, 256, 256, 8, BSP_FILL_ROW, UNIFORM, 256, "nonsquare_shortk_R256C256"); });
    // Random values (RAND mask, RAND C and D) on a larger random mask.
    r.push_back([] {
        bsr_matrix<float> mask(2048, 2048, 32, 32, 400, RAND, 13);
        dense_matrix<float> c(2048, 192, RAND), d(192, 2048, RAND);
        return Case{mask.bfloat16_cast(), c.bfloat16_cast(), d.bfloat16_cast(), "random_values_R32C32"};
    });
    return r;
}

bool cpu_structure_check(const Case& cs) {
    const auto& mask = std::get<0>(cs);
    const auto& c = std::get<1>(cs);
    bsp_bsr_desc d{(int64_t)mask.H, (int64_t)mask.W, (int64_t)mask.R, (int64_t)mask.C, (int64_t)mask.nblocks,
                   mask.indptr.data(), mask.indices.data()};
    if (bsp_validate_bsr(&d) != BSP_OK) return false;
    bsp_plan_info info{};
    if (bsp_sddmm_schedule(&d, (int64_t)c.W, 256, &info, nullptr, nullptr, nullptr, nullptr) != BSP_OK) return false;
    std::vector<int32_t> items(6 * (size_t)std::max(info.n_items, 1)), rows(std::max(info.n_entries, 1)),
        wg(std::max(info.grid, 1));
    std::vector<int64_t> offs(std::max(info.n_entries, 1));
    if (bsp_sddmm_schedule(&d, (int64_t)c.W, 256, &info, items.data(), rows.data(), offs.data(), wg.data()) != BSP_OK)
        return false;
    std::set<int64_t> seen(offs.begin(), offs.begin() + info.n_entries);
    const size_t subs = mask.nblocks * (mask.R / 32) * (mask.C / 32);
    return seen.size() == subs && (size_t)info.n_entries == subs;
}

int run_device(bsr_sddmm_host_code::SDDMMHostCodeFunctionPtr fn, Case& cs, float* pcc_out, double* worst_out) {
    auto& [mask, c, d, name] = cs;
    bsr_matrix<bfloat16> out;
    Device* dev = CreateDevice(0);
    fn(mask, c, d, out, mask.H, mask.W, c.W, mask.R, mask.C, 1, dev);
    CloseDevice(dev);
    if (out.H != mask.H || out.W != mask.W || out.R != mask.R || out.C != mask.C || out.nblocks != mask.nblocks ||
        out.indptr != mask.indptr || out.indices != mask.indices || out.data.size() != mask.nblocks * mask.R * mask.C) {
        std::printf("  structure mismatch\n");
        return 1;
    }
    std::vector<float> g(std::max<size_t>(1, out.data.size()));
    orc_sddmm(mask.indptr.data(), mask.indices.data(), reinterpret_cast<const uint16_t*>(mask.data.data()),
              mask.H / mask.R, mask.R, mask.C, reinterpret_cast<const uint16_t*>(c.data.data()), c.W,
              reinterpret_cast<const uint16_t*>(d.data.data()), d.W, 0, g.data(), 0, 0);
    std::vector<float> gb(out.data.size()), ob(out.data.size());
    double worst = 0.0;
    bool finite = true;
    const double ke = std::max<double>(32.0, (double)c.W);
    for (size_t i = 0; i < out.data.size(); ++i) {
        gb[i] = bfloat16(g[i]).to_float();
        ob[i] = out.data[i].to_float();
        if (!std::isfinite(ob[i])) finite = false;
        const double bound = 1e-2 * std::sqrt(ke / 32.0) * std::max(1.0, (double)std::fabs(g[i]));
        worst = std::max(worst, std::fabs((double)ob[i] - g[i]) / bound);
    }
    // The reference compares dense expansions (test_sddmm.cpp:250-256); with the
    // structure already equal, comparing block values is the same set of numbers
    // plus zeros.
    const float pcc = orc_pcc(gb.data(), ob.data(), (int64_t)gb.size());
    *pcc_out = pcc;
    *worst_out = worst;
    const bool degenerate = !std::isfinite(pcc);
    return (finite && worst <= 1.0 && (degenerate || pcc > 0.99f)) ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
    auto reg = registry();
    const int which = argc > 1 ? std::atoi(argv[1]) : -1;
    const int hc = argc > 2 ? std::atoi(argv[2]) : 0;
    auto& host_reg = bsr_sddmm_host_code::HostCodeRegistry;
    if (hc >= (int)(sizeof(host_reg) / sizeof(host_reg[0]))) {
        std::fprintf(stderr, "host code index out of range\n");
        return 2;
    }
    int passed = 0, failed = 0;
    for (size_t i = 0; i < reg.size(); ++i) {
        if (which >= 0 && (size_t)which != i) continue;
        seed_content(0x5EED1000ull + i);
        Case cs = reg[i]();
        const std::string& name = std::get<3>(cs);
        int rc;
        if (hc < 0) {
            rc = cpu_structure_check(cs) ? 0 : 1;
            std::printf("%-40s %s (%zu blocks)\n", name.c_str(), rc ? "FAIL" : "PASS", std::get<0>(cs).nblocks);
        } else {
            float pcc = 0;
            double worst = 0;
            rc = run_device(host_reg[hc].first, cs, &pcc, &worst);
            std::printf("%-40s %s (PCC=%.6f, max|err|/bound=%.4f, %zu blocks)\n", name.c_str(), rc ? "FAIL" : "PASS",
                        pcc, worst, std::get<0>(cs).nblocks);
        }
        std::fflush(stdout);
        (rc ? failed : passed)++;
    }
    std::printf("Host code: %s\nPassed: %d / %d\n", hc < 0 ? "CPU-only" : host_reg[hc].second.c_str(), passed,
                passed + failed);
    if (failed) std::printf("Failed: %d\n", failed);
    return passed + failed == 0 ? 2 : (failed ? 1 : 0);
}
