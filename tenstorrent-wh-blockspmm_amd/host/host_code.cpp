// Operator entry points over the C ABI (include/bsparse.h).
#include "host_code.hpp"

#include <stdexcept>

#include "bsparse.h"

namespace bsp_host {

namespace {

void check(int status) {
    if (status != BSP_OK)
        throw std::runtime_error(std::string("bsparse: ") + bsp_status_string(status) + ": " + bsp_last_error());
}

template <typename T>
bsp_bsr_desc desc_of(const bsr_matrix<T>& m) {
    bsp_bsr_desc d{};
    d.H = (int64_t)m.H;
    d.W = (int64_t)m.W;
    d.R = (int64_t)m.R;
    d.C = (int64_t)m.C;
    d.nblocks = (int64_t)m.nblocks;
    d.indptr = m.indptr.data();
    d.indices = m.indices.data();
    return d;
}

void check_dims(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(std::string("bsparse: argument mismatch: ") + what);
}

}  // namespace

Device* CreateDevice(int device_id) { return new Device{device_id}; }

bool CloseDevice(Device* device) {
    delete device;
    return true;
}

namespace bsr_host_code {

void bsr_spmm_mi355x(bsr_matrix<bfloat16>& a, dense_matrix<bfloat16>& b, dense_matrix<bfloat16>& output,
                     bool bcast_batch, uint32_t nnz_blocks, uint32_t M, uint32_t N, uint32_t K, uint32_t R,
                     uint32_t C, uint32_t B, Device* device) {
    check_dims(!bcast_batch && B == 1, "bcast_batch must be false and B == 1");
    check_dims(nnz_blocks == a.nblocks && M == a.H && K == a.W && R == a.R && C == a.C, "A's shape");
    check_dims(b.H == K && b.W == N, "B must be K x N");
    check_dims(output.H == M && output.W == N, "output must be M x N");
    check_dims(a.data.size() == a.nblocks * a.R * a.C, "A values");
    const bsp_bsr_desc d = desc_of(a);
    check(bsp_host_spmm(&d, reinterpret_cast<const uint16_t*>(a.data.data()),
                        reinterpret_cast<const uint16_t*>(b.data.data()), N, output.data.data(), BSP_DTYPE_BF16,
                        device ? device->ordinal : 0));
}

void bsr_spmm_mi355x_f32(bsr_matrix<bfloat16>& a, dense_matrix<bfloat16>& b, dense_matrix<float>& output,
                         uint32_t M, uint32_t N, uint32_t K, uint32_t R, uint32_t C, Device* device) {
    check_dims(M == a.H && K == a.W && R == a.R && C == a.C, "A's shape");
    check_dims(b.H == K && b.W == N && output.H == M && output.W == N, "B / output shape");
    check_dims(a.data.size() == a.nblocks * a.R * a.C, "A values");
    const bsp_bsr_desc d = desc_of(a);
    check(bsp_host_spmm(&d, reinterpret_cast<const uint16_t*>(a.data.data()),
                        reinterpret_cast<const uint16_t*>(b.data.data()), N, output.data.data(), BSP_DTYPE_F32,
                        device ? device->ordinal : 0));
}

}  // namespace bsr_host_code

namespace bsr_sddmm_host_code {

template <typename TO>
static void run_sddmm(bsr_matrix<bfloat16>& mask, dense_matrix<bfloat16>& c, dense_matrix<bfloat16>& d,
                      bsr_matrix<TO>& output, int dtype, Device* device) {
    check_dims(c.H == mask.H && d.W == mask.W && c.W == d.H, "C must be M x K and D K x N");
    check_dims(mask.data.size() == mask.nblocks * mask.R * mask.C, "mask values");
    std::vector<TO> vals(mask.nblocks * mask.R * mask.C);
    const bsp_bsr_desc desc = desc_of(mask);
    check(bsp_host_sddmm(&desc, reinterpret_cast<const uint16_t*>(mask.data.data()),
                         reinterpret_cast<const uint16_t*>(c.data.data()),
                         reinterpret_cast<const uint16_t*>(d.data.data()), (int64_t)c.W, vals.data(), dtype,
                         device ? device->ordinal : 0));
    output = bsr_matrix<TO>(std::move(vals), mask.indptr, mask.indices, mask.H, mask.W, mask.R, mask.C,
                            mask.nblocks);
}

void bsr_sddmm_mi355x(bsr_matrix<bfloat16>& sampling_mask, dense_matrix<bfloat16>& c,
                      dense_matrix<bfloat16>& d, bsr_matrix<bfloat16>& output, uint32_t M, uint32_t N,
                      uint32_t K, uint32_t R, uint32_t C_block, uint32_t B, Device* device) {
    check_dims(B == 1, "B must be 1");
    check_dims(M == sampling_mask.H && N == sampling_mask.W && R == sampling_mask.R &&
                   C_block == sampling_mask.C && K == c.W,
               "shape arguments");
    run_sddmm(sampling_mask, c, d, output, BSP_DTYPE_BF16, device);
}

void bsr_sddmm_mi355x_f32(bsr_matrix<bfloat16>& sampling_mask, dense_matrix<bfloat16>& c,
                          dense_matrix<bfloat16>& d, bsr_matrix<float>& output, Device* device) {
    run_sddmm(sampling_mask, c, d, output, BSP_DTYPE_F32, device);
}

}  // namespace bsr_sddmm_host_code

namespace bsr_spgemm_host_code {

template <typename TO>
static bsr_matrix<TO> run_spgemm(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b, int dtype,
                                 Device* device) {
    check_dims(a.W == b.H && a.C == b.R, "A's columns and block width must match B's rows and block height");
    check_dims(a.data.size() == a.nblocks * a.R * a.C && b.data.size() == b.nblocks * b.R * b.C,
               "A and B values");
    const bsp_bsr_desc da = desc_of(a), db = desc_of(b);
    int64_t nb = 0;
    check(bsp_spgemm_symbolic(&da, &db, &nb, nullptr, nullptr));
    std::vector<int> indptr(a.H / a.R + 1), indices(nb);
    std::vector<TO> vals((size_t)nb * a.R * b.C);
    check(bsp_host_spgemm(&da, reinterpret_cast<const uint16_t*>(a.data.data()), &db,
                          reinterpret_cast<const uint16_t*>(b.data.data()), indptr.data(), indices.data(),
                          vals.data(), dtype, device ? device->ordinal : 0));
    return bsr_matrix<TO>(std::move(vals), std::move(indptr), std::move(indices), a.H, b.W, a.R, b.C, (size_t)nb);
}

bsr_matrix<bfloat16> bsr_spgemm_mi355x(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b,
                                       Device* device) {
    return run_spgemm<bfloat16>(a, b, BSP_DTYPE_BF16, device);
}

bsr_matrix<float> bsr_spgemm_mi355x_f32(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b,
                                        Device* device) {
    return run_spgemm<float>(a, b, BSP_DTYPE_F32, device);
}

}  // namespace bsr_spgemm_host_code

}  // namespace bsp_host
