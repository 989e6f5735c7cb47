// Operator entry points with the reference's function-pointer shapes.
//
// SpMM:  HostCodeFunctionPtr, block_spmm/inc/host_code.hpp:165-177
//        (a, b, output, bcast_batch, nnz_blocks, M, N, K, R, C, B, device)
// SDDMM: SDDMMHostCodeFunctionPtr, block_sddmm/inc/host_code.hpp:104-115
//        (sampling_mask, c, d, output, M, N, K, R, C_block, B, device)
// SpGEMM: bsr_matrix<T>::spgemm(const bsr_matrix<T>& B),
//        sparse_common/bsr_matrix.hpp:741-810 (a CPU routine in the reference;
//        here the products run on the device)
// The reference passes an IDevice* from tt-metal's CreateDevice; here Device
// names a HIP device ordinal.  Buffers are the reference's untilized host
// layout (the reference tilizes at its call sites, test_block_spmm.cpp:77-78;
// that step is dropped).  Every call is blocking, like the reference's
// Finish(cq).  Errors throw std::runtime_error with the library's message (the
// reference aborts through TT_THROW / TT_ASSERT).
#pragma once

#include <cstdint>
#include <string>
#include <utility>

#include "bsr_matrix.hpp"

namespace bsp_host {

struct Device {
    int ordinal = 0;
};

Device* CreateDevice(int device_id);
bool CloseDevice(Device* device);

namespace bsr_host_code {

// C = A * B with bf16 output (the reference's dense_matrix<bfloat16> output).
// `output` must be M x N; every element is written.  bcast_batch and B are
// accepted for signature compatibility and must be false / 1.
void bsr_spmm_mi355x(bsr_matrix<bfloat16>& a, dense_matrix<bfloat16>& b, dense_matrix<bfloat16>& output,
                     bool bcast_batch, uint32_t nnz_blocks, uint32_t M, uint32_t N, uint32_t K, uint32_t R,
                     uint32_t C, uint32_t B, Device* device);

// Same product with fp32 output (the golden's own precision).
void bsr_spmm_mi355x_f32(bsr_matrix<bfloat16>& a, dense_matrix<bfloat16>& b, dense_matrix<float>& output,
                         uint32_t M, uint32_t N, uint32_t K, uint32_t R, uint32_t C, Device* device);

using HostCodeFunctionPtr = void (*)(bsr_matrix<bfloat16>& a, dense_matrix<bfloat16>& b,
                                     dense_matrix<bfloat16>& output, bool bcast_batch, uint32_t nnz_blocks,
                                     uint32_t M, uint32_t N, uint32_t K, uint32_t R, uint32_t C, uint32_t B,
                                     Device* device);

static std::pair<HostCodeFunctionPtr, std::string> HostCodeRegistry[] = {
    {bsr_spmm_mi355x, "bsr_spmm_mi355x"},
};

}  // namespace bsr_host_code

namespace bsr_sddmm_host_code {

// output = sampling_mask (.) (c * d); output gets the mask's structure and bf16
// values (assigned inside, as bsr_sddmm_multicore_naive.cpp:342-346 does).
void bsr_sddmm_mi355x(bsr_matrix<bfloat16>& sampling_mask, dense_matrix<bfloat16>& c,
                      dense_matrix<bfloat16>& d, bsr_matrix<bfloat16>& output, uint32_t M, uint32_t N,
                      uint32_t K, uint32_t R, uint32_t C_block, uint32_t B, Device* device);

// Same with fp32 output values.
void bsr_sddmm_mi355x_f32(bsr_matrix<bfloat16>& sampling_mask, dense_matrix<bfloat16>& c,
                          dense_matrix<bfloat16>& d, bsr_matrix<float>& output, Device* device);

using SDDMMHostCodeFunctionPtr = void (*)(bsr_matrix<bfloat16>& sampling_mask, dense_matrix<bfloat16>& c,
                                          dense_matrix<bfloat16>& d, bsr_matrix<bfloat16>& output, uint32_t M,
                                          uint32_t N, uint32_t K, uint32_t R, uint32_t C_block, uint32_t B,
                                          Device* device);

static std::pair<SDDMMHostCodeFunctionPtr, std::string> HostCodeRegistry[] = {
    {bsr_sddmm_mi355x, "bsr_sddmm_mi355x"},
};

}  // namespace bsr_sddmm_host_code

namespace bsr_spgemm_host_code {

// a * b as a new BSR matrix (H x b.W in R x b.C blocks) with bf16 values, the
// reference's spgemm result type; requires a.W == b.H and a.C == b.R.
bsr_matrix<bfloat16> bsr_spgemm_mi355x(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b,
                                       Device* device);

// Same with fp32 values (the golden's accumulator precision).
bsr_matrix<float> bsr_spgemm_mi355x_f32(const bsr_matrix<bfloat16>& a, const bsr_matrix<bfloat16>& b,
                                        Device* device);

}  // namespace bsr_spgemm_host_code

}  // namespace bsp_host
