"""Block-sparse attention pair on the GPU: S = mask (.) (Q K^T) by SDDMM with
K read as Y^T (BSP_COL_MAJOR), S cast to bf16, then O = S V by SpMM on the
same BSR structure; seq 8192, head dim 128, mask = 8 causal block diagonals
+ 1% global blocks.  Checked stage by stage against the oracle chain."""
import numpy as np
import pytest

from helpers import (W, assert_parity, capi, golden_sddmm, golden_spmm, run_sddmm, run_spmm,
                     spmm_k_eff)

pytestmark = pytest.mark.gpu


def test_attention_pair_full_size():
    w = W.workload_attention()
    mask, q, k, v = w["mask"], w["q"], w["k"], w["v"]
    d = w["d"]
    # Stage 1: SDDMM, bf16 output (it feeds the SpMM's bf16 A operand).
    s_vals = run_sddmm(mask, q, k, "bf16", y_layout=capi.COL_MAJOR)
    s_gold = golden_sddmm(mask, q, k, y_colmajor=True)
    assert_parity(s_vals, s_gold, d, "S = mask (.) QK^T")
    # Stage 2: SpMM on the GPU's own S (bf16), against the oracle on the same S.
    s_bf16 = W.bf16_from_f32(s_vals)
    a = W.BsrArrays(mask.H, mask.W, 32, 32, mask.indptr, mask.indices, s_bf16)
    o = run_spmm(a, v, "f32")
    assert_parity(o, golden_spmm(a, v), spmm_k_eff(a), "O = S V")
    # The structure of S is the mask's, bit for bit (values only are produced).
    assert s_vals.size == mask.nblocks * 1024
