"""Block-sparse attention pair on the GPU: S = mask (.) (Q K^T) by SDDMM with
K read as Y^T (BSP_COL_MAJOR), S cast to bf16, then O = S V by SpMM on the
same BSR structure; seq 8192, head dim 128, mask = 8 causal block diagonals
+ 1% global blocks.  Checked stage by stage against the oracle chain, then
the fused operator (bsp_attention, S kept on the compute unit) against the
same chain at every supported head dimension."""
import numpy as np
import pytest

from helpers import (W, assert_parity, bsr_of, capi, golden_attention, golden_sddmm, golden_spmm,
                     run_attention, run_sddmm, run_spmm, spmm_k_eff, with_values)

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


# ---- fused pair (bsp_attention): S stays on the compute unit ----------------

def test_fused_attention_full_size():
    w = W.workload_attention()
    mask, q, k, v = w["mask"], w["q"], w["k"], w["v"]
    gold, s_arr = golden_attention(mask, q, k, v)
    got = run_attention(mask, q, k, v, "f32")
    assert_parity(got, gold, spmm_k_eff(s_arr), "fused O = bf16(mask (.) QK^T) V")
    # The S quadrants meet in LDS behind the ring's barriers: the same bits on
    # every run.
    for _ in range(3):
        np.testing.assert_array_equal(run_attention(mask, q, k, v, "f32"), got)
    # Against the unfused GPU pipeline: the same S up to the bf16 rounding of
    # its fp32 sums, O up to fp32 summation order.
    s_vals = run_sddmm(mask, q, k, "bf16", y_layout=capi.COL_MAJOR)
    a = W.BsrArrays(mask.H, mask.W, 32, 32, mask.indptr, mask.indices, W.bf16_from_f32(s_vals))
    assert_parity(got, run_spmm(a, v, "f32"), spmm_k_eff(a), "fused vs SDDMM->SpMM")


@pytest.mark.parametrize("out", ["f32", "bf16"])
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("blk", [32, 64])
def test_fused_attention_shapes(d, out, blk):
    rng = np.random.default_rng(40 + d + blk)
    seq = 2048
    mask = with_values(W.random_positions(seq, seq, blk, blk, (seq // blk) ** 2 // 8, rng), "RAND", seed=d)
    std = np.float32(d ** -0.5)
    q, k, v = (W.bf16_from_f32(rng.standard_normal((seq, d), dtype=np.float32) * std) for _ in range(3))
    gold, s_arr = golden_attention(mask, q, k, v)
    assert_parity(run_attention(mask, q, k, v, out), gold, spmm_k_eff(s_arr), f"d={d} {out} R=C={blk}")


@pytest.mark.parametrize("split", [1, 3])
def test_fused_attention_split_rows(monkeypatch, split):
    monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    w = W.workload_attention(seq=2048, d=64)
    mask = with_values(w["mask"], "RAND", seed=7)
    plan = capi.AttentionPlan(bsr_of(mask), 64, "f32")
    assert plan.info()["n_split_rows"] > 0 and plan.info()["kind"] == 3
    gold, s_arr = golden_attention(mask, w["q"], w["k"], w["v"])
    got = run_attention(mask, w["q"], w["k"], w["v"], "f32", plan=plan)
    plan.close()
    assert_parity(got, gold, spmm_k_eff(s_arr), f"split={split}")


def test_fused_attention_empty_rows():
    rng = np.random.default_rng(41)
    seq, d = 1024, 128
    # Block rows 1, 4, 5 and the last are empty.
    rows = [[0], [], [0, 3, 7], [2], [], [], [1, 5], [6, 30], [], [4]] + [[i] for i in range(10, 31)] + [[]]
    indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    indices = np.array([c for r in rows for c in r], np.int32)
    mask = with_values(W.BsrArrays(seq, seq, 32, 32, indptr, indices, None), "RAND", seed=3)
    q, k, v = (W.bf16_from_f32(rng.standard_normal((seq, d), dtype=np.float32) * np.float32(0.1))
               for _ in range(3))
    gold, s_arr = golden_attention(mask, q, k, v)
    got = run_attention(mask, q, k, v, "f32")
    assert_parity(got, gold, spmm_k_eff(s_arr), "empty rows")
    for i, r in enumerate(rows):
        if not r:
            assert np.all(got[32 * i:32 * (i + 1)] == 0.0)
