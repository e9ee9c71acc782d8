"""CPU pins of the oracle's o_proj GEMM (dispatch_gemm_cols,
kernels/gemm.mojo:198-225): integer-valued operands whose sums are exact,
the identity weight, and float64 matmul to one bf16 rounding on random
operands, with and without a tail of cols % 32."""
import numpy as np
import pytest

import oracle
from tests.helpers import bf16_to_f32, bf16_ulp


def _bf(x) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32).ravel())


def test_integer_operands_give_the_rounded_integer_matmul():
    # |x|, |w| <= 3 and cols = 256: every partial sum is an integer below
    # 2^24, so f32 accumulation is exact in any order and the output is the
    # exact integer product rounded once to bf16.  A transposed or shifted
    # operand, or a dropped chunk, changes these integers.
    rng = np.random.default_rng(1)
    seq, rows, cols = 5, 48, 256
    x = rng.integers(-3, 4, (seq, cols))
    w = rng.integers(-3, 4, (rows, cols))
    got = oracle.gemm_cols(_bf(x), _bf(w), rows=rows, cols=cols)
    want = _bf((x @ w.T).astype(np.float32)).reshape(seq, rows)
    assert np.array_equal(got, want)


def test_identity_weight_copies_the_input():
    rng = np.random.default_rng(2)
    cols = 128
    x = _bf(rng.standard_normal((3, cols)))
    w = _bf(np.eye(cols))
    got = oracle.gemm_cols(x, w, rows=cols, cols=cols)
    assert np.array_equal(got.ravel(), x)


@pytest.mark.parametrize("cols", [512, 512 + 17])
def test_random_operands_match_float64_to_one_rounding(cols):
    rng = np.random.default_rng(cols)
    seq, rows = 6, 40
    xb = _bf(rng.standard_normal((seq, cols)) * 0.5)
    wb = _bf(rng.standard_normal((rows, cols)) * 0.05)
    got = bf16_to_f32(oracle.gemm_cols(xb, wb, rows=rows, cols=cols)).astype(np.float64)
    xf = bf16_to_f32(xb).astype(np.float64).reshape(seq, cols)
    wf = bf16_to_f32(wb).astype(np.float64).reshape(rows, cols)
    exact = xf @ wf.T
    # One bf16 rounding (half a spacing) plus f32 accumulation error.
    bound = 0.5 * bf16_ulp(exact) + 1e-5 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(got - exact) <= bound)
