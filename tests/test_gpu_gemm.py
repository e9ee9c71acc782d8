"""GPU parity of the o_proj GEMM after the attention (dispatch_gemm_cols,
kernels/gemm.mojo:198-225) through the C ABI: bit-exact on integer-valued
operands (exact sums), and within one bf16 spacing of the oracle on random
operands (the MFMA and VDPBF16PS add the same exact products in different
orders), at the decode shapes (split contraction) and multi-tile batches."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import bf16_to_f32, bf16_ulp, compare_bf16

pytestmark = pytest.mark.gpu


def _bf(x) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32).ravel())


def _run(xb, wb, seq, rows, cols) -> np.ndarray:
    out = empty_dev(max(seq * rows, 1), np.uint16)
    ws = A.gemm_cols_workspace(rows, cols, seq)
    A.dispatch_gemm_cols(to_dev(xb), to_dev(wb), out, rows=rows, cols=cols, seq_len=seq,
                         workspace=ws)
    return from_dev(out, np.uint16)[:seq * rows].reshape(seq, rows)


@pytest.mark.parametrize("seq,rows,cols", [(1, 2816, 4096), (64, 2816, 4096), (20, 80, 1024),
                                           (40, 2816, 512), (5, 48, 256), (130, 320, 512),
                                           (200, 192, 4096), (3, 64, 8192), (16, 32, 384)])
def test_gemm_cols_matches_oracle(seq, rows, cols):
    announce(f"gemm_cols seq={seq} rows={rows} cols={cols}")
    rng = np.random.default_rng(seq * 7 + rows)
    xb = _bf(rng.standard_normal((seq, cols)) * 0.5)
    wb = _bf(rng.standard_normal((rows, cols)) * 0.02)
    got = _run(xb, wb, seq, rows, cols)
    want = oracle.gemm_cols(xb, wb, rows=rows, cols=cols)
    r = compare_bf16(got, want)
    assert r["n_fail"] == 0 and r["n_nan"] == 0, r
    # Tighter than the bar: one bf16 spacing, plus the f32 accumulation error
    # of either order (2^-22 of sum |x||w|), which is what remains where the
    # sum cancels to near zero and a spacing is tiny.  A dropped or repeated
    # product (|x w| ~ 1e-2) exceeds it.
    a = bf16_to_f32(got).astype(np.float64)
    b = bf16_to_f32(want).astype(np.float64)
    xf = np.abs(bf16_to_f32(xb).astype(np.float64).reshape(seq, cols))
    wf = np.abs(bf16_to_f32(wb).astype(np.float64).reshape(rows, cols))
    bound = bf16_ulp(b) * 1.0001 + 2.0 ** -22 * (xf @ wf.T)
    assert np.all(np.abs(a - b) <= bound), float(np.max(np.abs(a - b) - bound))


@pytest.mark.parametrize("seq,rows,cols", [(3, 64, 256), (64, 2816, 4096), (70, 80, 384)])
def test_gemm_cols_integer_operands_bit_exact(seq, rows, cols):
    announce(f"gemm_cols exact seq={seq} rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols)
    x = rng.integers(-3, 4, (seq, cols))
    w = rng.integers(-3, 4, (rows, cols))
    got = _run(_bf(x), _bf(w), seq, rows, cols)
    want = oracle.gemm_cols(_bf(x), _bf(w), rows=rows, cols=cols)
    assert np.array_equal(got, want)


def test_gemm_cols_rejects_unsupported_shapes():
    from inferno_amd._lib import InfernoHipError

    x = empty_dev(64 * 512, np.uint16)
    w = empty_dev(64 * 512, np.uint16)
    out = empty_dev(64 * 64, np.uint16)
    with pytest.raises(InfernoHipError):
        A.dispatch_gemm_cols(x, w, out, rows=64, cols=200, seq_len=2)   # cols % 128
    with pytest.raises(InfernoHipError):
        A.dispatch_gemm_cols(x, w, out, rows=40, cols=128, seq_len=2)   # rows % 16
    assert A.gemm_cols_workspace(64, 512, 64) is not None  # this shape splits k
    with pytest.raises(InfernoHipError):
        A.dispatch_gemm_cols(x, w, out, rows=64, cols=512, seq_len=64)  # no workspace
