"""The matrix-core GEMM for prefill chunks (xjh_gemm) against the oracle's
matmul (src/xiaoju-pipe/core/xj_cpu.c:36-54), a float64 product of the same
dequantized weights, and the dot-product GEMV (xjh_gemv). The GEMM's
products are exact (f16 halves of the activations times small-integer
weights) and only its fp32 accumulation rounds: ~1e-7 of the float64
product; the GEMV's 21-bit activations put it ~1e-6 away."""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import rel_l2
from helpers import random_blocks

pytestmark = pytest.mark.gpu


def _weights(t, rows, k, seed):
    return xp.quantize(t, xp.fill_normal(rows * k, seed, 0.02).reshape(rows, k))


@pytest.mark.parametrize("t,rows,k", [
    (xp.Q4_K, 4096, 1024),     # Q4_K 4096 x 1024
    (xp.Q6_K, 3584, 1024),     # Q6_K 3584 x 1024
    (xp.Q4_K, 1000, 2560),     # rows not a multiple of 16 or 64
    (xp.Q6_K, 517, 9216),      # few rows: K split over work-groups, reduce launch
    (xp.Q4_K, 33, 256),        # one block per row
    (xp.Q4_K, 2560, 4096),     # 320 units: 160 work-groups of two (ssm_out / wo)
    (xp.Q6_K, 1024, 9216),     # 288 units: 144 work-groups of two, a row group over 18
])
@pytest.mark.parametrize("T", [1, 16, 17, 40, 64])
def test_gemm_matches_oracle_and_gemv(t, rows, k, T):
    blob = _weights(t, rows, k, 2000 + rows + k)
    xs = xp.fill_normal(T * k, 91 + T, 1.0).reshape(T, k)
    w = xp.DevWeight(t, blob, rows, k)
    got = xp.gemm(w, xs)
    want = orc.matmul(t, blob, k, rows, xs)
    assert rel_l2(got, want) < 1e-3
    wd = orc.dequant_rows(t, blob, rows, k).astype(np.float64)
    ref64 = xs.astype(np.float64) @ wd.T
    assert rel_l2(got, ref64) < 1e-6
    # the GEMV on the same inputs: both within ~1e-6 of the float64 product
    gv = np.concatenate([xp.gemv(w, xs[i:i + 5]) for i in range(0, T, 5)])
    assert rel_l2(gv, ref64) < 3e-6
    assert rel_l2(got, gv) < 3e-6
    assert np.max(np.abs(got - gv)) <= 5e-6 * np.max(np.abs(gv))


@pytest.mark.parametrize("t", [xp.Q4_K, xp.Q6_K])
def test_gemm_random_blocks_and_residual_add(t):
    """Blocks with every field random (edge fp16 scales included), and the
    residual-add form y += W x."""
    rows, k, T = 300, 1024, 37
    blob = random_blocks(t, rows, k, 5)
    w = xp.DevWeight(t, blob, rows, k)
    xs = xp.fill_normal(T * k, 8, 1.0).reshape(T, k)
    wd = orc.dequant_rows(t, blob, rows, k).astype(np.float64)
    finite = np.isfinite(wd).all(axis=1)
    ref64 = xs.astype(np.float64) @ np.where(np.isfinite(wd), wd, 0).T
    got = xp.gemm(w, xs)
    assert rel_l2(got[:, finite], ref64[:, finite]) < 1e-6
    base = xp.fill_normal(T * rows, 9, 1.0).reshape(T, rows)
    got2 = xp.gemm(w, xs, add_to=base)
    assert np.array_equal(got2[:, finite], (base + got)[:, finite])


def test_gemm_rejects_unsupported():
    blob = _weights(xp.Q4_K, 64, 256, 3)
    w = xp.DevWeight(xp.Q4_K, blob, 64, 256)
    with pytest.raises(xp.XjError):
        xp.gemm(w, np.zeros((65, 256), np.float32))
    q8 = xp.DevWeight(xp.Q8_0, _weights(xp.Q8_0, 64, 256, 4), 64, 256)
    with pytest.raises(xp.XjError):
        xp.gemm(q8, np.zeros((16, 256), np.float32))
