"""Per-kernel parity of the gfx950 library against the oracle (same seeded inputs).

Bars: dequantization bit-exact; GEMV within 1e-3 relative L2 of the oracle's
fp32 matmul (and of an fp64 evaluation of the same dequantized weights); row
results independent of T; norms, argmax and the delta rule as documented per
test.
"""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import rel_l2
from helpers import random_blocks

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t", [xp.Q4_K, xp.Q6_K, xp.Q8_0, xp.Q5_K, xp.F16, xp.BF16])
def test_dequant_bit_exact_random_blocks(t):
    rows, k = 96, 1024
    blob = random_blocks(t, rows, k, 11 + t)
    w = xp.DevWeight(t, blob, rows, k)
    got = xp.dequant(w)
    want = orc.dequant_rows(t, blob, rows, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [xp.Q4_K, xp.Q6_K, xp.Q8_0, xp.F32])
def test_dequant_bit_exact_quantized(t):
    rows, k = 64, 2560
    x = xp.fill_normal(rows * k, 123, 0.02).reshape(rows, k)
    blob = xp.quantize(t, x)
    w = xp.DevWeight(t, blob, rows, k)
    got = xp.dequant(w, 5, 40)
    want = orc.dequant_rows(t, blob, rows, k)[5:45]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _weights(t, rows, k, seed):
    x = xp.fill_normal(rows * k, seed, 0.02).reshape(rows, k)
    return xp.quantize(t, x)


@pytest.mark.parametrize("t,rows,k", [
    (xp.Q4_K, 4096, 1024),     # single Q4_K GEMV, 4096 x 1024
    (xp.Q6_K, 3584, 1024),     # mixed batch: Q6_K 3584 x 1024
    (xp.Q8_0, 1024, 3584),     # mixed batch: Q8_0 1024 x 3584
    (xp.Q4_K, 1000, 2560),     # rows not a multiple of 16
    (xp.Q6_K, 517, 9216),
    (xp.Q4_K, 33, 256),
    (xp.F32, 300, 512),
    (xp.Q8_0, 300, 9216),      # five tokens of K = 9216 need two launches of the looping kernel
    (xp.F32, 130, 9216),
])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5])
def test_gemv_matches_oracle(t, rows, k, T):
    blob = _weights(t, rows, k, 1000 + rows + k)
    xs = xp.fill_normal(T * k, 77 + T, 1.0).reshape(T, k)
    w = xp.DevWeight(t, blob, rows, k)
    got = xp.gemv(w, xs)
    want = orc.matmul(t, blob, k, rows, xs)
    assert rel_l2(got, want) < 1e-3
    # fp64 evaluation of the same dequantized weights: the oracle's own error is far below the bar
    wd = orc.dequant_rows(t, blob, rows, k).astype(np.float64)
    ref64 = xs.astype(np.float64) @ wd.T
    assert rel_l2(got, ref64) < 1e-5
    assert rel_l2(want, ref64) < 1e-5


def _secondary_weights(t, rows, k, seed):
    """Finite weights of the types no configuration uses: F16 / BF16 rounded
    (RNE) from normal samples; Q5_K blocks with every field random except d and
    dmin, drawn from a few ordinary fp16 scales (no quantizer for Q5_K exists)."""
    rng = np.random.default_rng(seed)
    if t in (xp.F16, xp.BF16):
        x = (rng.standard_normal((rows, k)) * 0.05).astype(np.float32)
        if t == xp.F16:
            return x.astype(np.float16).view(np.uint8).reshape(-1).copy()
        b = x.view(np.uint32).astype(np.uint64)
        b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16   # round to nearest even (finite inputs)
        return b.astype(np.uint16).view(np.uint8).reshape(-1).copy()
    rb = xp.row_bytes(t, k)
    blob = rng.integers(0, 256, rows * rb, dtype=np.uint8)
    blocks = blob.reshape(-1, 176)
    scales = np.array([0.004, 0.002, 0.0015, 0.003], np.float16).view(np.uint16)
    h = scales[rng.integers(0, len(scales), (blocks.shape[0], 2))]
    blocks[:, 0:4] = h.view(np.uint8).reshape(-1, 4)
    return blob


@pytest.mark.parametrize("t,rows,k", [(xp.Q5_K, 700, 2560), (xp.F16, 300, 1024), (xp.BF16, 257, 512)])
@pytest.mark.parametrize("T", [1, 3, 5])
def test_gemv_secondary_types(t, rows, k, T):
    blob = _secondary_weights(t, rows, k, 300 + t)
    xs = xp.fill_normal(T * k, 90 + T, 1.0).reshape(T, k)
    w = xp.DevWeight(t, blob, rows, k)
    got = xp.gemv(w, xs)
    want = orc.matmul(t, blob, k, rows, xs)
    assert rel_l2(got, want) < 1e-3
    wd = orc.dequant_rows(t, blob, rows, k).astype(np.float64)
    assert np.isfinite(wd).all()
    ref64 = xs.astype(np.float64) @ wd.T
    assert rel_l2(got, ref64) < 1e-5
    assert np.array_equal(xp.dequant(w).view(np.uint32), orc.dequant_rows(t, blob, rows, k).view(np.uint32))


@pytest.mark.parametrize("t,rows,k,tmax", [
    (xp.Q4_K, 777, 2560, 5), (xp.Q6_K, 777, 2560, 5), (xp.Q8_0, 777, 3584, 5),
    (xp.Q4_K, 763, 2560, 5), (xp.Q6_K, 763, 2560, 5),    # 3 rows per work-group: a team with one row
    (xp.Q4_K, 18432, 2560, 5),                            # gate | up of the 4B shape
    (xp.Q6_K, 18000, 2560, 5),                            # 8-lane teams of Q6_K rows
    (xp.Q4_K, 2560, 4096, 5),                             # ssm_out / wo
    (xp.Q6_K, 2560, 9216, 5),                             # down (five tokens staged in one per-CU launch)
    (xp.Q8_0, 2560, 9216, 5),                             # the looping kernel: five tokens as 4 + 1
    (xp.Q6_K, 3584, 1024, 5),                             # 14 rows per work-group, 64 lanes per row
    (xp.Q4_K, 7168, 1024, 5),                             # gate | up of the 0.8B shape: 32-lane teams
    (xp.Q6_K, 1024, 3584, 5),                             # down of the 0.8B shape: 16-lane teams
    (xp.Q4_K, 3, 1024, 5), (xp.Q6_K, 5, 9216, 5),         # one row per work-group: a pair with one row
])
def test_gemv_rows_do_not_depend_on_T(t, rows, k, tmax):
    """Row r of a T-token launch equals the single-token launch bit for bit
    (speculative verification reproduces greedy decoding), for every T."""
    blob = _weights(t, rows, k, 5)
    xs = xp.fill_normal(5 * k, 6, 1.0).reshape(5, k)
    w = xp.DevWeight(t, blob, rows, k)
    y1 = np.stack([xp.gemv(w, xs[i:i + 1])[0] for i in range(tmax)])
    for T in range(2, tmax + 1):
        yT = xp.gemv(w, xs[:T])
        assert np.array_equal(yT.view(np.uint32), y1[:T].view(np.uint32)), T


def test_gemv_residual_add():
    rows, k = 512, 1024
    blob = _weights(xp.Q4_K, rows, k, 9)
    xs = xp.fill_normal(2 * k, 10, 1.0).reshape(2, k)
    base = xp.fill_normal(2 * rows, 12, 1.0).reshape(2, rows)
    w = xp.DevWeight(xp.Q4_K, blob, rows, k)
    got = xp.gemv(w, xs, add_to=base)
    want = base + xp.gemv(w, xs)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("t", [xp.Q4_K, xp.Q6_K])
def test_gemv_lm_head_shape(t):
    """151936 x 1024 (the 0.8B model's LM-head shape; a single token loops
    over row groups with the next group's units in flight) at every
    speculative-verify width T = 1..5."""
    rows, k = 151936, 1024
    blob = _weights(t, rows, k, 31)
    w = xp.DevWeight(t, blob, rows, k)
    for T in (1, 2, 3, 4, 5):
        xs = xp.fill_normal(T * k, 40 + T, 1.0).reshape(T, k)
        got = xp.gemv(w, xs)
        want = orc.matmul(t, blob, k, rows, xs)
        assert rel_l2(got, want) < 1e-3
        assert np.array_equal(np.argmax(got, 1), np.argmax(want, 1))


@pytest.mark.parametrize("mode", [0, 1])
def test_norm(mode):
    x = xp.fill_normal(6 * 2560, 3, 1.5).reshape(6, 2560)
    w = 1 + 0.1 * xp.fill_normal(2560, 4, 1.0)
    got = xp.norm(x, w if mode == 0 else None, mode, 1e-6)
    for r in range(6):
        if mode == 0:
            want = orc.rmsnorm(x[r], w, 1e-6)
        else:
            ss = np.sum(x[r].astype(np.float64) ** 2)
            want = x[r] * np.float32(1.0 / np.sqrt(np.float32(ss) + np.float32(1e-6)))
        assert rel_l2(got[r], want) < 1e-6


def test_argmax_first_maximum():
    """`if (x[i] > x[b]) b = i` from b = 0: ties and -0 == +0 keep the lowest
    index, NaN never wins - except at index 0, where nothing compares above it."""
    x = xp.fill_normal(7 * 151936, 8, 1.0).reshape(7, 151936)
    x[1, 1000] = x[1, 50000] = x[1, 150000] = 99.0     # ties: lowest index wins
    x[2, :] = -3.0                                     # all equal -> index 0
    x[3, 151935] = 1e30
    x[4, 0] = np.nan                                   # NaN first: 0
    x[5, 77] = np.nan                                  # NaN elsewhere: ignored
    x[5, 78] = 50.0
    x[6, :] = -1.0
    x[6, 5], x[6, 7] = -0.0, 0.0                       # -0 first, +0 is not above it
    got = xp.argmax(x)
    want = [orc.olib().xjo_argmax(row.ctypes.data_as(orc.C.c_void_p), row.size) for row in x]
    assert got.tolist() == want
    assert got.tolist()[1:] == [1000, 0, 151935, 0, 78, 5]


def _delta_inputs(T, H, S, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, H, S)).astype(np.float32)
    k = rng.standard_normal((T, H, S)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, H, S)).astype(np.float32)
    sig = lambda z: 1 / (1 + np.exp(-z))
    decay = sig(rng.standard_normal((T, H))).astype(np.float32)
    beta = sig(rng.standard_normal((T, H))).astype(np.float32)
    return q, k, v, decay, beta


@pytest.mark.parametrize("S", [64, 128])
def test_delta_recurrent_matches_oracle(S):
    T, H = 48, 4
    q, k, v, dec, beta = _delta_inputs(T, H, S, 1)
    st0 = np.random.default_rng(2).standard_normal((H, S, S)).astype(np.float32) * 0.1
    qs = 1 / np.sqrt(S)
    go, gs = xp.delta(q, k, v, dec, beta, st0, qs)
    oo, os_ = orc.delta_recurrent(q, k, v, dec, beta, st0, qs)
    assert rel_l2(go, oo) < 1e-4
    assert rel_l2(gs, os_) < 1e-4


@pytest.mark.parametrize("T", [64, 200, 2048])
def test_delta_chunked_matches_recurrent(T):
    """2048-token chunk-wise prefill of a 16-head, d=128 layer vs the token-by-token oracle."""
    H, S = 16, 128
    q, k, v, dec, beta = _delta_inputs(T, H, S, 3 + T)
    st0 = np.zeros((H, S, S), np.float32)
    qs = 1 / np.sqrt(S)
    go, gs = xp.delta(q, k, v, dec, beta, st0, qs, chunk=64)
    oo, os_ = orc.delta_recurrent(q, k, v, dec, beta, st0, qs)
    assert rel_l2(go, oo) < 1e-3
    assert rel_l2(gs, os_) < 1e-3


def test_delta_prefill_then_decode():
    """2048-token chunked prefill followed by 256 single-token recurrent steps."""
    H, S, T0, T1 = 16, 128, 2048, 256
    q, k, v, dec, beta = _delta_inputs(T0 + T1, H, S, 99)
    qs = 1 / np.sqrt(S)
    st = np.zeros((H, S, S), np.float32)
    go0, gst = xp.delta(q[:T0], k[:T0], v[:T0], dec[:T0], beta[:T0], st, qs, chunk=64)
    outs = []
    for t in range(T0, T0 + T1):       # single-token steps of the recurrent kernel
        o, gst = xp.delta(q[t:t + 1], k[t:t + 1], v[t:t + 1], dec[t:t + 1], beta[t:t + 1], gst, qs)
        outs.append(o)
    oo, ost = orc.delta_recurrent(q, k, v, dec, beta, st, qs)
    assert rel_l2(go0, oo[:T0]) < 1e-3
    assert rel_l2(np.concatenate(outs), oo[T0:]) < 1e-3
    assert rel_l2(gst, ost) < 1e-3
