"""Per-op entry points of the gfx950 library against the oracle (same seeded
inputs): SwiGLU, NeoX RoPE, the causal conv + SiLU (the qkv GEMV's conv
epilogue run on its own), gated GQA attention through the token loop's
attention kernels (fused single-token and kv_store + split paths, more than 64
splits in the combine) and the DeltaNet step through both forms of the token
loop's recurrence kernel.

Bars, written per test: elementwise results within a few float32 roundings
(the device's expf and the compilers' fused multiply-adds differ from glibc's
by an ulp or two); copied state (conv windows, fp16 values) bit-exact; fp16
keys within one fp16 ulp; attention outputs within 1e-5 relative L2.
"""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from helpers import draw_from_order, slot_history_cases
from conftest import rel_l2
from test_oracle import attn_inputs

pytestmark = pytest.mark.gpu


def _close(got, want, rtol):
    scale = np.maximum(np.abs(want), np.abs(want).max() * 1e-3)
    return float(np.max(np.abs(got - want) / scale)) < rtol


@pytest.mark.parametrize("n", [1, 255, 100003])
def test_swiglu_matches_oracle(n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    assert _close(xp.swiglu(g, u), orc.swiglu(g, u), 1e-6)


@pytest.mark.parametrize("n_rot,D,pos0", [(64, 256, 0), (64, 256, 4093), (128, 128, 17)])
def test_rope_matches_oracle(n_rot, D, pos0):
    """Rows laid out as the attention queries are ([q(D) | gate(D)] per head):
    only the first n_rot dims of each head's q rotate; everything else is left
    bit for bit."""
    rng = np.random.default_rng(pos0 + n_rot)
    T, H = 5, 6
    x = rng.standard_normal((T, H * 2 * D)).astype(np.float32)
    got = xp.rope(x, n_rot, pos0, 1e7, head_stride=2 * D)
    want = x.copy().reshape(T, H, 2 * D)
    for t in range(T):
        for h in range(H):
            want[t, h, :D] = orc.rope(want[t, h, :D], n_rot, pos0 + t, 1e7)
    want = want.reshape(T, -1)
    assert _close(got, want, 1e-6)
    rot = np.zeros((H, 2 * D), bool)
    rot[:, :n_rot] = True
    keep = ~np.tile(rot.reshape(-1), (T, 1))
    assert np.array_equal(got[keep], x[keep])


@pytest.mark.parametrize("K,Cn,T,ck_n", [(4, 8192, 1, 0), (4, 6144, 5, 4), (2, 1000, 3, 3), (6, 777, 17, 16)])
def test_conv_silu_matches_oracle(K, Cn, T, ck_n):
    rng = np.random.default_rng(K * 1000 + T)
    x = rng.standard_normal((T, Cn)).astype(np.float32)
    w = rng.standard_normal((Cn, K)).astype(np.float32)
    st = rng.standard_normal((Cn, K - 1)).astype(np.float32)
    got, gst, gck = xp.conv_silu(x, w, st, ck_n)
    want, wst, wck = orc.conv_silu(x, w, st, ck_n)
    # the K-term sums may cancel: bound the difference by the float32 rounding of
    # a K-term dot product, K * eps * sum_k |w_k x_k| (silu' < 1.1), plus the
    # rounding of silu itself
    seq = np.abs(np.concatenate([st.T, x], axis=0)).astype(np.float64)
    mag = np.stack([np.einsum("kc,ck->c", seq[t:t + K], np.abs(w).astype(np.float64)) for t in range(T)])
    bound = 1.1 * K * 2.0**-23 * mag + 4 * 2.0**-24 * np.abs(want)
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    assert np.array_equal(gst, wst)
    if ck_n:
        assert np.array_equal(gck, wck)


def test_conv_silu_state_carries_across_calls():
    """Two calls of 3 and 4 tokens equal one call of 7."""
    rng = np.random.default_rng(5)
    K, Cn = 4, 512
    x = rng.standard_normal((7, Cn)).astype(np.float32)
    w = rng.standard_normal((Cn, K)).astype(np.float32)
    st = np.zeros((Cn, K - 1), np.float32)
    a, sa, _ = xp.conv_silu(x[:3], w, st)
    b, sb, _ = xp.conv_silu(x[3:], w, sa)
    c, sc, _ = xp.conv_silu(x, w, st)
    assert np.array_equal(np.concatenate([a, b]), c) and np.array_equal(sb, sc)


ATTN_CASES = [
    # T, H, Hkv, D, n_rot, n_past, n_ctx
    (1, 16, 4, 256, 64, 0, 64),        # first token
    (1, 16, 4, 256, 64, 777, 1024),    # fused single-token path
    (1, 8, 2, 256, 64, 2500, 4096),    # 40 splits of 64 positions
    (1, 8, 2, 128, 64, 4200, 4608),    # 66 splits (> 64) in the combine
    (4, 16, 4, 256, 64, 2600, 4096),   # kv_store + split path
    (3, 8, 2, 128, 128, 31, 128),      # the batch crosses a split boundary
    (5, 8, 8, 64, 32, 60, 96),         # G = 1
    (2, 8, 1, 64, 64, 10, 64),         # G = 8
]


@pytest.mark.parametrize("T,H,Hkv,D,n_rot,n_past,n_ctx", ATTN_CASES)
def test_attn_decode_matches_oracle(T, H, Hkv, D, n_rot, n_past, n_ctx):
    print(f"attn_decode T={T} H={H} Hkv={Hkv} D={D} n_past={n_past} n_ctx={n_ctx}", flush=True)
    qg, k, v, qn, kn, kc, vc = attn_inputs(T, H, Hkv, D, n_past, n_ctx, 50 + n_past)
    base, eps = 1e7, 1e-6
    got, gkc, gvc = xp.attn_decode(qg, k, v, qn, kn, kc, vc, n_past, n_rot, base, eps)
    f = lambda b: b.view(np.float16).astype(np.float32)
    want, wkc, wvc = orc.attn_decode(qg, k, v, qn, kn, f(kc), f(vc), n_past, n_rot, base, eps)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) < 1e-5
    new = slice(n_past, n_past + T)
    assert np.array_equal(gvc[new], wvc[new].astype(np.float16).view(np.uint16))
    kd = np.abs(gkc[new].astype(np.int32) - wkc[new].astype(np.float16).view(np.uint16).astype(np.int32))
    assert kd.max() <= 1
    # nothing else in the caches changed
    assert np.array_equal(gkc[:n_past], kc[:n_past]) and np.array_equal(gkc[n_past + T:], kc[n_past + T:])
    assert np.array_equal(gvc[:n_past], vc[:n_past]) and np.array_equal(gvc[n_past + T:], vc[n_past + T:])


def test_attn_decode_token_by_token_equals_batch():
    """Three single-token calls leave the same caches (bit for bit) and the same
    outputs (to the fp32 reassociation of the two launch forms) as one call of 3."""
    T, H, Hkv, D, n_past, n_ctx = 3, 16, 4, 256, 100, 256
    qg, k, v, qn, kn, kc, vc = attn_inputs(T, H, Hkv, D, n_past, n_ctx, 77)
    ob, kcb, vcb = xp.attn_decode(qg, k, v, qn, kn, kc, vc, n_past, 64, 1e7, 1e-6)
    kcs, vcs, outs = kc, vc, []
    for t in range(T):
        o, kcs, vcs = xp.attn_decode(qg[t:t + 1], k[t:t + 1], v[t:t + 1], qn, kn, kcs, vcs, n_past + t, 64, 1e7, 1e-6)
        outs.append(o)
    assert np.array_equal(kcs, kcb) and np.array_equal(vcs, vcb)
    assert rel_l2(np.concatenate(outs), ob) < 1e-6


def test_per_op_entries_reject_bad_shapes():
    with pytest.raises(xp.XjError):
        xp.conv_silu(np.zeros((2, 8), np.float32), np.zeros((8, 9), np.float32), np.zeros((8, 8), np.float32))
    qg, k, v, qn, kn, kc, vc = attn_inputs(2, 8, 2, 64, 62, 64, 1)
    with pytest.raises(xp.XjError):   # n_past + T > n_ctx
        xp.attn_decode(qg, k, v, qn, kn, kc, vc, 63, 64, 1e4, 1e-6)
    qg, k, v, qn, kn, kc, vc = attn_inputs(1, 6, 2, 64, 0, 8, 1)
    with pytest.raises(xp.XjError):   # H / Hkv = 3
        xp.attn_decode(qg, k, v, qn, kn, kc, vc, 0, 64, 1e4, 1e-6)


@pytest.mark.parametrize("split", ["1", "0"])
@pytest.mark.parametrize("T,Hk,Hv,S,ck_n", [(1, 16, 32, 128, 0), (5, 16, 32, 128, 4), (9, 4, 8, 64, 9), (2, 2, 6, 128, 1)])
def test_delta_step_matches_oracle(monkeypatch, split, T, Hk, Hv, S, ck_n):
    """Both forms of the token loop's DeltaNet kernel (32 value rows per
    work-group, and one work-group per head) against xjo_delta_step: outputs,
    final state and checkpoints within 1e-5 relative L2 (the 16-lane partial
    sums are combined in a butterfly instead of one running sum)."""
    from test_oracle import delta_step_inputs
    monkeypatch.setenv("XJ_DELTA_SPLIT", split)
    print(f"delta_step split={split} T={T} Hk={Hk} Hv={Hv} S={S} ck_n={ck_n}", flush=True)
    qkv, ko, vo, beta, alpha, dt, A, st = delta_step_inputs(T, Hk, Hv, S, 70 + T)
    qs = 1 / np.sqrt(np.float32(S))
    got, gst, gck = xp.delta_step(qkv, ko, vo, beta, alpha, dt, A, Hk, Hv, S, 1e-6, qs, st, ck_n)
    want, wst, wck = orc.delta_step(qkv, ko, vo, beta, alpha, dt, A, Hk, Hv, S, 1e-6, qs, st, ck_n)
    assert rel_l2(got, want) < 1e-5
    assert rel_l2(gst, wst) < 1e-5
    for t in range(ck_n):
        assert rel_l2(gck[t], wck[t]) < 1e-5
    if ck_n == T:
        assert np.array_equal(gck[-1], gst)


def test_delta_step_forms_agree_bit_for_bit(monkeypatch):
    """The per-row arithmetic of the two forms is the same, so their results are
    identical."""
    from test_oracle import delta_step_inputs
    qkv, ko, vo, beta, alpha, dt, A, st = delta_step_inputs(6, 16, 32, 128, 80)
    res = []
    for split in ("1", "0"):
        monkeypatch.setenv("XJ_DELTA_SPLIT", split)
        res.append(xp.delta_step(qkv, ko, vo, beta, alpha, dt, A, 16, 32, 128, 1e-6, 0.0883883, st, 5))
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("V", [40, 1000, 151936])
def test_sample_equal_values_match_the_app(V):
    """Logits with many exact ties (multiples of 1/4: equal values inside the
    kept set and values equal to the 40th straddling its edge), so the app's
    slot history and exchange sort decide the order: the device's draw equals
    the oracle's restatement of the app row by row."""
    rng = np.random.default_rng(V + 11)
    T = 12
    lg = (np.round(rng.standard_normal((T, V)) * 8) / 4).astype(np.float32)
    r30 = rng.integers(0, 1 << 30, T).astype(np.uint32)
    for temp in (0.0, 0.3, 1.0, 10.0):
        got = xp.sample(lg, temp, r30)
        want = [orc.sample(lg[t], temp, int(r30[t])) for t in range(T)]
        assert got.tolist() == want, temp
    lg = np.array([[3.0, 3.0, 5.0]], np.float32)
    assert xp.sample(lg, 10.0, np.array([1 << 29], np.uint32)).tolist() == [1]


def test_sample_slot_history_cases():
    """The hand-worked slot orders (all values equal, replacements of the first
    minimum, interleaved values, the exchange sort's swaps, -0 == +0): the
    device draws what a draw from that order gives, for draws landing on every
    kept position."""
    for lg, order in slot_history_cases():
        vals = lg[order]
        r = np.array([0, 1, (1 << 30) - 1] + [int(x * (1 << 30)) for x in np.linspace(0.01, 0.99, 37)], np.uint32)
        for temp in (1e4, 3.0):
            got = xp.sample(np.tile(lg, (len(r), 1)), temp, r)
            want = [draw_from_order(vals, order, temp, int(x)) for x in r]
            assert got.tolist() == want, (lg[:6], temp)


@pytest.mark.parametrize("V", [3, 39, 40, 41, 5000, 151936])
def test_sample_edge_rows_match_the_app(V):
    """Rows that leave the fast path: NaN at index 0 and elsewhere, signed
    zeros at the 40th place, one repeated value, a rising row (every element
    enters), a falling row, large equal runs at the top; plus a row of
    distinct values. Device draws equal the oracle's for every row, greedy
    included (first maximum; NaN at index 0 wins as in `x[i] > x[b]`)."""
    rng = np.random.default_rng(V)
    rows = []
    base = rng.standard_normal(V).astype(np.float32)
    rows.append(base.copy())
    r = base.copy(); r[0] = np.nan; rows.append(r)
    r = base.copy(); r[V // 2] = np.nan; rows.append(r)
    r = np.where(rng.random(V) < 0.5, np.float32(-0.0), np.float32(0.0)).astype(np.float32)
    r[: min(V, 30)] = np.abs(rng.standard_normal(min(V, 30))).astype(np.float32) + 1
    rows.append(r)
    rows.append(np.full(V, 0.25, np.float32))
    rows.append(np.linspace(-3, 3, V).astype(np.float32))
    rows.append(np.linspace(3, -3, V).astype(np.float32))
    r = (np.round(rng.standard_normal(V)) / 2).astype(np.float32); r[rng.integers(0, V, 50)] = 4.0; rows.append(r)
    lg = np.stack(rows)
    T = lg.shape[0]
    for temp in (0.0, 0.7, 2.0):
        r30 = rng.integers(0, 1 << 30, T).astype(np.uint32)
        got = xp.sample(lg, temp, r30)
        want = [orc.sample(lg[t], temp, int(r30[t])) for t in range(T)]
        assert got.tolist() == want, temp


@pytest.mark.parametrize("V", [25, 1000, 151936])
def test_sample_matches_oracle(V):
    """The device sampler against the oracle's restatement of the app's sampler,
    row by row, over temperatures from greedy to nearly uniform."""
    rng = np.random.default_rng(V + 7)
    T = 14
    lg = (rng.standard_normal((T, V)) * 2).astype(np.float32)
    r30 = rng.integers(0, 1 << 30, T).astype(np.uint32)
    for temp in (0.0, 0.05, 0.7, 1.3, 50.0):
        got = xp.sample(lg, temp, r30)
        want = [orc.sample(lg[t], temp, int(r30[t])) for t in range(T)]
        assert got.tolist() == want, temp
