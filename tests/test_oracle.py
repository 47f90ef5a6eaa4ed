"""Pins the oracle (the CPU restatement used as the checker) before anything is
compared with it:

  * the reference's own known-answer tests (src/xiaoju-pipe/tests/unit.c:17-51:
    f16 round trip, a hand-built Q8_0 block, a hand-built Q4_K block over both
    scale paths), plus a hand-built Q6_K block from the format's definition;
  * golden vectors written by the reference compiled from source
    (tests/golden/*.npz|json, see gen_golden.py);
  * live bit-for-bit comparison with that reference build where it exists
    (oracle/_ref), including an -march=native build against the portable one;
  * invariants the mathematics fixes for the delta rule;
  * float64 brute force from the definitions for the per-op restatements
    (SwiGLU, the causal conv + SiLU, gated GQA attention with its fp16 cache),
    plus the closed form of attention over a single position.
"""
import json
import os
import struct

import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import GOLDEN, rel_l2
from helpers import draw_from_order, np_sample, random_blocks, slot_history_cases

needs_ref = pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")


# ------------------------------------------------------------ unit.c KATs --

def test_kat_f16_round_trip():
    """unit.c:17-24"""
    for v in [0.0, 1.0, -2.5, 65504.0, 6.1035156e-05, 5.9604645e-08, 0.33325195, -1e-3]:
        back = orc.f16_to_f32(orc.f32_to_f16(v))
        assert abs(back - v) <= abs(v) * 1e-3 + 1e-7
    assert np.isinf(orc.f16_to_f32(orc.f32_to_f16(1e6)))


def test_f16_conversion_is_ieee_rne():
    """Every one of the 65536 fp16 patterns decodes as numpy's IEEE half does, and
    re-encodes to itself (NaNs excepted); encoding ties round to even."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.isnan(got[~finite & np.isnan(want)]).all()
    enc = np.array([orc.f32_to_f16(float(v)) for v in want[finite]], np.uint16)
    assert np.array_equal(enc, bits[finite])
    x = xp.fill_normal(20000, 3, 100.0)
    ours = np.array([orc.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))


def test_kat_q8_0_block():
    """unit.c:28-34"""
    blk = struct.pack("<H", orc.f32_to_f16(0.5)) + bytes((i - 16) & 0xFF for i in range(32))
    y = orc.dequant_rows(xp.Q8_0, np.frombuffer(blk, np.uint8), 1, 32)[0]
    assert np.array_equal(y, 0.5 * (np.arange(32) - 16))


def test_kat_q4_k_block_both_scale_paths():
    """unit.c:36-51: sub-blocks 0..3 scale j+1 / min j, 4..7 scale 2 / min 1 (high-bit path)."""
    b = bytearray(144)
    b[0:2] = struct.pack("<H", orc.f32_to_f16(0.25))
    b[2:4] = struct.pack("<H", orc.f32_to_f16(1.0))
    for j in range(4):
        b[4 + j] = j + 1
        b[8 + j] = j
    for j in range(4, 8):
        b[12 + j - 4] = 2 | (1 << 4)
    for i in range(128):
        b[16 + i] = (i % 16) | ((15 - i % 16) << 4)
    y = orc.dequant_rows(xp.Q4_K, np.frombuffer(bytes(b), np.uint8), 1, 256)[0]
    for e in range(256):
        j, l, g = e // 32, e % 32, e // 64
        byte = b[16 + 32 * g + l]
        q = byte >> 4 if j & 1 else byte & 15
        sc, mn = (j + 1, j) if j < 4 else (2, 1)
        assert abs(y[e] - (0.25 * sc * q - 1.0 * mn)) < 1e-6


def test_kat_q6_k_block():
    """A Q6_K block built from the format's definition: element e = 128h+32g+l has
    q = (nibble of ql[64h+32(g&1)+l], low for g<2) | 2 bits of qh[32h+l] >> 2g, minus 32,
    scale sc[e/16], value (d*sc)*q. The reference has no Q6_K KAT."""
    rng = np.random.default_rng(1)
    q = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16)
    d = 0.0137
    b = bytearray(210)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * h + 32 * g + l] for g in range(4))
            b[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.array(sc, np.int8).tobytes()
    dh = orc.f32_to_f16(d)
    b[208:210] = struct.pack("<H", dh)
    y = orc.dequant_rows(xp.Q6_K, np.frombuffer(bytes(b), np.uint8), 1, 256)[0]
    df = np.float32(orc.f16_to_f32(dh))
    want = (df * sc[np.arange(256) // 16].astype(np.float32)) * (q - 32).astype(np.float32)
    assert np.array_equal(y, want.astype(np.float32))


# ----------------------------------------------------------- golden files --

def test_golden_dequant():
    g = np.load(os.path.join(GOLDEN, "dequant_golden.npz"))
    for t in (xp.F16, xp.BF16, xp.Q8_0, xp.Q4_K, xp.Q5_K, xp.Q6_K):
        blob = g[f"blob_{t}"]
        want = g[f"ref_{t}"]
        got = orc.dequant_rows(t, blob, want.shape[0], want.shape[1])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), xp.TYPE_NAMES[t]
    bits = np.array([orc.f32_to_f16(float(v)) for v in g["f16_in"]], np.uint16)
    assert np.array_equal(bits, g["f16_bits"])


def test_golden_matmul():
    g = np.load(os.path.join(GOLDEN, "matmul_golden.npz"))
    for key in g.files:
        if not key.startswith("w_"):
            continue
        _, t, k = key.split("_")
        t, k = int(t), int(k)
        x, y = g[f"x_{t}_{k}"], g[f"y_{t}_{k}"]
        got = orc.matmul(t, g[key], k, y.shape[1], x)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32))


def test_golden_greedy_tiny(tiny_path):
    rec = json.load(open(os.path.join(GOLDEN, "greedy_tiny.json")))
    assert os.path.getsize(tiny_path) == rec["bytes"]
    m = xp.Model(tiny_path)
    L = m.hp.n_layer
    prompt = np.array(rec["prompt"], np.int32)
    for split in (0, 3):
        want = rec[f"ref_split{split}"]
        stages = [orc.CpuStage(m.ptr, 0, L, 256, 8, True)] if split == 0 else \
            [orc.CpuStage(m.ptr, 0, split, 256, 8, False), orc.CpuStage(m.ptr, split, L, 256, 8, True)]
        toks, mg = orc.greedy(stages, prompt, len(want["tokens"]))
        assert toks.tolist() == want["tokens"]
        assert np.array_equal(mg, np.array(want["margins"], np.float32))
        for s in stages:
            s.destroy()


# ---------------------------------------------- live reference comparison --

@needs_ref
@pytest.mark.parametrize("t", [xp.F16, xp.BF16, xp.Q8_0, xp.Q4_K, xp.Q5_K, xp.Q6_K])
def test_dequant_vs_reference_build(t):
    rows, k = 64, 1024
    blob = random_blocks(t, rows, k, 500 + t)
    a = orc.dequant_rows(t, blob, rows, k)
    b = orc.dequant_rows(t, blob, rows, k, lib=orc.rlib())
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("t,rows,k,T", [(xp.Q4_K, 300, 2560, 5), (xp.Q6_K, 200, 9216, 2), (xp.Q8_0, 100, 3584, 3),
                                        (xp.F32, 50, 256, 1)])
def test_matmul_vs_reference_build(t, rows, k, T):
    w = xp.quantize(t, xp.fill_normal(rows * k, t + k, 0.02).reshape(rows, k))
    x = xp.fill_normal(T * k, 3, 1.0).reshape(T, k)
    a = orc.matmul(t, w, k, rows, x)
    b = orc.matmul(t, w, k, rows, x, ref=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
def test_norm_rope_vs_reference_build():
    x = xp.fill_normal(2560, 1, 2.0)
    w = 1 + 0.1 * xp.fill_normal(2560, 2, 1.0)
    assert np.array_equal(orc.rmsnorm(x, w, 1e-6), orc.rmsnorm(x, w, 1e-6, ref=True))
    v = xp.fill_normal(256, 4, 1.0)
    for pos in (0, 1, 17, 1023, 1540, 40000):
        assert np.array_equal(orc.rope(v, 64, pos, 1e7), orc.rope(v, 64, pos, 1e7, ref=True))


@needs_ref
def test_greedy_vs_reference_pipeline(tiny_path):
    """The oracle's stage + loop against the reference's own pipeline and greedy driver
    (fp32 KV): same tokens and the same top-2 margins, so the logits agree bit for bit."""
    m = xp.Model(tiny_path)
    L = m.hp.n_layer
    prompt = np.random.default_rng(5).integers(0, m.hp.n_vocab, 29).astype(np.int32)
    want, wmg = orc.ref_greedy(tiny_path, prompt, 48, split=0, n_ctx=256, max_batch=8)
    st = orc.CpuStage(m.ptr, 0, L, 256, 8, True)
    got, gmg = orc.greedy([st], prompt, 48)
    assert got.tolist() == want.tolist()
    assert np.array_equal(gmg, wmg)


@needs_ref
def test_cpu_stage_rollback_vs_reference(tiny_path):
    m = xp.Model(tiny_path)
    L = m.hp.n_layer
    toks = np.random.default_rng(6).integers(0, m.hp.n_vocab, 12).astype(np.int32)
    outs = []
    for ref in (False, True):
        s = orc.CpuStage(m.ptr, 0, L, 64, 8, True, ref=ref)
        s.forward(np.stack([orc.embed(m.ptr, int(t)) for t in toks[:5]]))
        s.set_keep(4)
        s.forward(np.stack([orc.embed(m.ptr, int(t)) for t in toks[5:9]]))
        s.rollback(7)
        outs.append(s.forward(np.stack([orc.embed(m.ptr, int(t)) for t in toks[9:12]])))
        s.destroy()
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.skipif(not (orc.ref_available() and orc.ref_available(native=True)), reason="reference builds absent")
def test_reference_portable_build_equals_native(tiny_path):
    """The prebuilt (x86-64-v3) reference gives the same results as -march=native."""
    w = xp.quantize(xp.Q4_K, xp.fill_normal(64 * 2560, 9, 0.02).reshape(64, 2560))
    x = xp.fill_normal(2 * 2560, 10, 1.0).reshape(2, 2560)
    y = np.empty((2, 64), np.float32)
    for native in (False, True):
        L = orc.rlib(native)
        out = np.empty((2, 64), np.float32)
        L.ref_matmul(xp.Q4_K, w.ctypes.data_as(orc.C.c_void_p), 2560, 64, x.ctypes.data_as(orc.C.c_void_p),
                     out.ctypes.data_as(orc.C.c_void_p), 2)
        if native:
            assert np.array_equal(out, y)
        y = out


# -------------------------------------------------- delta-rule invariants --

def _unit(rng, shape):
    a = rng.standard_normal(shape).astype(np.float32)
    return a / np.linalg.norm(a, axis=-1, keepdims=True)


def test_delta_identity_gate_keeps_state():
    """decay = 1 and beta = 0: the state is unchanged and o = S q * qscale."""
    rng = np.random.default_rng(0)
    T, H, S = 5, 3, 64
    q, k = _unit(rng, (T, H, S)), _unit(rng, (T, H, S))
    v = rng.standard_normal((T, H, S)).astype(np.float32)
    st = rng.standard_normal((H, S, S)).astype(np.float32)
    out, st2 = orc.delta_recurrent(q, k, v, np.ones((T, H), np.float32), np.zeros((T, H), np.float32), st, 0.5)
    assert np.array_equal(st2, st)
    want = np.einsum("hji,thi->thj", st.astype(np.float64), q.astype(np.float64)) * 0.5
    assert rel_l2(out, want) < 1e-6


def test_delta_beta_one_writes_value():
    """beta = 1 with a unit key: after the update S k = v exactly (up to rounding)."""
    rng = np.random.default_rng(1)
    H, S = 2, 128
    k = _unit(rng, (1, H, S))
    v = rng.standard_normal((1, H, S)).astype(np.float32)
    st = rng.standard_normal((H, S, S)).astype(np.float32) * 0.3
    dec = np.full((1, H), 0.7, np.float32)
    _, st2 = orc.delta_recurrent(k, k, v, dec, np.ones((1, H), np.float32), st, 1.0)
    sk = np.einsum("hji,hi->hj", st2.astype(np.float64), k[0].astype(np.float64))
    assert rel_l2(sk, v[0]) < 1e-5


def test_delta_zero_state_linear_in_v():
    """From a zero state the outputs are linear in v (for fixed q, k, gates)."""
    rng = np.random.default_rng(2)
    T, H, S = 12, 2, 64
    q, k = _unit(rng, (T, H, S)), _unit(rng, (T, H, S))
    v1, v2 = rng.standard_normal((2, T, H, S)).astype(np.float32)
    dec = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    z = np.zeros((H, S, S), np.float32)
    o1, _ = orc.delta_recurrent(q, k, v1, dec, beta, z, 0.1)
    o2, _ = orc.delta_recurrent(q, k, v2, dec, beta, z, 0.1)
    o3, _ = orc.delta_recurrent(q, k, (2 * v1 - 3 * v2).astype(np.float32), dec, beta, z, 0.1)
    assert rel_l2(o3, 2 * o1.astype(np.float64) - 3 * o2) < 1e-5


def test_delta_matches_dense_definition():
    """Brute force in float64 from the definition S <- a S + beta (v - a S k) k^T."""
    rng = np.random.default_rng(3)
    T, H, S = 6, 2, 64
    q, k = _unit(rng, (T, H, S)), _unit(rng, (T, H, S))
    v = rng.standard_normal((T, H, S)).astype(np.float32)
    dec = rng.uniform(0.2, 1.0, (T, H)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (T, H)).astype(np.float32)
    st = rng.standard_normal((H, S, S)).astype(np.float32) * 0.2
    out, st2 = orc.delta_recurrent(q, k, v, dec, beta, st, 0.125)
    M = st.astype(np.float64)
    for t in range(T):
        for h in range(H):
            a = float(dec[t, h])
            M[h] = a * M[h]
            M[h] += float(beta[t, h]) * np.outer(v[t, h] - M[h] @ k[t, h], k[t, h])
            assert rel_l2(out[t, h], 0.125 * M[h] @ q[t, h]) < 1e-5
    assert rel_l2(st2, M) < 1e-5


def test_kv_f16_cache_rounds_only_the_cache(tiny_path):
    """The fp16-KV oracle differs from the fp32 one only through the rounded cache:
    outputs stay within fp16 rounding of each other."""
    m = xp.Model(tiny_path)
    L = m.hp.n_layer
    toks = np.random.default_rng(8).integers(0, m.hp.n_vocab, 10).astype(np.int32)
    x = np.stack([orc.embed(m.ptr, int(t)) for t in toks])
    a = orc.CpuStage(m.ptr, 0, L, 64, 16, True, kv_f16=False).forward(x.copy())
    b = orc.CpuStage(m.ptr, 0, L, 64, 16, True, kv_f16=True).forward(x.copy())
    assert 0 < rel_l2(b, a) < 5e-3


# ------------------------------------------- per-op restatements, brute force --

def _silu(x):
    return x / (1.0 + np.exp(-x))


def test_swiglu_matches_definition():
    rng = np.random.default_rng(20)
    g = (rng.standard_normal(4099) * 4).astype(np.float32)
    u = rng.standard_normal(4099).astype(np.float32)
    got = orc.swiglu(g, u)
    want = _silu(g.astype(np.float64)) * u
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30)) < 1e-5


@pytest.mark.parametrize("K", [2, 4, 6])
def test_conv_silu_matches_sliding_window(K):
    """out[t][c] = silu(sum_k w[c][k] * seq[t + k][c]) over seq = the K-1 stored
    inputs followed by the new ones; the state keeps the last K-1 inputs and
    checkpoint t is the state after token t."""
    rng = np.random.default_rng(21 + K)
    T, Cn = 9, 37
    x = rng.standard_normal((T, Cn)).astype(np.float32)
    w = rng.standard_normal((Cn, K)).astype(np.float32)
    st = rng.standard_normal((Cn, K - 1)).astype(np.float32)
    out, st2, ck = orc.conv_silu(x, w, st, ck_n=T - 1)
    seq = np.concatenate([st.T, x], axis=0).astype(np.float64)   # [K-1+T][C]
    want = np.stack([_silu(np.einsum("kc,ck->c", seq[t:t + K], w.astype(np.float64))) for t in range(T)])
    assert np.max(np.abs(out - want)) < 1e-5
    assert np.array_equal(st2, seq[T:T + K - 1].T.astype(np.float32))
    for t in range(T - 1):
        assert np.array_equal(ck[t], seq[t + 1:t + K].T.astype(np.float32))


def _np_rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def _np_rope(x, n_rot, pos, base):
    """NeoX RoPE with the angle formed in float32 as the reference does
    (theta = pos * powf(base, -2i/n_rot)), the rotation in float64."""
    x = x.copy()
    half = n_rot // 2
    i = np.arange(half, dtype=np.float32)
    inv = np.power(np.float32(base), np.float32(-2.0) * i / np.float32(n_rot), dtype=np.float32)
    th = (np.float32(pos) * inv).astype(np.float64)
    c, s = np.cos(th), np.sin(th)
    x0, x1 = x[:half].copy(), x[half:n_rot].copy()
    x[:half] = x0 * c - x1 * s
    x[half:n_rot] = x0 * s + x1 * c
    return x


def np_attn_decode(qg, k, v, qn, kn, kc, vc, n_past, n_rot, base, eps):
    """Gated GQA attention from its definition in float64, with the new keys and
    values rounded to fp16 in the cache."""
    T, H, D2 = qg.shape
    D, Hkv = D2 // 2, k.shape[1]
    kc, vc = kc.astype(np.float64), vc.astype(np.float64)
    for t in range(T):
        pos = n_past + t
        for g in range(Hkv):
            kk = _np_rope(_np_rms(k[t, g].astype(np.float64), kn, eps), n_rot, pos, base)
            kc[pos, g * D:(g + 1) * D] = kk.astype(np.float32).astype(np.float16)
            vc[pos, g * D:(g + 1) * D] = v[t, g].astype(np.float16)
    out = np.zeros((T, H * D))
    for t in range(T):
        pos = n_past + t
        for h in range(H):
            g = h // (H // Hkv)
            q = _np_rope(_np_rms(qg[t, h, :D].astype(np.float64), qn, eps), n_rot, pos, base)
            s = kc[:pos + 1, g * D:(g + 1) * D] @ q / np.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[t, h * D:(h + 1) * D] = (p @ vc[:pos + 1, g * D:(g + 1) * D]) / (1.0 + np.exp(-qg[t, h, D:].astype(np.float64)))
    return out, kc, vc


def attn_inputs(T, H, Hkv, D, n_past, n_ctx, seed):
    """Seeded inputs for one attention call: the cache below n_past holds fp16
    values; positions at and past n_past hold 0x7E00 (a NaN) so a read of an
    unwritten slot shows."""
    rng = np.random.default_rng(seed)
    qg = rng.standard_normal((T, H, 2 * D)).astype(np.float32)
    k = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((T, Hkv, D)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kc = np.full((n_ctx, Hkv * D), 0x7E00, np.uint16)
    vc = np.full((n_ctx, Hkv * D), 0x7E00, np.uint16)
    kc[:n_past] = (rng.standard_normal((n_past, Hkv * D)) * 2).astype(np.float16).view(np.uint16)
    vc[:n_past] = rng.standard_normal((n_past, Hkv * D)).astype(np.float16).view(np.uint16)
    return qg, k, v, qn, kn, kc, vc


@pytest.mark.parametrize("T,H,Hkv,D,n_rot,n_past", [(1, 4, 4, 64, 64, 0), (3, 8, 2, 64, 32, 40), (2, 8, 1, 128, 64, 70)])
def test_attn_decode_matches_definition(T, H, Hkv, D, n_rot, n_past):
    n_ctx = n_past + T + 3
    qg, k, v, qn, kn, kc, vc = attn_inputs(T, H, Hkv, D, n_past, n_ctx, 30 + T)
    f = lambda b: b.view(np.float16).astype(np.float32)
    out, kc2, vc2 = orc.attn_decode(qg, k, v, qn, kn, f(kc), f(vc), n_past, n_rot, 1e6, 1e-6)
    want, wkc, wvc = np_attn_decode(qg, k, v, qn, kn, f(kc), f(vc), n_past, n_rot, 1e6, 1e-6)
    assert rel_l2(out, want) < 1e-4
    new = slice(n_past, n_past + T)
    assert np.array_equal(vc2[new], wvc[new].astype(np.float32))
    # keys: the same fp16 value unless float32 and float64 round across a half-way point
    kd = np.abs(kc2[new].astype(np.float16).view(np.uint16).astype(np.int32) -
                wkc[new].astype(np.float16).view(np.uint16).astype(np.int32))
    assert kd.max() <= 1 and np.mean(kd) < 0.01
    assert np.array_equal(kc2[:n_past], f(kc)[:n_past])


def test_attn_decode_single_position_returns_gated_value():
    """At position 0 the softmax has one term: out = fp16(v) * sigmoid(gate) for
    every query head of the kv head, whatever q and k are."""
    T, H, Hkv, D = 1, 4, 2, 64
    qg, k, v, qn, kn, kc, vc = attn_inputs(T, H, Hkv, D, 0, 4, 40)
    f = lambda b: b.view(np.float16).astype(np.float32)
    out, _, _ = orc.attn_decode(qg, k, v, qn, kn, f(kc), f(vc), 0, D, 1e4, 1e-6)
    for h in range(H):
        g = h // (H // Hkv)
        want = v[0, g].astype(np.float16).astype(np.float64) / (1 + np.exp(-qg[0, h, D:].astype(np.float64)))
        assert rel_l2(out[0, h * D:(h + 1) * D], want) < 1e-6


def delta_step_inputs(T, Hk, Hv, S, seed):
    """Seeded inputs of the DeltaNet recurrence after the conv: qkv rows
    [q (Hk*S) | k (Hk*S) | v (Hv*S)], raw gates, dt, A < 0 and a state."""
    rng = np.random.default_rng(seed)
    kd = Hk * S
    qkv = rng.standard_normal((T, 2 * kd + Hv * S)).astype(np.float32)
    beta = rng.standard_normal((T, Hv)).astype(np.float32)
    alpha = rng.standard_normal((T, Hv)).astype(np.float32)
    dt = (0.5 * rng.standard_normal(Hv)).astype(np.float32)
    A = (-rng.uniform(0.05, 1.0, Hv)).astype(np.float32)
    st = (0.2 * rng.standard_normal((Hv, S, S))).astype(np.float32)
    return qkv, kd, 2 * kd, beta, alpha, dt, A, st


def test_delta_step_matches_definition():
    """xjo_delta_step against the float64 definition: L2-normalised q, k of key
    head hv % Hk; S <- a S; S <- S + b (v - S k) k^T; o = qscale S q, with
    a = exp(softplus(alpha + dt) A), b = sigmoid(beta); checkpoints hold the
    state after each token."""
    T, Hk, Hv, S = 4, 2, 6, 64
    qkv, ko, vo, beta, alpha, dt, A, st = delta_step_inputs(T, Hk, Hv, S, 60)
    out, st2, ck = orc.delta_step(qkv, ko, vo, beta, alpha, dt, A, Hk, Hv, S, 1e-6, 0.125, st, ck_n=3)
    M = st.astype(np.float64)
    for t in range(T):
        r = qkv[t].astype(np.float64)
        for hv in range(Hv):
            hk = hv % Hk
            q = r[hk * S:(hk + 1) * S]
            k = r[ko + hk * S:ko + (hk + 1) * S]
            q, k = q / np.sqrt(q @ q + 1e-6), k / np.sqrt(k @ k + 1e-6)
            v = r[vo + hv * S:vo + (hv + 1) * S]
            a = np.exp(np.log1p(np.exp(alpha[t, hv] + dt[hv])) * A[hv])
            b = 1 / (1 + np.exp(-float(beta[t, hv])))
            M[hv] *= a
            M[hv] += b * np.outer(v - M[hv] @ k, k)
            assert rel_l2(out[t, hv * S:(hv + 1) * S], 0.125 * M[hv] @ q) < 1e-5
        if t < 3:
            assert rel_l2(ck[t], M) < 1e-5
    assert rel_l2(st2, M) < 1e-5


def test_delta_step_equals_recurrent_with_derived_gates():
    """The layer's step equals the standalone rule fed the same normalised q, k
    and the gates it derives."""
    T, Hk, Hv, S = 3, 4, 4, 128
    qkv, ko, vo, beta, alpha, dt, A, st = delta_step_inputs(T, Hk, Hv, S, 61)
    out, st2, _ = orc.delta_step(qkv, ko, vo, beta, alpha, dt, A, Hk, Hv, S, 1e-6, 0.0883883, st)
    nrm = lambda x: (x / np.sqrt((x.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)).astype(np.float32)
    q = nrm(qkv[:, :ko].reshape(T, Hk, S))
    k = nrm(qkv[:, ko:vo].reshape(T, Hk, S))
    v = qkv[:, vo:].reshape(T, Hv, S)
    dec = np.exp(np.log1p(np.exp(alpha + dt)) * A).astype(np.float32)
    b = (1 / (1 + np.exp(-beta))).astype(np.float32)
    o2, s2 = orc.delta_recurrent(q, k, v, dec, b, st, 0.0883883)
    assert rel_l2(out, o2.reshape(T, -1)) < 1e-5 and rel_l2(st2, s2) < 1e-5


@needs_ref
def test_mtp_stage_vs_reference_build(model_dir):
    """The MTP stage (layer n_layer behind the [embedding | hidden] prologue, head
    through shared_head_norm) of the oracle and of the reference compiled from
    source, on one model: hidden states and logits bit for bit over three calls."""
    from conftest import synth_model
    path = synth_model(model_dir, xp.TINY_MTP, "tiny_mtp")
    err = orc.C.create_string_buffer(512)
    r = orc.rlib().ref_model_load(path.encode(), err, 512)
    assert r, err.value
    hp = r.contents.hp
    n, E = hp.n_layer, hp.n_embd
    ref = orc.CpuStage(r, n, n + 1, 64, 8, True, ref=True)
    ora = orc.CpuStage(r, n, n + 1, 64, 8, True)
    assert ref.s.mtp and ora.s.mtp
    rng = np.random.default_rng(90)
    for T in (3, 1, 2):
        x = rng.standard_normal((T, 2 * E)).astype(np.float32)
        xr, xo = ref.forward(x.copy()), ora.forward(x.copy())
        hr, ho = xr.reshape(-1)[:T * E].reshape(T, E), xo.reshape(-1)[:T * E].reshape(T, E)
        assert np.array_equal(hr.view(np.uint32), ho.view(np.uint32))
        assert np.array_equal(ref.logits(hr).view(np.uint32), ora.logits(ho).view(np.uint32))
    assert ref.n_past == ora.n_past == 6
    for s in (ref, ora):
        s.destroy()
    orc.rlib().ref_model_free(r)


@needs_ref
def test_reference_mtp_driver_over_oracle_stages(model_dir):
    """The reference's own speculative driver with an MTP stage drafting 3 tokens,
    run over the reference's CPU stages and over the oracle's (fp32 KV): the same
    tokens and the same draft statistics, and the tokens of plain greedy decoding
    (speculation never changes the output); with drafts taken from that output
    every draft is accepted."""
    from conftest import synth_model
    path = synth_model(model_dir, xp.TINY_MTP, "tiny_mtp")
    m = xp.Model(path)
    L = m.hp.n_layer
    err = orc.C.create_string_buffer(512)
    r = orc.rlib().ref_model_load(path.encode(), err, 512)
    assert r, err.value
    prompt = np.random.default_rng(91).integers(0, m.hp.n_vocab, 20).astype(np.int32)
    n_gen = 24

    def run(mp, ref, k, oracle=None):
        a = orc.CpuStage(mp, 0, L // 2, 128, 8, False, ref=ref)
        b = orc.CpuStage(mp, L // 2, L, 128, 8, True, ref=ref)
        mt = orc.CpuStage(mp, L, L + 1, 128, 8, True, ref=ref) if k else None
        out = orc.ref_spec_run(mp, a.ptr, b.ptr, mt.ptr if mt else None, k, prompt, n_gen, oracle, drafts=True)
        for s in (a, b, mt):
            if s:
                s.destroy()
        return out

    plain, _, _ = run(r, True, 0)
    spec_ref, st_ref, d_ref = run(r, True, 3)
    spec_orc, st_orc, d_orc = run(m.ptr, False, 3)
    assert spec_ref.tolist() == plain.tolist() and spec_orc.tolist() == plain.tolist()
    assert st_ref == st_orc and st_ref[0] > 0
    # the drafted tokens themselves, one per call of the MTP head, in order
    assert len(d_ref) == st_ref[1] and d_ref.tolist() == d_orc.tolist()
    _, st_all, _ = run(m.ptr, False, 3, oracle=plain)
    assert st_all[1] > 0 and st_all[2] == st_all[1]
    orc.rlib().ref_model_free(r)


def end_token_model(model_dir, cfg, name, prompt, n, min_pos=6, kind="eos"):
    """(path, greedy tokens, i): cfg's model rewritten with an end token that
    first appears at index i >= min_pos of its greedy output after `prompt`
    (the oracle's fp32-KV greedy loop on the same weights), as
    tokenizer.ggml.eos_token_id (kind "eos") or as the "<|im_end|>" entry of a
    token list (kind "eot")."""
    from conftest import synth_model
    base = xp.Model(synth_model(model_dir, cfg, name))
    L = base.hp.n_layer
    st = orc.CpuStage(base.ptr, 0, L, 256, 8, True)
    toks, _ = orc.greedy([st], prompt, n)
    st.destroy()
    base.close()
    i = next(j for j in range(min_pos, n) if toks[j] not in toks[:j])
    end = int(toks[i])
    ecfg = cfg.with_(eos_id=end) if kind == "eos" else cfg.with_(eot_id=end)
    return synth_model(model_dir, ecfg, f"{name}_{kind}{end}"), toks, i


@needs_ref
@pytest.mark.parametrize("kind", ["eos", "eot"])
def test_end_tokens_in_the_reference_driver(model_dir, kind):
    """A model whose end token (eos id key or "<|im_end|>" in its token list) is
    the greedy output's token at index i: the loader reads it as the reference
    does, and the reference driver over the oracle's stages and over its own
    stops there with the tokens of plain greedy decoding up to and including it,
    with and without MTP speculation (oracle drafts carry the end token into a
    verify batch)."""
    prompt = np.random.default_rng(95).integers(0, xp.TINY_MTP.n_vocab, 14).astype(np.int32)
    path, plain, i = end_token_model(model_dir, xp.TINY_MTP, "tiny_mtp", prompt, 40, kind=kind)
    m = xp.Model(path)
    err = orc.C.create_string_buffer(512)
    r = orc.rlib().ref_model_load(path.encode(), err, 512)
    assert r, err.value
    assert bytes(r.contents.hp) == bytes(m.m.hp)
    end = int(plain[i])
    assert (m.hp.eos if kind == "eos" else m.hp.eot) == end
    L = m.hp.n_layer

    def run(mp, ref, k, oracle=None):
        a = orc.CpuStage(mp, 0, L // 2, 128, 8, False, ref=ref)
        b = orc.CpuStage(mp, L // 2, L, 128, 8, True, ref=ref)
        mt = orc.CpuStage(mp, L, L + 1, 128, 8, True, ref=ref) if k else None
        out = orc.ref_spec_run(mp, a.ptr, b.ptr, mt.ptr if mt else None, k, prompt, 40, oracle)
        for s in (a, b, mt):
            if s:
                s.destroy()
        return out

    for mp, ref in ((r, True), (m.ptr, False)):
        for k, oracle in ((0, None), (3, None), (3, plain), (4, plain)):
            out, _ = run(mp, ref, k, oracle)
            assert out.tolist() == plain[:i + 1].tolist(), (ref, k, oracle is not None)
    orc.rlib().ref_model_free(r)


@pytest.mark.parametrize("n", [25, 1000, 151936])
def test_sampler_matches_definition(n):
    rng = np.random.default_rng(n)
    for trial in range(12):
        lg = (rng.standard_normal(n) * rng.uniform(0.5, 4)).astype(np.float32)
        temp = [0.0, 0.01, 0.3, 0.7, 1.0, 1.5, 100.0][trial % 7]
        r30 = int(rng.integers(0, 1 << 30))
        assert orc.sample(lg, temp, r30) == np_sample(lg, temp, r30), (trial, temp)
    lg = rng.standard_normal(n).astype(np.float32)
    top = int(np.argmax(lg))
    assert orc.sample(lg, 1e-4, (1 << 30) - 1) == top          # a tiny temperature keeps only the maximum
    assert orc.sample(lg, 1e4, 0) == top                        # r = 0 takes the first kept token


def test_sampler_equal_values_keep_the_apps_order():
    """Equal values inside the kept set: the app's exchange sort (ios/App/XJGlue.c:270)
    is not stable, so for logits [3, 3, 5] it ranks index 1 before index 0, and a
    draw landing on the second kept value returns 1, where ranking equal values
    by index (np_sample's rule) returns 0. The device follows the app
    (test_gpu_ops.py)."""
    lg = np.array([3.0, 3.0, 5.0], np.float32)
    r30 = 1 << 29                       # r = 0.5 of the mass: past p_0 = 1, within p_1
    assert orc.sample(lg, 10.0, r30) == 1
    assert np_sample(lg, 10.0, r30) == 0
    # without equal values the two orders agree
    lg = np.array([3.0, 3.5, 5.0], np.float32)
    assert orc.sample(lg, 10.0, r30) == np_sample(lg, 10.0, r30) == 1


def test_sampler_slot_history_closed_forms():
    """The oracle's draws equal draws from the hand-derived slot orders, for
    draws landing on every kept position, at two temperatures."""
    for lg, order in slot_history_cases():
        vals = lg[order]
        for temp in (1e4, 3.0):
            for r30 in [0, 1, (1 << 30) - 1] + [int(x * (1 << 30)) for x in np.linspace(0.01, 0.99, 37)]:
                assert orc.sample(lg, temp, r30) == draw_from_order(vals, order, temp, r30), (lg[:6], temp, r30)


def test_sampler_nan_cases():
    """NaN never compares true: with NaN at index 0 the greedy pick is 0 and no
    later value enters slot 0's minimum, p_0 is NaN and the draw falls through
    to the first kept index (0); a NaN elsewhere keeps its slot and makes the
    mass NaN, so the draw returns the first kept index after the sort."""
    lg = np.full(41, 1.0, np.float32)
    lg[0] = np.nan
    lg[40] = 2.0
    for temp, r30 in ((0.0, 0), (0.7, 0), (0.7, 123456), (5.0, (1 << 30) - 1)):
        assert orc.sample(lg, temp, r30) == 0
    lg = np.full(41, 1.0, np.float32)
    lg[1] = np.nan
    lg[40] = 2.0                                  # 40 takes slot 0 (the first non-NaN minimum), sorts first
    for r30 in (0, 1 << 29, (1 << 30) - 1):
        assert orc.sample(lg, 0.7, r30) == 40
    assert orc.sample(lg, 0.0, 0) == 40


def test_sampler_callback_draws_one_number_per_token(tiny_path):
    """The reference's own driver (xj_spec_next over oracle stages, k = 0) with
    the app's sample_cb over a stream of numbers: token g is the draw from the
    logits after the prompt and tokens < g, with number g."""
    m = xp.Model(tiny_path)
    L, V = m.hp.n_layer, m.hp.n_vocab
    rng = np.random.default_rng(404)
    prompt = rng.integers(0, V, 9).astype(np.int32)
    r30 = rng.integers(0, 1 << 30, 24).astype(np.uint32)
    a = orc.CpuStage(m.ptr, 0, L, 128, 8, True, kv_f16=True)
    out, _, used = orc.ref_spec_run(m.ptr, a.ptr, None, None, 0, prompt, 24, sampler=(0.7, r30))
    a.destroy()
    assert used == 24
    s = orc.CpuStage(m.ptr, 0, L, 128, 8, True, kv_f16=True)
    x = np.stack([orc.embed(m.ptr, int(t)) for t in prompt])
    x = np.concatenate([s.forward(x[:8].copy()), s.forward(x[8:].copy())])   # the driver's chunks of max_batch
    toks = []
    for g in range(24):
        t = orc.sample(s.logits(x[-1:])[0], 0.7, int(r30[g]))
        toks.append(t)
        x = s.forward(orc.embed(m.ptr, t)[None].copy())
    s.destroy()
    assert out.tolist() == toks
    # greedy draws no number
    a = orc.CpuStage(m.ptr, 0, L, 128, 8, True, kv_f16=True)
    _, _, used = orc.ref_spec_run(m.ptr, a.ptr, None, None, 0, prompt, 8, sampler=(0.0, r30))
    a.destroy()
    assert used == 0
