"""Pins the oracle (the CPU restatement used as the checker) before anything is
compared with it:

  * the reference's own known-answer tests (src/xiaoju-pipe/tests/unit.c:17-51:
    f16 round trip, a hand-built Q8_0 block, a hand-built Q4_K block over both
    scale paths), plus a hand-built Q6_K block from the format's definition;
  * golden vectors written by the reference compiled from source
    (tests/golden/*.npz|json, see gen_golden.py);
  * live bit-for-bit comparison with that reference build where it exists
    (oracle/_ref), including an -march=native build against the portable one;
  * invariants the mathematics fixes for the delta rule.
"""
import json
import os
import struct

import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import GOLDEN, rel_l2
from helpers import random_blocks

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
