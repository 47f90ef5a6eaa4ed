"""Host-side pieces of the library, no GPU: the GGUF loader against the
reference's loader, the synthetic-model writer, the quantizers and the
generator."""
import os

import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import rel_l2

FIELDS = ("file_off", "nbytes", "type", "ne0", "ne1")


def w_tuple(w):
    return tuple(getattr(w, f) for f in FIELDS)


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("cfg", ["TINY", "TINY_DRAFT", "TINY_MTP"])
def test_loader_builds_the_reference_model(model_dir, cfg):
    """xj_model_load here and the reference's xj_model_load give the same hparams,
    tensor table (offsets, sizes, types, shapes), layer pattern and fingerprint,
    and with an MTP layer the same layer n_layer and nextn tensors."""
    from conftest import synth_model
    path = synth_model(model_dir, getattr(xp, cfg), cfg.lower())
    m = xp.Model(path)
    err = orc.C.create_string_buffer(512)
    r = orc.rlib().ref_model_load(path.encode(), err, 512)
    assert r, err.value
    rm = r.contents
    assert bytes(rm.hp) == bytes(m.m.hp)
    assert rm.fingerprint == m.m.fingerprint
    for name in ("tok_embd", "output_norm", "output"):
        assert w_tuple(getattr(rm, name)) == w_tuple(getattr(m.m, name))
    for i in range(m.hp.n_layer):
        assert rm.layers[i].recurrent == m.m.layers[i].recurrent
        for f in xp._LAYER_W:
            assert w_tuple(getattr(rm.layers[i], f)) == w_tuple(getattr(m.m.layers[i], f)), (i, f)
    assert rm.has_mtp == m.m.has_mtp == bool(getattr(xp, cfg).nextn)
    if m.m.has_mtp:
        i = m.hp.n_layer
        assert rm.layers[i].recurrent == m.m.layers[i].recurrent == 0
        for f in xp._LAYER_W:
            assert w_tuple(getattr(rm.layers[i], f)) == w_tuple(getattr(m.m.layers[i], f)), ("mtp", f)
        for name in ("mtp_eh", "mtp_enorm", "mtp_hnorm", "mtp_head_norm"):
            assert w_tuple(getattr(rm, name)) == w_tuple(getattr(m.m, name)), name
    orc.rlib().ref_model_free(r)


def test_layer_pattern_and_shapes(tiny_path):
    m = xp.Model(tiny_path)
    hp = m.hp
    assert [m.m.layers[i].recurrent for i in range(hp.n_layer)] == [(i + 1) % 4 != 0 for i in range(hp.n_layer)]
    assert hp.conv_dim == 2 * hp.s_k * hp.h_k + hp.d_inner
    L0 = m.m.layers[0]
    assert (L0.ssm_qkv.ne0, L0.ssm_qkv.ne1, L0.ssm_qkv.type) == (hp.n_embd, hp.conv_dim, xp.Q4_K)
    assert (L0.ffn_down.ne0, L0.ffn_down.ne1, L0.ffn_down.type) == (hp.n_ff, hp.n_embd, xp.Q6_K)
    L3 = m.m.layers[3]
    assert L3.wv.type == xp.Q6_K and L3.wq.ne1 == 2 * hp.n_head * hp.head_dim
    assert m.m.output.type == xp.Q6_K and m.m.tok_embd.type == xp.Q4_K
    # norm weights 1 + 0.1 N, ssm_a negative
    nw = m.tensor_f32(m.m.output_norm)[0]
    assert abs(float(nw.mean()) - 1.0) < 0.05 and 0.05 < float(nw.std()) < 0.15
    assert (m.tensor_f32(L0.ssm_a) < 0).all()


def test_loader_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUF" + b"\x07\x00\x00\x00" + b"\x00" * 32)
    with pytest.raises(xp.XjError):
        xp.Model(str(p))
    p.write_bytes(b"NOPE" + b"\x00" * 40)
    with pytest.raises(xp.XjError):
        xp.Model(str(p))


def test_writer_is_deterministic(tmp_path):
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    xp.write_model(str(a), xp.TINY_DRAFT)
    xp.write_model(str(b), xp.TINY_DRAFT)
    assert a.read_bytes() == b.read_bytes()
    xp.write_model(str(b), xp.TINY_DRAFT.with_(seed=1))
    assert a.read_bytes() != b.read_bytes()


def test_generator_statistics():
    x = xp.fill_normal(1 << 20, 42, 0.02).astype(np.float64)
    assert abs(x.mean()) < 1e-4 and abs(x.std() - 0.02) < 2e-4
    assert np.array_equal(xp.fill_normal(1000, 1, 1.0), xp.fill_normal(1000, 1, 1.0))
    assert not np.array_equal(xp.fill_normal(1000, 1, 1.0), xp.fill_normal(1000, 2, 1.0))


@pytest.mark.parametrize("t,bound", [(xp.Q8_0, 0.01), (xp.Q6_K, 0.04), (xp.Q4_K, 0.12)])
def test_quantizer_round_trip(t, bound):
    """Quantize N(0,0.02) rows with the library, decode with the oracle: relative
    error within what each format's bit width allows."""
    rows, k = 64, 1024
    x = xp.fill_normal(rows * k, 3, 0.02).reshape(rows, k)
    y = orc.dequant_rows(t, xp.quantize(t, x), rows, k)
    assert rel_l2(y, x) < bound


def test_quantizer_edge_rows():
    rows, k = 4, 256
    x = np.zeros((rows, k), np.float32)
    x[1] = 1.0
    x[2, 7] = -3.0
    x[3] = np.linspace(-1, 1, k)
    for t in (xp.Q4_K, xp.Q6_K, xp.Q8_0):
        y = orc.dequant_rows(t, xp.quantize(t, x), rows, k)
        assert np.array_equal(y[0], x[0])
        assert np.isfinite(y).all()
        assert rel_l2(y[3], x[3]) < 0.1
