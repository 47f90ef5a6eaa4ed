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
    """xjh_model_load here and the reference's xj_model_load give the same hparams,
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


def _truncated_copy(src, dst, nbytes):
    with open(src, "rb") as f, open(dst, "wb") as g:
        g.write(f.read(nbytes))
    return dst


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("l0,l1,io", [(0, 4, False), (4, 8, False), (2, 3, False), (0, 2, True), (6, 8, True), (0, 8, True)])
def test_layer_range_loader_matches_the_reference(tiny_path, tmp_path, l0, l1, io):
    """xjh_model_load_layers and xjh_model_ranges against the reference's own
    xj_model_load_layers and xj_model_ranges
    (xj_model.c:214-233, 308-328): the same byte ranges, the same tensor table,
    the same tensors left unmapped (data NULL), and the mapped bytes equal to
    the file's. A file cut right after the last range still loads in both,
    while the full loader rejects it; bad ranges fail in both."""
    full = xp.Model(tiny_path)
    L = full.hp.n_layer
    part = xp.Model(tiny_path, layers=(l0, l1), with_io=io)
    err = orc.C.create_string_buffer(512)
    r = orc.rlib().ref_model_load_layers(tiny_path.encode(), l0, l1, io, err, 512)
    assert r, err.value
    rm = r.contents
    assert bytes(rm.hp) == bytes(part.m.hp) and rm.fingerprint == part.m.fingerprint == full.m.fingerprint

    rr = (orc.C.c_uint64 * 1024)()
    n = orc.rlib().ref_model_ranges(r, l0, l1, io, rr, 512)
    ranges = part.ranges(l0, l1, io)
    assert ranges == [(rr[2 * i], rr[2 * i + 1]) for i in range(n)]
    assert ranges == full.ranges(l0, l1, io)
    lo, hi = ranges[0][0], ranges[-1][1]
    map_lo = lo // os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PAGE_SIZE")  # the mapping starts on a page
    assert sum(b - a for a, b in ranges) >= xp.lib().xjh_model_layer_bytes(part.ptr, l0, l1)

    def check(mine, ref, whole):
        assert w_tuple(mine) == w_tuple(ref)
        assert (mine.data is None) == (ref.data is None)
        mapped = bool(mine.nbytes) and map_lo <= mine.file_off and mine.file_off + mine.nbytes <= hi
        assert (mine.data is not None) == mapped
        if mapped:
            assert np.array_equal(part.tensor_bytes(mine), full.tensor_bytes(whole))

    for name in ("tok_embd", "output_norm", "output"):
        check(getattr(part.m, name), getattr(rm, name), getattr(full.m, name))
    for i in range(L):
        for f in xp._LAYER_W:
            check(getattr(part.m.layers[i], f), getattr(rm.layers[i], f), getattr(full.m.layers[i], f))
    for i in range(l0, l1):
        assert part.m.layers[i].ffn_down.data is not None
    orc.rlib().ref_model_free(r)
    part.close()

    cut = _truncated_copy(tiny_path, str(tmp_path / "cut.gguf"), hi)
    if hi < os.path.getsize(tiny_path):
        with pytest.raises(xp.XjError):
            xp.Model(cut)
    p2 = xp.Model(cut, layers=(l0, l1), with_io=io)
    r2 = orc.rlib().ref_model_load_layers(cut.encode(), l0, l1, io, err, 512)
    assert r2, err.value
    for i in range(l0, l1):
        assert np.array_equal(p2.tensor_bytes(p2.m.layers[i].wo if not p2.m.layers[i].recurrent else p2.m.layers[i].ssm_out),
                              full.tensor_bytes(full.m.layers[i].wo if not full.m.layers[i].recurrent else full.m.layers[i].ssm_out))
    orc.rlib().ref_model_free(r2)
    p2.close()

    for a, b in ((l1, l0), (0, L + 1), (-1, 2)):
        with pytest.raises(xp.XjError):
            xp.Model(tiny_path, layers=(a, b))
        assert not orc.rlib().ref_model_load_layers(tiny_path.encode(), a, b, io, err, 512)


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
def test_attach_mtp_matches_the_reference(model_dir, tiny_path, tmp_path):
    """xjh_model_attach_mtp against the reference's xj_model_attach_mtp
    (xj_model.c:275-300): the MTP layer and nextn tensors of a second file of
    the same model land in layers[n_layer] with the same table entries, mapped
    from that file, bytes equal to the file's own; only the header and the MTP
    span need to be present (the rest zeroed here); a file without an MTP layer
    or of another shape is refused by both."""
    from conftest import synth_model
    mtp_path = synth_model(model_dir, xp.TINY_MTP, "tiny_mtp")
    whole = xp.Model(mtp_path)
    lo, hi = orc.C.c_uint64(), orc.C.c_uint64()
    rlo, rhi = orc.C.c_uint64(), orc.C.c_uint64()
    err = orc.C.create_string_buffer(512)
    assert xp.lib().xjh_model_mtp_range(mtp_path.encode(), orc.C.byref(lo), orc.C.byref(hi), err, 512) == 0, err.value
    assert orc.rlib().ref_model_mtp_range(mtp_path.encode(), orc.C.byref(rlo), orc.C.byref(rhi), err, 512) == 0
    assert (lo.value, hi.value) == (rlo.value, rhi.value) and lo.value < hi.value

    # a copy holding only the header and the MTP span
    raw = bytearray(open(mtp_path, "rb").read())
    first = min(t.file_off for t in (whole.m.tok_embd, whole.m.output_norm))
    holes = bytearray(len(raw))
    holes[:first] = raw[:first]
    holes[lo.value:hi.value] = raw[lo.value:hi.value]
    sparse = tmp_path / "mtp_only.gguf"
    sparse.write_bytes(bytes(holes))

    for src in (mtp_path, str(sparse)):
        m = xp.Model(tiny_path)
        assert not m.m.has_mtp
        m.attach_mtp(src)
        r = orc.rlib().ref_model_load(tiny_path.encode(), err, 512)
        assert r, err.value
        assert orc.rlib().ref_model_attach_mtp(r, src.encode(), err, 512) == 0, err.value
        rm = r.contents
        assert m.m.has_mtp and rm.has_mtp
        i = m.hp.n_layer
        assert bytes(rm.hp) == bytes(m.m.hp) and rm.fingerprint == m.m.fingerprint
        for f in xp._LAYER_W:
            mine, ref = getattr(m.m.layers[i], f), getattr(rm.layers[i], f)
            assert w_tuple(mine) == w_tuple(ref), f
            assert (mine.data is None) == (ref.data is None) == (mine.nbytes == 0), f
            if mine.nbytes:
                assert np.array_equal(m.tensor_bytes(mine), whole.tensor_bytes(getattr(whole.m.layers[i], f))), f
        for name in ("mtp_eh", "mtp_enorm", "mtp_hnorm", "mtp_head_norm"):
            mine = getattr(m.m, name)
            assert w_tuple(mine) == w_tuple(getattr(rm, name)) == w_tuple(getattr(whole.m, name)), name
            assert np.array_equal(m.tensor_bytes(mine), whole.tensor_bytes(getattr(whole.m, name))), name
        m.attach_mtp(src)                      # already attached: a no-op in both
        assert orc.rlib().ref_model_attach_mtp(r, src.encode(), err, 512) == 0
        orc.rlib().ref_model_free(r)
        m.close()

    draft = synth_model(model_dir, xp.TINY_DRAFT, "tiny_draft")
    for bad in (tiny_path, draft):             # no MTP layer / another model's shape
        m = xp.Model(tiny_path)
        with pytest.raises(xp.XjError):
            m.attach_mtp(bad)
        r = orc.rlib().ref_model_load(tiny_path.encode(), err, 512)
        assert orc.rlib().ref_model_attach_mtp(r, bad.encode(), err, 512) != 0
        orc.rlib().ref_model_free(r)
        m.close()


def _utf8_text(rng, n_chars):
    """Random text of 1- to 4-byte UTF-8 characters."""
    cps = []
    for _ in range(n_chars):
        w = rng.integers(0, 4)
        cps.append(chr(int(rng.integers(0x20, 0x7F) if w == 0 else rng.integers(0xA0, 0x800) if w == 1 else
                           rng.integers(0x4E00, 0x9FFF) if w == 2 else rng.integers(0x1F300, 0x1FAFF))))
    return "".join(cps).encode("utf-8")


def _pieces(rng, data, max_len):
    out, i = [], 0
    while i < len(data):
        n = int(rng.integers(0, max_len + 1))
        out.append(data[i:i + n])
        i += n
    return out


def test_utf8_stream_known_splits():
    """Characters split across pieces reach the callback whole
    (ios/App/XJGlue.c:285-305): the 3-byte CJK characters and a 4-byte emoji
    held back until their last byte arrives."""
    s = xp.Utf8Stream()
    seq = [(b"\xe4", b""), (b"\xbd\xa0\xe5", b"\xe4\xbd\xa0"), (b"\xa5\xbd", b"\xe5\xa5\xbd"), (b"", b""),
           (b"ab", b"ab"), (b"\xf0\x9f", b""), (b"\x98", b""), (b"\x80!", b"\xf0\x9f\x98\x80!")]
    for piece, want in seq:
        assert s.emit(piece) == (want, 0), piece
    assert s.pending == b""


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_utf8_stream_matches_the_app(seed):
    """Chunk by chunk equal to the oracle's restatement of the app's emit on
    random text split at random byte positions, pieces of up to 300 bytes
    (the app keeps the first 256 of a piece), and on random bytes that are
    not UTF-8 (stray continuation bytes, cut sequences)."""
    rng = np.random.default_rng(seed)
    streams = [_utf8_text(rng, 400), bytes(rng.integers(0, 256, 900, dtype=np.uint8)),
               bytes(rng.choice(np.array([0x41, 0x80, 0xBF, 0xC3, 0xE4, 0xF0], np.uint8), 600))]
    for data in streams:
        s, o = xp.Utf8Stream(), orc.Utf8Emit()
        for piece in _pieces(rng, data, 300):
            got, stop = s.emit(piece)
            assert stop == 0
            assert got == o.emit(piece)


def test_utf8_stream_round_trip():
    """With pieces of at most 256 bytes nothing is dropped: the chunks and the
    held-back bytes concatenate to the input, and every chunk is whole UTF-8."""
    rng = np.random.default_rng(9)
    data = _utf8_text(rng, 2000)
    s = xp.Utf8Stream()
    got = b""
    for piece in _pieces(rng, data, 256):
        chunk, _ = s.emit(piece)
        chunk.decode("utf-8")          # raises on a split character
        got += chunk
    assert got + s.pending == data
    assert s.pending == b""            # the text ends with a whole character


def test_utf8_stream_stop():
    """The callback's nonzero return is xjh_utf8_emit's (the app stops its token loop on it)."""
    s = xp.Utf8Stream(stop_after=2)
    assert s.emit(b"a") == (b"a", 0)
    assert s.emit(b"\xe4\xbd") == (b"", 0)     # nothing complete: the callback is not called
    assert s.emit(b"\xa0b") == (b"\xe4\xbd\xa0b", 1)
