"""The MTP stage on the GPU (the range [n_layer, n_layer + 1) of a model with an
MTP layer: [embedding | hidden] rows, each half RMS-normalised with its own
weights, eh_proj back to n_embd, the MTP layer, and a head through
shared_head_norm; xj_cpu.c:253-261, :287) against the oracle's MTP stage (fp16
KV cache, the same inputs): hidden states and logits within 1e-3 relative L2,
the same greedy token per row, across calls, a rollback and a reset.
"""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import rel_l2, synth_model

pytestmark = pytest.mark.gpu


def mtp_rows(m, rng, T):
    """T rows of [embedding of a random token | a hidden-like vector]."""
    E = m.hp.n_embd
    toks = rng.integers(0, m.hp.n_vocab, T)
    x = np.empty((T, 2 * E), np.float32)
    for t in range(T):
        x[t, :E] = orc.embed(m.ptr, int(toks[t]))
        x[t, E:] = rng.standard_normal(E).astype(np.float32) * 2
    return x


def run_pair(m, calls, seed):
    n, E = m.hp.n_layer, m.hp.n_embd
    g = xp.HipStage(m, n, n + 1, 256, 8, True)
    c = orc.CpuStage(m.ptr, n, n + 1, 256, 8, True, kv_f16=True)
    assert g.s.mtp and c.s.mtp
    rng = np.random.default_rng(seed)
    for T in calls:
        if T == "rollback":
            g.rollback(g.n_past - 2)
            c.rollback(c.n_past - 2)
            continue
        if T == "reset":
            g.reset()
            c.reset()
            continue
        x = mtp_rows(m, rng, T)
        xg, xc = g.forward(x.copy()), c.forward(x.copy())
        hg, hc = xg.reshape(-1)[:T * E].reshape(T, E), xc.reshape(-1)[:T * E].reshape(T, E)
        assert rel_l2(hg, hc) < 1e-3, T
        lg, lc = g.logits(hg), c.logits(hc)
        assert rel_l2(lg, lc) < 1e-3, T
        assert np.array_equal(np.argmax(lg, 1), np.argmax(lc, 1))
        assert g.n_past == c.n_past
    g.destroy()
    c.destroy()


def test_mtp_stage_matches_oracle(model_dir):
    m = xp.Model(synth_model(model_dir, xp.TINY_MTP, "tiny_mtp"))
    assert m.m.has_mtp
    run_pair(m, [3, 1, 2, "rollback", 1, 5, "reset", 4], 1)


def test_mtp_stage_0_8b_shape():
    m = xp.Model(xp.cached_model(xp.CONFIG_0_8B_MTP, "synth08b_mtp"))
    run_pair(m, [5, 1, 1, "rollback", 3], 2)


def test_main_stages_of_an_mtp_model_ignore_the_mtp_layer(model_dir):
    """The main layers of TINY_MTP are those of TINY: the same hidden states."""
    a = xp.Model(synth_model(model_dir, xp.TINY_MTP, "tiny_mtp"))
    b = xp.Model(synth_model(model_dir, xp.TINY, "tiny"))
    L = a.hp.n_layer
    toks = np.random.default_rng(3).integers(0, a.hp.n_vocab, 6)
    x = np.stack([orc.embed(a.ptr, int(t)) for t in toks]).astype(np.float32)
    ga, gb = xp.HipStage(a, 0, L, 64, 8, True), xp.HipStage(b, 0, L, 64, 8, True)
    ya, yb = ga.forward(x.copy()), gb.forward(x.copy())
    assert np.array_equal(ya, yb)
    ga.destroy()
    gb.destroy()


def _driver_run(mp, make, L, k, prompt, n_gen, oracle=None):
    a, b = make(0, L // 2, False), make(L // 2, L, True)
    mt = make(L, L + 1, True) if k else None
    out = orc.ref_spec_run(mp, a.ptr, b.ptr, mt.ptr if mt else None, k, prompt, n_gen, oracle)
    for s in (a, b, mt):
        if s:
            s.destroy()
    return out


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("shape", ["tiny", "0_8b"])
def test_reference_mtp_driver_over_hip_stages(model_dir, shape):
    """The reference's own pipeline and speculative driver (MTP drafting 3 tokens
    per step) run unchanged over HIP stages through the xj_stage vtable: the
    tokens equal plain greedy decoding on the same stages and the oracle's
    (fp16 KV) greedy tokens; with drafts from that output every draft is accepted."""
    if shape == "tiny":
        m, n_gen = xp.Model(synth_model(model_dir, xp.TINY_MTP, "tiny_mtp")), 24
    else:
        m, n_gen = xp.Model(xp.cached_model(xp.CONFIG_0_8B_MTP, "synth08b_mtp")), 32
    L = m.hp.n_layer
    prompt = np.random.default_rng(92).integers(0, m.hp.n_vocab, 20).astype(np.int32)
    hip = lambda l0, l1, head: xp.HipStage(m, l0, l1, 128, 8, head)
    cpu = lambda l0, l1, head: orc.CpuStage(m.ptr, l0, l1, 128, 8, head, kv_f16=True)
    print(f"mtp driver {shape}", flush=True)
    plain, _ = _driver_run(m.ptr, hip, L, 0, prompt, n_gen)
    spec, st = _driver_run(m.ptr, hip, L, 3, prompt, n_gen)
    want, _ = _driver_run(m.ptr, cpu, L, 0, prompt, n_gen)
    print(f"{shape}: verify steps {st[0]}, drafted {st[1]}, accepted {st[2]}")
    assert spec.tolist() == plain.tolist() == want.tolist()
    _, st_all = _driver_run(m.ptr, hip, L, 3, prompt, n_gen, oracle=plain)
    assert st_all[1] > 0 and st_all[2] == st_all[1]


@pytest.mark.parametrize("shape", ["tiny", "0_8b"])
def test_native_mtp_driver(model_dir, shape):
    """xjh_spec_generate_mtp over the device chain: the tokens of plain greedy
    decoding; the same draft statistics as the reference's driver over the same
    HIP stages (where that build exists); every draft accepted in the driver's
    test mode, and one in four perturbed drafts rejected."""
    if shape == "tiny":
        m, n_gen = xp.Model(synth_model(model_dir, xp.TINY_MTP, "tiny_mtp")), 24
    else:
        m, n_gen = xp.Model(xp.cached_model(xp.CONFIG_0_8B_MTP, "synth08b_mtp")), 32
    L = m.hp.n_layer
    prompt = np.random.default_rng(93).integers(0, m.hp.n_vocab, 20).astype(np.int32)
    print(f"native mtp driver {shape}", flush=True)
    st1 = xp.HipStage(m, 0, L, 128, 8, True)
    ch = xp.Chain([st1])
    plain = np.concatenate([ch.eval(prompt), ch.decode(n_gen - 1)])
    mt = xp.HipStage(m, L, L + 1, 128, 8, True)
    out, st, log = xp.spec_generate_mtp(ch, mt, 3, prompt, n_gen, draft_log=True)
    print(f"{shape}: steps {st.n_steps} drafted {st.n_drafted} accepted {st.n_accepted}")
    assert out.tolist() == plain.tolist()
    assert len(log) == st.n_drafted
    if orc.ref_available():
        # the reference driver over the same HIP stages proposes the same drafts
        # (hidden rows through output_norm, MTP outputs through shared_head_norm,
        # both as x * (sc * w)), so its statistics are the native driver's
        hip = lambda l0, l1, head: xp.HipStage(m, l0, l1, 128, 8, head)
        a, b, m2 = hip(0, L // 2, False), hip(L // 2, L, True), hip(L, L + 1, True)
        ref_out, ref_st, ref_log = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, m2.ptr, 3, prompt, n_gen, drafts=True)
        for s in (a, b, m2):
            s.destroy()
        assert ref_out.tolist() == plain.tolist()
        assert (st.n_steps, st.n_drafted, st.n_accepted) == ref_st
        assert log.tolist() == ref_log.tolist()
    out, st = xp.spec_generate_mtp(ch, mt, 3, prompt, n_gen, oracle=plain)
    assert out.tolist() == plain.tolist() and st.n_accepted == st.n_drafted > 0
    out, st = xp.spec_generate_mtp(ch, mt, 4, prompt, n_gen, oracle=plain, oracle_miss=4)
    assert out.tolist() == plain.tolist() and 0 < st.n_accepted < st.n_drafted
    ch.free()
    st1.destroy()
    mt.destroy()
