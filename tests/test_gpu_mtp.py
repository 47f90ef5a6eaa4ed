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
