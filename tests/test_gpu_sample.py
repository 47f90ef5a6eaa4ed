"""The app's sampler on the device-resident path (ios/App/XJGlue.c:248-282,
the draws of xj_spec_next, core/xj_spec.c:135,185).

With the chain's sampler on, every token the chain produces is the app's
top-k 40 / top-p 0.95 draw from its logits row with the next number of a
given stream (standing in for arc4random_uniform(1 << 30)). The references:

  * the reference's own driver (xj_pipeline + xj_spec_next, compiled from its
    sources) over HIP stages behind the xj_stage vtable, with the app's
    sample_cb (the oracle's restatement) drawing from the same numbers - the
    drop-in path the app would run;
  * a host loop over a HIP stage: logits to the host, the oracle's sampler.

Both see the logits the chain's kernels compute, so the tokens must be equal,
not just close. Speculative decoding with sampled acceptance must give the
tokens of plain sampled decoding with the same numbers, and the MTP driver the
reference driver's tokens, statistics and drafts.
"""
import os

import numpy as np
import pytest

import oracle as orc
import xjpipe as xp

pytestmark = pytest.mark.gpu

N = 40


def numbers(seed, n):
    return np.random.default_rng(seed).integers(0, 1 << 30, n).astype(np.uint32)


def sampled_chain(m, prompt, n, temp, r30, split=None):
    L = m.hp.n_layer
    if split:
        st = [xp.HipStage(m, 0, split, 256, 8, False), xp.HipStage(m, split, L, 256, 8, True)]
    else:
        st = [xp.HipStage(m, 0, L, 256, 8, True)]
    ch = xp.Chain(st)
    ch.set_sampler(temp, r30)
    ch.eval(prompt)
    out = np.concatenate([[ch.last_token], ch.decode(n - 1)]).astype(np.int32)
    used = ch.sampler_used
    ch.free()
    for s in st:
        s.destroy()
    return out, used


def host_loop(m, prompt, n, temp, r30):
    """A HIP stage behind the vtable, logits to the host, the oracle's sampler
    with number g for token g."""
    st = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
    x = np.stack([orc.embed(m.ptr, int(t)) for t in prompt])
    for i in range(0, len(x), 8):
        x[i:i + 8] = st.forward(x[i:i + 8].copy())
    toks, g = [], 0
    last = x[-1:]
    for _ in range(n):
        t = orc.sample(st.logits(last)[0], temp, int(r30[g]) if temp > 0 else 0)
        g += temp > 0
        toks.append(t)
        last = st.forward(orc.embed(m.ptr, t)[None].copy())
    st.destroy()
    return np.array(toks, np.int32)


@pytest.mark.parametrize("temp", [0.0, 0.7, 1.5])
def test_chain_sampled_decode_matches_the_apps_loop(tiny_path, temp):
    m = xp.Model(tiny_path)
    prompt = np.random.default_rng(500).integers(0, m.hp.n_vocab, 11).astype(np.int32)
    r30 = numbers(501, N + 8)
    print(f"sampled chain temp {temp}", flush=True)
    out, used = sampled_chain(m, prompt, N, temp, r30)
    assert used == (N if temp > 0 else 0)
    assert out.tolist() == host_loop(m, prompt, N, temp, r30).tolist()
    # two stages, and the decode steps launched one by one instead of the graph
    assert sampled_chain(m, prompt, N, temp, r30, split=3)[0].tolist() == out.tolist()
    os.environ["XJ_DECODE_GRAPH"] = "0"
    try:
        assert sampled_chain(m, prompt, N, temp, r30)[0].tolist() == out.tolist()
    finally:
        del os.environ["XJ_DECODE_GRAPH"]
    if temp > 0:
        assert len(set(out.tolist())) > N // 4         # a real draw, not the argmax over and over
    if orc.ref_available():
        L = m.hp.n_layer
        a, b = xp.HipStage(m, 0, 4, 256, 8, False), xp.HipStage(m, 4, L, 256, 8, True)
        ref, _, rused = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, None, 0, prompt, N, sampler=(temp, r30))
        a.destroy()
        b.destroy()
        assert ref.tolist() == out.tolist()
        assert rused == used


def test_sampler_numbers_run_out(tiny_path):
    m = xp.Model(tiny_path)
    prompt = np.arange(5, dtype=np.int32)
    st = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
    ch = xp.Chain([st])
    ch.set_sampler(0.7, numbers(7, 6))
    ch.eval(prompt)
    assert ch.sampler_used == 1
    with pytest.raises(xp.XjError):
        ch.decode(6)                                   # five numbers left
    assert ch.decode(5).size == 5 and ch.sampler_used == 6
    with pytest.raises(xp.XjError):
        ch.set_sampler(0.7, np.array([1 << 30], np.uint32))   # not below 2^30
    ch.free()
    st.destroy()


@pytest.mark.parametrize("mode", ["draft", "oracle_all", "oracle_miss"])
def test_draft_model_speculation_sampled(tiny_path, tiny_draft_path, mode):
    """Sampled acceptance: the target's draw at row i (number used + i) must
    equal draft i + 1. The output is plain sampled decoding's, whatever the
    drafts; the driver ends holding the next token, drawn (N + 1 numbers) and
    not fed, as its greedy form holds the next argmax."""
    m, dm = xp.Model(tiny_path), xp.Model(tiny_draft_path)
    prompt = np.random.default_rng(502).integers(0, m.hp.n_vocab, 12).astype(np.int32)
    r30 = numbers(503, N + 8)
    plain, used = sampled_chain(m, prompt, N + 1, 0.8, r30)
    t = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
    d = xp.HipStage(dm, 0, dm.hp.n_layer, 256, 8, True)
    tc, dc = xp.Chain([t]), xp.Chain([d])
    tc.set_sampler(0.8, r30)
    tc.eval(prompt)
    dc.eval(prompt)
    oracle = None if mode == "draft" else plain
    out, st = xp.spec_generate(tc, dc, 4, N, oracle=oracle, oracle_miss=3 if mode == "oracle_miss" else 0)
    print(f"draft spec sampled ({mode}): accepted {st.n_accepted} of {st.n_drafted}", flush=True)
    assert out.tolist() == plain[:N].tolist()
    assert tc.sampler_used == used and tc.last_token == plain[N]
    if mode == "oracle_all":
        assert st.n_accepted == st.n_drafted
    for o in (tc, dc):
        o.free()
    t.destroy()
    d.destroy()


def test_mtp_speculation_sampled(model_dir):
    """The native MTP driver with the target's sampler: plain sampled decoding's
    tokens; with the reference's driver over the same HIP stages and the app's
    sample_cb on the same numbers, the same tokens, statistics and drafts. When
    the last verification accepted every draft, the driver also holds the next
    token, drawn with number N."""
    from conftest import synth_model
    m = xp.Model(synth_model(model_dir, xp.TINY_MTP, "tiny_mtp"))
    L = m.hp.n_layer
    prompt = np.random.default_rng(504).integers(0, m.hp.n_vocab, 16).astype(np.int32)
    r30 = numbers(505, N + 8)
    plain, _ = sampled_chain(m, prompt, N + 1, 0.7, r30)
    st1 = xp.HipStage(m, 0, L, 256, 8, True)
    ch = xp.Chain([st1])
    mt = xp.HipStage(m, L, L + 1, 256, 8, True)
    for k, oracle in ((3, None), (3, plain[:N]), (4, plain[:N])):
        ch.set_sampler(0.7, r30)
        out, st, log = xp.spec_generate_mtp(ch, mt, k, prompt, N, oracle=oracle, draft_log=True)
        print(f"mtp sampled k={k} oracle={oracle is not None}: accepted {st.n_accepted} of {st.n_drafted}", flush=True)
        assert out.tolist() == plain[:N].tolist(), (k, oracle is not None)
        assert ch.sampler_used == N or (ch.sampler_used == N + 1 and ch.last_token == plain[N])
        if orc.ref_available():
            a, b = xp.HipStage(m, 0, L // 2, 256, 8, False), xp.HipStage(m, L // 2, L, 256, 8, True)
            m2 = xp.HipStage(m, L, L + 1, 256, 8, True)
            ref, rst, rlog, _ = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, m2.ptr, k, prompt, N, oracle, drafts=True,
                                                 sampler=(0.7, r30))
            assert ref.tolist() == out.tolist()
            assert (st.n_steps, st.n_drafted, st.n_accepted) == rst
            assert log.tolist() == rlog.tolist()
            for s in (a, b, m2):
                s.destroy()
    ch.free()
    st1.destroy()
    mt.destroy()


def test_0_8b_sampled_decode_matches_the_apps_loop():
    """The 0.8B shape (config 4 model), 512-token prompt, 64 tokens at the app's
    default temperature 0.7: the device chain's draws equal the host loop's
    (logits of a HIP stage, the oracle's sampler) token for token."""
    m = xp.Model(xp.cached_model(xp.CONFIG_0_8B, "synth08b"))
    prompt = np.random.default_rng(506).integers(0, m.hp.n_vocab, 512).astype(np.int32)
    r30 = numbers(507, 72)
    n = 64
    st = xp.HipStage(m, 0, m.hp.n_layer, 1024, 8, True)
    ch = xp.Chain([st])
    ch.set_sampler(0.7, r30)
    ch.eval(prompt)
    out = np.concatenate([[ch.last_token], ch.decode(n - 1)]).tolist()
    ch.free()
    st.destroy()
    st = xp.HipStage(m, 0, m.hp.n_layer, 1024, 8, True)
    x = np.stack([orc.embed(m.ptr, int(t)) for t in prompt])
    for i in range(0, len(x), 8):
        x[i:i + 8] = st.forward(x[i:i + 8].copy())
    last, toks = x[-1:], []
    for g in range(n):
        t = orc.sample(st.logits(last)[0], 0.7, int(r30[g]))
        toks.append(t)
        last = st.forward(orc.embed(m.ptr, t)[None].copy())
    st.destroy()
    assert out == toks
