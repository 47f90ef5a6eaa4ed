"""End tokens on the GPU (xj_spec.c:29,139,193-194; tools/xjpipe-host.c:129-136):
the device chain's greedy decode, the draft-model speculative driver and the
native MTP driver stop at the model's end token exactly where the reference's
own driver over the same HIP stages stops, with the state of having fed only
the tokens before it. The end token is placed in the greedy output of the
same weights, once inside the first window of the decode loop and once past
it (the decode loop runs 32-step windows with a saved state when the model
has end tokens)."""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import synth_model

pytestmark = pytest.mark.gpu

N = 64


def greedy_gpu(m, prompt, n):
    st = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
    ch = xp.Chain([st])
    out = np.concatenate([ch.eval(prompt), ch.decode(n - 1)])
    ch.free()
    st.destroy()
    return out


def end_models(model_dir, cfg, name, prompt, kind):
    """[(path, plain, i)]: cfg rewritten with the end token at greedy index i,
    one i in [6, 32) and one in [40, N) when the output has a new token there."""
    base = xp.Model(synth_model(model_dir, cfg, name))
    plain = greedy_gpu(base, prompt, N)
    base.close()
    res = []
    for lo, hi in ((6, 32), (40, N)):
        i = next((j for j in range(lo, hi) if plain[j] not in plain[:j]), None)
        if i is None:
            continue
        end = int(plain[i])
        ecfg = cfg.with_(eos_id=end) if kind == "eos" else cfg.with_(eot_id=end)
        res.append((synth_model(model_dir, ecfg, f"{name}_{kind}{end}"), plain, i))
    assert res
    return res


@pytest.mark.parametrize("kind", ["eos", "eot"])
def test_chain_decode_stops_at_the_end_token(model_dir, kind):
    prompt = np.random.default_rng(96).integers(0, xp.TINY.n_vocab, 11).astype(np.int32)
    for path, plain, i in end_models(model_dir, xp.TINY, "tiny", prompt, kind):
        m = xp.Model(path)
        print(f"decode end {kind} at {i}", flush=True)
        st = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
        ch = xp.Chain([st])
        first = ch.eval(prompt)
        out = ch.decode(N)
        assert [int(first[0])] + out.tolist() == plain[:i + 1].tolist()
        assert ch.n_past == len(prompt) + i                 # the end token was not fed
        assert ch.decode(5).size == 0                        # nothing follows an end token
        # the state is that of prompt + plain[:i]: a fresh chain fed those gives
        # the same next token for a probe token
        st2 = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
        c2 = xp.Chain([st2])
        assert int(c2.eval(np.concatenate([prompt, plain[:i]]))[0]) == int(plain[i])
        z = np.array([int(plain[i - 1])], np.int32)
        (a1, l1), (a2, l2) = ch.eval(z, want_logits=True), c2.eval(z, want_logits=True)
        assert int(a1[0]) == int(a2[0])
        assert np.linalg.norm(l1 - l2) <= 1e-3 * np.linalg.norm(l2)
        if orc.ref_available():
            a, b = xp.HipStage(m, 0, 4, 256, 8, False), xp.HipStage(m, 4, m.hp.n_layer, 256, 8, True)
            ref, _ = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, None, 0, prompt, N)
            assert ref.tolist() == plain[:i + 1].tolist()
            a.destroy()
            b.destroy()
        for o in (ch, c2):
            o.free()
        st.destroy()
        st2.destroy()


@pytest.mark.parametrize("mode", ["draft", "oracle_all", "oracle_miss"])
def test_draft_model_speculation_stops_at_the_end_token(model_dir, tiny_draft_path, mode):
    prompt = np.random.default_rng(97).integers(0, xp.TINY.n_vocab, 13).astype(np.int32)
    dm = xp.Model(tiny_draft_path)
    for path, plain, i in end_models(model_dir, xp.TINY, "tiny", prompt, "eos"):
        m = xp.Model(path)
        print(f"draft spec end at {i} ({mode})", flush=True)
        t = xp.HipStage(m, 0, m.hp.n_layer, 256, 8, True)
        d = xp.HipStage(dm, 0, dm.hp.n_layer, 256, 8, True)
        tc, dc = xp.Chain([t]), xp.Chain([d])
        tc.eval(prompt)
        dc.eval(prompt)
        oracle = None if mode == "draft" else plain
        out, st = xp.spec_generate(tc, dc, 4, N, oracle=oracle, oracle_miss=3 if mode == "oracle_miss" else 0)
        assert out.tolist() == plain[:i + 1].tolist()
        assert tc.n_past == len(prompt) + i and dc.n_past == len(prompt) + i
        for o in (tc, dc):
            o.free()
        t.destroy()
        d.destroy()


@pytest.mark.parametrize("kind", ["eos", "eot"])
def test_mtp_speculation_stops_at_the_end_token(model_dir, kind):
    """Native MTP driver vs the reference's driver over the same HIP stages on a
    model with an end token: the same tokens (plain greedy up to the end
    token), the same statistics and the same drafted tokens, with real drafts
    and with oracle drafts (which carry the end token into a verify batch)."""
    prompt = np.random.default_rng(98).integers(0, xp.TINY_MTP.n_vocab, 16).astype(np.int32)
    for path, plain, i in end_models(model_dir, xp.TINY_MTP, "tiny_mtp", prompt, kind):
        m = xp.Model(path)
        L = m.hp.n_layer
        print(f"mtp end {kind} at {i}", flush=True)
        st1 = xp.HipStage(m, 0, L, 256, 8, True)
        ch = xp.Chain([st1])
        mt = xp.HipStage(m, L, L + 1, 256, 8, True)
        for k, oracle in ((3, None), (3, plain), (4, plain)):
            out, st, log = xp.spec_generate_mtp(ch, mt, k, prompt, N, oracle=oracle, draft_log=True)
            assert out.tolist() == plain[:i + 1].tolist(), (k, oracle is not None)
            if orc.ref_available():
                a, b = xp.HipStage(m, 0, L // 2, 256, 8, False), xp.HipStage(m, L // 2, L, 256, 8, True)
                m2 = xp.HipStage(m, L, L + 1, 256, 8, True)
                ref, rst, rlog = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, m2.ptr, k, prompt, N, oracle, drafts=True)
                assert ref.tolist() == out.tolist()
                assert (st.n_steps, st.n_drafted, st.n_accepted) == rst
                assert log.tolist() == rlog.tolist()
                for s in (a, b, m2):
                    s.destroy()
        ch.free()
        st1.destroy()
        mt.destroy()
