"""Greedy token identity at the real model shapes, against the committed
oracle runs (tests/golden/greedy_*.json, fp16 KV like the GPU; the fixtures
also hold the reference's own fp32-KV run, whose agreement is reported).

  * 0.8B shape: 512-token prompt, 256 greedy steps, one stage
  * 4B shape:   1024-token prompt, 512 greedy steps, layers 0-15 and 16-31 as two
                stages run in sequence on one GPU (the reference's two-device split)
  * 4B with the 0.8B model drafting 4 tokens per step: the speculative output
    equals plain greedy decoding
"""
import json
import os

import numpy as np
import pytest

import xjpipe as xp
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def fixture(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} not generated")
    return json.load(open(path))


def check_model(path, rec):
    assert os.path.getsize(path) == rec["bytes"], "synthetic model drifted from the fixture"


def first_divergence(a, b):
    return next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), None)


@pytest.mark.parametrize("max_batch", [8, 64])
def test_0_8b_greedy_256_steps(max_batch):
    """max_batch 8 (the recorded runs' chunking: prefill on the GEMV) and 64
    (prefill chunks on the matrix-core GEMM and the chunked delta rule); the
    reference's tokens do not depend on the chunking."""
    rec = fixture("greedy_0_8b.json")
    path = xp.cached_model(xp.CONFIG_0_8B, "synth08b")
    check_model(path, rec)
    m = xp.Model(path)
    prompt = np.random.default_rng(rec["prompt_seed"]).integers(0, m.hp.n_vocab, rec["n_prompt"]).astype(np.int32)
    st = xp.HipStage(m, 0, m.hp.n_layer, rec["n_ctx"], max_batch, True)
    ch = xp.Chain([st])
    toks = np.concatenate([ch.eval(prompt), ch.decode(rec["n_gen"] - 1)]).tolist()
    want = rec["oracle_kvf16"]["tokens"]
    div = first_divergence(toks, want)
    print(f"0.8B: first divergence from the fp16-KV oracle: {div}; "
          f"from the reference (fp32 KV): {first_divergence(toks, rec['ref_kvf32']['tokens'])}")
    assert toks == want, f"diverges at step {div} (oracle top-2 margin there {rec['oracle_kvf16']['margins'][div]})"
    ch.free()
    st.destroy()


@pytest.mark.parametrize("max_batch", [8, 64])
def test_4b_two_stage_greedy_512_steps(max_batch):
    """As the 0.8B test: prefill chunks of 8 (GEMV) and of 64 (matrix-core GEMM,
    chunked delta rule)."""
    rec = fixture("greedy_4b.json")
    path = xp.cached_model(xp.CONFIG_4B, "synth4b")
    check_model(path, rec)
    m = xp.Model(path)
    prompt = np.random.default_rng(rec["prompt_seed"]).integers(0, m.hp.n_vocab, rec["n_prompt"]).astype(np.int32)
    a = xp.HipStage(m, 0, 16, rec["n_ctx"], max_batch, False)
    b = xp.HipStage(m, 16, 32, rec["n_ctx"], max_batch, True)
    ch = xp.Chain([a, b])
    toks = np.concatenate([ch.eval(prompt), ch.decode(rec["n_gen"] - 1)]).tolist()
    want = rec["oracle_kvf16"]["tokens"]
    div = first_divergence(toks, want)
    if "ref_kvf32_split16" in rec:
        print(f"4B: first divergence from the reference (fp32 KV): {first_divergence(toks, rec['ref_kvf32_split16']['tokens'])}")
    assert toks == want, f"diverges at step {div} (oracle top-2 margin there {rec['oracle_kvf16']['margins'][div]})"
    ch.free()
    a.destroy()
    b.destroy()


@pytest.mark.parametrize("mode", ["draft_0_8b", "oracle_drafts", "oracle_miss"])
def test_4b_speculative_with_0_8b_draft(mode):
    """Config 5 in full: the 4B shape split 0-15 | 16-31 on one GPU, the 0.8B
    model drafting 4 tokens per step, 1024-token prompt, 512 tokens; the
    output equals the committed greedy tokens of the 4B shape (the oracle's
    fp16-KV run, itself equal to the reference's) with the draft's own
    proposals, with proposals taken from that output, and with one in four of
    those perturbed."""
    rec = fixture("greedy_4b.json")
    path = xp.cached_model(xp.CONFIG_4B, "synth4b")
    check_model(path, rec)
    dpath = xp.cached_model(xp.CONFIG_0_8B, "synth08b")
    m, dm = xp.Model(path), xp.Model(dpath)
    prompt = np.random.default_rng(rec["prompt_seed"]).integers(0, m.hp.n_vocab, rec["n_prompt"]).astype(np.int32)
    n_gen, want = rec["n_gen"], rec["oracle_kvf16"]["tokens"]
    a = xp.HipStage(m, 0, 16, rec["n_ctx"], rec["max_batch"], False)
    b = xp.HipStage(m, 16, 32, rec["n_ctx"], rec["max_batch"], True)
    d = xp.HipStage(dm, 0, dm.hp.n_layer, rec["n_ctx"], rec["max_batch"], True)
    tc, dc = xp.Chain([a, b]), xp.Chain([d])
    tc.eval(prompt)
    dc.eval(prompt)
    oracle = None if mode == "draft_0_8b" else np.array(want, np.int32)
    out, stats = xp.spec_generate(tc, dc, 4, n_gen, oracle=oracle, oracle_miss=4 if mode == "oracle_miss" else 0)
    print(f"{mode}: steps {stats.n_steps}, drafted {stats.n_drafted}, accepted {stats.n_accepted}, "
          f"{n_gen / (stats.t_total_ms / 1e3):.1f} tok/s")
    assert out.tolist() == want, f"diverges at {first_divergence(out.tolist(), want)}"
    if mode == "oracle_drafts":
        assert stats.n_accepted == stats.n_drafted
    for o in (tc, dc):
        o.free()
    for s in (a, b, d):
        s.destroy()


def test_4b_verify_pass_equals_single_steps():
    """At the 4B shape a 4- and a 5-token verification pass (the widths whose
    GEMVs pair the rows of a team) give, bit for bit, the logits of feeding
    the same tokens one at a time."""
    path = xp.cached_model(xp.CONFIG_4B, "synth4b")
    m = xp.Model(path)
    L = m.hp.n_layer
    rng = np.random.default_rng(77)
    prompt = rng.integers(0, m.hp.n_vocab, 96).astype(np.int32)
    cand = rng.integers(0, m.hp.n_vocab, 5).astype(np.int32)
    stages = [xp.HipStage(m, 0, L, 128, 8, True) for _ in range(3)]
    chains = [xp.Chain([s]) for s in stages]
    for c in chains:
        c.eval(prompt)
    lg1 = np.stack([chains[0].eval(cand[i:i + 1], nlog=1, want_logits=True)[1][0] for i in range(5)])
    for c, T in ((chains[1], 4), (chains[2], 5)):
        _, lgT = c.eval(cand[:T], nlog=T, keep=True, want_logits=True)
        assert np.array_equal(lgT.view(np.uint32), lg1[:T].view(np.uint32)), T
    for c in chains:
        c.free()
    for s in stages:
        s.destroy()
