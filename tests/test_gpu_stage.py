"""The HIP stage behind the xj_stage vtable and the device chain, against the
oracle's CPU stage with an fp16 KV cache, on identical seeded inputs.

Mirrors the reference's own GPU-vs-CPU check (src/xiaoju-pipe/tools/xjpipe-check.c:61-109):
prefill 12 tokens then 3 single tokens, head top-1, keep/rollback equal to
never having computed the rolled-back tokens; plus greedy token identity.
"""
import numpy as np
import pytest

import oracle as orc
import xjpipe as xp
from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tiny_path):
    return xp.Model(tiny_path)


def embed(m, toks):
    return np.stack([orc.embed(m.ptr, int(t)) for t in toks]).astype(np.float32)


def prompt_ids(m, n, seed):
    return np.random.default_rng(seed).integers(0, m.hp.n_vocab, n).astype(np.int32)


def test_forward_and_head_match_oracle(tiny):
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 15, 1)
    g = xp.HipStage(m, 0, L, 128, 16, True)
    c = orc.CpuStage(m.ptr, 0, L, 128, 16, True, kv_f16=True)
    pos = 0
    for T in (12, 1, 1, 1):
        x = embed(m, toks[pos:pos + T])
        xg, xc = g.forward(x.copy()), c.forward(x.copy())
        assert rel_l2(xg, xc) < 1e-3, T
        pos += T
    assert g.n_past == c.n_past == 15
    lg, lc = g.logits(xg[-1:]), c.logits(xc[-1:])
    assert rel_l2(lg, lc) < 1e-3
    assert int(np.argmax(lg)) == int(np.argmax(lc))
    g.destroy()
    c.destroy()


def test_two_stages_equal_one(tiny):
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 10, 2)
    one = xp.HipStage(m, 0, L, 64, 8, True)
    a, b = xp.HipStage(m, 0, 4, 64, 8, False), xp.HipStage(m, 4, L, 64, 8, True)
    for T in (8, 2):
        x = embed(m, toks[:T]) if T == 8 else embed(m, toks[8:10])
        x1 = one.forward(x.copy())
        x2 = b.forward(a.forward(x.copy()))
        assert np.array_equal(x1, x2)
    for s in (one, a, b):
        s.destroy()


def test_keep_rollback_equals_never_computed(tiny):
    """forward 6, verify 4 with keep, roll back to 8, forward 2 others == forward the 10 kept tokens."""
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 14, 3)
    g = xp.HipStage(m, 0, L, 64, 8, True)
    g.forward(embed(m, toks[:6]))
    g.set_keep(4)
    g.forward(embed(m, toks[6:10]))
    assert g.s.ck_start == 6 and g.s.ck_T == 4
    g.rollback(8)
    assert g.n_past == 8
    x_after = g.forward(embed(m, toks[12:14]))
    ref = xp.HipStage(m, 0, L, 64, 16, True)
    seq = np.concatenate([toks[:8], toks[12:14]])
    xr = ref.forward(embed(m, seq))
    assert rel_l2(x_after, xr[8:]) < 1e-6
    c = orc.CpuStage(m.ptr, 0, L, 64, 16, True, kv_f16=True)
    xc = c.forward(embed(m, seq))
    assert rel_l2(x_after, xc[8:]) < 1e-3
    for s in (g, ref, c):
        s.destroy()


def test_rollback_rules(tiny):
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 8, 4)
    g = xp.HipStage(m, 0, L, 64, 8, True)
    g.forward(embed(m, toks[:4]))
    with pytest.raises(xp.XjError):       # no checkpoint window
        g.rollback(2)
    g.rollback(4)                          # unchanged position is a no-op
    g.set_keep(3)
    g.forward(embed(m, toks[4:7]))
    with pytest.raises(xp.XjError):       # outside [ck_start+1, ck_start+ck_T-1]
        g.rollback(4)
    g.rollback(6)
    # attention-only stage (layer 3 is full attention) truncates freely
    att = xp.HipStage(m, 3, 4, 64, 8, False)
    att.forward(embed(m, toks[:5]))
    att.rollback(2)
    assert att.n_past == 2
    with pytest.raises(xp.XjError):
        att.rollback(3)
    with pytest.raises(xp.XjError):       # T > max_batch
        g.forward(embed(m, np.zeros(9, np.int32)))
    g.destroy()
    att.destroy()


def test_reset_and_context_limit(tiny):
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 8, 5)
    g = xp.HipStage(m, 0, L, 8, 8, True)
    x1 = g.forward(embed(m, toks))
    with pytest.raises(xp.XjError):
        g.forward(embed(m, toks[:1]))      # context full
    g.reset()
    assert g.n_past == 0
    x2 = g.forward(embed(m, toks))
    assert np.array_equal(x1, x2)
    g.destroy()


def test_chain_greedy_matches_oracle(tiny):
    m, L = tiny, tiny.hp.n_layer
    prompt = prompt_ids(m, 21, 6)
    g = xp.HipStage(m, 0, L, 256, 8, True)
    ch = xp.Chain([g])
    toks = np.concatenate([ch.eval(prompt), ch.decode(63)])
    c = orc.CpuStage(m.ptr, 0, L, 256, 8, True, kv_f16=True)
    want, margins = orc.greedy([c], prompt, 64)
    assert np.array_equal(toks, want), (toks, want, margins)
    ch.free()
    g.destroy()
    c.destroy()


def test_decode_never_reads_unwritten_cache(tiny):
    """The cache slots at and past the decode position hold whatever the memory held (here an fp16 NaN in
    every slot) until a step writes them; a single-token step writes its own slot inside the attention
    kernel, so it must not combine those bytes, not even with a zero weight (0 * NaN = NaN)."""
    m, L = tiny, tiny.hp.n_layer
    prompt = prompt_ids(m, 21, 6)
    g = xp.HipStage(m, 0, L, 256, 8, True)
    ch = xp.Chain([g])
    first = ch.eval(prompt)
    g.fill_kv(len(prompt), 0x7E00)
    toks = np.concatenate([first, ch.decode(40)])
    c = orc.CpuStage(m.ptr, 0, L, 256, 8, True, kv_f16=True)
    want, margins = orc.greedy([c], prompt, 41)
    assert np.array_equal(toks, want), (toks, want, margins)
    ch.free()
    g.destroy()
    c.destroy()


def test_chain_split_and_vtable_agree(tiny):
    """Two chained stages on the device give the same tokens as the host-driven vtable loop."""
    m, L = tiny, tiny.hp.n_layer
    prompt = prompt_ids(m, 9, 7)
    a, b = xp.HipStage(m, 0, 4, 128, 8, False), xp.HipStage(m, 4, L, 128, 8, True)
    ch = xp.Chain([a, b])
    toks = np.concatenate([ch.eval(prompt), ch.decode(31)])
    ch.free()
    a.destroy()
    b.destroy()
    g = xp.HipStage(m, 0, L, 128, 8, True)
    x = g.forward(embed(m, prompt[:8]))
    x = g.forward(embed(m, prompt[8:]))
    host = []
    for _ in range(32):
        t = int(np.argmax(g.logits(x[-1:])[0]))
        host.append(t)
        x = g.forward(embed(m, [t]))
    assert toks.tolist() == host
    g.destroy()


@pytest.mark.parametrize("cuts", [(0, 4, 8), (0, 2, 5, 8)])
def test_pipelined_chain_prefill_equals_one_stage(tiny, cuts):
    """A prompt of many chunks through a chain whose stages run on their own
    streams, chunk k + 1 in stage i while chunk k is in stage i + 1
    (xj_net.c:561-604): the logits of the last rows, the hidden rows left for
    the drivers and the tokens decoded after it equal those of one stage
    computing the same chunks in order, bit for bit."""
    m, L = tiny, tiny.hp.n_layer
    assert cuts[-1] == L
    prompt = prompt_ids(m, 70, 29)            # max_batch 16: chunks 16 x 4 + 6
    one = xp.HipStage(m, 0, L, 128, 16, True)
    c1 = xp.Chain([one])
    am1, lg1 = c1.eval(prompt, nlog=3, want_logits=True)
    t1 = c1.decode(12)
    sts = [xp.HipStage(m, cuts[i], cuts[i + 1], 128, 16, i + 2 == len(cuts)) for i in range(len(cuts) - 1)]
    c2 = xp.Chain(sts)
    am2, lg2 = c2.eval(prompt, nlog=3, want_logits=True)
    assert np.array_equal(lg1.view(np.uint32), lg2.view(np.uint32))
    assert am1.tolist() == am2.tolist()
    assert c2.decode(12).tolist() == t1.tolist()
    # again from a reset state: the device positions restart with the host's
    c2.reset()
    c1.reset()
    a1 = c1.eval(prompt[:37])
    a2 = c2.eval(prompt[:37])
    assert a1.tolist() == a2.tolist()
    for c in (c1, c2):
        c.free()
    for st in [one] + sts:
        st.destroy()


def test_chain_verify_and_rollback(tiny):
    m, L = tiny, tiny.hp.n_layer
    prompt = prompt_ids(m, 16, 8)
    g = xp.HipStage(m, 0, L, 128, 8, True)
    ch = xp.Chain([g])
    ch.eval(prompt)
    greedy = ch.decode(5)                       # reference continuation
    g2 = xp.HipStage(m, 0, L, 128, 8, True)
    c2 = xp.Chain([g2])
    first = c2.eval(prompt)
    cand = np.concatenate([first, greedy[:4]])  # [t, d1..d4] all correct
    am = c2.eval(cand, nlog=5, keep=True)
    assert am.tolist() == greedy.tolist()
    c2.rollback(16 + 2)                          # keep t, d1
    nxt = c2.eval(greedy[1:2])
    assert int(nxt[0]) == int(greedy[2])
    for o in (ch, c2):
        o.free()
    g.destroy()
    g2.destroy()


def test_verify_pass_logits_equal_single_steps(tiny):
    """A 5-token verification pass gives, bit for bit, the logits of feeding
    the same tokens one at a time (the decode step's kernels)."""
    m, L = tiny, tiny.hp.n_layer
    prompt, cand = prompt_ids(m, 16, 8), prompt_ids(m, 5, 9)
    g1, g2 = xp.HipStage(m, 0, L, 128, 8, True), xp.HipStage(m, 0, L, 128, 8, True)
    c1, c2 = xp.Chain([g1]), xp.Chain([g2])
    c1.eval(prompt)
    c2.eval(prompt)
    _, lg5 = c1.eval(cand, nlog=5, keep=True, want_logits=True)
    lg1 = np.stack([c2.eval(cand[i:i + 1], nlog=1, want_logits=True)[1][0] for i in range(5)])
    assert np.array_equal(lg5.view(np.uint32), lg1.view(np.uint32))
    for o in (c1, c2):
        o.free()
    g1.destroy()
    g2.destroy()


@pytest.mark.parametrize("mode", ["draft", "oracle_all", "oracle_miss", "oracle_guess_miss"])
def test_spec_decode_equals_greedy(tiny, tiny_draft_path, mode):
    """Speculative generation equals plain greedy decoding. oracle_guess_miss:
    oracle drafts with wrong tokens at positions 15 and 31, where fully
    accepted rounds that overlap the next round's drafting with their
    verification guess the target's next token (the guess fails, the draft
    returns to its state after the round's last draft)."""
    m, L = tiny, tiny.hp.n_layer
    dm = xp.Model(tiny_draft_path)
    prompt = prompt_ids(m, 13, 9)
    n_gen = 40
    g = xp.HipStage(m, 0, L, 256, 8, True)
    ch = xp.Chain([g])
    plain = np.concatenate([ch.eval(prompt), ch.decode(n_gen - 1)])
    ch.free()
    g.destroy()
    t = xp.HipStage(m, 0, L, 256, 8, True)
    d = xp.HipStage(dm, 0, dm.hp.n_layer, 256, 8, True)
    tc, dc = xp.Chain([t]), xp.Chain([d])
    tc.eval(prompt)
    dc.eval(prompt)
    oracle = None if mode == "draft" else plain.copy()
    if mode == "oracle_guess_miss":
        V = int(m.hp.n_vocab)
        for gi in (15, 31):
            oracle[gi] = (oracle[gi] + 1) % V
    miss = 3 if mode == "oracle_miss" else 0
    out, st = xp.spec_generate(tc, dc, 4, n_gen, oracle=oracle, oracle_miss=miss)
    assert out.tolist() == plain.tolist()
    if mode == "oracle_all":
        assert st.n_accepted == st.n_drafted
        assert st.n_overlap_held == st.n_overlap > 0
    if mode == "oracle_guess_miss":
        assert 0 < st.n_overlap_held < st.n_overlap
    for o in (tc, dc):
        o.free()
    t.destroy()
    d.destroy()


def test_stage_over_a_layer_range_load(tiny, tiny_path, tmp_path):
    """A stage built from xj_model_load_layers on a file cut after its layers
    (a partial download, xj_model.c:214-233) computes bit for bit what the stage
    built from the whole file computes; a stage over layers outside the mapping
    is refused."""
    m, L = tiny, tiny.hp.n_layer
    part0 = xp.Model(tiny_path, layers=(0, L // 2))
    hi = part0.ranges(0, L // 2)[-1][1]
    part0.close()
    cut = str(tmp_path / "front.gguf")
    with open(tiny_path, "rb") as f, open(cut, "wb") as g:
        g.write(f.read(hi))
    part = xp.Model(cut, layers=(0, L // 2))
    toks = prompt_ids(m, 9, 5)
    x = embed(m, toks)
    a = xp.HipStage(part, 0, L // 2, 64, 16, False)
    b = xp.HipStage(m, 0, L // 2, 64, 16, False)
    xa, xb = a.forward(x[:8].copy()), b.forward(x[:8].copy())
    assert np.array_equal(xa, xb)
    xa, xb = a.forward(x[8:].copy()), b.forward(x[8:].copy())
    assert np.array_equal(xa, xb)
    a.destroy()
    b.destroy()
    with pytest.raises(xp.XjError, match="not mapped"):
        xp.HipStage(part, L // 2, L, 64, 16, False)
    with pytest.raises(xp.XjError, match="not mapped"):
        xp.HipStage(part, 0, L // 2, 64, 16, True)
    part.close()


class RefLoaded:
    """A model table built by the reference's own loader (xj_model_load,
    core/xj_model.c:204), seen through the boundary struct."""

    def __init__(self, path, mtp_from=None):
        err = orc.C.create_string_buffer(512)
        r = orc.rlib().ref_model_load(path.encode(), err, 512)
        assert r, err.value
        if mtp_from:
            assert orc.rlib().ref_model_attach_mtp(r, mtp_from.encode(), err, 512) == 0, err.value
        self.r = r
        self.ptr = orc.C.cast(r, orc.C.POINTER(xp.XjModel))

    @property
    def hp(self):
        return self.ptr.contents.hp

    def free(self):
        orc.rlib().ref_model_free(self.r)


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
def test_hip_stages_over_the_reference_loader(model_dir, tiny_path):
    """The literal drop-in (core/xj_stage.h:46): xj_hip_stage_new over a model
    that the reference's own loader built, driven by the reference's own
    pipeline and greedy driver (split 0-3 | 3-8, as xjpipe-host runs it):
    the oracle's fp16-KV greedy tokens, and bit for bit the tokens of HIP
    stages over this library's loader. The MTP layer attached by the
    reference's xj_model_attach_mtp (core/xj_model.c:275-300) from a second
    file serves a HIP MTP stage whose drafts leave the output unchanged."""
    from conftest import synth_model
    rec_prompt = prompt_ids(xp.Model(tiny_path), 24, 41)
    mine = xp.Model(tiny_path)
    L = mine.hp.n_layer
    ref = RefLoaded(tiny_path, mtp_from=synth_model(model_dir, xp.TINY_MTP, "tiny_mtp"))
    n_gen = 32

    def drive(model, k):
        a, b = xp.HipStage(model, 0, 3, 256, 8, False), xp.HipStage(model, 3, L, 256, 8, True)
        mt = xp.HipStage(model, L, L + 1, 256, 8, True) if k else None
        out, st = orc.ref_spec_run(model.ptr, a.ptr, b.ptr, mt.ptr if mt else None, k, rec_prompt, n_gen)
        for s in (a, b, mt):
            if s:
                s.destroy()
        return out, st

    c = orc.CpuStage(mine.ptr, 0, L, 256, 8, True, kv_f16=True)
    want, _ = orc.greedy([c], rec_prompt, n_gen)
    c.destroy()
    got_ref, _ = drive(ref, 0)
    got_mine, _ = drive(mine, 0)
    assert got_ref.tolist() == got_mine.tolist() == want.tolist()
    spec, st = drive(ref, 3)
    assert spec.tolist() == want.tolist() and st[1] > 0
    ref.free()


@pytest.mark.parametrize("T", [16, 40, 64])
def test_prefill_chunk_matches_oracle(tiny, T):
    """A prefill chunk of at least 16 tokens takes the matrix-core path: GEMM
    projections (RMSNorm scale per token after the dot products), the conv +
    SiLU launch, the chunked delta rule over prepared q/k/v/decay/beta (GQA
    heads: key head hv % Hk), the gated RMSNorm as ssm_out's prep. Hidden states
    against the oracle, then decode steps continue from the chunk's recurrent
    and KV state."""
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, T + 3, 21 + T)
    g = xp.HipStage(m, 0, L, 128, 64, True)
    c = orc.CpuStage(m.ptr, 0, L, 128, 64, True, kv_f16=True)
    x = embed(m, toks[:T])
    xg, xc = g.forward(x.copy()), c.forward(x.copy())
    assert rel_l2(xg, xc) < 1e-3
    for t in range(T, T + 3):
        x1 = embed(m, toks[t:t + 1])
        yg, yc = g.forward(x1.copy()), c.forward(x1.copy())
        assert rel_l2(yg, yc) < 1e-3, t
    lg, lc = g.logits(yg), c.logits(yc)
    assert rel_l2(lg, lc) < 1e-3
    assert int(np.argmax(lg)) == int(np.argmax(lc))
    g.destroy()
    c.destroy()


def test_prefill_chunk_with_checkpoints_rolls_back(tiny):
    """A 20-token chunk with keep: GEMM projections, the conv launch writing
    its checkpoints, the recurrent rule writing the state checkpoints; rolled
    back into the chunk it continues as a fresh stage fed the kept prefix
    (which itself takes the chunked rule, 18 tokens without keep)."""
    m, L = tiny, tiny.hp.n_layer
    toks = prompt_ids(m, 40, 22)
    g = xp.HipStage(m, 0, L, 128, 64, True)
    g.forward(embed(m, toks[:8]))
    g.set_keep(20)
    g.forward(embed(m, toks[8:28]))
    g.rollback(14)
    assert g.n_past == 14
    x_after = g.forward(embed(m, toks[30:34]))
    ref = xp.HipStage(m, 0, L, 128, 64, True)
    xr = ref.forward(embed(m, np.concatenate([toks[:14], toks[30:34]])))
    assert rel_l2(x_after, xr[14:]) < 1e-4
    c = orc.CpuStage(m.ptr, 0, L, 128, 64, True, kv_f16=True)
    xc = c.forward(embed(m, np.concatenate([toks[:14], toks[30:34]])))
    assert rel_l2(x_after, xc[14:]) < 1e-3
    for s_ in (g, ref, c):
        s_.destroy()

