"""Batch-1 greedy decode throughput of the synthetic hybrid 4B-shape model on one MI355X.

One step = one greedy decode token through all 32 layers and the LM head,
entirely on the device (one HIP graph launch: 24 DeltaNet + 8 gated-GQA
layers, Q6_K LM head, argmax, whose launch also writes the chosen token's
embedding as the next step's input). The prompt
(1024 uniform random ids) is prefilled first; W warm-up steps are not timed;
exactly K steps are timed between device synchronisations.

Also reported, on the same run:
  roofline      the fused dequant-GEMV kernel (the decode's dominant kernel):
                algorithmic bytes of the GEMV launches of one step divided by
                their GPU time, measured with HIP events on the chain's stream
                by replaying exactly those launches (weights 2.6 GB: cold).
                traffic = measured HBM bytes per GEMV launch from the committed
                counter summary profiles/traffic_gemv_4b_decode.json, if present.
  cpu_baseline  the reference CPU path compiled from the reference sources
                (oracle/_ref, OpenMP on this host's cores) on a bounded sample
                of the same workload; the oracle's C restatement if that
                library is absent.
  gemv_*        stand-alone cold-cache GEMV legs (Q4_K / Q6_K LM-head shapes), and
                at T = 1..5 activation rows the mixed-quant batch (Q6_K 3584x1024,
                Q8_0 1024x3584, Q4_K 151936x1024) and the 4B gate|up and down shapes.
  decode_sampled_4b  the same chain decoding with the app's sampler at temperature 0.7 (top-k 40,
                top-p 0.95; the draw is the decode graph's last launch), 128 steps.
  decode_0_8b   the same measurement on the 0.8B-shape model.
  prefill_1024_two_stages  the 1024-token prefill with the 4B shape split 0-15 | 16-31, the two
                stages' chunks pipelined on two streams.
  verify_4b     one pass of T = 1..5 tokens with checkpoints on the 4B shape (the
                speculative verification widths), ms per pass beside the decode step.
  speculative_4b  the 4B shape split 0-15 | 16-31 with the 0.8B model drafting
                4 tokens per step (5-row verify passes): real drafts, drafts
                from the plain greedy output, and one in four of them
                perturbed; tok/s and acceptance, each checked token-identical
                to plain greedy decoding.
  speculative_4b_mtp  the same with the model's own MTP layer drafting (the
                4B shape with one MTP layer added).

usage: python bench.py [--gpus 1] [--steps 512] [--warmup 16] [--no-cpu] [--no-extra]
                       [--copy-calibration MB] [--delta-c3] [--gemm-tokens]
--copy-calibration MB first copies MB megabytes device-to-device (one runtime
copy kernel of known size, to calibrate the HBM byte counters of a profiler run).
--gemm-tokens runs only the prefill-chunk GEMM legs (matrix-core GEMM vs
GEMV tiles at T = 16/32/64).
--delta-c3 runs only the Gated DeltaNet prefill comparison (16 heads, d=128,
2048 tokens: chunk-wise MFMA kernels vs the token-by-token kernel) and prints
its JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "meta-work_amd"))

import numpy as np  # noqa: E402

import xjpipe as xp  # noqa: E402

METRIC = "batch-1 decode tok/s (hybrid Q4_K 0.8B/4B shapes); GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_path(cfg, name):
    return xp.cached_model(cfg, name)


SAMPLED_STEPS = 128


def decode_run(cfg, name, n_prompt, steps, warmup, seed):
    m = xp.Model(model_path(cfg, name))
    hp = m.hp
    n_ctx = n_prompt + warmup + steps + SAMPLED_STEPS + 8
    t = time.time()
    # prefill chunks of 64 tokens (the GEMM and chunked DeltaNet path); decode is one token
    st = xp.HipStage(m, 0, hp.n_layer, n_ctx, 64, True)
    log(f"{name}: uploaded in {time.time() - t:.1f} s ({xp.tune_note()})")
    ch = xp.Chain([st])
    prompt = np.random.default_rng(seed).integers(0, hp.n_vocab, n_prompt).astype(np.int32)
    # warm-up of the prefill path over two chunks (so the pipelined parts' scratch
    # is allocated and their kernels loaded), then a fresh stage state
    ch.eval(prompt[:128])
    ch.reset()
    t = time.perf_counter()
    first = ch.eval(prompt)
    prefill_s = time.perf_counter() - t
    log(f"{name}: prefill {n_prompt} tokens in {prefill_s:.3f} s, first token {int(first[0])}")
    assert n_prompt >= 128
    if warmup:
        ch.decode(warmup)
    t0 = time.perf_counter()
    toks = ch.decode(steps)          # synchronises before and after the replayed graphs
    wall = time.perf_counter() - t0
    gpu_ms = ch.last_decode_ms
    return dict(m=m, st=st, ch=ch, prompt=prompt, first=int(first[0]), toks=toks, wall=wall, gpu_ms=gpu_ms,
                prefill_s=prefill_s)


def prefill_only(n_prompt=1024, reps=3, seed=20261107, split=None):
    """The 4B shape's 1024-token prefill (chunks of 64: the matrix-core GEMM and the chunked delta
    rule), reps times from a reset state, for a kernel trace of the prefill alone. split = l: two
    stages [0, l) | [l, n_layer) whose chunks are pipelined on two streams (the reference's 4B
    setup splits at 16)."""
    m = xp.Model(model_path(xp.CONFIG_4B, "synth4b"))
    hp = m.hp
    cuts = [0, hp.n_layer] if split is None else [0, split, hp.n_layer]
    sts = [xp.HipStage(m, cuts[i], cuts[i + 1], n_prompt + 8, 64, i + 2 == len(cuts)) for i in range(len(cuts) - 1)]
    ch = xp.Chain(sts)
    prompt = np.random.default_rng(seed).integers(0, hp.n_vocab, n_prompt).astype(np.int32)
    times, first = [], None
    for _ in range(reps):
        ch.reset()
        t0 = time.perf_counter()
        first = int(ch.eval(prompt)[0])
        times.append(time.perf_counter() - t0)
    ch.free()
    for st in sts:
        st.destroy()
    return {"prefill_tokens": n_prompt, "stages": len(sts), "prefill_s": [round(t, 4) for t in times], "first_token": first}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def oracle_mod():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    return orc


def cpu_baseline(cfg, name, n_prompt_cpu, n_steps_cpu, seed, at_pos=None):
    """Reference CPU path (oracle/_ref) or the oracle restatement on the host cores. With at_pos, the
    decode steps run at positions at_pos.. (the GPU run's context): after the n_prompt_cpu-token
    prompt the stage's n_past is set to at_pos, so each step attends over at_pos + 1 positions whose
    cache entries past the prompt stay as allocated - a timing sample, not a token-parity run (a
    real 1024-token CPU prefill would take about a minute)."""
    orc = oracle_mod()
    kind = "reference" if orc.ref_available() else "port"
    m = xp.Model(model_path(cfg, name))
    hp = m.hp
    n_ctx = (at_pos or n_prompt_cpu) + n_steps_cpu + 8
    stage = orc.CpuStage(m.ptr, 0, hp.n_layer, n_ctx, n_prompt_cpu, True, ref=(kind == "reference"))
    prompt = np.random.default_rng(seed).integers(0, hp.n_vocab, n_prompt_cpu).astype(np.int32)
    x = np.stack([orc.embed(m.ptr, int(t)) for t in prompt])
    stage.forward(x)
    tok = int(np.argmax(stage.logits(x[-1:])[0]))
    if at_pos:
        stage.ptr.contents.n_past = at_pos
    t0 = time.perf_counter()
    for _ in range(n_steps_cpu):
        x = orc.embed(m.ptr, tok)[None].copy()
        stage.forward(x)
        tok = int(np.argmax(stage.logits(x)[0]))
    dt = time.perf_counter() - t0
    stage.destroy()
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    where = (f"positions {at_pos}..{at_pos + n_steps_cpu - 1} (n_past set to {at_pos} after a {n_prompt_cpu}-token "
             f"prompt, as the GPU run's context)" if at_pos else f"after a {n_prompt_cpu}-token prompt")
    return {"value": round(n_steps_cpu / dt, 3), "unit": "tok/s", "cores": cores, "kind": kind, "cpu": cpu_model(),
            "sample": f"{name} model, {n_steps_cpu} timed greedy decode steps at {where} "
                      f"(fp32 KV, OpenMP over {cores} threads, {dt:.1f} s)"}


def cpu_configs(seed=20261107):
    """CPU figures of the smaller configs on the host cores (the reference's own C core when
    oracle/_ref is built, else the oracle restatement): the Q4_K GEMV 4096x1024 (config 1) and the
    mixed-quant batch at T = 1 and 5 (config 2) as us and effective GB/s, the standalone DeltaNet
    layer recurrence over 2048 + 256 tokens (config 3, the oracle's restatement: the reference runs
    it inside its layer), the 0.8B decode at its GPU context (config 4)."""
    orc = oracle_mod()
    ref = orc.ref_available()

    def matmul_leg(t, rows, k, T, reps):
        blob = xp.quantize(t, xp.fill_normal(rows * k, 17, 0.02).reshape(rows, k))
        x = xp.fill_normal(T * k, 5, 1.0).reshape(T, k)
        orc.matmul(t, blob, k, rows, x, ref=ref)
        t0 = time.perf_counter()
        for _ in range(reps):
            orc.matmul(t, blob, k, rows, x, ref=ref)
        dt = (time.perf_counter() - t0) / reps
        by = rows * xp.row_bytes(t, k) + T * k * 4 + T * rows * 4
        return {"shape": f"{xp.TYPE_NAMES[t]} {rows}x{k}", "T": T, "us": round(dt * 1e6, 1),
                "GBps": round(by / dt / 1e9, 2)}

    out = {"kind": "reference" if ref else "port", "cpu": cpu_model(),
           "cores": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))}
    out["config1"] = matmul_leg(xp.Q4_K, 4096, 1024, 1, 200)
    out["config2"] = [matmul_leg(t, r, k, T, 40 if r < 10000 else 5)
                      for (t, r, k) in ((xp.Q6_K, 3584, 1024), (xp.Q8_0, 1024, 3584), (xp.Q4_K, 151936, 1024))
                      for T in (1, 5)]
    T, H, S = 2048 + 256, 16, 128
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, H, S)).astype(np.float32)
    k = rng.standard_normal((T, H, S)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, H, S)).astype(np.float32)
    dec = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    t0 = time.perf_counter()
    orc.delta_recurrent(q, k, v, dec, beta, np.zeros((H, S, S), np.float32), 1 / np.sqrt(S))
    dt = time.perf_counter() - t0
    out["config3"] = {"shape": "H=16 d=128, 2048-token prefill + 256 steps (token by token, oracle)",
                      "ms": round(dt * 1e3, 1), "us_per_token": round(dt * 1e6 / T, 2),
                      "state_GBps": round(T * 2 * H * S * S * 4 / dt / 1e9, 2)}
    out["config4"] = cpu_baseline(xp.CONFIG_0_8B, "synth08b", 16, 24, seed=20261108, at_pos=512)
    return out


def dropin_run(n_prompt=1024, n_gen=64, seed=20261107):
    """The drop-in path: the reference's own driver (greedy loop, xjpipe-host.c:131-144, compiled
    from source in oracle/_ref) over HIP stages behind the xj_stage vtable - logits copied to the
    host every token, the argmax on the host - on the 4B shape, one stage, 1024-token prompt."""
    orc = oracle_mod()
    if not orc.ref_available():
        return None
    m = xp.Model(model_path(xp.CONFIG_4B, "synth4b"))
    hp = m.hp
    n_ctx = n_prompt + 2 * n_gen + 16
    a, b = xp.HipStage(m, 0, 16, n_ctx, 64, False), xp.HipStage(m, 16, hp.n_layer, n_ctx, 64, True)
    prompt = np.random.default_rng(seed).integers(0, hp.n_vocab, n_prompt).astype(np.int32)
    runs = {}
    for n in (1, n_gen):   # the prefill alone (one token generated), then the prefill and n_gen tokens
        for s_ in (a, b):
            s_.reset()
        t0 = time.perf_counter()
        toks, _ = orc.ref_spec_run(m.ptr, a.ptr, b.ptr, None, 0, prompt, n)
        runs[n] = (time.perf_counter() - t0, toks)
    for s_ in (a, b):
        s_.destroy()
    dec_s = runs[n_gen][0] - runs[1][0]
    return {"tok_s": round((n_gen - 1) / dec_s, 1), "prefill_s": round(runs[1][0], 3), "tokens": n_gen,
            "prompt": n_prompt, "first_token": int(runs[n_gen][1][0]),
            "note": ("the reference's own pipeline and greedy driver (compiled from source) over two HIP "
                     "stages (layers 0-15 | 16-31) behind the xj_stage vtable: the logits of every token "
                     "copied to the host, the argmax on the host; tok_s = decode steps after the first token")}


def gemv_leg(t, rows, k, copies, iters):
    """Cold-cache GEMV: `copies` distinct weights (> 512 MB in total) launched in rotation."""
    xs = xp.fill_normal(k, 5, 1.0)[None]
    blob = xp.quantize(t, xp.fill_normal(rows * k, 17, 0.02).reshape(rows, k))
    ws = [xp.DevWeight(t, blob, rows, k) for _ in range(copies)]
    ms = xp.gemv_time(ws, xs, iters)
    by = rows * xp.row_bytes(t, k) + k * 4 + rows * 4
    for w in ws:
        w.free()
    return {"shape": f"{xp.TYPE_NAMES[t]} {rows}x{k} T=1", "us": round(ms * 1e3, 2),
            "GBps": round(by / (ms * 1e-3) / 1e9, 1), "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}


def gemv_legs():
    """The LM-head shapes (151936x1024 of the 0.8B model, as Q4_K and as the synthetic model's Q6_K;
    Q6_K 151936x2560 of the 4B model) and config 1 (Q4_K 4096x1024), single token, cold weights."""
    return [gemv_leg(xp.Q4_K, 151936, 1024, 8, 64), gemv_leg(xp.Q6_K, 151936, 1024, 6, 48),
            gemv_leg(xp.Q6_K, 151936, 2560, 3, 24), gemv_leg(xp.Q4_K, 4096, 1024, 256, 512)]


def gemv_tokens(t, rows, k, iters=200):
    """One weight shape at T = 1..5 activation rows (the speculative-verify widths), cold weights
    (rotating copies totalling more than 600 MB): us per launch (the per-op entry, activations built
    in the GEMV's work-groups for T <= 2, by a prep launch beyond) and weight GB/s."""
    by = rows * xp.row_bytes(t, k)
    copies = max(4, -(-600_000_000 // by))
    blob = xp.quantize(t, xp.fill_normal(rows * k, 17, 0.02).reshape(rows, k))
    ws = [xp.DevWeight(t, blob, rows, k) for _ in range(copies)]
    out = []
    for T in range(1, 6):
        xs = np.stack([xp.fill_normal(k, 5 + i, 1.0) for i in range(T)])
        ms = xp.gemv_time(ws, xs, iters)
        out.append({"T": T, "us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1)})
    for w in ws:
        w.free()
    return {"shape": f"{xp.TYPE_NAMES[t]} {rows}x{k}", "by_T": out}


def gemm_tokens(t, rows, k, iters=50):
    """Prefill chunks of T = 16 / 32 / 64 tokens on one weight shape, cold weights: the matrix-core
    GEMM (xjh_gemm, its prep launch included) against the dot-product GEMV in tiles of 5 tokens
    (xjh_gemv at T = 5, scaled by T / 5), us per chunk and GFLOP/s (2 rows k T)."""
    by = rows * xp.row_bytes(t, k)
    copies = max(4, -(-600_000_000 // by))
    blob = xp.quantize(t, xp.fill_normal(rows * k, 17, 0.02).reshape(rows, k))
    ws = [xp.DevWeight(t, blob, rows, k) for _ in range(copies)]
    out = []
    for T in (16, 32, 64):
        xs = xp.fill_normal(T * k, 23 + T, 1.0).reshape(T, k)
        ms = xp.gemm_time(ws, xs, iters)
        mv = xp.gemv_time(ws, xs[:5], iters) * T / 5
        out.append({"T": T, "gemm_us": round(ms * 1e3, 1), "gemv_tiles_us": round(mv * 1e3, 1),
                    "gemm_GFLOPs": round(2.0 * rows * k * T / (ms * 1e-3) / 1e9, 1)})
    for w in ws:
        w.free()
    return {"shape": f"{xp.TYPE_NAMES[t]} {rows}x{k}", "by_T": out}


def spec_run(n_prompt=1024, n_gen=128, seed=20261109):
    """Speculative decode on the 4B shape, split 0-15 | 16-31 on one stream, with the 0.8B model
    drafting 4 tokens per step and the target verifying them as one 5-row pass: the real draft (random
    weights: acceptance near 0), drafts taken from the plain greedy output (every draft accepted), and
    the same with one draft in 4 perturbed. Every run must reproduce the plain greedy tokens."""
    m, dm = xp.Model(model_path(xp.CONFIG_4B, "synth4b")), xp.Model(model_path(xp.CONFIG_0_8B, "synth08b"))
    n_ctx = n_prompt + n_gen + 16
    prompt = np.random.default_rng(seed).integers(0, m.hp.n_vocab, n_prompt).astype(np.int32)
    a, b = xp.HipStage(m, 0, 16, n_ctx, 8, False), xp.HipStage(m, 16, 32, n_ctx, 8, True)
    d = xp.HipStage(dm, 0, dm.hp.n_layer, n_ctx, 8, True)
    tc, dc = xp.Chain([a, b]), xp.Chain([d])
    plain = np.concatenate([tc.eval(prompt), tc.decode(n_gen - 1)])
    res = {"prompt": n_prompt, "tokens": n_gen, "k": 4}
    for mode, orc, miss in (("draft_0_8b", None, 0), ("oracle_drafts", plain, 0), ("oracle_miss_1_in_4", plain, 4)):
        tc.reset()
        dc.reset()
        tc.eval(prompt)
        dc.eval(prompt)
        out, st = xp.spec_generate(tc, dc, 4, n_gen, oracle=orc, oracle_miss=miss)
        if out.tolist() != plain.tolist():
            raise RuntimeError(f"speculative decode ({mode}) diverged from plain greedy decoding")
        res[mode] = {"tok_s": round(n_gen / (st.t_total_ms / 1e3), 1), "verify_passes": st.n_steps,
                     "drafted": st.n_drafted, "accepted": st.n_accepted,
                     "draft_ms": round(st.t_draft_ms, 1), "total_ms": round(st.t_total_ms, 1)}
        log(f"spec {mode}: {res[mode]}")
    for o in (tc, dc):
        o.free()
    for s in (a, b, d):
        s.destroy()
    return res


def spec_mtp_run(n_prompt=1024, n_gen=128, seed=20261110):
    """Speculative decoding with the model's own MTP layer as the drafter (k = 4), on the 4B shape with
    one MTP layer added (its main layers are those of the 4B model): real drafts (random weights:
    acceptance near 0), drafts from the plain greedy output, one in four of them perturbed. Every run
    must reproduce the plain greedy tokens."""
    cfg = xp.CONFIG_4B.with_(nextn=1)
    m = xp.Model(model_path(cfg, "synth4b_mtp"))
    L = m.hp.n_layer
    n_ctx = n_prompt + n_gen + 16
    prompt = np.random.default_rng(seed).integers(0, m.hp.n_vocab, n_prompt).astype(np.int32)
    st = xp.HipStage(m, 0, L, n_ctx, 8, True)
    ch = xp.Chain([st])
    plain = np.concatenate([ch.eval(prompt), ch.decode(n_gen - 1)])
    mt = xp.HipStage(m, L, L + 1, n_ctx, 8, True)
    res = {"prompt": n_prompt, "tokens": n_gen, "k": 4}
    for mode, orc, miss in (("mtp_drafts", None, 0), ("oracle_drafts", plain, 0), ("oracle_miss_1_in_4", plain, 4)):
        out, s = xp.spec_generate_mtp(ch, mt, 4, prompt, n_gen, oracle=orc, oracle_miss=miss)
        if out.tolist() != plain.tolist():
            raise RuntimeError(f"MTP speculative decode ({mode}) diverged from plain greedy decoding")
        res[mode] = {"tok_s": round(n_gen / (s.t_total_ms / 1e3), 1), "verify_passes": s.n_steps,
                     "drafted": s.n_drafted, "accepted": s.n_accepted, "draft_ms": round(s.t_draft_ms, 1),
                     "total_ms": round(s.t_total_ms, 1)}
        log(f"spec mtp {mode}: {res[mode]}")
    ch.free()
    st.destroy()
    mt.destroy()
    return res


def verify_widths(widths=(1, 2, 3, 4, 5), n_prompt=1024, reps=30, seed=20261112, pause_s=0.0):
    """Speculative-verification passes on the 4B shape (one stage): after a 1024-token prompt, T = 1..5
    tokens fed as one pass with checkpoints, then rolled back to the first of them (the next pass starts
    one position later); ms per pass, median of `reps`, host round trip included. pause_s: an idle gap
    before the timed passes (marks them in a kernel trace)."""
    m = xp.Model(model_path(xp.CONFIG_4B, "synth4b"))
    st = xp.HipStage(m, 0, m.hp.n_layer, n_prompt + (len(widths) + 1) * reps + 16, 64, True)
    ch = xp.Chain([st])
    rng = np.random.default_rng(seed)
    ch.eval(rng.integers(0, m.hp.n_vocab, n_prompt).astype(np.int32))
    toks = rng.integers(0, m.hp.n_vocab, 5).astype(np.int32)

    def run(T, n):
        ts = []
        for _ in range(n):
            p0 = ch.n_past
            t0 = time.perf_counter()
            ch.eval(toks[:T], nlog=T, keep=True)
            ts.append(time.perf_counter() - t0)
            ch.rollback(p0 + 1)
        return float(np.median(ts)) * 1e3

    run(max(widths), 3)
    if pause_s:
        time.sleep(pause_s)
    out = [{"T": T, "ms": round(run(T, reps), 3)} for T in widths]
    ch.free()
    st.destroy()
    return out


def delta_c3(reps=3):
    """Gated DeltaNet prefill on the c3 shape (16 heads, d=128, 2048 tokens from a zero state): the chunk-wise
    MFMA kernels (chunk 64) next to the token-by-token kernel. Wall ms per call include the host copies; the
    kernel durations come from a rocprofv3 trace of `bench.py --delta-c3`."""
    T, H, S = 2048, 16, 128
    rng = np.random.default_rng(20261109)
    q = rng.standard_normal((T, H, S)).astype(np.float32)
    k = rng.standard_normal((T, H, S)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, H, S)).astype(np.float32)
    dec = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    st = np.zeros((H, S, S), np.float32)
    res = {}
    for name, chunk in (("chunked", 64), ("recurrent", 0)):
        best = None
        for _ in range(reps):
            t0 = time.perf_counter()
            o, s = xp.delta(q, k, v, dec, beta, st, 1 / np.sqrt(S), chunk=chunk)
            dt = (time.perf_counter() - t0) * 1e3
            best = dt if best is None else min(best, dt)
        res[name] = (o, s, best)
    rel = lambda a, b: float(np.linalg.norm(a - b) / np.linalg.norm(b))
    return {"shape": "H=16 d=128 T=2048 chunk 64", "chunked_wall_ms": round(res["chunked"][2], 2),
            "recurrent_wall_ms": round(res["recurrent"][2], 2),
            "out_rel_l2": rel(res["chunked"][0], res["recurrent"][0]),
            "state_rel_l2": rel(res["chunked"][1], res["recurrent"][1])}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the 0.8B run and the GEMV legs")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB")
    ap.add_argument("--greedy-only", action="store_true",
                    help="no sampled-decode leg (the counter runs: rocprofv3 --pmc has crashed in its own code on it)")
    ap.add_argument("--delta-c3", action="store_true", help="only the chunked vs token-by-token DeltaNet prefill")
    ap.add_argument("--gemm-tokens", action="store_true", help="only the prefill-chunk GEMM vs GEMV-tile legs")
    ap.add_argument("--prefill-only", action="store_true", help="only the 4B 1024-token prefill, three times")
    ap.add_argument("--gemv-legs", action="store_true", help="only the cold-cache single-token GEMV legs (LM heads)")
    ap.add_argument("--verify-only", nargs="?", const="1,2,3,4,5", default=None, metavar="WIDTHS",
                    help="only the 4B verification passes of the given widths (after a 0.2 s pause)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the token loop on a single MI355X and has no "
              f"multi-GPU path (--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    log(f"device: {xp.device_name()}")
    if args.gemm_tokens:
        print(json.dumps([gemm_tokens(xp.Q4_K, 18432, 2560), gemm_tokens(xp.Q6_K, 2560, 9216),
                          gemm_tokens(xp.Q4_K, 2560, 4096)]), flush=True)
        return
    if args.delta_c3:
        print(json.dumps(delta_c3()), flush=True)
        return
    if args.verify_only:
        print(json.dumps(verify_widths([int(w) for w in args.verify_only.split(",")], pause_s=0.2)), flush=True)
        return
    if args.prefill_only:
        print(json.dumps(prefill_only()), flush=True)
        print(json.dumps(prefill_only(split=16)), flush=True)
        return
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src, dst = xp.Dev(nbytes=n), xp.Dev(nbytes=n)
        if xp.lib().xjh_d2d(dst.ptr, src.ptr, n):
            raise SystemExit("calibration copy failed")
        log(f"calibration: copied {n} bytes device-to-device")
        src.free()
        dst.free()
    if args.gemv_legs:
        print(json.dumps(gemv_legs()), flush=True)
        return
    r = decode_run(xp.CONFIG_4B, "synth4b", 1024, args.steps, args.warmup, seed=20261107)
    tok_s = args.steps / r["wall"]
    ms_step = r["wall"] * 1e3 / args.steps
    log(f"4B decode: {tok_s:.1f} tok/s wall, {r['gpu_ms']:.3f} ms/step GPU events")

    g_ms, g_bytes, g_launch = r["ch"].time_gemv(8)
    achieved = g_bytes / (g_ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_gemv_4b_decode.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "gemv_kernel<1,...> / gemv_cu_kernel (fused dequant-GEMV, T=1, with its prologues/tails)",
                "bytes_per_launch": round(g_bytes / g_launch), "launches_per_step": g_launch,
                "us_per_launch": round(g_ms * 1e3 / g_launch, 3), "gemv_share_of_step": round(g_ms / r["gpu_ms"], 3)}
    log(f"GEMV leg: {g_launch} launches/step, {g_bytes / 1e9:.3f} GB/step, {g_ms:.3f} ms -> {achieved:.0f} GB/s")
    # the app's sampler on the same chain (temperature 0.7, the app's default): the decode graph's last
    # launch draws the token instead of taking the argmax
    sampled = None
    if not args.greedy_only:
        r["ch"].set_sampler(0.7, np.random.default_rng(20261113).integers(0, 1 << 30, SAMPLED_STEPS).astype(np.uint32))
        t0 = time.perf_counter()
        st_toks = r["ch"].decode(SAMPLED_STEPS)
        s_wall = time.perf_counter() - t0
        sampled = {"temperature": 0.7, "steps": int(st_toks.size), "tok_s": round(st_toks.size / s_wall, 1),
                   "gpu_ms_per_step": round(r["ch"].last_decode_ms, 4),
                   "distinct_tokens": int(len(set(st_toks.tolist())))}
        log(f"4B sampled decode: {sampled}")
    r["ch"].free()
    r["st"].destroy()

    extra = {}
    if not args.no_extra:
        r8 = decode_run(xp.CONFIG_0_8B, "synth08b", 512, 256, 8, seed=20261108)
        extra["decode_0_8b"] = {"tok_s": round(256 / r8["wall"], 1), "gpu_ms_per_step": round(r8["gpu_ms"], 4),
                                "prompt": 512, "steps": 256}
        extra["decode_0_8b"]["prefill_s"] = round(r8["prefill_s"], 4)
        r8["ch"].free()
        r8["st"].destroy()
        extra["gemv_legs"] = gemv_legs()
        # the mixed-quant batch (T = 1..5: Q6_K 3584x1024, Q8_0 1024x3584, Q4_K 151936x1024) and
        # the 4B shape's gate|up and down
        extra["gemv_tokens"] = [gemv_tokens(xp.Q6_K, 3584, 1024), gemv_tokens(xp.Q8_0, 1024, 3584),
                                gemv_tokens(xp.Q4_K, 151936, 1024), gemv_tokens(xp.Q4_K, 18432, 2560),
                                gemv_tokens(xp.Q6_K, 2560, 9216)]
        extra["gemm_tokens"] = [gemm_tokens(xp.Q4_K, 18432, 2560), gemm_tokens(xp.Q6_K, 2560, 9216),
                                gemm_tokens(xp.Q4_K, 2560, 4096)]
        p2 = prefill_only(split=16)
        extra["prefill_1024_two_stages"] = {"split": "0-15 | 16-31, chunks pipelined on two streams",
                                            "prefill_s": min(p2["prefill_s"]), "first_token": p2["first_token"]}
        extra["verify_4b"] = {"ms_per_pass": verify_widths(), "decode_ms_per_step": round(ms_step, 4),
                              "note": "T tokens fed as one pass with checkpoints at position ~1024, then rolled back"}
        extra["speculative_4b"] = spec_run()
        extra["speculative_4b_mtp"] = spec_mtp_run()
        d = dropin_run()
        if d:
            extra["dropin_vtable_4b"] = d
        log(f"extra: {extra}")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(xp.CONFIG_4B, "synth4b", 16, 48, seed=20261107, at_pos=1024)
        log(f"cpu baseline: {cpu}")
        if not args.no_extra:
            extra["cpu_configs"] = cpu_configs()
            log(f"cpu configs: {extra['cpu_configs']}")

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "dtype_note": ("fp32 arithmetic; the GEMV inputs enter as 21-bit fixed point per 32-element group "
                       "(three int8 digit planes, exact int32 sub-block sums, <= 2^-21 of the group maximum per "
                       "element); the prefill GEMM's as two f16 planes per 256-element block (exact f16 products "
                       "with integer-valued weights, fp32 accumulation); KV cache fp16"),
        "data": "synthetic (random-init weights, uniform random prompt ids)",
        "config": {"workload": "greedy decode, synthetic hybrid 4B shape: hidden 2560, 32 layers (24 Gated-DeltaNet "
                               "32x128 + 8 gated GQA 16q/4kv d256), FFN 9216, vocab 151936, Q4_K_M-style "
                               "(Q4_K + Q6_K v/down/head), fp16 KV cache, 1024-token prompt, batch 1",
                   "global_batch": 1, "prompt": 1024, "parallelism": "single GPU"},
        "gpu_ms_per_step": round(r["gpu_ms"], 4),
        "prefill_1024_s": round(r["prefill_s"], 4),
        "decode_sampled_4b": sampled,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
