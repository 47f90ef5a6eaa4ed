"""Writes the committed golden vectors of tests/golden/ from the reference CPU
path compiled from its own sources (oracle/_ref/libxjref.so, built by
`make -C oracle ref` in a container that has the reference tree).

    python tests/golden/gen_golden.py [dequant] [matmul] [tiny] [m08b]

Outputs (data only, no reference code):
  dequant_golden.npz   random blocks (every field arbitrary, fp16 scales from
                       an edge set) of F16/BF16/Q8_0/Q4_K/Q5_K/Q6_K and the
                       reference's xj_dequant_row of each
  matmul_golden.npz    reference matmul (xj_cpu.c:36-54) of quantized weights
  greedy_tiny.json     reference pipeline + greedy driver on the TINY model
                       (one stage and split 3:8), tokens and top-2 margins
  greedy_0_8b.json     0.8B-shape model, 512-token prompt, 256 greedy steps:
                       reference (fp32 KV) and oracle (fp32 and fp16 KV)
  greedy_4b.json       4B-shape model, 1024-token prompt, 512 greedy steps:
                       oracle (fp16 KV) and the reference split 0-15 | 16-31
The synthetic models are regenerated from (config, seed) by the library's
writer; each record stores the GGUF size and a checksum to detect drift.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "meta-work_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import oracle as orc  # noqa: E402
import xjpipe as xp  # noqa: E402
from helpers import random_blocks  # noqa: E402

TYPES = [xp.F16, xp.BF16, xp.Q8_0, xp.Q4_K, xp.Q5_K, xp.Q6_K]


def file_digest(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()[:16]


def gen_dequant():
    rows, k = 12, 512
    out = {}
    for t in TYPES:
        blob = random_blocks(t, rows, k, 100 + t)
        out[f"blob_{t}"] = blob
        out[f"ref_{t}"] = orc.dequant_rows(t, blob, rows, k, lib=orc.rlib())
    # fp32 -> fp16 -> fp32 of a sweep that covers rounding ties, subnormals and overflow
    vals = np.concatenate([np.array([0.0, 1.0, -2.5, 65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08,
                                     2.9802322e-08, 2.9802326e-08, 0.33325195, -1e-3, 1e6], np.float32),
                           xp.fill_normal(2000, 5, 30.0), xp.fill_normal(500, 6, 1e-5)])
    out["f16_in"] = vals.astype(np.float32)
    out["f16_bits"] = np.array([orc.rlib().ref_to_f16(float(v)) for v in vals], np.uint16)
    np.savez_compressed(os.path.join(HERE, "dequant_golden.npz"), **out)


def gen_matmul():
    out = {}
    for t, rows, k, T in [(xp.Q4_K, 64, 1024, 1), (xp.Q6_K, 48, 1024, 3), (xp.Q8_0, 40, 3584, 5), (xp.Q4_K, 24, 2560, 5)]:
        w = xp.quantize(t, xp.fill_normal(rows * k, 7 + t, 0.02).reshape(rows, k))
        x = xp.fill_normal(T * k, 8 + T, 1.0).reshape(T, k)
        out[f"w_{t}_{k}"] = w
        out[f"x_{t}_{k}"] = x
        out[f"y_{t}_{k}"] = orc.matmul(t, w, k, rows, x, ref=True)
    np.savez_compressed(os.path.join(HERE, "matmul_golden.npz"), **out)


def model_record(path, cfg, name):
    return {"config": name, "seed": cfg.seed, "bytes": os.path.getsize(path), "sha256_16": file_digest(path)}


def gen_tiny():
    path = "/tmp/xj_golden_tiny.gguf"
    xp.write_model(path, xp.TINY)
    prompt = np.random.default_rng(20261107).integers(0, xp.TINY.n_vocab, 40).astype(np.int32)
    rec = model_record(path, xp.TINY, "TINY")
    rec["prompt"] = prompt.tolist()
    for split in (0, 3):
        toks, mg = orc.ref_greedy(path, prompt, 64, split=split, n_ctx=256, max_batch=8)
        rec[f"ref_split{split}"] = {"tokens": toks.tolist(), "margins": [float(v) for v in mg]}
    with open(os.path.join(HERE, "greedy_tiny.json"), "w") as f:
        json.dump(rec, f)


def gen_m08b():
    path = "/tmp/xj_golden_08b.gguf"
    t = time.time()
    xp.write_model(path, xp.CONFIG_0_8B)
    print(f"0.8B model written in {time.time() - t:.1f} s", flush=True)
    cfg = xp.CONFIG_0_8B
    prompt = np.random.default_rng(20261108).integers(0, cfg.n_vocab, 512).astype(np.int32)
    rec = model_record(path, cfg, "CONFIG_0_8B")
    rec["prompt_seed"] = 20261108
    rec["n_prompt"], rec["n_gen"], rec["n_ctx"], rec["max_batch"] = 512, 256, 1024, 8
    m = xp.Model(path)
    for kv in (True, False):
        t = time.time()
        st = orc.CpuStage(m.ptr, 0, cfg.n_layer, 1024, 8, True, kv_f16=kv)
        toks, mg = orc.greedy([st], prompt, 256)
        st.destroy()
        rec["oracle_kvf16" if kv else "oracle_kvf32"] = {"tokens": toks.tolist(), "margins": [float(v) for v in mg]}
        print(f"oracle kv_f16={kv}: {time.time() - t:.1f} s", flush=True)
    t = time.time()
    toks, mg = orc.ref_greedy(path, prompt, 256, split=0, n_ctx=1024, max_batch=8)
    rec["ref_kvf32"] = {"tokens": toks.tolist(), "margins": [float(v) for v in mg]}
    print(f"reference: {time.time() - t:.1f} s", flush=True)
    with open(os.path.join(HERE, "greedy_0_8b.json"), "w") as f:
        json.dump(rec, f)


def gen_m4b():
    """4B-shape model, 1024-token prompt, 512 greedy tokens: oracle with the fp16
    KV cache (the GPU's parity target) and the reference itself (fp32 KV)."""
    path = "/tmp/xj_golden_4b.gguf"
    t = time.time()
    xp.write_model(path, xp.CONFIG_4B)
    print(f"4B model written in {time.time() - t:.1f} s", flush=True)
    cfg = xp.CONFIG_4B
    prompt = np.random.default_rng(20261107).integers(0, cfg.n_vocab, 1024).astype(np.int32)
    rec = model_record(path, cfg, "CONFIG_4B")
    rec["prompt_seed"] = 20261107
    rec["n_prompt"], rec["n_gen"], rec["n_ctx"], rec["max_batch"] = 1024, 512, 2048, 8
    m = xp.Model(path)
    t = time.time()
    st = orc.CpuStage(m.ptr, 0, cfg.n_layer, 2048, 8, True, kv_f16=True)
    toks, mg = orc.greedy([st], prompt, 512)
    st.destroy()
    rec["oracle_kvf16"] = {"tokens": toks.tolist(), "margins": [float(v) for v in mg]}
    print(f"oracle kv_f16: {time.time() - t:.1f} s", flush=True)
    with open(os.path.join(HERE, "greedy_4b.json"), "w") as f:
        json.dump(rec, f)
    t = time.time()
    toks, mg = orc.ref_greedy(path, prompt, 512, split=16, n_ctx=2048, max_batch=8)
    rec["ref_kvf32_split16"] = {"tokens": toks.tolist(), "margins": [float(v) for v in mg]}
    print(f"reference (layers 0-15 | 16-31): {time.time() - t:.1f} s", flush=True)
    with open(os.path.join(HERE, "greedy_4b.json"), "w") as f:
        json.dump(rec, f)


if __name__ == "__main__":
    if not orc.ref_available():
        sys.exit("oracle/_ref/libxjref.so is not built: run `make -C oracle ref` where the reference sources exist")
    what = sys.argv[1:] or ["dequant", "matmul", "tiny", "m08b"]
    for w in what:
        t = time.time()
        {"dequant": gen_dequant, "matmul": gen_matmul, "tiny": gen_tiny, "m08b": gen_m08b, "m4b": gen_m4b}[w]()
        print(f"{w}: {time.time() - t:.1f} s", flush=True)
