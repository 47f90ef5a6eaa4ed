"""Shared input builders for the tests and the golden-vector script."""
import numpy as np

import xjpipe as xp

# fp16 bit patterns for block scales: zero, subnormals, smallest normal, +-1, +-65504, others
EDGE_F16 = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x1234, 0x2E66, 0x8001, 0x5640]


def random_blocks(t, rows, k, seed):
    """Arbitrary bytes in every field of every block, with the fp16 scales drawn
    from EDGE_F16 (so every decode path, including subnormal scales, is hit)."""
    rng = np.random.default_rng(seed)
    rb = xp.row_bytes(t, k)
    blob = rng.integers(0, 256, rows * rb, dtype=np.uint8)
    if t == xp.F16:
        return np.array(EDGE_F16, np.uint16)[rng.integers(0, len(EDGE_F16), rows * k)].view(np.uint8).copy()
    if t in (xp.BF16, xp.F32):
        return blob
    _, bb = xp.BLOCK[t]
    blocks = blob.reshape(-1, bb)
    h = np.array(EDGE_F16, np.uint16)[rng.integers(0, len(EDGE_F16), (blocks.shape[0], 2))]
    hb = h.view(np.uint8).reshape(-1, 4)
    if t in (xp.Q4_K, xp.Q5_K):
        blocks[:, 0:4] = hb
    elif t == xp.Q6_K:
        blocks[:, 208:210] = hb[:, :2]
    elif t == xp.Q8_0:
        blocks[:, 0:2] = hb[:, :2]
    return blob


def np_sample(lg, temp, r30):
    """The sampler from its definition: the 40 largest by value (equal values
    in index order), p_i = exp((v_i - v_0) / temp), cut at 0.95 of the mass,
    r = r30 / 2^30 times the kept mass, first i where the running sum of p
    reaches r. This is the app's sampler (ios/App/XJGlue.c:251-282) whenever
    the kept values are distinct; the app orders equal kept values differently
    (test_oracle.py::test_sampler_equal_values_keep_the_apps_order) and the
    device sampler follows this rule."""
    if temp <= 0:
        return int(np.argmax(lg))
    order = np.argsort(-lg, kind="stable")[:40]
    v = lg[order]
    p = np.exp(((v - v[0]).astype(np.float32) / np.float32(temp)).astype(np.float64))
    tot = 0.0
    for x in p:
        tot += x
    acc, cut = 0.0, len(p)
    for i, x in enumerate(p):
        acc += x / tot
        if acc >= 0.95:
            cut = i + 1
            break
    s2 = 0.0
    for x in p[:cut]:
        s2 += x
    r = r30 / float(1 << 30) * s2
    for i in range(cut):
        r -= p[i]
        if r <= 0:
            return int(order[i])
    return int(order[0])
