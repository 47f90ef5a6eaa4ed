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
    the kept values are distinct; the app orders equal kept values by their
    slot history (test_oracle.py::test_sampler_equal_values_keep_the_apps_order,
    slot_history_cases below)."""
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


def draw_from_order(vals, idx, temp, r30):
    """The app's draw (XJGlue.c:272-281) from kept values already in their final
    order: p_i = exp((v_i - v_0) / temp) (float difference and quotient, then
    double), the cut where the running share first reaches 0.95, r = r30 / 2^30
    times the kept mass."""
    v = np.asarray(vals, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        p = [float(np.exp(np.float64((v[i] - v[0]) / np.float32(temp)))) for i in range(len(v))]
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
            return int(idx[i])
    return int(idx[0])


def slot_history_cases():
    """(logits, kept indices in the app's final order), each order worked out by
    hand from the loop's rules: the first 40 values fill slots 0..39; a later v
    enters only when v > the minimum and takes the first slot holding it; the
    exchange sort swaps position i with a later j only when val[j] > val[i]."""
    cases = []
    lg = np.full(100, 1.5, np.float32)            # all equal: nothing enters, no swap
    cases.append((lg, list(range(40))))
    lg = np.full(41, 1.0, np.float32)
    lg[40] = 2.0                                  # 40 replaces slot 0 (first minimum)
    cases.append((lg, [40] + list(range(1, 40))))
    lg = np.concatenate([np.full(40, 1.0), np.full(40, 2.0)]).astype(np.float32)
    cases.append((lg, list(range(40, 80))))       # 40+j replaces slot j
    lg = np.where(np.arange(200) % 2, 2.0, 1.0).astype(np.float32)
    # odd indices from 41 replace the even slots in turn (slot 2m <- 41+2m), then all equal
    cases.append((lg, [i for m in range(20) for i in (41 + 2 * m, 2 * m + 1)]))
    lg = np.array([1.0, 2.0, 1.0, 2.0], np.float32)
    # i=0: swap with 1 -> [1, 0, 2, 3]; i=1: value 1 at position 1, swap with 3 -> [1, 3, 2, 0]
    cases.append((lg, [1, 3, 2, 0]))
    lg = np.array([-0.0, 0.0, 1.0], np.float32)   # -0 == +0: i=0 swaps with 2 -> [2, 1, 0]
    cases.append((lg, [2, 1, 0]))
    return cases
