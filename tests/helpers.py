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
