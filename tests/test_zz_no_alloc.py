"""xjh_gemv_noalloc (the allocation-free variant of xjh_gemv, activations in
the library's static scratch) against xjh_gemv through the C ABI: bit-identical
outputs on two calls in a row, the second with a smaller input, with and
without the residual add; sizes beyond the scratch are refused with a message."""
import ctypes as C

import numpy as np
import pytest

import xjpipe as xp

pytestmark = pytest.mark.gpu


def _weights(t, rows, k, seed):
    return xp.quantize(t, xp.fill_normal(rows * k, seed, 0.02).reshape(rows, k))


def _noalloc(w, xs, add_to=None):
    T = xs.shape[0]
    dx = xp.Dev(np.ascontiguousarray(xs, np.float32))
    dy = xp.Dev(add_to.astype(np.float32)) if add_to is not None else xp.Dev(nbytes=T * w.rows * 4)
    err = C.create_string_buffer(512)
    rc = xp.lib().xjh_gemv_noalloc(w.t, w.ptr, w.rows, w.k, dx.ptr, T, dy.ptr, int(add_to is not None), err, 512)
    assert rc == 0, err.value
    return dy.get(np.float32, (T, w.rows))


def test_gemv_noalloc_equals_gemv():
    cases = [(xp.Q6_K, 2560, 9216, 5, 3), (xp.Q4_K, 4096, 1024, 1, 4)]   # the second call is smaller
    for t, rows, k, T, seed in cases:
        print(f"noalloc gemv type {t} {rows}x{k} T={T}", flush=True)
        w = xp.DevWeight(t, _weights(t, rows, k, seed), rows, k)
        xs = xp.fill_normal(T * k, seed + 10, 1.0).reshape(T, k)
        base = xp.fill_normal(T * rows, seed + 20, 1.0).reshape(T, rows)
        for add in (None, base):
            want = xp.gemv(w, xs, add_to=add)
            got = _noalloc(w, xs, add_to=add)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        w.free()


def test_gemv_noalloc_refuses_oversized_inputs():
    err = C.create_string_buffer(512)
    # 16 tokens of 16384 inputs need about 2 MB of scratch: refused before any launch
    rc = xp.lib().xjh_gemv_noalloc(xp.Q4_K, None, 16, 16384, None, 16, None, 0, err, 512)
    assert rc == -1 and b"maximum" in err.value
