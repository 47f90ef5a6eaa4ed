"""ctypes bindings of the oracle (oracle/_build/libxjoracle.so) and, when it was
built in this container, of the reference compiled from source
(oracle/_ref/libxjref.so).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the checker or the timed baseline,
never as part of the product.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.normpath(os.path.join(HERE, "..", "meta-work_amd")))
import xjpipe as xp  # noqa: E402  (ABI struct definitions only)

ORACLE_LIB = os.path.join(HERE, "_build", "libxjoracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libxjref.so")
REF_NATIVE_LIB = os.path.join(HERE, "_ref", "libxjref_native.so")
ERR = 512

_o = None
_r = {}


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def olib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError(f"{ORACLE_LIB} not built; run __graft_entry__.build()")
        L = C.CDLL(ORACLE_LIB)
        P, I, I64, U32, F, S, CP = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_float, C.c_size_t, C.c_char_p
        PS = C.POINTER(xp.XjStage)
        _sig(L, "xjo_f16", F, C.c_uint16)
        _sig(L, "xjo_to_f16", C.c_uint16, F)
        _sig(L, "xjo_row_bytes", C.c_uint64, U32, I64)
        _sig(L, "xjo_dequant_row", None, U32, P, P, I64)
        _sig(L, "xjo_matmul", None, U32, P, I64, I64, P, P, I)
        _sig(L, "xjo_rmsnorm", None, P, P, P, I, F)
        _sig(L, "xjo_l2norm", None, P, I, F)
        _sig(L, "xjo_rope", None, P, I, I, F)
        _sig(L, "xjo_embed", None, C.POINTER(xp.XjModel), C.c_int32, P)
        _sig(L, "xjo_stage_new", PS, C.POINTER(xp.XjModel), I, I, I, I, C.c_bool, I, CP, S)
        _sig(L, "xjo_greedy", I, C.POINTER(PS), I, P, I, I, P, P, CP, S)
        _sig(L, "xjo_argmax", I, P, I)
        _sig(L, "xjo_delta_recurrent", None, I, I, I, P, P, P, P, P, F, P, P)
        _sig(L, "xjo_conv_silu", None, I, I, P, P, P)
        _sig(L, "xjo_sample", I, P, I, F, U32)
        _sig(L, "xjo_sampler_cb", I, P, P, I)
        _sig(L, "xjo_utf8_emit", I, P, P, I, P)
        _sig(L, "xjo_swiglu", None, S, P, P)
        _sig(L, "xjo_delta_step", None, I, I, I, F, F, P, P, P, P, P, P, P, P, P, P)
        _sig(L, "xjo_attn_decode", None, I, I, I, I, I, F, F, I, I, P, P, P, P, P, P, P, P)
        _sig(L, "xjo_abi_offsets", I, C.POINTER(C.c_long), I)
        _o = L
    return _o


def ref_available(native=False):
    return os.path.exists(REF_NATIVE_LIB if native else REF_LIB)


def rlib(native=False):
    key = "native" if native else "v3"
    if key not in _r:
        path = REF_NATIVE_LIB if native else REF_LIB
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built (needs the reference sources; see oracle/Makefile)")
        L = C.CDLL(path)
        P, I, I64, U32, F, S, CP = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_float, C.c_size_t, C.c_char_p
        PS = C.POINTER(xp.XjStage)
        PM = C.POINTER(xp.XjModel)
        _sig(L, "ref_dequant_row", None, U32, P, P, I64)
        _sig(L, "ref_to_f16", C.c_uint16, F)
        _sig(L, "ref_f16", F, C.c_uint16)
        _sig(L, "ref_row_bytes", C.c_uint64, U32, I64)
        _sig(L, "ref_matmul", None, U32, P, I64, I64, P, P, I)
        _sig(L, "ref_rmsnorm", None, P, P, P, I, F)
        _sig(L, "ref_rope", None, P, I, I, F)
        _sig(L, "ref_model_load", PM, CP, CP, S)
        _sig(L, "ref_model_free", None, PM)
        _sig(L, "ref_model_load_layers", PM, CP, I, I, C.c_bool, CP, S)
        _sig(L, "ref_model_ranges", I, PM, I, I, C.c_bool, C.POINTER(C.c_uint64), I)
        _sig(L, "ref_model_attach_mtp", I, PM, CP, CP, S)
        _sig(L, "ref_model_mtp_range", I, CP, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), CP, S)
        _sig(L, "ref_stage_new", PS, PM, I, I, I, I, C.c_bool, CP, S)
        _sig(L, "ref_embed", None, PM, C.c_int32, P)
        _sig(L, "ref_greedy", I, PM, I, I, I, P, I, I, P, P, CP, S)
        _sig(L, "ref_abi_offsets", I, C.POINTER(C.c_long), I)
        _sig(L, "ref_spec_run", I, PM, PS, PS, PS, I, P, I, I, P, I, I, P, C.POINTER(C.c_long), P, I,
             C.POINTER(C.c_int), CP, S)
        _sig(L, "ref_spec_run_s", I, PM, PS, PS, PS, I, P, I, I, P, I, I, P, P, P, C.POINTER(C.c_long), P, I,
             C.POINTER(C.c_int), CP, S)
        _r[key] = L
    return _r[key]


class XjoSampler(C.Structure):
    _fields_ = [("temp", C.c_float), ("rand30", C.c_void_p), ("n", C.c_int), ("used", C.c_int)]


def ref_spec_run(model_ptr, a, b, mtp, k, prompt, n_gen, oracle=None, oracle_miss=0, drafts=False, sampler=None):
    """The reference's own pipeline + speculative driver over the given stage
    pointers (any backend behind the xj_stage vtable; b and mtp may be None),
    greedy, or with sampler = (temperature, rand30 numbers) the app's sampler
    (the oracle's restatement, xjo_sampler_cb) drawing one number per call.
    Stops after an end token, as xjpipe-host does (the token is kept).
    Returns (tokens, (verify steps, drafted, accepted)) and, with drafts, the
    MTP stage's proposals in order as a third item; with a sampler, the count
    of numbers drawn as the last item."""
    PS = C.POINTER(xp.XjStage)
    p = np.ascontiguousarray(prompt, np.int32)
    o = np.ascontiguousarray(oracle, np.int32) if oracle is not None else None
    out = np.empty(n_gen, np.int32)
    st = (C.c_long * 3)()
    cap = 4 * n_gen + 4
    log = np.full(cap, -1, np.int32)
    nd = C.c_int(0)
    err = C.create_string_buffer(ERR)
    if sampler is None:
        rc = rlib().ref_spec_run(C.cast(model_ptr, C.POINTER(xp.XjModel)), C.cast(a, PS), C.cast(b, PS) if b else None,
                                 C.cast(mtp, PS) if mtp else None, k, _ptr(p), len(p), n_gen,
                                 _ptr(o) if o is not None else None, len(o) if o is not None else 0, oracle_miss,
                                 _ptr(out), st, _ptr(log), cap, C.byref(nd), err, ERR)
    else:
        r = np.ascontiguousarray(sampler[1], np.uint32)
        ctx = XjoSampler(float(sampler[0]), _ptr(r), len(r), 0)
        cb = C.cast(olib().xjo_sampler_cb, C.c_void_p)
        rc = rlib().ref_spec_run_s(C.cast(model_ptr, C.POINTER(xp.XjModel)), C.cast(a, PS),
                                   C.cast(b, PS) if b else None, C.cast(mtp, PS) if mtp else None, k, _ptr(p), len(p),
                                   n_gen, _ptr(o) if o is not None else None, len(o) if o is not None else 0,
                                   oracle_miss, cb, C.byref(ctx), _ptr(out), st, _ptr(log), cap, C.byref(nd), err, ERR)
    if rc < 0:
        raise RuntimeError(err.value.decode())
    res = (out[:rc], (st[0], st[1], st[2]))
    if drafts:
        res = res + (log[:nd.value],)
    return res + (ctx.used,) if sampler is not None else res


# ---------------------------------------------------------------- oracle --

def f16_to_f32(h):
    return olib().xjo_f16(int(h))


def f32_to_f16(f):
    return olib().xjo_to_f16(float(f))


def dequant_rows(t, blob, rows, k, lib=None):
    L = lib or olib()
    fn = L.xjo_dequant_row if lib is None else L.ref_dequant_row
    rb = xp.row_bytes(t, k)
    blob = np.ascontiguousarray(blob, np.uint8)
    out = np.empty((rows, k), np.float32)
    for r in range(rows):
        fn(t, blob[r * rb:].ctypes.data_as(C.c_void_p), out[r].ctypes.data_as(C.c_void_p), k)
    return out


def matmul(t, blob, K, N, x, ref=False):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    y = np.empty((x.shape[0], N), np.float32)
    blob = np.ascontiguousarray(blob, np.uint8)
    f = rlib().ref_matmul if ref else olib().xjo_matmul
    f(t, _ptr(blob), K, N, _ptr(x), _ptr(y), x.shape[0])
    return y


def rmsnorm(x, w, eps, ref=False):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    f = rlib().ref_rmsnorm if ref else olib().xjo_rmsnorm
    f(_ptr(out), _ptr(x), _ptr(np.ascontiguousarray(w, np.float32)) if w is not None else None, x.size, eps)
    return out


def rope(v, n_rot, pos, base, ref=False):
    v = np.array(v, np.float32)
    f = rlib().ref_rope if ref else olib().xjo_rope
    f(_ptr(v), n_rot, pos, base)
    return v


def sample(lg, temp, rand30):
    lg = np.ascontiguousarray(lg, np.float32)
    return olib().xjo_sample(_ptr(lg), lg.size, temp, int(rand30))


class Utf8Emit:
    """The app's UTF-8 streaming (xjo_utf8_emit): emit(piece) returns the bytes
    the app would pass to its callback for that piece (b"" when none)."""

    def __init__(self):
        self._st = C.create_string_buffer(12)   # xjo_utf8: char[8] + int

    def emit(self, piece):
        piece = bytes(piece)
        out = C.create_string_buffer(8 + 256)
        n = olib().xjo_utf8_emit(self._st, piece, len(piece), out)
        return out.raw[:n]


def swiglu(g, u):
    g = np.array(g, np.float32)
    olib().xjo_swiglu(g.size, _ptr(g), _ptr(np.ascontiguousarray(u, np.float32)))
    return g


def conv_silu(x, w, state, ck_n=0):
    """Tokens of x [T][C] in order through xjo_conv_silu; returns (out, state,
    the state after each of the first ck_n tokens)."""
    x = np.array(x, np.float32)
    st = np.array(state, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    T, Cn = x.shape
    K = w.shape[1]
    ck = np.empty((ck_n, Cn, K - 1), np.float32)
    for t in range(T):
        olib().xjo_conv_silu(Cn, K, _ptr(x[t]), _ptr(w), _ptr(st))
        if t < ck_n:
            ck[t] = st
    return x, st, ck


def attn_decode(qg, k, v, q_norm, k_norm, kc, vc, n_past, n_rot, base, eps, kv_f16=True):
    """xjo_attn_decode on float caches kc, vc [n_ctx][Hkv*D] (copies updated and
    returned); qg [T][H][2D], k, v [T][Hkv][D]. Returns (out [T][H*D], kc, vc)."""
    qg = np.ascontiguousarray(qg, np.float32)
    T, H, D2 = qg.shape
    D = D2 // 2
    Hkv = k.shape[1]
    k = np.array(k, np.float32)
    kc, vc = np.array(kc, np.float32), np.array(vc, np.float32)
    out = np.empty((T, H * D), np.float32)
    olib().xjo_attn_decode(T, H, Hkv, D, n_rot, base, eps, n_past, int(kv_f16), _ptr(qg), _ptr(k),
                           _ptr(np.ascontiguousarray(v, np.float32)), _ptr(np.ascontiguousarray(q_norm, np.float32)),
                           _ptr(np.ascontiguousarray(k_norm, np.float32)), _ptr(kc), _ptr(vc), _ptr(out))
    return out, kc, vc


def delta_step(qkv, k_off, v_off, beta_raw, alpha_raw, dt, A, Hk, Hv, S, eps, qscale, state, ck_n=0):
    """Tokens of qkv [T][stride] in order through xjo_delta_step; returns (out
    [T][Hv*S], state, the state after each of the first ck_n tokens)."""
    qkv = np.array(qkv, np.float32)
    T = qkv.shape[0]
    st = np.array(state, np.float32)
    beta_raw, alpha_raw = np.ascontiguousarray(beta_raw, np.float32), np.ascontiguousarray(alpha_raw, np.float32)
    dt, A = np.ascontiguousarray(dt, np.float32), np.ascontiguousarray(A, np.float32)
    out = np.empty((T, Hv * S), np.float32)
    ck = np.empty((ck_n, Hv, S, S), np.float32)
    for t in range(T):
        r = qkv[t]
        base = r.ctypes.data
        olib().xjo_delta_step(Hk, Hv, S, eps, qscale, C.c_void_p(base), C.c_void_p(base + 4 * k_off),
                              C.c_void_p(base + 4 * v_off), _ptr(beta_raw[t]), _ptr(alpha_raw[t]), _ptr(dt), _ptr(A),
                              _ptr(st), _ptr(out[t]), _ptr(ck[t]) if t < ck_n else None)
    return out, st, ck


def delta_recurrent(q, k, v, decay, beta, state, qscale):
    T, H, S = q.shape
    st = np.ascontiguousarray(state, np.float32).copy()
    out = np.empty((T, H, S), np.float32)
    args = [np.ascontiguousarray(a, np.float32) for a in (q, k, v, decay, beta)]
    olib().xjo_delta_recurrent(H, S, T, *[_ptr(a) for a in args], qscale, _ptr(st), _ptr(out))
    return out, st


def abi_offsets(ref=False):
    buf = (C.c_long * 256)()
    n = (rlib().ref_abi_offsets if ref else olib().xjo_abi_offsets)(buf, 256)
    return list(buf[:n])


class CpuStage:
    """A CPU stage behind the xj_stage vtable: the oracle restatement (kv_f16 selects
    the fp16 KV cache) or, with ref=True, the reference's own xj_cpu_stage_new."""

    def __init__(self, model_ptr, l0, l1, n_ctx, max_batch, has_head, kv_f16=False, ref=False):
        err = C.create_string_buffer(ERR)
        if ref:
            self.ptr = rlib().ref_stage_new(model_ptr, l0, l1, n_ctx, max_batch, has_head, err, ERR)
        else:
            self.ptr = olib().xjo_stage_new(model_ptr, l0, l1, n_ctx, max_batch, has_head, int(kv_f16), err, ERR)
        if not self.ptr:
            raise RuntimeError(err.value.decode())
        self.E = model_ptr.contents.hp.n_embd
        self.V = model_ptr.contents.hp.n_vocab

    @property
    def s(self):
        return self.ptr.contents

    @property
    def n_past(self):
        return self.ptr.contents.n_past

    def forward(self, x):
        err = C.create_string_buffer(ERR)
        rc = self.s.forward(self.ptr, x.ctypes.data_as(C.POINTER(C.c_float)), x.shape[0], err, ERR)
        if rc:
            raise RuntimeError(err.value.decode())
        return x

    def logits(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty((x.shape[0], self.V), np.float32)
        err = C.create_string_buffer(ERR)
        rc = self.s.logits(self.ptr, x.ctypes.data_as(C.POINTER(C.c_float)), x.shape[0],
                           out.ctypes.data_as(C.POINTER(C.c_float)), err, ERR)
        if rc:
            raise RuntimeError(err.value.decode())
        return out

    def rollback(self, n_past):
        err = C.create_string_buffer(ERR)
        if self.s.rollback(self.ptr, n_past, err, ERR):
            raise RuntimeError(err.value.decode())

    def set_keep(self, k):
        self.ptr.contents.keep = k

    def reset(self):
        self.s.reset(self.ptr)

    def destroy(self):
        if self.ptr:
            self.s.destroy(self.ptr)
            self.ptr = None


def embed(model_ptr, token):
    out = np.empty(model_ptr.contents.hp.n_embd, np.float32)
    olib().xjo_embed(model_ptr, token, _ptr(out))
    return out


def greedy(stages, prompt, n_gen):
    """xjo_greedy over oracle CpuStages; returns (tokens, top1-top2 margins)."""
    arr = (C.POINTER(xp.XjStage) * len(stages))(*[s.ptr for s in stages])
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.empty(n_gen, np.int32)
    mg = np.empty(n_gen, np.float32)
    err = C.create_string_buffer(ERR)
    rc = olib().xjo_greedy(arr, len(stages), _ptr(p), len(p), n_gen, _ptr(out), _ptr(mg), err, ERR)
    if rc:
        raise RuntimeError(err.value.decode())
    return out, mg


def ref_greedy(path, prompt, n_gen, split=0, n_ctx=1024, max_batch=8):
    """The reference's own pipeline + greedy driver on its own loader (fp32 KV)."""
    L = rlib()
    err = C.create_string_buffer(ERR)
    m = L.ref_model_load(path.encode(), err, ERR)
    if not m:
        raise RuntimeError(err.value.decode())
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.empty(n_gen, np.int32)
    mg = np.empty(n_gen, np.float32)
    rc = L.ref_greedy(m, split, n_ctx, max_batch, _ptr(p), len(p), n_gen, _ptr(out), _ptr(mg), err, ERR)
    L.ref_model_free(m)
    if rc:
        raise RuntimeError(err.value.decode())
    return out, mg
