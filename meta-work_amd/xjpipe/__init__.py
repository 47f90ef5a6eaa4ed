"""Python bindings of libxjhip.so, the MI355X backend of the xiaoju-pipe token loop.

Everything here is a thin ctypes layer over the C ABI declared in
include/xj_hip.h; the compute runs in the hand-written gfx950 kernels of the
library. Importing this module never falls back to anything else: if the
library is missing it raises.

    import xjpipe as xp
    m = xp.Model(path)                       # xjh_model_load
    a = xp.HipStage(m, 0, m.hp.n_layer, n_ctx=1024, max_batch=8, has_head=True)
    x = m.embed_host(token)  ...             # or a device chain:
    c = xp.Chain([a]); c.eval(prompt); toks = c.decode(256)
"""
import ctypes as C
import os

import numpy as np

from .configs import CONFIG_0_8B, CONFIG_0_8B_MTP, CONFIG_4B, TINY, TINY_DRAFT, TINY_MTP, SynthConfig  # noqa: F401

HERE = os.path.dirname(os.path.abspath(__file__))
# XJ_HIP_LIB selects another build of the same library (e.g. a tuning variant)
LIB_PATH = os.environ.get("XJ_HIP_LIB") or os.path.normpath(os.path.join(HERE, "..", "_build", "libxjhip.so"))

# ggml type ids (include/xj_abi.h)
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 8, 12, 13, 14, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", BF16: "BF16"}
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def row_bytes(t, k):
    n, b = BLOCK[t]
    return (k // n) * b


# ------------------------------------------------------------------ ABI --

class XjW(C.Structure):
    _fields_ = [("data", C.c_void_p), ("file_off", C.c_uint64), ("nbytes", C.c_uint64),
                ("type", C.c_uint32), ("ne0", C.c_int64), ("ne1", C.c_int64)]


_LAYER_W = ["attn_norm", "post_norm", "wqkv", "wq", "wk", "wv", "wo", "q_norm", "k_norm",
            "ssm_qkv", "ssm_gate", "ssm_conv1d", "ssm_dt", "ssm_a", "ssm_beta", "ssm_alpha", "ssm_norm", "ssm_out",
            "ffn_gate", "ffn_up", "ffn_down"]


class XjLayer(C.Structure):
    _fields_ = [("recurrent", C.c_bool)] + [(n, XjW) for n in _LAYER_W]


class XjHparams(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_ff", "n_vocab", "n_head", "n_head_kv", "head_dim",
                                       "n_rot")] + \
               [("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n, C.c_int) for n in ("conv_k", "d_inner", "s_k", "h_k", "h_v", "s_v", "key_dim", "conv_dim",
                                       "full_attn_interval")] + \
               [("eos", C.c_uint32), ("eot", C.c_uint32)]


class XjModel(C.Structure):
    _fields_ = [("gguf", C.c_void_p), ("hp", XjHparams), ("tok_embd", XjW), ("output_norm", XjW), ("output", XjW),
                ("layers", XjLayer * 128), ("fingerprint", C.c_uint64), ("has_mtp", C.c_bool),
                ("mtp_eh", XjW), ("mtp_enorm", XjW), ("mtp_hnorm", XjW), ("mtp_head_norm", XjW), ("mtp_gguf", C.c_void_p)]


class XjStage(C.Structure):
    pass


_FWD = C.CFUNCTYPE(C.c_int, C.POINTER(XjStage), C.POINTER(C.c_float), C.c_int, C.c_char_p, C.c_size_t)
_LOG = C.CFUNCTYPE(C.c_int, C.POINTER(XjStage), C.POINTER(C.c_float), C.c_int, C.POINTER(C.c_float), C.c_char_p,
                   C.c_size_t)
_RB = C.CFUNCTYPE(C.c_int, C.POINTER(XjStage), C.c_int, C.c_char_p, C.c_size_t)
_VOID = C.CFUNCTYPE(None, C.POINTER(XjStage))
XjStage._fields_ = [("m", C.POINTER(XjModel)), ("l0", C.c_int), ("l1", C.c_int), ("n_ctx", C.c_int),
                    ("max_batch", C.c_int), ("n_past", C.c_int), ("has_head", C.c_bool), ("mtp", C.c_bool),
                    ("backend", C.c_char_p), ("keep", C.c_int), ("ck_start", C.c_int), ("ck_T", C.c_int),
                    ("forward", _FWD), ("logits", _LOG), ("rollback", _RB), ("reset", _VOID), ("destroy", _VOID),
                    ("impl", C.c_void_p)]


class XjhSpecStats(C.Structure):
    _fields_ = [("n_steps", C.c_long), ("n_drafted", C.c_long), ("n_accepted", C.c_long), ("acc_at", C.c_long * 4),
                ("t_total_ms", C.c_double), ("t_draft_ms", C.c_double), ("n_overlap", C.c_long),
                ("n_overlap_held", C.c_long)]


class XjsConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_ff", "n_vocab", "n_head", "n_head_kv", "head_dim",
                                       "n_rot")] + \
               [("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n, C.c_int) for n in ("conv_k", "s_k", "h_k", "h_v", "full_attn_interval")] + \
               [(n, C.c_uint32) for n in ("type_default", "type_embd", "type_out", "type_v", "type_down")] + \
               [("w_std", C.c_float), ("seed", C.c_uint64), ("nextn", C.c_int), ("eos_id", C.c_int32),
                ("eot_id", C.c_int32)]


# -------------------------------------------------------------- library --

_lib = None
ERR = 512


class XjError(RuntimeError):
    pass


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def lib():
    """Load libxjhip.so (built by __graft_entry__.build()); raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise XjError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    L = C.CDLL(LIB_PATH)
    P, I, I64, U32, U64, F, D, S = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_float, C.c_double, C.c_size_t
    CP = C.c_char_p
    PS = C.POINTER(XjStage)
    _sig(L, "xj_hip_stage_new", PS, C.POINTER(XjModel), I, I, I, I, C.c_bool, CP, S)
    _sig(L, "xj_hip_device_name", CP)
    _sig(L, "xj_hip_tune_note", CP)
    _sig(L, "xj_hip_stage_state_bytes", U64, C.POINTER(XjModel), I, I, I, I)
    _sig(L, "xj_hip_stage_snapshot", I, PS, I, CP, S)
    _sig(L, "xj_hip_stage_restore", I, PS, I, I, CP, S)
    _sig(L, "xj_hip_stage_fill_kv", I, PS, I, C.c_uint16, CP, S)
    _sig(L, "xjh_type_block", I, U32, C.POINTER(I))
    _sig(L, "xjh_row_bytes", U64, U32, I64)
    _sig(L, "xjh_type_name", CP, U32)
    _sig(L, "xjh_model_load", C.POINTER(XjModel), CP, CP, S)
    _sig(L, "xjh_model_free", None, C.POINTER(XjModel))
    _sig(L, "xjh_model_load_layers", C.POINTER(XjModel), CP, C.c_int, C.c_int, C.c_bool, CP, S)
    _sig(L, "xjh_model_ranges", C.c_int, C.POINTER(XjModel), C.c_int, C.c_int, C.c_bool, C.POINTER(C.c_uint64), C.c_int)
    _sig(L, "xjh_model_layer_bytes", C.c_uint64, C.POINTER(XjModel), C.c_int, C.c_int)
    _sig(L, "xjh_model_attach_mtp", I, C.POINTER(XjModel), CP, CP, S)
    _sig(L, "xjh_model_mtp_range", I, CP, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), CP, S)
    _sig(L, "xjs_fill_normal", None, P, I64, U64, F)
    _sig(L, "xjs_tensor_seed", U64, U64, CP)
    _sig(L, "xjs_quantize", I, U32, P, I64, I64, P, CP, S)
    _sig(L, "xjs_write_model", I64, CP, C.POINTER(XjsConfig), CP, S)
    _sig(L, "xjh_chain_new", P, C.POINTER(PS), I, CP, S)
    _sig(L, "xjh_chain_free", None, P)
    _sig(L, "xjh_chain_eval", I, P, P, I, I, I, P, P, CP, S)
    _sig(L, "xjh_chain_decode", I, P, I, P, CP, S)
    _sig(L, "xjh_chain_last_token", I, P)
    _sig(L, "xjh_chain_set_sampler", I, P, F, P, I, CP, S)
    _sig(L, "xjh_chain_sampler_used", I, P)
    _sig(L, "xjh_chain_rollback", I, P, I, CP, S)
    _sig(L, "xjh_chain_reset", None, P)
    _sig(L, "xjh_chain_n_past", I, P)
    _sig(L, "xjh_chain_last_decode_ms", D, P)
    _sig(L, "xjh_chain_time_gemv", I, P, I, C.POINTER(D), C.POINTER(D), C.POINTER(I), CP, S)
    _sig(L, "xjh_spec_generate", I, P, P, I, I, P, I, I, P, C.POINTER(XjhSpecStats), CP, S)
    _sig(L, "xjh_spec_generate_mtp", I, P, PS, I, P, I, I, P, I, I, P, C.POINTER(XjhSpecStats), P, I, CP, S)
    _sig(L, "xjh_malloc", P, S)
    _sig(L, "xjh_free", None, P)
    _sig(L, "xjh_h2d", I, P, P, S)
    _sig(L, "xjh_d2h", I, P, P, S)
    _sig(L, "xjh_d2d", I, P, P, S)
    _sig(L, "xjh_sync", I)
    _sig(L, "xjh_last_error", CP)
    _sig(L, "xjh_upload_weight", P, U32, P, I64, I64, CP, S)
    _sig(L, "xjh_dequant", I, U32, P, I64, I64, I64, I64, P, CP, S)
    _sig(L, "xjh_gemv", I, U32, P, I64, I64, P, I, P, I, CP, S)
    _sig(L, "xjh_gemv_noalloc", I, U32, P, I64, I64, P, I, P, I, CP, S)
    _sig(L, "xjh_gemm", I, U32, P, I64, I64, P, I, P, I, CP, S)
    _sig(L, "xjh_gemv_time", D, U32, C.POINTER(P), I, I64, I64, P, I, P, I, CP, S)
    _sig(L, "xjh_gemm_time", D, U32, C.POINTER(P), I, I64, I64, P, I, P, I, CP, S)
    _sig(L, "xjh_norm", I, I, P, P, I, I, F, P, CP, S)
    _sig(L, "xjh_argmax", I, P, I, I, P, CP, S)
    _sig(L, "xjh_delta_recurrent", I, I, I, I, P, P, P, P, P, F, P, P, CP, S)
    _sig(L, "xjh_delta_chunked", I, I, I, I, I, P, P, P, P, P, F, P, P, CP, S)
    _sig(L, "xjh_swiglu", I, P, P, I64, CP, S)
    _sig(L, "xjh_sample", I, P, I, I, F, P, P, CP, S)
    _sig(L, "xjh_utf8_reset", None, P)
    _sig(L, "xjh_utf8_emit", I, P, P, I, P, P)
    _sig(L, "xjh_delta_step", I, P, I, I, I, P, P, P, P, I, I, I, I, F, F, P, P, P, I, CP, S)
    _sig(L, "xjh_rope", I, P, I, I, I64, I64, I, I, F, CP, S)
    _sig(L, "xjh_conv_silu", I, P, P, P, I, I, I, P, I, CP, S)
    _sig(L, "xjh_attn_decode", I, I, I, I, I, I, F, F, I, I, P, P, P, P, P, P, P, P, CP, S)
    _lib = L
    return L


def _err():
    return C.create_string_buffer(ERR)


def _check(rc, err, what):
    if rc != 0:
        raise XjError(f"{what}: {err.value.decode(errors='replace')}")


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


# ----------------------------------------------------- synthetic models --

def config_struct(cfg):
    c = XjsConfig()
    for name, _ in XjsConfig._fields_:
        setattr(c, name, getattr(cfg, name))
    return c


def write_model(path, cfg):
    """Write the synthetic qwen35 GGUF of `cfg` to `path`; returns its size in bytes."""
    err = _err()
    c = config_struct(cfg)
    n = lib().xjs_write_model(path.encode(), C.byref(c), err, ERR)
    if n < 0:
        raise XjError(err.value.decode())
    return n


def cached_model(cfg, name):
    """Path of the synthetic model for cfg, written once per machine under
    $XJ_MODEL_DIR (default /tmp/xj_models) and reused afterwards."""
    import time
    d = os.environ.get("XJ_MODEL_DIR", "/tmp/xj_models")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, f"{name}_{cfg.seed}.gguf")
    if not os.path.exists(path):
        t = time.time()
        tmp = f"{path}.{os.getpid()}.tmp"
        n = write_model(tmp, cfg)
        os.replace(tmp, path)
        import sys
        print(f"wrote {path} ({n / 1e9:.2f} GB) in {time.time() - t:.1f} s", file=sys.stderr, flush=True)
    return path


def fill_normal(n, seed, std=1.0):
    out = np.empty(n, np.float32)
    lib().xjs_fill_normal(_ptr(out), n, seed, std)
    return out


def tensor_seed(seed, name):
    return lib().xjs_tensor_seed(seed, name.encode())


def quantize(t, x):
    """Quantize a [rows][k] float32 array with the library's quantizers; returns uint8 bytes."""
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    out = np.empty(rows * row_bytes(t, k), np.uint8)
    err = _err()
    _check(lib().xjs_quantize(t, _ptr(x), rows, k, _ptr(out), err, ERR), err, "quantize")
    return out


class Model:
    """xjh_model_load: the GGUF is mmapped; weights stay on the host until a stage uploads them.
    With layers=(l0, l1): xjh_model_load_layers, only the header is read and one mapping
    covers those layers (with_io: the embedding and head as well); other weights are NULL."""

    def __init__(self, path, layers=None, with_io=False):
        err = _err()
        if layers is None:
            self.ptr = lib().xjh_model_load(path.encode(), err, ERR)
        else:
            self.ptr = lib().xjh_model_load_layers(path.encode(), int(layers[0]), int(layers[1]), bool(with_io), err, ERR)
        if not self.ptr:
            raise XjError(err.value.decode())
        self.path = path

    @property
    def m(self):
        return self.ptr.contents

    @property
    def hp(self):
        return self.ptr.contents.hp

    def close(self):
        if self.ptr:
            lib().xjh_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def ranges(self, l0, l1, include_embd=False, max_ranges=512):
        """xjh_model_ranges: merged file byte ranges [(lo, hi), ...] of layers [l0, l1)."""
        r = (C.c_uint64 * (2 * max_ranges))()
        n = lib().xjh_model_ranges(self.ptr, l0, l1, include_embd, r, max_ranges)
        return [(r[2 * i], r[2 * i + 1]) for i in range(n)]

    def attach_mtp(self, path):
        """xjh_model_attach_mtp: take the MTP layer from another GGUF of the same model."""
        err = _err()
        _check(lib().xjh_model_attach_mtp(self.ptr, path.encode(), err, ERR), err, "attach_mtp")

    def tensor_bytes(self, w):
        """Raw GGUF bytes of an XjW as a numpy uint8 view (no copy)."""
        buf = (C.c_uint8 * w.nbytes).from_address(w.data)
        return np.frombuffer(buf, np.uint8)

    def tensor_f32(self, w):
        assert w.type == F32
        return self.tensor_bytes(w).view(np.float32).reshape(w.ne1, w.ne0)


# ---------------------------------------------------------------- stage --

class HipStage:
    """xj_hip_stage_new: layers [l0, l1) (+ head) in HBM behind the xj_stage vtable."""

    def __init__(self, model, l0, l1, n_ctx, max_batch, has_head):
        err = _err()
        self.model = model
        self.ptr = lib().xj_hip_stage_new(model.ptr, l0, l1, n_ctx, max_batch, has_head, err, ERR)
        if not self.ptr:
            raise XjError(err.value.decode())

    @property
    def s(self):
        return self.ptr.contents

    @property
    def n_past(self):
        return self.ptr.contents.n_past

    def forward(self, x):
        """x: float32 [T][n_embd], updated in place (vtable forward)."""
        assert x.dtype == np.float32 and x.flags.c_contiguous
        err = _err()
        rc = self.s.forward(self.ptr, x.ctypes.data_as(C.POINTER(C.c_float)), x.shape[0], err, ERR)
        _check(rc, err, "forward")
        return x

    def logits(self, x):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        out = np.empty((T, self.model.hp.n_vocab), np.float32)
        err = _err()
        rc = self.s.logits(self.ptr, x.ctypes.data_as(C.POINTER(C.c_float)), T,
                           out.ctypes.data_as(C.POINTER(C.c_float)), err, ERR)
        _check(rc, err, "logits")
        return out

    def rollback(self, n_past):
        err = _err()
        _check(self.s.rollback(self.ptr, n_past, err, ERR), err, "rollback")

    def set_keep(self, k):
        self.ptr.contents.keep = k

    def reset(self):
        self.s.reset(self.ptr)

    def snapshot(self, slot):
        err = _err()
        _check(lib().xj_hip_stage_snapshot(self.ptr, slot, err, ERR), err, "snapshot")

    def restore(self, slot, n_past):
        err = _err()
        _check(lib().xj_hip_stage_restore(self.ptr, slot, n_past, err, ERR), err, "restore")

    def fill_kv(self, pos0, bits):
        """Test hook: the fp16 pattern `bits` in every K/V cache slot from pos0 on."""
        err = _err()
        _check(lib().xj_hip_stage_fill_kv(self.ptr, pos0, bits, err, ERR), err, "fill_kv")

    def destroy(self):
        if self.ptr:
            self.s.destroy(self.ptr)
            self.ptr = None


class Chain:
    """Device-resident pipeline over HIP stages (embedding, layers, head, argmax on the GPU)."""

    def __init__(self, stages):
        self.stages = stages
        arr = (C.POINTER(XjStage) * len(stages))(*[s.ptr for s in stages])
        err = _err()
        self.ptr = lib().xjh_chain_new(arr, len(stages), err, ERR)
        if not self.ptr:
            raise XjError(err.value.decode())
        self.V = stages[-1].model.hp.n_vocab

    def eval(self, tokens, nlog=1, keep=False, want_logits=False):
        toks = np.ascontiguousarray(tokens, np.int32)
        nl = min(nlog, len(toks)) if nlog else 0
        am = np.empty(max(nl, 1), np.int32)
        lg = np.empty((max(nl, 1), self.V), np.float32) if want_logits else None
        err = _err()
        rc = lib().xjh_chain_eval(self.ptr, _ptr(toks), len(toks), nlog, int(keep),
                                  _ptr(lg) if lg is not None else None, _ptr(am), err, ERR)
        _check(rc, err, "chain eval")
        return (am[:nl], lg[:nl]) if want_logits else am[:nl]

    def set_sampler(self, temperature, rand30=()):
        """The app's sampler for every token this chain produces (temperature <= 0: greedy),
        drawing rand30[i] / 2^30 in order, one number per token."""
        r = np.ascontiguousarray(rand30, np.uint32).reshape(-1)
        err = _err()
        _check(lib().xjh_chain_set_sampler(self.ptr, float(temperature), _ptr(r) if r.size else None, r.size, err,
                                           ERR), err, "set sampler")

    @property
    def sampler_used(self):
        return lib().xjh_chain_sampler_used(self.ptr)

    def decode(self, n):
        """Up to n tokens (greedy, or drawn by the sampler); fewer when an end token came
        (it is the last one returned)."""
        out = np.empty(max(n, 1), np.int32)
        err = _err()
        rc = lib().xjh_chain_decode(self.ptr, n, _ptr(out), err, ERR)
        _check(rc < 0, err, "chain decode")
        return out[:rc]

    @property
    def last_token(self):
        return lib().xjh_chain_last_token(self.ptr)

    @property
    def n_past(self):
        return lib().xjh_chain_n_past(self.ptr)

    @property
    def last_decode_ms(self):
        return lib().xjh_chain_last_decode_ms(self.ptr)

    def rollback(self, n_past):
        err = _err()
        _check(lib().xjh_chain_rollback(self.ptr, n_past, err, ERR), err, "chain rollback")

    def time_gemv(self, iters):
        """(ms per step, algorithmic bytes per step, launches per step) of the GEMV launches of one decode step."""
        ms, by, n = C.c_double(), C.c_double(), C.c_int()
        err = _err()
        _check(lib().xjh_chain_time_gemv(self.ptr, iters, C.byref(ms), C.byref(by), C.byref(n), err, ERR), err,
               "time_gemv")
        return ms.value, by.value, n.value

    def reset(self):
        lib().xjh_chain_reset(self.ptr)

    def free(self):
        if self.ptr:
            lib().xjh_chain_free(self.ptr)
            self.ptr = None


def spec_generate(target, draft, k, n_gen, oracle=None, oracle_miss=0):
    out = np.empty(n_gen, np.int32)
    st = XjhSpecStats()
    err = _err()
    orc = np.ascontiguousarray(oracle, np.int32) if oracle is not None else None
    rc = lib().xjh_spec_generate(target.ptr, draft.ptr, k, n_gen, _ptr(orc) if orc is not None else None,
                                 len(orc) if orc is not None else 0, oracle_miss, _ptr(out), C.byref(st), err, ERR)
    _check(rc < 0, err, "spec generate")
    return out[:rc], st


def spec_generate_mtp(target, mtp_stage, k, prompt, n_gen, oracle=None, oracle_miss=0, draft_log=False):
    """Speculative decoding with the model's MTP stage drafting k tokens; feeds the prompt itself.
    Returns (tokens, stats) or, with draft_log, (tokens, stats, drafted tokens in order)."""
    out = np.empty(n_gen, np.int32)
    st = XjhSpecStats()
    err = _err()
    p = np.ascontiguousarray(prompt, np.int32)
    orc = np.ascontiguousarray(oracle, np.int32) if oracle is not None else None
    cap = 4 * n_gen + 4
    log = np.full(cap, -1, np.int32)
    rc = lib().xjh_spec_generate_mtp(target.ptr, mtp_stage.ptr, k, _ptr(p), len(p), n_gen,
                                     _ptr(orc) if orc is not None else None, len(orc) if orc is not None else 0,
                                     oracle_miss, _ptr(out), C.byref(st), _ptr(log) if draft_log else None,
                                     cap if draft_log else 0, err, ERR)
    _check(rc < 0, err, "MTP speculative generate")
    if draft_log:
        return out[:rc], st, log[:min(st.n_drafted, cap)]
    return out[:rc], st


# --------------------------------------------------------- device memory --

class Dev:
    """A device buffer holding a numpy array's bytes."""

    def __init__(self, arr=None, nbytes=None):
        if arr is not None:
            arr = np.ascontiguousarray(arr)
            nbytes = arr.nbytes
        self.nbytes = nbytes
        self.ptr = lib().xjh_malloc(nbytes)
        if not self.ptr:
            raise XjError(lib().xjh_last_error().decode())
        if arr is not None:
            self.put(arr)

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        if lib().xjh_h2d(self.ptr, _ptr(arr), arr.nbytes):
            raise XjError("h2d copy failed")

    def get(self, dtype, shape):
        out = np.empty(shape, dtype)
        if lib().xjh_d2h(_ptr(out), self.ptr, out.nbytes):
            raise XjError("d2h copy failed")
        return out

    def free(self):
        if self.ptr:
            lib().xjh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DevWeight:
    """A GGUF tensor repacked into the kernels' device layout."""

    def __init__(self, t, blob, rows, k):
        err = _err()
        blob = np.ascontiguousarray(blob, np.uint8)
        assert blob.nbytes == rows * row_bytes(t, k)
        self.t, self.rows, self.k = t, rows, k
        self.ptr = lib().xjh_upload_weight(t, _ptr(blob), rows, k, err, ERR)
        if not self.ptr:
            raise XjError(err.value.decode())

    def free(self):
        if self.ptr:
            lib().xjh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def dequant(w, r0=0, n=None):
    n = w.rows - r0 if n is None else n
    y = Dev(nbytes=max(1, n * w.k * 4))
    err = _err()
    _check(lib().xjh_dequant(w.t, w.ptr, w.rows, w.k, r0, n, y.ptr, err, ERR), err, "dequant")
    return y.get(np.float32, (n, w.k))


def gemv(w, x, add_to=None):
    """y[t] = W x[t] on the GPU; x float32 [T][k]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w.k)
    T = x.shape[0]
    dx = Dev(x)
    dy = Dev(add_to.astype(np.float32)) if add_to is not None else Dev(nbytes=T * w.rows * 4)
    err = _err()
    _check(lib().xjh_gemv(w.t, w.ptr, w.rows, w.k, dx.ptr, T, dy.ptr, int(add_to is not None), err, ERR), err, "gemv")
    return dy.get(np.float32, (T, w.rows))


def gemm(w, x, add_to=None):
    """y[t] = W x[t] on the matrix cores (xjh_gemm); x float32 [T][k], T <= 64."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w.k)
    T = x.shape[0]
    dx = Dev(x)
    dy = Dev(add_to.astype(np.float32)) if add_to is not None else Dev(nbytes=T * w.rows * 4)
    err = _err()
    _check(lib().xjh_gemm(w.t, w.ptr, w.rows, w.k, dx.ptr, T, dy.ptr, int(add_to is not None), err, ERR), err, "gemm")
    return dy.get(np.float32, (T, w.rows))


def gemm_time(weights, x, iters):
    """Mean ms per xjh_gemm call over rotating copies (HIP events on the library stream)."""
    w0 = weights[0]
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w0.k)
    T = x.shape[0]
    dx, dy = Dev(x), Dev(nbytes=T * w0.rows * 4)
    arr = (C.c_void_p * len(weights))(*[w.ptr for w in weights])
    err = _err()
    ms = lib().xjh_gemm_time(w0.t, arr, len(weights), w0.rows, w0.k, dx.ptr, T, dy.ptr, iters, err, ERR)
    if ms < 0:
        raise XjError(err.value.decode())
    return ms


def gemv_time(weights, x, iters):
    """Mean ms per GEMV launch over rotating copies (HIP events on the library stream)."""
    w0 = weights[0]
    x = np.ascontiguousarray(x, np.float32).reshape(-1, w0.k)
    T = x.shape[0]
    dx, dy = Dev(x), Dev(nbytes=T * w0.rows * 4)
    arr = (C.c_void_p * len(weights))(*[w.ptr for w in weights])
    err = _err()
    ms = lib().xjh_gemv_time(w0.t, arr, len(weights), w0.rows, w0.k, dx.ptr, T, dy.ptr, iters, err, ERR)
    if ms < 0:
        raise XjError(err.value.decode())
    return ms


def norm(x, w, mode, eps):
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    dx, dout = Dev(x), Dev(nbytes=x.nbytes)
    dw = Dev(np.ascontiguousarray(w, np.float32)) if w is not None else None
    err = _err()
    _check(lib().xjh_norm(mode, dx.ptr, dw.ptr if dw else None, n, rows, eps, dout.ptr, err, ERR), err, "norm")
    return dout.get(np.float32, x.shape)


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None]
    dx = Dev(x)
    out = np.empty(x.shape[0], np.int32)
    err = _err()
    _check(lib().xjh_argmax(dx.ptr, x.shape[1], x.shape[0], _ptr(out), err, ERR), err, "argmax")
    return out


def delta(q, k, v, decay, beta, state, qscale, chunk=0):
    """Gated delta rule on the GPU; q,k,v [T][H][S], decay,beta [T][H], state [H][S][S].
    chunk=0 runs the recurrent kernel, chunk=64 the chunk-wise one. Returns (out, new_state)."""
    T, H, S = q.shape
    dq, dk, dv = Dev(q.astype(np.float32)), Dev(k.astype(np.float32)), Dev(v.astype(np.float32))
    dd, db = Dev(decay.astype(np.float32)), Dev(beta.astype(np.float32))
    ds, do = Dev(state.astype(np.float32)), Dev(nbytes=T * H * S * 4)
    err = _err()
    if chunk:
        rc = lib().xjh_delta_chunked(H, S, T, chunk, dq.ptr, dk.ptr, dv.ptr, dd.ptr, db.ptr, qscale, ds.ptr, do.ptr,
                                     err, ERR)
    else:
        rc = lib().xjh_delta_recurrent(H, S, T, dq.ptr, dk.ptr, dv.ptr, dd.ptr, db.ptr, qscale, ds.ptr, do.ptr,
                                       err, ERR)
    _check(rc, err, "delta")
    return do.get(np.float32, (T, H, S)), ds.get(np.float32, (H, S, S))


_PIECE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_char), C.c_int)


class Utf8Stream:
    """Streams generated text pieces as whole UTF-8 characters (xjh_utf8_emit):
    emit(piece) returns the bytes passed to the callback for that piece (b""
    when the piece ends inside a character and nothing is complete yet);
    stop_after makes the callback ask to stop (return 1) once that many
    chunks were passed."""

    def __init__(self, stop_after=None):
        self._st = C.create_string_buffer(12)   # xjh_utf8_state: char[8] + int32
        lib().xjh_utf8_reset(self._st)
        self.chunks, self.stop_after = [], stop_after

        def cb(ctx, p, n):
            self.chunks.append(C.string_at(p, n))
            return 1 if self.stop_after is not None and len(self.chunks) >= self.stop_after else 0

        self._cb = _PIECE_FN(cb)

    def emit(self, piece):
        piece = bytes(piece)
        before = len(self.chunks)
        stop = lib().xjh_utf8_emit(self._st, piece, len(piece), self._cb, None)
        return (self.chunks[before] if len(self.chunks) > before else b""), stop

    @property
    def pending(self):
        n = int.from_bytes(self._st.raw[8:12], "little", signed=True)
        return self._st.raw[:n]


def sample(logits, temperature, rand30):
    """Top-k 40 / top-p 0.95 sampling on the GPU of each row of logits [T][V] with
    rand30[t] / 2^30 as the uniform number; temperature <= 0: greedy."""
    lg = np.ascontiguousarray(logits, np.float32)
    if lg.ndim == 1:
        lg = lg[None]
    r = np.ascontiguousarray(rand30, np.uint32).reshape(-1)
    d = Dev(lg)
    out = np.empty(lg.shape[0], np.int32)
    err = _err()
    _check(lib().xjh_sample(d.ptr, lg.shape[1], lg.shape[0], temperature, _ptr(r), _ptr(out), err, ERR), err, "sample")
    return out


def swiglu(g, u):
    """silu(g) * u on the GPU (float32, any shape)."""
    g = np.ascontiguousarray(g, np.float32)
    dg, du = Dev(g), Dev(np.ascontiguousarray(u, np.float32))
    err = _err()
    _check(lib().xjh_swiglu(dg.ptr, du.ptr, g.size, err, ERR), err, "swiglu")
    return dg.get(np.float32, g.shape)


def rope(x, n_rot, pos0, base, head_stride=None):
    """NeoX RoPE on the GPU of x [T][n_heads * head_stride] (the first n_rot
    elements of each head's head_stride rotated), token t at position pos0 + t."""
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    hs = head_stride or x.shape[1]
    nh = x.shape[1] // hs
    dx = Dev(x)
    err = _err()
    _check(lib().xjh_rope(dx.ptr, T, nh, x.shape[1], hs, n_rot, pos0, base, err, ERR), err, "rope")
    return dx.get(np.float32, x.shape)


def conv_silu(x, w, state, ck_n=0):
    """Depthwise causal conv + SiLU on the GPU: x [T][C], w [C][K], state [C][K-1].
    Returns (out, new_state, checkpoints [ck_n][C][K-1])."""
    x = np.ascontiguousarray(x, np.float32)
    T, Cn = x.shape
    K = w.shape[1]
    dx, dw, ds = Dev(x), Dev(np.ascontiguousarray(w, np.float32)), Dev(np.ascontiguousarray(state, np.float32))
    dck = Dev(nbytes=max(1, ck_n * Cn * (K - 1) * 4))
    err = _err()
    _check(lib().xjh_conv_silu(dx.ptr, ds.ptr, dw.ptr, Cn, K, T, dck.ptr if ck_n else None, ck_n, err, ERR), err,
           "conv_silu")
    return (dx.get(np.float32, x.shape), ds.get(np.float32, (Cn, K - 1)),
            dck.get(np.float32, (ck_n, Cn, K - 1)) if ck_n else None)


def attn_decode(qg, k, v, q_norm, k_norm, kc, vc, n_past, n_rot, base, eps):
    """Gated GQA attention on the GPU for T tokens at n_past.. (the token loop's
    kernels). qg [T][H][2D], k, v [T][Hkv][D], kc, vc uint16 fp16 bits
    [n_ctx][Hkv*D] (updated copies are returned). Returns (out [T][H*D], kc, vc)."""
    qg = np.ascontiguousarray(qg, np.float32)
    T, H, D2 = qg.shape
    D = D2 // 2
    Hkv = k.shape[1]
    n_ctx = kc.shape[0]
    dq, dk, dv = Dev(qg), Dev(np.ascontiguousarray(k, np.float32)), Dev(np.ascontiguousarray(v, np.float32))
    dqn, dkn = Dev(np.ascontiguousarray(q_norm, np.float32)), Dev(np.ascontiguousarray(k_norm, np.float32))
    dkc, dvc = Dev(np.ascontiguousarray(kc, np.uint16)), Dev(np.ascontiguousarray(vc, np.uint16))
    do = Dev(nbytes=T * H * D * 4)
    err = _err()
    _check(lib().xjh_attn_decode(T, H, Hkv, D, n_rot, base, eps, n_past, n_ctx, dq.ptr, dk.ptr, dv.ptr, dqn.ptr,
                                 dkn.ptr, dkc.ptr, dvc.ptr, do.ptr, err, ERR), err, "attn_decode")
    return (do.get(np.float32, (T, H * D)), dkc.get(np.uint16, kc.shape), dvc.get(np.uint16, vc.shape))


def delta_step(qkv, k_off, v_off, beta_raw, alpha_raw, dt, A, Hk, Hv, S, eps, qscale, state, ck_n=0):
    """DeltaNet recurrence on the GPU (the token loop's kernel) for the T rows of
    qkv [T][stride] (after the conv). Returns (out [T][Hv*S], state, checkpoints)."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    T = qkv.shape[0]
    dq, db, da = Dev(qkv), Dev(np.ascontiguousarray(beta_raw, np.float32)), Dev(np.ascontiguousarray(alpha_raw, np.float32))
    ddt, dA = Dev(np.ascontiguousarray(dt, np.float32)), Dev(np.ascontiguousarray(A, np.float32))
    ds, do = Dev(np.ascontiguousarray(state, np.float32)), Dev(nbytes=T * Hv * S * 4)
    dck = Dev(nbytes=max(1, ck_n * Hv * S * S * 4))
    err = _err()
    _check(lib().xjh_delta_step(dq.ptr, qkv.shape[1], k_off, v_off, db.ptr, da.ptr, ddt.ptr, dA.ptr, Hk, Hv, S, T, eps,
                                qscale, ds.ptr, do.ptr, dck.ptr if ck_n else None, ck_n, err, ERR), err, "delta_step")
    return (do.get(np.float32, (T, Hv * S)), ds.get(np.float32, (Hv, S, S)),
            dck.get(np.float32, (ck_n, Hv, S, S)) if ck_n else None)


def device_name():
    return lib().xj_hip_device_name().decode()


def tune_note():
    return lib().xj_hip_tune_note().decode()
