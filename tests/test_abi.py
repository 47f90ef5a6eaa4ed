"""The C-ABI boundary: the library loads, exports every function the public
headers declare, and lays out the boundary structs exactly as the reference's
headers do (src/xiaoju-pipe/core/xj_model.h:13-61, xj_stage.h:13-39).
No GPU calls."""
import ctypes as C
import os
import re
import subprocess

import pytest

import oracle as orc
import xjpipe as xp
from conftest import ROOT


def declared_functions():
    names = set()
    for h in ("xj_abi.h", "xj_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(xj[a-z]*_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_function():
    lib = xp.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", xp.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    decl = declared_functions()
    assert len(decl) > 30
    missing = sorted(decl - exported)
    assert not missing, missing
    for n in decl:
        getattr(lib, n)


def test_ctypes_layout_matches_header():
    """The Python ABI mirror and the C header agree (oracle/xjo_abi.c dumps the header's offsets)."""
    off = orc.abi_offsets()
    w = xp.XjW
    assert off[0] == C.sizeof(w) == 48
    assert off[1:7] == [getattr(w, f).offset for f in ("data", "file_off", "nbytes", "type", "ne0", "ne1")]
    assert off[7] == C.sizeof(xp.XjLayer)
    i = off.index(C.sizeof(xp.XjModel))
    assert off[i + 1:i + 6] == [getattr(xp.XjModel, f).offset for f in ("gguf", "hp", "tok_embd", "output_norm", "output")]
    j = off.index(C.sizeof(xp.XjStage), i + 1)
    names = ["m", "l0", "l1", "n_ctx", "max_batch", "n_past", "has_head", "mtp", "backend", "keep", "ck_start", "ck_T",
             "forward", "logits", "rollback", "reset", "destroy", "impl"]
    assert off[j + 1:j + 1 + len(names)] == [getattr(xp.XjStage, f).offset for f in names]


@pytest.mark.skipif(not orc.ref_available(), reason="reference build (oracle/_ref) not present")
def test_layout_matches_reference_headers():
    assert orc.abi_offsets() == orc.abi_offsets(ref=True)


def test_stage_constructor_fails_cleanly_without_gpu_or_with_bad_range(tiny_path):
    m = xp.Model(tiny_path)
    with pytest.raises(xp.XjError):
        xp.HipStage(m, 5, 3, 64, 8, True)      # l0 > l1
    with pytest.raises(xp.XjError):
        xp.HipStage(m, 0, m.hp.n_layer + 1, 64, 8, True)
