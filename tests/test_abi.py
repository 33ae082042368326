"""The C-ABI library loads and exports every function the headers in include/
declare (stories_lm.h: lm_*, ane_gen.h: ane_*)."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b((?:lm|ane)_\w+)\s*\(", src, flags=re.M))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("lm_init", "lm_create", "lm_load_llama2c", "lm_forward", "lm_forward_batch",
                 "lm_prefill", "lm_prefill_batch", "lm_generate_greedy", "lm_free"):
        assert must in names


def declared_constants():
    """Every integer #define and explicitly valued enumerator of the headers
    (status codes, dtypes, options, logits modes): name -> value."""
    out = {}
    for h in HEADERS:
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for name, val in re.findall(r"^#define\s+((?:LM|ANE)_\w+)\s+\(?(-?\d+)\)?\s*$", src, flags=re.M):
            out[name] = int(val)
        for body in re.findall(r"enum\s*\{([^}]*)\}", src):   # enumerators with explicit values
            for name, val in re.findall(r"((?:LM|ANE)_\w+)\s*=\s*(-?\d+)", body):
                out[name] = int(val)
    return out


def test_binding_constants_match_the_header(lm):
    """The ctypes mirror's status codes, dtypes, options and logits modes carry
    the header's values (a renumbered option would otherwise set another)."""
    consts = declared_constants()
    assert {"LM_OK", "LM_ERR_HIP", "LM_OPT_USE_GRAPH", "LM_OPT_PREFILL_FOLD", "LM_LOGITS_LAST"} <= set(consts)
    mirrored = {n: v for n, v in vars(lm).items() if n.startswith("LM_") and isinstance(v, int)}
    assert mirrored, "no constants in the binding"
    wrong = {n: (v, consts.get(n)) for n, v in mirrored.items() if consts.get(n) != v}
    assert not wrong, wrong
    missing = [n for n in consts if n.startswith(("LM_OPT_", "LM_ERR_", "LM_DTYPE_", "LM_LOGITS_"))
               and n not in mirrored]
    assert not missing, missing


def test_library_exports_every_declared_symbol(lm):
    L = lm.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


@pytest.mark.skipif(os.path.exists("/dev/kfd"),
                    reason="compiler check: runs where the library is built, not on a GPU host "
                           "(no child processes next to an initialised GPU)")
def test_header_compiles_as_plain_c(tmp_path):
    c = tmp_path / "t.c"
    c.write_text('#include "stories_lm.h"\n#include "ane_gen.h"\n'
                 'int main(void){Config c={0};ANEGenConfig g=ane_gen_default_config();(void)c;(void)g;'
                 'return lm_strerror(0)==0;}\n')
    rc = os.system(f"gcc -std=c99 -Wall -Werror -I{ROOT}/include -c {c} -o {tmp_path}/t.o")
    assert rc == 0


def test_status_strings(lm):
    assert lm.strerror(0) == "ok"
    assert "gfx950" in lm.strerror(lm.LM_ERR_NOT_GFX950)
    assert lm.strerror(12345) == "unknown status"


def test_null_arguments_rejected_before_device(lm):
    L = lm.lib()
    st = ctypes.c_int(99)
    assert not L.lm_create(None, None, 1, 1, ctypes.byref(st))
    assert st.value == lm.LM_ERR_INVALID
    assert L.lm_forward_batch(None, None, None, 1, None, None) == lm.LM_ERR_INVALID
    assert L.lm_prefill(None, 0, 0, None, 1, None) == lm.LM_ERR_INVALID
    assert L.lm_prefill_loss(None, 1, None, None, 2, None, None) == lm.LM_ERR_INVALID
    assert L.lm_generate_greedy(None, 1, None, None, 1, None) == lm.LM_ERR_INVALID
    assert not L.lm_forward(None, 0, 0)
    L.lm_free(None)


def test_create_layers_rejects_null_entries_before_device(lm):
    """lm_create_layers checks every per-layer pointer before any device call
    (here: layer 1 of wq missing), and split_layers' per-layer copies hold the
    contiguous buffer's values."""
    from conftest import TINY_GQA
    cfg = lm.make_config(**TINY_GQA)
    w16 = lm.synth_weights_f16(cfg, 3, 0.02, True)
    t = lm.split_layers(cfg, w16, True)
    names = ("token_embedding",) + lm.LAYER_TENSORS + ("rms_final_w", "wcls")
    flat = np.concatenate([np.concatenate(t[n]) if n in lm.LAYER_TENSORS else t[n] for n in names])
    assert np.array_equal(flat, w16)
    assert all(len(t[n]) == cfg.n_layers for n in lm.LAYER_TENSORS)
    t["wq"][1] = None
    w = lm.LMLayerWeights()
    w.dtype = lm.LM_DTYPE_F16
    w.token_embedding = t["token_embedding"].ctypes.data
    keep = []
    for n in lm.LAYER_TENSORS:
        ptrs = (ctypes.c_void_p * cfg.n_layers)(*[a.ctypes.data if a is not None else None for a in t[n]])
        keep.append(ptrs)
        setattr(w, n, ctypes.cast(ptrs, ctypes.POINTER(ctypes.c_void_p)))
    w.rms_final_w = t["rms_final_w"].ctypes.data
    st = ctypes.c_int(99)
    assert not lm.lib().lm_create_layers(ctypes.byref(cfg), ctypes.byref(w), 1, 16, ctypes.byref(st))
    assert st.value == lm.LM_ERR_INVALID
    w.wq = None
    assert not lm.lib().lm_create_layers(ctypes.byref(cfg), ctypes.byref(w), 1, 16, ctypes.byref(st))
    assert st.value == lm.LM_ERR_INVALID
