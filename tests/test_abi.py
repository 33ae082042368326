"""The C-ABI library loads and exports every function include/stories_lm.h declares."""
import ctypes
import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "stories_lm.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(lm_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("lm_init", "lm_create", "lm_load_llama2c", "lm_forward", "lm_forward_batch",
                 "lm_prefill", "lm_prefill_batch", "lm_generate_greedy", "lm_free"):
        assert must in names


def test_library_exports_every_declared_symbol(lm):
    L = lm.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_header_compiles_as_plain_c(tmp_path):
    c = tmp_path / "t.c"
    c.write_text('#include "stories_lm.h"\nint main(void){Config c={0};(void)c;return lm_strerror(0)==0;}\n')
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
    assert L.lm_generate_greedy(None, 1, None, None, 1, None) == lm.LM_ERR_INVALID
    assert not L.lm_forward(None, 0, 0)
    L.lm_free(None)
