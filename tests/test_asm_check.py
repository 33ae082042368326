"""The build check of the tiled GEMM's inline LDS reads (CPU only): the checker
flags a planted use of an in-flight read register, passes the clean form, and
passes the library's own device assembly."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ane-training_amd")
sys.path.insert(0, PKG)

import check_lds_asm  # noqa: E402
import pytest  # noqa: E402

HEAD = "_Z11k_gemm_tileILi64ELi64ELi0EEvPKtiS1_i7EpiArgsii:\n"
TAIL = ".Lfunc_end0:\n"


def test_flags_planted_use_of_pending_register():
    asm = HEAD + ("\tds_read_b128 v[4:7], v1\n"
                  "\tv_mfma_f32_32x32x16_f16 a[0:15], v[4:7], v[8:11], a[0:15]\n"
                  "\ts_waitcnt lgkmcnt(0)\n") + TAIL
    names, bad = check_lds_asm.check(asm)
    assert len(names) == 1 and len(bad) == 1


def test_flags_copy_of_pending_register():
    asm = HEAD + ("\tds_read_b128 v[4:7], v1\n"
                  "\tv_mov_b32 v20, v5\n"
                  "\ts_waitcnt lgkmcnt(0)\n") + TAIL
    assert len(check_lds_asm.check(asm)[1]) == 1


def test_passes_use_after_wait_and_unrelated_work():
    asm = HEAD + ("\tds_read_b128 v[4:7], v1\n"
                  "\tv_mfma_f32_32x32x16_f16 a[16:31], v[12:15], v[8:11], a[16:31]\n"
                  "\ts_waitcnt lgkmcnt(0)\n"
                  "\tv_mfma_f32_32x32x16_f16 a[0:15], v[4:7], v[8:11], a[0:15]\n") + TAIL
    names, bad = check_lds_asm.check(asm)
    assert len(names) == 1 and not bad


def test_partial_wait_retires_only_older_reads():
    """lgkmcnt(1) after two LDS reads retires the older one only (LDS operations
    complete in order)."""
    two = "\tds_read_b128 v[4:7], v1\n\tds_read_b128 v[8:11], v1 offset:32\n\ts_waitcnt lgkmcnt(1)\n"
    assert not check_lds_asm.check(HEAD + two + "\tv_mul_f32_e32 v20, v4, v20\n" + TAIL)[1]
    assert len(check_lds_asm.check(HEAD + two + "\tv_mul_f32_e32 v20, v8, v20\n" + TAIL)[1]) == 1


def test_partial_wait_with_scalar_load_retires_nothing():
    """A scalar load in flight can complete out of order: lgkmcnt(1) then
    retires no LDS read."""
    asm = HEAD + ("\tds_read_b128 v[4:7], v1\n"
                  "\ts_load_dwordx2 s[0:1], s[4:5], 0x0\n"
                  "\ts_waitcnt lgkmcnt(1)\n"
                  "\tv_mul_f32_e32 v20, v4, v20\n") + TAIL
    assert len(check_lds_asm.check(asm)[1]) == 1


@pytest.mark.skipif(os.path.exists("/dev/kfd"),
                    reason="build check: runs where the library is built, not on a GPU host "
                           "(no child processes next to an initialised GPU)")
def test_library_assembly_is_clean():
    r = subprocess.run(["make", "-C", PKG, "check"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
