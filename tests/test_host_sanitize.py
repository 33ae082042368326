"""The host-only C code (weight-file readers, fp16 conversion, RoPE table,
tokenizer, samplers, mean loss) and the CPU oracle built with gcc's
AddressSanitizer and UndefinedBehaviorSanitizer (no device code; a run stops
at the first report) and run over valid, truncated and garbled files:
every valid file reads, every damaged one is refused with a status and no
out-of-bounds access, leak or undefined operation (tests/host_sanitize.c)."""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from test_checkpoint_gen import D_SMALL, blzt_tensors, write_blzt
from test_text import write_tokenizer

# bytes of the embedding's last row plus the writer's 7 trailing floats: cut
# there, the file ends inside the embedding
V_BLZT_TAIL = 4 * (D_SMALL["dim"] + 7)

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
SOURCES = ["tests/host_sanitize.c", "ane-training_amd/csrc/lm_weights.c", "ane-training_amd/csrc/lm_text.c",
           "oracle/oracle.c"]

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")


def build(out):
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fopenmp", "-mavx2", "-mfma", "-ffp-contract=off",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", "-Iinclude", "-Iane-training_amd/csrc",
           "-Ioracle"] + SOURCES + ["-lm", "-o", str(out)]
    subprocess.run(cmd, cwd=ROOT, check=True, capture_output=True, text=True)


def llama2c_bytes(cfg7, w):
    return struct.pack("<7i", *cfg7) + np.asarray(w, np.float32).tobytes()


def write_inputs(d):
    """Files the driver reads, each name with the status it must return (0 or
    any negative status, "<0")."""
    want = {}
    cfg = (256, 512, 2, 4, 2, -300, 32)                       # untied
    dim, hid, L, H, KV, V = 256, 512, 2, 4, 2, 300
    hd = dim // H
    per_layer = dim + dim * H * hd + 2 * dim * KV * hd + H * hd * dim + dim + 3 * dim * hid
    n_untied = V * dim + L * per_layer + dim + V * dim
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(n_untied) * 0.02).astype(np.float32)
    good = llama2c_bytes(cfg, w)
    tied = llama2c_bytes((256, 512, 2, 4, 2, 300, 32), w[:n_untied - V * dim])

    def put(name, blob, status):
        with open(os.path.join(d, name), "wb") as f:
            f.write(blob)
        want[name] = status
    put("good.llama2c", good, 0)
    put("tied.llama2c", tied, 0)
    put("empty.llama2c", b"", "<0")
    put("header_only.llama2c", good[:28], "<0")
    put("short_header.llama2c", good[:17], "<0")
    put("one_float_short.llama2c", good[:-4], "<0")
    put("mid_tensor.llama2c", good[:28 + 4 * (V * dim + 1000)], "<0")
    for name, c in {"zero_dim": (0, 512, 2, 4, 2, 300, 32), "heads_not_dividing": (256, 512, 2, 3, 3, 300, 32),
                    "kv_not_dividing": (256, 512, 2, 4, 3, 300, 32), "neg_layers": (256, 512, -2, 4, 2, 300, 32),
                    "huge_dims": (1 << 30, 1 << 30, 1 << 20, 1 << 10, 1 << 10, 1 << 30, 1 << 20),
                    "zero_vocab": (256, 512, 2, 4, 2, 0, 32),
                    # consistent headers over short files: refused before the
                    # weights (up to ~470 TB for the first) are allocated
                    "consistent_huge": (1 << 16, 1 << 16, 4096, 1024, 1024, -(1 << 24), 64),
                    "stories_short": (768, 2048, 12, 12, 12, -32000, 256)}.items():
        put(f"{name}.llama2c", llama2c_bytes(c, w[:4096]), "<0")

    layers, rf, emb = blzt_tensors(D_SMALL, 6)
    write_blzt(os.path.join(d, "good.blzt"), D_SMALL, layers, rf, emb)
    want["good.blzt"] = 0
    for name, kw in {"magic": dict(magic=0x12345678), "version": dict(version=3),
                     "truncated": dict(truncate=7 * 4 + 100), "cut_header": dict(truncate=0),
                     "adam_cut": dict(truncate=V_BLZT_TAIL)}.items():
        path = os.path.join(d, f"bad_{name}.blzt")
        write_blzt(path, D_SMALL, layers, rf, emb, **kw)
        if name == "cut_header":
            with open(path, "r+b") as f:
                f.truncate(40)
        want[f"bad_{name}.blzt"] = "<0"

    vocab = [b"<unk>", b"a", b"b", b"c", b" ", b"ab", b"bc", b"abc", b"ca", b" a", b"\xff"]
    scores = [0.0, -1.0, -1.0, -1.0, -2.0, 1.0, 2.0, 3.0, 0.5, 0.25, -5.0]
    V_tok = len(vocab)
    write_tokenizer(os.path.join(d, f"good.{V_tok}.tok"), vocab, scores)
    want[f"good.{V_tok}.tok"] = 0
    with open(os.path.join(d, f"good.{V_tok}.tok"), "rb") as f:
        tok = f.read()
    put(f"truncated.{V_tok}.tok", tok[:-3], "<0")
    put(f"more_entries_than_file.{V_tok + 5}.tok", tok, "<0")
    bad_len = bytearray(tok)
    struct.pack_into("<i", bad_len, 4 + 4, 1 << 30)           # first entry's length
    put(f"huge_len.{V_tok}.tok", bytes(bad_len), "<0")
    neg_len = bytearray(tok)
    struct.pack_into("<i", neg_len, 4 + 4, -7)
    put(f"negative_len.{V_tok}.tok", bytes(neg_len), "<0")
    put(f"empty.{V_tok}.tok", b"", "<0")
    return want


def test_host_code_under_sanitizers(tmp_path):
    exe = tmp_path / "host_sanitize"
    try:
        build(exe)
    except subprocess.CalledProcessError as e:
        pytest.fail(f"sanitizer build failed:\n{e.stderr[-3000:]}")
    d = tmp_path / "files"
    d.mkdir()
    want = write_inputs(str(d))
    env = dict(os.environ, OMP_NUM_THREADS="2",
               ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=99",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=98")
    r = subprocess.run([str(exe), str(d)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, f"exit {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}"
    got = {}
    for line in r.stdout.splitlines():
        parts = line.split()
        if len(parts) == 2 and parts[0] in want:
            got[parts[0]] = int(parts[1])
    assert set(got) == set(want), f"files not reported: {set(want) - set(got)}"
    for name, status in want.items():
        if status == 0:
            assert got[name] == 0, f"{name}: status {got[name]}"
        else:
            assert got[name] < 0, f"{name} was accepted"
    assert "checks failed: 0" in r.stdout
