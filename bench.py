"""Benchmark of the Stories / Llama-2 token loop on one MI355X.

Headline (``value``): configuration C0 of the baseline — Stories-110M
(dim 768, 12 layers, 12 heads, SwiGLU 2048, vocab 32000, untied classifier),
seeded N(0, 0.02) fp16 weights, batch-1 greedy decode of 256 tokens from token
id 1, fp32 accumulation, K/V cache in fp32 like the reference forward
(training/forward.h:118-128), so the greedy ids are the reference's (--kv16
switches to a binary16 cache).  A step is one such 256-token sequence: --steps
K times exactly K of them (K x 256 tokens), after --warmup W untimed ones.  The
timed region replays captured 16-token hipGraphs with the argmax fed back on
the device, inputs and weights already resident in HBM; value is tokens/s.

Alongside the headline the JSON line carries:
  roofline      the dominant kernel of the decode step: algorithmic bytes per
                launch / mean launch duration, the duration measured after the
                timed region over the 254 decode steps of one sequence of the same
                chain, each kernel launched with events at its own dispatch's
                device start and end (lm_profile_chain); every family's time is
                in kernel_us_per_launch.  traffic: the kernel's FETCH_SIZE +
                WRITE_SIZE per dispatch from the committed C0 profile's counter
                line, or null when no counter pass of it has completed
  step_roofline the whole token: algorithmic bytes per token / time per token
  configs       C1-C4 (MFMA paths), C0 in the reference's own algorithm (a
                256-position window forward per token, generate.m:427-516),
                C0 with the binary16 K/V cache, and C0 per-token time warm
                against after a sweep that evicts the Infinity Cache
  device_copy_rate  a plain device-to-device copy's bytes read + written per
                second on this GPU (what a stream reaches, beside the
                published 8 TB/s the fractions use)
  cpu_baseline  the reference's portable CPU forward with OpenBLAS in place of
                Accelerate (oracle/cpu_ref.c) on this host's cores: C0 KV-cache
                decode (its ids compared with the GPU's), and under "configs"
                C0 in the reference's own algorithm, C1 and C3, each a bounded
                sample
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "ane-training_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
_T0 = time.perf_counter()


def progress(msg):
    """One progress line on stderr per phase (the JSON line alone goes to
    stdout), flushed, so a run that stops can be placed."""
    print(f"[bench {time.perf_counter() - _T0:7.1f}s] {msg}", file=sys.stderr, flush=True)
# Published reference figure for this metric: Stories-110M B=1 greedy decode on
# the ANE (libane, fp16), M3 Pro: 41.7 tok/s (full 256-window recompute).
LIB_FUSE_DEFAULT = 3     # LM_OPT_FUSE_QKV_ATTN after lm_load / lm_create
REF_TOK_S = 41.7
SEQ = 256


PROFILE_C0 = os.path.join(ROOT, "profiles", "decode_b1_stories110m_chain.md")


def profiled_traffic(kernel_prefix):
    """HBM bytes per launch of the kernel named by kernel_prefix, from the
    counter line of the committed C0 profile: FETCH_SIZE and WRITE_SIZE per
    dispatch of that kernel in two rocprofv3 --pmc runs, each scaled by what
    the same counter reads for a device copy of known size in the same run.
    The line reads `counters <kernel> fetch_bytes=F write_bytes=W`; None when
    the profile holds no such line (no completed counter pass)."""
    import re
    try:
        text = open(PROFILE_C0).read()
    except OSError:
        return None
    want = kernel_prefix.replace(" ", "")
    for mt in re.finditer(r"^counters (\S+) fetch_bytes=(\d+) write_bytes=(\d+)", text, re.M):
        if mt.group(1).startswith(want):
            return {"fetch": int(mt.group(2)), "write": int(mt.group(3)), "kernel": mt.group(1)}
    return None


def algorithmic_bytes(cfg, B, mean_ctx, kv_bytes=2, logits=False):
    """Bytes each decode kernel family must move per launch (weights read once,
    activations read/written once; K/V read over mean_ctx cached positions)."""
    D, F, V = cfg.dim, cfg.hidden_dim, abs(cfg.vocab_size)
    hd = D // cfg.n_heads
    NQ, NKV = cfg.n_heads * hd, cfg.n_kv_heads * hd
    nblk = (V + 31) // 32          # argmax partials: one per 32 classifier rows
    return {
        "qkv": (NQ + 2 * NKV) * D * 2 + D * 4 + B * (D * 4 + NQ * 4 + 2 * NKV * kv_bytes + hd * 4),
        "attn": B * (2 * mean_ctx * NKV * kv_bytes + 2 * NQ * 4),
        "wo": D * NQ * 2 + B * (NQ * 4 + 2 * D * 4),
        "w13": 2 * F * D * 2 + D * 4 + B * (D * 4 + F * 4),
        "w2": D * F * 2 + B * (F * 4 + 2 * D * 4),
        "cls": V * D * 2 + D * 4 + B * (D * 4 + nblk * 8 + (V * 4 if logits else 0)),
        "argmax": B * (nblk * 8 + 12),
    }


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, vendor, family,
    model and stepping numbers (which identify the part when the name is
    generic, as in some virtual machines), and the online core count."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "vendor_id", "cpu family", "model", "stepping") and k not in info:
                info[k] = v.strip()
    except OSError:
        pass
    name = info.get("model name", "unknown")
    ids = ", ".join(f"{k} {info[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in info)
    return f"{name} ({ids}; {os.cpu_count()} online cores)" if ids else name


def cpu_threads():
    """Threads for the CPU baseline: the count `nproc` prints, the processing
    units this process may use.  As GNU nproc does, that is the affinity
    mask's CPUs, replaced by OMP_NUM_THREADS when it is set and capped by
    OMP_THREAD_LIMIT.  The GPU box sets OMP_NUM_THREADS to its CPU share for
    one GPU (16 of the host's cores; the others serve its other GPUs)."""
    def env_int(k):
        try:
            return int(os.environ.get(k, "").split(",")[0])
        except ValueError:
            return 0
    n = len(os.sched_getaffinity(0))
    if env_int("OMP_NUM_THREADS") > 0:
        n = env_int("OMP_NUM_THREADS")
    if env_int("OMP_THREAD_LIMIT") > 0:
        n = min(n, env_int("OMP_THREAD_LIMIT"))
    return max(1, n)


def cpu_baseline(cfg7, w16, S, gpu_ids, seconds):
    """The reference's portable CPU forward (oracle/cpu_ref.c: stories_cpu_ops.h
    RMSNorm, forward.h RoPE and attention, OpenBLAS sgemv/sgemm for the
    projections) on this host: C0 KV-cache greedy decode from token 1, as many
    whole passes over its first tokens as fit about `seconds`; its ids are
    compared with the GPU's.  Under "configs", bounded samples of C0 in the
    reference's own algorithm (every token a 256-position window forward with
    the classifier on the last row, generate.m:427-516), C1 (one 256-token
    prompt, all logits) and C3 (two of its eight prompts)."""
    import cpu_ref as R
    n = cpu_threads()
    R.set_threads(n)
    w32 = S.f16_to_f32(w16)
    r = R.CpuRef(cfg7, w32, True, SEQ)
    # C0 KV decode: 64 tokens per pass, passes until the budget is spent
    ntok, passes, ids = 64, 0, None
    t0 = time.perf_counter()
    while True:
        got = r.greedy(1, 0, ntok)
        if ids is None:
            ids = got
        elif not np.array_equal(got, ids):
            raise RuntimeError("CPU baseline decode is not repeatable")
        passes += 1
        if time.perf_counter() - t0 > seconds * 0.5:
            break
    dt = time.perf_counter() - t0
    out = {"value": round(passes * ntok / dt, 2), "unit": "tok/s", "cores": n, "kind": "port",
           "cpu_model": cpu_model(), "nproc_all": os.cpu_count(), "blas": R.blas_name(),
           "ids_match_gpu": bool(np.array_equal(ids, gpu_ids[:ntok])),
           "sample": f"C0 KV-cache greedy decode of the first {ntok} tokens from id 1, {passes} passes, "
                     f"{dt:.1f} s, {n} threads (oracle/cpu_ref.c: the reference forward with OpenBLAS)"}
    cfgs = {}
    win = np.concatenate([[1], gpu_ids[:SEQ - 1]]).astype(np.int32)
    t0 = time.perf_counter()
    k = 0
    while k < 2 or (time.perf_counter() - t0 < seconds * 0.25 and k < 64):
        r.forward(win, last_only=True)
        k += 1
    dt = time.perf_counter() - t0
    cfgs["c0_reference_algorithm"] = {
        "value": round(k / dt, 3), "unit": "tok/s",
        "sample": f"{k} tokens, each a full {SEQ}-position window forward + last-row classifier, {dt:.1f} s"}
    toks = np.random.default_rng(101).integers(0, 32000, SEQ).astype(np.int32)
    t0 = time.perf_counter()
    r.forward(toks)
    dt = time.perf_counter() - t0
    cfgs["c1_prefill_256"] = {"value": round(SEQ / dt, 1), "unit": "tok/s", "ms": round(dt * 1e3, 1),
                              "sample": "one 256-token prompt, all 256 x 32000 logits"}
    toks = np.random.default_rng(103).integers(0, 32000, (8, SEQ)).astype(np.int32)
    t0 = time.perf_counter()
    for i in range(8):
        r.forward(toks[i])
    dt = time.perf_counter() - t0
    cfgs["c3_forward_8x256"] = {"value": round(8 * SEQ / dt, 1), "unit": "tok/s",
                                "sample": f"the 8 prompts of 256 tokens one after another, all logits, {dt:.1f} s"}
    r.close()
    out["configs"] = cfgs
    return out


def reference_algorithm_gpu(S, cfg, w16, ids, n_tokens=48):
    """C0 in the reference's own algorithm on the GPU: every token recomputes
    the full 256-position window (BOS + the newest 255 tokens, generate.m:
    427-516 with its window shift, 504-508) through the MFMA prefill with the
    classifier on the last row, the logits copied to the host and the argmax
    taken there, as the session API does once its window is full; wall-clock
    ms per token over n_tokens after one untimed token."""
    m = S.Model.create(cfg, w16, True, 1, SEQ)
    m.set_option(S.LM_OPT_KV_F32, 1)
    win = np.concatenate([[1], ids[:SEQ - 1]]).astype(np.int32)

    def step(w):
        lg = m.prefill_batch(w[None], mode=S.LM_LOGITS_LAST)
        nxt = S.sample_argmax(lg[0])
        return np.concatenate([w[:1], w[2:], [nxt]]).astype(np.int32)
    win = step(win)
    t0 = time.perf_counter()
    for _ in range(n_tokens):
        win = step(win)
    dt = time.perf_counter() - t0
    m.close()
    return {"value": round(n_tokens / dt, 1), "unit": "tok/s", "ms_per_token": round(dt * 1e3 / n_tokens, 4),
            "sample": f"{n_tokens} tokens with a full window, each one {SEQ}-row MFMA prefill (last-row "
                      f"classifier) + logits to the host + host argmax, wall clock"}


def c0_kv16(S, cfg, w16, ids, direct, seqs=8):
    """C0 with the binary16 K/V cache (north_star's storage; the headline uses
    the reference forward's fp32 K/V): tok/s over `seqs` timed 256-token greedy
    sequences after one untimed, and the first step whose id differs from the
    fp32-cache run (a near tie that the cache rounding flips), if any."""
    m = S.Model.create(cfg, w16, True, 1, SEQ)
    if direct:
        m.set_option(S.LM_OPT_USE_GRAPH, 0)
    got = m.generate_greedy([1], [0], SEQ)[:, 0]
    m.sync()
    m.timer_begin()
    for _ in range(seqs):
        m.generate_greedy([1], [0], SEQ)
    ms = m.timer_end()
    m.close()
    diff = np.nonzero(np.asarray(got) != np.asarray(ids))[0]
    return {"value": round(seqs * SEQ / (ms / 1e3), 1), "unit": "tok/s",
            "us_per_token": round(ms * 1e3 / (seqs * SEQ), 3),
            "first_id_differing_from_fp32_cache": int(diff[0]) if diff.size else None,
            "sample": f"{seqs} timed 256-token greedy sequences from token id 1"}


def c0_cold_cache(S, cfg, w16, ids, sweep_mib=512):
    """C0 with and without a cache sweep before every token.  The decode
    working set (219 MB of fp16 weights, the K/V cache and activations) fits
    the 256 MB Infinity Cache, so a warm token may be served partly from it
    rather than from HBM.  Both legs run the 255 decode steps of a C0 sequence
    one call each (lm_generate_greedy of one step: its graph replay, the id
    copied back to the host), timed by hipEvents on the model's stream around
    the call; the cold leg first copies a sweep_mib MiB buffer into another
    (sweep_mib MiB read + written, twice the cache) and waits for the copy, so
    the token starts with the weights evicted from the L2s and the Infinity
    Cache.  cold_minus_warm_us is the cost of fetching from HBM what a warm
    token finds in the caches."""
    import ctypes
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hip = ctypes.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    n = int(sweep_mib) << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), n) or hip.hipMalloc(ctypes.byref(b), n):
        raise SystemExit("c0_cold_cache: hipMalloc failed")
    if hip.hipMemset(a, 1, ctypes.c_size_t(n)) or hip.hipDeviceSynchronize():
        raise SystemExit("c0_cold_cache: hipMemset failed")
    m = S.Model.create(cfg, w16, True, 1, SEQ)
    m.set_option(S.LM_OPT_KV_F32, 1)
    toks = np.concatenate([[1], np.asarray(ids[:SEQ - 2])]).astype(np.int32)

    def leg(cold):
        total = 0.0
        for p, t in enumerate(toks):
            if cold and (hip.hipMemcpy(b, a, n, 3) or hip.hipDeviceSynchronize()):
                raise SystemExit("c0_cold_cache: sweep copy failed")
            m.timer_begin()
            got = m.generate_greedy([int(t)], [p], 1)[0, 0]
            total += m.timer_end()
            if got != ids[p]:
                raise SystemExit(f"c0_cold_cache: step {p} gave id {got}, the timed run {ids[p]}")
        return total * 1e3 / toks.size
    leg(False)
    warm = leg(False)
    cold = leg(True)
    m.close()
    hip.hipFree(a)
    hip.hipFree(b)
    return {"warm_us_per_token": round(warm, 3), "cold_us_per_token": round(cold, 3),
            "cold_minus_warm_us": round(cold - warm, 3),
            "sample": f"the {toks.size} decode steps of one C0 sequence, one lm_generate_greedy call "
                      f"each (graph replay + id to the host), cold: a {2 * sweep_mib} MiB device copy "
                      f"(read + write) before every step"}


MFMA_PEAK_TFLOPS = 2500.0      # dense fp16


def _timed(m, fn, reps):
    """Device milliseconds per call of fn over reps calls (hipEvents on the
    model's stream; fn's host copies of the results are excluded by design of
    the calls used: they keep logits on the device)."""
    fn()
    m.sync()
    m.timer_begin()
    for _ in range(reps):
        fn()
    return m.timer_end() / reps


def model_bytes(cfg):
    D, F, V, L = cfg.dim, cfg.hidden_dim, abs(cfg.vocab_size), cfg.n_layers
    hd = D // cfg.n_heads
    NQ, NKV = cfg.n_heads * hd, cfg.n_kv_heads * hd
    mats = L * ((NQ + 2 * NKV) * D + D * NQ + 3 * F * D) + V * D
    return 2 * mats, 2 * mats // 2          # bytes of fp16 matrices, matrix parameters


def linear_flops(cfg, rows):
    _, params = model_bytes(cfg)
    return 2.0 * params * rows


def attn_flops_prefill(cfg, S, nseq):
    hd = cfg.dim // cfg.n_heads
    return nseq * cfg.n_layers * cfg.n_heads * 2 * 2 * hd * S * (S + 1) / 2


def bench_extra(S, w16_stories, reps_prefill=10, reps_decode=2, direct=False, only=None, c4_steps=128):
    """Configs C1-C4 of the baseline (MFMA paths), as extra entries.  direct:
    launch decode kernels directly instead of replaying graphs; only: run just
    these configs ("c1" .. "c4")."""
    out = {}

    def want(c):
        return only is None or c in only
    cfg = S.make_config(**S.STORIES_110M)
    wbytes, _ = model_bytes(cfg)
    V = 32000
    # C1: 256-token causal prefill, all 256 x 32000 fp32 logits (kept on the device)
    if want("c1"):
        progress("C1: 256-token prefill, all logits")
        m = S.Model.create(cfg, w16_stories, True, 1, 256)
        toks = np.random.default_rng(101).integers(0, V, 256).astype(np.int32)
        ms = _timed(m, lambda: m.prefill(toks, want_logits=False), reps_prefill)
        fl = linear_flops(cfg, 256) + attn_flops_prefill(cfg, 256, 1)
        by = wbytes + 256 * V * 4
        out["c1_prefill_256"] = {"value": round(256 / (ms * 1e-3), 1), "unit": "tok/s", "ms": round(ms, 4),
                                 "hbm_frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                 "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                                 "algorithmic_bytes": int(by), "flops": fl}
        m.close()
    # C3: 8 x 256 = 2048-token causal forward with all logits (MFMA bound)
    if want("c3"):
        progress("C3: 8 x 256-token forward")
        m = S.Model.create(cfg, w16_stories, True, 8, 256)
        toks = np.random.default_rng(103).integers(0, V, (8, 256)).astype(np.int32)
        ms = _timed(m, lambda: m.prefill_batch(toks, mode=S.LM_LOGITS_ALL, want_logits=False), reps_prefill)
        fl = linear_flops(cfg, 2048) + attn_flops_prefill(cfg, 256, 8)
        out["c3_forward_8x256"] = {"value": round(2048 / (ms * 1e-3), 1), "unit": "tok/s", "ms": round(ms, 4),
                                   "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                                   "tflops": round(fl / (ms * 1e-3) / 1e12, 1), "flops": fl}
        # the same forward with model_forward's loss taken on the device
        ms_loss = _timed(m, lambda: m.prefill_loss(toks), reps_prefill)
        out["c3_forward_8x256"]["with_loss_ms"] = round(ms_loss, 4)
        m.close()
    # C2: 64 sequences, 192-token prompts prefilled, then 64 greedy steps each
    if want("c2"):
        progress("C2: 64 x 192-token prefill, then 64 greedy steps")
        m = S.Model.create(cfg, w16_stories, True, 64, 256)
        if direct:
            m.set_option(S.LM_OPT_USE_GRAPH, 0)
        rng = np.random.default_rng(102)
        prompts = rng.integers(0, V, (64, 192)).astype(np.int32)
        ms_pf = _timed(m, lambda: m.prefill_batch(prompts, mode=S.LM_LOGITS_LAST, want_logits=False), 2)
        lg = m.prefill_batch(prompts, mode=S.LM_LOGITS_LAST)
        first = np.argmax(lg, axis=1).astype(np.int32)
        pos = np.full(64, 192, np.int32)
        ms = _timed(m, lambda: m.generate_greedy(first, pos, 64), reps_decode)
        kv_step = 64 * 12 * 2 * 768 * 2 * (192 + 64 / 2 + 0.5)    # mean context 224.5
        by_step = wbytes + kv_step + 64 * V * 0 + 64 * 2 * 12 * 768 * 2
        t_step = ms * 1e-3 / 64
        out["c2_decode_b64"] = {"value": round(64 * 64 / (ms * 1e-3), 1), "unit": "tok/s",
                                "ms_per_step": round(ms / 64, 4),
                                "hbm_frac": round(by_step / t_step / 1e9 / HBM_PEAK_GBS, 4),
                                "algorithmic_bytes_per_step": int(by_step),
                                "prefill_64x192_tok_s": round(64 * 192 / (ms_pf * 1e-3), 1)}
        m.close()
    # C4: scaled Llama-2 model, 32 sequences, 512-token contexts, 128 greedy steps
    if want("c4"):
        d4 = dict(dim=2048, hidden_dim=5632, n_layers=16, n_heads=16, n_kv_heads=16, vocab_size=32000,
                  seq_len=640)
        cfg4 = S.make_config(**d4)
        progress("C4: synthesising the scaled model's weights")
        w4 = S.synth_weights_f16(cfg4, 4, 0.02, True)
        progress("C4: creating the model (weights to the device)")
        m = S.Model.create(cfg4, w4, True, 32, 640)
        if direct:
            m.set_option(S.LM_OPT_USE_GRAPH, 0)
        del w4
        prompts = np.random.default_rng(104).integers(0, V, (32, 512)).astype(np.int32)
        progress("C4: 32 x 512-token prefill")
        lg = m.prefill_batch(prompts, mode=S.LM_LOGITS_LAST)
        first = np.argmax(lg, axis=1).astype(np.int32)
        pos = np.full(32, 512, np.int32)
        progress(f"C4: {c4_steps} greedy steps, untimed then timed")
        ms = _timed(m, lambda: m.generate_greedy(first, pos, c4_steps), 1)
        wb4, _ = model_bytes(cfg4)
        kv4 = 32 * 16 * 2 * 2048 * 2 * (512 + c4_steps / 2 + 0.5)
        t4 = ms * 1e-3 / c4_steps
        out["c4_scaled_decode_b32"] = {"value": round(32 * c4_steps / (ms * 1e-3), 1), "unit": "tok/s",
                                       "ms_per_step": round(ms / c4_steps, 4), "steps": c4_steps,
                                       "hbm_frac": round((wb4 + kv4) / t4 / 1e9 / HBM_PEAK_GBS, 4),
                                       "algorithmic_bytes_per_step": int(wb4 + kv4)}
        m.close()
    return out


def calibration_copy(mbytes):
    """One device-to-device copy of mbytes MiB (hipMemcpy, the runtime's copy
    kernel): the known-size reference that scales rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters to bytes."""
    import ctypes
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hip = ctypes.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    n = int(mbytes) << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), n) or hip.hipMalloc(ctypes.byref(b), n):
        raise SystemExit("calibration copy: hipMalloc failed")
    rc = hip.hipMemset(a, 0, ctypes.c_size_t(n)) or hip.hipMemcpy(b, a, n, 3) or hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)
    if rc:
        raise SystemExit("calibration copy failed")


def device_copy_rate(mib=1024, reps=5):
    """The device-to-device copy rate on this GPU (hipMemcpy of mib MiB, the
    runtime's copy kernel, timed by hipEvents over reps queued copies after one
    untimed): bytes read + written per second.  Context for the HBM fractions,
    which are against the published 8 TB/s: this is what a plain stream
    reaches here."""
    import ctypes
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hip = ctypes.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
    vp = ctypes.c_void_p
    hip.hipMalloc.argtypes = [ctypes.POINTER(vp), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpyAsync.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, vp]
    hip.hipMemset.argtypes = [vp, ctypes.c_int, ctypes.c_size_t]
    hip.hipFree.argtypes = [vp]
    hip.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
    hip.hipEventRecord.argtypes = [vp, vp]
    hip.hipEventSynchronize.argtypes = [vp]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    hip.hipEventDestroy.argtypes = [vp]
    n = int(mib) << 20
    a, b, e0, e1 = vp(), vp(), vp(), vp()
    if hip.hipMalloc(ctypes.byref(a), n) or hip.hipMalloc(ctypes.byref(b), n):
        raise SystemExit("device_copy_rate: hipMalloc failed")
    ms = ctypes.c_float(0)
    rc = hip.hipMemset(a, 1, ctypes.c_size_t(n)) or hip.hipMemcpy(b, a, n, 3) or \
        hip.hipEventCreate(ctypes.byref(e0)) or hip.hipEventCreate(ctypes.byref(e1)) or \
        hip.hipEventRecord(e0, None)
    for _ in range(reps):   # queued back to back on the null stream
        rc = rc or hip.hipMemcpyAsync(b, a, n, 3, None)
    rc = rc or hip.hipEventRecord(e1, None) or hip.hipEventSynchronize(e1) or \
        hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1)
    hip.hipEventDestroy(e0)
    hip.hipEventDestroy(e1)
    hip.hipFree(a)
    hip.hipFree(b)
    if rc or ms.value <= 0:
        raise SystemExit("device_copy_rate: copy timing failed")
    return {"value": round(2 * n * reps / (ms.value * 1e-3) / 1e9, 1), "unit": "GB/s",
            "sample": f"{reps} device-to-device copies of {mib} MiB (hipMemcpy), bytes read + written"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32, help="timed 256-token C0 sequences")
    ap.add_argument("--warmup", type=int, default=2, help="untimed 256-token C0 sequences")
    ap.add_argument("--direct", action="store_true", help="launch kernels directly, no graphs")
    ap.add_argument("--fuse", type=int, choices=[0, 1, 2, 3, 4], default=None,
                    help="LM_OPT_FUSE_QKV_ATTN for the C0 chain (A/B; default: the library's)")
    ap.add_argument("--kv16", action="store_true",
                    help="binary16 K/V cache (default fp32, as the reference forward keeps K/V)")
    ap.add_argument("--cpu-seconds", type=float, default=16.0, help="budget of the CPU baseline samples")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip configs C1-C4")
    ap.add_argument("--no-chain-timing", action="store_true",
                    help="skip the per-dispatch timing of the decode chain (lm_profile_chain)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="first copy this many MiB device to device (counter calibration)")
    ap.add_argument("--c4-steps", type=int, default=128,
                    help="greedy steps of the C4 leg (fewer for counter passes)")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4"],
                    help="run just this config of C1-C4 (for profiling) and print its entry")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (one MI355X per box); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)
    import stories_lm as S
    progress("lm_init")
    rc = S.init()
    if rc:
        raise SystemExit(f"lm_init: {S.strerror(rc)}")
    if args.calib_copy_mb:
        progress(f"calibration copy of {args.calib_copy_mb} MiB")
        calibration_copy(args.calib_copy_mb)
    cfg = S.make_config(**S.STORIES_110M)
    w16 = None
    if args.only != "c4":
        progress("synthesising the Stories-110M weights")
        w16 = S.synth_weights_f16(cfg, 1, 0.02, True)
    if args.only:
        print(json.dumps(bench_extra(S, w16, direct=args.direct, only={args.only},
                                     c4_steps=args.c4_steps)), flush=True)
        progress("done")
        return
    progress("creating the C0 model")
    m = S.Model.create(cfg, w16, True, 1, SEQ)
    if not args.kv16:
        m.set_option(S.LM_OPT_KV_F32, 1)
    if args.direct:
        m.set_option(S.LM_OPT_USE_GRAPH, 0)
    if args.fuse is not None:
        m.set_option(S.LM_OPT_FUSE_QKV_ATTN, args.fuse)

    progress(f"C0: {args.warmup} warm-up sequence(s)")
    for _ in range(args.warmup):
        m.generate_greedy([1], [0], SEQ)
    m.sync()
    progress(f"C0: {args.steps} timed sequence(s) of {SEQ} tokens")
    m.timer_begin()
    t0 = time.perf_counter()
    ids = None
    for _ in range(args.steps):
        ids = m.generate_greedy([1], [0], SEQ)[:, 0]
    ms = m.timer_end()
    wall = time.perf_counter() - t0
    tokens = args.steps * SEQ
    tok_s = tokens / (ms / 1e3)
    us_tok = ms * 1e3 / tokens

    mean_ctx = (SEQ + 1) / 2
    kvb = 2 if args.kv16 else 4
    algo = algorithmic_bytes(cfg, 1, mean_ctx, kvb)
    chain_timing = not args.no_chain_timing
    fuse_level = LIB_FUSE_DEFAULT if args.fuse is None else args.fuse
    launches = None
    if chain_timing:
        progress("per-dispatch timing of the decode chain (lm_profile_chain, 254 steps)")
        # device time per launch of each kernel family inside the decode chain over
        # the positions of a timed sequence (254 steps from position 0): every
        # kernel timed by hipEvents at its own dispatch's start and end
        us, launches = m.profile_chain([1], [0], SEQ - 2)
    m.close()
    if launches is None:   # the chain's launch counts: one per layer, attention (Wo from
        # level 2, the FFN at 3) inside the QKV launch, classifier and argmax once
        fz = fuse_level
        inside = {"attn": fz >= 1, "wo": fz >= 2, "w13": fz >= 3, "w2": fz >= 3, "argmax": fz >= 3}
        launches = {k: (0 if inside.get(k) else 1 if k in ("cls", "argmax") else cfg.n_layers)
                    for k in algo}
    if launches.get("argmax") == 0:   # the argmax runs inside the classifier launch
        algo["cls"] += algo.pop("argmax")
        launches.pop("argmax")
    folded = []
    for k in ("attn", "wo", "w13", "w2"):    # families that run inside the QKV launch
        if launches.get(k) == 0:
            folded.append(k)
            algo["qkv"] += algo.pop(k)
            launches.pop(k)
    step_bytes = sum(algo[k] * launches[k] for k in algo)
    step_gbs = step_bytes / (us_tok * 1e-6) / 1e9
    out = {
        "metric": "Stories-110M decode tok/s at B=1 and B=64; prefill tok/s; % HBM/MFMA roofline",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": round(tok_s / REF_TOK_S, 1),
        "vs_baseline_note": "value / 41.7 tok/s, the reference's published B=1 decode on the ANE (M3 Pro), "
                            "which recomputes the 256-token window per token; the same algorithm on this "
                            "GPU is configs.c0_reference_algorithm (vs_baseline_same_algorithm)",
        "dtype": "f32", "storage": "f16 weights, f%d K/V cache" % (8 * kvb),
        "data": "synthetic (seeded N(0,0.02) fp16 weights, greedy from token id 1)",
        "config": {"workload": "C0: Stories-110M batch-1 greedy decode, 256-token sequences "
                               "from token id 1, untied classifier; one step = one 256-token sequence",
                   "batch": 1, "seq_len": SEQ, "tokens_timed": tokens, "graphs": not args.direct},
        "us_per_token": round(us_tok, 3),
        "launches_per_token": int(sum(launches.values())),
        "wall_s": round(wall, 3),
        "step_roofline": {"bytes_per_token": int(step_bytes), "achieved": round(step_gbs, 1),
                          "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
    }
    if chain_timing:
        # the fused QKV + attention launch is the largest kernel of the step
        dom = "qkv" if "attn" not in algo else "attn"
        dur_us = us[dom]
        achieved = algo[dom] / (dur_us * 1e-6) / 1e9
        traffic, tsrc = None, "no completed counter pass of this kernel in " + os.path.relpath(PROFILE_C0, ROOT)
        fused = dom == "qkv" and fuse_level == 3 and not args.kv16
        if fused:
            c = profiled_traffic("k_qkv_attn<768, 1, float, 64, true, 2048>")
            if c:
                traffic = c["fetch"] + c["write"]
                tsrc = (f"FETCH_SIZE + WRITE_SIZE of {c['kernel']} per dispatch, rocprofv3 --pmc "
                        f"(one counter per run, each scaled by the same counter over a known device copy), "
                        f"{os.path.relpath(PROFILE_C0, ROOT)}")
        out["roofline"] = {"bound": "hbm", "kernel": "k_qkv_attn" if dom == "qkv" else dom,
                           "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                           "traffic_source": tsrc,
                           "bytes_per_launch": int(algo[dom]), "launch_us": round(dur_us, 3),
                           "launch_us_source": "device start/end timestamps of every dispatch of the "
                                               "kernel over the 254 decode steps of one sequence, direct "
                                               "launches (lm_profile_chain: hipExtLaunchKernelGGL events); "
                                               "the kernel trace of the same dispatches is in "
                                               + os.path.relpath(PROFILE_C0, ROOT)}
        out["kernel_us_per_launch"] = {k: round(v, 3) for k, v in us.items() if launches.get(k)}
    if not args.no_extra:
        out["configs"] = bench_extra(S, w16, direct=args.direct)
        progress("C0 in the reference's algorithm (window recompute) on the GPU")
        ra = reference_algorithm_gpu(S, cfg, w16, ids)
        out["configs"]["c0_reference_algorithm"] = ra
        if not args.kv16:
            progress("C0 with the binary16 K/V cache")
            out["configs"]["c0_kv16"] = c0_kv16(S, cfg, w16, ids, args.direct)
            progress("C0 warm and cold (Infinity Cache sweep) tokens")
            out["configs"]["c0_cold_cache"] = c0_cold_cache(S, cfg, w16, ids)
        progress("device copy rate")
        out["device_copy_rate"] = device_copy_rate()
        out["vs_baseline_same_algorithm"] = round(ra["value"] / REF_TOK_S, 1)
    if not args.no_cpu:
        progress("CPU baseline (oracle/cpu_ref.c with OpenBLAS)")
        out["cpu_baseline"] = cpu_baseline(cfg.astuple(), w16, S, ids, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    progress("done")


if __name__ == "__main__":
    main()
