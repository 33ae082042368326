"""Benchmark of the Stories-110M token loop on one MI355X (first version).

A step is one greedy decode token at batch 1 (config C0: 256-token sequences
from token id 1, fp32 accumulation, fp32 K/V cache), replayed as captured
hipGraphs with the argmax fed back on the device.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "ane-training_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--path", type=int, default=0)
    ap.add_argument("--direct", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import stories_lm as S
    rc = S.init()
    if rc:
        raise SystemExit(f"lm_init: {S.strerror(rc)}")
    cfg = S.make_config(**S.STORIES_110M)
    w16 = S.synth_weights_f16(cfg, 1, 0.02, True)
    m = S.Model.create(cfg, w16, True, 1, 256)
    m.set_option(S.LM_OPT_KV_F32, 1)
    if args.direct:
        m.set_option(S.LM_OPT_USE_GRAPH, 0)
    if args.path:
        m.set_option(S.LM_OPT_DECODE_PATH, args.path)

    def run(n):
        done = 0
        while done < n:
            k = min(256, n - done)
            m.generate_greedy([1], [0], k)
            done += k

    run(args.warmup)
    m.sync()
    m.timer_begin()
    t0 = time.perf_counter()
    run(args.steps)
    ms = m.timer_end()
    wall = time.perf_counter() - t0
    tok_s = args.steps / (ms / 1e3)
    print(json.dumps({"metric": "Stories-110M decode tok/s at B=1", "value": round(tok_s, 1),
                      "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "ms_per_step": ms / args.steps, "wall_s": wall, "higher_is_better": True}),
          flush=True)


if __name__ == "__main__":
    main()
