"""Decode-step driver for kernel profiling (run it under rocprofv3).

    python3 -m undertow_amd.profile_decode --config c4 --prompt 512 --tokens 32

Builds the synthetic model on the device, prefills a uniform-random prompt,
then runs `--tokens` single-row decode steps and `--tokens // 2` two-row
verify steps (the MTP verify width at depth 1), each phase separated from
the next by an idle second so a kernel trace splits cleanly at the gaps.
Prints the host-timed ms per step of each phase.
"""
from __future__ import annotations

import argparse
import sys
import time
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c4", choices=["c1", "c4"])
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--tokens", type=int, default=32)
    ap.add_argument("--seed", type=int, default=42)
    args = ap.parse_args()

    import numpy as np
    import torch
    import undertow_amd as U
    from undertow_amd.configs import C1, C4

    cfg = {"c1": C1, "c4": C4}[args.config]
    ctx = U.Context(0)
    m = U.Model(ctx, cfg)
    m.synthesize(args.seed, 0.02, U.INT4, U.INT8)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg["vocab_size"], args.prompt).tolist()
    s = m.session()
    s.prefill(prompt, want_logits=False)
    nxt = s.last_argmax[-1]
    torch.cuda.synchronize()
    time.sleep(1.0)
    t0 = time.perf_counter()
    for _ in range(args.tokens):
        s.prefill([nxt], want_logits=False)
        nxt = s.last_argmax[-1]
    t1 = time.perf_counter()
    print(f"decode {args.tokens} tokens: {(t1 - t0) / args.tokens * 1e3:.3f} ms/token", flush=True)
    torch.cuda.synchronize()
    time.sleep(1.0)
    n = max(args.tokens // 2, 1)
    t0 = time.perf_counter()
    for _ in range(n):
        s.prefill([nxt, nxt], want_logits=False)
        nxt = s.last_argmax[-1]
    t1 = time.perf_counter()
    print(f"verify (2 rows) {n} steps: {(t1 - t0) / n * 1e3:.3f} ms/step", flush=True)


if __name__ == "__main__":
    main()
