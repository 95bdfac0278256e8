"""A/B of whole requests across builds of libsys1hip.so in one process on one GPU.

Each build loads the same seeded synthetic ModernBERT-large checkpoint with sys1rust's
DEFAULT_TUNING settings; for every shape the builds are timed in turn (A B, then B A, ...),
`--steps` forwards each after 3 warm-ups, and the median forward time of each round is kept, so
that the drift of one box between runs cancels. The logits and pooled rows of every build are
compared with the first build's (0 when the kernels are the same bits).

Run on the GPU host from the repo root, e.g. with a second build copied beside the first:
  python3 sys1rust_amd/microbench/request_ab.py sys1rust_amd/libsys1hip.so /tmp/other/libsys1hip.so
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from sys1rust_amd import _lib  # noqa: E402
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, synth_checkpoint  # noqa: E402
from sys1rust_amd.workloads import AGENT, MODERNBERT_LARGE, SCORER_WIDTH, workload  # noqa: E402


def load(path: str) -> C.CDLL:
    lib = C.CDLL(os.path.abspath(path))
    for name, (res, args) in _lib.SIGNATURES.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("libs", nargs="+", help="builds of libsys1hip.so")
    ap.add_argument("--shapes", default="state128_1q,state512_1q,state512_10q")
    ap.add_argument("--rounds", type=int, default=4)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--settings", default=DEFAULT_TUNING)
    ap.add_argument("--seed", type=int, default=2024)
    a = ap.parse_args()

    import torch

    assert torch.cuda.is_available(), "needs a GPU"
    libs = [(p, load(p)) for p in a.libs]
    enc, ag = json.dumps(MODERNBERT_LARGE), json.dumps(AGENT)
    # The backend module calls _lib.lib(); pointing it at a build before each call routes the call
    # (and the model handle it uses) to that build.
    _lib._lib = libs[0][1]
    ckpt = synth_checkpoint(enc, ag, seed=a.seed, scorer_width=SCORER_WIDTH)
    models = {}
    for p, lib in libs:
        _lib._lib = lib
        m = HipBackend(ckpt, enc, ag, settings=a.settings)
        m.warmup()
        models[p] = m
        print(f"{p}: {m.active_kernels()}", flush=True)
    for shape in a.shapes.split(","):
        b = workload(shape, seed=a.seed)
        times = {p: [] for p, _ in libs}
        outs = {}
        for r in range(a.rounds):
            for p, lib in (libs if r % 2 == 0 else libs[::-1]):
                _lib._lib = lib
                m = models[p]
                for _ in range(3):
                    m.forward(b)
                ts = []
                for _ in range(a.steps):
                    t0 = time.perf_counter()
                    out = m.forward(b)
                    ts.append((time.perf_counter() - t0) * 1e3)
                times[p].append(float(np.median(ts)))
                outs[p] = out
        first = libs[0][0]
        for p, _ in libs:
            v = sorted(times[p])
            dl = float(np.abs(outs[p].logits - outs[first].logits).max()) if outs[p].logits.size else 0.0
            dp = float(np.abs(outs[p].pooled - outs[first].pooled).max())
            print(f"{shape} {p}: forward {v[len(v) // 2]:.4f} ms (median of round medians; rounds "
                  f"{' '.join(f'{x:.3f}' for x in times[p])}); max |logit - first| {dl:.2e}, "
                  f"max |pooled - first| {dp:.2e}", flush=True)
    for p, lib in libs:
        _lib._lib = lib
        models[p].close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
