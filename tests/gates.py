"""Correctness gates shared by the GPU parity tests.

Identical argmax choice per choice question, answer probabilities within 5e-3 absolute (after the
f64 temperature softmax of decode.rs), final hidden states within 2e-2 relative per real token
(||gpu - ref|| / ||ref||).
"""
from __future__ import annotations

import numpy as np

from sys1rust_amd.decode import decode_answers
from sys1rust_amd.workloads import Batch

HIDDEN_REL_GATE = 2e-2
PROB_ABS_GATE = 5e-3


def say(*a):
    print(*a, flush=True)


def hidden_rel(gpu_hidden: np.ndarray, ref: np.ndarray, b: Batch) -> float:
    g = gpu_hidden.reshape(b.n, b.len, -1)
    am = b.attention_mask.reshape(b.n, b.len).astype(bool)
    d = np.linalg.norm(g[am] - ref[am], axis=-1) / np.linalg.norm(ref[am], axis=-1)
    return float(d.max())


def check_answers(lg_gpu, lg_ref, b: Batch, tag: str):
    a = decode_answers(lg_gpu, b.kmax, b.marker_count, b.qtype)
    r = decode_answers(lg_ref, b.kmax, b.marker_count, b.qtype)
    worst = 0.0
    for i, (x, y) in enumerate(zip(a, r)):
        worst = max(worst, float(np.abs(x["probabilities"] - y["probabilities"]).max()))
        if x["type"] == "choice":
            p = np.sort(y["probabilities"])
            margin = p[-1] - p[-2]
            say(f"{tag} row {i}: choice gpu={x['choice']} oracle={y['choice']} margin={margin:.2e}")
            assert x["choice"] == y["choice"], (tag, i, x["probabilities"], y["probabilities"])
    say(f"{tag}: max |dp| = {worst:.2e}")
    assert worst <= PROB_ABS_GATE, (tag, worst)
    return worst
