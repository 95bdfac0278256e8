"""Answer-position decode on the CPU: `decode_answers` of
runtime/crates/laya-core/src/decode.rs:309-399 (probabilities and typed answers only; the act
head and JSON rendering are not on this path).

For each question row r with k = marker_count[r] options: z = logits[r, :k] / T, T the clamped
temperature of the (qtype, k) bucket (decode.rs:16-86); p = softmax in f64; choice = argmax with
the first maximum winning (decode.rs:335-338), score = sum_i i * p_i, noul = p[1].
"""
from __future__ import annotations

import math

import numpy as np

TEMP_MIN, TEMP_MAX = 0.5, 5.0
QTYPE_NAMES = ["choice", "score", "noul"]


def clamp_temperature(v) -> float:
    """decode.rs:19-30."""
    try:
        if isinstance(v, bool):
            t = 1.0 if v else 0.0
        elif isinstance(v, str):
            t = float(v.strip())
        else:
            t = float(v)
    except (TypeError, ValueError):
        return 1.0
    if not math.isfinite(t):
        return 1.0
    return min(max(t, TEMP_MIN), TEMP_MAX)


def temp_bucket(qtype: int, k: int) -> str:
    """decode.rs:71-82."""
    size = "2" if k <= 2 else "3-5" if k <= 5 else "6-10" if k <= 10 else "11+"
    return f"{QTYPE_NAMES[qtype]}:{size}"


def softmax_f64(z: np.ndarray) -> np.ndarray:
    """decode.rs:95-100."""
    m = np.max(z)
    e = np.exp(z - m)
    return e / e.sum()


def decode_answers(logits: np.ndarray, kmax: int, marker_count, qtype, temperature=(1.0, 1.0, 1.0),
                   temperature_by_options: dict | None = None):
    by_type = [clamp_temperature(t) for t in temperature]
    by_opt = {k: clamp_temperature(v) for k, v in (temperature_by_options or {}).items()}
    out = []
    for r in range(len(qtype)):
        k = int(marker_count[r])
        qt = int(qtype[r])
        t = by_opt.get(temp_bucket(qt, k), by_type[qt])
        z = logits[r * kmax: r * kmax + k].astype(np.float64) / t
        p = softmax_f64(z) if k else np.zeros(0)
        ans = {"type": QTYPE_NAMES[qt], "probabilities": p}
        if qt == 0:
            best = 0
            for i in range(k):
                if p[i] > p[best]:
                    best = i
            ans["choice"] = best
        elif qt == 1:
            ans["score"] = float(sum(i * x for i, x in enumerate(p)))
        else:
            ans["noul"] = float(p[1]) if k > 1 else 0.0
        out.append(ans)
    return out
