"""Answer-position decode on the CPU: `decode_answers` of
runtime/crates/laya-core/src/decode.rs:309-399, with the action head (decode.rs:117-259); the
JSON rendering of labels is not on this path.

For each question row r with k = marker_count[r] options: z = logits[r, :k] / T, T the clamped
temperature of the (qtype, k) bucket (decode.rs:16-86); p = softmax in f64; choice = argmax with
the first maximum winning (decode.rs:335-338), score = sum_i i * p_i, noul = p[1];
confidence = 1 - H(p) / ln k (decode.rs:88-94) on choice and score, max(p_yes, p_no) on noul;
answer_confidence = the probability of the reported answer. With an action head,
act_probability = ActHead.probs(pooled[r], act_features(logits[r], k))[0] (decode.rs:319-331), the
head's rows evaluated together.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf as _erf

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


def confidence_from_probs(p, k: int) -> float:
    """decode.rs:88-94: normalised Shannon-entropy confidence 1 - H(p) / ln k, in [0, 1]."""
    if k < 2:
        return 1.0
    ent = float(sum(-x * math.log(min(max(x, 1e-12), 1.0)) for x in p[:k]))
    return min(max(1.0 - ent / math.log(k), 0.0), 1.0)


def gelu_f64(x):
    """decode.rs:111-115: exact-erf GELU evaluated in f64, returned as f32."""
    xf = np.asarray(x, dtype=np.float64)
    return (0.5 * xf * (1.0 + _erf(xf / math.sqrt(2.0)))).astype(np.float32)


def softmax_f32(z) -> np.ndarray:
    """decode.rs:104-109."""
    z = np.asarray(z, dtype=np.float32)
    e = np.exp(z - z.max()).astype(np.float32)
    return (e / e.sum(dtype=np.float32)).astype(np.float32)


def act_features(logits_row, marker_count: int) -> np.ndarray:
    """decode.rs:250-259: [top1, top1 - top2, normalised entropy, k / 255] of the softmax over the
    whole masked logits row (masked slots hold -1e4 and weigh nothing), k = max(marker_count, 2).
    An empty row (kmax 0) has no probabilities: top1 = top2 = 0 and the entropy sum is -0.0."""
    k = np.float32(max(int(marker_count), 2))
    if np.asarray(logits_row).size == 0:  # a batch without answer slots: no probabilities
        return np.array([0.0, 0.0, -0.0, k / np.float32(255.0)], dtype=np.float32)
    p = softmax_f32(logits_row)
    ent = np.float32(-(p * np.log(np.maximum(p, np.float32(1e-9)))).sum(dtype=np.float32) / np.log(k))
    srt = np.sort(p)[::-1]
    top1 = srt[0] if srt.size else np.float32(0)
    top2 = srt[1] if srt.size > 1 else np.float32(0)
    return np.array([top1, top1 - top2, ent, k / np.float32(255.0)], dtype=np.float32)


def act_features_rows(logits, kmax: int, marker_count) -> np.ndarray:
    """act_features of every row of a [n * kmax] logits buffer at once -> [n, 4]."""
    n = len(marker_count)
    if kmax == 0:
        return np.stack([act_features(np.zeros(0, np.float32), c) for c in marker_count]).reshape(n, 4)
    z = np.asarray(logits, dtype=np.float32)[: n * kmax].reshape(n, kmax)
    e = np.exp(z - z.max(axis=1, keepdims=True)).astype(np.float32)
    p = (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    k = np.maximum(np.asarray(marker_count, dtype=np.int64), 2).astype(np.float32)
    ent = (-(p * np.log(np.maximum(p, np.float32(1e-9)))).sum(axis=1, dtype=np.float32) / np.log(k)).astype(np.float32)
    srt = -np.sort(-p, axis=1)
    top1 = srt[:, 0] if kmax else np.zeros(n, np.float32)
    top2 = srt[:, 1] if kmax > 1 else np.zeros(n, np.float32)
    return np.stack([top1, top1 - top2, ent, k / np.float32(255.0)], axis=1).astype(np.float32)


class ActHead:
    """decode.rs:117-246: act_head = Linear(d + 4, hidden) -> GELU -> Linear(hidden, n_act) ->
    softmax, on the CPU in f32, from the checkpoint's act_head.{0,2}.{weight,bias}."""

    def __init__(self, w0, b0, w2, b2):
        w0, b0, w2, b2 = (np.asarray(a, dtype=np.float32) for a in (w0, b0, w2, b2))
        if w0.ndim != 2 or w2.ndim != 2 or w2.shape[1] != w0.shape[0]:
            raise ValueError(f"act_head shapes {w0.shape} / {w2.shape} are not a 2-layer MLP")
        if w0.shape[1] <= 4:
            raise ValueError("act_head.0.weight needs an input width of at least 5")
        if b0.shape != (w0.shape[0],) or b2.shape != (w2.shape[0],):
            raise ValueError("act_head biases do not match their layers")
        self.w0, self.b0, self.w2, self.b2 = w0, b0, w2, b2
        self.d_in, self.hidden, self.n_act = w0.shape[1], w0.shape[0], w2.shape[0]

    @classmethod
    def from_weights(cls, w: dict) -> "ActHead":
        return cls(w["act_head.0.weight"], w["act_head.0.bias"], w["act_head.2.weight"], w["act_head.2.bias"])

    @classmethod
    def from_safetensors(cls, st: bytes) -> "ActHead":
        """The act_head tensors of a safetensors image (F32, F16 or BF16), read as laya-core reads
        them at load (decode.rs:130-136)."""
        import json
        import struct

        n = struct.unpack("<Q", st[:8])[0]
        header = json.loads(st[8:8 + n])
        w = {}
        for name in ("act_head.0.weight", "act_head.0.bias", "act_head.2.weight", "act_head.2.bias"):
            if name not in header:
                raise ValueError(f"checkpoint has no {name}")
            e = header[name]
            a, z = (8 + n + o for o in e["data_offsets"])
            raw = st[a:z]
            if e["dtype"] == "F32":
                v = np.frombuffer(raw, np.float32)
            elif e["dtype"] == "F16":
                v = np.frombuffer(raw, np.float16).astype(np.float32)
            elif e["dtype"] == "BF16":
                v = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
            else:
                raise ValueError(f"{name}: dtype {e['dtype']} is not F32, F16 or BF16")
            w[name] = v.reshape(e["shape"])
        return cls.from_weights(w)

    def pooled_width(self) -> int:
        return self.d_in - 4

    def probs(self, pooled, feats) -> np.ndarray:
        return self.probs_rows(np.asarray(pooled, dtype=np.float32)[None], np.asarray(feats, dtype=np.float32)[None])[0]

    def probs_rows(self, pooled, feats) -> np.ndarray:
        """probs() of every row at once: pooled [n, d], feats [n, 4] -> [n, n_act]."""
        x = np.concatenate([np.asarray(pooled, dtype=np.float32), np.asarray(feats, dtype=np.float32)], axis=1)
        h = gelu_f64((x @ self.w0.T + self.b0).astype(np.float32))
        out = (h @ self.w2.T + self.b2).astype(np.float32)
        e = np.exp(out - out.max(axis=1, keepdims=True)).astype(np.float32)
        return (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)


def round_dp(x: float, n: int = 4) -> float:
    return round(float(x), n)


# From this many rows on, the [n, kmax] array form is faster than a loop over the rows (numpy's
# fixed cost per call outweighs a short loop: one row takes 9 µs looped, 36 µs as arrays).
VECTOR_ROWS = 4


def _answers_looped(logits, kmax: int, ks, qts, temps):
    """Softmax, choice, confidence, score and noul row by row (decode.rs:309-399)."""
    out = []
    for r, (k, qt, t) in enumerate(zip(ks, qts, temps)):
        z = logits[r * kmax: r * kmax + k].astype(np.float64) / t
        p = softmax_f64(z) if k else np.zeros(0)
        if qt == 2:  # noul reads p[1] alone
            out.append((p, 0, 0.0, 0.0, 0.0, float(p[1]) if k > 1 else 0.0))
            continue
        best = 0
        for i in range(k):  # the first maximum wins (decode.rs:335-338)
            if p[i] > p[best]:
                best = i
        score = float(sum(i * x for i, x in enumerate(p))) if qt == 1 else 0.0
        out.append((p, best, confidence_from_probs(p, k), float(p[best]) if k else 0.0, score, 0.0))
    return out


def _answers_arrays(logits, kmax: int, ks, qts, temps):
    """The same as [n, kmax] arrays, the slots past a row's k masked out (a probability of 0 that
    adds nothing), read out row by row."""
    n = len(ks)
    z = np.asarray(logits)[: n * kmax].reshape(n, kmax).astype(np.float64) / np.asarray(temps)[:, None]
    valid = np.arange(kmax)[None, :] < np.asarray(ks, dtype=np.int64)[:, None]
    zm = np.where(valid, z, -np.inf)
    m = zm.max(axis=1, keepdims=True)
    e = np.exp(zm - np.where(np.isfinite(m), m, 0.0))  # rows without options: all zeros
    tot = e.sum(axis=1, keepdims=True)
    P = e / np.where(tot > 0.0, tot, 1.0)
    # decode.rs:88-94 per row: 1 - H(p) / ln k, clamped to [0, 1]; 1 for k < 2
    ent = -(P * np.log(np.clip(P, 1e-12, 1.0))).sum(axis=1)
    lnk = np.log(np.maximum(np.asarray(ks, dtype=np.float64), 2.0))
    conf = np.where(np.asarray(ks) < 2, 1.0, np.clip(1.0 - ent / lnk, 0.0, 1.0))
    best = P.argmax(axis=1)  # the first maximum wins (decode.rs:335-338)
    pbest = P[np.arange(n), best]
    score = (P * np.arange(kmax, dtype=np.float64)[None, :]).sum(axis=1)
    p1 = P[:, 1] if kmax > 1 else np.zeros(n)
    return [(P[r, :k], int(best[r]) if k else 0, float(conf[r]) if k else 1.0, float(pbest[r]) if k else 0.0,
             float(score[r]) if k else 0.0, float(p1[r]) if k > 1 else 0.0) for r, k in enumerate(ks)]


def decode_answers(logits: np.ndarray, kmax: int, marker_count, qtype, temperature=(1.0, 1.0, 1.0),
                   temperature_by_options: dict | None = None, pooled=None, act_head: ActHead | None = None):
    by_type = [clamp_temperature(t) for t in temperature]
    by_opt = {k: clamp_temperature(v) for k, v in (temperature_by_options or {}).items()}
    n = len(qtype)
    ks = [int(c) for c in marker_count[:n]]
    qts = [int(q) for q in qtype[:n]]
    act = None
    if act_head is not None:
        # The action head of every row in one product (the rows are independent).
        d = act_head.pooled_width()
        feats = act_features_rows(logits, kmax, marker_count)
        act = act_head.probs_rows(np.asarray(pooled, dtype=np.float32)[: n * d].reshape(n, d), feats)
    temps = [by_opt.get(temp_bucket(q, k), by_type[q]) for q, k in zip(qts, ks)]
    if kmax and n >= VECTOR_ROWS:
        rows = _answers_arrays(logits, kmax, ks, qts, temps)
    else:
        rows = _answers_looped(logits, kmax, ks, qts, temps)
    out = []
    for r, (p, best, conf, pbest, score, p1) in enumerate(rows):
        qt = qts[r]
        ans = {"type": QTYPE_NAMES[qt], "probabilities": p}
        if qt == 0:
            ans["choice"] = best
            ans["confidence"] = conf
            ans["answer_confidence"] = pbest
        elif qt == 1:
            ans["score"] = score
            ans["confidence"] = conf
            ans["answer_confidence"] = pbest
        else:
            ans["noul"] = p1
            ans["confidence"] = ans["answer_confidence"] = max(p1, 1.0 - p1)
        if act is not None:
            ans["act_probability"] = float(act[r, 0])
        out.append(ans)
    return out
