"""The dtype=f32 path (the reference's BackendOptions::f32, runtime/crates/laya-core/src/backend.rs:
25-27, checked upstream by laya-mlx/tests/parity.rs:54-65) against the oracle, which is f32 too.

Both sides compute in float32 with the same f32 weights, so the gates here are tighter than the
16-bit path's: hidden states within 1e-3 relative per position, logits within 1e-3 absolute,
pooled rows within 1e-3 relative, answer probabilities within 1e-4, every decision identical.
The differences left are summation order (GEMM k order, softmax sums) and the erf and exp
implementations.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from oracle.torch_ref import TorchOracle
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, synth_checkpoint
from sys1rust_amd.decode import ActHead, decode_answers
from sys1rust_amd.workloads import AGENT, MODERNBERT_LARGE, Batch, workload

from gates import decisive_checkpoint, hidden_rel, random_batch, say

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
HIDDEN_REL_F32 = 1e-3
LOGIT_ABS_F32 = 1e-3
POOLED_REL_F32 = 1e-3
PROB_ABS_F32 = 1e-4


def gate_f32(m, b, ref_hidden, lg_ref, pl_ref, act, tag, padding=True):
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    rel = hidden_rel(hid, ref_hidden, b, padding=padding)
    out = m.forward(b)
    dl = float(np.abs(out.logits - lg_ref).max()) if b.kmax else 0.0
    pg, pr = out.pooled.reshape(b.n, -1), pl_ref.reshape(b.n, -1)
    dp = float((np.linalg.norm(pg - pr, axis=-1) / np.linalg.norm(pr, axis=-1)).max())
    dprob = dact = 0.0
    same = True
    if b.kmax:  # answers need answer slots
        a = decode_answers(out.logits, b.kmax, b.marker_count, b.qtype, pooled=out.pooled, act_head=act)
        r = decode_answers(lg_ref, b.kmax, b.marker_count, b.qtype, pooled=pl_ref, act_head=act)
        dprob = max((float(np.abs(x["probabilities"] - y["probabilities"]).max()) for x, y in zip(a, r)
                     if len(y["probabilities"])), default=0.0)
        dact = max(abs(x["act_probability"] - y["act_probability"]) for x, y in zip(a, r))
        same = all(x.get("choice") == y.get("choice") for x, y in zip(a, r))
    say(f"{tag}: hidden rel {rel:.2e}, logits {dl:.2e}, pooled rel {dp:.2e}, probabilities {dprob:.2e}, "
        f"act {dact:.2e}, choices identical {same}")
    assert rel <= HIDDEN_REL_F32, (tag, rel)
    assert dl <= LOGIT_ABS_F32, (tag, dl)
    assert dp <= POOLED_REL_F32, (tag, dp)
    assert dprob <= PROB_ABS_F32 and dact <= PROB_ABS_F32, (tag, dprob, dact)
    assert same, tag


@pytest.fixture(scope="module")
def small():
    z = np.load(GOLDEN / "golden_small.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    return cfg, agent, st, b


@pytest.mark.parametrize("settings", ["", "mask=bool,dense_upto=0", "band=1,fuserope", DEFAULT_TUNING])
def test_f32_small_model_matches_the_oracle(small, settings):
    """The golden batch (3 ragged rows, window 16) at every position, padding included, and the
    forward's logits, pooled rows and answers, under several mask paths."""
    cfg, agent, st, b = small
    spec = ",".join(x for x in [settings, "dtype=f32"] if x)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=spec)
    assert m.name() == "hip(gfx950,f32)"
    assert m.active_kernels() == []  # the plain f32 kernels only
    o = O.Oracle(st, cfg, agent, settings=settings)
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    gate_f32(m, b, ref, lg, pl, ActHead.from_weights(o.w), f"f32 small {settings[:30]!r}")
    m.close()


def test_f32_short_rows_and_no_markers(small):
    """Rows of 1, 3 and 9 tokens, and a batch without answer markers (kmax 0)."""
    cfg, agent, st, _ = small
    lens, L = [1, 3, 9], 9
    rng = np.random.default_rng(7)
    ids = rng.integers(5, 1000, size=(3, L)).astype(np.uint32)
    am = np.zeros((3, L), np.uint32)
    for r, n in enumerate(lens):
        am[r, :n] = 1
        ids[r, n:] = 1002
    o = O.Oracle(st, cfg, agent)
    act = ActHead.from_weights(o.w)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f32")
    for kmax, mp, mc in [(2, [[0, 0], [2, 0], [4, 8]], [0, 1, 2]), (0, None, [0, 0, 0])]:
        b = Batch(3, L, kmax, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64),
                  np.array(mp, np.uint32).reshape(-1) if mp else np.zeros(0, np.uint32), np.array(mc, np.uint64),
                  np.array([0, 1, 2], np.uint32))
        ref = o.encoder_hidden(b)
        lg, pl = o.forward(b, ref)
        gate_f32(m, b, ref, lg, pl, act, f"f32 short rows kmax={kmax}")
    m.close()


def test_f32_modernbert_large_512_tokens():
    """The 28-layer ModernBERT-large shape over a 512-token state with one question, and a padded
    600-position batch at every position (chunked local attention for the padding), against the
    oracle's torch f32 restatement on the GPU."""
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    m = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings="dtype=f32")
    o = O.Oracle(st, MODERNBERT_LARGE, AGENT)
    t = TorchOracle(o, "cuda")
    act = ActHead.from_weights(o.w)
    b = workload("state512_1q", seed=5)
    say(f"f32 large: n={b.n} len={b.len} T={b.total_tokens()}")
    ref = t.encoder_hidden(b)
    lg, pl = t.forward(b, ref)
    gate_f32(m, b, ref, lg, pl, act, "f32 large state512_1q")
    lens, L = [600, 300, 20], 600
    rng = np.random.default_rng(17)
    ids = rng.integers(5, 50000, size=(3, L)).astype(np.uint32)
    am = np.zeros((3, L), np.uint32)
    for r, n in enumerate(lens):
        am[r, :n] = 1
        ids[r, n:] = 50283
    bp = Batch(3, L, 0, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64), np.zeros(0, np.uint32),
               np.zeros(3, np.uint64), np.zeros(3, np.uint32))
    rel = hidden_rel(m.encoder_hidden(bp).reshape(3, L, -1), t.encoder_hidden(bp), bp, padding=True)
    say(f"f32 large padded 600: hidden rel at every position {rel:.2e}")
    assert rel <= HIDDEN_REL_F32, rel
    m.close()


def test_f32_mmbert_golden_batch():
    """The mmBERT-base shape (hidden 768, 12 heads, GeGLU 1152) on its golden fixture's batch,
    against the oracle at every position, padding included."""
    z = np.load(GOLDEN / "golden_mmbert.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f32")
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    gate_f32(m, b, ref, lg, pl, ActHead.from_weights(o.w), "f32 mmbert golden")
    m.close()


@pytest.mark.parametrize("case", ["golden_small", "golden_large", "golden_mmbert"])
def test_f32_against_the_independent_fixtures(case):
    """The f32 option straight against the golden fixtures written by transformers'
    ModernBertModel (hidden states) and torch's TransformerEncoderLayer head and scorer (logits,
    pooled rows), at the tolerances the oracle itself meets against them."""
    z = np.load(GOLDEN / f"{case}.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f32")
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    sel = z["hidden_sel"]
    g = hid[sel[:, 0], sel[:, 1]]
    rel = float((np.linalg.norm(g - z["hidden"], axis=-1) / np.linalg.norm(z["hidden"], axis=-1)).max())
    out = m.forward(b)
    dl = float(np.abs(out.logits - z["logits"]).max())
    pg, pr = out.pooled.reshape(b.n, -1), z["pooled"].reshape(b.n, -1)
    dp = float((np.linalg.norm(pg - pr, axis=-1) / np.linalg.norm(pr, axis=-1)).max())
    say(f"f32 {case} against the fixture: hidden rel {rel:.2e}, logits {dl:.2e}, pooled rel {dp:.2e}")
    assert rel < 1e-4 and dl < 1e-5 and dp < 1e-4, (rel, dl, dp)
    m.close()


def test_f32_random_batches(small):
    """Six of the seeded random batches (ragged rows of 1-300 tokens, 0-6 answer slots) on the
    decisive-scorer checkpoint, every position of encoder_hidden included."""
    cfg, agent, st, _ = small
    st = decisive_checkpoint(st)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f32")
    o = O.Oracle(st, cfg, agent)
    act = ActHead.from_weights(o.w)
    rng = np.random.default_rng(20261202)
    for case in range(6):
        b = random_batch(rng, cfg["vocab_size"], cfg["pad_token_id"])
        ref = o.encoder_hidden(b)
        lg, pl = o.forward(b, ref)
        gate_f32(m, b, ref, lg, pl, act, f"f32 random {case} n={b.n} len={b.len} kmax={b.kmax}")
    m.close()
