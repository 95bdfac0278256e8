"""The multilingual checkpoint's encoder shape on the GPU: mmBERT-base (22 layers, hidden 768,
12 heads, GeGLU 1152, vocabulary 256,000), with its 12-head decision head and a 768-wide scorer,
served by sys1rust like the English checkpoints (runtime/crates/sys1rust/src/config.rs:31-35;
the reference's parity suite for it is laya-mlx/tests/parity.rs:68-80).

Gates as for ModernBERT-large (tests/gates.py): against the golden fixture written by
transformers' ModernBertModel at this shape, and against the oracle on every row of a 1- and a
10-question request over a 512-token state.
"""
from __future__ import annotations

import copy
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, synth_checkpoint
from sys1rust_amd.decode import ActHead
from sys1rust_amd.workloads import MMBERT_BASE, Batch, workload

from gates import FUSED, HIDDEN_REL_GATE, gate_model, hidden_rel, random_batch, say

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
AGENT_ML = {"head_layers": 2, "max_len": 1024, "head_max_len": 256}


def test_mmbert_golden_batch():
    """The fixture's ragged 2-row batch: hidden states against transformers' values, and every
    gate against the oracle."""
    z = np.load(GOLDEN / "golden_mmbert.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    assert (cfg["hidden_size"], cfg["num_attention_heads"], cfg["intermediate_size"]) == (768, 12, 1152)
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    say("mmbert golden: create")
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
    assert m.active_kernels() == FUSED
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    sel = z["hidden_sel"]
    g = hid[sel[:, 0], sel[:, 1]]
    gr = float((np.linalg.norm(g - z["hidden"], axis=-1) / np.linalg.norm(z["hidden"], axis=-1)).max())
    say(f"mmbert golden: hidden rel vs transformers {gr:.3e}")
    assert gr <= HIDDEN_REL_GATE, gr
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    gate_model(m, b, ref, lg, pl, ActHead.from_weights(o.w), "mmbert golden batch")
    m.close()


@pytest.fixture(scope="module")
def mmbert():
    say("mmbert: synth checkpoint")
    st = synth_checkpoint(json.dumps(MMBERT_BASE), json.dumps(AGENT_ML), seed=99, scorer_width=768)
    say("mmbert: create")
    m = HipBackend(st, json.dumps(MMBERT_BASE), json.dumps(AGENT_ML), settings=DEFAULT_TUNING)
    o = O.Oracle(st, MMBERT_BASE, AGENT_ML)
    return m, o, st, ActHead.from_weights(o.w)


@pytest.mark.parametrize("name", ["state128_1q", "state512_1q", "state512_10q"])
def test_mmbert_base_requests_every_row(mmbert, name):
    m, o, st, act = mmbert
    b = workload(name, seed=2, agent=AGENT_ML)
    say(f"mmbert {name}: n={b.n} len={b.len} T={b.total_tokens()}")
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    gate_model(m, b, ref, lg, pl, act, f"mmbert {name}")


def test_mmbert_random_batches(mmbert):
    """Four seeded random batches (1-9 ragged rows of 1-300 tokens, 0-6 answer slots) at this
    shape, whose 128-token local window is the widest the staged local kernel takes."""
    m, o, st, act = mmbert
    rng = np.random.default_rng(768)
    for case in range(4):
        b = random_batch(rng, MMBERT_BASE["vocab_size"], MMBERT_BASE["pad_token_id"])
        tag = f"mmbert random {case}: n={b.n} len={b.len} kmax={b.kmax} T={b.total_tokens()}"
        say(tag)
        ref = o.encoder_hidden(b)
        lg, pl = o.forward(b, ref)
        gate_model(m, b, ref, lg, pl, act, tag)


def test_mmbert_base_f16(mmbert):
    """dtype=f16 (the checkpoint's stored type) at this shape: gates against the oracle."""
    m, o, st, act = mmbert
    m16 = HipBackend(st, json.dumps(MMBERT_BASE), json.dumps(AGENT_ML), settings=DEFAULT_TUNING + ",dtype=f16")
    # Every fused kernel passes its load check at this width, in both types.
    assert m16.active_kernels() == FUSED and m.active_kernels() == FUSED, (m16.active_kernels(), m.active_kernels())
    b = workload("state512_1q", seed=3, agent=AGENT_ML)
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    gate_model(m16, b, ref, lg, pl, act, "mmbert f16 state512_1q")
    m16.close()


@pytest.mark.parametrize("settings", ["", DEFAULT_TUNING + ",dtype=f16"])
def test_mmbert_encoder_hidden_padding_positions(mmbert, settings):
    """encoder_hidden at every position at this shape (window 64): a 300-position padded length,
    chunked local attention under the default settings and dense under DEFAULT_TUNING
    (dense_upto=1024), rows of 300, 40 and 2 real tokens, against the oracle under the same
    settings."""
    _, o0, st, _ = mmbert
    lens, L = [300, 40, 2], 300
    rng = np.random.default_rng(23)
    ids = rng.integers(5, 250000, size=(len(lens), L)).astype(np.uint32)
    am = np.zeros((len(lens), L), np.uint32)
    for r, l in enumerate(lens):
        am[r, :l] = 1
        ids[r, l:] = MMBERT_BASE["pad_token_id"]
    b = Batch(len(lens), L, 0, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64), np.zeros(0, np.uint32),
              np.zeros(len(lens), np.uint64), np.zeros(len(lens), np.uint32))
    o = copy.copy(o0)
    o.opts = O.mask_options(settings)
    m = HipBackend(st, json.dumps(MMBERT_BASE), json.dumps(AGENT_ML), settings=settings)
    say(f"mmbert padding {settings[:30]!r}: n={b.n} len={b.len}")
    ref = o.encoder_hidden(b)
    rel = hidden_rel(m.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b, padding=True)
    say(f"mmbert padding {settings[:30]!r}: hidden rel at every position {rel:.2e}")
    assert rel <= HIDDEN_REL_GATE, rel
    m.close()
