"""Parity at the throughput sizes: the 64-request varlen sweep and one 8192-token state.

The numpy oracle needs minutes per row at these lengths, so the reference here is its torch float32
restatement (oracle/torch_ref.py) on the GPU; tests/test_oracle.py pins that restatement to the
numpy oracle and the golden fixtures. The first test re-pins it on the GPU against the numpy
oracle at a size the latter finishes in seconds.

Gates as elsewhere: identical decisions per question (choice, score level, noul side),
probabilities and act_probability within 5e-3, logits within 0.15, hidden states within 2e-2
relative, on every row of the sweep. Properties at full size: rows
are independent, so a subset of the packed batch run alone must give the same answers, and every
output is finite. The model runs sys1rust's production settings (DEFAULT_TUNING).
"""
from __future__ import annotations

import copy
import json

import numpy as np
import pytest

from oracle import oracle as O
from oracle.torch_ref import TorchOracle
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, synth_checkpoint
from sys1rust_amd.decode import ActHead
from sys1rust_amd.workloads import AGENT, MODERNBERT_LARGE, Batch, workload

from gates import FUSED, HIDDEN_REL_GATE, check_act, check_answers, check_logits, hidden_rel, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def big_ckpt():
    say("big: synth checkpoint")
    return synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)


@pytest.fixture(scope="module")
def big(big_ckpt):
    st = big_ckpt
    say("big: create")
    m = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings=DEFAULT_TUNING)
    o = O.Oracle(st, MODERNBERT_LARGE, AGENT)
    return m, o, TorchOracle(o, "cuda")


def test_torch_checker_matches_numpy_oracle_on_gpu(big):
    _, o, t = big
    b = workload("state128_1q", seed=3)
    say(f"checker pin: T={b.total_tokens()}")
    ref = o.encoder_hidden(b)
    enc = t.encoder_hidden(b)
    rel = hidden_rel(enc, ref, b)
    say(f"checker pin: torch-on-GPU vs numpy hidden rel {rel:.2e}")
    assert rel < 1e-4
    lt, _ = t.forward(b, ref)
    lo, _ = o.forward(b, ref)
    assert float(np.abs(lt - lo).max()) < 1e-4


def test_state8192_single_question(big):
    m, _, t = big
    b = workload("state8192_1q", seed=1)
    say(f"state8192_1q: n={b.n} len={b.len} T={b.total_tokens()}")
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    out = m.forward(b)
    assert np.isfinite(hid).all() and np.isfinite(out.logits).all()
    say("state8192_1q: checker")
    ref = t.encoder_hidden(b)
    rel = hidden_rel(hid, ref, b)
    say(f"state8192_1q: hidden rel {rel:.3e}")
    assert rel <= HIDDEN_REL_GATE
    lg_ref, pl_ref = t.forward(b, ref)
    check_answers(out.logits, lg_ref, b, "state8192_1q")
    check_logits(out.logits, lg_ref, b, "state8192_1q")
    check_act(out.logits, out.pooled, lg_ref, pl_ref, b, ActHead.from_weights(t.o.w), "state8192_1q")
    pr = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
    say(f"state8192_1q: pooled rel {pr:.3e}")
    assert pr <= HIDDEN_REL_GATE


def test_state8192_f16(big):
    """The f16 path on the longest row: gates against the torch restatement, and closer than bf16."""
    m, o, t = big
    b = workload("state8192_1q", seed=1)
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    m16 = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings=DEFAULT_TUNING + ",dtype=f16")
    assert m16.active_kernels() == FUSED, m16.active_kernels()
    say(f"state8192_1q f16: T={b.total_tokens()}")
    ref = t.encoder_hidden(b)
    r16 = hidden_rel(m16.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    rbf = hidden_rel(m.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    say(f"state8192_1q f16: hidden rel {r16:.3e} (bf16 {rbf:.3e})")
    assert r16 <= HIDDEN_REL_GATE and r16 <= 0.2 * rbf, (r16, rbf)
    lg_ref, _ = t.forward(b, ref)
    check_answers(m16.forward(b).logits, lg_ref, b, "state8192_1q f16")
    m16.close()


def test_sweep64_packed_batch_every_row(big):
    """All 192 rows of the 64-request sweep, packed into one forward, against the torch restatement."""
    m, o, t = big
    b = workload("sweep64", seed=1)
    T = b.total_tokens()
    say(f"sweep64: n={b.n} len={b.len} T={T}")
    out = m.forward(b)
    assert np.isfinite(out.logits).all() and np.isfinite(out.pooled).all()
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    act = ActHead.from_weights(o.w)
    lens = b.seq_lens.astype(np.int64)
    lg_all = out.logits.reshape(b.n, b.kmax)
    pl_all = out.pooled.reshape(b.n, -1)
    worst = 0.0
    # The torch restatement in chunks of rows (its padded [rows, len] layout is what bounds its memory).
    order = np.argsort(lens)
    for c in range(0, b.n, 16):
        rows = sorted(int(r) for r in order[c:c + 16])
        sub = b.rows(rows)
        L = int(lens[rows].max())
        sub = Batch(sub.n, L, sub.kmax, np.ascontiguousarray(sub.input_ids.reshape(sub.n, b.len)[:, :L].reshape(-1)),
                    np.ascontiguousarray(sub.attention_mask.reshape(sub.n, b.len)[:, :L].reshape(-1)),
                    sub.seq_lens, sub.marker_pos, sub.marker_count, sub.qtype)
        ref = t.encoder_hidden(sub)
        rel = hidden_rel(hid[rows][:, :L], ref, sub)
        worst = max(worst, rel)
        assert rel <= HIDDEN_REL_GATE, (rows, rel)
        lg_ref, pl_ref = t.forward(sub, ref)
        lg, pl = lg_all[rows].reshape(-1), pl_all[rows].reshape(-1)
        check_answers(lg, lg_ref, sub, f"sweep64 rows {rows[0]}..")
        check_logits(lg, lg_ref, sub, f"sweep64 rows {rows[0]}..")
        check_act(lg, pl, lg_ref, pl_ref, sub, act, f"sweep64 rows {rows[0]}..")
    say(f"sweep64: every row checked; worst hidden rel {worst:.3e}")
    # Rows are independent: the shortest, the longest and one row of each type run alone answer
    # the same (other tile shapes and splits change bf16 rounding in the last bits, so compare
    # at the answer gates).
    rows = {int(np.argmin(lens)), int(np.argmax(lens))}
    for qt in np.unique(b.qtype):
        of = np.flatnonzero(b.qtype == qt)
        rows.add(int(of[np.argmax(lens[of])]))
    rows = sorted(rows)
    sub = b.rows(rows)
    alone = m.forward(sub)
    check_answers(alone.logits, lg_all[rows].reshape(-1), sub, "sweep64 rows alone")


@pytest.mark.parametrize("settings", ["", "mask=bool", DEFAULT_TUNING])
def test_encoder_hidden_padding_positions_large(big, big_ckpt, settings):
    """The ModernBERT-large encoder at a 600-position padded length, where the reference's local
    layers run chunked (default settings, boolean masks) or banded (DEFAULT_TUNING: band=512):
    every position of rows with 600, 300 and 20 real tokens (padding far past the window, and
    padding queries in the first chunk), against the torch checker under the same masks."""
    m0, o0, t0 = big
    lens, L = [600, 300, 20], 600
    rng = np.random.default_rng(17)
    ids = rng.integers(5, 50000, size=(len(lens), L)).astype(np.uint32)
    am = np.zeros((len(lens), L), np.uint32)
    for r, l in enumerate(lens):
        am[r, :l] = 1
        ids[r, l:] = 50283
    b = Batch(len(lens), L, 0, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64), np.zeros(0, np.uint32),
              np.zeros(len(lens), np.uint64), np.zeros(len(lens), np.uint32))
    o = copy.copy(o0)
    o.opts = O.mask_options(settings)
    t = copy.copy(t0)
    t.o = o
    m = m0 if settings == DEFAULT_TUNING else HipBackend(big_ckpt, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT),
                                                         settings=settings)
    say(f"padding large {settings[:40]!r}: n={b.n} len={b.len}")
    ref = t.encoder_hidden(b)
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    rel = hidden_rel(hid, ref, b, padding=True)
    say(f"padding large {settings[:40]!r}: hidden rel at every position {rel:.2e}")
    assert rel <= HIDDEN_REL_GATE, rel
    if m is not m0:
        m.close()
