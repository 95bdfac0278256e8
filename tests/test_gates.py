"""The parity gates themselves, on hand-made logits (CPU): a changed choice fails unless the
reference's top two are tied at the gate's resolution, and a probability moved past 5e-3 fails."""
from __future__ import annotations

import numpy as np
import pytest

from sys1rust_amd.workloads import Batch

from gates import LOGITS_ABS_GATE, SCORER_GAINS, check_answers, check_logits, decisive_checkpoint


def batch(k: int) -> Batch:
    z = np.zeros(1, np.uint32)
    return Batch(1, 1, k, z, np.ones(1, np.uint32), np.ones(1, np.uint64), np.zeros(k, np.uint32),
                 np.array([k], np.uint64), z)


def test_a_changed_choice_fails():
    ref = np.log(np.array([0.40, 0.35, 0.25], np.float32))
    gpu = np.log(np.array([0.35, 0.40, 0.25], np.float32))
    with pytest.raises(AssertionError):
        check_answers(gpu, ref, batch(3), "planted flip")


def test_a_near_tie_may_rank_either_way():
    ref = np.log(np.array([0.3340, 0.3330, 0.3330], np.float32))
    gpu = np.log(np.array([0.3332, 0.3338, 0.3330], np.float32))
    check_answers(gpu, ref, batch(3), "near tie")
    # the GPU's pick must still be one of the tied options
    gpu = np.log(np.array([0.3320, 0.3300, 0.3380], np.float32))
    check_answers(gpu, ref, batch(3), "near tie, third option within the band")
    ref = np.log(np.array([0.36, 0.355, 0.285], np.float32))
    gpu = np.log(np.array([0.3565, 0.357, 0.2865], np.float32))
    with pytest.raises(AssertionError):  # a third option outside the band cannot win
        check_answers(np.log(np.array([0.355, 0.355, 0.29], np.float32)) + np.array([0, 0, 0.3], np.float32),
                      ref, batch(3), "outside the band")
    check_answers(gpu, ref, batch(3), "tie within 1e-2")


def test_a_probability_past_the_gate_fails():
    ref = np.log(np.array([0.6, 0.4], np.float32))
    gpu = np.log(np.array([0.606, 0.394], np.float32))
    with pytest.raises(AssertionError):
        check_answers(gpu, ref, batch(2), "drift")


def batch_typed(k: int, qtype: int) -> Batch:
    z = np.zeros(1, np.uint32)
    return Batch(1, 1, k, z, np.ones(1, np.uint32), np.ones(1, np.uint64), np.zeros(k, np.uint32),
                 np.array([k], np.uint64), np.array([qtype], np.uint32))


def test_score_and_noul_decisions_are_gated_too():
    """compare.py:15-17: score by its argmax level, noul by p >= 0.5, not only choice."""
    ref = np.log(np.array([0.1, 0.42, 0.38, 0.1], np.float32))
    gpu = np.log(np.array([0.1, 0.38, 0.42, 0.1], np.float32))
    with pytest.raises(AssertionError):
        check_answers(gpu, ref, batch_typed(4, 1), "score flip", prob_gate=None)
    ref = np.log(np.array([0.47, 0.53], np.float32))
    gpu = np.log(np.array([0.53, 0.47], np.float32))
    with pytest.raises(AssertionError):
        check_answers(gpu, ref, batch_typed(2, 2), "noul flip", prob_gate=None)
    # a noul within the tie band may land on either side, and is counted as waived
    ref = np.log(np.array([0.498, 0.502], np.float32))
    gpu = np.log(np.array([0.501, 0.499], np.float32))
    s = check_answers(gpu, ref, batch_typed(2, 2), "noul tie")
    assert s["waived"] == 1 and s["near_ties"] == 1 and s["min_margin"] < 0.01


def test_decisive_rows_report_no_waiver():
    ref = np.log(np.array([0.6, 0.3, 0.1], np.float32))
    s = check_answers(ref + np.float32(1e-4), ref, batch(3), "decisive")
    assert s["waived"] == 0 and s["near_ties"] == 0 and abs(s["min_margin"] - 0.3) < 1e-5


def test_logits_gate():
    b = batch(3)
    ref = np.array([1.0, -2.0, 0.5], np.float32)
    assert check_logits(ref + np.float32(0.1), ref, b, "within") <= LOGITS_ABS_GATE
    with pytest.raises(AssertionError):
        check_logits(ref + np.array([0, 0.2, 0], np.float32), ref, b, "past the bound")
    # slots past marker_count (masked to -1e4 by the forward) are not compared
    b2 = Batch(1, 1, 3, b.input_ids, b.attention_mask, b.seq_lens, b.marker_pos, np.array([2], np.uint64), b.qtype)
    check_logits(np.array([1.0, -2.0, 7.0], np.float32), ref, b2, "masked slot")


def test_decisive_checkpoint_scales_exactly():
    """The decisive checkpoint multiplies scorer.1 and scorer.3 by 8 and 4 and leaves every other
    byte alone; the multiplications are exact (powers of two), so with scorer.3 (weight and bias)
    alone scaled the oracle's logits are exactly 4 times the plain checkpoint's."""
    import json

    from oracle import oracle as O
    from sys1rust_amd.backend import synth_checkpoint
    from sys1rust_amd.workloads import AGENT, collate, small_config

    cfg = small_config(layers=1, vocab=300, d=128, heads=2, inter=128)
    st = synth_checkpoint(json.dumps(cfg), json.dumps(AGENT), seed=5, scorer_width=128)
    dc = decisive_checkpoint(st)
    assert len(dc) == len(st)
    a, c = O.load_safetensors(st), O.load_safetensors(dc)
    for name in a:
        want = a[name] * SCORER_GAINS.get(name, 1.0)
        assert np.array_equal(c[name], want), name
    rng = np.random.default_rng(1)
    b = collate([([290] + rng.integers(0, 280, 20).tolist() + [291], [3, 7, 9], 0)], pad_id=292)
    l0, _ = O.Oracle(st, cfg, AGENT).forward(b)
    l3, _ = O.Oracle(decisive_checkpoint(st, {"scorer.3.weight": 4.0, "scorer.3.bias": 4.0}), cfg, AGENT).forward(b)
    assert np.array_equal(l3, 4 * l0)
