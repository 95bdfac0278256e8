"""End-to-end parity of the HIP forward against the oracle, through the C ABI (HipBackend).

Gates: identical argmax choice per choice question, answer probabilities
within 5e-3 absolute (after the f64 temperature softmax of decode.rs), and final hidden states
within 2e-2 relative (per real token, ||gpu - oracle|| / ||oracle||). The oracle is float32 with
the same bf16 weights; the GPU computes in bf16 with f32 accumulation and an f32 residual stream.

Workloads: a reduced 4-layer encoder on a ragged 3-row batch, then the ModernBERT-large shape at
a 128-token state with 1 question, a 512-token state with 1 question, and a 512-token state with
10 questions (the oracle runs a subset of its rows; rows are independent). Settings variants
(unfused RoPE / GeGLU, no head pruning) must agree with the default path.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from sys1rust_amd.backend import HipBackend, synth_checkpoint
from sys1rust_amd.workloads import AGENT, MODERNBERT_LARGE, Batch, workload

from gates import HIDDEN_REL_GATE, PROB_ABS_GATE, check_answers, hidden_rel, say

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def small_model():
    z = np.load(GOLDEN / "golden_small.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    return cfg, agent, st, b, z


def test_small_encoder_matches_oracle_and_golden(small_model):
    cfg, agent, st, b, z = small_model
    say("small: create")
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    assert m.name() == "hip(gfx950,bf16)"
    say("small: encoder_hidden")
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    rel = hidden_rel(hid, ref, b)
    say(f"small: hidden rel {rel:.3e}")
    assert rel <= HIDDEN_REL_GATE
    # padding positions are not computed
    am = b.attention_mask.reshape(b.n, b.len).astype(bool)
    assert np.all(hid[~am] == 0)
    # against the independent golden values too
    sel = z["hidden_sel"]
    g = hid[sel[:, 0], sel[:, 1]]
    gr = float((np.linalg.norm(g - z["hidden"], axis=-1) / np.linalg.norm(z["hidden"], axis=-1)).max())
    assert gr <= HIDDEN_REL_GATE, gr
    say("small: forward")
    out = m.forward(b)
    lg_ref, pl_ref = o.forward(b, ref)
    assert np.all(out.logits[np.arange(b.n * b.kmax) % b.kmax >= np.repeat(b.marker_count, b.kmax)] == -1e4)
    check_answers(out.logits, lg_ref, b, "small")
    prel = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
    say(f"small: pooled rel {prel:.3e}")
    assert prel <= HIDDEN_REL_GATE


@pytest.mark.parametrize("settings", ["fuserope=0", "fusegeglu=0", "headprune=0", "fuseln=0",
                                      "fuserope=0,fusegeglu=0,headprune=0,fuseln=0"])
def test_settings_variants_agree(small_model, settings):
    cfg, agent, st, b, z = small_model
    say(f"variant {settings}")
    base = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    var = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
    o1, o2 = base.forward(b), var.forward(b)
    assert np.abs(o1.logits - o2.logits).max() <= 5e-3
    assert np.linalg.norm(o1.pooled - o2.pooled) / np.linalg.norm(o1.pooled) <= 1e-2
    h1, h2 = base.encoder_hidden(b), var.encoder_hidden(b)
    assert np.linalg.norm(h1 - h2) / np.linalg.norm(h1) <= 1e-2
    if "fuserope=0" in settings:
        assert "fuserope" not in var.active_kernels()
    if "headprune=0" in settings:
        assert "headprune" not in var.active_kernels()
    if settings == "fuseln=0":  # same arithmetic in one kernel instead of two
        assert "fuseln" not in var.active_kernels() and "fuseln" in base.active_kernels()
        assert np.array_equal(o1.logits, o2.logits) and np.array_equal(o1.pooled, o2.pooled)
        assert np.array_equal(h1, h2)


@pytest.mark.parametrize("settings", ["", "graphs=0"])
def test_row_subsets_after_other_batches_match_oracle(small_model, settings):
    """One model, batches of different shapes in a row: each must match the oracle on its own.
    The arena is re-planned for each shape (split-K workspaces, graph capture per shape), and
    what a launch reads must be its own batch's data, not what an earlier layout left there
    (rows are independent, so any subset has known answers)."""
    cfg, agent, st, b, z = small_model
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
    o = O.Oracle(st, cfg, agent)
    for rows in ([0, 1, 2], [1, 2], [0, 1, 2], [2], [0, 2], [1, 2], [1]):
        bb = b.rows(rows)
        out = m.forward(bb)
        lg_ref, pl_ref = o.forward(bb)
        check_answers(out.logits, lg_ref, bb, f"rows {rows}")
        prel = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
        say(f"rows {rows}: pooled rel {prel:.3e}")
        assert prel <= HIDDEN_REL_GATE, (rows, prel)


def _reencode(st: bytes, dtype: str) -> bytes:
    """The same tensors re-encoded as F16 or F32 safetensors."""
    tensors = O.load_safetensors(st)
    header, chunks, off = {}, [], 0
    for name, a in tensors.items():
        raw = np.ascontiguousarray(a.astype(np.float16 if dtype == "F16" else np.float32)).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        chunks.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(chunks)


@pytest.mark.parametrize("dtype", ["F32", "F16"])
def test_f32_and_f16_checkpoints_load_like_bf16(small_model, dtype):
    """The real checkpoints ship F16 tensors, converted on load (weights.rs:82-103); the loader
    rounds F16 and F32 tensors to bf16. The bf16 weights re-encoded as F32 give the same bits;
    as F16 they are exact except below F16's normal range (|w| < 6.1e-5), so compare at the gates."""
    cfg, agent, st, b, z = small_model
    say(f"checkpoint as {dtype}")
    m0 = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    m1 = HipBackend(_reencode(st, dtype), json.dumps(cfg), json.dumps(agent))
    o0, o1 = m0.forward(b), m1.forward(b)
    if dtype == "F32":
        assert np.array_equal(o0.logits, o1.logits) and np.array_equal(o0.pooled, o1.pooled)
    else:
        check_answers(o1.logits, o0.logits, b, "f16 checkpoint")
        assert np.linalg.norm(o1.pooled - o0.pooled) / np.linalg.norm(o0.pooled) <= 1e-2
    m0.close()
    m1.close()


def test_f16_matches_oracle_closer_than_bf16(small_model):
    """dtype=f16 runs every kernel on f16 operands (three more mantissa bits than bf16, the
    checkpoints' own type). It passes the gates, and its distance to the f32 oracle is well under
    the bf16 path's: a kernel left on bf16 conversions, or on the bf16 MFMA, would not be."""
    cfg, agent, st, b, z = small_model
    say("f16: create")
    m16 = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f16")
    mbf = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    assert m16.name() == "hip(gfx950,f16)"
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    r16 = hidden_rel(m16.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    rbf = hidden_rel(mbf.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    say(f"f16: hidden rel {r16:.3e} (bf16 {rbf:.3e})")
    assert r16 <= HIDDEN_REL_GATE and r16 <= 0.2 * rbf, (r16, rbf)
    lg_ref, pl_ref = o.forward(b, ref)
    for name in ("fuserope=0,fusegeglu=0,fuseln=0,headprune=0", ""):
        mm = m16 if not name else HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f16," + name)
        out = mm.forward(b)
        check_answers(out.logits, lg_ref, b, f"f16 {name or 'default'}")
        p16 = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
        pbf = float(np.linalg.norm(mbf.forward(b).pooled - pl_ref) / np.linalg.norm(pl_ref))
        say(f"f16 {name or 'default'}: pooled rel {p16:.3e} (bf16 {pbf:.3e})")
        assert p16 <= 0.2 * pbf, (name, p16, pbf)
    m16.close()
    mbf.close()


def test_f16_model_keeps_f16_checkpoint_bits(small_model):
    """With dtype=f16 an F16 checkpoint's tensors are used as stored; the bf16 checkpoint's are
    rounded to f16 on load (round to nearest even, as numpy's astype(float16) that wrote the F16
    file), so both give the same weights and the same bits out."""
    cfg, agent, st, b, z = small_model
    say("f16 checkpoint with dtype=f16")
    a = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f16")
    c = HipBackend(_reencode(st, "F16"), json.dumps(cfg), json.dumps(agent), settings="dtype=f16")
    oa, oc = a.forward(b), c.forward(b)
    assert np.array_equal(oa.logits, oc.logits) and np.array_equal(oa.pooled, oc.pooled)
    assert np.array_equal(a.encoder_hidden(b), c.encoder_hidden(b))
    a.close()
    c.close()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_graph_replays_match_eager_runs(small_model, dtype):
    """Repeated shapes replay a captured HIP graph: every replay, interleaved with other shapes
    and with eager work, gives the eager path's bits."""
    cfg, agent, st, b, z = small_model
    say(f"graphs: replay vs eager ({dtype})")
    g = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=f"dtype={dtype}")
    e = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=f"dtype={dtype},graphs=0")
    b2 = b.rows([1, 2])
    want = {0: e.forward(b), 1: e.forward(b2)}
    want_h = e.encoder_hidden(b)
    for i, (k, bb) in enumerate([(0, b), (0, b), (1, b2), (0, b), (1, b2), (1, b2), (0, b), (0, b)]):
        out = g.forward(bb)
        assert np.array_equal(out.logits, want[k].logits), i
        assert np.array_equal(out.pooled, want[k].pooled), i
        if i % 3 == 0:
            assert np.array_equal(g.encoder_hidden(b), want_h), i


@pytest.fixture(scope="module")
def large():
    say("large: synth checkpoint")
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    say("large: create")
    m = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT))
    m.warmup()
    o = O.Oracle(st, MODERNBERT_LARGE, AGENT)
    return m, o


@pytest.mark.parametrize("name", ["state128_1q", "state512_1q"])
def test_modernbert_large_single_question(large, name):
    m, o = large
    b = workload(name, seed=1)
    say(f"{name}: n={b.n} len={b.len} T={b.total_tokens()}")
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    ref = o.encoder_hidden(b)
    rel = hidden_rel(hid, ref, b)
    say(f"{name}: hidden rel {rel:.3e}")
    assert rel <= HIDDEN_REL_GATE
    out = m.forward(b)
    lg_ref, pl_ref = o.forward(b, ref)
    check_answers(out.logits, lg_ref, b, name)


def test_modernbert_large_ten_questions(large):
    m, o = large
    b = workload("state512_10q", seed=1)
    say(f"state512_10q: n={b.n} len={b.len} T={b.total_tokens()}")
    out = m.forward(b)
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    rows = [0, 4, 7]  # one question of each type
    sub = b.rows(rows)
    ref = o.encoder_hidden(sub)
    rel = hidden_rel(hid[rows], ref, sub)
    say(f"state512_10q rows {rows}: hidden rel {rel:.3e}")
    assert rel <= HIDDEN_REL_GATE
    lg_ref, _ = o.forward(sub, ref)
    lg = out.logits.reshape(b.n, b.kmax)[rows].reshape(-1)
    check_answers(lg, lg_ref, sub, "state512_10q")
    # Rows are independent: the same rows alone give the same answers. (A smaller batch takes
    # other GEMM splits, so bf16 rounding differs in the last bits; compare at the answer gates.)
    alone = m.forward(sub)
    check_answers(alone.logits, lg, sub, "state512_10q rows alone")


@pytest.mark.parametrize("name", ["state128_1q", "state512_1q", "state512_10q"])
def test_modernbert_large_f16(large, name):
    """The f16 path at the full shape: gates against the oracle, and closer than bf16."""
    m, o = large
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    m16 = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings="dtype=f16")
    b = workload(name, seed=1)
    rows = [0] if b.n == 1 else [0, 4, 7]
    sub = b.rows(rows)
    say(f"f16 {name}: T={b.total_tokens()}")
    ref = o.encoder_hidden(sub)
    r16 = hidden_rel(m16.encoder_hidden(b).reshape(b.n, b.len, -1)[rows], ref, sub)
    rbf = hidden_rel(m.encoder_hidden(b).reshape(b.n, b.len, -1)[rows], ref, sub)
    say(f"f16 {name}: hidden rel {r16:.3e} (bf16 {rbf:.3e})")
    assert r16 <= HIDDEN_REL_GATE and r16 <= 0.2 * rbf, (r16, rbf)
    lg_ref, _ = o.forward(sub, ref)
    lg = m16.forward(b).logits.reshape(b.n, b.kmax)[rows].reshape(-1)
    check_answers(lg, lg_ref, sub, f"f16 {name}")
    m16.close()


def test_fused_split_k_layernorm_bit_exact(large):
    """At one short request Wo and Wo2 split K and finish inside the next LayerNorm's kernel;
    with fuseln=0 the same sums run in the GEMM's reduce kernel and a separate LayerNorm."""
    m, _ = large
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    sep = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings="fuseln=0")
    for name in ("state128_1q", "state512_1q"):
        b = workload(name, seed=3)
        say(f"fuseln {name}: T={b.total_tokens()}")
        o1, o2 = m.forward(b), sep.forward(b)
        assert np.array_equal(o1.logits, o2.logits) and np.array_equal(o1.pooled, o2.pooled), name
        assert np.array_equal(m.encoder_hidden(b), sep.encoder_hidden(b)), name
    sep.close()


def test_blaslt_residual_gemms_agree_and_replay(large):
    """With the opt-in setting blaslt, from 2048 rows the unsplit residual GEMMs run in hipBLASLt:
    the answers agree with the hand-written kernels' (the default) at the gates, and graph
    replays of that path (first sight eager, then captured, then replayed) give the eager run's
    bits."""
    m, o = large
    assert "blaslt" not in m.active_kernels()
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    lt = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings="blaslt")
    eager = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings="blaslt,graphs=0")
    assert "blaslt" in lt.active_kernels()
    b = workload("state512_10q", seed=4)
    say(f"blaslt: T={b.total_tokens()}")
    want = eager.forward(b)
    for i in range(4):
        out = lt.forward(b)
        assert np.array_equal(out.logits, want.logits) and np.array_equal(out.pooled, want.pooled), i
    own = m.forward(b)
    check_answers(want.logits, own.logits, b, "blaslt vs own kernels")
    assert np.linalg.norm(want.pooled - own.pooled) / np.linalg.norm(own.pooled) <= 1e-2
    h1, h2 = lt.encoder_hidden(b), m.encoder_hidden(b)
    assert np.linalg.norm(h1 - h2) / np.linalg.norm(h2) <= 1e-2
    lt.close()
    eager.close()


def test_warmup_and_repeat_determinism(large):
    m, _ = large
    b = workload("state128_1q", seed=5)
    a1 = m.forward(b)
    a2 = m.forward(b)
    assert np.array_equal(a1.logits, a2.logits) and np.array_equal(a1.pooled, a2.pooled)
    assert m.padded_len(170, 1) == 170
