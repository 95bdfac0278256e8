"""End-to-end parity of the HIP forward against the oracle, through the C ABI (HipBackend).

Gates: identical argmax choice per choice question, answer probabilities and act_probability
within 5e-3 absolute (after the f64 temperature softmax and the CPU action head of decode.rs),
and final hidden states within 2e-2 relative (per real token, ||gpu - oracle|| / ||oracle||).
The oracle is float32 with the same bf16 weights; the GPU computes in bf16 (or f16) with f32
accumulation and an f32 residual stream.

Workloads: a reduced 4-layer encoder on a ragged 3-row batch (the golden fixture's), then the
ModernBERT-large shape at a 128-token state with 1 question, a 512-token state with 1 question,
and a 512-token state with 10 questions, every row of it. Every settings variant is held to the
oracle itself, not only to another variant: sys1rust's production settings (DEFAULT_TUNING), the
backend's defaults, each fusion and work reduction switched off, and f16.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, S1Error, synth_checkpoint
from sys1rust_amd.decode import ActHead
from sys1rust_amd.workloads import AGENT, MODERNBERT_LARGE, Batch, workload

from gates import (HIDDEN_REL_GATE, FUSED, check_answers, decisive_checkpoint, gate_model, hidden_rel,
                   random_batch, say)

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


@pytest.fixture(scope="module")
def small_ref(small_model):
    cfg, agent, st, b, z = small_model
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    lg, pl = o.forward(b, ref)
    return o, ref, lg, pl, ActHead.from_weights(o.w)


def test_small_encoder_matches_oracle_and_golden(small_model, small_ref):
    cfg, agent, st, b, z = small_model
    o, ref, lg_ref, pl_ref, act = small_ref
    say("small: create")
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    assert m.name() == "hip(gfx950,bf16)"
    # The backend's own fusions are on by default; the reference's settings default off.
    assert m.active_kernels() == ["fusegeglu", "fuseln"]
    gate_model(m, b, ref, lg_ref, pl_ref, act, "small default")
    hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
    # every position, padding included, as the oracle computes it under the same (default) masks
    assert hidden_rel(hid, ref, b, padding=True) <= HIDDEN_REL_GATE
    # against the independent golden values too
    sel = z["hidden_sel"]
    g = hid[sel[:, 0], sel[:, 1]]
    gr = float((np.linalg.norm(g - z["hidden"], axis=-1) / np.linalg.norm(z["hidden"], axis=-1)).max())
    assert gr <= HIDDEN_REL_GATE, gr


# The reference's local-attention mask paths (lib.rs:1241-1310) that tell the padding positions
# apart, on the small model (window 16, dense up to 64 positions by default).
PADDING_MODES = ["", "dense_upto=0", "band=1,fuserope", "mask=bool", "mask=bool,dense_upto=0", DEFAULT_TUNING,
                 "windowed=0,dtype=f16"]


@pytest.mark.parametrize("settings", PADDING_MODES)
def test_encoder_hidden_padding_positions(small_model, settings):
    """encoder_hidden at every position, padding included, under each mask path the reference
    takes (dense, chunked, banded, boolean dense and chunked): the padding queries' key sets
    differ per path, and the oracle runs the same path. Rows with padding within the window of
    their last real token and beyond it, a far padding query in the first chunk (5 real tokens),
    a 1-token row and a full row."""
    cfg, agent, st, b0, z = small_model
    o = O.Oracle(st, cfg, agent, settings=settings)
    lens, L = [5, 40, 1], 40
    rng = np.random.default_rng(11)
    ids = rng.integers(5, 1000, size=(len(lens), L)).astype(np.uint32)
    am = np.zeros((len(lens), L), np.uint32)
    for r, l in enumerate(lens):
        am[r, :l] = 1
        ids[r, l:] = 1002
    b1 = Batch(len(lens), L, 0, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64), np.zeros(0, np.uint32),
               np.zeros(len(lens), np.uint64), np.zeros(len(lens), np.uint32))
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
    for tag, b in (("golden batch", b0), ("short rows", b1)):
        say(f"padding {settings!r}: {tag} n={b.n} len={b.len}")
        ref = o.encoder_hidden(b)
        hid = m.encoder_hidden(b).reshape(b.n, b.len, -1)
        rel = hidden_rel(hid, ref, b, padding=True)
        say(f"padding {settings!r}: {tag}: hidden rel at every position {rel:.2e}")
        assert rel <= HIDDEN_REL_GATE, (settings, tag, rel)
        # the same call again (graph replay of the padded layout)
        assert np.array_equal(hid, m.encoder_hidden(b).reshape(b.n, b.len, -1))
    m.close()


@pytest.mark.parametrize("head_layers", [0, 1])
def test_decision_head_depths(small_model, head_layers):
    """Agents with no decision-head layer (the scorer reads the encoder's stream, which headprune
    then leaves whole) and with one (the only layer is the pruned one), against the oracle."""
    cfg, agent, _, b, z = small_model
    ag = dict(agent, head_layers=head_layers)
    st = synth_checkpoint(json.dumps(cfg), json.dumps(ag), int(z["seed"]), int(z["scorer_width"]), 2, True)
    o = O.Oracle(st, cfg, ag)
    ref = o.encoder_hidden(b)
    lg_ref, pl_ref = o.forward(b, ref)
    act = ActHead.from_weights(o.w)
    outs = []
    for settings in (DEFAULT_TUNING, DEFAULT_TUNING + ",headprune=0", DEFAULT_TUNING + ",fuseln=0"):
        m = HipBackend(st, json.dumps(cfg), json.dumps(ag), settings=settings)
        outs.append(gate_model(m, b, ref, lg_ref, pl_ref, act, f"head_layers={head_layers} {settings}")[0])
        m.close()
    assert np.array_equal(outs[0].logits, outs[2].logits) and np.array_equal(outs[0].pooled, outs[2].pooled)


def test_encoder_hidden_positions_past_max_pos(small_model):
    """The padded layout gives every position a RoPE angle, so encoder_hidden refuses a len past
    max_position_embeddings (a Batch error naming it), while forward, which runs the real tokens
    only, serves the same batch; a token id past the vocabulary is refused by both."""
    cfg0, agent, _, _, _ = small_model
    cfg = dict(cfg0, max_position_embeddings=64, num_hidden_layers=2)
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), 5, 256, 2, True)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    n, L = 2, 80
    ids = np.full((n, L), 1002, np.uint32)
    ids[:, :10] = np.arange(5, 15, dtype=np.uint32)
    am = np.zeros((n, L), np.uint32)
    am[:, :10] = 1
    b = Batch(n, L, 1, ids.reshape(-1), am.reshape(-1), np.array([10, 10], np.uint64), np.array([3, 4], np.uint32),
              np.array([1, 1], np.uint64), np.array([0, 0], np.uint32))
    out = m.forward(b)
    assert np.all(np.isfinite(out.logits)) and np.all(np.isfinite(out.pooled))
    with pytest.raises(S1Error, match="max_position_embeddings"):
        m.encoder_hidden(b)
    bad = Batch(n, 12, 1, np.full(n * 12, 5000, np.uint32), np.ones(n * 12, np.uint32), np.array([12, 12], np.uint64),
                np.array([3, 4], np.uint32), np.array([1, 1], np.uint64), np.array([0, 0], np.uint32))
    for call in (m.forward, m.encoder_hidden):
        with pytest.raises(S1Error, match="vocabulary"):
            call(bad)
    m.close()


def test_very_short_rows(small_model):
    """Rows of 1, 3 and 9 tokens in one packed batch (a 1-token row has no room for a marker):
    every kernel on tiles far shorter than their blocks, against the oracle."""
    cfg, agent, st, _, _ = small_model
    lens = [1, 3, 9]
    n, L, K = len(lens), max(lens), 2
    rng = np.random.default_rng(7)
    ids = rng.integers(5, 1000, size=(n, L)).astype(np.uint32)
    am = np.zeros((n, L), np.uint32)
    for r, l in enumerate(lens):
        am[r, :l] = 1
        ids[r, l:] = 1002
    mp = np.array([[0, 0], [2, 0], [4, 8]], np.uint32)
    mc = np.array([0, 1, 2], np.uint64)
    b = Batch(n, L, K, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64), mp.reshape(-1), mc,
              np.array([0, 1, 2], np.uint32))
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    lg_ref, pl_ref = o.forward(b, ref)
    act = ActHead.from_weights(o.w)
    for settings in (DEFAULT_TUNING, DEFAULT_TUNING + ",headprune=0"):
        m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
        gate_model(m, b, ref, lg_ref, pl_ref, act, f"short rows {settings}")
        m.close()


@pytest.mark.parametrize("d,inter", [(640, 448), (1536, 1024), (2048, 1408)])
def test_hidden_widths(small_model, d, inter):
    """Hidden sizes the row kernels take besides 512, 768 and 1024: a partial 512-column chunk
    (640), three chunks (1536) and the widest (2048), on a 2-layer encoder with the small model's
    batch; in bf16 and f16, every fused kernel checked at load, against the oracle."""
    cfg0, agent, _, b, z = small_model
    cfg = dict(cfg0, hidden_size=d, num_attention_heads=d // 64, intermediate_size=inter, num_hidden_layers=2)
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), 5, 256, 2, True)
    o = O.Oracle(st, cfg, agent)
    ref = o.encoder_hidden(b)
    lg_ref, pl_ref = o.forward(b, ref)
    act = ActHead.from_weights(o.w)
    for settings in (DEFAULT_TUNING, DEFAULT_TUNING + ",dtype=f16", DEFAULT_TUNING + ",fuseln=0"):
        say(f"width {d}: {settings}")
        m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
        if "fuseln=0" not in settings:
            assert m.active_kernels() == FUSED, (settings, m.active_kernels())
        gate_model(m, b, ref, lg_ref, pl_ref, act, f"width {d} {settings}")
        m.close()


def test_batch_without_markers(small_model):
    """kmax = 0 (no answer markers in any row): no logits, only the pooled rows, which the pruned
    head's last kernel writes on its own. Pooled against the oracle, and bit for bit between the
    fused and unfused ends of the head."""
    cfg, agent, st, b0, z = small_model
    b = Batch(b0.n, b0.len, 0, b0.input_ids, b0.attention_mask, b0.seq_lens, np.zeros(0, np.uint32),
              np.zeros(b0.n, np.uint64), b0.qtype)
    o = O.Oracle(st, cfg, agent)
    _, pl_ref = o.forward(b)
    outs = []
    for settings in (DEFAULT_TUNING, DEFAULT_TUNING + ",fuseln=0", DEFAULT_TUNING + ",headprune=0"):
        say(f"no markers: {settings}")
        m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
        out = m.forward(b)
        m.close()
        assert out.logits.size == 0
        prel = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
        say(f"no markers {settings}: pooled rel {prel:.3e}")
        assert prel <= HIDDEN_REL_GATE, (settings, prel)
        outs.append(out.pooled)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("settings", [
    DEFAULT_TUNING,
    DEFAULT_TUNING + ",fuserope=0",
    DEFAULT_TUNING + ",fusegeglu=0",
    DEFAULT_TUNING + ",headprune=0",
    DEFAULT_TUNING + ",fuseln=0",
    "fusegeglu=0,fuseln=0,graphs=0",
    DEFAULT_TUNING + ",mask=bool,windowed=0,band=0,nax=0,geglu=plain,addmm=0,wcopy=t,unpad=0",
])
def test_settings_variants_match_oracle(small_model, small_ref, settings):
    """Each settings variant on its own against the oracle. The MLX-only keys of the last variant
    are accepted without effect on the forward: the same kernels run, so its bits equal
    DEFAULT_TUNING's (mask / windowed / band choose only the padding positions' keys in
    encoder_hidden)."""
    cfg, agent, st, b, z = small_model
    o, ref, lg_ref, pl_ref, act = small_ref
    say(f"variant {settings}")
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
    want = [k for k in FUSED if f"{k}=0" not in settings and (k != "fuserope" or "fuserope" in settings)]
    assert m.active_kernels() == want, (m.active_kernels(), want)
    out, _ = gate_model(m, b, ref, lg_ref, pl_ref, act, f"small {settings}")
    if "mask=bool" in settings or settings.endswith(",fuseln=0"):
        base = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
        o1 = base.forward(b)
        assert np.array_equal(o1.logits, out.logits) and np.array_equal(o1.pooled, out.pooled)
        # at the real tokens: mask=bool gives the padding positions other keys, as in the reference
        real = np.repeat(b.attention_mask.astype(bool), cfg["hidden_size"])
        assert np.array_equal(base.encoder_hidden(b)[real], m.encoder_hidden(b)[real])
        base.close()
    m.close()


@pytest.mark.parametrize("kernel", FUSED)
def test_load_check_turns_off_a_wrong_kernel(small_model, small_ref, kernel, capfd, monkeypatch):
    """The load-time check (lib.rs:319-362): a fused kernel whose output does not match its unfused
    twin is turned off for the load with one stderr line, is missing from active_kernels, and the
    forward runs the unfused kernels, which pass the gates and give the bits of a model loaded
    with that setting off. SYS1HIP_CHECK_FAULT (read at create, tests only) perturbs one value of
    the fused output inside the check (a wrong result, not a fault)."""
    cfg, agent, st, b, z = small_model
    o, ref, lg_ref, pl_ref, act = small_ref
    say(f"load check with a wrong {kernel}")
    capfd.readouterr()
    monkeypatch.setenv("SYS1HIP_CHECK_FAULT", kernel)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
    monkeypatch.delenv("SYS1HIP_CHECK_FAULT")
    err = capfd.readouterr().err
    assert f"libsys1hip: {kernel} is off for this load" in err, err
    assert err.count("libsys1hip:") == 1, err
    assert m.active_kernels() == [k for k in FUSED if k != kernel]
    out, _ = gate_model(m, b, ref, lg_ref, pl_ref, act, f"fallback {kernel}")
    off = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=f"{DEFAULT_TUNING},{kernel}=0")
    o2 = off.forward(b)
    assert np.array_equal(out.logits, o2.logits) and np.array_equal(out.pooled, o2.pooled)
    m.close()
    off.close()


def test_per_tensor_create_matches_image_create(small_model):
    """s1_model_create_from_tensors (the views of Weights::view()) loads the same model as the
    safetensors image: the same bits out."""
    cfg, agent, st, b, z = small_model
    a = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
    t = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING, per_tensor=True)
    oa, ot = a.forward(b), t.forward(b)
    assert np.array_equal(oa.logits, ot.logits) and np.array_equal(oa.pooled, ot.pooled)
    assert np.array_equal(a.encoder_hidden(b), t.encoder_hidden(b))
    a.close()
    t.close()


def test_layers_clear_and_warm_settings(small_model, capfd):
    """`layers` prints one line of per-layer times per forward; `clear` gives the arena back after
    every call and recomputes the same bits; `buckets` + `warm` run forwards at load and pad
    lengths to the buckets (padded_len, lib.rs:1826-1831)."""
    cfg, agent, st, b, z = small_model
    base = HipBackend(st, json.dumps(cfg), json.dumps(agent))
    want = base.forward(b)
    capfd.readouterr()
    lay = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="layers")
    out = lay.forward(b)
    lines = [l for l in capfd.readouterr().err.splitlines() if l.startswith("layers us:")]
    assert len(lines) == 1 and len(lines[0].split()) == 2 + cfg["num_hidden_layers"], lines
    assert np.array_equal(out.logits, want.logits)
    clr = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="clear")
    for _ in range(3):
        out = clr.forward(b)
        assert np.array_equal(out.logits, want.logits) and np.array_equal(out.pooled, want.pooled)
    warm = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="buckets=64:128,warm=1:2,pad=8")
    assert warm.padded_len(50, 1) == 64 and warm.padded_len(100, 3) == 128 and warm.padded_len(130, 1) == 136
    out = warm.forward(b)
    assert np.array_equal(out.logits, want.logits)
    for m in (base, lay, clr, warm):
        m.close()


@pytest.mark.parametrize("settings", ["", "graphs=0"])
def test_row_subsets_after_other_batches_match_oracle(small_model, settings):
    """One model, batches of different shapes in a row: each must match the oracle on its own.
    The arena is re-planned for each shape (split-K workspaces, graph capture per shape), and
    what a launch reads must be its own batch's data, not what an earlier layout left there
    (rows are independent, so any subset has known answers)."""
    cfg, agent, st, b, z = small_model
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=",".join(x for x in [DEFAULT_TUNING, settings] if x))
    o = O.Oracle(st, cfg, agent)
    for rows in ([0, 1, 2], [1, 2], [0, 1, 2], [2], [0, 2], [1, 2], [1]):
        bb = b.rows(rows)
        out = m.forward(bb)
        lg_ref, pl_ref = o.forward(bb)
        check_answers(out.logits, lg_ref, bb, f"rows {rows}")
        prel = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
        say(f"rows {rows}: pooled rel {prel:.3e}")
        assert prel <= HIDDEN_REL_GATE, (rows, prel)


@pytest.mark.parametrize("settings", ["", DEFAULT_TUNING, "dtype=f16"])
def test_random_batches_match_oracle(small_model, settings):
    """Twelve seeded random batches (ragged rows of 1-300 tokens, so one to three 128-query local
    tiles and one or two 256-query global tiles per row and head, 0-6 answer slots, markers
    anywhere in the row) through encoder_hidden and forward, each against the oracle with every
    gate, on the decisive-scorer checkpoint."""
    cfg, agent, st, _, _ = small_model
    st = decisive_checkpoint(st)
    m = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=settings)
    o = O.Oracle(st, cfg, agent)
    act = ActHead.from_weights(o.w)
    rng = np.random.default_rng(20261202)
    for case in range(12):
        b = random_batch(rng, cfg["vocab_size"], cfg["pad_token_id"])
        tag = f"random {case} ({settings[:12]!r}) n={b.n} len={b.len} kmax={b.kmax} T={b.total_tokens()}"
        say(tag)
        ref = o.encoder_hidden(b)
        lg, pl = o.forward(b, ref)
        gate_model(m, b, ref, lg, pl, act, tag)
    m.close()


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


def test_f16_matches_oracle_closer_than_bf16(small_model, small_ref):
    """dtype=f16 runs every kernel on f16 operands (three more mantissa bits than bf16, the
    checkpoints' own type). It passes the gates, and its distance to the f32 oracle is well under
    the bf16 path's: a kernel left on bf16 conversions, or on the bf16 MFMA, would not be."""
    cfg, agent, st, b, z = small_model
    o, ref, lg_ref, pl_ref, act = small_ref
    say("f16: create")
    m16 = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING + ",dtype=f16")
    mbf = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
    assert m16.name() == "hip(gfx950,f16)"
    # Every fused kernel passes its load check in f16 too (fuseln's is bit for bit).
    assert m16.active_kernels() == FUSED, m16.active_kernels()
    r16 = hidden_rel(m16.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    rbf = hidden_rel(mbf.encoder_hidden(b).reshape(b.n, b.len, -1), ref, b)
    say(f"f16: hidden rel {r16:.3e} (bf16 {rbf:.3e})")
    assert r16 <= HIDDEN_REL_GATE and r16 <= 0.2 * rbf, (r16, rbf)
    for name in ("fusegeglu=0,fuseln=0", DEFAULT_TUNING):
        mm = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings="dtype=f16," + name)
        out, _ = gate_model(mm, b, ref, lg_ref, pl_ref, act, f"f16 {name}")
        p16 = float(np.linalg.norm(out.pooled - pl_ref) / np.linalg.norm(pl_ref))
        pbf = float(np.linalg.norm(mbf.forward(b).pooled - pl_ref) / np.linalg.norm(pl_ref))
        say(f"f16 {name}: pooled rel {p16:.3e} (bf16 {pbf:.3e})")
        assert p16 <= 0.2 * pbf, (name, p16, pbf)
        mm.close()
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
    g = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=f"{DEFAULT_TUNING},dtype={dtype}")
    e = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=f"{DEFAULT_TUNING},dtype={dtype},graphs=0")
    b2 = b.rows([1, 2])
    want = {0: e.forward(b), 1: e.forward(b2)}
    want_h = e.encoder_hidden(b)
    for i, (k, bb) in enumerate([(0, b), (0, b), (1, b2), (0, b), (1, b2), (1, b2), (0, b), (0, b)]):
        out = g.forward(bb)
        assert np.array_equal(out.logits, want[k].logits), i
        assert np.array_equal(out.pooled, want[k].pooled), i
        if i % 3 == 0:
            assert np.array_equal(g.encoder_hidden(b), want_h), i


def test_graph_cache_eviction(small_model):
    """More request shapes than the graph cache holds (32): each shape is captured on its second
    request, the least recently used graphs are destroyed to make room, and a shape whose graph
    was evicted is captured again. Every output equals the eager path's."""
    cfg, agent, st, _, _ = small_model
    g = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING)
    e = HipBackend(st, json.dumps(cfg), json.dumps(agent), settings=DEFAULT_TUNING + ",graphs=0")
    rng = np.random.default_rng(11)

    def batch(l0):
        lens, L = [l0, 12], 48
        ids = rng.integers(5, 1000, size=(2, L)).astype(np.uint32)
        am = np.zeros((2, L), np.uint32)
        for r, l in enumerate(lens):
            am[r, :l] = 1
            ids[r, l:] = 1002
        return Batch(2, L, 2, ids.reshape(-1), am.reshape(-1), np.array(lens, np.uint64),
                     np.array([2, 5, 3, 7], np.uint32), np.array([2, 2], np.uint64), np.array([0, 2], np.uint32))

    shapes = {l0: batch(l0) for l0 in range(10, 46)}
    want = {l0: e.forward(b) for l0, b in shapes.items()}
    say(f"graph cache: {len(shapes)} shapes")
    for rnd in range(2):
        for l0, b in shapes.items():
            for _ in range(2):
                out = g.forward(b)
                assert np.array_equal(out.logits, want[l0].logits) and np.array_equal(out.pooled, want[l0].pooled), (rnd, l0)
    g.close()
    e.close()


@pytest.fixture(scope="module")
def large():
    say("large: synth checkpoint")
    st = synth_checkpoint(json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), seed=2024, scorer_width=1024)
    say("large: create")
    m = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings=DEFAULT_TUNING)
    assert m.active_kernels() == FUSED
    m.warmup()
    o = O.Oracle(st, MODERNBERT_LARGE, AGENT)
    return m, o, st, ActHead.from_weights(o.w)


@pytest.mark.parametrize("name", ["state128_1q", "state512_1q"])
def test_modernbert_large_single_question(large, name):
    m, o, st, act = large
    b = workload(name, seed=1)
    say(f"{name}: n={b.n} len={b.len} T={b.total_tokens()}")
    ref = o.encoder_hidden(b)
    lg_ref, pl_ref = o.forward(b, ref)
    gate_model(m, b, ref, lg_ref, pl_ref, act, name)


@pytest.fixture(scope="module")
def ten_questions(large):
    """The 10-question request and the oracle's answers for every one of its rows."""
    m, o, st, act = large
    b = workload("state512_10q", seed=1)
    say(f"state512_10q: n={b.n} len={b.len} T={b.total_tokens()}: oracle on all rows")
    ref = o.encoder_hidden(b)
    lg_ref, pl_ref = o.forward(b, ref)
    return b, ref, lg_ref, pl_ref


@pytest.mark.parametrize("settings", [DEFAULT_TUNING, "", DEFAULT_TUNING + ",fuserope=0",
                                      DEFAULT_TUNING + ",fusegeglu=0", DEFAULT_TUNING + ",headprune=0",
                                      DEFAULT_TUNING + ",dtype=f16"])
def test_modernbert_large_ten_questions_every_row(large, ten_questions, settings):
    """Every row of the 10-question request against the oracle, under the production settings and
    with each variant on its own."""
    m, o, st, act = large
    b, ref, lg_ref, pl_ref = ten_questions
    mm = m if settings == DEFAULT_TUNING else HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT),
                                                         settings=settings)
    gate_model(mm, b, ref, lg_ref, pl_ref, act, f"state512_10q [{settings or 'defaults'}]")
    if mm is not m:
        mm.close()


def test_ten_question_rows_alone_answer_the_same(large, ten_questions):
    """Rows are independent: rows of the batch run alone answer as inside it (other GEMM splits
    change bf16 rounding in the last bits, so compare at the answer gates)."""
    m, o, st, act = large
    b, ref, lg_ref, pl_ref = ten_questions
    rows = [0, 4, 7]
    sub = b.rows(rows)
    lg = m.forward(b).logits.reshape(b.n, b.kmax)[rows].reshape(-1)
    check_answers(m.forward(sub).logits, lg, sub, "state512_10q rows alone")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_fused_split_k_layernorm_bit_exact(large, dtype):
    """At one short request Wo and Wo2 split K and finish inside the next LayerNorm's kernel;
    with fuseln=0 the same sums run in the GEMM's reduce kernel and a separate LayerNorm. In f16
    as in bf16: the fused kernels must not round differently from the separate ones."""
    m, _, st, _ = large
    if dtype != "bf16":
        m = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT), settings=DEFAULT_TUNING + f",dtype={dtype}")
    assert "fuseln" in m.active_kernels(), m.active_kernels()
    sep = HipBackend(st, json.dumps(MODERNBERT_LARGE), json.dumps(AGENT),
                     settings=DEFAULT_TUNING + f",fuseln=0,dtype={dtype}")
    for name in ("state128_1q", "state512_1q"):
        b = workload(name, seed=3)
        say(f"fuseln {dtype} {name}: T={b.total_tokens()}")
        o1, o2 = m.forward(b), sep.forward(b)
        assert np.array_equal(o1.logits, o2.logits) and np.array_equal(o1.pooled, o2.pooled), name
        assert np.array_equal(m.encoder_hidden(b), sep.encoder_hidden(b)), name
    sep.close()
    if dtype != "bf16":
        m.close()


def test_warmup_and_repeat_determinism(large):
    m, _, _, _ = large
    b = workload("state128_1q", seed=5)
    a1 = m.forward(b)
    a2 = m.forward(b)
    assert np.array_equal(a1.logits, a2.logits) and np.array_equal(a1.pooled, a2.pooled)
    assert m.padded_len(170, 1) == 170
