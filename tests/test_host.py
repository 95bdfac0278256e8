"""Host-side logic of libsys1hip and the harness, without a GPU: the C ABI's exports, strict
settings, config and weight errors, the packing tables, the synthetic checkpoint, the row layout
of build_sequence / collate and the answer decode."""
from __future__ import annotations

import ctypes as C
import json
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from sys1rust_amd import _lib
from sys1rust_amd._lib import S1Error, check, i32p, u32p, u64p
from sys1rust_amd.backend import HipBackend, synth_checkpoint
from sys1rust_amd.decode import clamp_temperature, decode_answers, temp_bucket
from sys1rust_amd.workloads import (AGENT, CLS, MASK, SEP, Batch, Question, build_sequence, collate, encoder_json,
                                    small_config, workload)

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "sys1hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s1k?_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


@pytest.mark.parametrize("M,d,v_ld,needle", [
    (10, 1000, 24, "d must be a multiple of 64"),
    (10, 1024, 8, "v_ld must be a multiple of 8"),   # below M rounded up to 8
    (10, 1024, 20, "v_ld must be a multiple of 8"),  # 16-byte V^T stores need 8-element rows
])
def test_split_rope_entry_checks_shapes_before_any_launch(M, d, v_ld, needle):
    # The checks come before any device call, so null pointers never reach a kernel.
    with pytest.raises(S1Error) as e:
        check(_lib.lib().s1k_split_rope(None, M, d, None, 0.0, None, None, None, v_ld, None))
    assert e.value.kind == "Config" and needle in str(e.value)


SMALL = json.dumps(small_config(layers=2, vocab=512))


@pytest.fixture(scope="module")
def small_ckpt():
    return synth_checkpoint(SMALL, json.dumps(AGENT), seed=3, scorer_width=256)


@pytest.mark.parametrize("spec,needle", [
    ("bogus", "unknown setting `bogus`"),
    ("trace=2", "`2` is not 0 or 1"),
    ("pad=0", "pad must be at least 1"),
    ("pad=x", "is not a whole number"),
    ("buckets", "needs a value"),
    ("headprune,nax=all", "unknown setting `nax`"),
    ("dtype=fp8", "dtype must be bf16 or f16"),
    ("dtype", "dtype must be bf16 or f16"),
])
def test_settings_are_strict(small_ckpt, spec, needle):
    with pytest.raises(S1Error) as e:
        HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=spec)
    assert e.value.kind == "Config" and needle in str(e.value), str(e.value)


@pytest.mark.parametrize("spec", ["dtype=f16", "dtype=bf16", "dtype=f16,dtype=bf16"])
def test_dtype_setting_is_accepted(small_ckpt, spec):
    """A valid dtype passes the settings check: without a GPU the create fails later, at the
    device (a Backend error), never as a Config error."""
    try:
        m = HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=spec)
    except S1Error as e:
        assert e.kind != "Config", str(e)
        return
    want = "f16" if spec.endswith("f16") else "bf16"
    assert m.name() == f"hip(gfx950,{want})"
    m.close()


@pytest.mark.parametrize("mutate,needle", [
    (lambda c: c.update(model_type="bert"), "only 'modernbert'"),
    (lambda c: c.pop("num_hidden_layers"), "missing integer 'num_hidden_layers'"),
    (lambda c: c.update(global_attn_every_n_layers=0), "at least 1"),
    (lambda c: c.update(num_attention_heads=3), "not a multiple of num_attention_heads"),
    (lambda c: c.update(local_attention=1), "local_attention must be at least 2"),
    (lambda c: c.update(num_attention_heads=16), "head dim of 64"),
])
def test_config_errors(small_ckpt, mutate, needle):
    c = json.loads(SMALL)
    mutate(c)
    with pytest.raises(S1Error) as e:
        HipBackend(small_ckpt, json.dumps(c), json.dumps(AGENT))
    assert e.value.kind == "Config" and needle in str(e.value), str(e.value)


def test_truncated_or_missing_weights_are_weight_errors(small_ckpt, tmp_path):
    # weights.rs:22-43 and laya-mlx tests/loading.rs: every truncation is an error, never a crash
    for cut in [0, 4, 8, 20, len(small_ckpt) // 2, len(small_ckpt) - 1]:
        with pytest.raises(S1Error) as e:
            HipBackend(small_ckpt[:cut], SMALL, json.dumps(AGENT))
        assert e.value.kind == "Weights", (cut, str(e.value))
    with pytest.raises(S1Error) as e:
        HipBackend(str(tmp_path / "missing.safetensors"), SMALL, json.dumps(AGENT))
    assert e.value.kind == "Weights" and "cannot open" in str(e.value)
    # a tensor of the wrong shape names the tensor
    other = synth_checkpoint(json.dumps(small_config(layers=2, vocab=512, inter=256)), json.dumps(AGENT), 3, 256)
    with pytest.raises(S1Error) as e:
        HipBackend(other, SMALL, json.dumps(AGENT))
    assert e.value.kind == "Weights" and "mlp.Wi.weight" in str(e.value)


def test_synthetic_checkpoint_layout_and_determinism(small_ckpt):
    w = O.load_safetensors(small_ckpt)
    c = json.loads(SMALL)
    d, I = c["hidden_size"], c["intermediate_size"]
    assert w["encoder.embeddings.tok_embeddings.weight"].shape == (512, d)
    assert "encoder.layers.0.attn_norm.weight" not in w
    assert w["encoder.layers.1.attn_norm.weight"].shape == (d,)
    assert w["encoder.layers.1.mlp.Wi.weight"].shape == (2 * I, d)
    assert w["encoder.layers.1.mlp.Wo.weight"].shape == (d, I)
    assert w["head.layers.1.linear1.weight"].shape == (4 * d, d)
    assert w["scorer.1.weight"].shape == (256, d) and w["scorer.3.weight"].shape == (1, 256)
    assert w["act_head.0.weight"].shape == (256, d + 4)
    x = w["encoder.layers.1.attn.Wqkv.weight"]
    assert abs(float(x.std()) - 0.02) < 5e-4 and abs(float(x.mean())) < 5e-4
    g = w["encoder.layers.1.mlp_norm.weight"]
    assert abs(float(g.mean()) - 1.0) < 5e-3
    again = synth_checkpoint(SMALL, json.dumps(AGENT), seed=3, scorer_width=256)
    assert again == small_ckpt
    other = synth_checkpoint(SMALL, json.dumps(AGENT), seed=4, scorer_width=256)
    assert other != small_ckpt and len(other) == len(small_ckpt)


def pack_tables(b: Batch):
    L = _lib.lib()
    rs = np.zeros(b.n + 1, dtype=np.int32)
    pack = np.zeros(b.n * b.len, dtype=np.int32)
    row = np.zeros(b.n * b.len, dtype=np.int32)
    sc = np.zeros(b.n * (1 + b.kmax), dtype=np.int32)
    t = C.c_uint32(0)
    mp = b.marker_pos if b.marker_pos.size else np.zeros(1, np.uint32)
    check(L.s1_pack_tables(b.n, b.len, b.kmax, b.attention_mask.ctypes.data_as(u32p), b.seq_lens.ctypes.data_as(u64p),
                           mp.ctypes.data_as(u32p), b.marker_count.ctypes.data_as(u64p), rs.ctypes.data_as(i32p),
                           pack.ctypes.data_as(i32p), row.ctypes.data_as(i32p), sc.ctypes.data_as(i32p), C.byref(t)))
    T = t.value
    return rs, pack[:T], row[:T], sc


def test_packing_indexes_real_tokens_and_scorer_rows():
    """The reference's known-answer test, runtime/crates/laya-mlx/src/lib.rs:2008-2032."""
    b = Batch(3, 4, 2,
              np.array([1, 2, 0, 0, 3, 4, 5, 6, 7, 0, 0, 0], np.uint32),
              np.array([1, 1, 0, 0, 1, 1, 1, 1, 1, 0, 0, 0], np.uint32),
              np.array([2, 4, 1], np.uint64),
              np.array([1, 0, 1, 3, 0, 0], np.uint32),
              np.array([1, 2, 0], np.uint64),
              np.array([0, 1, 2], np.uint32))
    rs, pack, row, sc = pack_tables(b)
    assert rs[:3].tolist() == [0, 2, 6]
    assert pack.tolist() == [0, 1, 4, 5, 6, 7, 8]
    assert row.tolist() == [0, 0, 1, 1, 1, 1, 2]
    assert sc.tolist() == [0, 1, 0, 2, 3, 5, 6, 6, 6]


@pytest.mark.parametrize("bad,needle", [
    ("nonprefix", "right-padded"),
    ("seq_zero", "is not in 1..len"),
    ("marker_past", "points past the row"),
    ("count_over", "exceeds kmax"),
])
def test_malformed_batches_are_rejected(bad, needle):
    b = collate([([CLS, 5, 6, SEP], [1, 2], 0), ([CLS, 7, SEP], [1], 2)])
    if bad == "nonprefix":
        b.attention_mask[1] = 0
    elif bad == "seq_zero":
        b.seq_lens[1] = 0
    elif bad == "marker_past":
        b.marker_pos[2 + 0] = 3
    elif bad == "count_over":
        b.marker_count[0] = 3
    with pytest.raises(S1Error) as e:
        pack_tables(b)
    assert e.value.kind == "Batch" and needle in str(e.value)


def test_build_sequence_layout():
    """sequence.rs:43-96: [CLS] head [SEP] ([MASK] opt)* [SEP] state [SEP], options capped at 48."""
    q = Question("choice", [10, 11, 12], [[20, 21], [22] * 60])
    ids, markers = build_sequence(list(range(100, 110)), False, q, 512, 192)
    assert ids[:5] == [CLS, 10, 11, 12, SEP]
    assert markers == [5, 8]
    assert ids[5:8] == [MASK, 20, 21]
    assert ids[8] == MASK and ids[9:57] == [22] * 48
    assert ids[57] == SEP and ids[58:68] == list(range(100, 110)) and ids[68] == SEP
    # max_len truncates the state first and keeps the final [SEP]
    ids2, m2 = build_sequence(list(range(100, 600)), False, q, 80, 192)
    assert len(ids2) == 80 and ids2[-1] == SEP and ids2[58] == 100
    # a left-truncated (array) state keeps its tail
    ids3, _ = build_sequence(list(range(100, 600)), True, q, 80, 192)
    assert ids3[-2] == 599


def test_workloads_have_the_documented_shapes():
    b = workload("state512_10q", seed=0)
    assert b.n == 10 and b.kmax == 5
    assert b.qtype.tolist() == [0] * 4 + [1] * 3 + [2] * 3
    assert 540 <= b.seq_lens.min() and b.seq_lens.max() <= 600
    assert b.marker_count[4:7].tolist() == [4, 4, 4] and b.marker_count[7:].tolist() == [2, 2, 2]
    c0 = workload("state128_1q", seed=0)
    assert c0.n == 1 and 150 <= c0.len <= 185
    c2 = workload("state512_1q", seed=0)
    assert c2.n == 1 and 540 <= c2.len <= 590 and c2.marker_count[0] == 3
    ids = c2.input_ids.reshape(c2.n, c2.len)
    for k in range(3):
        assert ids[0, c2.marker_pos[k]] == MASK


def test_decode_known_answers():
    """decode.rs:407-418 (temperature clamp and buckets) and the f64 softmax decode."""
    assert clamp_temperature(0.1006) == 0.5
    assert clamp_temperature(7.0) == 5.0
    assert clamp_temperature("1.5") == 1.5
    assert clamp_temperature("abc") == 1.0
    assert clamp_temperature(None) == 1.0
    assert temp_bucket(0, 20) == "choice:11+"
    assert temp_bucket(2, 2) == "noul:2"
    assert temp_bucket(1, 5) == "score:3-5"
    assert temp_bucket(0, 6) == "choice:6-10"
    logits = np.array([1.0, 3.0, 3.0, -1e4, 0.0, 0.0, 0.0, 0.0, 2.0, 0.0, -1e4, -1e4], np.float32)
    ans = decode_answers(logits, 4, [3, 4, 2], [0, 1, 2], temperature=[1.0, 1.0, 2.0])
    assert ans[0]["choice"] == 1  # first maximum wins
    np.testing.assert_allclose(ans[0]["probabilities"].sum(), 1.0)
    assert abs(ans[1]["score"] - 1.5) < 1e-12
    e = np.exp(np.array([2.0, 0.0]) / 2.0)
    assert abs(ans[2]["noul"] - e[1] / e.sum()) < 1e-12
