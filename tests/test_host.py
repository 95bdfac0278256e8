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
from sys1rust_amd.backend import DEFAULT_TUNING, HipBackend, check_settings, synth_checkpoint, tensor_views
from sys1rust_amd.decode import (ActHead, act_features, clamp_temperature, confidence_from_probs, decode_answers,
                                 round_dp, temp_bucket)
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
    ("nax=1", "`1` is not one of 0, all"),
    ("dtype=fp8", "`fp8` is not one of bf16, f16, f32"),
    ("dtype", "needs a value"),
    # warm's load-time forwards are checked before any device memory is allocated
    ("buckets=2:64,warm=1", "warm needs buckets of at least 3 tokens"),
    ("buckets=9000,warm=1", "warm bucket 9000 is longer than max_position_embeddings (8192)"),
])
def test_settings_are_strict(small_ckpt, spec, needle):
    with pytest.raises(S1Error) as e:
        HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=spec)
    assert e.value.kind == "Config" and needle in str(e.value), str(e.value)


def test_production_settings_string_is_accepted(small_ckpt):
    """sys1rust passes DEFAULT_TUNING (runtime/crates/sys1rust/src/config.rs:29) as
    BackendOptions::tuning to every model it serves, and checks it with check_settings at startup
    (config.rs:657). Both must accept it verbatim; a create with it gets past the settings and
    the weights (here it stops at the device: there is no GPU in this container)."""
    check_settings(DEFAULT_TUNING)
    try:
        m = HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=DEFAULT_TUNING)
    except S1Error as e:
        assert e.kind == "Backend" and "device" in str(e), str(e)
        return
    m.close()


# Every key of laya-mlx's Knobs with a valid value (lib.rs:196-256), and this backend's own.
KNOBS_KEYS = ["geglu=shapeless", "geglu=compiled", "geglu=plain", "addmm", "addmm=0", "mask=bool", "mask=additive",
              "windowed=0", "clear", "trace", "layers", "ops=0", "wcopy=view", "wcopy=gpu", "wcopy=t", "f16gelu",
              "buckets=512:128:256", "pad=8", "warm=1:4", "cache=512", "wired=2048", "dense_upto=1024", "headprune",
              "unpad", "fuserope", "band=512", "band=0", "nax=all", "nax=0", "directload", "sharehead",
              "parallel_load", "parallel_load=0"]
OWN_KEYS = ["fusegeglu=0", "fuseln=0", "graphs=0", "dtype=f16", "dtype=bf16", "dtype=f32"]


@pytest.mark.parametrize("spec", KNOBS_KEYS + OWN_KEYS + [
    "", ",f16gelu,,", "f16gelu,f16gelu=0", "mask=bool,mask=additive", "band=512,band=0", "nax=all,nax=0",
    "directload=1,sharehead=1,directload=0,sharehead=0,parallel_load=0",
    "dense_upto=512,headprune,unpad,fuserope", "headprune=0,unpad=0,fuserope=0", "fuserope=1",
    "f16gelu,addmm=0,mask=bool,geglu=compiled,wcopy=t,buckets=512:128:256,pad=8,warm=1:4,cache=512,wired=2048",
    "f16gelu,cache=512,wired=2048"])
def test_check_settings_accepts_what_knobs_accepts(spec):
    """knobs_default_off_and_parse and settings_parse_every_kind_of_value (lib.rs:1927-1954,
    2034-2047): every key and value form Knobs takes, the last mention winning."""
    check_settings(spec)


@pytest.mark.parametrize("spec,needle", [
    # settings_reject_unknown_keys_and_bad_values (lib.rs:2050-2072), item for item
    ("f16gelu,cache=512x", "`cache=512x`"),
    ("f16gelu,chache=512", "unknown setting `chache`"),
    ("geglu=fast", "`fast` is not one of shapeless, compiled, plain"),
    ("mask=1", "`mask=1`"),
    ("wcopy=copy", "`wcopy=copy`"),
    ("f16gelu=yes", "`yes` is not 0 or 1"),
    ("buckets=128:abc", "`abc` is not a whole number"),
    ("buckets=", "`buckets=`"),
    ("pad=0", "pad must be at least 1"),
    ("pad=-1", "`-1` is not a whole number"),
    ("cache", "needs a value"),
    ("dense_upto=abc", "`abc` is not a whole number"),
    ("dense_upto", "needs a value"),
    ("unpad=yes", "`yes` is not 0 or 1"),
    ("headprune=on", "`on` is not 0 or 1"),
    ("fuserope=split", "`split` is not 0 or 1"),
    ("wired=2048,f16gelu,cache=512 ", "`cache=512 `"),
    # knobs_default_off_and_parse (lib.rs:1941-1954)
    ("band", "needs a value"),
    ("band=-1", "`-1` is not a whole number"),
    ("nax", "needs a value"),
    ("nax=split", "`split` is not one of 0, all"),
    ("directload=2", "`2` is not 0 or 1"),
    ("sharehead=yes", "`yes` is not 0 or 1"),
    ("parallel_load=2", "`2` is not 0 or 1"),
    # the load checks' fault injection is for tests only and is no setting
    ("check_fault=fuseln", "unknown setting `check_fault`"),
])
def test_check_settings_rejects_what_knobs_rejects(small_ckpt, spec, needle):
    """A bad item is a Config error naming it, from check_settings and from a create alike."""
    with pytest.raises(S1Error) as e:
        check_settings(spec)
    assert e.value.kind == "Config" and needle in str(e.value), str(e.value)
    with pytest.raises(S1Error) as e2:
        HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=spec)
    assert e2.value.kind == "Config" and str(e2.value) == str(e.value)


def test_per_tensor_create_checks_the_views(small_ckpt):
    """s1_model_create_from_tensors takes the (name, dtype, shape, bytes) views of
    Weights::view(): a view whose byte length does not match its shape, a duplicate name or an
    unknown dtype is a Weights error; well-formed views get past the weights (to the device)."""
    L = _lib.lib()
    arr, count, keep = tensor_views(small_ckpt)
    out = C.c_void_p()
    rc = L.s1_model_create_from_tensors(arr, count, SMALL.encode(), json.dumps(AGENT).encode(), b"", 0, C.byref(out))
    assert rc == _lib.S1_ERR_BACKEND, L.s1_last_error()
    for mutate, needle in [
        (lambda a: setattr(a[0], "nbytes", a[0].nbytes - 2), "byte length does not match"),
        (lambda a: setattr(a[1], "name", a[0].name), "given twice"),
        (lambda a: setattr(a[0], "dtype", 9), "unsupported dtype"),
    ]:
        arr, count, keep = tensor_views(small_ckpt)
        mutate(arr)
        rc = L.s1_model_create_from_tensors(arr, count, SMALL.encode(), json.dumps(AGENT).encode(), b"", 0,
                                            C.byref(out))
        assert rc == _lib.S1_ERR_WEIGHTS, L.s1_last_error()
        assert needle in L.s1_last_error().decode()
    # a missing tensor names it, as from the safetensors image
    arr, count, keep = tensor_views(small_ckpt)
    names = [arr[i].name.decode() for i in range(count)]
    drop = names.index("encoder.final_norm.weight")
    arr2 = (_lib.S1Tensor * (count - 1))(*[arr[i] for i in range(count) if i != drop])
    rc = L.s1_model_create_from_tensors(arr2, count - 1, SMALL.encode(), json.dumps(AGENT).encode(), b"", 0,
                                        C.byref(out))
    assert rc == _lib.S1_ERR_WEIGHTS and "encoder.final_norm.weight" in L.s1_last_error().decode()


@pytest.mark.parametrize("spec", ["dtype=f16", "dtype=bf16", "dtype=f16,dtype=bf16", "dtype=bf16,dtype=f32"])
def test_dtype_setting_is_accepted(small_ckpt, spec):
    """A valid dtype passes the settings check: without a GPU the create fails later, at the
    device (a Backend error), never as a Config error."""
    try:
        m = HipBackend(small_ckpt, SMALL, json.dumps(AGENT), settings=spec)
    except S1Error as e:
        assert e.kind != "Config", str(e)
        return
    want = spec.rsplit("=", 1)[1]
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


def test_answer_confidence_known_answers():
    """answer_confidence_per_type and confidence (decode.rs:519-524, 560-638): one row per type,
    temperatures 1, so the probabilities are plain softmaxes."""
    assert confidence_from_probs([1.0], 1) == 1.0
    assert abs(confidence_from_probs([0.5, 0.5], 2)) < 1e-12
    assert abs(confidence_from_probs([1.0, 0.0], 2) - 1.0) < 1e-9
    logits = np.array([2.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, -1.0, -1e4], np.float32)
    pick, rate, yes = decode_answers(logits, 3, [3, 3, 2], [0, 1, 2])
    assert pick["choice"] == 0 and round_dp(pick["answer_confidence"]) == 0.787
    assert round_dp(rate["answer_confidence"]) == 0.5761 == round_dp(rate["probabilities"][1])
    assert round_dp(yes["noul"]) == 0.2689 and round_dp(yes["confidence"]) == 0.7311
    assert yes["answer_confidence"] == yes["confidence"]


def test_act_features_invariants():
    """act_features (decode.rs:250-259) on rows whose answers are fixed by symmetry: equal
    logits give top1 = 1/k, margin 0 and a normalised entropy of exactly 1; masked slots (-1e4)
    change nothing; one dominant logit gives top1 -> 1, margin -> 1, entropy -> 0; the count
    feature is max(k, 2) / 255."""
    for k in (2, 3, 5):
        f = act_features(np.zeros(k, np.float32), k)
        np.testing.assert_allclose(f, [1.0 / k, 0.0, 1.0, k / 255.0], rtol=1e-6, atol=1e-6)
        padded = np.concatenate([np.zeros(k, np.float32), np.full(3, -1e4, np.float32)])
        np.testing.assert_allclose(act_features(padded, k), f, rtol=1e-6, atol=1e-7)
    f = act_features(np.array([30.0, 0.0, 0.0], np.float32), 3)
    assert f[0] > 1 - 1e-6 and f[1] > 1 - 1e-6 and f[2] < 1e-5
    assert act_features(np.array([1.0], np.float32), 1)[3] == np.float32(2.0 / 255.0)
    # top2 is the second largest, whatever the order
    f = act_features(np.log(np.array([0.2, 0.5, 0.3], np.float32)), 3)
    np.testing.assert_allclose(f[:2], [0.5, 0.2], rtol=1e-5)
    # an empty row (a batch with kmax 0): the softmax of nothing has no top entries
    # (unwrap_or(0.0)), its entropy sum is 0 negated, and k = max(0, 2)
    f = act_features(np.zeros(0, np.float32), 0)
    np.testing.assert_array_equal(f, np.array([0.0, 0.0, -0.0, 2.0 / 255.0], np.float32))
    assert np.signbit(f[2])


def test_act_features_rows_match_one_row_at_a_time():
    """act_features_rows (the decode's batched form) equals act_features row by row, with and
    without answer slots."""
    from sys1rust_amd.decode import act_features_rows

    rng = np.random.default_rng(2)
    for kmax, counts in [(4, [4, 2, 1, 0]), (0, [0, 0])]:
        lg = rng.normal(size=len(counts) * kmax).astype(np.float32)
        for r, c in enumerate(counts):
            lg[r * kmax + c: (r + 1) * kmax] = -1e4
        got = act_features_rows(lg, kmax, counts)
        want = np.stack([act_features(lg[r * kmax:(r + 1) * kmax], c) for r, c in enumerate(counts)])
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_decode_batch_matches_one_row_at_a_time():
    """decode_answers over a batch (the [n, kmax] array form from VECTOR_ROWS rows on) gives what
    each row decoded alone gives (the loop over rows): rows are independent. Random logits at
    three scales, exact ties, rows with 0 and 1 options, every question type, clamped and
    per-bucket temperatures."""
    from sys1rust_amd.decode import VECTOR_ROWS, decode_answers

    rng = np.random.default_rng(3)
    for trial in range(300):
        n = int(rng.integers(VECTOR_ROWS, 12))
        kmax = int(rng.integers(1, 14))
        mc = rng.integers(0, kmax + 1, size=n).astype(np.uint64)
        qt = rng.integers(0, 3, size=n).astype(np.uint32)
        lg = (rng.standard_normal(n * kmax) * [0.01, 1.0, 30.0][trial % 3]).astype(np.float32)
        if trial % 7 == 0:
            lg[:] = np.float32(0.5)  # every option tied: the first one wins
        for r in range(n):
            lg[r * kmax + int(mc[r]): (r + 1) * kmax] = np.float32(-1e4)
        temps = [(1.0, 1.0, 1.0), (0.7, 2.0, "3"), (True, None, float("nan"))][trial % 3]
        tbo = {"choice:3-5": 0.9, "noul:2": 4.0} if trial % 5 == 0 else None
        batch = decode_answers(lg, kmax, mc, qt, temps, tbo)
        for r in range(n):
            one = decode_answers(lg[r * kmax:(r + 1) * kmax], kmax, mc[r:r + 1], qt[r:r + 1], temps, tbo)[0]
            x = batch[r]
            assert x.keys() == one.keys() and x["type"] == one["type"]
            np.testing.assert_allclose(x["probabilities"], one["probabilities"], rtol=1e-12, atol=1e-15)
            for key in x:
                if key == "choice":
                    assert x[key] == one[key], (trial, r, x, one)
                elif key not in ("type", "probabilities"):
                    assert abs(x[key] - one[key]) <= 1e-12, (trial, r, key, x[key], one[key])


def test_act_head_matches_torch_mlp():
    """ActHead.probs (decode.rs:226-246) against torch's Linear -> GELU -> Linear -> softmax, an
    independent implementation, on the synthetic checkpoint's act_head; a head of zeros gives the
    uniform distribution (the reference's zero_act_head)."""
    import torch

    ck = synth_checkpoint(SMALL, json.dumps(AGENT), seed=5, scorer_width=256, n_act=3)
    w = O.load_safetensors(ck)
    head = ActHead.from_weights(w)
    d = json.loads(SMALL)["hidden_size"]
    assert head.pooled_width() == d and head.n_act == 3
    mlp = torch.nn.Sequential(torch.nn.Linear(d + 4, head.hidden), torch.nn.GELU(), torch.nn.Linear(head.hidden, 3))
    with torch.no_grad():
        mlp[0].weight.copy_(torch.from_numpy(w["act_head.0.weight"]))
        mlp[0].bias.copy_(torch.from_numpy(w["act_head.0.bias"]))
        mlp[2].weight.copy_(torch.from_numpy(w["act_head.2.weight"]))
        mlp[2].bias.copy_(torch.from_numpy(w["act_head.2.bias"]))
    rng = np.random.default_rng(0)
    for _ in range(4):
        pooled = rng.normal(size=d).astype(np.float32)
        feats = act_features(rng.normal(size=4).astype(np.float32), 3)
        with torch.no_grad():
            want = torch.softmax(mlp(torch.from_numpy(np.concatenate([pooled, feats]))), -1).numpy()
        np.testing.assert_allclose(head.probs(pooled, feats), want, rtol=1e-5, atol=1e-6)
    zero = ActHead(np.zeros((1, d + 4)), np.zeros(1), np.zeros((2, 1)), np.zeros(2))
    np.testing.assert_array_equal(zero.probs(np.ones(d), np.ones(4)), [0.5, 0.5])
    with pytest.raises(ValueError):
        ActHead(np.zeros((4, 4)), np.zeros(4), np.zeros((2, 4)), np.zeros(2))  # no room for the hidden state
    # read straight from the checkpoint image, as the bench's decode does: the same head
    direct = ActHead.from_safetensors(ck)
    for a, b in [(direct.w0, head.w0), (direct.b0, head.b0), (direct.w2, head.w2), (direct.b2, head.b2)]:
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("entry", ["s1k_gemm", "s1k_gemm_noalloc"])
def test_geglu_gemm_refuses_a_bias(entry):
    """The GeGLU epilogue has no bias term (the reference's Wi has none, lib.rs:1671): a bias
    given with epi=2 is refused with a Config error before anything reaches the GPU, instead of
    being dropped. (An unsplit shape, so no workspace is touched; the buffers are never read.)"""
    L = _lib.lib()
    buf = C.create_string_buffer(64)
    bias = (C.c_float * 256)()
    M, N, K = 2048, 256, 64
    rc = getattr(L, entry)(buf, K, buf, K, buf, N // 2, bias, M, N, K, 2, 0, None)
    assert rc == _lib.S1_ERR_CONFIG, L.s1_last_error()
    assert "GeGLU epilogue takes no bias" in L.s1_last_error().decode()


@pytest.mark.parametrize("entry", ["s1k_gemm", "s1k_gemm_noalloc"])
@pytest.mark.parametrize("which", ["A", "W"])
def test_gemm_refuses_operands_it_cannot_address(entry, which):
    """The GEMM's direct loads address A and W by 32-bit byte offsets from their starts. W must
    span less than 4 GiB ((N - 1) ldw + K 16-bit elements); an A that spans more runs as row
    pieces, which needs 8 rows to span less than 4 GiB. Either is refused with a Config error
    before anything reaches the GPU. One k-tile (K = 64) keeps the plan unsplit, so no workspace
    is touched; the buffers are never read."""
    L = _lib.lib()
    buf = C.create_string_buffer(64)
    K = 64
    if which == "W":
        ld = 1024
        big = (1 << 32) // (2 * ld) + 128  # (big - 1) ld + K elements pass 4 GiB; a multiple of 128
        assert ((big - 1) * ld + K) * 2 >= 1 << 32 and ((big - 129) * ld + K) * 2 < 1 << 32
        M, N, lda, ldw = 256, big, K, ld
        want = "W must span less than 4 GiB"
    else:
        lda = 1 << 29  # 8 rows span 7 GiB
        assert (7 * lda + K) * 2 >= 1 << 32
        M, N, ldw = 16, 256, K
        want = "rows under 512 MiB"
    rc = getattr(L, entry)(buf, lda, buf, ldw, buf, N, None, M, N, K, 0, 0, None)
    assert rc == _lib.S1_ERR_CONFIG, L.s1_last_error()
    assert want in L.s1_last_error().decode()


def test_answer_gate_takes_questions_with_one_option():
    """The parity gate's decisions (tests/gates.py) read the decode's own fields: a noul question
    with a single option has noul 0 (decode.rs) and no second probability to read."""
    from gates import check_answers
    from sys1rust_amd.workloads import Batch

    lg = np.array([0.3, -1e4, 1.5, -0.2, 0.7, -1e4], np.float32)
    b = Batch(3, 4, 2, np.zeros(12, np.uint32), np.ones(12, np.uint32), np.full(3, 4, np.uint64),
              np.array([1, 0, 1, 2, 3, 0], np.uint32), np.array([1, 2, 1], np.uint64), np.array([2, 2, 0], np.uint32))
    summary = check_answers(lg, lg, b, "one-option rows")
    assert summary["rows"] == 3 and summary["waived"] == 0 and summary["max_dp"] == 0.0
