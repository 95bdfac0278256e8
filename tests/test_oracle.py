"""The oracle against the golden fixtures, closed forms and planted mistakes (CPU only).

The fixtures come from transformers' ModernBertModel and torch's TransformerEncoderLayer
(tests/golden/make_golden.py), an implementation independent of the oracle. A planted-mistake
test changes one thing in the oracle (window width, RoPE base, GeGLU order, head scale, a
dropped bias) and checks that the golden comparison then fails, so the fixtures do pin each of
those choices.
"""
from __future__ import annotations

import functools
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from sys1rust_amd.backend import synth_checkpoint
from sys1rust_amd.workloads import Batch

GOLDEN = Path(__file__).resolve().parent / "golden"

# f32 restatement vs f32 torch: differences are summation order and RoPE angle rounding.
HIDDEN_REL_TOL = 1e-4
LOGIT_ABS_TOL = 1e-5
POOLED_REL_TOL = 1e-4


@functools.lru_cache(maxsize=None)
def load_case(name: str):
    z = np.load(GOLDEN / f"{name}.npz")
    cfg = json.loads(str(z["encoder_config"]))
    agent = json.loads(str(z["agent_config"]))
    b = Batch(int(z["n"]), int(z["len"]), int(z["kmax"]), z["input_ids"], z["attention_mask"], z["seq_lens"],
              z["marker_pos"], z["marker_count"], z["qtype"])
    st = synth_checkpoint(json.dumps(cfg), json.dumps(agent), int(z["seed"]), int(z["scorer_width"]), 2, True)
    return z, cfg, agent, b, st


@pytest.fixture(scope="module")
def small():
    return load_case("golden_small")


def compare(z, o: O.Oracle, b: Batch):
    enc = o.encoder_hidden(b)
    lg, pl = o.forward(b, enc)
    sel = z["hidden_sel"]
    hid = enc[sel[:, 0], sel[:, 1]]
    ref = z["hidden"]
    rel = float((np.linalg.norm(hid - ref, axis=-1) / np.linalg.norm(ref, axis=-1)).max())
    dl = float(np.abs(lg - z["logits"]).max())
    dp = float(np.linalg.norm(pl - z["pooled"]) / np.linalg.norm(z["pooled"]))
    return rel, dl, dp


def test_oracle_matches_golden_small(small):
    z, cfg, agent, b, st = small
    rel, dl, dp = compare(z, O.Oracle(st, cfg, agent), b)
    assert rel < HIDDEN_REL_TOL, rel
    assert dl < LOGIT_ABS_TOL, dl
    assert dp < POOLED_REL_TOL, dp


def test_oracle_matches_golden_modernbert_large():
    z, cfg, agent, b, st = load_case("golden_large")
    rel, dl, dp = compare(z, O.Oracle(st, cfg, agent), b)
    assert rel < HIDDEN_REL_TOL, rel
    assert dl < LOGIT_ABS_TOL, dl
    assert dp < POOLED_REL_TOL, dp


def test_oracle_matches_golden_mmbert_base():
    """The multilingual checkpoint's encoder shape (mmBERT-base: d 768, 12 heads, I 1152, 22
    layers, vocabulary 256,000; laya-mlx/tests/parity.rs:68-80 is the reference's suite for it)."""
    z, cfg, agent, b, st = load_case("golden_mmbert")
    assert (cfg["hidden_size"], cfg["num_attention_heads"], cfg["intermediate_size"]) == (768, 12, 1152)
    rel, dl, dp = compare(z, O.Oracle(st, cfg, agent), b)
    assert rel < HIDDEN_REL_TOL, rel
    assert dl < LOGIT_ABS_TOL, dl
    assert dp < POOLED_REL_TOL, dp


@pytest.mark.parametrize("case", ["golden_small", "golden_large", "golden_mmbert"])
def test_torch_restatement_matches_oracle_and_golden(case):
    """oracle/torch_ref.py (the reference for the 8192-token and 64-request GPU cases) performs
    the oracle's steps in torch: it must meet the golden fixtures at the oracle's own tolerances
    and agree with the numpy oracle to float32 rounding."""
    import torch

    from oracle.torch_ref import TorchOracle

    z, cfg, agent, b, st = load_case(case)
    o = O.Oracle(st, cfg, agent)
    t = TorchOracle(o, "cpu")
    with torch.no_grad():
        rel, dl, dp = compare(z, t, b)
    assert rel < HIDDEN_REL_TOL, rel
    assert dl < LOGIT_ABS_TOL, dl
    assert dp < POOLED_REL_TOL, dp
    enc_t, enc_o = t.encoder_hidden(b), o.encoder_hidden(b)
    am = b.attention_mask.reshape(b.n, b.len).astype(bool)
    d = np.linalg.norm(enc_t[am] - enc_o[am], axis=-1) / np.linalg.norm(enc_o[am], axis=-1)
    assert float(d.max()) < 2e-5, float(d.max())
    lt, _ = t.forward(b, enc_o)
    lo, _ = o.forward(b, enc_o)
    assert float(np.abs(lt - lo).max()) < 1e-5


@pytest.mark.parametrize("headprune", [True, False])
@pytest.mark.parametrize("case", ["golden_small", "golden_large"])
def test_batched_torch_restatement_matches_oracle(case, headprune):
    """TorchOracle.forward_batched, the CPU baseline's forward (the whole padded batch per layer,
    torch's fused layer_norm / gelu / attention, the pruned last head layer), gives the oracle's
    logits and pooled rows to float32 rounding, with and without head pruning."""
    import torch

    from oracle.torch_ref import TorchOracle

    z, cfg, agent, b, st = load_case(case)
    o = O.Oracle(st, cfg, agent)
    lo, po = o.forward(b)
    with torch.no_grad():
        lt, pt = TorchOracle(o, "cpu").forward_batched(b, headprune=headprune)
    assert lt.shape == lo.shape and pt.shape == po.shape
    assert float(np.abs(lt - lo).max()) < 1e-4, float(np.abs(lt - lo).max())
    assert float(np.linalg.norm(pt - po) / np.linalg.norm(po)) < 1e-5
    assert np.array_equal(lt == O.LOGIT_MASKED, lo == O.LOGIT_MASKED)
    # a planted mistake in the batched path is visible at these tolerances: the window one wider
    o.window += 1
    with torch.no_grad():
        lw, pw = TorchOracle(o, "cpu").forward_batched(b, headprune=headprune)
    assert float(np.linalg.norm(pw - po) / np.linalg.norm(po)) > 1e-4


@pytest.mark.parametrize("mistake", ["window+1", "theta_swap", "geglu_order", "head_scale", "drop_out_proj_bias",
                                     "emb_norm_weight_dropped", "rope_traditional"])
def test_planted_mistakes_fail_the_golden_check(small, mistake, monkeypatch):
    z, cfg, agent, b, st = small
    o = O.Oracle(st, cfg, agent)
    if mistake == "window+1":
        o.window += 1
    elif mistake == "theta_swap":
        o.tables = {False: o.tables[True], True: o.tables[False]}
    elif mistake == "geglu_order":
        I = o.inter
        for l in range(o.layers):
            k = f"encoder.layers.{l}.mlp.Wi.weight"
            o.w[k] = np.concatenate([o.w[k][I:], o.w[k][:I]], axis=0)
    elif mistake == "head_scale":
        o.head_heads = o.head_heads // 2
    elif mistake == "drop_out_proj_bias":
        for j in range(o.head_layers):
            o.w[f"head.layers.{j}.self_attn.out_proj.bias"] = np.zeros_like(o.w[f"head.layers.{j}.self_attn.out_proj.bias"])
    elif mistake == "emb_norm_weight_dropped":
        o.w["encoder.embeddings.norm.weight"] = np.ones(o.d, dtype=np.float32)
    elif mistake == "rope_traditional":
        def rope_interleaved(x, cos, sin):
            L = x.shape[-2]
            c, s = cos[:L], sin[:L]
            x1, x2 = x[..., 0::2], x[..., 1::2]
            y = np.empty_like(x)
            y[..., 0::2] = x1 * c - x2 * s
            y[..., 1::2] = x1 * s + x2 * c
            return y

        monkeypatch.setattr(O, "rope", rope_interleaved)
    rel, dl, dp = compare(z, o, b)
    assert rel > 10 * HIDDEN_REL_TOL or dl > 10 * LOGIT_ABS_TOL or dp > 10 * POOLED_REL_TOL, (mistake, rel, dl, dp)


def test_layer_norm_closed_form():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(5, 64)).astype(np.float32) * 3 + 1
    w = rng.normal(size=64).astype(np.float32)
    b = rng.normal(size=64).astype(np.float32)
    y = O.layer_norm(x, w, b, 1e-5)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + 1e-5) * w + b
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_gelu_special_values():
    x = np.array([0.0, 1.0, -1.0, 3.0, -3.0], dtype=np.float32)
    # 0.5 x (1 + erf(x / sqrt 2)) at known points: Phi(1) = 0.8413447460685429
    ref = np.array([0.0, 0.8413447460685429, -0.15865525393145707, 3 * 0.9986501019683699,
                    -3 * 0.0013498980316301], dtype=np.float64)
    np.testing.assert_allclose(O.gelu(x), ref, rtol=1e-6, atol=1e-7)


def test_rope_rotation_invariants():
    cos, sin = O.rope_tables(160000.0, 8192, 64)
    # position 0 is the identity, split_rope.rs:718-719
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    rng = np.random.default_rng(1)
    x = rng.normal(size=(2, 8192, 64)).astype(np.float32)
    y = O.rope(x, cos, sin)
    # each (i, i + 32) pair keeps its norm
    n0 = np.hypot(x[..., :32], x[..., 32:])
    n1 = np.hypot(y[..., :32], y[..., 32:])
    np.testing.assert_allclose(n0, n1, rtol=2e-6, atol=2e-6)
    # frequency i is theta^(-i/32): at p = 1 the angle is exactly inv_freq (to f32 rounding)
    inv = 160000.0 ** (-np.arange(32) / 32.0)
    np.testing.assert_allclose(np.arctan2(sin[1], cos[1]), inv, rtol=1e-6)
    # relative-position property: <R_p q, R_{p+t} k> depends on t only
    q, k = rng.normal(size=64).astype(np.float32), rng.normal(size=64).astype(np.float32)
    qq = O.rope(np.tile(q, (8192, 1)), cos, sin)
    kk = O.rope(np.tile(k, (8192, 1)), cos, sin)
    d1 = float(qq[10] @ kk[17])
    d2 = float(qq[100] @ kk[107])
    assert abs(d1 - d2) < 1e-4


def test_rows_are_independent_and_padding_invariant(small):
    z, cfg, agent, b, st = small
    o = O.Oracle(st, cfg, agent)
    enc = o.encoder_hidden(b)
    am = b.attention_mask.reshape(b.n, b.len)
    for r in range(b.n):
        one = b.rows([r])
        L = int(one.seq_lens[0])
        trimmed = Batch(1, L, one.kmax, one.input_ids[:L].copy(), one.attention_mask[:L].copy(), one.seq_lens,
                        one.marker_pos, one.marker_count, one.qtype)
        e1 = o.encoder_hidden(trimmed)[0]
        np.testing.assert_allclose(e1, enc[r][:L], rtol=2e-5, atol=2e-5)
        lg1, _ = o.forward(trimmed, o.encoder_hidden(trimmed))
        lg, _ = o.forward(b, enc)
        np.testing.assert_allclose(lg1, lg[r * b.kmax:(r + 1) * b.kmax], rtol=1e-5, atol=1e-5)
        assert am[r].sum() == L


def test_local_window_is_exactly_local(small):
    """A token beyond the window cannot change a local layer's output: with all layers local and
    one layer, perturbing a token at distance W + 1 leaves the query's output unchanged, while
    distance W changes it."""
    z, cfg, agent, b, st = small
    c = dict(cfg)
    c["num_hidden_layers"] = 1
    c["layer_types"] = ["sliding_attention"]
    o = O.Oracle(st, c, agent)
    W = o.window
    L = 40
    ids = b.input_ids[:L].astype(np.int64).copy()
    am = np.ones(L, dtype=np.uint32)
    base = o._encode_row(ids, am)
    for dist, changed in [(W + 1, False), (W, True)]:
        ids2 = ids.copy()
        ids2[2 + dist] = (ids2[2 + dist] + 1) % 1000
        out = o._encode_row(ids2, am)
        diff = float(np.abs(out[2] - base[2]).max())
        assert (diff > 0) == changed, (dist, diff)
