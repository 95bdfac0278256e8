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


# ---- the local-attention paths the reference picks per batch length (lib.rs:1241-1310)
MODES = {
    "dense": "windowed=0",
    "chunked": "dense_upto=0",
    "banded": "band=1,fuserope",
    "bool_dense": "mask=bool,windowed=0",
    "bool_chunked": "mask=bool,dense_upto=0",
}


def test_chunk_tables_known_answers():
    """The reference's own fixture (lib.rs:2175-2180): S = 2, len = 7, row 0 all real, row 1 three
    real tokens. Tables written out by hand from the position rule (slot j of chunk c holds
    position (c - 1) S + j); row 1's fourth chunk holds no valid key (lib.rs:2246-2247)."""
    T, F = True, False
    rows = [np.ones(7, np.uint32), np.array([1, 1, 1, 0, 0, 0, 0], np.uint32)]
    want_keys = [
        [[F, F, T, T, T, T], [T, T, T, T, T, T], [T, T, T, T, T, F], [T, T, T, F, F, F]],
        [[F, F, T, T, T, F], [T, T, T, F, F, F], [T, F, F, F, F, F], [F, F, F, F, F, F]],
    ]
    want_padded = [
        [[F, F], [F, F], [F, F], [F, T]],
        [[F, F], [F, T], [T, T], [T, T]],
    ]
    for am, wk, wp in zip(rows, want_keys, want_padded):
        assert O.window_key_valid(am, 2, 4).tolist() == wk
        assert O.window_query_padded(am, 2, 4).tolist() == wp
    # lib.rs:2202-2210: band[i, j] iff i + 2S >= j >= i
    assert O.band_allows(2).tolist() == [[T, T, T, T, T, F], [F, T, T, T, T, T]]


def _brute_local(q, k, v, am, scale, S, mode):
    """One query at a time, one key slot at a time, from the rules as the reference states them:
    dense masks over the row's keys, or the chunk's 3S gathered slots (position (c - 1) S + j,
    clamped to the row; zero outside it when banded), -1e4 per failed test (additive) or
    exclusion (boolean, padding queries seeing every valid key / every slot)."""
    H, L, hd = q.shape
    out = np.zeros_like(q, dtype=np.float64)
    chunked = mode in ("chunked", "banded", "bool_chunked")
    boolean = mode.startswith("bool")
    for h in range(H):
        for t in range(L):
            pad_q = am[t] != 1
            scores, vals = [], []
            slots = range(3 * S) if chunked else range(L)
            for j in slots:
                p = (t // S - 1) * S + j if chunked else j
                inside = 0 <= p < L
                pc = min(max(p, 0), L - 1)
                valid = inside and am[pc] == 1
                inband = abs(t - p) <= S
                kk, vv = k[h, pc].astype(np.float64), v[h, pc].astype(np.float64)
                if mode == "banded" and not inside:
                    kk, vv = np.zeros(hd), np.zeros(hd)
                s = float(q[h, t].astype(np.float64) @ kk) * scale
                if boolean:
                    if not ((valid and inband) or (pad_q and (chunked or valid))):
                        continue
                else:  # the masks are added to the f32 score in f32, as the oracle and MLX's f32 path do
                    s = float(np.float32(s) + np.float32((0.0 if valid else -1e4) + (0.0 if inband else -1e4)))
                scores.append(s)
                vals.append(vv)
            sc = np.array(scores)
            w = np.exp(sc - sc.max())
            out[h, t] = (w[:, None] * np.array(vals)).sum(0) / w.sum()
    return out


@pytest.mark.parametrize("mode", list(MODES))
def test_local_attention_paths_brute_force(mode):
    """oracle.local_attention on every path against the slot-by-slot restatement, at every query
    of rows with padding up to and beyond the window, and a length that is not a multiple of S."""
    rng = np.random.default_rng(3)
    H, hd, S = 2, 8, 4
    opts = O.mask_options(MODES[mode])
    for L, real in [(23, 9), (16, 16), (13, 1), (8, 5)]:
        q, k, v = (rng.standard_normal((H, L, hd)).astype(np.float32) for _ in range(3))
        am = (np.arange(L) < real).astype(np.uint32)
        got = O.local_attention(q, k, v, am, 0.35, S, opts)
        want = _brute_local(q, k, v, am, 0.35, S, mode)
        # 1e-3: a score near -1e4 holds 2^-10 in f32, so an f32 rounding flip there moves a weight by 0.1 %
        np.testing.assert_allclose(got, want, rtol=2e-4, atol=1e-3, err_msg=f"{mode} L={L} real={real}")
        real_rows = np.arange(L) < real
        np.testing.assert_allclose(got[:, real_rows], want[:, real_rows], rtol=2e-4, atol=2e-5)


def test_local_attention_paths_agree_at_real_tokens():
    """Every path gives a real token the same attention (the real keys of its window): they differ
    at padding queries only, and there each path's padding outputs differ from the dense ones."""
    rng = np.random.default_rng(5)
    H, hd, S, L, real = 2, 8, 4, 29, 11
    q, k, v = (rng.standard_normal((H, L, hd)).astype(np.float32) for _ in range(3))
    am = (np.arange(L) < real).astype(np.uint32)
    outs = {m: O.local_attention(q, k, v, am, 0.35, S, O.mask_options(s)) for m, s in MODES.items()}
    for m, o in outs.items():
        np.testing.assert_allclose(o[:, :real], outs["dense"][:, :real], rtol=1e-5, atol=1e-6, err_msg=m)
        if m != "dense":
            assert float(np.abs(o[:, real + S + 1:] - outs["dense"][:, real + S + 1:]).max()) > 1e-3, m


def test_mask_path_follows_len():
    """Chunked local attention from dense_upto + 1 (default 4 * window) when windowed, banded from
    `band` when fuserope is on, dense otherwise: the oracle's choice, seen through the padding
    outputs."""
    rng = np.random.default_rng(9)
    H, hd, S = 1, 8, 2
    for L, settings, path in [(8, "", "dense"), (9, "", "chunked"), (9, "windowed=0", "dense"),
                              (9, "dense_upto=9", "dense"), (6, "band=6,fuserope", "banded"),
                              (6, "band=6", "dense"), (5, "band=6,fuserope", "dense")]:
        q, k, v = (rng.standard_normal((H, L, hd)).astype(np.float32) for _ in range(3))
        am = (np.arange(L) < 2).astype(np.uint32)
        got = O.local_attention(q, k, v, am, 0.35, S, O.mask_options(settings))
        np.testing.assert_allclose(got, _brute_local(q, k, v, am, 0.35, S, path), rtol=2e-4, atol=1e-3,
                                   err_msg=f"L={L} {settings}")


def test_mask_paths_change_the_padding_hidden_states(small):
    """On the golden batch (window 16; a row with padding past the window of its last real token),
    the mask paths give the same hidden states at the real tokens and, at the padding positions,
    states apart by more than twice the GPU parity gate (2e-2 relative): that gate tells the
    paths apart."""
    z, cfg, agent, b, st = small
    am = b.attention_mask.reshape(b.n, b.len).astype(bool)
    encs = {m: O.Oracle(st, cfg, agent, settings=s).encoder_hidden(b) for m, s in MODES.items()}
    base = encs["dense"]
    for m, e in encs.items():
        np.testing.assert_allclose(e[am], base[am], rtol=1e-5, atol=1e-5, err_msg=m)
        for m2, e2 in encs.items():
            if m2 <= m:
                continue
            rel = np.linalg.norm(e[~am] - e2[~am], axis=-1) / np.linalg.norm(e2[~am], axis=-1)
            assert float(rel.max()) > 0.05, (m, m2, float(rel.max()))
