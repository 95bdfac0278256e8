"""The oracle: a CPU restatement, in numpy f32, of sys1rust's decision-model forward.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to check the HIP path's results (or as the timed CPU baseline);
the product path (libsys1hip) never calls it.

It follows MlxBackend op for op in the padded layout that `encoder_hidden` uses
(runtime/crates/laya-mlx/src/lib.rs:1525-1800, 1869-1878):

  encode        lib.rs:1525-1693  h = LN(tok_emb[ids]); 28 x {attn_norm (not layer 0), Wqkv,
                                  split + RoPE (split_rope.rs:44-54), SDPA with the additive
                                  -1e4 pad mask (global, lib.rs:1227-1235) or, on local layers,
                                  the path attn_ctx picks (lib.rs:1241-1310): pad + |i-j| <= W
                                  window masks (dense), chunked or banded windows, additive or
                                  boolean masks (local_attention), h += att Wo^T,
                                  mlp_norm, Wi, GeGLU (lib.rs:494-510), h += act Wo2^T};
                                  final_norm
  head_forward  lib.rs:1698-1765  h + type_emb[qtype]; pre-norm layers with biases, 16 heads,
                                  scale 1/sqrt(d/heads) (lib.rs:576-578), ReLU FFN
  score         lib.rs:1768-1800  LN_b at the marker rows, scorer1, exact GELU, scorer3; pooled
  forward       lib.rs:1852-1856  logits past marker_count set to -1e4

Numerics: weights are the checkpoint's bf16 values widened to f32; all arithmetic is f32 (the
reference's `f32` option, backend.rs:26-28). RoPE angles use the reference kernel's arithmetic
(split_rope.metal:46-49): inv_freq = exp2(-(i / half) * log2 theta) and p * inv_freq in f32,
with the cosine and sine of that f32 angle taken in double.

Pinned by tests/test_oracle.py against tests/golden/ fixtures written by transformers'
ModernBertModel and torch's TransformerEncoderLayer (an independent implementation of the same
model), against closed forms (LayerNorm, GELU, the RoPE rotation) and against brute-force
invariants (row independence, padding invariance, window locality); the mask paths against the
reference's chunk-table fixture (lib.rs:2175-2247) and a slot-by-slot brute force.
"""
from __future__ import annotations

import json
import struct

import numpy as np
from scipy.special import erf

MASK_NEG = np.float32(-1e4)  # lib.rs:43
LOGIT_MASKED = np.float32(-1e4)  # lib.rs:45


def load_safetensors(b: bytes) -> dict:
    """name -> f32 array (weights.rs:82-103 to_f32)."""
    (hlen,) = struct.unpack("<Q", b[:8])
    header = json.loads(b[8: 8 + hlen])
    base = 8 + hlen
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        s, e = t["data_offsets"]
        raw = b[base + s: base + e]
        dt = t["dtype"]
        if dt == "BF16":
            u = np.frombuffer(raw, dtype=np.uint16).astype(np.uint32) << 16
            a = u.view(np.float32)
        elif dt == "F16":
            a = np.frombuffer(raw, dtype=np.float16).astype(np.float32)
        elif dt == "F32":
            a = np.frombuffer(raw, dtype=np.float32).copy()
        elif dt == "F64":
            a = np.frombuffer(raw, dtype=np.float64).astype(np.float32)
        else:
            raise ValueError(f"unsupported dtype {dt}")
        out[name] = a.reshape(t["shape"])
    return out


def layer_norm(x: np.ndarray, w: np.ndarray, b, eps: float) -> np.ndarray:
    """fast::layer_norm over the last axis (lib.rs:631-641): f32 mean and biased variance."""
    x = x.astype(np.float32, copy=False)
    mu = x.mean(axis=-1, keepdims=True, dtype=np.float32)
    c = x - mu
    var = (c * c).mean(axis=-1, keepdims=True, dtype=np.float32)
    y = c * (np.float32(1.0) / np.sqrt(var + np.float32(eps))) * w
    if b is not None:
        y = y + b
    return y.astype(np.float32, copy=False)


def gelu(x: np.ndarray) -> np.ndarray:
    """Exact GELU, 0.5 x (1 + erf(x / sqrt 2)) (lib.rs:494-510)."""
    x = x.astype(np.float32, copy=False)
    return (np.float32(0.5) * x * (np.float32(1.0) + erf(x * np.float32(0.7071067811865476)).astype(np.float32)))


def rope_tables(theta: float, max_pos: int, head_dim: int):
    """cos, sin [max_pos, head_dim / 2] f32 with the angle arithmetic of split_rope.metal:46-49."""
    half = head_dim // 2
    th = np.float32(theta)
    lbase = np.float32(np.log2(np.float64(th)))
    i = np.arange(half, dtype=np.float32)
    ex = (-(i / np.float32(half))) * lbase  # f32
    inv = np.exp2(ex.astype(np.float64)).astype(np.float32)
    p = np.arange(max_pos, dtype=np.float32)
    ang = p[:, None] * inv[None, :]  # f32 product
    return np.cos(ang.astype(np.float64)).astype(np.float32), np.sin(ang.astype(np.float64)).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Half-split rotation (MLX fast::rope, traditional=false): x [..., len, hd], pairs (i, i+hd/2)."""
    half = x.shape[-1] // 2
    L = x.shape[-2]
    c, s = cos[:L], sin[:L]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1).astype(np.float32)


def sdpa(q, k, v, scale: float, mask) -> np.ndarray:
    """softmax(q k^T scale + mask) v for one row: q, k, v [H, L, hd]; mask broadcastable to [H, L, L]."""
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * np.float32(scale)
    s = s + mask
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(p, v).astype(np.float32)


# ---- local attention as the reference chooses it per batch length (lib.rs:1241-1310, 1428-1475)
MASK_KEYS = ("mask", "windowed", "dense_upto", "band", "fuserope")


def mask_options(settings: str = "") -> dict:
    """The Knobs keys (lib.rs:196-256) that choose the attention masks, from a settings string:
    mask (additive | bool), windowed (flag, default on), dense_upto (None: 4 * window), band
    (0: off) and fuserope (band needs it, lib.rs:330-361). Other keys are ignored."""
    o = {"bool_mask": False, "windowed": True, "dense_upto": None, "band": 0, "fuserope": False}
    for kv in filter(None, settings.split(",")):
        key, _, val = kv.partition("=")
        flag = val in ("", "1")
        if key == "mask":
            o["bool_mask"] = val == "bool"
        elif key == "windowed":
            o["windowed"] = flag
        elif key == "dense_upto":
            o["dense_upto"] = int(val)
        elif key == "band":
            o["band"] = int(val)
        elif key == "fuserope":
            o["fuserope"] = flag
    return o


def band_allows(s: int) -> np.ndarray:
    """[S, 3S] bool (lib.rs:512-523): query i of a chunk may see gathered slot j iff |S + i - j| <= S."""
    i = np.arange(s)[:, None]
    j = np.arange(3 * s)[None, :]
    return np.abs(s + i - j) <= s


def window_positions(s: int, nc: int) -> np.ndarray:
    """[nc, 3S] int: slot j of chunk c holds position (c - 1) S + j (lib.rs:804-814, before the clamp)."""
    return (np.arange(nc)[:, None] - 1) * s + np.arange(3 * s)[None, :]


def window_key_valid(am: np.ndarray, s: int, nc: int) -> np.ndarray:
    """[nc, 3S] bool for one row (lib.rs:542-557): the slot's position lies in the row and is real."""
    pos = window_positions(s, nc)
    inside = (pos >= 0) & (pos < am.shape[0])
    return inside & (am[np.clip(pos, 0, am.shape[0] - 1)] == 1)


def window_query_padded(am: np.ndarray, s: int, nc: int) -> np.ndarray:
    """[nc, S] bool for one row (lib.rs:559-571): query c S + i is past the row or padding."""
    padded = np.ones(nc * s, dtype=bool)
    padded[: am.shape[0]] = am != 1
    return padded.reshape(nc, s)


def local_attention(q, k, v, am, scale: float, window: int, opts: dict) -> np.ndarray:
    """Local-layer attention of one padded row, q, k, v [H, len, hd], by the path the reference
    takes for this len (lib.rs:1241-1270): dense pad + window masks, chunked (1428-1475: queries
    in chunks of S = window against the 3S gathered keys of chunks c - 1, c, c + 1, clamped to
    the row), or banded (the chunked sdpa on a layout that is zero outside the row,
    split_rope.rs:56-59 and its test mlx_path_band_is_the_chunked_view, 622-657). Additive masks add -1e4 per failed test; boolean masks exclude, and
    padding queries may see every valid key (dense) or every gathered slot (chunked)."""
    L = q.shape[1]
    S = window
    dense_upto = opts["dense_upto"] if opts["dense_upto"] is not None else 4 * S
    banded = opts["band"] > 0 and opts["fuserope"] and not opts["bool_mask"] and L >= opts["band"]
    chunked = banded or (opts["windowed"] and L > dense_upto)
    real = am == 1
    if not chunked:
        idx = np.arange(L)
        inwin = np.abs(idx[:, None] - idx[None, :]) <= S
        if opts["bool_mask"]:  # lib.rs:1259-1264
            allowed = (inwin | ~real[:, None]) & real[None, :]
            mask = np.where(allowed, np.float32(0), np.float32(-np.inf)).astype(np.float32)
        else:  # pad + window (lib.rs:1265-1266)
            mask = (np.where(real, np.float32(0), MASK_NEG)[None, :] + np.where(inwin, np.float32(0), MASK_NEG)).astype(np.float32)
        return sdpa(q, k, v, scale, mask[None])
    H, hd = q.shape[0], q.shape[2]
    nc = -(-L // S)
    lp = nc * S
    qp = np.zeros((H, lp, hd), np.float32)
    qp[:, :L] = q
    qp = qp.reshape(H, nc, S, hd)
    pos = window_positions(S, nc)
    idx = np.clip(pos, 0, L - 1)
    kg, vg = k[:, idx], v[:, idx]  # [H, nc, 3S, hd]
    if banded:
        out = (pos < 0) | (pos >= L)
        kg[:, out] = 0
        vg[:, out] = 0
    key_ok = window_key_valid(am, S, nc)
    band = band_allows(S)
    if opts["bool_mask"]:  # lib.rs:1279-1291
        allowed = (key_ok[:, None, :] & band[None]) | window_query_padded(am, S, nc)[:, :, None]
        mask = np.where(allowed, np.float32(0), np.float32(-np.inf)).astype(np.float32)
    else:  # lib.rs:1292-1297
        mask = (np.where(key_ok, np.float32(0), MASK_NEG)[:, None, :] + np.where(band, np.float32(0), MASK_NEG)[None]).astype(np.float32)
    att = sdpa(qp, kg, vg, scale, mask[None])  # [H, nc, S, hd]
    return att.reshape(H, lp, hd)[:, :L]


class Oracle:
    def __init__(self, st_bytes: bytes, encoder_config: dict, agent_config: dict | None = None, settings: str = ""):
        """settings: the backend settings string; its mask keys (mask_options) choose the local
        attention of the padded layout, which only the padding positions tell apart."""
        self.w = load_safetensors(st_bytes)
        self.opts = mask_options(settings)
        c = encoder_config
        self.d = c["hidden_size"]
        self.layers = c["num_hidden_layers"]
        self.heads = c["num_attention_heads"]
        self.hd = self.d // self.heads
        self.inter = c["intermediate_size"]
        self.eps = c.get("norm_eps", c.get("layer_norm_eps", 1e-5))
        every = c.get("global_attn_every_n_layers", 3)
        self.window = c.get("local_attention", 128) // 2
        g_theta = c.get("global_rope_theta", 160000.0)
        l_theta = c.get("local_rope_theta", 10000.0)
        rp = c.get("rope_parameters") or {}
        g_theta = (rp.get("full_attention") or {}).get("rope_theta", g_theta)
        l_theta = (rp.get("sliding_attention") or {}).get("rope_theta", l_theta)
        lt = c.get("layer_types")
        if lt and len(lt) == self.layers:
            self.local = [t == "sliding_attention" for t in lt]
        else:
            self.local = [i % every != 0 for i in range(self.layers)]
        self.max_pos = c.get("max_position_embeddings", 8192)
        self.tables = {False: rope_tables(g_theta, self.max_pos, self.hd), True: rope_tables(l_theta, self.max_pos, self.hd)}
        a = agent_config or {}
        self.head_layers = a.get("head_layers", 2)
        self.head_heads = max(1, self.d // 64)

    # ---- encoder (lib.rs:1525-1693), one padded row at a time
    def _encode_row(self, ids: np.ndarray, am: np.ndarray) -> np.ndarray:
        w, d, H, hd = self.w, self.d, self.heads, self.hd
        L = ids.shape[0]
        h = layer_norm(w["encoder.embeddings.tok_embeddings.weight"][ids], w["encoder.embeddings.norm.weight"], None, self.eps)
        # the key-padding mask of global layers (lib.rs:1227-1235; boolean: exclusion)
        pad_neg = np.float32(-np.inf) if self.opts["bool_mask"] else MASK_NEG
        pad = np.where(am == 1, np.float32(0), pad_neg).astype(np.float32)[None, None, :]  # [1, 1, L]
        scale = 1.0 / np.sqrt(np.float32(hd))
        for l in range(self.layers):
            p = f"encoder.layers.{l}"
            a = h if l == 0 else layer_norm(h, w[f"{p}.attn_norm.weight"], None, self.eps)
            qkv = a @ w[f"{p}.attn.Wqkv.weight"].T
            q = qkv[:, :d].reshape(L, H, hd).transpose(1, 0, 2)
            k = qkv[:, d: 2 * d].reshape(L, H, hd).transpose(1, 0, 2)
            v = qkv[:, 2 * d:].reshape(L, H, hd).transpose(1, 0, 2)
            cos, sin = self.tables[self.local[l]]
            q, k = rope(q, cos, sin), rope(k, cos, sin)
            if self.local[l]:
                att = local_attention(q, k, np.ascontiguousarray(v), am, scale, self.window, self.opts)
            else:
                att = sdpa(q, k, np.ascontiguousarray(v), scale, pad)
            att = att.transpose(1, 0, 2).reshape(L, d)
            h = h + att @ w[f"{p}.attn.Wo.weight"].T
            m = layer_norm(h, w[f"{p}.mlp_norm.weight"], None, self.eps)
            wi = m @ w[f"{p}.mlp.Wi.weight"].T
            act = gelu(wi[:, : self.inter]) * wi[:, self.inter:]
            h = h + act @ w[f"{p}.mlp.Wo.weight"].T
        return layer_norm(h, w["encoder.final_norm.weight"], None, self.eps)

    def encoder_hidden(self, b) -> np.ndarray:
        """Backend::encoder_hidden: [n, len, d] f32, padding positions included."""
        ids = b.input_ids.reshape(b.n, b.len).astype(np.int64)
        am = b.attention_mask.reshape(b.n, b.len)
        return np.stack([self._encode_row(ids[r], am[r]) for r in range(b.n)]).astype(np.float32)

    # ---- head (lib.rs:1698-1765) and scorer (lib.rs:1768-1800)
    def _head_row(self, enc: np.ndarray, am: np.ndarray, qtype: int) -> np.ndarray:
        w, d = self.w, self.d
        H = self.head_heads
        hd = d // H
        L = enc.shape[0]
        h = enc + w["type_emb.weight"][qtype]
        pad = np.where(am == 1, np.float32(0), MASK_NEG).astype(np.float32)[None, None, :]
        scale = 1.0 / np.sqrt(np.float32(hd))
        for j in range(self.head_layers):
            p = f"head.layers.{j}"
            x = layer_norm(h, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], 1e-5)
            qkv = x @ w[f"{p}.self_attn.in_proj_weight"].T + w[f"{p}.self_attn.in_proj_bias"]
            q = qkv[:, :d].reshape(L, H, hd).transpose(1, 0, 2)
            k = qkv[:, d: 2 * d].reshape(L, H, hd).transpose(1, 0, 2)
            v = qkv[:, 2 * d:].reshape(L, H, hd).transpose(1, 0, 2)
            att = sdpa(q, k, np.ascontiguousarray(v), scale, pad).transpose(1, 0, 2).reshape(L, d)
            h = h + att @ w[f"{p}.self_attn.out_proj.weight"].T + w[f"{p}.self_attn.out_proj.bias"]
            x = layer_norm(h, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], 1e-5)
            x = np.maximum(x @ w[f"{p}.linear1.weight"].T + w[f"{p}.linear1.bias"], np.float32(0))
            h = h + x @ w[f"{p}.linear2.weight"].T + w[f"{p}.linear2.bias"]
        return h.astype(np.float32)

    def forward(self, b, enc: np.ndarray | None = None):
        """Backend::forward: (logits [n*kmax], pooled [n*d]), f32."""
        w = self.w
        if enc is None:
            enc = self.encoder_hidden(b)
        am = b.attention_mask.reshape(b.n, b.len)
        logits = np.zeros(b.n * b.kmax, dtype=np.float32)
        pooled = np.zeros((b.n, self.d), dtype=np.float32)
        for r in range(b.n):
            h = self._head_row(enc[r], am[r], int(b.qtype[r]))
            pooled[r] = h[0]
            if b.kmax == 0:
                continue
            rows = h[b.marker_pos.reshape(b.n, b.kmax)[r].astype(np.int64)]
            s = layer_norm(rows, w["scorer.0.weight"], w["scorer.0.bias"], 1e-5)
            s = gelu(s @ w["scorer.1.weight"].T + w["scorer.1.bias"])
            lg = (s @ w["scorer.3.weight"].T + w["scorer.3.bias"]).reshape(-1)
            lg = np.where(np.arange(b.kmax) < int(b.marker_count[r]), lg, LOGIT_MASKED)
            logits[r * b.kmax: (r + 1) * b.kmax] = lg
        return logits, pooled.reshape(-1)
