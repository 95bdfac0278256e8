"""The oracle's forward restated in torch float32, for checks at sizes numpy cannot finish.

TEST INFRASTRUCTURE, under the same rule as oracle.py: only tests/ may import it, as a checker.

It takes an oracle.Oracle (the parsed config, the checkpoint widened to f32 and the RoPE tables)
and performs the same steps in the same order as Oracle._encode_row, Oracle._head_row and
Oracle.forward (runtime/crates/laya-mlx/src/lib.rs:1525-1800): LayerNorm with f32 mean and
biased variance, exact-erf GELU, the half-split RoPE rotation, softmax attention with the -1e4
additive pad and window masks, all in float32 on any torch device. On a GPU it runs the
8192-token state and the rows of the 64-request sweep in seconds, where the numpy oracle needs
minutes (its attention is a dense [H, L, L] product per row either way).

Pinned by tests/test_oracle.py: on the golden batches it agrees with oracle.py to float32
rounding, and through it with the transformers / torch fixtures that pin oracle.py.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O


class TorchOracle:
    def __init__(self, o: O.Oracle, device: str = "cpu"):
        # f32 products must stay f32 (no reduced-precision inner products).
        torch.backends.cuda.matmul.allow_tf32 = False
        self.o = o
        self.dev = torch.device(device)
        self.w = {k: torch.from_numpy(np.ascontiguousarray(v)).to(self.dev) for k, v in o.w.items()}
        self.tables = {k: tuple(torch.from_numpy(t).to(self.dev) for t in v) for k, v in o.tables.items()}

    # ---- the oracle's helpers (oracle.layer_norm, gelu, rope, sdpa)
    @staticmethod
    def layer_norm(x, w, b, eps: float):
        mu = x.mean(dim=-1, keepdim=True)
        c = x - mu
        var = (c * c).mean(dim=-1, keepdim=True)
        y = c * (1.0 / torch.sqrt(var + eps)) * w
        return y + b if b is not None else y

    @staticmethod
    def gelu(x):
        return 0.5 * x * (1.0 + torch.erf(x * 0.7071067811865476))

    @staticmethod
    def rope(x, cos, sin):
        half = x.shape[-1] // 2
        L = x.shape[-2]
        c, s = cos[:L], sin[:L]
        x1, x2 = x[..., :half], x[..., half:]
        return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], dim=-1)

    @staticmethod
    def sdpa(q, k, v, scale: float, mask):
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
        s = s + mask
        s = s - s.amax(dim=-1, keepdim=True)
        e = torch.exp(s)
        p = e / e.sum(dim=-1, keepdim=True)
        return torch.matmul(p, v.contiguous())

    # ---- encoder (Oracle._encode_row)
    def _encode_row(self, ids: np.ndarray, am: np.ndarray) -> torch.Tensor:
        o, w = self.o, self.w
        d, H, hd = o.d, o.heads, o.hd
        L = ids.shape[0]
        idt = torch.from_numpy(ids.astype(np.int64)).to(self.dev)
        amt = torch.from_numpy(am.astype(np.int64)).to(self.dev)
        h = self.layer_norm(w["encoder.embeddings.tok_embeddings.weight"][idt], w["encoder.embeddings.norm.weight"],
                            None, o.eps)
        neg = torch.tensor(float(O.MASK_NEG), device=self.dev)
        zero = torch.tensor(0.0, device=self.dev)
        pad = torch.where(amt == 1, zero, neg)[None, None, :]
        idx = torch.arange(L, device=self.dev)
        win = torch.where((idx[:, None] - idx[None, :]).abs() > o.window, neg, zero)
        scale = float(1.0 / np.sqrt(np.float32(hd)))
        for l in range(o.layers):
            p = f"encoder.layers.{l}"
            a = h if l == 0 else self.layer_norm(h, w[f"{p}.attn_norm.weight"], None, o.eps)
            qkv = a @ w[f"{p}.attn.Wqkv.weight"].T
            q = qkv[:, :d].reshape(L, H, hd).transpose(0, 1)
            k = qkv[:, d: 2 * d].reshape(L, H, hd).transpose(0, 1)
            v = qkv[:, 2 * d:].reshape(L, H, hd).transpose(0, 1)
            cos, sin = self.tables[o.local[l]]
            q, k = self.rope(q, cos, sin), self.rope(k, cos, sin)
            mask = pad + win[None] if o.local[l] else pad
            att = self.sdpa(q, k, v, scale, mask).transpose(0, 1).reshape(L, d)
            h = h + att @ w[f"{p}.attn.Wo.weight"].T
            m = self.layer_norm(h, w[f"{p}.mlp_norm.weight"], None, o.eps)
            wi = m @ w[f"{p}.mlp.Wi.weight"].T
            act = self.gelu(wi[:, : o.inter]) * wi[:, o.inter:]
            h = h + act @ w[f"{p}.mlp.Wo.weight"].T
        return self.layer_norm(h, w["encoder.final_norm.weight"], None, o.eps)

    @torch.no_grad()
    def encoder_hidden(self, b) -> np.ndarray:
        """[n, len, d] f32 like Oracle.encoder_hidden (padding positions included)."""
        ids = b.input_ids.reshape(b.n, b.len)
        am = b.attention_mask.reshape(b.n, b.len)
        return np.stack([self._encode_row(ids[r], am[r]).cpu().numpy() for r in range(b.n)]).astype(np.float32)

    # ---- head and scorer (Oracle._head_row, Oracle.forward)
    def _head_row(self, enc: torch.Tensor, am: np.ndarray, qtype: int) -> torch.Tensor:
        o, w = self.o, self.w
        d, H = o.d, o.head_heads
        hd = d // H
        L = enc.shape[0]
        h = enc + w["type_emb.weight"][qtype]
        amt = torch.from_numpy(am.astype(np.int64)).to(self.dev)
        pad = torch.where(amt == 1, torch.tensor(0.0, device=self.dev),
                          torch.tensor(float(O.MASK_NEG), device=self.dev))[None, None, :]
        scale = float(1.0 / np.sqrt(np.float32(hd)))
        for j in range(o.head_layers):
            p = f"head.layers.{j}"
            x = self.layer_norm(h, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], 1e-5)
            qkv = x @ w[f"{p}.self_attn.in_proj_weight"].T + w[f"{p}.self_attn.in_proj_bias"]
            q = qkv[:, :d].reshape(L, H, hd).transpose(0, 1)
            k = qkv[:, d: 2 * d].reshape(L, H, hd).transpose(0, 1)
            v = qkv[:, 2 * d:].reshape(L, H, hd).transpose(0, 1)
            att = self.sdpa(q, k, v, scale, pad).transpose(0, 1).reshape(L, d)
            h = h + att @ w[f"{p}.self_attn.out_proj.weight"].T + w[f"{p}.self_attn.out_proj.bias"]
            x = self.layer_norm(h, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], 1e-5)
            x = torch.clamp_min(x @ w[f"{p}.linear1.weight"].T + w[f"{p}.linear1.bias"], 0.0)
            h = h + x @ w[f"{p}.linear2.weight"].T + w[f"{p}.linear2.bias"]
        return h

    @torch.no_grad()
    def forward(self, b, enc: np.ndarray):
        """(logits [n*kmax], pooled [n*d]) f32 like Oracle.forward, from encoder_hidden's output."""
        o, w = self.o, self.w
        am = b.attention_mask.reshape(b.n, b.len)
        logits = np.zeros(b.n * b.kmax, dtype=np.float32)
        pooled = np.zeros((b.n, o.d), dtype=np.float32)
        for r in range(b.n):
            h = self._head_row(torch.from_numpy(np.ascontiguousarray(enc[r])).to(self.dev), am[r], int(b.qtype[r]))
            pooled[r] = h[0].cpu().numpy()
            if b.kmax == 0:
                continue
            mp = torch.from_numpy(b.marker_pos.reshape(b.n, b.kmax)[r].astype(np.int64)).to(self.dev)
            s = self.layer_norm(h[mp], w["scorer.0.weight"], w["scorer.0.bias"], 1e-5)
            s = self.gelu(s @ w["scorer.1.weight"].T + w["scorer.1.bias"])
            lg = (s @ w["scorer.3.weight"].T + w["scorer.3.bias"]).reshape(-1).cpu().numpy()
            lg = np.where(np.arange(b.kmax) < int(b.marker_count[r]), lg, O.LOGIT_MASKED)
            logits[r * b.kmax: (r + 1) * b.kmax] = lg
        return logits, pooled.reshape(-1)
