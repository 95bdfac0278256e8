"""The oracle's forward restated in torch float32, for checks at sizes numpy cannot finish.

TEST INFRASTRUCTURE, under the same rule as oracle.py: only tests/ may import it, as a checker.

It takes an oracle.Oracle (the parsed config, the checkpoint widened to f32 and the RoPE tables)
and performs the same steps in the same order as Oracle._encode_row, Oracle._head_row and
Oracle.forward (runtime/crates/laya-mlx/src/lib.rs:1525-1800): LayerNorm with f32 mean and
biased variance, exact-erf GELU, the half-split RoPE rotation, softmax attention with the
reference's masks (dense, chunked or banded local attention by the oracle's mask options), all
in float32 on any torch device. On a GPU it runs the
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

    def local_attention(self, q, k, v, am: np.ndarray, scale: float):
        """oracle.local_attention in torch: dense, chunked or banded by the oracle's mask options."""
        o = self.o
        opts, S = o.opts, o.window
        L = q.shape[1]
        dense_upto = opts["dense_upto"] if opts["dense_upto"] is not None else 4 * S
        banded = opts["band"] > 0 and opts["fuserope"] and not opts["bool_mask"] and L >= opts["band"]
        chunked = banded or (opts["windowed"] and L > dense_upto)
        real = torch.from_numpy(am == 1).to(self.dev)
        zero = torch.tensor(0.0, device=self.dev)
        neg = torch.tensor(float(O.MASK_NEG), device=self.dev)
        ninf = torch.tensor(float("-inf"), device=self.dev)
        if not chunked:
            idx = torch.arange(L, device=self.dev)
            inwin = (idx[:, None] - idx[None, :]).abs() <= S
            if opts["bool_mask"]:
                mask = torch.where((inwin | ~real[:, None]) & real[None, :], zero, ninf)
            else:
                mask = torch.where(real, zero, neg)[None, :] + torch.where(inwin, zero, neg)
            return self.sdpa(q, k, v, scale, mask[None])
        H, hd = q.shape[0], q.shape[2]
        nc = -(-L // S)
        qp = torch.zeros((H, nc * S, hd), device=self.dev)
        qp[:, :L] = q
        qp = qp.reshape(H, nc, S, hd)
        pos = torch.from_numpy(O.window_positions(S, nc)).to(self.dev)
        idx = pos.clamp(0, L - 1)
        kg, vg = k[:, idx], v[:, idx]
        if banded:
            out = (pos < 0) | (pos >= L)
            kg[:, out] = 0
            vg[:, out] = 0
        key_ok = torch.from_numpy(O.window_key_valid(am, S, nc)).to(self.dev)
        band = torch.from_numpy(O.band_allows(S)).to(self.dev)
        if opts["bool_mask"]:
            padded = torch.from_numpy(O.window_query_padded(am, S, nc)).to(self.dev)
            mask = torch.where((key_ok[:, None, :] & band[None]) | padded[:, :, None], zero, ninf)
        else:
            mask = torch.where(key_ok, zero, neg)[:, None, :] + torch.where(band, zero, neg)[None]
        att = self.sdpa(qp, kg, vg, scale, mask[None])
        return att.reshape(H, nc * S, hd)[:, :L]

    # ---- encoder (Oracle._encode_row)
    def _encode_row(self, ids: np.ndarray, am: np.ndarray) -> torch.Tensor:
        o, w = self.o, self.w
        d, H, hd = o.d, o.heads, o.hd
        L = ids.shape[0]
        idt = torch.from_numpy(ids.astype(np.int64)).to(self.dev)
        amt = torch.from_numpy(am.astype(np.int64)).to(self.dev)
        h = self.layer_norm(w["encoder.embeddings.tok_embeddings.weight"][idt], w["encoder.embeddings.norm.weight"],
                            None, o.eps)
        neg = torch.tensor(float("-inf") if o.opts["bool_mask"] else float(O.MASK_NEG), device=self.dev)
        zero = torch.tensor(0.0, device=self.dev)
        pad = torch.where(amt == 1, zero, neg)[None, None, :]
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
            att = self.local_attention(q, k, v, am, scale) if o.local[l] else self.sdpa(q, k, v, scale, pad)
            att = att.transpose(0, 1).reshape(L, d)
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

    # ---- the whole padded batch at once, as the reference's CPU path runs it
    @torch.no_grad()
    def forward_batched(self, b, headprune: bool = True):
        """(logits [n*kmax], pooled [n*d]) for the padded batch in one pass per layer: the
        reference's forward as its CPU device runs it (MlxBackend::forward on BackendOptions
        device Cpu, lib.rs:1525-1863, backend.rs:14-20): [n, len] rows with the -1e4 pad mask
        and, on local layers, the dense window mask (dense_upto, lib.rs:1399-1417,1646-1649);
        with headprune the last head layer keeps every key and value but runs its queries,
        out_proj, norm2 and FFN at the scorer's rows only (lib.rs:1728-1748). The same
        operations as the per-row methods above, through torch's fused CPU kernels (layer_norm,
        gelu, scaled_dot_product_attention); pinned to them by tests/test_oracle.py."""
        import torch.nn.functional as F

        o, w = self.o, self.w
        d, H, hd, n, L = o.d, o.heads, o.hd, b.n, b.len
        ids = torch.from_numpy(b.input_ids.reshape(n, L).astype(np.int64)).to(self.dev)
        am = torch.from_numpy(b.attention_mask.reshape(n, L).astype(np.int64)).to(self.dev)
        neg = float(O.MASK_NEG)
        pad = torch.where(am == 1, 0.0, neg).to(torch.float32)[:, None, None, :]  # [n, 1, 1, L]
        idx = torch.arange(L, device=self.dev)
        win = torch.where((idx[:, None] - idx[None, :]).abs() > o.window, neg, 0.0).to(torch.float32)
        masks = {False: pad, True: pad + win}
        scale = float(1.0 / np.sqrt(np.float32(hd)))

        def heads(x, rows, nh):  # [n, rows, nh * 64] -> [n, nh, rows, 64]
            return x.view(n, rows, nh, -1).transpose(1, 2)

        def rope(x, cos, sin):
            half = x.shape[-1] // 2
            x1, x2 = x[..., :half], x[..., half:]
            return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)

        h = F.layer_norm(w["encoder.embeddings.tok_embeddings.weight"][ids], (d,),
                         w["encoder.embeddings.norm.weight"], None, o.eps)
        for l in range(o.layers):
            p = f"encoder.layers.{l}"
            a = h if l == 0 else F.layer_norm(h, (d,), w[f"{p}.attn_norm.weight"], None, o.eps)
            q, k, v = (a @ w[f"{p}.attn.Wqkv.weight"].T).split(d, dim=-1)
            cos, sin = (t[:L] for t in self.tables[o.local[l]])
            q, k, v = rope(heads(q, L, H), cos, sin), rope(heads(k, L, H), cos, sin), heads(v, L, H)
            att = F.scaled_dot_product_attention(q, k, v, attn_mask=masks[o.local[l]], scale=scale)
            h = h + att.transpose(1, 2).reshape(n, L, d) @ w[f"{p}.attn.Wo.weight"].T
            m = F.layer_norm(h, (d,), w[f"{p}.mlp_norm.weight"], None, o.eps)
            x, g = (m @ w[f"{p}.mlp.Wi.weight"].T).split(o.inter, dim=-1)
            h = h + (F.gelu(x) * g) @ w[f"{p}.mlp.Wo.weight"].T
        h = F.layer_norm(h, (d,), w["encoder.final_norm.weight"], None, o.eps)

        # decision head (Oracle._head_row), rows of the scorer: position 0, then the markers
        Hh = o.head_heads
        h = h + w["type_emb.weight"][torch.from_numpy(b.qtype.astype(np.int64)).to(self.dev)][:, None, :]
        kmax = b.kmax
        pick = torch.zeros(n, 1 + kmax, dtype=torch.int64, device=self.dev)
        if kmax:
            pick[:, 1:] = torch.from_numpy(b.marker_pos.reshape(n, kmax).astype(np.int64)).to(self.dev)
        for j in range(o.head_layers):
            p = f"head.layers.{j}"
            x = F.layer_norm(h, (d,), w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], 1e-5)
            wq, wk, wv = w[f"{p}.self_attn.in_proj_weight"].split(d, dim=0)
            bq, bk, bv = w[f"{p}.self_attn.in_proj_bias"].split(d, dim=0)
            k, v = heads(x @ wk.T + bk, L, Hh), heads(x @ wv.T + bv, L, Hh)
            last = headprune and j == o.head_layers - 1
            if last:  # queries and everything after them at the picked rows only
                gidx = pick[:, :, None].expand(n, 1 + kmax, d)
                x, h = x.gather(1, gidx), h.gather(1, gidx)
            rows = x.shape[1]
            q = heads(x @ wq.T + bq, rows, Hh)
            att = F.scaled_dot_product_attention(q, k, v, attn_mask=pad, scale=1.0 / np.sqrt(d // Hh))
            h = h + att.transpose(1, 2).reshape(n, rows, d) @ w[f"{p}.self_attn.out_proj.weight"].T \
                + w[f"{p}.self_attn.out_proj.bias"]
            x = F.layer_norm(h, (d,), w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], 1e-5)
            x = torch.clamp_min(x @ w[f"{p}.linear1.weight"].T + w[f"{p}.linear1.bias"], 0.0)
            h = h + x @ w[f"{p}.linear2.weight"].T + w[f"{p}.linear2.bias"]
        if h.shape[1] != 1 + kmax:
            h = h.gather(1, pick[:, :, None].expand(n, 1 + kmax, d))
        pooled = h[:, 0].reshape(-1).cpu().numpy().astype(np.float32)
        if kmax == 0:
            return np.zeros(0, np.float32), pooled
        s = F.layer_norm(h[:, 1:], (d,), w["scorer.0.weight"], w["scorer.0.bias"], 1e-5)
        s = F.gelu(s @ w["scorer.1.weight"].T + w["scorer.1.bias"])
        lg = (s @ w["scorer.3.weight"].T + w["scorer.3.bias"]).reshape(n, kmax).cpu().numpy()
        live = np.arange(kmax)[None, :] < b.marker_count.astype(np.int64)[:, None]
        return np.where(live, lg, O.LOGIT_MASKED).astype(np.float32).reshape(-1), pooled

