"""Kernel-level parity on the GPU, through the C ABI's s1k_* entry points.

GEMM epilogues are checked against a float32 torch product of the same bf16 operands; the fused
Wqkv + split + RoPE product (the isolated M=512, K=1024, N=3072 case at both RoPE bases), the
standalone split + RoPE pass, attention and LayerNorm against the oracle's formulas in float32.
Tolerances are bf16-output tolerances: the kernels accumulate in f32 and round once to bf16
(relative step 2^-8).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _lib():
    from sys1rust_amd import _lib as L

    return L


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "gpu tests need a GPU"
    return torch.device("cuda:0")


def ptr(t):
    return C.c_void_p(t.data_ptr())


def stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def bf16_bits(t):
    return t.to(torch.bfloat16).contiguous().view(torch.int16)


def gemm(A, W, M, N, K, epi=0, act=0, bias=None, C_out=None):
    L = _lib()
    dev = A.device
    if C_out is None:
        if epi in (1, 3):
            C_out = torch.zeros(M, N, dtype=torch.float32, device=dev)
        elif epi == 2:
            C_out = torch.zeros(M, N // 2, dtype=torch.int16, device=dev)
        else:
            C_out = torch.zeros(M, N, dtype=torch.int16, device=dev)
    ldc = C_out.shape[1]
    L.check(L.lib().s1k_gemm(ptr(A), K, ptr(W), K, ptr(C_out), ldc, ptr(bias) if bias is not None else None, M, N, K,
                             epi, act, stream()))
    torch.cuda.synchronize()
    return C_out


def as_f32(bits):
    return bits.contiguous().view(torch.bfloat16).float()


# Tile configurations: small (M <= 1024 or few tiles, split-K below 96 tiles), mid (1024-wide
# outputs), large and wide (192-row tiles; 2001 and 11372 also end on partial row tiles).
SHAPES = [(1, 128, 64), (37, 256, 128), (170, 3072, 1024), (257, 1024, 1024), (563, 1024, 2624), (600, 5248, 1024),
          (1000, 4096, 1024), (2001, 5248, 1024), (5686, 1024, 1024), (11372, 1024, 2624)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_f32_and_bf16_outputs(dev, M, N, K):
    say(f"gemm M={M} N={N} K={K}")
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N)
    A = bf16_bits(torch.randn(M, K, generator=g)).to(dev)
    W = bf16_bits(torch.randn(N, K, generator=g) * 0.02).to(dev)
    ref = as_f32(A) @ as_f32(W).T
    out = gemm(A, W, M, N, K, epi=3)
    scale = float(ref.abs().max())
    err = float((out - ref).abs().max())
    assert err <= 2e-5 * scale + 1e-6, (err, scale)
    ob = as_f32(gemm(A, W, M, N, K, epi=0))
    err = (ob - ref).abs()
    assert bool((err <= ref.abs() * 2 ** -8 + 1e-5 * scale).all()), float(err.max())


@pytest.mark.parametrize("M,N", [(100, 1024), (300, 1024), (1500, 1024), (3100, 3072)])  # split-K, small, wide
def test_gemm_epilogues_bias_relu_gelu_residual_geglu(dev, M, N):
    K = 512
    g = torch.Generator(device="cpu").manual_seed(5)
    A = bf16_bits(torch.randn(M, K, generator=g)).to(dev)
    W = bf16_bits(torch.randn(N, K, generator=g) * 0.05).to(dev)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    ref = as_f32(A) @ as_f32(W).T + bias
    for act, f in [(1, torch.relu), (2, lambda x: torch.nn.functional.gelu(x))]:
        say(f"epilogue act={act}")
        ob = as_f32(gemm(A, W, M, N, K, epi=0, act=act, bias=bias))
        r = f(ref)
        assert bool(((ob - r).abs() <= r.abs() * 2 ** -8 + 1e-4).all())
    say("epilogue residual")
    h0 = torch.randn(M, N, generator=g).to(dev)
    h = h0.clone()
    gemm(A, W, M, N, K, epi=1, bias=bias, C_out=h)
    assert float((h - (h0 + ref)).abs().max()) < 1e-4
    say("epilogue geglu")
    # Wi = [x rows | gate rows]; the kernel wants them interleaved by blocks of 32 rows.
    I = N // 2
    Wf = as_f32(W)
    Wi = torch.cat([Wf[:I].reshape(I // 32, 32, K), Wf[I:].reshape(I // 32, 32, K)], dim=1).reshape(N, K)
    Wi_bits = bf16_bits(Wi)
    act = as_f32(gemm(A, Wi_bits, M, N, K, epi=2))
    x = as_f32(A) @ Wf[:I].T
    gate = as_f32(A) @ Wf[I:].T
    r = torch.nn.functional.gelu(x) * gate
    assert bool(((act - r).abs() <= r.abs() * 2 ** -7 + 1e-4).all()), float((act - r).abs().max())


@pytest.mark.parametrize("M", [5686, 5000])
def test_gemm_long_k_one_round_pipelined(dev, M):
    """One round of 192 x 128 tiles (200 to 256 of them) with K >= 2048 takes the pipelined
    one-workgroup-per-CU k-loop: Wo2 of a 10-question request (5686 x 1024 x 2624) and a shorter
    M ending on a partial row tile. f32, bf16 and residual outputs against a float32 product."""
    N, K = 1024, 2624
    say(f"long-K gemm M={M}")
    g = torch.Generator(device="cpu").manual_seed(M)
    A = bf16_bits(torch.randn(M, K, generator=g)).to(dev)
    W = bf16_bits(torch.randn(N, K, generator=g) * 0.02).to(dev)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    ref = as_f32(A) @ as_f32(W).T
    scale = float(ref.abs().max())
    out = gemm(A, W, M, N, K, epi=3)
    assert float((out - ref).abs().max()) <= 2e-5 * scale + 1e-6
    ob = as_f32(gemm(A, W, M, N, K, epi=0))
    assert bool(((ob - ref).abs() <= ref.abs() * 2 ** -8 + 1e-5 * scale).all())
    h0 = torch.randn(M, N, generator=g).to(dev)
    h = h0.clone()
    gemm(A, W, M, N, K, epi=1, bias=bias, C_out=h)
    assert float((h - (h0 + ref + bias)).abs().max()) <= 2e-5 * scale + 1e-5


def test_gemm_a_spanning_4_gib_runs_as_row_pieces(dev):
    """The GEMM's direct loads address A by 32-bit byte offsets from its start, so an A that
    spans 4 GiB or more ((M - 1) lda + K 16-bit elements) runs as row pieces, each a launch of
    its own. Here A's rows are 2 MiB apart (lda = 2^20), so 2100 rows span 4.4 GB and run as
    pieces of 1152 and 948 rows; every epilogue must give the bits of the same product over a
    contiguous A (lda = K), whose single launch takes the same tile configuration and k order."""
    M, N, K, lda = 2100, 256, 256, 1 << 20
    assert ((M - 1) * lda + K) * 2 >= 1 << 32
    say(f"gemm over a 4 GiB A: M={M} N={N} K={K} lda={lda}")
    L = _lib()
    g = torch.Generator(device="cpu").manual_seed(11)
    A = bf16_bits(torch.randn(M, K, generator=g)).to(dev)
    W = bf16_bits(torch.randn(N, K, generator=g) * 0.05).to(dev)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    big = torch.empty(M, lda, dtype=torch.int16, device=dev)  # 4.4 GB; only the first K columns are read
    big[:, :K] = A
    h0 = torch.randn(M, N, generator=g).to(dev)
    for epi, act, b in [(0, 2, bias), (1, 0, bias), (2, 0, None), (3, 0, bias)]:
        outs = []
        for src, ld in [(A, K), (big, lda)]:
            if epi == 1:
                out = h0.clone()
            elif epi == 3:
                out = torch.zeros(M, N, dtype=torch.float32, device=dev)
            else:
                out = torch.zeros(M, N // 2 if epi == 2 else N, dtype=torch.int16, device=dev)
            L.check(L.lib().s1k_gemm(ptr(src), ld, ptr(W), K, ptr(out), out.shape[1], ptr(b) if b is not None else None,
                                     M, N, K, epi, act, stream()))
            torch.cuda.synchronize()
            outs.append(out)
        say(f"  epi={epi}: bit-identical {torch.equal(outs[0], outs[1])}")
        assert torch.equal(outs[0], outs[1]), epi
    ref = as_f32(A) @ as_f32(W).T + bias
    assert float((outs[1] - ref).abs().max()) <= 2e-5 * float(ref.abs().max()) + 1e-5
    del big
    torch.cuda.empty_cache()


def test_split_k_back_to_back_shapes(dev):
    """Split-K launches of other shapes and split counts in a row, each reusing the workspace
    the previous one left: every result is complete and repeats bit for bit."""
    g = torch.Generator(device="cpu").manual_seed(77)
    cases = [(170, 1024, 2624), (170, 3072, 1024), (170, 1024, 2624), (64, 1024, 1024), (170, 1024, 2624)]
    for M, N, K in cases:
        say(f"split-K M={M} N={N} K={K}")
        A = bf16_bits(torch.randn(M, K, generator=g)).to(dev)
        W = bf16_bits(torch.randn(N, K, generator=g) * 0.02).to(dev)
        ref = as_f32(A) @ as_f32(W).T
        out = gemm(A, W, M, N, K, epi=3)
        scale = float(ref.abs().max())
        assert float((out - ref).abs().max()) <= 2e-5 * scale + 1e-6
        again = gemm(A, W, M, N, K, epi=3)
        assert torch.equal(out, again)  # partials summed in split order


@pytest.mark.parametrize("M", [170, 512, 2048, 4100])  # 170: split-K, including the transposed v blocks; 4100: wide
@pytest.mark.parametrize("theta", [160000.0, 10000.0])
def test_fused_wqkv_split_rope(dev, theta, M):
    """Isolated fused Wqkv GEMM + split + RoPE at M=512 (and 2048, the whole-K path), K=1024,
    N=3072, A ~ N(0,1), W ~ N(0,0.02), positions 0..M-1."""
    say(f"qkv_rope theta={theta} M={M}")
    d = 1024
    g = torch.Generator(device="cpu").manual_seed(int(theta) % 97)
    A = bf16_bits(torch.randn(M, d, generator=g)).to(dev)
    W = bf16_bits(torch.randn(3 * d, d, generator=g) * 0.02).to(dev)
    pos = torch.arange(M, dtype=torch.int32, device=dev)
    L = _lib()
    ldv = L.vt_ld(M)
    q, k = (torch.zeros(16, M, 64, dtype=torch.int16, device=dev) for _ in range(2))
    vt = torch.full((16, 64, ldv), -1, dtype=torch.int16, device=dev)
    L.check(L.lib().s1k_qkv_rope(ptr(A), ptr(W), M, d, ptr(pos), theta, ptr(q), ptr(k), ptr(vt), ldv, stream()))
    torch.cuda.synchronize()
    m8 = (M + 7) // 8 * 8  # v columns [M, m8) are written as zeros, the rest of the slack is not written
    assert bool((vt[:, :, M:m8] == 0).all()) and bool((vt[:, :, m8:] == -1).all())
    v = vt[:, :, :M].transpose(1, 2)  # v is written transposed, [H, 64, ldv]
    qkv = (as_f32(A) @ as_f32(W).T).cpu().numpy()
    cos, sin = O.rope_tables(theta, M, 64)
    want = []
    for part in range(3):
        x = qkv[:, part * d:(part + 1) * d].reshape(M, 16, 64).transpose(1, 0, 2)
        want.append(O.rope(x, cos, sin) if part < 2 else x)
    for got, ref in zip((q, k, v), want):
        g_ = as_f32(got).cpu().numpy()
        err = np.abs(g_ - ref)
        assert np.all(err <= np.abs(ref) * 2 ** -8 + 2e-4), float(err.max())


@pytest.mark.parametrize("M", [700, 5, 64])
@pytest.mark.parametrize("theta", [160000.0, 10000.0, 0.0])
def test_split_rope_pass(dev, theta, M):
    say(f"split_rope theta={theta} M={M}")
    d = 1024
    g = torch.Generator(device="cpu").manual_seed(3)
    qkv = bf16_bits(torch.randn(M, 3 * d, generator=g)).to(dev)
    pos = torch.arange(M, dtype=torch.int32, device=dev) * 11  # positions up to 7689
    L = _lib()
    ldv = L.vt_ld(M)
    q, k = (torch.zeros(16, M, 64, dtype=torch.int16, device=dev) for _ in range(2))
    vt = torch.full((16, 64, ldv), -1, dtype=torch.int16, device=dev)
    L.check(L.lib().s1k_split_rope(ptr(qkv), M, d, ptr(pos), theta, ptr(q), ptr(k), ptr(vt), ldv, stream()))
    torch.cuda.synchronize()
    m8 = (M + 7) // 8 * 8  # v columns [M, m8) are written as zeros, the rest of the slack is not written
    assert bool((vt[:, :, M:m8] == 0).all()) and bool((vt[:, :, m8:] == -1).all())
    v = vt[:, :, :M].transpose(1, 2)
    x = as_f32(qkv).cpu().numpy()
    p = pos.cpu().numpy()
    for part, got in enumerate((q, k, v)):
        ref = x[:, part * d:(part + 1) * d].reshape(M, 16, 64).transpose(1, 0, 2)
        if part < 2 and theta > 0:
            cos, sin = O.rope_tables(theta, int(p.max()) + 1, 64)
            c, s = cos[p], sin[p]
            ref = np.concatenate([ref[..., :32] * c - ref[..., 32:] * s, ref[..., :32] * s + ref[..., 32:] * c], -1)
        g_ = as_f32(got).cpu().numpy()
        if part == 2 or theta == 0:
            assert np.array_equal(g_, ref)  # an exact copy
        else:
            assert np.all(np.abs(g_ - ref) <= np.abs(ref) * 2 ** -8 + 1e-6)


def attention_ref(q, k, v, starts, window, scale):
    """float32 per-row softmax(q k^T scale) v with the row and window masks."""
    H, T, _ = q.shape
    out = torch.zeros(T, H * 64, dtype=torch.float32)
    for r in range(len(starts) - 1):
        a, b = starts[r], starts[r + 1]
        qq, kk, vv = q[:, a:b], k[:, a:b], v[:, a:b]
        s = (qq @ kk.transpose(1, 2)) * scale
        if window >= 0:
            i = torch.arange(b - a)
            s = s.masked_fill((i[:, None] - i[None, :]).abs() > window, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out[a:b] = (p @ vv).transpose(0, 1).reshape(b - a, H * 64)
    return out


# window 64 and 16 take the staged local kernel ([2048], 24 rows of 600, and the 28 mixed rows
# of 1 to 600 tokens, whose tiles include one-token rows and waves past their tile's queries) or,
# for the shorter batches, 32-query tiles of the window range with the keys split over 4 waves;
# 100 takes the chunked one; -1 the global one, whose tiles hold 32 queries with the keys split
# over 4 waves ([8, 200], [700, 1], [513]), 128 (the other short batches) or 256 (24 rows of 600)
@pytest.mark.parametrize("window", [-1, 64, 16, 100])
@pytest.mark.parametrize("lens", [[1, 37, 129, 300, 600], [8, 200], [700, 1], [513], [2048], [5, 3, 250, 1, 700, 9],
                                  [600] * 24, [1, 2, 130, 7, 64, 600, 3] * 4])
def test_attention_varlen(dev, window, lens):
    say(f"attention window={window} lens={lens}")
    H = 16
    starts = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(starts[-1])
    g = torch.Generator(device="cpu").manual_seed(T + window)
    q, k, v = (torch.randn(H, T, 64, generator=g) for _ in range(3))
    qb, kb, vb = (bf16_bits(x).to(dev) for x in (q, k, v))
    L = _lib()
    ldv = L.vt_ld(T)
    # v transposed, [H, 64, ldv]: columns [T, T rounded up to 8) hold zeros, as every v writer
    # leaves them; the slack past that holds NaN bits, which must never reach the output
    vt = torch.full((H, 64, ldv), -1, dtype=torch.int16, device=dev)
    vt[:, :, :T] = vb.transpose(1, 2)
    vt[:, :, T:(T + 7) // 8 * 8] = 0
    out = torch.zeros(T, H * 64, dtype=torch.int16, device=dev)
    st = np.ascontiguousarray(starts)
    L.check(L.lib().s1k_attention(ptr(qb), ptr(kb), ptr(vt), ldv, T, H, st.ctypes.data_as(L.i32p), len(lens),
                                  window, 0.125, ptr(out), stream()))
    torch.cuda.synchronize()
    ref = attention_ref(as_f32(qb.cpu()), as_f32(kb.cpu()), as_f32(vb.cpu()), starts.tolist(), window, 0.125)
    got = as_f32(out.cpu())
    # P is rounded to bf16 before the PV product: allow ~2^-8 relative on each term
    err = (got - ref).abs()
    assert float(err.max()) <= 2e-2, float(err.max())
    assert float(err.mean()) <= 2e-3, float(err.mean())


def test_layernorm(dev):
    say("layernorm")
    M, d = 333, 1024
    g = torch.Generator(device="cpu").manual_seed(9)
    x = (torch.randn(M, d, generator=g) * 3 + 0.5).to(dev)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    b = (0.1 * torch.randn(d, generator=g)).to(dev)
    y = torch.zeros(M, d, dtype=torch.int16, device=dev)
    L = _lib()
    L.check(L.lib().s1k_layernorm(ptr(x), ptr(w), ptr(b), 1e-5, M, d, ptr(y), stream()))
    torch.cuda.synchronize()
    ref = O.layer_norm(x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy(), 1e-5)
    got = as_f32(y).cpu().numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -8 + 1e-5)
