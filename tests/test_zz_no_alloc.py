"""s1k_gemm_noalloc, the allocation-free variant of s1k_gemm, through the C ABI: the same bits as
the allocating entry point on shapes that split K (so the static scratch holds the partials),
on two calls in a row, the second with a smaller input, for each epilogue."""
from __future__ import annotations

import ctypes as C

import pytest

from sys1rust_amd import _lib

pytestmark = pytest.mark.gpu


def _run(fn, A, W, Cout, bias, M, N, K, epi, act):
    import torch

    st = torch.cuda.current_stream().cuda_stream
    rc = fn(C.c_void_p(A.data_ptr()), K, C.c_void_p(W.data_ptr()), K, C.c_void_p(Cout.data_ptr()),
            Cout.shape[1], C.c_void_p(bias.data_ptr() if bias is not None else 0), M, N, K, epi, act, C.c_void_p(st))
    _lib.check(rc)
    torch.cuda.synchronize()


@pytest.mark.parametrize("epi,act,bias", [(0, 0, False), (0, 2, True), (1, 0, True), (3, 0, False)])
def test_noalloc_gemm_matches_allocating_gemm(epi, act, bias):
    import torch

    L = _lib.lib()
    g = torch.Generator(device="cuda").manual_seed(7 + epi)
    # Both shapes split K (few output tiles): 4 splits, then 10 splits of a smaller product.
    for M, N, K in [(128, 1024, 1024), (40, 512, 2624)]:
        print(f"noalloc: epi={epi} act={act} bias={bias} M={M} N={N} K={K}", flush=True)
        A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        W = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(torch.bfloat16)
        bv = torch.randn(N, device="cuda", generator=g) if bias else None
        f32 = epi in (1, 3)
        base = torch.randn(M, N, device="cuda", generator=g) if epi == 1 else torch.zeros(M, N, device="cuda")
        c1 = base.clone() if f32 else torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
        c2 = base.clone() if f32 else torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
        _run(L.s1k_gemm, A, W, c1, bv, M, N, K, epi, act)
        _run(L.s1k_gemm_noalloc, A, W, c2, bv, M, N, K, epi, act)
        assert torch.equal(c1.view(torch.int16) if not f32 else c1.view(torch.int32),
                           c2.view(torch.int16) if not f32 else c2.view(torch.int32)), (M, N, K)
        # and against a float32 reference of the same product, to the bf16 output's precision
        ref = A.float() @ W.float().T + (bv if bias else 0)
        if act == 2:
            ref = torch.nn.functional.gelu(ref)
        if epi == 1:
            ref = ref + base
        err = (c2.float() - ref).abs().max().item()
        assert err <= 2e-2 * max(1.0, ref.abs().max().item()), err


def test_noalloc_gemm_under_graph_capture():
    """The captured call replays the eager call's bits: a split-K product (its partials in the
    static scratch) captured in a graph after one eager call on the GPU, replayed several times
    with eager work and new inputs between the replays, each replay checked against s1k_gemm."""
    import torch

    L = _lib.lib()
    g = torch.Generator(device="cuda").manual_seed(11)
    M, N, K = 128, 1024, 1024
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    W = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(torch.bfloat16)
    bias = torch.randn(N, device="cuda", generator=g)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    want = torch.zeros_like(out)

    def call(fn, C_, st):
        return fn(C.c_void_p(A.data_ptr()), K, C.c_void_p(W.data_ptr()), K, C.c_void_p(C_.data_ptr()), N,
                  C.c_void_p(bias.data_ptr()), M, N, K, 0, 2, C.c_void_p(st))

    _run(L.s1k_gemm_noalloc, A, W, out, bias, M, N, K, 0, 2)  # first call on this GPU: outside capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call(L.s1k_gemm_noalloc, out, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    for i in range(4):
        print(f"noalloc graph: replay {i}", flush=True)
        out.zero_()
        if i:
            A.copy_(torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _run(L.s1k_gemm, A, W, want, bias, M, N, K, 0, 2)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), i
