"""GEMM timing at the 10-question request's shapes (M = 5686 tokens of the ModernBERT-large
encoder): s1k_gemm of one or more builds of libsys1hip.so, and hipBLASLt through torch.matmul for
comparison (bf16 out, no epilogue).

Shapes (N, K, epilogue): wqkv 3072 x 1024 bf16 out; wo 1024 x 1024 and wo2 1024 x 2624 with the
f32 residual add (epi 1), or f32 stores only (`*_f32`, epi 3), or bf16 stores (`*_bf16`, epi 0);
wi 5248 x 1024 with the GeGLU epilogue (epi 2). The weights rotate over copies filling 600 MB, so
every launch reads them cold from HBM as the model's per-layer weights are. Each build is timed
over `--reps` launches with HIP events, in `--rounds` rounds whose order alternates between the
builds; the median round is reported. `--check` compares every build's output with the first's.

Run on the GPU host from the repo root:
  python3 sys1rust_amd/microbench/gemm_shapes.py sys1rust_amd/libsys1hip.so --blas
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from sys1rust_amd._lib import SIGNATURES  # noqa: E402

SHAPES = {"wqkv": (3072, 1024, 0), "wo": (1024, 1024, 1), "wi": (5248, 1024, 2), "wo2": (1024, 2624, 1),
          "wo_f32": (1024, 1024, 3), "wo_bf16": (1024, 1024, 0), "wo2_f32": (1024, 2624, 3),
          "wo2_bf16": (1024, 2624, 0)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("libs", nargs="+", help="builds of libsys1hip.so to time")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--rounds", type=int, default=4)
    ap.add_argument("--blas", action="store_true", help="also time torch.matmul (hipBLASLt)")
    ap.add_argument("--M", type=int, default=5686)
    ap.add_argument("--shapes", default="wqkv,wo,wi,wo2")
    ap.add_argument("--check", action="store_true")
    a = ap.parse_args()
    assert torch.cuda.is_available(), "needs a GPU"

    libs = []
    for p in a.libs:
        lib = C.CDLL(os.path.abspath(p))
        lib.s1k_gemm.restype, lib.s1k_gemm.argtypes = SIGNATURES["s1k_gemm"]
        lib.s1_last_error.restype = C.c_char_p
        libs.append((p, lib))
    dev = torch.device("cuda:0")
    M = a.M
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for name in a.shapes.split(","):
        N, K, epi = SHAPES[name]
        A = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        ncopy = max(2, int(600e6 // (N * K * 2)))
        Ws = [(torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(ncopy)]
        if epi == 2:
            out = torch.empty(M, N // 2, device=dev, dtype=torch.bfloat16)
        elif epi in (1, 3):
            out = torch.zeros(M, N, device=dev, dtype=torch.float32)
        else:
            out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        ldc = out.shape[1]
        # The output buffer holds exactly what the epilogue writes: M rows of ldc elements of its type.
        assert out.numel() * out.element_size() == M * ldc * (4 if epi in (1, 3) else 2)
        flop = 2.0 * M * N * K
        times, outs = {}, {}
        for r in range(a.rounds):
            for p, lib in (libs if r % 2 == 0 else libs[::-1]):
                def run(i, lib=lib):
                    rc = lib.s1k_gemm(C.c_void_p(A.data_ptr()), K, C.c_void_p(Ws[i % ncopy].data_ptr()), K,
                                      C.c_void_p(out.data_ptr()), ldc, None, M, N, K, epi, 0, stream)
                    if rc:
                        raise RuntimeError(lib.s1_last_error().decode())
                for i in range(3):
                    run(i)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for i in range(a.reps):
                    run(i)
                e1.record()
                torch.cuda.synchronize()
                times.setdefault(p, []).append(e0.elapsed_time(e1) * 1e3 / a.reps)
                if a.check and r == 0:
                    if epi == 1:
                        out.zero_()
                    run(0)
                    torch.cuda.synchronize()
                    outs[p] = out.clone()
            if a.blas:
                for i in range(3):
                    torch.matmul(A, Ws[i % ncopy].t())
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for i in range(a.reps):
                    torch.matmul(A, Ws[i % ncopy].t())
                e1.record()
                torch.cuda.synchronize()
                times.setdefault("hipblaslt", []).append(e0.elapsed_time(e1) * 1e3 / a.reps)
        for p, v in times.items():
            v = sorted(v)
            med = v[len(v) // 2]
            print(f"{name:8s} {p}: median {med:.2f} µs, min {v[0]:.2f}, {flop / med / 1e6:.1f} TFLOP/s", flush=True)
        if a.check and len(outs) > 1:
            first = next(iter(outs))
            for p in list(outs)[1:]:
                print(f"  {p} against {first}: bit-identical {torch.equal(outs[p], outs[first])}, max |diff| "
                      f"{(outs[p].float() - outs[first].float()).abs().max().item():.3e}", flush=True)
        del A, Ws, out
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
