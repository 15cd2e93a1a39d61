"""qlin_run_noalloc (the entry point that allocates nothing, scratch in a static device
array) against the existing entry points through the C ABI: bit for bit equal to
qlin_run / qlin_run_rmsnorm on two calls in a row, the second with a smaller input, on
the decode GEMV (fused and separate quantization) and the prefill GEMM (with split-K),
W4 and W8, SiLU-gate and RMSNorm; sizes beyond its limits are refused."""
import ctypes

import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import _lib
from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run_noalloc(w, A, flags=0, gamma=None, eps=1e-6, out_dtype=torch.float16, err=None):
    M = A.shape[0]
    ncols = w.N // 2 if flags & ql.QLIN_SWIGLU else w.N
    out = torch.full((M, ncols), float("nan"), dtype=out_dtype, device=A.device)
    rc = _lib.load().qlin_run_noalloc(w.handle, M, ql._ptr(A), ql._DT[A.dtype], A.stride(0),
                                      ql._ptr(gamma) if gamma is not None else None, eps, ql._ptr(out),
                                      ql._DT[out_dtype], out.stride(0), flags,
                                      ql._ptr(err) if err is not None else None, ql._stream())
    return rc, out


def weights(bits, K, N, seed):
    packed, _, sc = synth.make_linear(N, K, bits, seed, device=DEV)
    return ql.Weights.from_packed_device(bits, K, N, packed, sc)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N,swiglu,norm,rows", [
    (2560, 19456, True, True, (4, 1)),      # decode GEMV, RMSNorm fused, then one row
    (4096, 2560, False, False, (16, 3)),    # GEMV on separately quantized rows, then fused
    (9728, 2560, False, False, (512, 200)),  # GEMM with split-K, then a smaller GEMM
    (2560, 6144, False, True, (1024, 17)),  # GEMM after RMSNorm-quantize
    (2560, 2000, True, False, (300, 2)),    # SiLU-gate at N % 64 != 0
    (2560, 6144, False, False, (8, 5)),     # 5..8-row fused decode GEMV
    (4096, 2560, False, False, (24, 20)),   # 17..32 quantized rows: the GEMV's two row blocks
])
def test_noalloc_matches_workspace_entry(bits, K, N, swiglu, norm, rows):
    w = weights(bits, K, N, 800 + K % 97 + N % 89 + bits)
    ws = ql.Workspace(max(rows), K, N)
    gamma = synth.gamma(K, seed=801, device=DEV) if norm else None
    flags = ql.QLIN_SWIGLU if swiglu else 0
    for M in rows:
        A = synth.activations(M, K, seed=802 + M, device=DEV)
        print(f"[noalloc] bits={bits} K={K} N={N} M={M}", flush=True)
        ref = ql.run(ws, w, A, flags=flags, gamma=gamma, eps=1e-6)
        rc, out = run_noalloc(w, A, flags, gamma)
        torch.cuda.synchronize()
        assert rc == 0, _lib.strerror(rc)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (M, (out != ref).sum().item())
    ws.close()
    w.close()


@pytest.mark.parametrize("bits,K,N,swiglu,norm,M", [
    (4, 2560, 19456, True, True, 1),     # fused decode GEMV with RMSNorm and SiLU-gate
    (8, 9728, 2560, False, False, 512),  # prefill GEMM with split-K (counters reused per replay)
])
def test_noalloc_under_graph_capture(bits, K, N, swiglu, norm, M):
    """qlin_run_noalloc captured in a HIP graph (the callers it is for), replayed with a
    new input each time and eager workspace runs between the replays: every replay equals
    qlin_run bit for bit."""
    w = weights(bits, K, N, 820 + bits)
    ws = ql.Workspace(M, K, N)
    gamma = synth.gamma(K, seed=821, device=DEV) if norm else None
    flags = ql.QLIN_SWIGLU if swiglu else 0
    ncols = N // 2 if swiglu else N
    A = synth.activations(M, K, seed=822, device=DEV)
    out = torch.empty((M, ncols), dtype=torch.float16, device=DEV)
    lib = _lib.load()

    def call():
        return lib.qlin_run_noalloc(w.handle, M, ql._ptr(A), ql.QLIN_F16, A.stride(0),
                                    ql._ptr(gamma) if gamma is not None else None, 1e-6, ql._ptr(out), ql.QLIN_F16,
                                    out.stride(0), flags, None, ql._stream())

    assert call() == 0  # eager first: code objects load outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = call()
    assert rc == 0
    for rep in range(4):
        print(f"[noalloc graph] bits={bits} K={K} N={N} M={M} replay {rep}", flush=True)
        A.copy_(synth.activations(M, K, seed=823 + rep, device=DEV))
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = ql.run(ws, w, A, flags=flags, gamma=gamma, eps=1e-6)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (rep, (got != ref).sum().item())
    del g
    ws.close()
    w.close()


def test_noalloc_error_word_and_limits():
    w = weights(4, 2560, 1024, 810)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    A = synth.activations(2, 2560, seed=811, device=DEV)
    A[1, 7] = float("inf")
    rc, _ = run_noalloc(w, A, err=err)
    torch.cuda.synchronize()
    assert rc == 0 and int(err.item()) & 1
    err.zero_()
    rc, _ = run_noalloc(w, A[:1].contiguous(), err=err)
    torch.cuda.synchronize()
    assert rc == 0 and int(err.item()) == 0
    # more rows than the static scratch holds: refused before any launch
    big = torch.zeros((4097, 2560), dtype=torch.float16, device=DEV)
    rc, _ = run_noalloc(w, big)
    assert rc == _lib.QLIN_ERR_UNSUPPORTED
    rc = _lib.load().qlin_run_noalloc(None, 1, None, 1, 8, None, 0.0, None, 1, 8, 0, None, None)
    assert rc == _lib.QLIN_ERR_PARAM
    w.close()
