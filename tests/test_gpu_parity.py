"""Parity of the HIP path against the CPU oracle, through the C ABI.

Bar: int8 q, f32 s and int32 acc bit-exact; f32 and fp16 outputs of the plain
linear bit-exact (both sides perform the same singly-rounded f32 operations and
round to fp16 to nearest even); SwiGLU outputs within 1e-3 relative for fp16
(|a-e| <= 1e-3 * max(|e|, 1), the reference's compare form) and the reference's
3e-5 for f32, since exp() differs between libm and the device.
"""
import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from tests import refcases

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
F16_TOL = 1e-3
SWIGLU_F32_TOL = 3e-5


def roundup(x, a):
    return (x + a - 1) // a * a


def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make_weights(bits, codes_nk: np.ndarray, scales: np.ndarray):
    codes_kn = np.ascontiguousarray(codes_nk.T)
    return ql.Weights.from_codes_kn(bits, codes_kn, scales)


@pytest.fixture(scope="module")
def ws():
    w = ql.Workspace(4096, 9728, 19456)
    yield w
    w.close()


# ------------------------------------------------------------------ quantize


def tie_rows(K):
    """Rows whose x*(1/s) land exactly on k + 0.5 (s = 1 when absmax = 127)."""
    A = np.zeros((3, K), np.float32)
    A[0, 0] = 127
    A[0, 1:] = (np.arange(K - 1) % 100).astype(np.float32) + 0.5
    A[0, 1:] *= np.where(np.arange(K - 1) % 2, -1, 1)
    A[1, :] = 0  # zero row -> s = 1
    A[2, 0] = 6.0e-8  # fp16 subnormal only
    return A


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 2560), (3, 100), (7, 9728), (64, 4096), (5, 13), (2, 256)])
@pytest.mark.parametrize("rne", [False, True])
def test_quantize_bitexact(oracle, dtype, M, K, rne):
    g = torch.Generator().manual_seed(M * 1000 + K)
    A = torch.randn((M, K), generator=g) * torch.tensor([10.0 ** (i % 5 - 2) for i in range(M)])[:, None]
    A[:, ::37] *= 20
    if K >= 3:
        A = torch.cat([A, torch.from_numpy(tie_rows(K))], 0)
    A = A.to(dtype)
    Ad = A.to(DEV)
    ldq = roundup(K, 256)
    q, s = ql.quantize(Ad, ldq=ldq, flags=ql.QLIN_ROUND_HALF_EVEN if rne else 0)
    torch.cuda.synchronize()
    qo, so, bad = oracle.quantize(A.float().numpy(), oracle.ROUND_EVEN if rne else oracle.ROUND_AWAY)
    assert bad == 0
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    qn = q.cpu().numpy()
    assert np.array_equal(qn[:, :K], qo)
    assert not qn[:, K:].any()


def test_quantize_nonfinite_flag(oracle):
    A = torch.randn((4, 512), dtype=torch.float32)
    A[1, 7] = float("nan")
    A[3, 0] = float("inf")
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    q, s = ql.quantize(A.to(DEV), ldq=512, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    qo, so, bad = oracle.quantize(A.numpy())
    assert bad == 2
    assert np.array_equal(q.cpu().numpy(), qo)  # same NaN -> 0, s = inf handling
    err.zero_()
    ql.quantize(torch.randn((4, 512), device=DEV), ldq=512, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0


@pytest.mark.parametrize("order", ["neon16", "seq"])
@pytest.mark.parametrize("M,K", [(1, 2560), (5, 100), (3, 9728), (33, 4096)])
def test_rmsnorm_quantize_bitexact(oracle, order, M, K):
    x = synth.activations(M, K, seed=K + M, device="cpu", dist="student_t3")
    gam = synth.gamma(K, seed=K, device="cpu")
    flags = ql.QLIN_NORM_SEQUENTIAL if order == "seq" else 0
    q, s = ql.quantize(x.to(DEV), ldq=roundup(K, 256), gamma=gam.to(DEV), eps=1e-6, flags=flags)
    torch.cuda.synchronize()
    y = oracle.rmsnorm(x.float().numpy(), gam.numpy(), 1e-6, order)
    qo, so, _ = oracle.quantize(y)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(q.cpu().numpy()[:, :K], qo)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("order", ["neon16", "seq"])
@pytest.mark.parametrize("M,K", [(1027, 2560), (1030, 104), (1025, 9728)])
def test_rmsnorm_quantize_many_rows(oracle, dtype, order, M, K):
    """Many rows take one wave per row: rows and RMSNorm weights in registers (fp16 rows up to
    K = 4096, the chain-major sum for K % 512 == 0 in the chain order; f32 rows up to K = 2048),
    else the staged kernel (64-thread workgroups)."""
    x = synth.activations(M, K, seed=K + M, device="cpu", dist="student_t3").to(dtype)
    gam = synth.gamma(K, seed=K, device="cpu")
    flags = ql.QLIN_NORM_SEQUENTIAL if order == "seq" else 0
    ldq = roundup(K, 256)
    q, s = ql.quantize(x.to(DEV), ldq=ldq, gamma=gam.to(DEV), eps=1e-6, flags=flags)
    torch.cuda.synchronize()
    y = oracle.rmsnorm(x.float().numpy(), gam.numpy(), 1e-6, order)
    qo, so, _ = oracle.quantize(y)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, :K], qo)
    assert not qh[:, K:].any()  # the zero tail up to ldq


# every register-resident instance of the one-wave-per-row RMSNorm kernel: chunks of 16
# bytes per lane NC = 2, 4, 5, 8 for fp16 (chain-major sum when K % 512 == 0 in the chain
# order, row-major otherwise) and f32 rows
@pytest.mark.parametrize("order", ["neon16", "seq"])
@pytest.mark.parametrize("dtype,K", [
    (torch.float16, 1024),  # NC 2, chain-major
    (torch.float16, 1536),  # NC 3 -> 4, chain-major
    (torch.float16, 2000),  # NC 4, row-major (K % 512 != 0)
    (torch.float16, 4096),  # NC 8, chain-major
    (torch.float32, 1024),  # NC 4
    (torch.float32, 1280),  # NC 5
    (torch.float32, 2048),  # NC 8
])
def test_rmsnorm_quantize_many_rows_register_paths(oracle, order, dtype, K):
    M = 1024
    x = synth.activations(M, K, seed=K + 3, device="cpu", dist="student_t3").to(dtype)
    gam = synth.gamma(K, seed=K + 1, device="cpu")
    flags = ql.QLIN_NORM_SEQUENTIAL if order == "seq" else 0
    ldq = roundup(K, 256)
    q, s = ql.quantize(x.to(DEV), ldq=ldq, gamma=gam.to(DEV), eps=1e-6, flags=flags)
    torch.cuda.synchronize()
    y = oracle.rmsnorm(x.float().numpy(), gam.numpy(), 1e-6, order)
    qo, so, _ = oracle.quantize(y)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, :K], qo)
    assert not qh[:, K:].any()


@pytest.mark.parametrize("dtype,K", [(torch.float16, 2560), (torch.float16, 104), (torch.float32, 2560)])
def test_rmsnorm_quantize_many_rows_nonfinite(oracle, dtype, K):
    """Rows holding NaN, Inf or -Inf among 1030 RMSNorm rows (fp16 K = 2560: the chain-major
    sum; K = 104: the row-major sum; f32 K = 2560: the staged kernel): the error word is set,
    the oracle counts three bad rows, every row's codes equal the oracle's and the finite rows'
    scales do too."""
    M = 1030
    x = synth.activations(M, K, seed=K + 7, device="cpu", dist="student_t3").to(dtype)
    x[3, 5] = float("nan")
    x[700, K - 1] = float("inf")
    x[M - 1, 0] = float("-inf")
    gam = synth.gamma(K, seed=K, device="cpu")
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    ldq = roundup(K, 256)
    q, s = ql.quantize(x.to(DEV), ldq=ldq, gamma=gam.to(DEV), eps=1e-6, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    y = oracle.rmsnorm(x.float().numpy(), gam.numpy(), 1e-6, "neon16")
    qo, so, bad = oracle.quantize(y)
    assert bad == 3
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, :K], qo)
    assert not qh[:, K:].any()
    finite = np.ones(M, dtype=bool)
    finite[[3, 700, M - 1]] = False
    assert np.array_equal(s.cpu().numpy().view(np.uint32)[finite], so.view(np.uint32)[finite])


# ------------------------------------------------------------------ integer accumulators


GEMM_SHAPES = [(256, 256), (2560, 64), (4096, 2560), (9728, 2560), (2560, 6144), (300, 200)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N", GEMM_SHAPES)
def test_acc_bitexact(oracle, ws, bits, K, N):
    seed = bits * 7 + K + N
    codes = synth.codes(N, K, bits, seed).numpy()
    sc = synth.scales(N, bits, seed).numpy()
    w = make_weights(bits, codes, sc)
    rows_list = [1, 2, 5, 16, 17, 129] if K * N <= 2560 * 6144 else [1, 16, 300]
    for M in rows_list:
        q = torch.randint(-127, 128, (M, w.K_padded), dtype=torch.int8)
        q[:, K:] = 0
        acc = ql.gemm_i32(ws, w, q.to(DEV))
        torch.cuda.synchronize()
        expect = oracle.gemm_i32_nk(q[:, :K].numpy(), codes)
        got = acc.cpu().numpy()
        assert np.array_equal(got, expect), f"bits={bits} K={K} N={N} M={M}: {np.argwhere(got != expect)[:4]}"
    w.close()


# ------------------------------------------------------------------ full linear


def oracle_linear(oracle, A16: torch.Tensor, codes_nk, sc, swiglu, gamma=None, round_mode=0):
    """f32 outputs of the oracle from fp16 activations (optionally RMSNorm first)."""
    x = A16.float().numpy()
    if gamma is not None:
        x = oracle.rmsnorm(x, gamma, 1e-6, "neon16")
    q, s, _ = oracle.quantize(x, round_mode)
    acc = oracle.gemm_i32_nk(q, codes_nk)
    out = oracle.dequant(acc, s, sc)
    return oracle.swiglu(out) if swiglu else out


def compare_f16_tol(oracle, got_f32, expect_f32, tol):
    """fp16 results within tol; values beyond the fp16 range must be inf of the same sign."""
    exp16 = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(expect_f32))
    big = np.abs(expect_f32) > 65504.0 * (1 + tol)
    small = np.abs(expect_f32) < 65504.0 * (1 - tol)
    assert np.array_equal(got_f32[big], exp16[big])
    refcases.compare(got_f32[small], expect_f32[small], tol)


def check_outputs(oracle, out_dev, expect_f32, swiglu, dtype):
    got = out_dev.cpu()
    if dtype == torch.float32:
        if swiglu:
            refcases.compare(got.numpy(), expect_f32, SWIGLU_F32_TOL)
        else:
            assert np.array_equal(got.numpy().view(np.uint32), expect_f32.view(np.uint32))
    else:
        if swiglu:
            compare_f16_tol(oracle, got.float().numpy(), expect_f32, F16_TOL)
        else:
            g16, e16 = f16_bits(got), oracle.f32_to_f16_bits(expect_f32)
            bad = np.argwhere(g16 != e16)
            assert len(bad) == 0, f"{len(bad)} fp16 mismatches, first {bad[:3].tolist()}"



@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16, 17, 64, 512])
@pytest.mark.parametrize("swiglu", [False, True])
def test_linear_small_shapes(oracle, ws, bits, M, swiglu):
    K, N = 2560, 1024
    codes = synth.codes(N, K, bits, 5 + bits).numpy()
    sc = synth.scales(N, bits, 6 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=M)
    expect = oracle_linear(oracle, A, codes, sc, swiglu)
    flags = ql.QLIN_SWIGLU if swiglu else 0
    for extra in (0, ql.QLIN_NO_FUSED_QUANT):
        for dtype in (torch.float16, torch.float32):
            out = ql.run(ws, w, A.to(DEV), out_dtype=dtype, flags=flags | extra)
            torch.cuda.synchronize()
            check_outputs(oracle, out, expect, swiglu, dtype)
    # f32 activations take the same path
    out = ql.run(ws, w, A.float().to(DEV), out_dtype=torch.float32, flags=flags)
    torch.cuda.synchronize()
    check_outputs(oracle, out, expect, swiglu, torch.float32)
    w.close()


@pytest.mark.parametrize("M", [1, 4, 512])
def test_qwen3_layer(oracle, ws, M):
    """The four Qwen3-4B projections (W4) at decode and prefill sizes."""
    for p, (name, K, N) in enumerate(synth.LAYER):
        seed = synth.linear_seed(0, p)
        packed, codes, sc = synth.make_linear(N, K, 4, seed)
        w = make_weights(4, codes.numpy(), sc.numpy())
        A = synth.activations(M, K, seed=seed + 1)
        swiglu = name == "gate_up"
        out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU if swiglu else 0)
        torch.cuda.synchronize()
        expect = oracle_linear(oracle, A, codes.numpy(), sc.numpy(), swiglu)
        check_outputs(oracle, out, expect, swiglu, torch.float16)
        w.close()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 600])
@pytest.mark.parametrize("bits", [4, 8])
def test_rmsnorm_linear(oracle, ws, M, bits):
    K, N = 2560, 2048
    codes = synth.codes(N, K, bits, 77).numpy()
    sc = synth.scales(N, bits, 78).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=90 + M, dist="student_t3")
    gam = synth.gamma(K, seed=91)
    for swiglu in (False, True):
        out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU if swiglu else 0,
                     gamma=gam.to(DEV), eps=1e-6)
        torch.cuda.synchronize()
        expect = oracle_linear(oracle, A, codes, sc, swiglu, gamma=gam.numpy())
        check_outputs(oracle, out, expect, swiglu, torch.float16)
    w.close()


def test_packed_weights_match_codes(oracle, ws):
    """qlin_weights_create_packed_device (the device layout) equals the [K,N] repack."""
    N, K = 512, 2560
    for bits in (4, 8):
        packed, codes, sc = synth.make_linear(N, K, bits, 1234 + bits, device=DEV)
        w1 = ql.Weights.from_packed_device(bits, K, N, packed, sc)
        w2 = make_weights(bits, codes.cpu().numpy(), sc.cpu().numpy())
        A = synth.activations(3, K, seed=3, device=DEV)
        o1 = ql.run(ws, w1, A)
        o2 = ql.run(ws, w2, A)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        w1.close()
        w2.close()


def test_nonfinite_activation_sets_status(ws):
    K, N = 256, 128
    codes = synth.codes(N, K, 8, 1).numpy()
    w = make_weights(8, codes, synth.scales(N, 8, 2).numpy())
    ws.status(clear=True)
    A = torch.randn((2, K), device=DEV, dtype=torch.float16)
    ql.run(ws, w, A)
    assert ws.status(clear=True) == 0
    A[1, 3] = float("inf")
    ql.run(ws, w, A)
    assert ws.status(clear=True) == ql._lib.QLIN_ERR_NONFINITE
    ql.run(ws, w, torch.randn((40, K), device=DEV, dtype=torch.float16))
    assert ws.status(clear=True) == 0
    w.close()


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("M", [1, 4, 6, 40, 1030])
def test_nonfinite_row_sets_status_every_path(ws, M, norm):
    """One Inf in the last activation row sets the sticky error word on every path: the
    fused-quantization GEMV (1, 4 and, without RMSNorm, 6 rows; 6 rows with RMSNorm take the
    separate quantize launch), the quantize launch before the GEMM (40 rows) and
    the many-rows quantize kernels (1030 rows), with and without RMSNorm; a clean run after it
    leaves the word clear."""
    K, N = 2560, 256
    codes = synth.codes(N, K, 4, 3).numpy()
    w = make_weights(4, codes, synth.scales(N, 4, 4).numpy())
    g = synth.gamma(K, seed=3, device=DEV) if norm else None
    A = synth.activations(M, K, seed=M, device=DEV)
    ws.status(clear=True)
    ql.run(ws, w, A, gamma=g, eps=1e-6)
    assert ws.status(clear=True) == 0
    bad = A.clone()
    bad[M - 1, 17] = float("inf")
    ql.run(ws, w, bad, gamma=g, eps=1e-6)
    assert ws.status(clear=True) == ql._lib.QLIN_ERR_NONFINITE
    ql.run(ws, w, A, gamma=g, eps=1e-6)
    assert ws.status(clear=True) == 0
    w.close()


# ------------------------------------------------------------------ reference test cases


@pytest.mark.parametrize("bits", [4, 8])
def test_reference_padding_case_host_api(ws, bits):
    """src/npu.rs:1161-1224 through the synchronous host-buffer entry points."""
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.npz"))
    codes, scales, inp = refcases.padding_case(bits)
    w = ql.Weights.from_codes_kn(bits, codes, scales)
    ref = gold[f"pad_w{bits}_out"]
    for rows in refcases.PADDING_ROWS:
        out = ql.run_host_f32(ws, w, inp[:rows])
        assert np.array_equal(out.view(np.uint32), ref[:rows].view(np.uint32)), rows
        refcases.compare(out, ref[:rows], 2e-5)
        if bits == 4 and rows >= 32:
            mid = ql.run_host_f32(ws, w, inp[:rows], swiglu=True)
            refcases.compare(mid, gold["pad_w4_swiglu"][:rows], 3e-5)
    # gate/up fusion is also offered below 32 rows and for W8
    mid = ql.run_host_f32(ws, w, inp[:5], swiglu=True)
    g, u = ref[:5, :128].astype(np.float64), ref[:5, 128:].astype(np.float64)
    refcases.compare(mid, (g / (1 + np.exp(-g)) * u).astype(np.float32), 3e-5)
    w.close()


@pytest.mark.parametrize("n", [32, 64])
def test_reference_narrow_case(ws, n):
    """src/npu/narrow_projection.rs:3-68: W8, K=2560, rows 1..7."""
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_cases.npz"))
    codes, scales, inp = refcases.narrow_case(n, 7)
    w = ql.Weights.from_codes_kn(8, codes, scales)
    for rows in refcases.NARROW_ROWS:
        out = ql.run_host_f32(ws, w, inp[:rows])
        assert np.array_equal(out.view(np.uint32), gold[f"narrow_n{n}_out"][:rows].view(np.uint32))
    w.close()


def test_host_api_rejects_nonfinite(ws):
    codes, scales, inp = refcases.padding_case(8)
    w = ql.Weights.from_codes_kn(8, codes, scales)
    bad = inp[:3].copy()
    bad[2, 5] = np.nan
    with pytest.raises(ql._lib.QlinError) as e:
        ql.run_host_f32(ws, w, bad)
    assert e.value.rc == ql._lib.QLIN_ERR_NONFINITE
    out = ql.run_host_f32(ws, w, inp[:3])  # the workspace recovers
    assert np.isfinite(out).all()
    w.close()


def test_graph_replay_matches_eager(ws):
    """Captured launches (GEMV with split-K counters, fused SwiGLU, GEMM) replayed several
    times between eager work reproduce the eager results bit for bit: the split-K
    partials and counters re-zero themselves, so no memset enters the graph."""
    specs = [(4, 2560, 6144, 1, 0), (4, 2560, 2048, 1, ql.QLIN_SWIGLU), (8, 4096, 2560, 1, 0),
             (4, 9728, 2560, 64, 0), (8, 2560, 1024, 3, ql.QLIN_SWIGLU)]
    ws_list, eager = [], []
    for i, (bits, K, N, M, fl) in enumerate(specs):
        packed, codes, sc = synth.make_linear(N, K, bits, 500 + i, device=DEV)
        w = ql.Weights.from_packed_device(bits, K, N, packed, sc)
        A = synth.activations(M, K, seed=600 + i, device=DEV)
        out = torch.empty((M, N // 2 if fl else N), dtype=torch.float16, device=DEV)
        ql.run(ws, w, A, out=out, flags=fl)
        torch.cuda.synchronize()
        ws_list.append((w, A, out, fl))
        eager.append(out.clone())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for w, A, out, fl in ws_list:
            ql.run(ws, w, A, out=out, flags=fl)
    for rep in range(3):
        for _, _, out, _ in ws_list:
            out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        for i, (_, _, out, _) in enumerate(ws_list):
            assert torch.equal(out, eager[i]), f"replay {rep} spec {i}"
        # eager work between replays on the same workspace
        w, A, out, fl = ws_list[0]
        ql.run(ws, w, A, out=out, flags=fl)
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0])
    for w, _, _, _ in ws_list:
        w.close()


@pytest.mark.parametrize("M", [1, 4, 64])
def test_lm_head_w8(oracle, M):
    """W8 output head at the vocabulary width (N = 151,936, K = 2560): one GEMV with 9,496
    channel groups at decode, the GEMM for a batched scoring pass."""
    K, N = 2560, 151936
    codes = synth.codes(N, K, 8, 960).numpy()
    sc = synth.scales(N, 8, 961).numpy()
    w = make_weights(8, codes, sc)
    ws_head = ql.Workspace(64, K, N)
    A = synth.activations(M, K, seed=962 + M)
    out = ql.run(ws_head, w, A.to(DEV), out_dtype=torch.float16)
    torch.cuda.synchronize()
    check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, False), False, torch.float16)
    w.close()
    ws_head.close()
