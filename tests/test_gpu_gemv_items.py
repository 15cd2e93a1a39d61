"""Decode GEMV with several 16-channel items per workgroup (more items than CUs, fused
quantization): against the oracle, and bit for bit against the one-item-per-workgroup
launch of the same shapes (QLIN_GEMV_GRID=0 forces it; the arithmetic is the same)."""
import os

import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from tests.test_gpu_parity import check_outputs, f16_bits, make_weights, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ws():
    w = ql.Workspace(8, 4096, 24000)
    yield w
    w.close()


def override_ws(ws, **env):
    """A workspace like ws whose kernel-variant overrides are the QLIN_* values given
    (a workspace reads the overrides once, when it is created)."""
    for k, v in env.items():
        os.environ[k] = str(v)
    try:
        return ql.Workspace(ws.max_rows, ws.max_k, ws.max_n)
    finally:
        for k in env:
            del os.environ[k]


def run_both(ws, w, A, **kw):
    """Output of the default launch and of the one-item-per-workgroup launch."""
    out = ql.run(ws, w, A, **kw)
    torch.cuda.synchronize()
    ws1 = override_ws(ws, QLIN_GEMV_GRID=0)
    ref = ql.run(ws1, w, A, **kw)
    torch.cuda.synchronize()
    assert ql.plan(ws1, w, A, kw.get("flags", 0), kw.get("gamma"))["grid"] == ql.plan(ws1, w, A, kw.get("flags", 0),
                                                                                      kw.get("gamma"))["items"]
    ws1.close()
    return out, ref


# item counts: 300 and 1000 plain (2 and 4 per workgroup on 256 CUs), 700 SwiGLU (3 each)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,swiglu", [(16 * 300, False), (16 * 1000, False), (2 * 16 * 700, True)])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_items_match_oracle_and_single_item(oracle, ws, bits, N, swiglu, M):
    K = 1024 if bits == 8 else 2560
    codes = synth.codes(N, K, bits, 300 + bits).numpy()
    sc = synth.scales(N, bits, 301 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=302 + M)
    flags = ql.QLIN_SWIGLU if swiglu else 0
    expect = oracle_linear(oracle, A, codes, sc, swiglu)
    for dt in (torch.float16, torch.float32):
        out, ref = run_both(ws, w, A.to(DEV).to(dt), out_dtype=torch.float16, flags=flags)
        assert np.array_equal(f16_bits(out), f16_bits(ref))
        check_outputs(oracle, out, expect, swiglu, torch.float16)
    w.close()


def test_items_rmsnorm_and_rne(oracle, ws):
    """RMSNorm prologue and round-half-even with several items per workgroup."""
    K, N = 2560, 2 * 16 * 600
    codes = synth.codes(N, K, 4, 310).numpy()
    sc = synth.scales(N, 4, 311).numpy()
    w = make_weights(4, codes, sc)
    A = synth.activations(1, K, seed=312, dist="student_t3")
    gam = synth.gamma(K, seed=313)
    out, ref = run_both(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU, gamma=gam.to(DEV), eps=1e-6)
    assert np.array_equal(f16_bits(out), f16_bits(ref))
    check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, True, gamma=gam.numpy()), True, torch.float16)
    out, ref = run_both(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU | ql.QLIN_ROUND_HALF_EVEN)
    assert np.array_equal(f16_bits(out), f16_bits(ref))
    check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, True, round_mode=oracle.ROUND_EVEN), True,
                  torch.float16)
    w.close()


@pytest.mark.parametrize("iw", [1, 5, 10, 13, 16])
@pytest.mark.parametrize("bits,N,swiglu", [(4, 2560, False), (8, 2 * 1312, True), (4, 6144, False)])
def test_item_width_matches_oracle(oracle, ws, iw, bits, N, swiglu):
    """Items narrower than the 16-row MFMA tile (QLIN_GEMV_ITEM_WIDTH): rows past the width
    re-read the item's last row and are not stored; every output channel once, bit for bit
    equal to the default width and within the bar of the oracle, fused and unfused."""
    K = 2560
    codes = synth.codes(N, K, bits, 320 + iw).numpy()
    sc = synth.scales(N, bits, 321 + iw).numpy()
    w = make_weights(bits, codes, sc)
    flags = ql.QLIN_SWIGLU if swiglu else 0
    for M, extra in ((1, 0), (3, 0), (1, ql.QLIN_NO_FUSED_QUANT)):
        A = synth.activations(M, K, seed=322 + M)
        ref = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, flags=flags | extra)
        torch.cuda.synchronize()
        ws1 = override_ws(ws, QLIN_GEMV_ITEM_WIDTH=iw)
        assert ql.plan(ws1, w, A.to(DEV), flags | extra)["item_width"] == iw
        out = ql.run(ws1, w, A.to(DEV), out_dtype=torch.float16, flags=flags | extra)
        torch.cuda.synchronize()
        ws1.close()
        assert np.array_equal(f16_bits(out), f16_bits(ref))
        check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, swiglu), swiglu, torch.float16)
    w.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("order", ["neon16", "seq"])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_rmsnorm_rows_fused(oracle, ws, bits, order, M):
    """RMSNorm of 2-4 rows inside the GEMV prologue (one wave per row sums its squares;
    the launch plan confirms the fused path ran): against the oracle, and bit for bit
    against the separate RMSNorm-quantize launch (QLIN_NO_FUSED_QUANT) and the
    one-item-per-workgroup launch, fp16 and f32 rows."""
    K = 2560
    flags0 = ql.QLIN_NORM_SEQUENTIAL if order == "seq" else 0
    for N, swiglu in ((2 * 16 * 600, True), (16 * 300, False), (2560, False)):
        codes = synth.codes(N, K, bits, 320 + bits + N % 7).numpy()
        sc = synth.scales(N, bits, 321 + bits).numpy()
        w = make_weights(bits, codes, sc)
        A = synth.activations(M, K, seed=322 + M, dist="student_t3")
        gam = synth.gamma(K, seed=323)
        flags = flags0 | (ql.QLIN_SWIGLU if swiglu else 0)
        x = oracle.rmsnorm(A.float().numpy(), gam.numpy(), 1e-6, order)
        q, s, _ = oracle.quantize(x, 0)
        expect = oracle.dequant(oracle.gemm_i32_nk(q, codes), s, sc)
        if swiglu:
            expect = oracle.swiglu(expect)
        for dt in (torch.float16, torch.float32):
            a = A.to(DEV).to(dt)
            # RMSNorm of 2-4 rows at K = 2560 runs inside the GEMV, except W8 N = 2560 at 4
            # rows: its 16-wave workgroups cannot hold 4 normalized rows, and at 4 rows the
            # separate launch is kept rather than fewer waves
            fused = not (bits == 8 and N == 2560 and M == 4)
            path = ql.plan(ws, w, a, flags, gam.to(DEV))["path"]
            assert path == (ql.QLIN_PATH_GEMV_FUSED if fused else ql.QLIN_PATH_GEMV), (N, M, path)
            out, ref = run_both(ws, w, a, out_dtype=torch.float16, flags=flags, gamma=gam.to(DEV), eps=1e-6)
            sep = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags | ql.QLIN_NO_FUSED_QUANT,
                         gamma=gam.to(DEV), eps=1e-6)
            torch.cuda.synchronize()
            assert np.array_equal(f16_bits(out), f16_bits(ref)), (N, dt)
            assert np.array_equal(f16_bits(out), f16_bits(sep)), (N, dt)
            check_outputs(oracle, out, expect, swiglu, torch.float16)
        w.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K", [4096, 9728])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_fused_rows_fewer_waves(oracle, bits, K, M):
    """o / down shapes (N = 2560): 16-wave workgroups hold 4 activation groups of 8 values
    per thread, so K = 4096 quantizes inside the GEMV up to 4 rows, and 3 and 4 rows of
    K = 9728 (two groups per row) take the 8-slot instances.  Every case equals the
    separate-quantize launch bit for bit and the oracle."""
    N = 2560
    ws = ql.Workspace(4, K, N)  # the separate quantization needs room for K columns
    codes = synth.codes(N, K, bits, 330 + bits + K % 11).numpy()
    sc = synth.scales(N, bits, 331 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=332 + M)
    expect = oracle_linear(oracle, A, codes, sc, False)
    fused = True
    for dt in (torch.float16, torch.float32):
        a = A.to(DEV).to(dt)
        pl = ql.plan(ws, w, a)
        assert pl["path"] == (ql.QLIN_PATH_GEMV_FUSED if fused else ql.QLIN_PATH_GEMV), pl
        assert ql.plan(ws, w, a, ql.QLIN_NO_FUSED_QUANT)["path"] == ql.QLIN_PATH_GEMV
        out = ql.run(ws, w, a, out_dtype=torch.float16)
        sep = ql.run(ws, w, a, out_dtype=torch.float16, flags=ql.QLIN_NO_FUSED_QUANT)
        torch.cuda.synchronize()
        assert np.array_equal(f16_bits(out), f16_bits(sep)), dt
        check_outputs(oracle, out, expect, False, torch.float16)
    w.close()
    ws.close()



@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2])
def test_fused_rows_three_groups_per_thread(oracle, bits, M):
    """K = 20480 at 16 waves: three activation groups of each row per thread, the slot
    layout chosen at run time (8-slot instances at two rows; one and two groups per thread
    take instances with the layout fixed at compile time).  Equal to the separate-quantize
    launch bit for bit and to the oracle."""
    K, N = 20480, 512
    ws = ql.Workspace(2, K, N)
    codes = synth.codes(N, K, bits, 340 + bits).numpy()
    sc = synth.scales(N, bits, 341 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=342 + M)
    expect = oracle_linear(oracle, A, codes, sc, False)
    a = A.to(DEV).to(torch.float16)
    pl = ql.plan(ws, w, a)
    assert pl["path"] == ql.QLIN_PATH_GEMV_FUSED and pl["waves"] == 16, pl
    out = ql.run(ws, w, a, out_dtype=torch.float16)
    sep = ql.run(ws, w, a, out_dtype=torch.float16, flags=ql.QLIN_NO_FUSED_QUANT)
    torch.cuda.synchronize()
    assert np.array_equal(f16_bits(out), f16_bits(sep))
    check_outputs(oracle, out, expect, False, torch.float16)
    w.close()
    ws.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N,swiglu", [(2560, 6144, False), (4096, 2560, False), (2560, 2 * 9728, True),
                                        (9728, 2560, False), (1024, 2 * 1000, True), (512, 600, False)])
@pytest.mark.parametrize("M", [5, 6, 7, 8])
def test_fused_rows_five_to_eight(oracle, bits, K, N, swiglu, M):
    """5..8 rows quantize inside the GEMV in the 8-row instances (8 waves, one activation
    group per thread per row) wherever a row holds at most 512 groups (K <= 4096: the qkv, o
    and gate_up shapes), equal bit for bit to the separate-quantize launch and to the
    oracle; K = 9728 (down) takes the separate launch."""
    ws = ql.Workspace(8, K, N)
    codes = synth.codes(N, K, bits, 340 + bits + K % 13 + M).numpy()
    sc = synth.scales(N, bits, 341 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=342 + M, dist="student_t3")
    flags = ql.QLIN_SWIGLU if swiglu else 0
    fused = K <= 4096
    for dt in (torch.float16, torch.float32):
        a = A.to(DEV).to(dt)
        pl = ql.plan(ws, w, a, flags)
        assert pl["path"] == (ql.QLIN_PATH_GEMV_FUSED if fused else ql.QLIN_PATH_GEMV), pl
        if fused:
            assert pl["waves"] == 8, pl
        out = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags)
        sep = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags | ql.QLIN_NO_FUSED_QUANT)
        torch.cuda.synchronize()
        assert np.array_equal(f16_bits(out), f16_bits(sep)), dt
        check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, swiglu), swiglu, torch.float16)
    w.close()
    ws.close()


@pytest.mark.parametrize("K", [2560, 4096, 9728])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8])
def test_fused_nonfinite_rows_match_separate(oracle, M, K):
    """Rows holding NaN and Inf through the fused prologue (whichever instance the plan
    takes) equal the separate quantize launch, which equals the oracle: the row maximum is
    the reference's fold of f32::max over |x| (src/npu.rs:1101-1106), NaN ignored and Inf
    kept.  Row 0 holds a NaN in the same 8-value group as its largest value, so dropping
    that group from the maximum would change the row's scale; with two or more rows the last
    row holds an Inf (scale Inf, every output of the row NaN).  fp16 and f32 rows, with and
    without RMSNorm (which turns a NaN or Inf row into NaN values throughout: maximum 0, scale
    1, every code 0); the status word reports the non-finite input on both paths."""
    N = 2560
    ws = ql.Workspace(8, K, N)
    codes = synth.codes(N, K, 4, 350 + M + K % 17).numpy()
    sc = synth.scales(N, 4, 351).numpy()
    w = make_weights(4, codes, sc)
    A = synth.activations(M, K, seed=352 + M).float()
    A[0, 43] = float("nan")
    A[0, 42] = 3000.0  # the row's largest value, in the NaN's group (columns 40..47)
    if M >= 2:
        A[M - 1, 3] = float("inf")
    gam = synth.gamma(K, seed=353)
    for norm in (False, True):
        x = oracle.rmsnorm(A.numpy(), gam.numpy(), 1e-6, "neon16") if norm else A.numpy()
        q_ref, s_ref, nbad = oracle.quantize(x)
        assert nbad == min(M, 2)
        if not norm:
            assert s_ref[0] == np.float32(np.float32(3000.0) / np.float32(127.0))
            assert M == 1 or s_ref[M - 1] == np.inf
        g = gam.to(DEV) if norm else None
        for dt in (torch.float16, torch.float32):
            a = A.to(dt).to(DEV)
            ws.status(clear=True)
            out = ql.run(ws, w, a, out_dtype=torch.float32, gamma=g, eps=1e-6)
            assert ws.status(clear=True) == ql._lib.QLIN_ERR_NONFINITE
            sep = ql.run(ws, w, a, out_dtype=torch.float32, flags=ql.QLIN_NO_FUSED_QUANT, gamma=g, eps=1e-6)
            assert ws.status(clear=True) == ql._lib.QLIN_ERR_NONFINITE
            q, s = ql.quantize(a, ldq=w.K_padded, gamma=g, eps=1e-6)
            torch.cuda.synchronize()
            assert np.array_equal(q.cpu().numpy()[:, :K], q_ref), (norm, dt)
            assert np.array_equal(s.cpu().numpy(), s_ref), (norm, dt)
            o, e = out.cpu().numpy(), sep.cpu().numpy()
            assert np.array_equal(o, e, equal_nan=True), (norm, dt, np.argwhere(~((o == e) | (np.isnan(o) & np.isnan(e))))[:3])
            if not norm:
                assert np.isfinite(o[0]).all() and np.isnan(o[M - 1]).all() == (M >= 2)
    w.close()
    ws.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,N,swiglu", [(2560, 6144, False), (2560, 2 * 9728, True), (4096, 2560, False),
                                        (9728, 2560, False), (1024, 2 * 1000, True)])
@pytest.mark.parametrize("M", [17, 20, 31, 32])
def test_gemv_two_row_blocks(oracle, bits, K, N, swiglu, M):
    """17..32 rows, quantized by a separate launch, take the GEMV with two 16-row blocks per
    weight fragment (the items kernel, at most 8 waves) up to 20 rows, and up to 32 rows for
    at most 4096 output channels; the GEMM otherwise.  Against the oracle (plain fp16
    bit-exact, SiLU-gate within 1e-3), fp16 and f32 rows, and on the GEMV bit for bit with
    every item in a workgroup of its own."""
    ws = ql.Workspace(32, K, N)
    codes = synth.codes(N, K, bits, 360 + bits + K % 13 + M).numpy()
    sc = synth.scales(N, bits, 361 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=362 + M, dist="student_t3")
    flags = ql.QLIN_SWIGLU if swiglu else 0
    expect = oracle_linear(oracle, A, codes, sc, swiglu)
    for dt in (torch.float16, torch.float32):
        a = A.to(DEV).to(dt)
        pl = ql.plan(ws, w, a, flags)
        if M <= 20 or N <= 4096:
            assert pl["path"] == ql.QLIN_PATH_GEMV and pl["waves"] <= 8, pl
            out, ref = run_both(ws, w, a, out_dtype=torch.float16, flags=flags)
            torch.cuda.synchronize()
            assert np.array_equal(f16_bits(out), f16_bits(ref)), dt
        else:
            assert pl["path"] == ql.QLIN_PATH_GEMM, pl
            out = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags)
        check_outputs(oracle, out, expect, swiglu, torch.float16)
    w.close()
    ws.close()


@pytest.mark.parametrize("K", [2560, 4096])
@pytest.mark.parametrize("rne", [False, True])
def test_fused_edge_rows_match_separate(oracle, K, rne):
    """Rows whose x * (1/s) land exactly on k + 0.5 (the rounding ties), an all-zero row
    (s = 1) and a row holding only an fp16 subnormal, through the fused prologue one row at a
    time, as 3 rows and as 6 rows (with 3 ordinary rows: the 5..8-row instances), in both
    rounding modes: every output bit for bit equal to the separate quantize launch and to the
    oracle (plain fp16 outputs)."""
    from tests.test_gpu_parity import tie_rows
    N = 2560
    ws = ql.Workspace(8, K, N)
    codes = synth.codes(N, K, 4, 370 + K % 7 + rne).numpy()
    sc = synth.scales(N, 4, 371).numpy()
    w = make_weights(4, codes, sc)
    edge = torch.from_numpy(tie_rows(K))
    rows = [edge[i:i + 1] for i in range(3)] + [edge, torch.cat([edge, synth.activations(3, K, seed=372).float()], 0)]
    flags = ql.QLIN_ROUND_HALF_EVEN if rne else 0
    mode = oracle.ROUND_EVEN if rne else oracle.ROUND_AWAY
    for A in rows:
        M = A.shape[0]
        for dt in (torch.float16, torch.float32):
            expect = oracle_linear(oracle, A.to(dt), codes, sc, False, round_mode=mode)  # the rows as the GPU sees them
            a = A.to(dt).to(DEV)
            assert ql.plan(ws, w, a, flags)["path"] == ql.QLIN_PATH_GEMV_FUSED, M
            out = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags)
            sep = ql.run(ws, w, a, out_dtype=torch.float16, flags=flags | ql.QLIN_NO_FUSED_QUANT)
            torch.cuda.synchronize()
            assert np.array_equal(f16_bits(out), f16_bits(sep)), (M, dt)
            check_outputs(oracle, out, expect, False, torch.float16)
    w.close()
    ws.close()
