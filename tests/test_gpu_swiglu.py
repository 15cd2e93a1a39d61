"""SiLU-gate for any even N, and the device SiLU-gate on the unfused layout.

The reference fuses SwiGLU only when N % 64 == 0 (src/npu.rs:1011) and otherwise runs
the linear, then Cpu::swiglu on the [M, 2F] output (src/model/dense.rs:508-522,
src/model/cpu.rs:119-152,327-351).  Here the fused epilogue takes every even N, and
qlin_swiglu is the device form of that fallback for callers holding an unfused output.
Bar: the oracle within 1e-3 (fp16) / 3e-5 (f32); the fallback route equal bit for bit
to the fused epilogue (both apply the same f32 SiLU-gate to the same f32 values).
"""
import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from open_rknpu2_lm_infer_amd._lib import QLIN_ERR_UNSUPPORTED, QlinError
from tests import refcases
from tests.test_gpu_parity import check_outputs, f16_bits, make_weights, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ws():
    w = ql.Workspace(512, 2560, 4096)
    yield w
    w.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("F", [1000, 1001, 20, 1])
def test_fused_swiglu_any_even_n(oracle, ws, bits, F):
    K, N = 2560, 2 * F
    codes = synth.codes(N, K, bits, 700 + F % 97 + bits).numpy()
    sc = synth.scales(N, bits, 701 + bits).numpy()
    w = make_weights(bits, codes, sc)
    for M in (1, 4, 64, 512):
        A = synth.activations(M, K, seed=702 + M)
        expect = oracle_linear(oracle, A, codes, sc, True)
        path = ql.plan(ws, w, A.to(DEV), ql.QLIN_SWIGLU)["path"]
        assert path == ql.QLIN_PATH_GEMM if M > 32 else path in (ql.QLIN_PATH_GEMV_FUSED, ql.QLIN_PATH_GEMV)
        for dtype in (torch.float16, torch.float32):
            out = ql.run(ws, w, A.to(DEV), out_dtype=dtype, flags=ql.QLIN_SWIGLU)
            # the fallback route: plain f32 linear, then the device SiLU-gate
            plain = ql.run(ws, w, A.to(DEV), out_dtype=torch.float32)
            via = ql.swiglu(plain, out_dtype=dtype)
            torch.cuda.synchronize()
            check_outputs(oracle, out, expect, True, dtype)
            assert torch.equal(out, via), (M, dtype)
    # the synchronous host entry point (rk_npu_w4a8_run_swiglu_f32's drop-in) takes it too
    A = synth.activations(3, K, seed=709)
    got = ql.run_host_f32(ws, w, A.float().numpy(), swiglu=True)
    refcases.compare(got, oracle_linear(oracle, A, codes, sc, True), 3e-5)
    w.close()


def test_odd_n_swiglu_unsupported(ws):
    K, N = 256, 65
    codes = synth.codes(N, K, 4, 710).numpy()
    w = make_weights(4, codes, synth.scales(N, 4, 711).numpy())
    A = synth.activations(1, K, seed=712).to(DEV)
    with pytest.raises(QlinError) as e:
        ql.run(ws, w, A, flags=ql.QLIN_SWIGLU)
    assert e.value.rc == QLIN_ERR_UNSUPPORTED
    w.close()


@pytest.mark.parametrize("F", [9728, 1000, 13])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.float16, torch.float16),
                                     (torch.float32, torch.float16)])
def test_swiglu_unfused_layout(oracle, F, xdt, ydt):
    rng = np.random.default_rng(F)
    M = 5
    x = (rng.standard_normal((M, 2 * F)) * rng.choice([0.5, 4, 40], size=(M, 1))).astype(np.float32)
    x[0, :3] = [-100.0, 0.0, 100.0]
    X = torch.from_numpy(x).to(xdt)
    # a row stride wider than 2F: the gate and up blocks are found from the row start
    Xpad = torch.zeros((M, 2 * F + 8), dtype=xdt)
    Xpad[:, :2 * F] = X
    Y = ql.swiglu(Xpad.to(DEV)[:, :2 * F], out_dtype=ydt)
    Y2 = ql.swiglu(X.to(DEV).contiguous(), out_dtype=ydt)
    torch.cuda.synchronize()
    assert torch.equal(Y, Y2)
    expect = oracle.swiglu(X.float().numpy())
    check_outputs(oracle, Y, expect, True, ydt)
