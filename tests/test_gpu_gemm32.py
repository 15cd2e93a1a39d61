"""The 32x32x32 MFMA GEMM in each of its tile configurations, forced through QLIN_GEMM_CFG
(a workspace reads the override when it is created), against the oracle: int32 sums
bit-exact, plain fp16 outputs bit-exact, SiLU-gate within 1e-3, the residual update
bit-exact; ragged M and N, split K, W4 and W8 (configuration 3 is W4 only).  By default the
library takes this kernel only for large grids (e.g. the M = 4096 gate_up) and for the
SiLU-gate GEMM whose 256 x 192 grid covers the CUs about once (the M = 512 gate_up), so these
tests keep every configuration covered."""
import os

import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from tests.test_gpu_parity import check_outputs, f16_bits, make_weights, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def cfg_ws(cfg, rows, K, N, splits=None):
    os.environ["QLIN_GEMM_CFG"] = str(cfg)
    if splits:
        os.environ["QLIN_GEMM_SPLITS"] = str(splits)
    try:
        return ql.Workspace(rows, K, N)
    finally:
        del os.environ["QLIN_GEMM_CFG"]
        os.environ.pop("QLIN_GEMM_SPLITS", None)


# every (configuration, bits) pair the kernel has: configuration 3 exists for W4 only
@pytest.mark.parametrize("cfg,bits", [(c, b) for b in (4, 8) for c in ((0, 1, 2, 3) if b == 4 else (0, 1, 2))])
@pytest.mark.parametrize("K,N,M,splits", [(2560, 1024, 300, None), (4096, 640, 33, 3), (1024, 2000, 513, 2)])
def test_gemm32_configs_match_oracle(oracle, cfg, bits, K, N, M, splits):
    codes = synth.codes(N, K, bits, 600 + cfg + K % 7 + bits).numpy()
    sc = synth.scales(N, bits, 601 + bits).numpy()
    w = make_weights(bits, codes, sc)
    ws = cfg_ws(cfg, M, K, N, splits)
    A = synth.activations(M, K, seed=602 + M)
    pl = ql.plan(ws, w, A.to(DEV))
    assert pl["path"] == ql.QLIN_PATH_GEMM
    if splits:
        assert pl["splits"] == splits, pl
    # int32 sums
    q, s = ql.quantize(A.to(DEV), ldq=w.K_padded)
    acc = ql.gemm_i32(ws, w, q)
    torch.cuda.synchronize()
    qh = q.cpu().numpy()[:, :K]
    assert np.array_equal(acc.cpu().numpy(), oracle.gemm_i32_nk(qh, codes))
    # plain fp16 and f32 outputs, and SiLU-gate
    for dtype in (torch.float16, torch.float32):
        out = ql.run(ws, w, A.to(DEV), out_dtype=dtype)
        torch.cuda.synchronize()
        check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, False), False, dtype)
    out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU)
    torch.cuda.synchronize()
    check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, True), True, torch.float16)
    # residual update in the epilogue: R + y * 0.5, f32 roundings, fp16 rows
    R = synth.activations(M, N, seed=603).to(DEV)
    out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, residual=R, residual_scale=0.5)
    torch.cuda.synchronize()
    y = oracle_linear(oracle, A, codes, sc, False)
    ref = oracle.residual_add(R.float().cpu().numpy(), y, 0.5)
    assert np.array_equal(f16_bits(out), oracle.f32_to_f16_bits(ref))
    ws.close()
    w.close()


def test_gemm32_is_default_for_large_grids():
    """The M = 4096 gate_up (1216 tiles of 256 x 256) takes the 32x32x32 kernel by default,
    and its output equals the 16x16x64 kernel's bit for bit."""
    name, K, N = synth.LAYER[2]
    packed, codes, sc = synth.make_linear(N, K, 4, synth.linear_seed(0, 2), device=DEV)
    w = ql.Weights.from_packed_device(4, K, N, packed, sc)
    ws = ql.Workspace(4096, K, N)
    A = synth.activations(4096, K, seed=610, device=DEV)
    pl = ql.plan(ws, w, A, ql.QLIN_SWIGLU)
    assert pl["tile_m"] == 256 and pl["tile_n"] == 128, pl
    out = ql.run(ws, w, A, flags=ql.QLIN_SWIGLU)
    os.environ["QLIN_GEMM_KERNEL"] = "16"
    try:
        ws16 = ql.Workspace(4096, K, N)
    finally:
        del os.environ["QLIN_GEMM_KERNEL"]
    assert ql.plan(ws16, w, A, ql.QLIN_SWIGLU)["tile_m"] == 128
    ref = ql.run(ws16, w, A, flags=ql.QLIN_SWIGLU)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    ws.close()
    ws16.close()
    w.close()


def test_gemm32_gate_up_512_takes_256x192():
    """The M = 512 gate_up (W4, SiLU-gate) takes the 256 x 192 tiles by default (204 tiles for
    256 CUs), and its output equals the 16x16x64 kernel's bit for bit; so do a ragged M = 500
    and, with the tiles forced, the residual-free plain output of the same weights."""
    name, K, N = synth.LAYER[2]
    packed, codes, sc = synth.make_linear(N, K, 4, synth.linear_seed(0, 2), device=DEV)
    w = ql.Weights.from_packed_device(4, K, N, packed, sc)
    ws = ql.Workspace(512, K, N)
    os.environ["QLIN_GEMM_KERNEL"] = "16"
    try:
        ws16 = ql.Workspace(512, K, N)
    finally:
        del os.environ["QLIN_GEMM_KERNEL"]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for M in (512, 500):
        A = synth.activations(M, K, seed=611 + M, device=DEV)
        pl = ql.plan(ws, w, A, ql.QLIN_SWIGLU)
        if cus == 256:
            assert pl["tile_m"] == 256 and pl["tile_n"] == 96 and pl["splits"] == 1, pl
        assert ql.plan(ws16, w, A, ql.QLIN_SWIGLU)["tile_m"] == 128
        out = ql.run(ws, w, A, flags=ql.QLIN_SWIGLU)
        ref = ql.run(ws16, w, A, flags=ql.QLIN_SWIGLU)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), M
    ws.close()
    ws16.close()
    w.close()
