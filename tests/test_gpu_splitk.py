"""Split K in the 16x16x64 GEMM kernel, forced through QLIN_GEMM_KERNEL=16 and
QLIN_GEMM_SPLITS (a workspace reads both when it is created), against the oracle.

The splits of a tile are adjacent in the per-XCD workgroup order: with a tile count
divisible by 8 all splits of a tile run on one XCD, otherwise they may straddle XCDs (and a
grid whose size is not a multiple of 8 is not remapped at all).  Both kinds of grid must
give bit-exact int32 sums and fp16 outputs and SiLU-gate outputs within 1e-3 (the partials
are exchanged with device-coherent stores and loads either way).  Each shape runs twice on
one workspace, so the second run also checks that the tile counters reset themselves."""
import os

import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from tests.test_gpu_parity import check_outputs, make_weights, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def split_ws(rows, K, N, splits):
    os.environ["QLIN_GEMM_KERNEL"] = "16"
    os.environ["QLIN_GEMM_SPLITS"] = str(splits)
    try:
        return ql.Workspace(rows, K, N)
    finally:
        del os.environ["QLIN_GEMM_KERNEL"]
        del os.environ["QLIN_GEMM_SPLITS"]


# (M, K, N, splits, plain tiles of 128 x 128): 8 and 24 tiles keep a tile's splits on one
# XCD; 10 and 20 tiles (grids of 30 and 60) do not
SHAPES = [(256, 2048, 512, 2, 8), (256, 2048, 512, 4, 8), (200, 3072, 1536, 3, 24), (130, 4096, 640, 3, 10),
          (33, 9728, 2560, 3, 20)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,K,N,splits,tiles", SHAPES)
def test_split_k_matches_oracle(oracle, bits, M, K, N, splits, tiles):
    codes = synth.codes(N, K, bits, 700 + K % 11 + bits).numpy()
    sc = synth.scales(N, bits, 701 + bits).numpy()
    w = make_weights(bits, codes, sc)
    ws = split_ws(M, K, N, splits)
    A = synth.activations(M, K, seed=702 + M)
    pl = ql.plan(ws, w, A.to(DEV))
    assert pl["path"] == ql.QLIN_PATH_GEMM and pl["splits"] == splits, pl
    assert (pl["tile_m"], pl["tile_n"]) == (128, 128) and pl["grid"] == tiles * splits, pl
    q, s = ql.quantize(A.to(DEV), ldq=w.K_padded)
    ref = oracle.gemm_i32_nk(q.cpu().numpy()[:, :K], codes)
    for _ in range(2):
        acc = ql.gemm_i32(ws, w, q)
        torch.cuda.synchronize()
        assert np.array_equal(acc.cpu().numpy(), ref)
    y = oracle_linear(oracle, A, codes, sc, False)
    for _ in range(2):
        out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16)
        torch.cuda.synchronize()
        check_outputs(oracle, out, y, False, torch.float16)
    out = ql.run(ws, w, A.to(DEV), out_dtype=torch.float16, flags=ql.QLIN_SWIGLU)
    torch.cuda.synchronize()
    check_outputs(oracle, out, oracle_linear(oracle, A, codes, sc, True), True, torch.float16)
    ws.close()
    w.close()
