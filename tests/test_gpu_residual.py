"""Residual update fused into the linear's epilogue (qlin_run_residual and chain stages
with QLIN_RESIDUAL): the decoder's projected *= residual_multiplier; hidden += projected
(src/model/dense.rs:478-489, 528-537).

Bar: bit-exact against the oracle in f32 and fp16 (the linear's f32 value, then one f32
multiply and one f32 add, then the store rounding), for the decode GEMV (fused and
separate quantization) and the prefill GEMM, fp16 and f32 residual rows, in place and
out of place; chain stages equal qlin_run_residual on their own inputs bit for bit.
"""
import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from open_rknpu2_lm_infer_amd._lib import QLIN_ERR_PARAM, QlinError
from tests.test_gpu_parity import check_outputs, f16_bits, make_weights, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ws():
    w = ql.Workspace(600, 9728, 19456)
    yield w
    w.close()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 4, 6, 16, 17, 32, 512])
def test_residual_linear_bitexact(oracle, ws, bits, M):
    K, N = 4096, 2560  # the o projection's shape
    codes = synth.codes(N, K, bits, 70 + bits).numpy()
    sc = synth.scales(N, bits, 71 + bits).numpy()
    w = make_weights(bits, codes, sc)
    A = synth.activations(M, K, seed=72 + M)
    y = oracle_linear(oracle, A, codes, sc, False)
    for r_dtype, c_dtype, mult in ((torch.float16, torch.float16, 1.0), (torch.float32, torch.float32, 0.5),
                                   (torch.float16, torch.float32, 1.41421356), (torch.float32, torch.float16, 1.0)):
        R = synth.activations(M, N, seed=73 + M).to(r_dtype)
        expect = oracle.residual_add(R.float().numpy(), y, mult)
        for extra in (0, ql.QLIN_NO_FUSED_QUANT):
            out = ql.run(ws, w, A.to(DEV), out_dtype=c_dtype, flags=extra, residual=R.to(DEV), residual_scale=mult)
            torch.cuda.synchronize()
            check_outputs(oracle, out, expect, False, c_dtype)
        if r_dtype == c_dtype:
            # in place: the reference's hidden += projected
            h = R.to(DEV).clone()
            ql.run(ws, w, A.to(DEV), out=h, residual=h, residual_scale=mult)
            torch.cuda.synchronize()
            check_outputs(oracle, h, expect, False, c_dtype)
    w.close()


def test_residual_rejects_swiglu_and_bad_args(ws):
    K, N = 256, 128
    codes = synth.codes(N, K, 4, 80).numpy()
    w = make_weights(4, codes, synth.scales(N, 4, 81).numpy())
    A = synth.activations(1, K, seed=82).to(DEV)
    R = torch.zeros((1, N), dtype=torch.float16, device=DEV)
    with pytest.raises(QlinError) as e:
        ql.run(ws, w, A, flags=ql.QLIN_SWIGLU, out=torch.empty((1, N // 2), dtype=torch.float16, device=DEV),
               residual=R)
    assert e.value.rc == QLIN_ERR_PARAM
    with pytest.raises(QlinError) as e:  # a non-finite multiplier
        ql.run(ws, w, A, out=R, residual=R, residual_scale=float("inf"))
    assert e.value.rc == QLIN_ERR_PARAM
    w.close()


def linear(bits, K, N, seed):
    packed, codes, sc = synth.make_linear(N, K, bits, seed, stack=True)
    return ql.Weights.from_packed_device(bits, K, N, packed.to(DEV), sc.to(DEV))


def decoder_stages(layers, gammas):
    """Per layer: RMSNorm -> qkv (W4); o (W8) on the q columns, hidden += o; RMSNorm ->
    gate_up (W4, SwiGLU) on that hidden; down (W8), hidden += down.  Stage 4l + 1 and
    4l + 3 carry the residual stream."""
    (_, Kq, Nq), (_, Ko, No), (_, Kg, Ng), (_, Kd, Nd) = synth.LAYER
    stages = []
    for l in range(layers):
        b = 4 * l
        hid = b - 1 if l else -1  # the hidden rows entering this layer
        stages += [
            dict(weights=linear(4, Kq, Nq, synth.linear_seed(l, 0, workload=7)), gamma=gammas[2 * l], eps=1e-6,
                 input=hid, offset=0),
            dict(weights=linear(8, Ko, No, synth.linear_seed(l, 1, workload=7)), input=b, offset=0, residual=hid,
                 residual_scale=1.0),
            dict(weights=linear(4, Kg, Ng, synth.linear_seed(l, 2, workload=7)), flags=ql.QLIN_SWIGLU,
                 gamma=gammas[2 * l + 1], eps=1e-6, input=b + 1, offset=0),
            dict(weights=linear(8, Kd, Nd, synth.linear_seed(l, 3, workload=7)), input=b + 2, offset=0,
                 residual=b + 1, residual_scale=1.0),
        ]
    return stages


@pytest.mark.parametrize("rows", [1, 4])
def test_chain_residual_stages_match_single_linears(ws, rows):
    layers = 2
    gam = [synth.gamma(synth.HIDDEN, seed=950 + i).to(DEV) for i in range(2 * layers)]
    stages = decoder_stages(layers, gam)
    chain = ql.Chain(stages, max_rows=4)
    x = synth.activations(rows, synth.HIDDEN, seed=960 + rows, device=DEV)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    outs = [chain.stage_output(s, rows) for s in range(len(stages) - 1)] + [y]
    for s, st in enumerate(stages):
        src = x if st["input"] == -1 else outs[st["input"]]
        inp = src[:, st["offset"]:st["offset"] + st["weights"].K].contiguous()
        res = st.get("residual")
        kw = {}
        if res is not None:
            kw = dict(residual=(x if res == -1 else outs[res]).contiguous(), residual_scale=st["residual_scale"])
        ref = ql.run(ws, st["weights"], inp, out_dtype=torch.float16, flags=st.get("flags", 0),
                     gamma=st.get("gamma"), eps=st.get("eps", 1e-6), **kw)
        torch.cuda.synchronize()
        g, e = f16_bits(outs[s]), f16_bits(ref)
        bad = np.argwhere(g != e)
        assert len(bad) == 0, f"stage {s}: {len(bad)} fp16 mismatches, first {bad[:3].tolist()}"
        assert torch.isfinite(outs[s].float()).all()
    # launched again: the stage counters reset themselves and the result repeats
    y2 = chain.run(x)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and chain.status() == 0
    chain.close()


def test_chain_residual_rejects_bad_stages(ws):
    w0 = linear(4, 256, 512, 990)
    w1 = linear(8, 512, 256, 991)
    bad = [
        [dict(weights=w0, input=-1, offset=0), dict(weights=w1, input=0, offset=0, residual=1)],  # not earlier
        [dict(weights=w0, input=-1, offset=0), dict(weights=w1, input=0, offset=0, residual=0, residual_offset=384)],
        [dict(weights=w0, input=-1, offset=0, flags=ql.QLIN_SWIGLU, residual=-1),
         dict(weights=w1, input=0, offset=0)],
    ]
    for stages in bad:
        with pytest.raises(QlinError) as e:
            ql.Chain(stages, max_rows=1)
        assert e.value.rc == QLIN_ERR_PARAM
