"""Decode chain (qlin_chain_*): several linears in one persistent launch.

Each stage must equal the single-linear entry point (qlin_run / qlin_run_rmsnorm)
applied to that stage's input, bit for bit in fp16: the chain fuses launches, not
arithmetic.  Stage inputs are taken from the chain's own previous outputs, so each
stage is checked on exactly what it consumed.  Against the oracle, each stage is
checked with the same bar as the single linear (plain outputs bit-exact, SwiGLU
within 1e-3 relative in fp16).
"""
import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from open_rknpu2_lm_infer_amd._lib import QLIN_ERR_NONFINITE, QLIN_ERR_PARAM, QlinError
from tests.test_gpu_parity import check_outputs, f16_bits, oracle_linear

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ws():
    w = ql.Workspace(16, 9728, 19456)
    yield w
    w.close()


def linear(bits, K, N, seed, stack=False):
    packed, codes, sc = synth.make_linear(N, K, bits, seed, stack=stack)
    w = ql.Weights.from_packed_device(bits, K, N, packed.to(DEV), sc.to(DEV))
    return w, codes.numpy(), sc.numpy()


def linear_unit(bits, K, N, seed):
    """A linear whose outputs keep an O(1) magnitude through SiLU-gate stages: scales
    1 / (code std * sqrt(K)) so short chains of small, oddly shaped stages stay finite."""
    codes = synth.codes(N, K, bits, seed)
    std = 4.6 if bits == 4 else 73.3
    sc = (torch.rand((N,), generator=synth.gen(seed + 7, "cpu")) * 0.4 + 0.8) / (std * K ** 0.5)
    packed = synth.pack_w4(codes) if bits == 4 else codes.contiguous()
    w = ql.Weights.from_packed_device(bits, K, N, packed.to(DEV), sc.float().to(DEV))
    return w, codes.numpy(), sc.float().numpy()


def stage_inputs(chain, stages, x, y, rows):
    """Input of every stage as the chain saw it, from its own outputs."""
    outs = [chain.stage_output(s, rows) for s in range(len(stages) - 1)] + [y]
    ins = []
    for st in stages:
        src = x if st["input"] == -1 else outs[st["input"]]
        ins.append(src[:, st["offset"]:st["offset"] + st["weights"].K].contiguous())
    return ins, outs


def check_against_single(ws, chain, stages, x, y, rows):
    ins, outs = stage_inputs(chain, stages, x, y, rows)
    for s, st in enumerate(stages):
        ref = ql.run(ws, st["weights"], ins[s], out_dtype=torch.float16, flags=st.get("flags", 0),
                     gamma=st.get("gamma"), eps=st.get("eps", 1e-6))
        torch.cuda.synchronize()
        g, e = f16_bits(outs[s]), f16_bits(ref)
        bad = np.argwhere(g != e)
        assert len(bad) == 0, f"stage {s}: {len(bad)} fp16 mismatches, first {bad[:3].tolist()}"
    return ins, outs


def build_small(seed0):
    w0 = linear(4, 512, 768, seed0)
    w1 = linear(8, 256, 512, seed0 + 1)
    w2 = linear(4, 512, 1024, seed0 + 2)
    w3 = linear(8, 512, 320, seed0 + 3)
    w4 = linear(4, 256, 96, seed0 + 4)
    g0 = synth.gamma(512, seed=seed0 + 5).to(DEV)
    g2 = synth.gamma(512, seed=seed0 + 6).to(DEV)
    stages = [
        dict(weights=w0[0], flags=0, gamma=g0, eps=1e-6, input=-1, offset=0),
        dict(weights=w1[0], flags=0, input=0, offset=128),
        dict(weights=w2[0], flags=ql.QLIN_SWIGLU, gamma=g2, eps=1e-6, input=1, offset=0),
        dict(weights=w3[0], flags=0, input=2, offset=0),
        dict(weights=w4[0], flags=0, input=-1, offset=256),
    ]
    host = [w0, w1, w2, w3, w4]
    return stages, host


@pytest.mark.parametrize("rows", [1, 3, 4])
def test_chain_small_matches_single_linears(oracle, ws, rows):
    stages, host = build_small(900)
    chain = ql.Chain(stages, max_rows=4)
    x = synth.activations(rows, 512, seed=901 + rows, device=DEV)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    ins, outs = check_against_single(ws, chain, stages, x, y, rows)
    # and each stage against the oracle on its own input
    for s, st in enumerate(stages):
        _, codes, sc = host[s]
        g = st.get("gamma")
        expect = oracle_linear(oracle, ins[s].cpu(), codes, sc, bool(st["flags"] & ql.QLIN_SWIGLU),
                               gamma=None if g is None else g.cpu().numpy())
        check_outputs(oracle, outs[s], expect, bool(st["flags"] & ql.QLIN_SWIGLU), torch.float16)
    chain.close()


def qwen_layer_stages(layer, gammas):
    """qkv (W4, RMSNorm) -> o (W8, the q columns of qkv) -> gate_up (W4, RMSNorm, SwiGLU)
    -> down (W8): the mixed W4/W8 decode layer with attention left out (stack scales)."""
    (_, Kq, Nq), (_, Ko, No), (_, Kg, Ng), (_, Kd, Nd) = synth.LAYER
    wq = linear(4, Kq, Nq, synth.linear_seed(layer, 0), stack=True)
    wo = linear(8, Ko, No, synth.linear_seed(layer, 1), stack=True)
    wg = linear(4, Kg, Ng, synth.linear_seed(layer, 2), stack=True)
    wd = linear(8, Kd, Nd, synth.linear_seed(layer, 3), stack=True)
    base = 4 * layer
    stages = [
        dict(weights=wq[0], flags=0, gamma=gammas[0], eps=1e-6, input=base - 1 if layer else -1, offset=0),
        dict(weights=wo[0], flags=0, input=base, offset=0),
        dict(weights=wg[0], flags=ql.QLIN_SWIGLU, gamma=gammas[1], eps=1e-6, input=base + 1, offset=0),
        dict(weights=wd[0], flags=0, input=base + 2, offset=0),
    ]
    return stages, [wq, wo, wg, wd]


@pytest.mark.parametrize("rows", [1, 4])
def test_chain_qwen_layer(ws, rows):
    gam = [synth.gamma(synth.HIDDEN, seed=910).to(DEV), synth.gamma(synth.HIDDEN, seed=911).to(DEV)]
    stages, host = qwen_layer_stages(0, gam)
    chain = ql.Chain(stages, max_rows=rows)
    x = synth.activations(rows, synth.HIDDEN, seed=912, device=DEV)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    check_against_single(ws, chain, stages, x, y, rows)
    chain.close()


def test_chain_two_layers_repeat(ws):
    """Eight stages; three launches in a row give identical results (the completion
    flags of one launch never satisfy the waits of the next)."""
    gam = [synth.gamma(synth.HIDDEN, seed=920 + i).to(DEV) for i in range(4)]
    s0, h0 = qwen_layer_stages(0, gam[:2])
    s1, h1 = qwen_layer_stages(1, gam[2:])
    stages = s0 + s1
    chain = ql.Chain(stages, max_rows=1)
    x = synth.activations(1, synth.HIDDEN, seed=925, device=DEV)
    first = chain.run(x).clone()
    torch.cuda.synchronize()
    check_against_single(ws, chain, stages, x, first, 1)
    for _ in range(2):
        y = chain.run(x)
        torch.cuda.synchronize()
        assert torch.equal(y, first)
    assert chain.status() == 0
    chain.close()


def test_chain_graph_replay():
    gam = [synth.gamma(synth.HIDDEN, seed=930).to(DEV), synth.gamma(synth.HIDDEN, seed=931).to(DEV)]
    stages, host = qwen_layer_stages(0, gam)
    chain = ql.Chain(stages, max_rows=4)
    x = synth.activations(4, synth.HIDDEN, seed=932, device=DEV)
    y = torch.empty((4, synth.HIDDEN), dtype=torch.float16, device=DEV)
    chain.run(x, out=y)
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        chain.run(x, out=y)
    for rep in range(3):
        y.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep}"
        chain.run(x, out=y)  # eager launch between replays
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    assert chain.status() == 0
    chain.close()


def test_chain_rejects_bad_stages():
    w_a = linear(4, 256, 512, 940)[0]
    w_b = linear(8, 512, 256, 941)[0]
    w_c = linear(4, 256, 97, 942)[0]  # odd N: no SiLU-gate pairing
    cases = [
        ([dict(weights=w_a, input=-1, offset=0), dict(weights=w_b, input=0, offset=4)], QLIN_ERR_PARAM),  # offset % 8
        ([dict(weights=w_a, input=-1, offset=0), dict(weights=w_b, input=1, offset=0)], QLIN_ERR_PARAM),  # not earlier
        ([dict(weights=w_a, input=-1, offset=0), dict(weights=w_b, input=0, offset=8)], QLIN_ERR_PARAM),  # past the end
        ([dict(weights=w_c, flags=ql.QLIN_SWIGLU, input=-1, offset=0)], QLIN_ERR_PARAM),
        ([dict(weights=w_a, input=0, offset=0)], QLIN_ERR_PARAM),  # stage 0 must read the input
    ]
    for stages, rc in cases:
        with pytest.raises(QlinError) as e:
            ql.Chain(stages, max_rows=1)
        assert e.value.rc == rc
    with pytest.raises(QlinError):
        ql.Chain([dict(weights=w_a, input=-1, offset=0)], max_rows=5)
    chain = ql.Chain([dict(weights=w_a, input=-1, offset=0)], max_rows=2)
    with pytest.raises(QlinError):
        chain.run(torch.zeros((3, 256), dtype=torch.float16, device=DEV))  # rows > max_rows
    chain.close()


def test_chain_nonfinite_status():
    w = linear(4, 256, 512, 950)[0]
    chain = ql.Chain([dict(weights=w, input=-1, offset=0)], max_rows=1)
    x = synth.activations(1, 256, seed=951, device=DEV)
    x[0, 7] = float("inf")
    chain.run(x)
    assert chain.status(clear=True) == QLIN_ERR_NONFINITE
    assert chain.status() == 0
    chain.close()


def test_chain_wait_give_up_and_recover(ws):
    """A stage wait that gives up (forced from the host with a wait limit of zero polls:
    every kernel still exits normally) is reported as QLIN_ERR_DEVICE by qlin_chain_status,
    which reads and clears the error word.  A run that gave up leaves no state behind: the
    next launch's epoch makes every completion flag fresh, so the same chain then runs
    correctly again with the default limit (src/model/dense.rs:398-540 stages, two layers)."""
    gam = [synth.gamma(synth.HIDDEN, seed=940 + i).to(DEV) for i in range(4)]
    s0, h0 = qwen_layer_stages(0, gam[:2])
    s1, h1 = qwen_layer_stages(1, gam[2:])
    stages = s0 + s1
    chain = ql.Chain(stages, max_rows=1)
    x = synth.activations(1, synth.HIDDEN, seed=945, device=DEV)
    chain.set_wait_limit(0)
    chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == ql._lib.QLIN_ERR_DEVICE
    chain.set_wait_limit(1 << 22)
    for _ in range(2):
        y = chain.run(x)
        torch.cuda.synchronize()
        assert chain.status() == 0
        check_against_single(ws, chain, stages, x, y, 1)
    with pytest.raises(QlinError):
        chain.set_wait_limit(-1)
    chain.close()


def test_chain_new_input_every_launch(oracle, ws):
    """Five launches with a different input each, eager and from a graph whose input
    buffer is refilled between replays: every stage of every launch equals the single
    linears on what it consumed, so no stage read a stale row of an earlier launch."""
    gam = [synth.gamma(synth.HIDDEN, seed=960 + i).to(DEV) for i in range(4)]
    s0, h0 = qwen_layer_stages(0, gam[:2])
    s1, h1 = qwen_layer_stages(1, gam[2:])
    stages = s0 + s1
    chain = ql.Chain(stages, max_rows=4)
    x = torch.empty((3, synth.HIDDEN), dtype=torch.float16, device=DEV)
    y = torch.empty((3, stages[-1]["weights"].N), dtype=torch.float16, device=DEV)
    g = torch.cuda.CUDAGraph()
    x.copy_(synth.activations(3, synth.HIDDEN, seed=969, device=DEV))
    chain.run(x, out=y)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        chain.run(x, out=y)
    for launch in range(5):
        x.copy_(synth.activations(3, synth.HIDDEN, seed=970 + launch, device=DEV))
        if launch % 2:
            g.replay()
        else:
            chain.run(x, out=y)
        torch.cuda.synchronize()
        assert chain.status() == 0
        check_against_single(ws, chain, stages, x, y, 3)
    chain.close()


def test_chain_swiglu_any_even_width(oracle, ws):
    """SiLU-gate stages whose half width is not a multiple of 16 or 64 (96 -> 48, 2 x 1000
    -> 1000): output channels are dealt to workgroups one by one, so any even N works."""
    wa = linear_unit(4, 512, 96, 980)
    wb = linear_unit(8, 48, 2000, 981)
    wc = linear_unit(4, 1000, 256, 982)
    stages = [
        dict(weights=wa[0], flags=ql.QLIN_SWIGLU, input=-1, offset=0),
        dict(weights=wb[0], flags=ql.QLIN_SWIGLU, input=0, offset=0),
        dict(weights=wc[0], flags=0, input=1, offset=0),
    ]
    chain = ql.Chain(stages, max_rows=2)
    x = synth.activations(2, 512, seed=983, device=DEV)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    ins, outs = check_against_single(ws, chain, stages, x, y, 2)
    for s, (st, host) in enumerate(zip(stages, (wa, wb, wc))):
        expect = oracle_linear(oracle, ins[s].cpu(), host[1], host[2], bool(st["flags"] & ql.QLIN_SWIGLU))
        check_outputs(oracle, outs[s], expect, bool(st["flags"] & ql.QLIN_SWIGLU), torch.float16)
    chain.close()


@pytest.mark.parametrize("rows", [1, 4])
def test_chain_w8_gate_up_in_rounds(oracle, ws, rows):
    """All-W8 Qwen3-4B MLP: RMSNorm -> gate_up (W8, K=2560, N=19456, SiLU-gate) -> down (W8).
    The gate_up share of a CU is 120 weight steps, more than the 80 the compute waves hold
    in registers, so the stage streams in two rounds; every stage equals the single-linear
    launch bit for bit, and the gate_up stage the oracle (src/npu.rs:1052-1062 W8 path)."""
    (_, Kg, Ng), (_, Kd, Nd) = synth.LAYER[2], synth.LAYER[3]
    wg = linear(8, Kg, Ng, synth.linear_seed(0, 2, workload=8), stack=True)
    wd = linear(8, Kd, Nd, synth.linear_seed(0, 3, workload=8), stack=True)
    gam = synth.gamma(synth.HIDDEN, seed=990).to(DEV)
    stages = [dict(weights=wg[0], flags=ql.QLIN_SWIGLU, gamma=gam, eps=1e-6, input=-1, offset=0),
              dict(weights=wd[0], flags=0, input=0, offset=0)]
    chain = ql.Chain(stages, max_rows=rows)
    x = synth.activations(rows, synth.HIDDEN, seed=991 + rows, device=DEV)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    ins, outs = check_against_single(ws, chain, stages, x, y, rows)
    expect = oracle_linear(oracle, ins[0].cpu(), wg[1], wg[2], True, gamma=gam.cpu().numpy())
    check_outputs(oracle, outs[0], expect, True, torch.float16)
    chain.close()
