"""Parity at the benchmarked workloads' own shapes, sizes and distributions, through the
C ABI, against the CPU oracle.

- W8 decode GEMV, M=1, K=N=2560, int8 codes U[-127,127], scales U(0.002, 0.02), fp16
  N(0,1) activations with 1% x20 outlier channels (src/npu.rs:1052-1062, the W8 dynamic
  path), in both rounding modes and through the synchronous host entry point.
- One W4 layer at M=4096 with Student-t(3) activations: RMSNorm fused into the
  quantization of qkv and gate_up, SiLU-gate epilogue on gate_up.  q and s on every row;
  int32 sums and fp16 outputs against the oracle on two rows of every 128-row tile over
  all channels; every row's int32 sums against the platform's int8 GEMM (torch._int_mm,
  exact integer arithmetic) on the same q and codes, and every output against the
  oracle's dequant of those sums; the whole output free of NaN.
- The 36-layer mixed W4/W8 decoder stack at M=1 and M=4 (src/model/dense.rs:398-540:
  RMSNorm -> qkv -> o (+ residual) -> RMSNorm -> gate_up + SiLU-gate -> down
  (+ residual)), run as one launch per linear and as the one-launch decode chain; every
  stage of every layer is checked against the oracle applied to the stage's own input.

Bar: q, s, int32 sums and plain fp16 outputs bit-exact; SiLU-gate outputs within 1e-3
relative (|a-e| <= 1e-3 * max(|e|, 1)).
"""
import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import qlinear as ql
from open_rknpu2_lm_infer_amd import synth
from tests.test_gpu_parity import check_outputs, f16_bits

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def say(msg):
    print(f"[configs] {msg}", flush=True)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ W8 GEMV, M=1, 2560 x 2560


@pytest.mark.parametrize("rne", [False, True])
def test_w8_gemv_2560(oracle, rne):
    K = N = 2560
    packed, codes, sc = synth.make_linear(N, K, 8, synth.linear_seed(0, 0, workload=1), device=DEV)
    w = ql.Weights.from_packed_device(8, K, N, packed, sc)
    codes, sc = host(codes), host(sc)
    assert sc.min() >= 0.002 and sc.max() <= 0.02
    A = synth.activations(1, K, seed=synth.linear_seed(0, 0, workload=1) + 1, device=DEV)
    ws = ql.Workspace(1, K, N)
    rmode = oracle.ROUND_EVEN if rne else oracle.ROUND_AWAY
    flags = ql.QLIN_ROUND_HALF_EVEN if rne else 0
    say(f"w8 gemv 2560x2560 rne={rne}")

    x = A.float().cpu().numpy()
    q_ref, s_ref, bad = oracle.quantize(x, rmode)
    assert bad == 0
    q, s = ql.quantize(A, ldq=w.K_padded, flags=flags)
    torch.cuda.synchronize()
    assert np.array_equal(host(q)[:, :K], q_ref)
    assert np.array_equal(host(s).view(np.uint32), s_ref.view(np.uint32))

    acc_ref = oracle.gemm_i32_nk(q_ref, codes)
    assert np.array_equal(host(ql.gemm_i32(ws, w, q)), acc_ref)
    out_ref = oracle.dequant(acc_ref, s_ref, sc)
    for extra in (0, ql.QLIN_NO_FUSED_QUANT):
        for dtype in (torch.float16, torch.float32):
            out = ql.run(ws, w, A, out_dtype=dtype, flags=flags | extra)
            torch.cuda.synchronize()
            check_outputs(oracle, out, out_ref, False, dtype)
    if not rne:
        # the drop-in for rk_npu_f32i8f32_run_dynamic: host f32 in, host f32 out
        got = ql.run_host_f32(ws, w, x)
        assert np.array_equal(got.view(np.uint32), out_ref.view(np.uint32))
    ws.close()
    w.close()


# ------------------------------------------------------------------ W4 layer, M=4096, Student-t(3)


def sample_rows(M, tile=128):
    """Two rows of every 128-row tile, at positions that move from tile to tile, plus the last row."""
    rows = []
    for t in range((M + tile - 1) // tile):
        for r in ((t * 37) % tile, tile - 1 - (t * 11) % tile):
            if t * tile + r < M:
                rows.append(t * tile + r)
    rows.append(M - 1)
    return np.unique(np.array(rows))


@pytest.fixture(scope="module")
def ws4096():
    w = ql.Workspace(4096, 9728, 19456)
    yield w
    w.close()


@pytest.mark.parametrize("p", range(4))
def test_long_prefill_m4096(oracle, ws4096, p):
    M = 4096
    name, K, N = synth.LAYER[p]
    swiglu = name == "gate_up"
    say(f"M=4096 {name} {K}x{N}")
    packed, codes_d, sc = synth.make_linear(N, K, 4, synth.linear_seed(0, p), device=DEV)
    w = ql.Weights.from_packed_device(4, K, N, packed, sc)
    codes, sc = host(codes_d), host(sc)
    del packed
    A = synth.activations(M, K, seed=50100 + p, device=DEV, dist="student_t3")
    gamma = synth.gamma(K, seed=50000 + p // 2, device=DEV) if name in ("qkv", "gate_up") else None
    flags = ql.QLIN_SWIGLU if swiglu else 0

    out = ql.run(ws4096, w, A, out_dtype=torch.float16, flags=flags, gamma=gamma, eps=1e-6)
    q, s = ql.quantize(A, ldq=w.K_padded, gamma=gamma, eps=1e-6)
    torch.cuda.synchronize()

    # q and s on every row
    x = A.float().cpu().numpy()
    if gamma is not None:
        x = oracle.rmsnorm(x, host(gamma), 1e-6, "neon16")
    q_ref, s_ref, bad = oracle.quantize(x)
    assert bad == 0
    qg = host(q)
    assert np.array_equal(qg[:, :K], q_ref)
    assert not qg[:, K:].any()
    assert np.array_equal(host(s).view(np.uint32), s_ref.view(np.uint32))

    # int32 sums and outputs on two rows of every m tile, all channels
    rows = sample_rows(M)
    acc = ql.gemm_i32(ws4096, w, q)
    torch.cuda.synchronize()
    acc_ref = oracle.gemm_i32_nk(q_ref[rows], codes)
    got = host(acc[torch.as_tensor(rows, device=DEV)])
    bad = np.argwhere(got != acc_ref)
    assert len(bad) == 0, f"{len(bad)} int32 mismatches, first {bad[:3].tolist()}"
    ref = oracle.dequant(acc_ref, s_ref[rows], sc)
    if swiglu:
        ref = oracle.swiglu(ref)
    check_outputs(oracle, out[torch.as_tensor(rows, device=DEV)], ref, swiglu, torch.float16)
    assert not torch.isnan(out).any()

    # every row: the int32 sums against the platform's int8 GEMM (torch._int_mm, exact
    # integer products and sums) on the same q and codes, then every output against the
    # oracle's dequant (+ SiLU-gate) of those sums
    blas = torch._int_mm(q[:, :K].contiguous(), codes_d.t())
    torch.cuda.synchronize()
    assert torch.equal(acc, blas), f"{int((acc != blas).sum())} int32 mismatches against torch._int_mm"
    del blas, codes_d
    acc_all = host(acc)
    del acc
    ref = oracle.dequant(acc_all, s_ref, sc)
    del acc_all
    if swiglu:
        ref = oracle.swiglu(ref)
    check_outputs(oracle, out, ref, swiglu, torch.float16)
    w.close()


# ------------------------------------------------------------------ 36-layer mixed stack, M=1 and M=4


def oracle_stage(oracle, x16, codes, sc, gamma=None, swiglu=False, residual16=None):
    """fp16 bits of one decoder linear on fp16 input rows (the oracle, f32 math)."""
    x = x16.float().cpu().numpy()
    if gamma is not None:
        x = oracle.rmsnorm(x, gamma, 1e-6, "neon16")
    q, s, bad = oracle.quantize(x)
    assert bad == 0
    y = oracle.dequant(oracle.gemm_i32_nk(q, codes), s, sc)
    if swiglu:
        y = oracle.swiglu(y)
    if residual16 is not None:
        y = oracle.residual_add(residual16.float().cpu().numpy(), y, 1.0)
    return y


def assert_stage(oracle, got16, ref_f32, swiglu, what):
    if swiglu:
        check_outputs(oracle, got16, ref_f32, True, torch.float16)
        return
    g, e = f16_bits(got16), oracle.f32_to_f16_bits(ref_f32)
    bad = np.argwhere(g != e)
    assert len(bad) == 0, f"{what}: {len(bad)} fp16 mismatches, first {bad[:3].tolist()}"


@pytest.fixture(scope="module")
def stack():
    """36 layers: qkv, gate_up W4 (scales U(0.01, 0.1)), o, down W8 (variance-preserving
    scales), RMSNorm weights U(0.8, 1.2); the seeds of the benchmark's stack."""
    L = synth.N_LAYERS
    layers = []
    for l in range(L):
        ws_ = []
        for p, (name, K, N) in enumerate(synth.LAYER):
            bits = synth.layer_bits(name, True)
            seed = synth.linear_seed(l, p) if bits == 4 else synth.linear_seed(l, p, workload=4)
            packed, codes, sc = synth.make_linear(N, K, bits, seed, device=DEV, stack=bits == 8)
            ws_.append(ql.Weights.from_packed_device(bits, K, N, packed, sc))
            del packed, codes, sc
        g = (synth.gamma(synth.HIDDEN, seed=40000 + 2 * l, device=DEV),
             synth.gamma(synth.HIDDEN, seed=40001 + 2 * l, device=DEV))
        layers.append((ws_, g))
    torch.cuda.synchronize()
    yield layers
    for ws_, _ in layers:
        for w in ws_:
            w.close()


def host_codes(l, p):
    """Codes and scales of layer l, projection p, regenerated from their seeds."""
    name, K, N = synth.LAYER[p]
    bits = synth.layer_bits(name, True)
    seed = synth.linear_seed(l, p) if bits == 4 else synth.linear_seed(l, p, workload=4)
    _, codes, sc = synth.make_linear(N, K, bits, seed, device=DEV, stack=bits == 8)
    return host(codes), host(sc)


@pytest.mark.parametrize("M", [1, 4])
def test_stack_36_layers(oracle, stack, M):
    L = len(stack)
    ws = ql.Workspace(16, 9728, 19456)
    x = synth.activations(M, synth.HIDDEN, seed=40100 + M, device=DEV)
    say(f"stack {L} layers M={M}: launches")
    # one launch per linear; every stage output kept
    outs = []
    h = x
    for l, (w, g) in enumerate(stack):
        qkv = ql.run(ws, w[0], h, gamma=g[0], eps=1e-6)
        h1 = ql.run(ws, w[1], qkv[:, :4096], residual=h)
        mid = ql.run(ws, w[2], h1, flags=ql.QLIN_SWIGLU, gamma=g[1], eps=1e-6)
        h2 = ql.run(ws, w[3], mid, residual=h1)
        outs.append((h, qkv, h1, mid, h2))
        h = h2
    torch.cuda.synchronize()
    assert ws.status() == 0

    say(f"stack {L} layers M={M}: chain")
    stages = []
    for l, (w, g) in enumerate(stack):
        b = 4 * l
        hid = b - 1 if l else -1
        stages += [dict(weights=w[0], gamma=g[0], eps=1e-6, input=hid),
                   dict(weights=w[1], input=b, offset=0, residual=hid),
                   dict(weights=w[2], flags=ql.QLIN_SWIGLU, gamma=g[1], eps=1e-6, input=b + 1),
                   dict(weights=w[3], input=b + 2, residual=b + 1)]
    chain = ql.Chain(stages, max_rows=M)
    y = chain.run(x)
    torch.cuda.synchronize()
    assert chain.status() == 0
    couts = [chain.stage_output(s, M) for s in range(len(stages) - 1)] + [y]

    say(f"stack {L} layers M={M}: oracle")
    for l in range(L):
        h, qkv, h1, mid, h2 = outs[l]
        cin = x if l == 0 else couts[4 * l - 1]
        cq, ch1, cmid, ch2 = couts[4 * l: 4 * l + 4]
        gam = [host(stack[l][1][0]), host(stack[l][1][1])]
        cs = [host_codes(l, p) for p in range(4)]
        for tag, (hh, qq, hh1, mm, hh2) in (("launches", (h, qkv, h1, mid, h2)), ("chain", (cin, cq, ch1, cmid, ch2))):
            what = f"layer {l} {tag}"
            assert_stage(oracle, qq, oracle_stage(oracle, hh, *cs[0], gamma=gam[0]), False, what + " qkv")
            assert_stage(oracle, hh1, oracle_stage(oracle, qq[:, :4096], *cs[1], residual16=hh), False, what + " o")
            assert_stage(oracle, mm, oracle_stage(oracle, hh1, *cs[2], gamma=gam[1], swiglu=True), True,
                         what + " gate_up")
            assert_stage(oracle, hh2, oracle_stage(oracle, mm, *cs[3], residual16=hh1), False, what + " down")
    # the two executions agree bit for bit, and the stack stays finite
    assert torch.equal(y, outs[-1][4])
    assert torch.isfinite(y.float()).all()
    chain.close()
    ws.close()
