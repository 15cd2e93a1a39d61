"""Seeded synthetic inputs for the five quantized-linear workloads.

All draws come from torch generators seeded from a base seed of 42 plus a stream
offset, on the device the data is made on (the same seed gives the same data on
the same device type).  Activations are drawn in f32 and rounded to fp16; the
oracle then reads those exact fp16 values.

Workloads (Qwen3-4B layer linears: hidden 2560, FFN 9728, q 4096 + k 1024 + v 1024):
  1. W8 GEMV, M=1, K=N=2560, int8 codes U[-127,127], scales U(0.002, 0.02)
  2. W4 GEMV over one layer, M=1: qkv 2560->6144, o 4096->2560,
     gate_up 2560->19456 (SiLU-gate fused), down 9728->2560; codes U[-8,7], scales U(0.01, 0.1)
  3. the same four linears at M=512 on the MFMA GEMM
  4. 36 such layers with o/down W8 and qkv/gate_up W4, M in {1, 4}, RMSNorm before qkv/gate_up
  5. one W4 layer at M=4096 with Student-t(3) activations and RMSNorm fused into the quantizer
Activations: N(0,1) with 1% of the K channels (seeded choice) scaled by 20.
"""
from __future__ import annotations

import math

import torch

BASE_SEED = 42
HIDDEN, FFN, QKV = 2560, 9728, 6144
LAYER = (
    ("qkv", HIDDEN, QKV),
    ("o", 4096, HIDDEN),
    ("gate_up", HIDDEN, 2 * FFN),
    ("down", FFN, HIDDEN),
)
N_LAYERS = 36


def gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(BASE_SEED + seed)
    return g


def activations(M: int, K: int, seed: int, device="cpu", dist: str = "normal",
                outlier_frac: float = 0.01, outlier_scale: float = 20.0) -> torch.Tensor:
    """fp16 [M, K]: N(0,1) (or Student-t with 3 dof) with outlier channels."""
    g = gen(seed, device)
    x = torch.randn((M, K), generator=g, device=device, dtype=torch.float32)
    if dist == "student_t3":
        chi2 = torch.randn((3, M, K), generator=g, device=device, dtype=torch.float32).square().sum(0)
        x = x / torch.sqrt(chi2 / 3.0)
    n_out = int(round(outlier_frac * K))
    if n_out:
        idx = torch.randperm(K, generator=g, device=device)[:n_out]
        x[:, idx] *= outlier_scale
    return x.to(torch.float16)


def codes(N: int, K: int, bits: int, seed: int, device="cpu") -> torch.Tensor:
    """int8 [N, K] uniform in [-8, 7] (W4) or [-127, 127] (W8)."""
    g = gen(seed, device)
    lo, hi = (-8, 7) if bits == 4 else (-127, 127)
    return torch.randint(lo, hi + 1, (N, K), generator=g, device=device, dtype=torch.int8)


def pack_w4(codes_nk: torch.Tensor) -> torch.Tensor:
    """[N, K] int8 codes -> [N, K/2] uint8, low nibble = even k."""
    c = codes_nk.to(torch.uint8) & 0xF
    return (c[:, 0::2] | (c[:, 1::2] << 4)).contiguous()


def scales(N: int, bits: int, seed: int, device="cpu") -> torch.Tensor:
    g = gen(seed, device)
    lo, hi = (0.01, 0.1) if bits == 4 else (0.002, 0.02)
    return (torch.rand((N,), generator=g, device=device, dtype=torch.float32) * (hi - lo) + lo).contiguous()


def gamma(K: int, seed: int, device="cpu") -> torch.Tensor:
    """RMSNorm weight U(0.8, 1.2), stored at fp16 precision (held as f32)."""
    g = gen(seed, device)
    x = torch.rand((K,), generator=g, device=device, dtype=torch.float32) * 0.4 + 0.8
    return x.to(torch.float16).to(torch.float32)


def linear_seed(layer: int, proj: int, workload: int = 2) -> int:
    return workload * 100000 + layer * 16 + proj


def layer_bits(name: str, mixed: bool) -> int:
    """Mixed W4/W8 stack: o and down are W8, qkv and gate_up W4."""
    if mixed and name in ("o", "down"):
        return 8
    return 4


def stack_scales(N: int, K: int, bits: int, seed: int, device="cpu") -> torch.Tensor:
    """Per-channel scales for a layer stack: W4 as in scales(); W8 variance preserving,
    U(0.5, 1.5) / (73 sqrt(K)) (73 ~ the std of uniform [-127, 127] codes), so an
    un-normalized W8 input (o, down) keeps its magnitude instead of growing ~50x per
    projection and overflowing fp16 a layer later.  The stack workload names no W8
    scale range; the single-linear U(0.002, 0.02) is kept for single linears."""
    if bits == 4:
        return scales(N, bits, seed, device)
    g = gen(seed, device)
    u = torch.rand((N,), generator=g, device=device, dtype=torch.float32) + 0.5
    return u / (73.0 * math.sqrt(K))


def make_linear(N: int, K: int, bits: int, seed: int, device="cpu", stack: bool = False):
    """(packed codes (W4: low nibble = even k), codes [N,K] int8, scales [N]) for one linear; stack=True
    draws W8 scales from stack_scales()."""
    c = codes(N, K, bits, seed, device)
    s = stack_scales(N, K, bits, seed + 7, device) if stack else scales(N, bits, seed + 7, device)
    packed = pack_w4(c) if bits == 4 else c.contiguous()
    return packed, c, s
