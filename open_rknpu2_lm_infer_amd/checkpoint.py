"""compressed-tensors checkpoints straight to device weights.

Mirrors the reference loader (src/model/checkpoint.rs:213-423): the quantization
scheme of each module is found and validated exactly as QuantLoader::scheme / bits
do (symmetric static per-channel int W4/W8, dynamic per-token int8 activations, no
group scales, no actorder, no output quantization), the module's tensors are read
(weight_packed I32 + weight_shape for `pack-quantized`, weight I8 for
`int-quantized` W8, weight_scale [N, 1] in f32/f16/bf16), and the fused projections
are concatenated along N in module order.  Instead of unpacking to a host [K, N]
int8 matrix, the raw tensors go to qlin_weights_create_compressed, which writes the
device layout directly.

    ckpt = CompressedCheckpoint("/path/to/model")          # config.json + *.safetensors
    w = ckpt.weights(["model.layers.0.self_attn.q_proj", "...k_proj", "...v_proj"], [4096, 1024, 1024], 2560)

codes_kn() restates the reference's host decode (the QuantMatrix layout) for checks.
"""
from __future__ import annotations

import ctypes
import json
import os
import re

import numpy as np

from . import _lib


class CheckpointError(ValueError):
    pass


def _ensure(cond, msg):
    if not cond:
        raise CheckpointError(msg)


def _matches(target: str, module: str) -> bool:
    """src/model/checkpoint.rs:213-221."""
    if target == "Linear" or target == module:
        return True
    if target.startswith("re:"):
        return re.fullmatch(f"(?:{target[3:]})", module) is not None
    return False


def _symmetric(q, bits, strategy, dynamic):
    """src/model/checkpoint.rs:222-235."""
    q = q or {}
    ok = (q.get("num_bits") == bits and q.get("type") == "int" and q.get("strategy") == strategy
          and q.get("symmetric") is True
          and (q["dynamic"] is dynamic if "dynamic" in q else not dynamic)
          and q.get("group_size") is None and q.get("actorder") is None)
    _ensure(ok, "expected symmetric static channel W4/W8 and dynamic token A8; unsupported group scales/actorder")


class CompressedCheckpoint:
    """A compressed-tensors checkpoint: config.json (or a config dict) plus safetensors files."""

    def __init__(self, path: str, config: dict | None = None):
        self.path = path
        if config is None:
            with open(os.path.join(path, "config.json")) as f:
                config = json.load(f)
        quant = config.get("quantization_config") or {}
        _ensure(quant.get("quant_method") == "compressed-tensors" and quant.get("quantization_status") == "compressed",
                "expected a compressed-tensors compressed checkpoint")
        for key in ("sparsity_config", "transform_config"):
            v = quant.get(key)
            _ensure(v is None or v == {}, f"unsupported compressed-tensors {key}")
        _ensure(quant.get("kv_cache_scheme") is None, "quantized KV cache schemes are unsupported")
        _ensure(isinstance(quant.get("config_groups"), dict), "missing quantization config_groups")
        self.quant = quant
        files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors")) if os.path.isdir(path) else []
        _ensure(files, f"no safetensors files under {path}")
        from safetensors import safe_open
        self._files = {}
        self._where = {}
        for f in files:
            h = safe_open(os.path.join(path, f), framework="pt")
            self._files[f] = h
            for name in h.keys():
                self._where[name] = f

    # ---- tensors -----------------------------------------------------------------
    def contains(self, name: str) -> bool:
        return name in self._where

    def tensor(self, name: str):
        _ensure(name in self._where, f"missing tensor {name}")
        return self._files[self._where[name]].get_tensor(name)

    # ---- schemes -------------------------------------------------------------------
    def scheme(self, module: str) -> dict:
        """src/model/checkpoint.rs:276-305."""
        for target in self.quant.get("ignore") or []:
            _ensure(not _matches(target, module), f"required projection excluded from quantization: {module}")
        found = None
        for value in self.quant["config_groups"].values():
            targets = value.get("targets")
            _ensure(isinstance(targets, list), "missing quantization targets")
            for t in targets:
                if _matches(t, module):
                    _ensure(found is None or found == value, f"ambiguous quantization scheme: {module}")
                    found = value
        _ensure(found is not None, f"no quantization scheme for {module}")
        return found

    def bits(self, module: str) -> int:
        """src/model/checkpoint.rs:306-319."""
        s = self.scheme(module)
        bits = (s.get("weights") or {}).get("num_bits")
        _ensure(bits in (4, 8), "only W4A8 and W8A8 are supported")
        _symmetric(s.get("weights"), bits, "channel", False)
        _symmetric(s.get("input_activations"), 8, "token", True)
        _ensure(s.get("output_activations") is None, f"quantized linear output is unsupported: {module}")
        return bits

    def _module(self, module: str, n: int, k: int):
        """Validated raw tensors of one module: (bits, format, data uint8 bytes, scales f32 [n])."""
        import torch
        _ensure(n > 0 and k > 0, "invalid linear dimensions")
        bits = self.bits(module)
        _ensure(not self.contains(f"{module}.bias"), f"linear bias is unsupported: {module}")
        _ensure(not self.contains(f"{module}.weight_g_idx"), f"weight_g_idx/actorder unsupported: {module}")
        scale = self.tensor(f"{module}.weight_scale")
        _ensure(tuple(scale.shape) == (n, 1), f"unexpected shape: weight_scale: {tuple(scale.shape)}, expected {(n, 1)}")
        _ensure(scale.dtype in (torch.float32, torch.float16, torch.bfloat16), "weight_scale must be floating")
        scales = scale.float().reshape(n).numpy().copy()
        _ensure(bool(np.all(scales > 0)), f"nonpositive scale: {module}")
        if self.contains(f"{module}.weight_zero_point"):
            _ensure(not bool(self.tensor(f"{module}.weight_zero_point").any()), f"nonzero weight zero point: {module}")
        fmt = self.scheme(module).get("format") or self.quant.get("format") or ""
        if fmt == "pack-quantized":
            packed = self.tensor(f"{module}.weight_packed")
            columns = -(-k // (32 // bits))
            _ensure(tuple(packed.shape) == (n, columns),
                    f"unexpected shape: weight_packed: {tuple(packed.shape)}, expected {(n, columns)}")
            _ensure(packed.dtype == torch.int32, "weight_packed must be I32")
            shape = self.tensor(f"{module}.weight_shape")
            _ensure(tuple(shape.shape) == (2,), "unexpected shape: weight_shape")
            _ensure(int(shape[0]) == n and int(shape[1]) == k, f"weight_shape mismatch: {module}")
            return bits, _lib.QLIN_PACK_QUANTIZED, packed.contiguous().numpy().view(np.uint8), scales
        if fmt == "int-quantized" and bits == 8:
            w = self.tensor(f"{module}.weight")
            _ensure(tuple(w.shape) == (n, k), f"unexpected shape: weight: {tuple(w.shape)}, expected {(n, k)}")
            _ensure(w.dtype == torch.int8, "W8 weight must be signed I8")
            return bits, _lib.QLIN_INT_QUANTIZED, w.contiguous().numpy().view(np.uint8), scales
        raise CheckpointError(f"unsupported compressed-tensors storage: {fmt}")

    # ---- device weights ---------------------------------------------------------------
    def weights(self, modules: list, ns: list, k: int):
        """One device weight for the modules concatenated along N (q, k, v / gate, up),
        written in the device layout by qlin_weights_create_compressed."""
        from . import qlinear as ql
        parts = [self._module(m, n, k) for m, n in zip(modules, ns)]
        bits, fmt = parts[0][0], parts[0][1]
        _ensure(all(p[0] == bits for p in parts), "fused projections require identical bit widths and K")
        _ensure(all(p[1] == fmt for p in parts), "fused projections require one storage format")
        cfg = _lib.WeightConfig(bits, k, int(sum(ns)))
        n_parts = len(parts)
        part_n = (ctypes.c_int32 * n_parts)(*ns)
        data = (ctypes.c_void_p * n_parts)(*[p[2].ctypes.data for p in parts])
        scal = (ctypes.c_void_p * n_parts)(*[p[3].ctypes.data for p in parts])
        h = ctypes.c_void_p()
        _lib.check(_lib.load().qlin_weights_create_compressed(ctypes.byref(cfg), fmt, n_parts, part_n, data, scal,
                                                              ctypes.byref(h)), "qlin_weights_create_compressed")
        return ql.Weights(h)

    # ---- the reference's host decode, for checks ------------------------------------------
    def codes_kn(self, module: str, n: int, k: int):
        """(codes int8 [K, N], scales f32 [N]) as QuantLoader::load returns them."""
        bits, fmt, data, scales = self._module(module, n, k)
        if fmt == _lib.QLIN_INT_QUANTIZED:
            return np.ascontiguousarray(data.view(np.int8).reshape(n, k).T), scales
        factor = 32 // bits
        words = data.view(np.uint32).reshape(n, -1)
        kk = np.arange(k)
        fields = (words[:, kk // factor] >> ((kk % factor) * bits).astype(np.uint32)) & ((1 << bits) - 1)
        codes = fields.astype(np.int32) - (1 << (bits - 1))
        return np.ascontiguousarray(codes.astype(np.int8).T), scales
