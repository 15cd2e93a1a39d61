"""compressed-tensors loader: scheme validation and host decode on the CPU (against the
oracle's restatement of src/model/checkpoint.rs:352-378), device weights on the GPU
(against weights built from the host-decoded [K, N] codes)."""
import json

import numpy as np
import pytest
import torch

from open_rknpu2_lm_infer_amd import synth
from open_rknpu2_lm_infer_amd.checkpoint import CheckpointError, CompressedCheckpoint


def scheme(bits, fmt="pack-quantized", **over):
    w = {"num_bits": bits, "type": "int", "strategy": "channel", "symmetric": True, "dynamic": False,
         "group_size": None, "actorder": None}
    w.update(over)
    return {"targets": ["Linear"], "format": fmt, "weights": w,
            "input_activations": {"num_bits": 8, "type": "int", "strategy": "token", "symmetric": True,
                                  "dynamic": True, "group_size": None, "actorder": None},
            "output_activations": None}


def config(groups, **extra):
    q = {"quant_method": "compressed-tensors", "quantization_status": "compressed", "config_groups": groups}
    q.update(extra)
    return {"quantization_config": q}


def pack_words(codes_nk: np.ndarray, bits: int) -> np.ndarray:
    """Encode codes [N, K] as compressed-tensors I32 words (field = code + 2^(bits-1), LSB first)."""
    n, k = codes_nk.shape
    factor = 32 // bits
    cols = -(-k // factor)
    fields = np.zeros((n, cols * factor), np.uint32)
    fields[:, :k] = (codes_nk.astype(np.int32) + (1 << (bits - 1))).astype(np.uint32)
    words = np.zeros((n, cols), np.uint32)
    for i in range(factor):
        words |= fields[:, i::factor] << np.uint32(i * bits)
    return words.view(np.int32)


def write_ckpt(tmp_path, tensors: dict, cfg: dict):
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    return CompressedCheckpoint(str(tmp_path))


def module_tensors(name, codes_nk, bits, fmt, scale_dtype=torch.float32, seed=0):
    n, k = codes_nk.shape
    g = torch.Generator().manual_seed(seed)
    sc = (torch.rand((n, 1), generator=g) * 0.09 + 0.01).to(scale_dtype)
    t = {f"{name}.weight_scale": sc}
    if fmt == "pack-quantized":
        t[f"{name}.weight_packed"] = torch.from_numpy(pack_words(codes_nk, bits))
        t[f"{name}.weight_shape"] = torch.tensor([n, k], dtype=torch.int64)
    else:
        t[f"{name}.weight"] = torch.from_numpy(codes_nk.astype(np.int8))
    return t


@pytest.mark.parametrize("bits,fmt,k", [(4, "pack-quantized", 100), (4, "pack-quantized", 256),
                                        (8, "pack-quantized", 130), (8, "int-quantized", 96)])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.bfloat16])
def test_host_decode_matches_oracle(tmp_path, oracle, bits, fmt, k, scale_dtype):
    n = 48
    lo, hi = (-8, 7) if bits == 4 else (-128, 127)
    codes = np.random.default_rng(k + bits).integers(lo, hi + 1, (n, k)).astype(np.int8)
    ck = write_ckpt(tmp_path, module_tensors("m.proj", codes, bits, fmt, scale_dtype), config({"g": scheme(bits, fmt)}))
    got, sc = ck.codes_kn("m.proj", n, k)
    assert np.array_equal(got, codes.T)
    if fmt == "pack-quantized":
        words = pack_words(codes, bits).view(np.uint32)
        assert np.array_equal(oracle.unpack_compressed(words, n, k, bits), codes.T)
    assert sc.dtype == np.float32 and sc.shape == (n,)


def test_scheme_validation(tmp_path):
    codes = np.zeros((16, 64), np.int8)
    t = module_tensors("m.proj", codes, 4, "pack-quantized")
    bad = [
        config({"g": scheme(4, group_size=128)}),                  # group scales
        config({"g": scheme(4, strategy="tensor")}),               # not per channel
        config({"g": scheme(4, symmetric=False)}),                 # asymmetric
        config({"g": scheme(4)}, ignore=["m.proj"]),               # excluded module
        config({"g": scheme(4), "h": dict(scheme(4), weights=dict(scheme(4)["weights"], num_bits=8))}),  # ambiguous
        config({"g": dict(scheme(4), targets=["re:other.*"])}),    # no scheme
        config({"g": scheme(4)}, kv_cache_scheme={"num_bits": 8}),  # quantized KV cache
    ]
    for i, cfg in enumerate(bad):
        d = tmp_path / f"c{i}"
        d.mkdir()
        with pytest.raises(CheckpointError):
            write_ckpt(d, t, cfg).codes_kn("m.proj", 16, 64)
    d = tmp_path / "regex"
    d.mkdir()
    ok = write_ckpt(d, t, config({"g": dict(scheme(4), targets=["re:m\\.pro.*"])}))
    assert ok.bits("m.proj") == 4
    # tensor-level checks
    for key, val in [("m.proj.bias", torch.zeros(16)), ("m.proj.weight_g_idx", torch.zeros(64, dtype=torch.int32)),
                     ("m.proj.weight_zero_point", torch.ones((16, 1), dtype=torch.int8))]:
        d = tmp_path / key.replace(".", "_")
        d.mkdir()
        with pytest.raises(CheckpointError):
            write_ckpt(d, dict(t, **{key: val}), config({"g": scheme(4)})).codes_kn("m.proj", 16, 64)
    d = tmp_path / "shape"
    d.mkdir()
    with pytest.raises(CheckpointError):
        write_ckpt(d, dict(t, **{"m.proj.weight_shape": torch.tensor([16, 63])}),
                   config({"g": scheme(4)})).codes_kn("m.proj", 16, 64)
    d = tmp_path / "negscale"
    d.mkdir()
    with pytest.raises(CheckpointError):
        write_ckpt(d, dict(t, **{"m.proj.weight_scale": -torch.ones((16, 1))}),
                   config({"g": scheme(4)})).codes_kn("m.proj", 16, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("bits,fmt,k", [(4, "pack-quantized", 2560), (4, "pack-quantized", 100),
                                        (8, "pack-quantized", 260), (8, "int-quantized", 4096)])
def test_device_weights_match_host_decode(tmp_path, bits, fmt, k):
    """Fused q, k, v style parts: the device layout written from the raw tensors gives the
    same int32 sums and outputs as weights built from the host-decoded [K, N] codes."""
    from open_rknpu2_lm_infer_amd import qlinear as ql
    ns = [128, 64, 64]
    lo, hi = (-8, 7) if bits == 4 else (-127, 127)
    rng = np.random.default_rng(bits * 1000 + k)
    tensors, names = {}, []
    for i, n in enumerate(ns):
        name = f"layer.p{i}"
        names.append(name)
        tensors.update(module_tensors(name, rng.integers(lo, hi + 1, (n, k)).astype(np.int8), bits, fmt,
                                      torch.bfloat16 if i == 1 else torch.float32, seed=i))
    ck = write_ckpt(tmp_path, tensors, config({"g": scheme(bits, fmt)}))
    w_dev = ck.weights(names, ns, k)
    host = [ck.codes_kn(nm, n, k) for nm, n in zip(names, ns)]
    codes_kn = np.concatenate([c for c, _ in host], axis=1)
    scales = np.concatenate([s for _, s in host])
    w_ref = ql.Weights.from_codes_kn(bits, codes_kn, scales)
    ws = ql.Workspace(64, max(k, 256), sum(ns))
    for M in (1, 40):
        A = synth.activations(M, k, seed=M + k, device="cuda:0")
        q, s = ql.quantize(A, ldq=w_ref.K_padded)
        assert torch.equal(ql.gemm_i32(ws, w_dev, q), ql.gemm_i32(ws, w_ref, q))
        assert torch.equal(ql.run(ws, w_dev, A), ql.run(ws, w_ref, A))
    for w in (w_dev, w_ref):
        w.close()
    ws.close()
