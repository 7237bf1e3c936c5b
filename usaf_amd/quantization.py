"""4-bit per-group expert-weight codec on the GPU.

Drop-in for the reference's ``usaf/quantization.py`` surface (same function
names, arguments, return structure and error types).  The arithmetic runs in
hand-written HIP kernels (``csrc/codec.hip``) over HBM-resident tensors;
results stay on the GPU.  Inputs on the CPU are copied to the current GPU
first.  There is no CPU path.

Format (quantization.py:47-85): the tensor is flattened row-major and cut into
groups of ``group_size`` (``min(group_size, numel)`` if smaller; the last
group zero-padded, the padding taking part in min/max).  Per group the fp16
``zero`` is the group minimum and the fp16 ``scale`` is
``max((max-min)/15, 1e-12)``; codes ``rint((x-min)/scale)`` clamped to
[0, 15] are computed with the fp32 scale/min and packed two per byte, element
2j in the low nibble of byte j.
"""
from __future__ import annotations

import math
from typing import Any, Dict, Tuple

import torch

from . import _native as N


def _resolve_device(*tensors: torch.Tensor, device=None) -> torch.device:
    if device is not None:
        N.require_gpu()
        return torch.device(device)
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return t.device
    return N.default_device()


def quantize_4bit(
    tensor: torch.Tensor,
    group_size: int = 128,
    *,
    device=None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Size]:
    """Quantize a float tensor to the 4-bit per-group format.

    Mirrors quantization.py:21-85.  Returns ``(packed int8 [groups,
    ceil(gs/2)], scale fp16 [groups], zero fp16 [groups], shape)`` with every
    tensor on the GPU.
    """
    if tensor.dim() == 0:
        raise ValueError("Scalar tensors cannot be quantized; skip them explicitly.")
    dev = _resolve_device(tensor, device=device)
    shape = tensor.shape
    x = tensor.detach()
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        x = x.float()
    x = N.on_device(x.reshape(-1), dev)
    numel = x.numel()
    if numel == 0:
        raise ValueError("quantize_4bit: empty tensors cannot be quantized")
    egs = min(group_size, numel)
    n_groups = (numel + egs - 1) // egs
    packed = torch.empty((n_groups, (egs + 1) // 2), dtype=torch.int8, device=dev)
    scale = torch.empty(n_groups, dtype=torch.float16, device=dev)
    zero = torch.empty(n_groups, dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        N.call("usaf_hip_quantize_q4", x.data_ptr(), N.dtype_code(x.dtype), numel, group_size,
               packed.data_ptr(), scale.data_ptr(), zero.data_ptr(), N.stream_ptr(dev))
    return packed, scale, zero, shape


def dequantize_4bit(
    q_int4: torch.Tensor,
    scale: torch.Tensor,
    zero: torch.Tensor,
    shape: torch.Size,
    group_size: int = 128,
    *,
    out_dtype: torch.dtype = torch.float16,
    out: torch.Tensor | None = None,
    device=None,
) -> torch.Tensor:
    """Dequantize a packed 4-bit tensor (quantization.py:88-132) on the GPU.

    ``x = fp16(fp16(q * scale) + zero)``, bit-identical to the reference's fp16
    arithmetic.  ``out_dtype=torch.bfloat16`` returns the round-to-nearest-even
    bf16 of that fp16 value.  ``out`` (contiguous, ``numel`` elements, right
    dtype, on the GPU) receives the result in place when given.
    """
    if q_int4.dim() != 2:
        raise ValueError(f"q_int4 must be 2-D [groups, packed_cols], got shape {tuple(q_int4.shape)}")
    dev = _resolve_device(q_int4, scale, zero, out, device=device)
    n_groups, packed_cols = int(q_int4.shape[0]), int(q_int4.shape[1])
    numel = 1
    for s in shape:
        numel *= int(s)
    egs = min(group_size, numel)
    if n_groups * egs > 2 * n_groups * packed_cols:
        raise RuntimeError(
            f"shape '[{n_groups}, {egs}]' is invalid for input of size {2 * n_groups * packed_cols}")
    if numel > n_groups * egs:
        raise RuntimeError(f"shape '{list(shape)}' is invalid for input of size {n_groups * egs}")
    if scale.numel() < n_groups or zero.numel() < n_groups:
        raise ValueError(f"scale/zero must hold {n_groups} entries")
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("out_dtype must be torch.float16 or torch.bfloat16")
    q = N.on_device(q_int4, dev, torch.int8) if q_int4.dtype != torch.uint8 else N.on_device(q_int4.view(torch.int8), dev)
    s = N.on_device(scale.reshape(-1)[:n_groups], dev, torch.float16)
    z = N.on_device(zero.reshape(-1)[:n_groups], dev, torch.float16)
    if out is None:
        out = torch.empty(numel, dtype=out_dtype, device=dev)
    else:
        if out.dtype != out_dtype or not out.is_contiguous() or out.numel() != numel or out.device != dev:
            raise ValueError("out must be a contiguous tensor of numel elements, dtype out_dtype, on the target GPU")
    with torch.cuda.device(dev):
        N.call("usaf_hip_dequant_q4", q.data_ptr(), s.data_ptr(), z.data_ptr(), n_groups, packed_cols,
               group_size, numel, out.data_ptr(), N.dtype_code(out_dtype), N.stream_ptr(dev))
    return out.view(shape)


def quantize_state_dict(
    state_dict: Dict[str, torch.Tensor],
    group_size: int = 128,
    min_size: int = 256,
    *,
    device=None,
) -> Dict[str, Any]:
    """Quantize every tensor with at least ``min_size`` elements (quantization.py:135-169).

    Small and 0-dim tensors are kept as fp16; other entries pass through.
    Quantized entries are ``{"q", "s", "z", "shape", "group_size"}`` dicts.
    """
    out: Dict[str, Any] = {}
    for name, param in state_dict.items():
        if not isinstance(param, torch.Tensor):
            out[name] = param
            continue
        if param.dim() == 0 or param.numel() < min_size:
            out[name] = param.detach().to(torch.float16)
            continue
        q, s, z, shape = quantize_4bit(param, group_size=group_size, device=device)
        out[name] = {"q": q, "s": s, "z": z, "shape": shape, "group_size": group_size}
    return out


def dequantize_state_dict(q_dict: Dict[str, Any], *, out_dtype: torch.dtype = torch.float16,
                          device=None) -> Dict[str, torch.Tensor]:
    """Inverse of ``quantize_state_dict`` (quantization.py:172-196), on the GPU."""
    out: Dict[str, torch.Tensor] = {}
    for name, entry in q_dict.items():
        if isinstance(entry, dict) and "q" in entry:
            out[name] = dequantize_4bit(entry["q"], entry["s"], entry["z"], entry["shape"],
                                        group_size=entry.get("group_size", 128), out_dtype=out_dtype,
                                        device=device)
        elif isinstance(entry, torch.Tensor):
            out[name] = entry.to(torch.float16)
        else:
            out[name] = entry
    return out


def estimate_quantized_size(num_params: int, bits: int = 4) -> Dict[str, float]:
    """Memory estimate in MiB (quantization.py:199-224; same formula, including
    its per-element fp16 scale/zero accounting)."""
    to_mib = 1.0 / (1024 * 1024)
    weight_mb = math.ceil(num_params * bits / 8) * to_mib
    scale_mb = num_params * 2 * to_mib
    zero_mb = scale_mb
    return {
        "weight_mb": round(weight_mb, 4),
        "scale_mb": round(scale_mb, 4),
        "zero_mb": round(zero_mb, 4),
        "total_mb": round(weight_mb + scale_mb + zero_mb, 4),
    }


def estimate_quantized_state_dict_size(
    state_dict: Dict[str, torch.Tensor],
    group_size: int = 128,
    min_size: int = 256,
) -> Dict[str, Any]:
    """Size accounting of a quantized state dict (quantization.py:227-285)."""
    to_mib = 1.0 / (1024 * 1024)
    original_bytes = quantized_bytes = 0
    per_param: list[dict] = []
    for name, param in state_dict.items():
        if not isinstance(param, torch.Tensor) or param.dim() == 0:
            continue
        n = param.numel()
        orig_b = n * param.element_size()
        if n < min_size:
            original_bytes += orig_b
            quantized_bytes += orig_b
            continue
        gs = min(group_size, n)
        groups = math.ceil(n / gs)
        q_total = groups * ((gs + 1) // 2) + 2 * groups * 2
        original_bytes += orig_b
        quantized_bytes += q_total
        per_param.append({"name": name, "elements": n, "orig_mb": round(orig_b * to_mib, 4),
                          "quant_mb": round(q_total * to_mib, 4)})
    original_mb = original_bytes * to_mib
    quantized_mb = quantized_bytes * to_mib
    ratio = original_mb / quantized_mb if quantized_mb > 0 else 1.0
    return {"original_mb": round(original_mb, 2), "quantized_mb": round(quantized_mb, 2),
            "compression_ratio": round(ratio, 2), "per_param": per_param}


def reconstruction_error(original: torch.Tensor, dequantized: torch.Tensor) -> float:
    """mse(dequant, orig) / var(orig), 0.0 for a constant tensor (quantization.py:288-315)."""
    orig = original.detach().float()
    deq = dequantized.detach().float().to(orig.device)
    if deq.shape != orig.shape:
        deq = deq.view(orig.shape)
    mse = ((deq - orig) ** 2).mean().item()
    var = orig.var(unbiased=False).item()
    if var < 1e-12:
        return 0.0
    return mse / var


def quantize_with_outliers(
    tensor: torch.Tensor,
    group_size: int = 128,
    outlier_fraction: float = 0.01,
    *,
    device=None,
) -> Dict[str, torch.Tensor]:
    """Outlier-split quantization (quantization.py:327-378): the top
    ``outlier_fraction`` by magnitude are kept in fp16, the rest quantized."""
    if tensor.dim() == 0:
        raise ValueError("Scalar tensors cannot be quantized.")
    dev = _resolve_device(tensor, device=device)
    shape = tensor.shape
    x = N.on_device(tensor.detach().reshape(-1).float(), dev)
    numel = x.numel()
    num_outliers = max(1, int(numel * outlier_fraction))
    _, top_indices = torch.topk(x.abs(), num_outliers)
    outlier_vals = x[top_indices].to(torch.float16)
    mask = torch.ones(numel, dtype=torch.bool, device=dev)
    mask[top_indices] = False
    q, s, z, _ = quantize_4bit(x[mask], group_size=group_size, device=dev)
    return {"q": q, "s": s, "z": z, "shape": shape, "group_size": group_size,
            "outlier_indices": top_indices.to(torch.int64), "outlier_values": outlier_vals}


def dequantize_with_outliers(packed: Dict[str, torch.Tensor], *, device=None) -> torch.Tensor:
    """Inverse of ``quantize_with_outliers`` (quantization.py:381-407)."""
    q, s, z, shape = packed["q"], packed["s"], packed["z"], packed["shape"]
    group_size = packed.get("group_size", 128)
    dev = _resolve_device(q, device=device)
    outlier_idx = packed["outlier_indices"].to(dev)
    outlier_val = packed["outlier_values"].to(dev)
    numel = 1
    for d in shape:
        numel *= int(d)
    clean_numel = numel - outlier_idx.numel()
    clean = dequantize_4bit(q, s, z, torch.Size([clean_numel]), group_size=group_size,
                            device=dev).reshape(-1).float()
    x_flat = torch.empty(numel, dtype=torch.float32, device=dev)
    mask = torch.ones(numel, dtype=torch.bool, device=dev)
    mask[outlier_idx] = False
    x_flat[mask] = clean
    x_flat[outlier_idx] = outlier_val.float()
    return x_flat.view(shape).to(torch.float16)
