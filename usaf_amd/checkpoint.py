"""Export of trained weights back to the 4-bit checkpoint format, on the GPU
(drop-in for usaf/checkpoint.py:58-92 ``export_merged_weights``).

For every entry of the quantized state dict (``experts_q4.pt``): dequantize
to fp16 (kernel a), write the trained fp32 masters of its active positions
into the fp16 tensor (fp16 rounding, as the reference's
``masters.to(float16)`` + ``scatter_``), re-quantize with the reference's
scheme (``usaf_hip_quantize_q4``), and save the result with ``torch.save``
as CPU tensors in the same dict layout.  Each tensor makes the round trip in
HBM, one at a time, so the largest intermediate is one fp16 tensor.
Entries that are neither 4-bit dicts nor tensors are dropped, as there.
"""
from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from . import _native as N
from .moe_loader import overlay_scatter
from .quantization import dequantize_4bit, quantize_state_dict


def merge_masters(q_dict: Dict[str, Any], masters: Dict[str, torch.Tensor], active_idx: Dict[str, torch.Tensor],
                  group_size: int = 128, device=None) -> Dict[str, Any]:
    """The merged, re-quantized state dict (CPU tensors) without touching disk."""
    dev = torch.device(device) if device is not None else N.default_device()
    out: Dict[str, Any] = {}
    for name, entry in q_dict.items():
        if isinstance(entry, dict) and "q" in entry:
            t = dequantize_4bit(entry["q"], entry["s"], entry["z"], entry["shape"],
                                group_size=entry.get("group_size", group_size), out_dtype=torch.float16,
                                device=dev)
        elif isinstance(entry, torch.Tensor):
            t = entry.detach().to(device=dev, dtype=torch.float16)
        else:
            continue
        if name in masters and name in active_idx:
            t = t.contiguous()
            overlay_scatter(t, active_idx[name], masters[name])
        # re-quantized and moved to the host before the next tensor is dequantized:
        # the HBM peak is one fp16 tensor and its codes
        q = quantize_state_dict({name: t}, group_size=group_size, device=dev)[name]
        del t
        out[name] = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in q.items()} \
            if isinstance(q, dict) else q.cpu()
        del q
    return out


def export_merged_weights(quant_path: str, masters: Dict[str, torch.Tensor], active_idx: Dict[str, torch.Tensor],
                          output_path: str, group_size: int = 128, *, device: Optional[torch.device] = None) -> str:
    """usaf/checkpoint.py:58-92: merge the masters into the 4-bit weights of
    ``quant_path`` and save the re-quantized dict to ``output_path``."""
    q_dict = torch.load(quant_path, map_location="cpu", weights_only=True)
    torch.save(merge_masters(q_dict, masters, active_idx, group_size, device), output_path)
    return output_path
