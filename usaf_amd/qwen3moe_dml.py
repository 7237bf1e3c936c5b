"""Drop-in replacements for the reference's patched Qwen3-MoE forwards.

``patch_qwen3moe_for_dml()`` installs, exactly like usaf/qwen3moe_dml.py:89-94,

* ``Qwen3MoeExperts.forward(self, hidden_states [N, H], weights [N, E])`` and
* ``Qwen3MoeSparseMoeBlock.forward(self, hidden_states [B, S, H])``,

but the expert math runs on the routed tokens only, through the fused 4-bit
dequant-GEMM kernels (when the module carries HBM 4-bit tensors in
``module._usaf_q4``, set by ``moe_loader.setup_quantized_streaming``) or the
dense-weight variant of the same kernels (``self.gate_up_proj`` /
``self.down_proj``).  The result equals the reference's dense-masked sum:
non-routed experts contribute exact zeros there.

Grad capture keeps the reference protocol: with
``module._grad_capture = (store, prefix)`` the weight gradients of
``{prefix}.gate_up_proj`` / ``{prefix}.down_proj`` go to ``store`` -- sampled
at the active positions for ``usaf_amd.moe_loader.SparseGradStore``, as dense
per-expert tensors (``store.add(name, ei, g)`` or a dict of fp16 buffers) for
other stores.  The expert weights themselves receive no ``.grad``, as in the
reference (it detaches every per-expert slice).
"""
from __future__ import annotations

import torch

from .moe import ExpertWeights, RouteTopKFn, routed_experts


def _expert_weights(module) -> ExpertWeights:
    q4 = getattr(module, "_usaf_q4", None)
    if q4:
        gu, dn = q4.get("gate_up_proj"), q4.get("down_proj")
        if gu is None or dn is None:
            raise RuntimeError("module._usaf_q4 must hold gate_up_proj and down_proj")
        ew = ExpertWeights(gu, dn)
        # trained values over the 4-bit weights (QuantizedExpertCache.sync_resident)
        for local, ov in (getattr(module, "_usaf_q4_overlays", None) or {}).items():
            ew.overlays[local.replace("_proj", "")] = ov
        return ew
    gu = getattr(module, "gate_up_proj", None)
    dn = getattr(module, "down_proj", None)
    if gu is None or dn is None:
        raise RuntimeError("expert module has no weights: attach 4-bit tensors (module._usaf_q4) or "
                           "dense gate_up_proj/down_proj")
    return ExpertWeights(gu.detach(), dn.detach())


def _slot_cache_of(module, hidden_states: torch.Tensor, weights: torch.Tensor, capture):
    """The per-expert copy cache for this forward, if it may serve it: no
    gradient is wanted, the module carries no trained values (their masters
    change every step; the fused GEMMs read them through overlay tables) and
    the activations are in the copies' dtype."""
    slots = getattr(module, "_usaf_slots", None)
    if slots is None or capture is not None or getattr(module, "_usaf_q4_overlays", None):
        return None
    if torch.is_grad_enabled() and (hidden_states.requires_grad or weights.requires_grad):
        return None
    cache, name = slots
    return slots if hidden_states.dtype == cache.dtype else None


def dml_qwen3_experts_forward(self, hidden_states: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """qwen3moe_dml.py:24-64: [N, H] x routing weights [N, E] -> [N, H]."""
    capture = None
    if torch.is_grad_enabled() and getattr(self, "_grad_capture", None) is not None:
        capture = self._grad_capture
    slots = _slot_cache_of(self, hidden_states, weights, capture)
    if slots is not None:
        cache, name = slots
        return cache.forward(name, hidden_states.contiguous(), weights.to(cache.dtype).contiguous())
    return routed_experts(hidden_states, weights, _expert_weights(self), capture)


def dml_qwen3_moe_block_forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
    """qwen3moe_dml.py:67-86: router linear, fp32 softmax, >=-threshold top-k
    mask, optional renormalisation, routed experts."""
    batch_size, sequence_length, hidden_dim = hidden_states.shape
    hs = hidden_states.view(-1, hidden_dim)
    router = self.gate
    router_logits = torch.nn.functional.linear(hs, router.weight)
    weights = RouteTopKFn.apply(router_logits, int(router.top_k), bool(getattr(router, "norm_topk_prob", False)),
                                hs.dtype)
    final = self.experts(hs, weights)
    return final.view(batch_size, sequence_length, hidden_dim)


def patch_qwen3moe_for_dml():
    """Install the forwards on transformers' Qwen3-MoE classes (all instances)."""
    from transformers.models.qwen3_moe import modeling_qwen3_moe
    modeling_qwen3_moe.Qwen3MoeExperts.forward = dml_qwen3_experts_forward
    modeling_qwen3_moe.Qwen3MoeSparseMoeBlock.forward = dml_qwen3_moe_block_forward
    return modeling_qwen3_moe
