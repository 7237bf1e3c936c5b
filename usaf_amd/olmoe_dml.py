"""Drop-in replacements for the reference's patched OLMoE forwards.

``patch_olmoe_for_dml()`` installs, like usaf/olmoe_dml.py:59-64,

* ``OlmoeExperts.forward(self, hidden_states [N, H], weights [N, E])`` and
* ``OlmoeSparseMoeBlock.forward(self, hidden_states [B, S, H])``.

The reference runs the expert math of this variant in fp32 so that fp16
activations cannot overflow (olmoe_dml.py:10-21).  Here the experts run routed
on the MFMA kernels in bf16 -- the exponent range of fp32 -- with fp32
accumulation, and the result is returned in the activations' dtype; the
expert weights are taken from ``module._usaf_q4`` (4-bit, HBM) when present,
else from the module's dense Parameters, which then receive dense gradients
as with the reference's autograd (olmoe_streaming.py:91-97 captures them).
"""
from __future__ import annotations

import torch

from .moe import ExpertWeights, RouteTopKFn, routed_experts

_COMPUTE = torch.bfloat16


def dml_experts_forward(self, hidden_states: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """olmoe_dml.py:10-33: [N, H] x routing weights [N, E] -> [N, H]."""
    q4 = getattr(self, "_usaf_q4", None)
    params = None
    if q4:
        ew = ExpertWeights(q4["gate_up_proj"], q4["down_proj"])
    else:
        wg, wd = self.gate_up_proj, self.down_proj
        ew = ExpertWeights(wg.detach().to(_COMPUTE).contiguous(), wd.detach().to(_COMPUTE).contiguous())
        params = (wg, wd)
    capture = None
    if torch.is_grad_enabled() and getattr(self, "_grad_capture", None) is not None:
        capture = self._grad_capture
    out = routed_experts(hidden_states.to(_COMPUTE), weights.to(_COMPUTE), ew, capture, params)
    return out.to(hidden_states.dtype)


def dml_moe_block_forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
    """olmoe_dml.py:36-56: router linear, fp32 softmax, >=-threshold top-k mask
    (no gradient through the mask), optional renormalisation, routed experts."""
    batch_size, sequence_length, hidden_dim = hidden_states.shape
    hs = hidden_states.view(-1, hidden_dim)
    router = self.gate
    router_logits = torch.nn.functional.linear(hs, router.weight)
    weights = RouteTopKFn.apply(router_logits, int(router.top_k), bool(getattr(router, "norm_topk_prob", False)),
                                hs.dtype)
    final = self.experts(hs, weights)
    return final.view(batch_size, sequence_length, hidden_dim)


def patch_olmoe_for_dml():
    """Install the forwards on transformers' OLMoE classes (all instances)."""
    from transformers.models.olmoe import modeling_olmoe
    modeling_olmoe.OlmoeExperts.forward = dml_experts_forward
    modeling_olmoe.OlmoeSparseMoeBlock.forward = dml_moe_block_forward
    return modeling_olmoe
