"""OLMoE expert placement and gradient capture (drop-in for usaf/olmoe_streaming.py).

The reference streams each expert module's Parameters from host memory to
the device around its forward (pre/post hooks) and catches their gradients
with post-accumulate hooks, because its 12 GB GPU cannot hold the experts
(olmoe_streaming.py:39-136).  One MI355X holds every expert of the model in
HBM, so ``setup_streaming`` moves the whole model to the device once, in
place (``module.to``: Parameter objects, and the optimizers holding them,
stay valid) and streams nothing.  The reference's protocol around it is kept:

* every trainable expert Parameter reports its accumulated gradient into
  ``model._expert_grads`` ({full name: grad}) after backward;
* ``apply_captured_expert_grads(model, scale)`` turns those into
  ``param.grad`` (times ``scale``, fp32 math, cast to the Parameter's dtype)
  and empties the store; it is what the reference trainer calls before its
  optimizer step;
* ``model._stream_state`` counts expert modules inside their forward.

Gradient checkpointing, which the reference needs for memory, is opt-in here.
"""
from __future__ import annotations

import functools
from typing import Dict

import torch
import torch.nn as nn

EXPERT_SUFFIX = ".mlp.experts"


def _record_grad(store: Dict[str, torch.Tensor], full_name: str, param: nn.Parameter) -> None:
    """Post-accumulate hook body: keep a reference to the accumulated gradient."""
    if param.grad is not None:
        store[full_name] = param.grad.detach()


def capture_expert_grads(model: nn.Module, suffix: str = EXPERT_SUFFIX) -> int:
    """Install gradient capture on every trainable Parameter of the modules whose
    name ends with ``suffix``; returns the number of Parameters hooked."""
    store = model.__dict__.setdefault("_expert_grads", {})
    hooked = 0
    for mname, mod in model.named_modules():
        if not mname.endswith(suffix):
            continue
        for pname, param in mod.named_parameters(recurse=False):
            if param.requires_grad:
                param.register_post_accumulate_grad_hook(functools.partial(_record_grad, store, f"{mname}.{pname}"))
                hooked += 1
    return hooked


def apply_captured_expert_grads(model: nn.Module, scale: float = 1.0) -> int:
    """usaf/olmoe_streaming.py:139-167 (and moe_loader.py:778-802): each captured
    gradient, times ``scale`` in fp32, becomes ``.grad`` of the Parameter of the
    same name (in its dtype, on its device); the store is emptied.  Returns how
    many Parameters received a gradient."""
    store: Dict[str, torch.Tensor] = getattr(model, "_expert_grads", None) or {}
    if not store:
        return 0
    by_name = dict(model.named_parameters())
    given = 0
    for name in list(store):
        grad = store.pop(name)
        target = by_name.get(name)
        if target is None:
            continue
        target.grad = grad.detach().float().mul(scale).to(device=target.device, dtype=target.dtype)
        given += 1
    return given


def sync_expert_grads_to_cpu(model: nn.Module) -> int:
    """usaf/olmoe_streaming.py:170-173: the reference's older name for
    apply_captured_expert_grads (scale 1)."""
    return apply_captured_expert_grads(model)


def setup_streaming(model: nn.Module, device: torch.device, verbose: bool = True, *,
                    gradient_checkpointing: bool = False) -> nn.Module:
    """usaf/olmoe_streaming.py:39-136 for an MI355X: the whole model resident in
    HBM, expert gradients captured into ``model._expert_grads``, a residency
    counter in ``model._stream_state``.  ``gradient_checkpointing=True``
    enables the transformers mixin's reentrant checkpointing as the reference
    always does (it trades recompute for memory HBM does not lack)."""
    device = torch.device(device)
    tally = {True: [0, 0], False: [0, 0]}  # is-expert -> [tensors, bytes]
    for mname, mod in model.named_modules():
        for param in mod.parameters(recurse=False):
            entry = tally[mname.endswith(EXPERT_SUFFIX)]
            entry[0] += 1
            entry[1] += param.numel() * param.element_size()
    model.to(device)
    hooked = capture_expert_grads(model)
    state = {"resident": 0, "max": 0}

    def entered(_module, _args):
        state["resident"] += 1
        state["max"] = max(state["max"], state["resident"])

    def left(_module, _args, output):
        state["resident"] -= 1
        return output

    n_modules = 0
    for mname, mod in model.named_modules():
        if mname.endswith(EXPERT_SUFFIX):
            mod.register_forward_pre_hook(entered)
            mod.register_forward_hook(left)
            n_modules += 1
    model._stream_state = state
    if verbose:
        print(f"  HBM: {tally[False][0]} non-expert tensors ({tally[False][1] / 1e9:.2f} GB), "
              f"{tally[True][0]} expert tensors ({tally[True][1] / 1e9:.2f} GB); "
              f"gradient capture on {hooked} tensors of {n_modules} expert modules")
    if gradient_checkpointing:
        enable = getattr(model, "gradient_checkpointing_enable", None)
        if enable is None:
            if verbose:
                print("  gradient checkpointing: the model has no gradient_checkpointing_enable")
        else:
            enable(gradient_checkpointing_kwargs={"use_reentrant": True})
            if verbose:
                print("  gradient checkpointing: enabled (reentrant)")
    return model
