"""Expert parameter placement and gradient capture for OLMoE (usaf/olmoe_streaming.py).

The reference keeps the expert Parameters in host memory and copies them to
the device around every expert forward (pre/post hooks), capturing their
gradients with post-accumulate hooks (olmoe_streaming.py:39-136).  An MI355X
holds every expert of the model in HBM, so ``setup_streaming`` places all
Parameters on the device once; the hook protocol is kept -- expert gradients
are captured into ``model._expert_grads`` and ``apply_captured_expert_grads``
hands them to the canonical Parameters -- so callers of the reference work
unchanged.
"""
from __future__ import annotations

from typing import Dict

import torch
import torch.nn as nn


def _is_expert_module(name: str) -> bool:
    return name.endswith(".mlp.experts")


def _move_module_tensors(module: nn.Module, target: torch.device) -> None:
    """Move one module's Parameters (reassigned, .grad carried over) and buffers."""
    for pname, p in list(module._parameters.items()):
        if p is None or p.device == target:
            continue
        new = nn.Parameter(p.detach().to(target), requires_grad=p.requires_grad)
        if p.grad is not None:
            new.grad = p.grad.to(target)
        module._parameters[pname] = new
    for bname, b in list(module._buffers.items()):
        if b is not None and b.device != target:
            module._buffers[bname] = b.to(target)


def setup_streaming(model: nn.Module, device: torch.device, verbose: bool = True) -> nn.Module:
    """olmoe_streaming.py:39-136: every Parameter on ``device``; expert
    Parameters get gradient-capture hooks; forward hooks count resident expert
    modules (``model._stream_state``); gradient checkpointing as the reference."""
    device = torch.device(device)
    n_exp = n_other = 0
    bytes_exp = bytes_other = 0
    expert_modules = []
    for mname, mod in model.named_modules():
        is_expert = _is_expert_module(mname)
        for p in mod._parameters.values():
            if p is None:
                continue
            nb = p.numel() * p.element_size()
            if is_expert:
                n_exp += 1
                bytes_exp += nb
            else:
                n_other += 1
                bytes_other += nb
        _move_module_tensors(mod, device)
        if is_expert:
            expert_modules.append((mname, mod))
    if verbose:
        print(f"  HBM (resident): {n_other} tensors, {bytes_other / 1e9:.2f}GB")
        print(f"  HBM (experts):  {n_exp} tensors, {bytes_exp / 1e9:.2f}GB")

    if not hasattr(model, "_expert_grads"):
        model._expert_grads = {}
    grad_store: Dict[str, torch.Tensor] = model._expert_grads
    state = {"resident": 0, "max": 0}

    for mname, mod in expert_modules:
        for pname, p in mod._parameters.items():
            if p is None or not p.requires_grad:
                continue
            full = f"{mname}.{pname}"

            def _cap(param: nn.Parameter, _full: str = full) -> None:
                if param.grad is not None:
                    grad_store[_full] = param.grad.detach()

            p.register_post_accumulate_grad_hook(_cap)

        def pre_hook(module, _args):
            state["resident"] += 1
            state["max"] = max(state["max"], state["resident"])

        def post_hook(module, _args, output):
            state["resident"] -= 1
            return output

        mod.register_forward_pre_hook(pre_hook)
        mod.register_forward_hook(post_hook)
    model._stream_state = state
    if verbose:
        print(f"  capture hooks on {len(expert_modules)} expert modules")
    try:
        model.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": True})
        if verbose:
            print("  gradient checkpointing: enabled (reentrant)")
    except Exception as exc:  # models without the transformers mixin
        if verbose:
            print(f"  gradient checkpointing: unavailable ({exc})")
    return model


def apply_captured_expert_grads(model: nn.Module, scale: float = 1.0) -> int:
    """olmoe_streaming.py:139-167: captured gradients x scale (fp32 math) ->
    ``param.grad`` of the canonical Parameters; clears the store."""
    store: Dict[str, torch.Tensor] = getattr(model, "_expert_grads", {})
    if not store:
        return 0
    params = dict(model.named_parameters())
    applied = 0
    for full, g in store.items():
        p = params.get(full)
        if p is not None:
            p.grad = (g.detach().float() * scale).to(device=p.device, dtype=p.dtype)
            applied += 1
    store.clear()
    return applied


def sync_expert_grads_to_cpu(model: nn.Module) -> int:
    """olmoe_streaming.py:170-173: alias of apply_captured_expert_grads."""
    return apply_captured_expert_grads(model)
