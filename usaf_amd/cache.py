"""Per-step activation capture of decoder blocks (usaf/cache.py:5-90).

Same interface as the reference's ``ActivationCache``: forward hooks on every
module whose class name marks a transformer block record its (detached)
outputs per forward call, on ``device`` -- pass the GPU to keep them in HBM.
As in the reference (cache.py:34-49), a copy to another device is a blocking
``.to(device)``: a GPU output cached on the CPU has landed when the hook
returns, so ``get_cached`` right after the forward reads finished data; an
output already on ``device`` is kept as a detached alias, not copied.
``memory_estimate_mb`` also counts the tensors inside tuple outputs (the
reference counts bare tensors only).
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Any, Dict, List, Optional, Set

import torch

_BLOCK_NAMES = ("DecoderLayer", "TransformerBlock", "GemmaDecoderLayer", "Gemma4DecoderLayer", "Block")


def _detach_to(x: Any, device: torch.device) -> Any:
    if isinstance(x, torch.Tensor):
        return x.detach().to(device)
    if isinstance(x, tuple):
        return tuple(_detach_to(t, device) for t in x)
    return x


class ActivationCache:
    def __init__(self, device: torch.device = torch.device("cpu")):
        self.device = torch.device(device)
        self._cache: "OrderedDict[str, List[Any]]" = OrderedDict()
        self._invalidated_modules: Set[str] = set()
        self._hooks: list = []
        self._step = 0

    def register_hooks(self, model: torch.nn.Module) -> None:
        """cache.py:13-21: hook every transformer block of ``model``."""
        self._hooks = []
        for name, module in model.named_modules():
            if self._is_transformer_block(module):
                self._hooks.append(module.register_forward_hook(self._make_hook(name)))
                self._cache[name] = []

    @staticmethod
    def _is_transformer_block(module: torch.nn.Module) -> bool:
        cls = type(module).__name__
        return any(b in cls for b in _BLOCK_NAMES)

    def _make_hook(self, name: str):
        def hook(module, inputs, output):
            if name in self._invalidated_modules:
                return output
            self._cache.setdefault(name, []).append(_detach_to(output, self.device))
            return output
        return hook

    def get_cached(self, name: str, step: int) -> Optional[Any]:
        """cache.py:53-59: output of block ``name`` at forward call ``step`` (None if absent)."""
        entries = self._cache.get(name)
        if entries is None or step >= len(entries):
            return None
        return entries[step]

    def invalidate(self, module_names: Set[str]) -> None:
        for name in module_names:
            self._invalidated_modules.add(name)
            self._cache.pop(name, None)

    def reset(self) -> None:
        self._cache.clear()
        self._invalidated_modules.clear()
        self._step = 0

    def advance_step(self) -> None:
        self._step += 1

    def remove_hooks(self) -> None:
        for h in self._hooks:
            h.remove()
        self._hooks.clear()

    @property
    def cached_modules(self) -> Set[str]:
        return set(self._cache.keys())

    def memory_estimate_mb(self) -> float:
        total = 0
        for entries in self._cache.values():
            for t in entries:
                if isinstance(t, torch.Tensor):
                    total += t.numel() * t.element_size()
                elif isinstance(t, tuple):
                    total += sum(x.numel() * x.element_size() for x in t if isinstance(x, torch.Tensor))
        return total / (1024 * 1024)
