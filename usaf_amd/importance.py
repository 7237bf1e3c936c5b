"""Active-set selection on the GPU: the importance pass and the RigL reselect
of the reference trainer (usaf/moe_loader.py:584-631, train.py:536-613).

* ``topk_abs`` -- positions of the k largest |x| by a device-side radix
  select (usaf_hip_topk_abs), in ascending position order;
* ``TopKImportanceStore`` -- the reference's capture store: per expert slice
  the top ``frac * cand_mult`` |grad| candidates, then one global top-k per
  tensor in ``select``; every selection runs on the GPU;
* ``dequant_at`` -- dequantized values at flat positions of a 4-bit tensor
  (usaf_hip_dequant_q4_at), without dequantizing the tensor;
* ``reselect_active`` -- the reference's merge of the old active set with a
  new selection: keep the intersection, grow the smallest-index newcomers up
  to the old size, carry the kept masters over and seed the grown ones from
  the 4-bit weights.

Selections equal torch.topk's index sets whenever the k-th and (k+1)-th
magnitudes differ; on a tie this build takes the lowest positions (torch
leaves the choice unspecified).  Orders differ: the reference returns
candidates by descending magnitude, this build by position; every consumer
(``SparseGradStore``, ``SparseAdam``, set arithmetic) is order-free.
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch

from . import _native as N
from .moe import Q4Tensor


def topk_abs(x: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(pos int64 [min(k, n)], |x[pos]| fp32) of the k largest magnitudes of the
    flattened GPU tensor ``x`` (fp32, fp16 or bf16)."""
    if not x.is_cuda:
        raise ValueError("topk_abs runs on the GPU; pass a cuda tensor")
    flat = x.detach().reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    n = flat.numel()
    k = max(0, min(int(k), n))
    dev = flat.device
    pos = torch.empty(k, dtype=torch.int64, device=dev)
    vals = torch.empty(k, dtype=torch.float32, device=dev)
    if k == 0:
        return pos, vals
    ws = torch.empty(int(N.load().usaf_hip_topk_abs_ws_ints(n)), dtype=torch.int32, device=dev)
    N.call("usaf_hip_topk_abs", flat.data_ptr(), N.dtype_code(flat.dtype), n, k, pos.data_ptr(), vals.data_ptr(),
           ws.data_ptr(), N.stream_ptr(dev))
    return pos, vals


def dequant_at(entry: Any, idx: torch.Tensor, device=None) -> torch.Tensor:
    """fp32 of the fp16 dequantized values of a 4-bit tensor at flat positions
    ``idx`` (the reference's dequantize_4bit(...).reshape(-1)[idx].float());
    ``entry`` is a Q4Tensor, a quantize_state_dict entry or a dense tensor."""
    if isinstance(entry, torch.Tensor):
        dev = torch.device(device) if device is not None else entry.device
        return entry.detach().reshape(-1).to(dev)[idx.to(dev).long()].float()
    q = entry if isinstance(entry, Q4Tensor) else Q4Tensor.from_entry(entry, device)
    dev = q.device
    idx = idx.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    out = torch.empty(idx.numel(), dtype=torch.float32, device=dev)
    if idx.numel() == 0:
        return out
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    N.call("usaf_hip_dequant_q4_at", q.q.data_ptr(), q.s.data_ptr(), q.z.data_ptr(), q.q.shape[0], q.q.shape[1],
           q.group_size, q.numel(), idx.data_ptr(), idx.numel(), out.data_ptr(), bad.data_ptr(),
           N.stream_ptr(dev))
    if bool(bad.item()):
        raise IndexError("dequant_at: position outside the tensor")
    return out


class TopKImportanceStore:
    """usaf/moe_loader.py:584-631 with GPU selection.  The same ``add`` protocol
    as SparseGradStore: ``add(full_name, ei, g)`` receives expert ei's dense
    gradient slice and keeps its top ``numel * frac * cand_mult`` |g| candidates
    (at least one) as fp32 magnitudes and global flat indices;
    ``select(frac)`` returns, per tensor, the global indices of the top
    ``numel * frac`` (at least one, at most all) candidates."""

    def __init__(self, shapes: Dict[str, Any], frac: float, cand_mult: float = 2.0) -> None:
        self._shapes = {name: tuple(int(d) for d in shape) for name, shape in shapes.items()}
        self._frac = frac
        self._cand = cand_mult
        self._found: Dict[str, Dict[int, Tuple[torch.Tensor, torch.Tensor]]] = {n: {} for n in self._shapes}

    def zero_(self) -> None:
        for per_expert in self._found.values():
            per_expert.clear()

    def add(self, full_name: str, ei: int, g: torch.Tensor) -> None:
        per_expert = self._found.get(full_name)
        if per_expert is None:
            return
        if not g.is_cuda:
            g = g.to(N.default_device())
        width = g.numel()
        want = max(1, int(width * self._frac * self._cand))
        pos, mags = topk_abs(g, want)
        per_expert[int(ei)] = (mags, pos + int(ei) * width)

    def select(self, frac: Optional[float] = None) -> Dict[str, torch.Tensor]:
        frac = self._frac if frac is None else frac
        chosen: Dict[str, torch.Tensor] = {}
        for name, shape in self._shapes.items():
            per_expert = self._found[name]
            if not per_expert:
                continue
            mags = torch.cat([per_expert[e][0] for e in sorted(per_expert)])
            gidx = torch.cat([per_expert[e][1] for e in sorted(per_expert)])
            numel = 1
            for d in shape:
                numel *= d
            k = min(max(1, int(numel * frac)), mags.numel())
            pos, _ = topk_abs(mags, k)
            chosen[name] = gidx[pos]
        return chosen

    def n_captured(self) -> int:
        return sum(len(per_expert) for per_expert in self._found.values())


def _last_position_of(sorted_keys: torch.Tensor, order: torch.Tensor, wanted: torch.Tensor) -> torch.Tensor:
    """Position in the unsorted array of the last occurrence of each wanted key
    (all present): ``sorted_keys`` = keys sorted stably, ``order`` its permutation."""
    at = torch.searchsorted(sorted_keys, wanted, right=True) - 1
    return order[at]


def reselect_active(old_idx: torch.Tensor, old_masters: torch.Tensor, new_idx: Optional[torch.Tensor],
                    entry: Any) -> Tuple[torch.Tensor, torch.Tensor, Dict[str, int]]:
    """The reference's reselect merge for one tensor (train.py:556-597) on the GPU.

    old_idx: current active flat indices; old_masters: their fp32 master values
    (aligned); new_idx: the importance pass's selection (None / empty: keep the
    old set); entry: the tensor's 4-bit entry (or dense weight) for seeding
    newly grown positions.  Returns (final_idx, final_masters, counts) with
    final_idx = sorted(old & new) followed by the smallest
    |old| - |old & new| indices of sorted(new - old), the kept positions' old
    master values (the last occurrence for a repeated old index, as the
    reference's reverse map) and the grown positions' dequantized values."""
    old = old_idx.reshape(-1).long()
    dev = old.device
    if new_idx is None or new_idx.numel() == 0:
        return old.clone(), old_masters.detach().reshape(-1).float().clone(), \
            {"kept": int(old.numel()), "dropped": 0, "grown": 0}
    new = new_idx.reshape(-1).to(dev).long()
    old_u = torch.unique(old)
    new_u = torch.unique(new)
    kept = old_u[torch.isin(old_u, new_u)]
    newcomers = new_u[~torch.isin(new_u, old_u)]
    fill = max(0, old_u.numel() - kept.numel())
    grown = newcomers[:fill]
    final = torch.cat([kept, grown])
    vals = torch.empty(final.numel(), dtype=torch.float32, device=dev)
    if kept.numel():
        sorted_old, order = torch.sort(old, stable=True)
        vals[:kept.numel()] = old_masters.detach().reshape(-1).to(dev).float()[
            _last_position_of(sorted_old, order, kept)]
    if grown.numel():
        vals[kept.numel():] = dequant_at(entry, grown, device=dev)
    counts = {"kept": int(kept.numel()), "dropped": int(old_u.numel() - kept.numel()), "grown": int(grown.numel())}
    return final, vals, counts
