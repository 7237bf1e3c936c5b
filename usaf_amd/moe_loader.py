"""HBM-resident quantized expert cache and sparse gradient stores.

Drop-in for usaf/moe_loader.py.  Differences of placement, not of interface:

* ``QuantizedExpertCache`` keeps every 4-bit entry in HBM (the reference keeps
  them in CPU RAM) and fills its LRU of fp16 expert copies with the dequant
  kernel instead of a CPU dequant + PCIe copy.  ``get_q4`` additionally hands
  the 4-bit tensors to the fused expert GEMMs.  Resident copies of trainable
  layers and their overlays also live in HBM.
* ``SparseGradStore`` keeps its compact fp32 gradients in HBM and accepts
  sampled gradients straight from the fused backward (``add_sampled``) besides
  the reference's dense per-expert ``add``.
"""
from __future__ import annotations

import fnmatch
import functools
from collections import OrderedDict
from typing import Any, Dict, List, Optional, Tuple, Union

import torch
import torch.nn as nn

from . import _native as N
from .importance import TopKImportanceStore  # noqa: F401  (moe_loader.py:584-631, GPU selection)
from .expert_cache import ExpertSlotCache
from .moe import ExpertWeights, OverlayTooDense, Q4Overlay, Q4Tensor, timed_call
from .olmoe_streaming import _record_grad, apply_captured_expert_grads  # noqa: F401  (moe_loader.py:778-802)
from .quantization import dequantize_4bit


def save_quantized_state_dict(q_dict: Dict[str, Any], path: str, *, _use_new_zipfile_serialization: bool = True
                              ) -> None:
    """moe_loader.py:25-37: torch.save of the quantized dict (tensors moved to CPU first)."""
    def cpu(x):
        if isinstance(x, torch.Tensor):
            return x.detach().cpu()
        if isinstance(x, dict):
            return {k: cpu(v) for k, v in x.items()}
        if isinstance(x, tuple):
            return tuple(cpu(v) for v in x)
        return x
    torch.save(cpu(q_dict), path, _use_new_zipfile_serialization=_use_new_zipfile_serialization)


def load_quantized_state_dict(path: str, map_location: Union[str, torch.device] = "cpu") -> Dict[str, Any]:
    """moe_loader.py:40-57 (weights_only load; raises TypeError if not a dict)."""
    loaded = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(loaded, dict):
        raise TypeError(f"Expected quantized state dict (dict), got {type(loaded).__name__}")
    return loaded


def _is_q4_entry(entry) -> bool:
    return isinstance(entry, Q4Tensor) or (isinstance(entry, dict) and "q" in entry) or \
        (isinstance(entry, tuple) and len(entry) == 4)


class QuantizedExpertCache:
    """LRU of dequantized fp16 expert modules over an HBM-resident 4-bit store.

    Mirrors moe_loader.py:60-524.  Keys are expert module names
    (``model.layers.L.mlp.experts``); each holds that module's parameters
    (``gate_up_proj``, ``down_proj``).

    Args:
        quantized_dict: output of ``quantize_state_dict`` (dict or tuple entries);
                        moved to ``device`` once.
        device:         GPU holding the 4-bit store and the fp16 copies.
        max_cached:     LRU size in expert modules.
        group_size:     group size of the 4-bit entries.
        max_cached_bytes: optional byte cap on the fp16 LRU (checked with max_cached).
        dtype:          dtype of the dequantized copies (fp16 as the reference, or bf16).
    """

    def __init__(self, quantized_dict: Dict[str, Any], device: torch.device, max_cached: int = 2,
                 group_size: int = 128, *, max_cached_bytes: Optional[int] = None,
                 dtype: torch.dtype = torch.float16) -> None:
        N.require_gpu()
        self._device = torch.device(device)
        if self._device.type != "cuda":
            raise ValueError("QuantizedExpertCache holds its store in GPU memory; pass a cuda device")
        self._max_cached = max(max_cached, 1)
        self._max_bytes = max_cached_bytes
        self._group_size = group_size
        self._dtype = dtype
        self._q_dict: Dict[str, Any] = {}
        for name, entry in quantized_dict.items():
            if _is_q4_entry(entry):
                self._q_dict[name] = Q4Tensor.from_entry(entry, self._device, group_size)
            elif isinstance(entry, torch.Tensor):
                self._q_dict[name] = entry.detach().to(self._device)
            else:
                self._q_dict[name] = entry
        self._cache: "OrderedDict[str, Dict[str, torch.Tensor]]" = OrderedDict()
        self.overlays: Dict[str, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._prefetched: Dict[str, Tuple[Dict[str, torch.Tensor], torch.cuda.Event]] = {}
        self._prefetch_stream: Optional[torch.cuda.Stream] = None
        self._prefetch_disabled = False
        self._expert_to_params: Dict[str, List[Tuple[str, str]]] = {}
        self._build_index()
        self._resident: Dict[str, Dict[str, torch.Tensor]] = {}
        self._resident_active = False
        # fused path: trained values of 4-bit tensors as the fused GEMMs read them
        # (FusedOverlay: Q4Overlay tables, or a dense copy for over-dense masks),
        # built from ``overlays`` / sync_resident for this activation dtype
        self.fused_overlays: Dict[str, "FusedOverlay"] = {}
        self.fused_dtype: Optional[torch.dtype] = None
        # fused views whose values were written from the masters since the last
        # evict_all: the reference re-applies ``overlays`` with their current values
        # whenever a module is dequantized again after an eviction, so a fused view
        # not in this set takes the current values at its next access
        self._fused_fresh: set = set()
        # optional per-expert LRU of dequantized copies (make_slot_cache), used by
        # forwards that need no gradients through layers without trained values
        self.slot_cache: Optional[ExpertSlotCache] = None
        self.hits = 0
        self.misses = 0

    # ---- indexing -----------------------------------------------------------------

    def _build_index(self) -> None:
        """moe_loader.py:111-128: group keys by expert module name."""
        e2p: Dict[str, List[Tuple[str, str]]] = {}
        for full_name in self._q_dict:
            parts = full_name.rsplit(".", 1)
            if len(parts) != 2:
                continue
            e2p.setdefault(parts[0], []).append((full_name, parts[1]))
        self._expert_to_params = e2p

    # ---- 4-bit access for the fused path --------------------------------------------

    def get_q4(self, expert_module_name: str) -> Dict[str, Any]:
        """The weights the fused GEMMs read for a module, by local name: the HBM
        4-bit tensor (Q4Tensor), or the dense copy of a tensor whose trained
        positions are too dense for overlay tables, or a dense entry."""
        self._fused_from_overlays(expert_module_name)
        out = {}
        for full_name, local in self._expert_to_params.get(expert_module_name, []):
            fo = self.fused_overlays.get(full_name)
            if fo is not None and fo.dense is not None:
                out[local] = fo.dense
                continue
            entry = self._q_dict.get(full_name)
            if entry is not None:
                out[local] = entry
        return out

    def get_q4_overlays(self, expert_module_name: str) -> Dict[str, Any]:
        """The overlay tables (Q4Overlay) of a module's 4-bit tensors, by local name."""
        self._fused_from_overlays(expert_module_name)
        out = {}
        for full_name, local in self._expert_to_params.get(expert_module_name, []):
            fo = self.fused_overlays.get(full_name)
            if fo is not None and fo.ov is not None:
                out[local] = fo.ov
        return out

    # ---- dequantized copies --------------------------------------------------------

    def _nbytes(self, params: Dict[str, torch.Tensor]) -> int:
        return sum(t.numel() * t.element_size() for t in params.values())

    def _dequant(self, expert_module_name: str, stream=None, skip=()) -> Dict[str, torch.Tensor]:
        """HBM dequant of a module's params with overlays applied (moe_loader.py:183-224);
        params named in ``skip`` are left out."""
        out: Dict[str, torch.Tensor] = {}
        ctx = torch.cuda.stream(stream) if stream is not None else torch.cuda.device(self._device)
        with ctx:
            for full_name, local in self._expert_to_params.get(expert_module_name, []):
                if local in skip:
                    continue
                entry = self._q_dict.get(full_name)
                if isinstance(entry, Q4Tensor):
                    t = entry.dequantize(self._dtype)
                elif isinstance(entry, torch.Tensor):
                    t = entry.to(self._dtype).clone()
                else:
                    continue
                ov = self.overlays.get(full_name)
                if ov is not None:
                    overlay_scatter(t, ov[0], ov[1])
                out[local] = t
        return out

    # the reference's name for the same step (it ran on the CPU there)
    _dequant_cpu = _dequant

    def _get_resident(self, expert_module_name: str) -> Dict[str, torch.Tensor]:
        """moe_loader.py:226-247: resident base with overlays applied (a fresh copy)."""
        out = {}
        for local, base in self._resident[expert_module_name].items():
            t = base.clone()
            ov = self.overlays.get(f"{expert_module_name}.{local}")
            if ov is not None:
                overlay_scatter(t, ov[0], ov[1])
            out[local] = t
        return out

    def _evict_for(self, incoming_bytes: int) -> None:
        while self._cache and (len(self._cache) >= self._max_cached or (
                self._max_bytes is not None and
                sum(self._nbytes(p) for p in self._cache.values()) + incoming_bytes > self._max_bytes)):
            self._cache.popitem(last=False)

    def get_expert_weights(self, expert_module_name: str) -> Dict[str, torch.nn.Parameter]:
        """moe_loader.py:130-181: fp16 Parameters of a module on the GPU (LRU)."""
        if expert_module_name in self._cache:
            self.hits += 1
            self._cache.move_to_end(expert_module_name)
            cached = self._cache[expert_module_name]
            return {p: torch.nn.Parameter(t, requires_grad=t.requires_grad) for p, t in cached.items()}
        self.misses += 1
        if expert_module_name in self._resident:
            # resident modules join the cache without evicting others (moe_loader.py:153-164);
            # only params the resident copy lacks are dequantized
            params = self._get_resident(expert_module_name)
            params.update(self._dequant(expert_module_name, skip=params.keys()))
        else:
            pending = self._prefetched.pop(expert_module_name, None)
            if pending is not None:
                params, ev = pending
                torch.cuda.current_stream(self._device).wait_event(ev)
                for t in params.values():
                    t.record_stream(torch.cuda.current_stream(self._device))
            else:
                params = self._dequant(expert_module_name)
            self._evict_for(self._nbytes(params))
        self._cache[expert_module_name] = params
        return {p: torch.nn.Parameter(t, requires_grad=True) for p, t in params.items()}

    def free_frozen(self, detach_at: int) -> None:
        """moe_loader.py:249-261: drop 4-bit entries of layers 0..detach_at."""
        for li in range(detach_at + 1):
            prefix = f"model.layers.{li}."
            for key in list(self._q_dict.keys()):
                if key.startswith(prefix):
                    del self._q_dict[key]
            name = f"model.layers.{li}.mlp.experts"
            self._expert_to_params.pop(name, None)
            self._prefetched.pop(name, None)
            if self.slot_cache is not None:
                self.slot_cache.drop_layer(name)

    def make_slot_cache(self, max_bytes: int, dtype: Optional[torch.dtype] = None) -> ExpertSlotCache:
        """A per-expert LRU of dequantized copies in one HBM arena of ``max_bytes``
        (ExpertSlotCache) over every module whose gate_up/down are 4-bit: the
        reference's dequant-on-demand cache at expert granularity, copies made
        when the routing first selects a missing expert.  ``dtype``: of the
        copies, the activation dtype of the forwards it serves (default the
        fused path's, else fp16)."""
        layers = {}
        for name in self._expert_to_params:
            gu, dn = self._q_dict.get(f"{name}.gate_up_proj"), self._q_dict.get(f"{name}.down_proj")
            if isinstance(gu, Q4Tensor) and isinstance(dn, Q4Tensor) and gu.fused_ok() and dn.fused_ok():
                layers[name] = ExpertWeights(gu, dn)
        if not layers:
            raise ValueError("make_slot_cache: no module holds 4-bit gate_up_proj and down_proj")
        dt = dtype or self.fused_dtype or torch.float16
        self.slot_cache = ExpertSlotCache(layers, self._device, max_bytes, dtype=dt)
        return self.slot_cache

    def make_resident(self, train_layers, dequant_batch: int = 8, only_params=None) -> None:
        """moe_loader.py:263-299: dequantize trainable layers once into HBM fp16."""
        self._resident_active = False
        for li in sorted(train_layers):
            name = f"model.layers.{li}.mlp.experts"
            entries = self._expert_to_params.get(name)
            if not entries:
                continue
            res: Dict[str, torch.Tensor] = {}
            for full_name, local in entries:
                if only_params is not None and local not in only_params:
                    continue
                entry = self._q_dict.get(full_name)
                if isinstance(entry, Q4Tensor):
                    res[local] = entry.dequantize(self._dtype)
                elif isinstance(entry, torch.Tensor):
                    res[local] = entry.to(self._dtype).clone()
            self._resident[name] = res
        self._resident_active = True

    def setup_vk_dequant(self, train_layers) -> None:
        """moe_loader.py:301-350 uploaded codes to Vulkan buffers; the codes already
        live in HBM here and the dequant kernel always runs on the GPU."""
        return None

    def setup_vk_streaming(self, max_layers: int = 999) -> None:
        """moe_loader.py:352-409 counterpart; nothing to upload (see setup_vk_dequant)."""
        return None

    def apply_resident_overlays(self, active_idx, masters) -> None:
        """moe_loader.py:411-423: scatter master values into the resident copies
        (and into the fused GEMMs' view of the 4-bit tensors)."""
        self._sync_fused(active_idx, masters)
        self._scatter_masters(active_idx, masters)

    def sync_resident(self, active_idx, masters) -> None:
        """moe_loader.py:425-443: propagate optimizer masters into the resident copies
        and, for 4-bit tensors the fused GEMMs read (setup_quantized_streaming with
        fused=True), into their overlay tables."""
        self._sync_fused(active_idx, masters)
        if not self._resident_active:
            return
        self._scatter_masters(active_idx, masters)

    # ---- the fused GEMMs' view of the trained values -----------------------------------

    def _fused_target(self, fname: str) -> Optional[Q4Tensor]:
        entry = self._q_dict.get(fname)
        local = fname.rsplit(".", 1)[-1]
        if (self.fused_dtype is None or not isinstance(entry, Q4Tensor) or local not in ("gate_up_proj", "down_proj")
                or not entry.fused_ok()):
            return None
        return entry

    def _sticky(self, fname: str) -> bool:
        """Whether a position dropped from the active set keeps its last trained
        value: the reference scatters masters into its resident copies in place
        (moe_loader.py:411-443), so a resident tensor keeps every value it was
        ever given, while a streamed one is re-dequantized with the current
        overlays only (moe_loader.py:183-224)."""
        name, local = fname.rsplit(".", 1)
        return self._resident_active and name in self._resident and local in self._resident[name]

    def _sync_one(self, fname: str, aidx: torch.Tensor, vals, refresh: bool) -> None:
        """Make the fused view of ``fname`` hold ``vals`` at ``aidx``: refresh the
        values when the positions are the ones it was built for (``refresh``, or
        when ``vals`` is another tensor than last time), otherwise rebuild it.
        The view then counts as written since the last evict_all."""
        entry = self._fused_target(fname)
        if entry is None:
            return
        fo = self.fused_overlays.get(fname)
        v = vals.data if isinstance(vals, torch.nn.Parameter) else vals
        v = v.detach().reshape(-1).to(device=self._device, dtype=torch.float32).contiguous()
        self._fused_fresh.add(fname)
        if fo is not None and fo.same_positions(aidx):
            if refresh or fo.vals_src is not vals:
                fo.refresh(v)
                fo.vals_src = vals
            return
        retired = fo.retired_after(aidx) if (fo is not None and self._sticky(fname)) else None
        local = fname.rsplit(".", 1)[-1]
        self.fused_overlays[fname] = FusedOverlay(entry, local.replace("_proj", ""), aidx, v, self.fused_dtype,
                                                  retired)
        self.fused_overlays[fname].vals_src = vals

    def _sync_fused(self, active_idx, masters) -> None:
        if self.fused_dtype is None:
            return
        for fname, aidx in active_idx.items():
            if fname in masters:
                self._sync_one(fname, aidx, masters[fname], refresh=True)

    def _fused_from_overlays(self, expert_module_name: str) -> None:
        """Before a fused forward: the trained values set in ``overlays`` (the
        trainer sets them at start-up, after a resume and after a reselect,
        train.py:467, 607) reach the fused view of each 4-bit tensor, with the
        values they hold now when the view was not written since the last
        evict_all (the reference dequantizes an evicted module again with the
        current overlay values, moe_loader.py:183-247); a view written since
        (sync_resident, an earlier access) is not rewritten."""
        if self.fused_dtype is None:
            return
        for full_name, _ in self._expert_to_params.get(expert_module_name, []):
            ov = self.overlays.get(full_name)
            if ov is not None:
                self._sync_one(full_name, ov[0], ov[1], refresh=full_name not in self._fused_fresh)

    def _scatter_masters(self, active_idx, masters) -> None:
        for fname, aidx in active_idx.items():
            parts = fname.rsplit(".", 1)
            if len(parts) != 2:
                continue
            name, local = parts
            if name not in self._resident or local not in self._resident[name]:
                continue
            overlay_scatter(self._resident[name][local], aidx, masters[fname].data)

    def prefetch(self, expert_module_name: str) -> None:
        """moe_loader.py:445-471: dequantize ahead on a side stream."""
        if self._prefetch_disabled:
            return
        if (expert_module_name in self._cache or expert_module_name in self._prefetched
                or expert_module_name not in self._expert_to_params or expert_module_name in self._resident):
            return
        if self._prefetch_stream is None:
            self._prefetch_stream = torch.cuda.Stream(device=self._device)
        self._prefetch_stream.wait_stream(torch.cuda.current_stream(self._device))
        params = self._dequant(expert_module_name, stream=self._prefetch_stream)
        ev = torch.cuda.Event()
        ev.record(self._prefetch_stream)
        self._prefetched[expert_module_name] = (params, ev)

    def clear_prefetch(self) -> None:
        """moe_loader.py:473-486: drop pending prefetches (waiting for them)."""
        for _, ev in self._prefetched.values():
            ev.synchronize()
        self._prefetched.clear()

    def evict(self, expert_module_name: str) -> None:
        self._cache.pop(expert_module_name, None)

    def evict_all(self) -> None:
        self._cache.clear()
        self._fused_fresh.clear()

    @property
    def cached_experts(self) -> List[str]:
        return list(reversed(self._cache.keys()))

    @property
    def device(self) -> torch.device:
        return self._device

    def estimate_vram_mb(self) -> float:
        """MiB held by the fp16 LRU (moe_loader.py:506-512)."""
        return sum(self._nbytes(p) for p in self._cache.values()) / (1024 * 1024)

    def estimate_cpu_mb(self) -> float:
        """MiB of the 4-bit store (moe_loader.py:514-524; it sits in HBM here)."""
        total = 0
        for entry in self._q_dict.values():
            if isinstance(entry, Q4Tensor):
                total += entry.nbytes()
            elif isinstance(entry, torch.Tensor):
                total += entry.numel() * entry.element_size()
        return total / (1024 * 1024)


class FusedOverlay:
    """Trained values over one HBM 4-bit expert tensor as the fused GEMMs read
    them: its Q4Overlay tables (``ov``) or, when the positions are too dense
    for the tables (OverlayTooDense), a dense copy of the weights in the
    activation dtype (``dense``: dequant to fp16, the masters scattered as
    fp16, converted -- the reference's fp16 weights after its scatter,
    moe_loader.py:218-221, in the activation dtype).

    ``idx`` / ``vals``: the active positions and their fp32 masters (aligned);
    ``retired``: optional (positions, values) kept from an earlier set
    (QuantizedExpertCache._sticky).  ``refresh(vals)`` writes new masters."""

    def __init__(self, entry: Q4Tensor, role: str, idx: torch.Tensor, vals: torch.Tensor, dtype: torch.dtype,
                 retired: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
        dev = entry.device
        # index tensors known to hold these positions, with their versions (the
        # trainer passes the same positions as several tensor objects)
        self._known = [(idx, idx._version)]
        self.active = idx.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
        self.n_active = int(self.active.numel())
        if vals.numel() != self.n_active:
            raise ValueError(f"overlay has {self.n_active} positions and {vals.numel()} values")
        if retired is not None and retired[0].numel():
            self.positions = torch.cat([self.active, retired[0]])
            self.values = torch.cat([vals, retired[1]])
        else:
            self.positions = self.active
            self.values = vals.clone()
        self.vals_src = None
        shape = entry.shape
        inter = int(shape[1]) // 2 if role == "gate_up" else int(shape[2])
        self.ov: Optional[Q4Overlay] = None
        self.dense: Optional[torch.Tensor] = None
        try:
            self.ov = Q4Overlay(role, self.positions, shape, inter, dtype, self.values)
        except OverlayTooDense:
            base = entry.dequantize(torch.float16)
            overlay_scatter(base, self.positions, self.values)
            self.dense = base if dtype == torch.float16 else base.to(dtype)

    def same_positions(self, idx: torch.Tensor) -> bool:
        """Whether ``idx`` names the active positions this view was built for (the
        same tensor, unmodified, or equal values)."""
        if any(idx is t and idx._version == v for t, v in self._known):
            return True
        if idx.numel() != self.n_active:
            return False
        same = bool(torch.equal(idx.reshape(-1).to(device=self.active.device, dtype=torch.int64), self.active))
        if same:
            self._known = [(t, v) for t, v in self._known if t._version == v][-3:] + [(idx, idx._version)]
        return same

    def retired_after(self, new_idx: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(positions, values) of this view that ``new_idx`` does not name."""
        new = new_idx.reshape(-1).to(device=self.positions.device, dtype=torch.int64)
        keep = ~torch.isin(self.positions, new)
        return self.positions[keep], self.values[keep]

    def refresh(self, vals: torch.Tensor) -> None:
        """New fp32 masters of the active positions (aligned with ``idx``)."""
        if vals.numel() != self.n_active:
            raise ValueError(f"overlay refresh needs {self.n_active} values, got {vals.numel()}")
        self.values[:self.n_active].copy_(vals.reshape(-1))
        if self.ov is not None:
            self.ov.refresh(self.values)
        else:
            # dtype(fp16(master)): the fp16 value is exact in fp32
            overlay_scatter(self.dense, self.positions, self.values.half().float())


def overlay_scatter(base: torch.Tensor, idx: torch.Tensor, vals: torch.Tensor) -> None:
    """base.flat[idx] = base.dtype(vals) on the GPU (moe_loader.py:218-221)."""
    if not base.is_contiguous():
        raise ValueError("overlay target must be contiguous")
    dev = base.device
    idx = idx.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    vals = vals.detach().reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    if idx.numel() != vals.numel():
        raise ValueError(f"overlay has {idx.numel()} indices and {vals.numel()} values")
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    N.call("usaf_hip_overlay_scatter", base.data_ptr(), N.dtype_code(base.dtype), base.numel(), idx.data_ptr(),
           vals.data_ptr(), idx.numel(), bad.data_ptr(), N.stream_ptr(dev))
    if bool(bad.item()):
        raise IndexError("overlay index out of range")


class SparseGradStore:
    """Compact fp32 gradients at the active positions of each expert tensor, in HBM.

    Mirrors moe_loader.py:527-581 (``compact``, ``zero_``, ``add``,
    ``n_captured``).  ``add_sampled`` is the fused path: it receives the
    slot-major operands of a weight gradient from the expert backward and
    computes only the active entries (usaf_hip_sddmm_masked).
    """

    def __init__(self, active_idx: Dict[str, torch.Tensor], shapes: Dict[str, Any], device=None) -> None:
        dev = torch.device(device) if device is not None else N.default_device()
        self.device = dev
        self._compact: Dict[str, torch.Tensor] = {}
        self._zero_pending: set = set()
        self._csr: Dict[str, tuple] = {}
        self._maps: Dict[str, Dict[int, Tuple[torch.Tensor, torch.Tensor]]] = {}
        # the compact gradients are consecutive slices of one buffer (``flat``), so
        # that a whole-store pass (finite check, copy) is one launch
        self.spans: Dict[str, Tuple[int, int]] = {}
        total = 0
        for name, idx in active_idx.items():
            self.spans[name] = (total, int(idx.numel()))
            total += int(idx.numel())
        self._flat = torch.zeros(total, dtype=torch.float32, device=dev)
        for name, idx in active_idx.items():
            idx = idx.reshape(-1).to(device=dev, dtype=torch.long)
            shape = [int(s) for s in shapes[name]]
            start, n = self.spans[name]
            self._compact[name] = self._flat[start:start + n]
            if len(shape) < 2:
                raise ValueError(f"{name}: expert tensors are [E, rows, ...], got shape {shape}")
            E, R = shape[0], shape[1]
            C = 1
            for s in shape[2:]:
                C *= s
            order = torch.argsort(idx, stable=True)
            sidx = idx[order]
            identity = bool(torch.equal(order, torch.arange(idx.numel(), device=dev)))
            rows = torch.div(sidx, C, rounding_mode="floor")
            cols = (sidx - rows * C).to(torch.int32)
            if E * R >= 2 ** 31 or C >= 2 ** 31:
                raise ValueError(f"{name}: rows E*R and columns C must fit in int32, shape {shape}")
            row_ptr = torch.zeros(E * R + 1, dtype=torch.int64, device=dev)
            if idx.numel():
                if int(sidx[0]) < 0 or int(sidx[-1]) >= E * R * C:
                    raise IndexError(f"{name}: active index out of range for shape {shape}")
                row_ptr[1:] = torch.cumsum(torch.bincount(rows, minlength=E * R), 0)
            if E > 1024 or R >= 2 ** 21:
                raise ValueError(f"{name}: the sampled-gradient kernel needs E <= 1024 and rows < 2^21, shape {shape}")
            e_of = torch.div(rows, R, rounding_mode="floor")
            row_code = ((e_of << 21) | (rows - e_of * R)).to(torch.int32).contiguous()  # e << 21 | o
            self._csr[name] = (row_ptr, row_code, cols.contiguous(), None if identity else order.contiguous(), E, R, C)

    @property
    def compact(self) -> Dict[str, torch.Tensor]:
        """name -> compact fp32 gradient (moe_loader.py:541-562)."""
        for name in list(self._zero_pending):
            self._materialize(name)
        return self._compact

    @property
    def flat(self) -> torch.Tensor:
        """All compact gradients as one fp32 buffer: ``compact[name]`` is
        ``flat[start:start + n]`` with ``(start, n) = spans[name]``."""
        for name in list(self._zero_pending):
            self._materialize(name)
        return self._flat

    def _materialize(self, name: str) -> None:
        if name in self._zero_pending:
            self._zero_pending.discard(name)
            self._compact[name].zero_()

    def zero_(self) -> None:
        """Zero every compact gradient.  The zeroing is deferred: the first
        sampled add into a tensor writes 0 + sum instead of accumulating, so a
        step that fills the store from the fused backward launches no fill."""
        self._zero_pending = set(self._compact)

    def add_sampled(self, full_name: str, rowT: torch.Tensor, colT: torch.Tensor, offsets: torch.Tensor,
                    dtype: torch.dtype) -> None:
        """compact[name] += dtype(rowT[o, slots_e] . colT[i, slots_e]) at each active (e, o, i).

        rowT / colT: slot-major operands [R or C, >= S] (usaf_amd.moe.slot_major), or
        usaf_amd.moe.BlockedSlots built with the same offsets (usaf_amd.moe.slot_blocked)."""
        csr = self._csr.get(full_name)
        if csr is None:
            return
        _, row_code, cols, pos_map, E, R, C = csr
        if not isinstance(rowT, torch.Tensor):  # BlockedSlots
            if rowT.cols != R or colT.cols != C:
                raise ValueError(f"{full_name}: blocked operands of {rowT.cols} / {colT.cols} rows do not match "
                                 f"the weight rows {R} x cols {C}")
            if rowT.offsets.data_ptr() != offsets.data_ptr() or colT.offsets.data_ptr() != offsets.data_ptr():
                raise ValueError(f"{full_name}: blocked operands were built with other expert offsets")
            first = full_name in self._zero_pending
            timed_call("usaf_hip_sddmm_blocked", rowT.data.data_ptr(), colT.data.data_ptr(), rowT.table.data_ptr(), E,
                       R, C, cols.numel(), row_code.data_ptr(), cols.data_ptr(), N.ptr(pos_map), N.dtype_code(dtype),
                       self._compact[full_name].data_ptr(), 0 if first else 1, N.stream_ptr(self.device))
            self._zero_pending.discard(full_name)
            return
        if rowT.shape[0] != R or colT.shape[0] != C or rowT.shape[1] != colT.shape[1]:
            raise ValueError(f"{full_name}: operands {tuple(rowT.shape)} / {tuple(colT.shape)} do not match "
                             f"the weight rows {R} x cols {C}")
        ldT = rowT.stride(0)
        if rowT.stride(1) != 1 or colT.stride(1) != 1 or colT.stride(0) != ldT or ldT % 8:
            raise ValueError("slot-major operands need unit column stride and one row stride, a multiple of 8 "
                             "(use usaf_amd.moe.slot_major)")
        self._materialize(full_name)
        N.call("usaf_hip_sddmm_masked", rowT.data_ptr(), colT.data_ptr(), ldT, offsets.data_ptr(), E, R, C,
               cols.numel(), row_code.data_ptr(), cols.data_ptr(), N.ptr(pos_map), N.dtype_code(dtype),
               self._compact[full_name].data_ptr(), N.stream_ptr(self.device))

    def add(self, full_name: str, ei: int, g: torch.Tensor) -> None:
        """Reference protocol (moe_loader.py:564-578): dense grad of expert ei."""
        csr = self._csr.get(full_name)
        if csr is None:
            return
        row_ptr, _, cols, pos_map, E, R, C = csr
        ei = int(ei)
        p0, p1 = int(row_ptr[ei * R]), int(row_ptr[(ei + 1) * R])
        if p0 == p1:
            return
        rows = torch.searchsorted(row_ptr, torch.arange(p0, p1, device=row_ptr.device), right=True) - 1
        local = (rows - ei * R) * C + cols[p0:p1].long()
        pos = pos_map[p0:p1] if pos_map is not None else torch.arange(p0, p1, device=row_ptr.device)
        vals = g.detach().to(self.device).reshape(-1).gather(0, local).float()
        self._materialize(full_name)
        self._compact[full_name].index_add_(0, pos, vals)

    def n_captured(self) -> int:
        return len(self._compact)


def setup_quantized_streaming(model: nn.Module, quantized_dict: Dict[str, Any], device: torch.device, *,
                              max_cached_experts: int = 2, group_size: int = 128,
                              expert_pattern: str = "*.mlp.experts", verbose: bool = True,
                              fused: bool = True, expert_cache_bytes: Optional[int] = None) -> nn.Module:
    """moe_loader.py:650-769.  The expert modules lose their Parameters (their
    weights live in the cache's HBM 4-bit store); everything else moves to the
    GPU in place.  Each expert module gets a pre-hook that attaches its HBM 4-bit
    tensors (``module._usaf_q4``, read by the fused forward) -- or, with
    ``fused=False``, dequantized fp16 Parameters from the LRU as the reference
    does, their gradients captured into ``model._expert_grads`` -- and a
    post-hook that detaches them again.  ``expert_cache_bytes`` (fused path):
    also keep a per-expert LRU of dequantized copies of that size
    (QuantizedExpertCache.make_slot_cache, attached as ``module._usaf_slots``);
    the patched experts forward runs on the copies when it needs no gradients
    and the module has no trained values, and on the fused 4-bit GEMMs
    otherwise."""
    cache = QuantizedExpertCache(quantized_dict, device=device, max_cached=max_cached_experts,
                                 group_size=group_size)
    expert_names = [name for name, _ in model.named_modules() if fnmatch.fnmatch(name, expert_pattern)]
    experts = set(expert_names)
    for name, mod in model.named_modules():
        if name in experts:
            mod._parameters.clear()
    resident = [p for p in model.parameters()]
    model.to(device)
    if verbose:
        nbytes = sum(p.numel() * p.element_size() for p in resident)
        print(f"  GPU (resident): {len(resident)} tensors, {nbytes / 1e9:.2f}GB")
        print(f"  HBM (4-bit):    {len(quantized_dict)} entries, ~{cache.estimate_cpu_mb() / 1024:.2f}GiB")
    state: Dict[str, int] = {"resident": 0, "max": 0}
    grads: Dict[str, torch.Tensor] = {}
    model._expert_grads = grads

    if fused:
        dtypes = {p.dtype for p in resident if p.is_floating_point()}
        act = torch.bfloat16 if torch.bfloat16 in dtypes else torch.float16
        cache.fused_dtype = act  # the overlay tables hold trained values in the activation dtype
        if expert_cache_bytes:
            cache.make_slot_cache(int(expert_cache_bytes), act)

    def attach(mod_name: str):
        def pre_hook(module: nn.Module, _args) -> None:
            if fused:
                module._usaf_q4 = cache.get_q4(mod_name)
                module._usaf_q4_overlays = cache.get_q4_overlays(mod_name)
                # the copies hold the plain 4-bit values: modules with trained values
                # (overlay tables or a dense fallback) stay on the fused path
                sc = cache.slot_cache
                trained = any(n in cache.fused_overlays for n, _ in cache._expert_to_params.get(mod_name, []))
                module._usaf_slots = (sc, mod_name) if sc is not None and mod_name in sc.layers and not trained \
                    else None
            else:
                for pname, param in cache.get_expert_weights(mod_name).items():
                    module._parameters[pname] = param
                    param.register_post_accumulate_grad_hook(
                        functools.partial(_record_grad, grads, f"{mod_name}.{pname}"))
            state["resident"] += 1
            state["max"] = max(state["max"], state["resident"])
        return pre_hook

    def detach(module: nn.Module, _args, output):
        module._parameters.clear()
        module._usaf_q4 = None
        module._usaf_q4_overlays = None
        module._usaf_slots = None
        state["resident"] -= 1
        return output

    model._stream_state = state
    for name, mod in model.named_modules():
        if name in experts:
            mod.register_forward_pre_hook(attach(name))
            mod.register_forward_hook(detach)
    model._quantized_cache = cache
    return model


def get_quantized_cache(model: nn.Module) -> Optional[QuantizedExpertCache]:
    return getattr(model, "_quantized_cache", None)


def load_and_stream(model: nn.Module, quantized_path: str, device: torch.device, **stream_kwargs: Any) -> nn.Module:
    """moe_loader.py:805-824."""
    return setup_quantized_streaming(model, load_quantized_state_dict(quantized_path), device, **stream_kwargs)
