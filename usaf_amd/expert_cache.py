"""Per-expert LRU of dequantized copies in one HBM slot arena.

The reference's ``QuantizedExpertCache`` keeps whole expert modules (one MoE
layer's fused gate_up/down tensors, 1.2 GB in fp16) in an LRU and dequantizes
a module on the CPU when it is missing (usaf/moe_loader.py:130-181).  On an
MI355X every layer's 4-bit weights stay resident in HBM (15.4 GB for the 48
layers of Qwen3-30B-A3B) and the copies are per expert:

* one arena of ``n_slots`` slots is allocated once (``max_bytes`` of HBM, at
  most one slot per expert of the model); a slot holds one expert's
  dequantized gate_up [2I, H] and down [H, I] slices in the activation dtype;
* ``touch(layer, experts)`` applies the reference's LRU policy to the keys
  (layer, expert) in the given order -- a hit moves the key to the most
  recent end, a miss takes a free slot or evicts the least recently used key
  -- and fills every missed slot with one batched dequant launch per tensor
  (usaf_hip_dequant_q4_slices_frag), reading the 4-bit slices from HBM;
* ``forward`` buckets the tokens first and touches only the experts the
  routing selected (one host read of the per-expert counts): a copy is made
  on demand, when an expert is used and missing, as the reference dequantizes
  a module when its forward asks for it (usaf/moe_loader.py:130-181);
* the layer's slot table (int32 [E] on the device) then feeds the arena
  GEMMs (usaf_hip_moe_gate_up_fwd_slots / _down_fwd_slots), so no expert is
  ever copied into a contiguous [E, ...] tensor.

A slot is written in the order the arena GEMMs read it
(usaf_hip_dequant_q4_slices_frag): the four 16-byte weight registers each
lane of a wave loads per 64-wide k-step sit next to each other, so every load
instruction of the GEMM reads 1 KiB in a row instead of 64 rows' worth of
cache lines.  ``copy_of`` gives a slot back in natural [rows, cols] order.

Copies hold the reference's fp16 dequantized values (dtype fp16, the default,
with fp16 activations) or their bf16 rounding (dtype bf16, for bf16
activations: the MFMA operands of one product share a type).  A layer's
experts must fit the arena together (n_slots >= E), so a touch never evicts a
key it inserted itself.  Slot tables of layers that lost experts to eviction
are refreshed by their next touch, which every forward starts with.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Dict, Iterable, List, Optional, Tuple

import torch

from . import _native as N
from .moe import ExpertWeights, Q4Tensor, bucket_by_expert, combine


class ExpertSlotCache:
    def __init__(self, layers: Dict[str, ExpertWeights], device, max_bytes: int,
                 dtype: torch.dtype = torch.float16) -> None:
        if not layers:
            raise ValueError("ExpertSlotCache needs at least one layer")
        self.device = torch.device(device)
        self.dtype = dtype
        first = next(iter(layers.values()))
        self.E, self.H, self.I = first.E, first.H, first.I
        for name, ew in layers.items():
            if not ew.is_q4 or (ew.E, ew.H, ew.I) != (self.E, self.H, self.I):
                raise ValueError(f"{name}: every layer must hold 4-bit experts of one shape")
            for q in (ew.gate_up, ew.down):
                if not q.fused_ok():
                    raise ValueError(f"{name}: the slot cache needs group size 128 along whole rows")
        self.layers = dict(layers)
        if self.H % 128 or self.I % 128:
            raise ValueError("the slot cache needs hidden and intermediate sizes that are multiples of 128")
        # fragment-order slots: rows padded to whole GEMM tiles
        self.gu_elems = int(N.load().usaf_hip_frag_slot_elems(2 * self.I, self.H, self.I))
        self.dn_elems = int(N.load().usaf_hip_frag_slot_elems(self.H, self.I, 0))
        elem = torch.empty(0, dtype=dtype).element_size()
        self.slot_bytes = (self.gu_elems + self.dn_elems) * elem
        self.n_slots = int(min(len(layers) * self.E, max_bytes // self.slot_bytes))
        if self.n_slots < self.E:
            raise ValueError(f"max_bytes={max_bytes} holds {self.n_slots} expert slots; one layer needs {self.E}")
        self.gu_arena = torch.empty(self.n_slots, self.gu_elems, dtype=dtype, device=self.device)
        self.dn_arena = torch.empty(self.n_slots, self.dn_elems, dtype=dtype, device=self.device)
        self._lru: "OrderedDict[Tuple[str, int], int]" = OrderedDict()
        self._free: List[int] = list(range(self.n_slots - 1, -1, -1))
        self._host_tables: Dict[str, List[int]] = {n: [0] * self.E for n in layers}
        self._tables: Dict[str, torch.Tensor] = {n: torch.zeros(self.E, dtype=torch.int32, device=self.device)
                                                  for n in layers}
        self.hits = self.misses = self.evictions = 0
        self.dequant_bytes = 0
        self.dequant_events: Optional[list] = None  # set to a list to time the fill launches

    # ---- bookkeeping ------------------------------------------------------------

    @property
    def cached_keys(self) -> List[Tuple[str, int]]:
        """(layer, expert) keys, least recently used first."""
        return list(self._lru.keys())

    def slot_of(self, layer: str, expert: int) -> Optional[int]:
        return self._lru.get((layer, int(expert)))

    def nbytes(self) -> int:
        return self.n_slots * self.slot_bytes

    def drop_layer(self, layer: str) -> None:
        """Forget a layer (its 4-bit weights are being freed): its copies' slots
        return to the free list."""
        if layer not in self.layers:
            return
        for key in [k for k in self._lru if k[0] == layer]:
            self._free.append(self._lru.pop(key))
        del self.layers[layer], self._host_tables[layer], self._tables[layer]

    def touch(self, layer: str, experts: Optional[Iterable[int]] = None) -> torch.Tensor:
        """Mark ``experts`` (default: all of the layer's) used, in order; dequantize
        the misses; return the layer's slot table (int32 [E], device)."""
        if layer not in self.layers:
            raise KeyError(layer)
        order = range(self.E) if experts is None else [int(e) for e in experts]
        missed: List[Tuple[int, int]] = []
        for e in order:
            key = (layer, e)
            slot = self._lru.get(key)
            if slot is not None:
                self._lru.move_to_end(key)
                self.hits += 1
                continue
            self.misses += 1
            if self._free:
                slot = self._free.pop()
            else:
                _, slot = self._lru.popitem(last=False)
                self.evictions += 1
            self._lru[key] = slot
            missed.append((e, slot))
        if missed:
            self._fill(layer, missed)
            table = self._host_tables[layer]
            for e, slot in missed:
                table[e] = slot
            staged = torch.tensor(table, dtype=torch.int32).pin_memory()
            self._tables[layer].copy_(staged, non_blocking=True)
        return self._tables[layer]

    def _fill(self, layer: str, missed: List[Tuple[int, int]]) -> None:
        ew = self.layers[layer]
        jobs = torch.tensor([[e for e, _ in missed], [s for _, s in missed]], dtype=torch.int64).pin_memory()
        jobs = jobs.to(self.device, non_blocking=True)
        st = N.stream_ptr(self.device)
        ev = self.dequant_events
        if ev is not None:
            a = torch.cuda.Event(enable_timing=True)
            a.record()
        for q, arena, rows, k, inter in ((ew.gate_up, self.gu_arena, 2 * self.I, self.H, self.I),
                                         (ew.down, self.dn_arena, self.H, self.I, 0)):
            N.call("usaf_hip_dequant_q4_slices_frag", q.q.data_ptr(), q.s.data_ptr(), q.z.data_ptr(), self.E, rows, k,
                   inter, len(missed), jobs[0].data_ptr(), jobs[1].data_ptr(), self.n_slots, arena.data_ptr(),
                   N.dtype_code(self.dtype), st)
        if ev is not None:
            b = torch.cuda.Event(enable_timing=True)
            b.record()
            ev.append((a, b, len(missed)))
        # algorithmic bytes: codes + scale/zero in, dequantized copies out
        n = len(missed) * 3 * self.H * self.I
        self.dequant_bytes += int(n * (0.5 + 4.0 / 128 + torch.empty(0, dtype=self.dtype).element_size()))
        # keep the job tensor alive until the launches have read it
        self._last_jobs = jobs

    def copy_of(self, slot: int, role: str) -> torch.Tensor:
        """Slot ``slot``'s copy of the gate_up [2I, H] or down [H, I] slice, in
        natural row order (for checks; the arena holds fragment order)."""
        if role == "gate_up":
            arena, rows, k, inter = self.gu_arena, 2 * self.I, self.H, self.I
        elif role == "down":
            arena, rows, k, inter = self.dn_arena, self.H, self.I, 0
        else:
            raise ValueError(role)
        idx = frag_chunk_index(rows, k, inter).to(arena.device)
        frag = arena[slot].view(-1, 8)
        keep = idx >= 0
        out = torch.empty(rows * k // 8, 8, dtype=arena.dtype, device=arena.device)
        out[idx[keep]] = frag[keep]
        return out.view(rows, k)

    # ---- forward --------------------------------------------------------------------

    def forward(self, layer: str, hs: torch.Tensor, weights: torch.Tensor,
                top_k: Optional[int] = None) -> torch.Tensor:
        """The routed experts of ``layer`` (qwen3moe_dml.py:24-64, forward only) on
        the cached copies: hs [T, H] and routing weights [T, E] in the cache dtype.
        Only the experts the routing selected are touched (and filled when
        missing), in ascending expert order.  ``top_k`` sizes the slot buffers
        for T * (top_k + 1) routed pairs without a host read of the slot count
        (bucket_by_expert's capacity mode); a routing beyond that, or no
        ``top_k``, buckets exactly."""
        if hs.dtype != self.dtype or weights.dtype != self.dtype:
            raise TypeError("activations and routing weights must be in the cache dtype")
        T = hs.shape[0]
        if top_k is not None:
            cap = T * min(top_k + 1, self.E)
            overflow = torch.zeros(1, dtype=torch.int32, device=self.device)
            b = bucket_by_expert(weights, cap, overflow)
            counts = b.counts.cpu()  # the one host read: which experts the routing selected
            if int(counts.sum()) > cap:
                b = bucket_by_expert(weights)
        else:
            b = bucket_by_expert(weights)
            counts = b.counts.cpu()
        table = self.touch(layer, counts.nonzero().reshape(-1).tolist())
        S = b.n_slots
        st = N.stream_ptr(self.device)
        code = N.dtype_code(self.dtype)
        gu = torch.empty(S, 2 * self.I, dtype=self.dtype, device=self.device)
        act = torch.empty(S, self.I, dtype=self.dtype, device=self.device)
        y = torch.empty(S, self.H, dtype=self.dtype, device=self.device)
        N.call("usaf_hip_moe_gate_up_fwd_slots", hs.data_ptr(), T, self.H, b.token_idx.data_ptr(),
               b.offsets.data_ptr(), S, self.E, self.I, self.gu_arena.data_ptr(), table.data_ptr(), self.n_slots,
               code, gu.data_ptr(), act.data_ptr(), st)
        N.call("usaf_hip_moe_down_fwd_slots", act.data_ptr(), self.I, b.offsets.data_ptr(), S, self.E, self.H,
               self.dn_arena.data_ptr(), table.data_ptr(), self.n_slots, code, y.data_ptr(), st)
        return combine(y, weights, b.pair_slot, self.dtype)


def frag_chunk_index(w_rows: int, K: int, inter: int) -> torch.Tensor:
    """For each 16-byte chunk of a fragment-order slot, the natural chunk
    (row * K / 8 + col / 8) it holds, or -1 for padding rows: chunk
    c = (((nt * 8 + w) * nk + ks) * 4 + j) * 64 + l holds row wrow(nt, w, l),
    columns 64 ks + 32 (l >> 5) + 8 j + [0, 8)."""
    nk = K // 64
    n_nt = (inter + 127) // 128 if inter > 0 else (w_rows + 255) // 256
    nt = torch.arange(n_nt).view(-1, 1, 1, 1, 1)
    w = torch.arange(8).view(1, -1, 1, 1, 1)
    ks = torch.arange(nk).view(1, 1, -1, 1, 1)
    j = torch.arange(4).view(1, 1, 1, -1, 1)
    lane = torch.arange(64).view(1, 1, 1, 1, -1)
    if inter > 0:
        n = nt * 128 + 16 * w + (lane & 15)
        valid = n < inter
        row = torch.where((lane & 16) != 0, inter, 0) + n
    else:
        row = nt * 256 + 32 * w + (lane & 31)
        valid = row < w_rows
    col8 = ks * 8 + 4 * (lane >> 5) + j
    idx = row * (K // 8) + col8
    return torch.where(valid, idx, -1).reshape(-1)


def q4_expert_slice(q: Q4Tensor, expert: int, dtype: torch.dtype) -> torch.Tensor:
    """Expert ``expert``'s dequantized slice of a 4-bit [E, rows, cols] tensor
    (for checks): the codec's dequant of that expert's groups."""
    E, rows, cols = (int(d) for d in q.shape)
    per = rows * cols // q.group_size
    sub = Q4Tensor(q.q[expert * per:(expert + 1) * per], q.s[expert * per:(expert + 1) * per],
                   q.z[expert * per:(expert + 1) * per], torch.Size([rows, cols]), q.group_size)
    return sub.dequantize(dtype)
