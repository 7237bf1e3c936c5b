"""Routed MoE expert layer on the GPU: routing, bucketing, fused 4-bit
dequant-GEMMs, combine, and their backward, as torch autograd Functions over
the C-ABI kernels.

Numerics follow the reference's dense-masked forward
(usaf/qwen3moe_dml.py:24-86) restricted to routed tokens
(benchmarks/kaggle_t4_bench.py:253-328): activations in the layer dtype
(bf16/fp16) with each op's output rounded to it, fp32 accumulation on MFMA,
and an fp32 combine over experts in ascending expert order.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional, Tuple

import torch

from . import _native as N


# ---------------------------------------------------------------------------
# 4-bit expert tensors
# ---------------------------------------------------------------------------

@dataclass
class Q4Tensor:
    """An HBM-resident tensor in the reference's 4-bit format (quantization.py:21-85)."""
    q: torch.Tensor        # int8 [groups, ceil(gs/2)]
    s: torch.Tensor        # fp16 [groups]
    z: torch.Tensor        # fp16 [groups]
    shape: torch.Size
    group_size: int = 128
    _sz: Optional[torch.Tensor] = field(default=None, repr=False, compare=False)
    _t: Optional[Tuple[torch.Tensor, torch.Tensor]] = field(default=None, repr=False, compare=False)

    @classmethod
    def from_entry(cls, entry: Any, device=None, group_size: int = 128) -> "Q4Tensor":
        """Accepts a quantize_state_dict entry ({"q","s","z","shape"[,"group_size"]})
        or a (q, s, z, shape) tuple (moe_loader.py:203-212)."""
        if isinstance(entry, Q4Tensor):
            q, s, z, shape, gs = entry.q, entry.s, entry.z, entry.shape, entry.group_size
        elif isinstance(entry, dict) and "q" in entry:
            q, s, z, shape = entry["q"], entry["s"], entry["z"], entry["shape"]
            gs = entry.get("group_size", group_size)
        elif isinstance(entry, (tuple, list)) and len(entry) == 4:
            q, s, z, shape = entry
            gs = group_size
        else:
            raise TypeError(f"not a 4-bit entry: {type(entry).__name__}")
        dev = torch.device(device) if device is not None else (q.device if q.is_cuda else N.default_device())
        return cls(N.on_device(q, dev, torch.int8) if q.dtype != torch.uint8 else N.on_device(q.view(torch.int8), dev),
                   N.on_device(s, dev, torch.float16), N.on_device(z, dev, torch.float16),
                   torch.Size(shape), int(gs))

    @classmethod
    def quantize(cls, tensor: torch.Tensor, group_size: int = 128, device=None) -> "Q4Tensor":
        from .quantization import quantize_4bit
        q, s, z, shape = quantize_4bit(tensor, group_size, device=device)
        return cls(q, s, z, shape, group_size)

    @property
    def device(self) -> torch.device:
        return self.q.device

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.q, self.s, self.z))

    def dequantize(self, out_dtype: torch.dtype = torch.float16, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        from .quantization import dequantize_4bit
        return dequantize_4bit(self.q, self.s, self.z, self.shape, self.group_size, out_dtype=out_dtype, out=out)

    def scale_zero(self) -> torch.Tensor:
        """int32 [groups]: scale bits | zero bits << 16, the form the fused GEMMs
        read (built once, on the tensor's device)."""
        if self._sz is None or self._sz.device != self.q.device:
            sz = torch.empty(self.s.numel(), dtype=torch.int32, device=self.q.device)
            N.call("usaf_hip_pack_scale_zero", self.s.data_ptr(), self.z.data_ptr(), self.s.numel(), sz.data_ptr(),
                   N.stream_ptr(self.q.device))
            self._sz = sz
        return self._sz

    def transposed(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(codes int8 [E, cols, rows/2], scale/zero int32 [E, cols/128, rows/2, 2]):
        the copy of W^T per expert that the grad-input GEMMs read (usaf_hip_q4_transpose),
        built once on the tensor's device and kept with it."""
        if self._t is None or self._t[0].device != self.q.device:
            E, rows, cols = (int(d) for d in self.shape)
            qt = torch.empty(E * cols * rows // 2, dtype=torch.int8, device=self.q.device)
            szt = torch.empty(E * (cols // 128) * (rows // 2) * 2, dtype=torch.int32, device=self.q.device)
            N.call("usaf_hip_q4_transpose", self.q.data_ptr(), self.s.data_ptr(), self.z.data_ptr(), E, rows, cols,
                   qt.data_ptr(), szt.data_ptr(), N.stream_ptr(self.q.device))
            self._t = (qt, szt)
        return self._t

    def transposed_ok(self) -> bool:
        """True when the transposed copy exists for this shape (rows % 64 == 0 on top of fused_ok)."""
        return self.fused_ok() and int(self.shape[1]) % 64 == 0

    def fused_ok(self) -> bool:
        """True when the layout is the one the fused GEMMs read directly:
        group size 128 along whole rows (last dim % 128 == 0)."""
        return self.group_size == 128 and len(self.shape) == 3 and int(self.shape[-1]) % 128 == 0 \
            and self.q.shape[1] == 64


# grad-input GEMMs on the transposed copies: shapes and expert counts they serve
_T_MAX_E = 255


# ---------------------------------------------------------------------------
# overlays: trained values over the 4-bit weights
# ---------------------------------------------------------------------------

# the four fused 4-bit GEMMs and how each reads its weight W [E, R, C]:
#   gate_up_fwd  W = gate_up, output column n = row r (gate rows r < I pair with up rows I + r), k = column
#   down_fwd     W = down,    n = r, k = c
#   down_bwd     W = down^T (transposed copy), n = c, k = r
#   gate_up_bwd  W = gate_up^T,                n = c, k = r
_OVL_KINDS = {"gate_up": ("gate_up_fwd", "gate_up_bwd"), "down": ("down_fwd", "down_bwd")}
_OVL_CAP = 16  # entries per (wave, k-step, fragment register): one 16-bit LDS store by each of 16 lanes
_OVL_WAVES, _OVL_WORDS = 8, 64  # waves per n-tile, entry words per wave and k-step


class OverlayTooDense(ValueError):
    """A set of trained positions puts more than 16 into one fragment register's
    32 x 16 weight block of a fused GEMM: the overlay tables cannot hold it."""


def overlay_entries(kind: str, idx: torch.Tensor, shape, inter: int):
    """Where each flat position ``idx`` of an expert tensor ``shape`` = [E, R, C]
    sits in the fused GEMM ``kind``'s weight fragments, as the entry tables of
    usaf_hip_moe_*(overlay=...) name it.  Returns (word int32 [n], byte offset
    int32 [n], table words).

    The GEMM's tile unit u = (e * n_nt + nt) * 8 + w is wave w of n-tile nt of
    expert e; the wave holds 32 weight rows l32 = 0..31 (tile rows 32 w + l32),
    and per k-step of 64 contraction elements lane l32 + 32 h holds k = 32 h +
    8 j + [0, 8) of its row as fragment registers j = 0..3.  Register j goes
    through a 1 KiB image that puts lane l's copy at byte 16 l, so the weight at
    k-step offset kk = 32 h + 8 j + 2 q + b (b: low or high half of dword q)
    sits at byte (l32 + 32 h) * 16 + 4 q + 2 b of register j's image.  Tile
    rows: n-tile nt covers weight rows 256 nt + [0, 256); for the SwiGLU
    forward it covers n = 128 nt + [0, 128), wave w taking gate rows n = 128 nt
    + 16 w + [0, 16) as its rows 0-15 and the up rows I + n as rows 16-31.
    The entries of one (u, k-step, j) are ranked in position order; rank r goes
    to word (u * nk + ks) * 64 + 16 j + r (lane 16 j + r stores it).  More than
    16 positions in one register's 32 x 16 block of a wave (3 % local density)
    raise OverlayTooDense (a ValueError)."""
    E, R, C = (int(d) for d in shape)
    idx = idx.reshape(-1).to(torch.int64)
    e = torch.div(idx, R * C, rounding_mode="floor")
    rc = idx - e * (R * C)
    r = torch.div(rc, C, rounding_mode="floor")
    c = rc - r * C
    if kind == "gate_up_fwd":
        n, k, K = r, c, C
        up = (n >= inter).to(torch.int64)
        g = n - up * inter
        n_nt = (inter + 127) // 128
        nt = torch.div(g, 128, rounding_mode="floor")
        w = torch.div(g % 128, 16, rounding_mode="floor")
        l32 = 16 * up + g % 16
    else:
        if kind == "down_fwd":
            n, k, N, K = r, c, R, C
        elif kind in ("down_bwd", "gate_up_bwd"):
            n, k, N, K = c, r, C, R
        else:
            raise ValueError(f"unknown overlay kind {kind!r}")
        n_nt = (N + 255) // 256
        nt = torch.div(n, 256, rounding_mode="floor")
        w = torch.div(n % 256, 32, rounding_mode="floor")
        l32 = n % 32
    if K % 128:
        raise ValueError(f"overlay: contraction length {K} is not a multiple of 128")
    nk = K // 64
    ks = torch.div(k, 64, rounding_mode="floor")
    kk = k % 64
    lane = l32 + 32 * torch.div(kk, 32, rounding_mode="floor")
    j = torch.div(kk % 32, 8, rounding_mode="floor")
    off = lane * 16 + 4 * torch.div(kk % 8, 2, rounding_mode="floor") + 2 * (kk % 2)
    group = ((e * n_nt + nt) * _OVL_WAVES + w) * nk + ks
    key = group * 4 + j
    order = torch.argsort(key, stable=True)
    sk = key[order]
    first = torch.searchsorted(sk, sk)  # start of each key's run
    rank_sorted = torch.arange(sk.numel(), device=sk.device) - first
    rank = torch.empty_like(rank_sorted)
    rank[order] = rank_sorted
    if rank.numel() and int(rank.max()) >= _OVL_CAP:
        raise OverlayTooDense(f"overlay ({kind}): more than {_OVL_CAP} trained positions in one 32 x 16 weight "
                              f"block; use dense expert weights with overlay_scatter for such masks")
    word = group * _OVL_WORDS + 16 * j + rank
    n_words = E * n_nt * _OVL_WAVES * nk * _OVL_WORDS
    return word.to(torch.int32), off.to(torch.int32), n_words


def overlay_table(n_words: int, word: torch.Tensor, off: torch.Tensor) -> torch.Tensor:
    """Entry table with offsets set, values 0: unused words point into the dummy
    area [1024, 2048) of the wave's epilogue tile, one 16-bit slot per word."""
    dev = word.device
    table = 1024 + 2 * (torch.arange(n_words, dtype=torch.int32, device=dev) % 512)
    table[word.long()] = off
    return table


class Q4Overlay:
    """Trained values at a fixed set of flat positions of one 4-bit expert
    tensor, held as the entry tables the fused GEMMs read: the reference's
    overlay scatter of the optimizer masters into its fp16 expert weights
    (usaf/moe_loader.py:218-221, 425-443 sync_resident; train.py:666) without
    materialising the weights.  ``role`` is "gate_up" or "down"; the tables
    (forward and grad-input GEMM) are built for one activation dtype.
    ``refresh(values)`` writes new fp32 values (aligned with ``idx``, e.g. the
    SparseAdam masters) into both tables."""

    def __init__(self, role: str, idx: torch.Tensor, shape, inter: int, dtype: torch.dtype,
                 values: torch.Tensor):
        if role not in _OVL_KINDS:
            raise ValueError(f"overlay role must be 'gate_up' or 'down', got {role!r}")
        if dtype not in (torch.float16, torch.bfloat16):
            raise TypeError("overlay dtype must be fp16 or bf16 (the activation dtype)")
        dev = values.device
        self.role, self.dtype, self.shape = role, dtype, torch.Size(shape)
        self.n = int(idx.numel())
        self.tables = {}
        for kind in _OVL_KINDS[role]:
            word, off, n_words = overlay_entries(kind, idx.to(dev), shape, inter)
            # refresh order: by word, so that each cache line of the table is written in one burst
            order = torch.argsort(word)
            self.tables[kind] = (overlay_table(n_words, word, off), word[order].contiguous(),
                                 order.to(torch.int32), n_words)
        self.bad = torch.zeros(1, dtype=torch.int32, device=dev)
        self.refresh(values)

    def table(self, kind: str, dtype: torch.dtype):
        """(pointer, words) of GEMM ``kind``'s entry table."""
        if dtype != self.dtype:
            raise TypeError(f"overlay built for {self.dtype} activations, used with {dtype}")
        t = self.tables[kind][0]
        return t.data_ptr(), t.numel()

    def refresh(self, values: torch.Tensor) -> None:
        """New values (fp32 [n], on the tables' device) into both tables."""
        v = values.detach().reshape(-1)
        if v.dtype != torch.float32 or not v.is_contiguous() or v.numel() != self.n:
            raise ValueError(f"overlay refresh needs {self.n} contiguous fp32 values")
        (ta, wa, ia, na), (tb, wb, ib, nb) = (self.tables[k] for k in _OVL_KINDS[self.role])
        N.call("usaf_hip_overlay_refresh", v.data_ptr(), self.n, wa.data_ptr(), ia.data_ptr(), ta.data_ptr(), na,
               wb.data_ptr(), ib.data_ptr(), tb.data_ptr(), nb, N.dtype_code(self.dtype), self.bad.data_ptr(),
               N.stream_ptr(v.device))


class ExpertWeights:
    """The two fused expert tensors of one MoE layer, either 4-bit (Q4Tensor)
    or dense 16-bit tensors of the activation dtype:
    gate_up [E, 2I, H] and down [E, H, I] (transformers' fused layout)."""

    def __init__(self, gate_up, down):
        self.gate_up = gate_up
        self.down = down
        gs = gate_up.shape
        ds = down.shape
        if len(gs) != 3 or len(ds) != 3 or gs[0] != ds[0] or gs[2] != ds[1] or gs[1] != 2 * ds[2]:
            raise ValueError(f"expert shapes do not form gate_up [E,2I,H] / down [E,H,I]: {tuple(gs)}, {tuple(ds)}")
        self.E, self.H, self.I = int(gs[0]), int(gs[2]), int(ds[2])
        self.overlays: dict = {}  # "gate_up" / "down" -> Q4Overlay

    @property
    def is_q4(self) -> bool:
        return isinstance(self.gate_up, Q4Tensor)

    def set_overlay(self, which: str, idx: torch.Tensor, values: torch.Tensor, dtype: torch.dtype) -> "Q4Overlay":
        """Trained values ``values`` (fp32) at flat positions ``idx`` of the 4-bit
        tensor ``which`` ("gate_up" / "down"), seen by every fused GEMM from now on
        (Q4Overlay; refresh its values after each optimizer step)."""
        w = self.gate_up if which == "gate_up" else self.down
        if not isinstance(w, Q4Tensor) or not w.fused_ok():
            raise NotImplementedError("overlays apply to 4-bit weights on the fused GEMMs; scatter dense weights "
                                      "with overlay_scatter instead")
        ov = Q4Overlay(which, idx, w.shape, self.I, dtype, values)
        self.overlays[which] = ov
        return ov

    def clear_overlay(self, which: Optional[str] = None) -> None:
        if which is None:
            self.overlays.clear()
        else:
            self.overlays.pop(which, None)

    def _ovl(self, kind: str, dtype: torch.dtype):
        """(entry table pointer, words) of GEMM ``kind`` (overlay_entries), or (None, 0)."""
        ov = self.overlays.get("gate_up" if kind.startswith("gate_up") else "down")
        return (None, 0) if ov is None else ov.table(kind, dtype)

    def _ptrs_t(self, which):
        """(codes, scale/zero) pointers of the transposed 4-bit copy for the
        grad-input GEMM of `which`, or None when that path does not apply
        (dense weights, unsupported shapes)."""
        w = self.gate_up if which == "gate_up" else self.down
        if not isinstance(w, Q4Tensor) or not w.transposed_ok() or self.E > _T_MAX_E:
            return None
        # down_bwd_t: N = I, K = H; gate_up_bwd_t: N = H, K = 2I
        n, k = (self.I, self.H) if which == "down" else (self.H, 2 * self.I)
        if n % 128 or k % 128:
            return None
        qt, szt = w.transposed()
        return qt.data_ptr(), szt.data_ptr()

    def _ptrs(self, which, dtype: torch.dtype):
        w = self.gate_up if which == "gate_up" else self.down
        if isinstance(w, Q4Tensor):
            if not w.fused_ok():
                raise NotImplementedError(
                    f"fused 4-bit GEMM needs group_size 128 along whole rows (shape {tuple(w.shape)}, "
                    f"group_size {w.group_size})")
            return w.q.data_ptr(), w.scale_zero().data_ptr(), None
        if w.dtype != dtype:
            raise TypeError(f"dense expert weight dtype {w.dtype} must match the activations ({dtype})")
        if not w.is_contiguous():
            raise ValueError("dense expert weights must be contiguous")
        return None, None, w.data_ptr()


# ---------------------------------------------------------------------------
# routing and bucketing
# ---------------------------------------------------------------------------

def route_topk(logits: torch.Tensor, top_k: int, norm_topk_prob: bool, out_dtype: torch.dtype,
               with_probs: bool = True):
    """qwen3moe_dml.py:73-83 on the GPU: (weights [T,E] out_dtype, probs fp32 [T,E] or None)."""
    if logits.dim() != 2:
        raise ValueError("logits must be [T, E]")
    logits = logits.contiguous()
    T, E = logits.shape
    dev = logits.device
    weights = torch.empty(T, E, dtype=out_dtype, device=dev)
    probs = torch.empty(T, E, dtype=torch.float32, device=dev) if with_probs else None
    N.call("usaf_hip_route_topk", logits.data_ptr(), N.dtype_code(logits.dtype), T, E, int(top_k),
           1 if norm_topk_prob else 0, weights.data_ptr(), N.dtype_code(out_dtype), N.ptr(probs), N.stream_ptr(dev))
    return weights, probs


@dataclass
class Buckets:
    counts: torch.Tensor     # int32 [E]
    offsets: torch.Tensor    # int32 [E+1]
    token_idx: torch.Tensor  # int32 [S]
    slot_w: torch.Tensor     # fp32 [S]
    pair_slot: torch.Tensor  # int32 [T, E]
    n_slots: int
    blk_table: Optional[torch.Tensor] = None  # layout table of the blocked sampled-gradient operands (lazy)


def bucket_by_expert(weights: torch.Tensor, capacity: Optional[int] = None,
                     overflow: Optional[torch.Tensor] = None) -> Buckets:
    """Stable bucketing of routed pairs by expert (kaggle_t4_bench.py:293-306).

    Default: reads back the slot count once (the reference's batched path also
    syncs, on `counts.max().item()`) to size the slot buffers exactly.

    capacity + overflow (int32 [>= 1] device tensor): no host read.  The slot
    buffers hold `capacity` slots, n_slots = capacity, and the slots past the
    routed pairs carry token 0 and weight 0; pairs beyond capacity are dropped
    and set overflow[0] = 1, which the caller must check before trusting the
    step (e.g. capacity = T * top_k, exceeded only by ties at the top-k
    threshold).
    """
    weights = weights.contiguous()
    T, E = weights.shape
    dev = weights.device
    lib = N.load()
    if (capacity is None) != (overflow is None):
        raise ValueError("bucket_by_expert: give both capacity and overflow, or neither")
    if overflow is not None and (overflow.dtype != torch.int32 or overflow.device != dev or overflow.numel() < 1):
        raise ValueError("bucket_by_expert: overflow must be an int32 tensor on the weights' device")
    ws = torch.empty(max(1, int(lib.usaf_hip_bucket_workspace_ints(T, E))), dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    cap = T * E if capacity is None else int(capacity)
    token_idx = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    slot_w = torch.empty(max(cap, 1), dtype=torch.float32, device=dev)
    pair_slot = torch.empty(T, E, dtype=torch.int32, device=dev)
    N.call("usaf_hip_bucket_by_expert", weights.data_ptr(), N.dtype_code(weights.dtype), T, E, ws.data_ptr(),
           counts.data_ptr(), offsets.data_ptr(), token_idx.data_ptr(), slot_w.data_ptr(), pair_slot.data_ptr(),
           cap, N.ptr(overflow), N.stream_ptr(dev))
    S = int(offsets[E].item()) if capacity is None else cap
    return Buckets(counts, offsets, token_idx[:S], slot_w[:S], pair_slot, S)


def combine(y_slots: torch.Tensor, weights: Optional[torch.Tensor], pair_slot: torch.Tensor, dtype: torch.dtype):
    T, E = pair_slot.shape
    H = y_slots.shape[1]
    out = torch.empty(T, H, dtype=dtype, device=pair_slot.device)
    N.call("usaf_hip_moe_combine", y_slots.data_ptr(), N.ptr(weights), pair_slot.data_ptr(), T, E, H,
           N.dtype_code(dtype), out.data_ptr(), N.stream_ptr(pair_slot.device))
    return out


# ---------------------------------------------------------------------------
# grad capture (usaf/qwen3moe_dml.py:30-56 protocol)
# ---------------------------------------------------------------------------

def _sampled_blocked(capture, b: "Buckets") -> bool:
    """Whether _capture takes the blocked sampled-gradient path for this store."""
    return capture is not None and hasattr(capture[0], "add_sampled") and b.offsets.numel() - 1 <= 1024


def _capture(capture, which: str, dy: torch.Tensor, x: torch.Tensor, x_rows: Optional[torch.Tensor],
             b: "Buckets", full_shape, dtype, dy_blocked: Optional["BlockedSlots"] = None,
             x_blocked: Optional["BlockedSlots"] = None) -> None:
    """Deliver the weight gradient of ``{prefix}.{which}`` (dW_e = dy_e^T @ x_e over
    expert e's slots; x_e = x[x_rows] when x_rows is given) to the capture store.

    SparseGradStore (``add_sampled``): only the active positions, by the
    sampled-product kernel (dy_blocked / x_blocked: the operands already in
    the blocked layout of b.blk_table, written by the kernels that produced them).  Other stores get dense per-expert gradients in
    the activation dtype, as F.linear's weight grad in the reference:
    ``store.add(name, ei, g)`` or, for a dict store, accumulation into
    per-tensor fp16 CPU buffers (usaf/qwen3moe_dml.py:34-47).
    """
    store, prefix = capture
    name = f"{prefix}.{which}"
    if hasattr(store, "add_sampled"):
        if _sampled_blocked(capture, b) and _blocked_ok(dy) and _blocked_ok(x):
            if b.blk_table is None:
                b.blk_table = blocked_layout(b.offsets, b.n_slots)
            if dy_blocked is None:
                dy_blocked = slot_blocked(dy, b.offsets, b.n_slots, table=b.blk_table)
            if x_blocked is None:
                x_blocked = slot_blocked(x, b.offsets, b.n_slots, rows=x_rows, table=b.blk_table)
            store.add_sampled(name, dy_blocked, x_blocked, b.offsets, dtype)
        else:
            store.add_sampled(name, slot_major(dy), slot_major(x, rows=x_rows), b.offsets, dtype)
        return
    offs = b.offsets.tolist()
    for ei in range(len(offs) - 1):
        s0, s1 = offs[ei], offs[ei + 1]
        if s0 == s1:
            continue
        xe = x.index_select(0, x_rows[s0:s1].long()) if x_rows is not None else x[s0:s1]
        g = torch.mm(dy[s0:s1].t(), xe)  # library GEMM, dtype output as F.linear's weight grad
        if isinstance(store, dict):
            buf = store.get(name)
            if buf is None:
                buf = torch.zeros(tuple(full_shape), dtype=torch.float16, device="cpu")
                store[name] = buf
            buf[ei] += g.detach().to(device="cpu", dtype=torch.float16)
        else:
            store.add(name, ei, g)


# ---------------------------------------------------------------------------
# the routed expert layer
# ---------------------------------------------------------------------------

# Optional per-launch timing of the fused GEMMs and the sampled gradient: None,
# or a dict that collects entry-point name -> [(start, end) HIP events recorded
# on the launch stream].  bench.py sets it over its timed steps.
launch_events: Optional[dict] = None


def timed_call(name, *args):
    ev = launch_events
    if ev is None:
        N.call(name, *args)
        return
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    N.call(name, *args)
    b.record()
    ev.setdefault(name, []).append((a, b))


class RoutedExpertsFn(torch.autograd.Function):
    """out = sum_e w[:, e] * down_e(silu(gate_e(x)) * up_e(x)) over routed pairs."""

    @staticmethod
    def forward(ctx, hs: torch.Tensor, weights: torch.Tensor, ew: ExpertWeights, capture,
                w_gate_up: Optional[torch.Tensor] = None, w_down: Optional[torch.Tensor] = None,
                slots: Optional[Tuple[int, torch.Tensor]] = None, link: Optional["HsGradLink"] = None):
        # w_gate_up / w_down: the dense expert Parameters the kernels' weights were
        # taken from, passed only so that autograd delivers their gradients;
        # slots: (capacity, overflow) for bucketing without a host read (bucket_by_expert)
        dt = hs.dtype
        if dt not in (torch.float16, torch.bfloat16):
            raise TypeError(f"activations must be fp16 or bf16, got {dt}")
        hs = hs.contiguous()
        weights = weights.to(dt).contiguous()
        T, H = hs.shape
        E, I = ew.E, ew.I
        if H != ew.H or weights.shape != (T, E):
            raise ValueError(f"shape mismatch: hs {tuple(hs.shape)}, weights {tuple(weights.shape)}, "
                             f"experts E={E} H={ew.H} I={I}")
        dev = hs.device
        st = N.stream_ptr(dev)
        code = N.dtype_code(dt)
        b = bucket_by_expert(weights) if slots is None else bucket_by_expert(weights, *slots)
        S = b.n_slots
        gu = torch.empty(S, 2 * I, dtype=dt, device=dev)
        act = torch.empty(S, I, dtype=dt, device=dev)
        y = torch.empty(S, H, dtype=dt, device=dev)
        act_blk = None
        if S > 0 and _sampled_blocked(capture, b):
            # the down projection's sampled gradient reads act blocked slot-major:
            # written by the gate_up epilogue, with act
            if b.blk_table is None:
                b.blk_table = blocked_layout(b.offsets, S)
            n_blk = max(1, int(N.load().usaf_hip_blocked_elems(S, E, I)))
            act_blk = BlockedSlots(torch.empty(n_blk, dtype=dt, device=dev), I, b.offsets, b.blk_table)
        if S > 0:
            q, sz, w16 = ew._ptrs("gate_up", dt)
            timed_call("usaf_hip_moe_gate_up_fwd", hs.data_ptr(), T, H, b.token_idx.data_ptr(), b.offsets.data_ptr(),
                       S, E, I, q, sz, w16, code, gu.data_ptr(), act.data_ptr(),
                       None if act_blk is None else act_blk.data.data_ptr(),
                       None if act_blk is None else b.blk_table.data_ptr(), *ew._ovl("gate_up_fwd", dt), st)
            q, sz, w16 = ew._ptrs("down", dt)
            timed_call("usaf_hip_moe_down_fwd", act.data_ptr(), I, b.offsets.data_ptr(), S, E, H, q, sz, w16,
                       code, y.data_ptr(), *ew._ovl("down_fwd", dt), st)
        out = combine(y, weights, b.pair_slot, dt)
        ctx.ew = ew
        ctx.capture = capture
        ctx.link = link
        ctx.b = b
        ctx.act_blk = act_blk
        ctx.wdt = (None if w_gate_up is None else w_gate_up.dtype, None if w_down is None else w_down.dtype)
        ctx.save_for_backward(hs, gu, act, y)
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        hs, gu, act, y = ctx.saved_tensors
        ew, b, capture = ctx.ew, ctx.b, ctx.capture
        dt = hs.dtype
        dout = dout.to(dt).contiguous()
        T, H = hs.shape
        E, I = ew.E, ew.I
        S = b.n_slots
        dev = hs.device
        st = N.stream_ptr(dev)
        code = N.dtype_code(dt)
        dweights = torch.zeros(T, E, dtype=dt, device=dev)
        want_gu, want_dn = ctx.needs_input_grad[4], ctx.needs_input_grad[5]
        d_wgu = torch.zeros(E, 2 * I, H, dtype=ctx.wdt[0], device=dev) if want_gu else None
        d_wdn = torch.zeros(E, H, I, dtype=ctx.wdt[1], device=dev) if want_dn else None
        if S == 0:
            return torch.zeros_like(hs), dweights, None, None, d_wgu, d_wdn, None
        dcur = torch.empty(S, H, dtype=dt, device=dev)
        dcur_blk = None
        if _sampled_blocked(capture, b) and _blocked_ok(dout) and _blocked_ok(y):
            # the down projection's sampled gradient reads dcur slot-major: written here, with dcur
            if b.blk_table is None:
                b.blk_table = blocked_layout(b.offsets, S)
            lib = N.load()
            blk = torch.empty(max(1, int(lib.usaf_hip_blocked_elems(S, E, H))), dtype=dt, device=dev)
            ws = torch.empty(max(1, int(lib.usaf_hip_combine_bwd_blocked_ws_floats(S, H))), dtype=torch.float32,
                             device=dev)
            N.call("usaf_hip_moe_combine_bwd_blocked", dout.data_ptr(), y.data_ptr(), b.token_idx.data_ptr(),
                   b.slot_w.data_ptr(), b.offsets.data_ptr(), b.blk_table.data_ptr(), S, E, H, code,
                   dcur.data_ptr(), blk.data_ptr(), dweights.data_ptr(), ws.data_ptr(), st)
            dcur_blk = BlockedSlots(blk, H, b.offsets, b.blk_table)
        else:
            N.call("usaf_hip_moe_combine_bwd", dout.data_ptr(), y.data_ptr(), b.token_idx.data_ptr(),
                   b.slot_w.data_ptr(), b.offsets.data_ptr(), S, E, H, code, dcur.data_ptr(), dweights.data_ptr(), st)
        dgu = torch.empty(S, 2 * I, dtype=dt, device=dev)
        tq = ew._ptrs_t("down")
        if tq is not None:
            timed_call("usaf_hip_moe_down_bwd_t", dcur.data_ptr(), H, gu.data_ptr(), b.offsets.data_ptr(), S, E, I,
                       *tq, code, dgu.data_ptr(), *ew._ovl("down_bwd", dt), st)
        else:
            _no_overlay(ew, "down")
            q, sz, w16 = ew._ptrs("down", dt)
            timed_call("usaf_hip_moe_down_bwd", dcur.data_ptr(), H, gu.data_ptr(), b.offsets.data_ptr(), S, E, I,
                       q, sz, w16, code, dgu.data_ptr(), st)
        if capture is not None:
            _capture(capture, "down_proj", dcur, act, None, b, (E, H, I), dt, dy_blocked=dcur_blk,
                     x_blocked=ctx.act_blk)
        if want_dn:
            _dense_weight_grad(d_wdn, dcur, act, None, b)
        dx_slots = torch.empty(S, H, dtype=dt, device=dev)
        tq = ew._ptrs_t("gate_up")
        if tq is not None:
            timed_call("usaf_hip_moe_gate_up_bwd_t", dgu.data_ptr(), I, b.offsets.data_ptr(), S, E, H, *tq,
                       code, dx_slots.data_ptr(), *ew._ovl("gate_up_bwd", dt), st)
        else:
            _no_overlay(ew, "gate_up")
            q, sz, w16 = ew._ptrs("gate_up", dt)
            timed_call("usaf_hip_moe_gate_up_bwd", dgu.data_ptr(), I, b.offsets.data_ptr(), S, E, H, q, sz, w16,
                       code, dx_slots.data_ptr(), st)
        # the sum over experts right behind the GEMM that wrote dx_slots, while they
        # are still in the last-level cache (after the sampled gradient's
        # transposes they come from HBM: 35 against 26.5 us at cfg2)
        dhs = combine(dx_slots, None, b.pair_slot, dt)
        if capture is not None:
            _capture(capture, "gate_up_proj", dgu, hs, b.token_idx, b, (E, 2 * I, H), dt)
        if want_gu:
            _dense_weight_grad(d_wgu, dgu, hs, b.token_idx, b)
        if ctx.link is not None and dweights is not None:
            # the router's backward (next, it needs dweights) adds its grad-input to
            # this one in the same kernel: one sum instead of autograd's extra add
            ctx.link.dx = dhs
            dhs = None
        return dhs, dweights, None, None, d_wgu, d_wdn, None, None


def _no_overlay(ew: ExpertWeights, which: str) -> None:
    if which in ew.overlays:
        raise NotImplementedError(f"the grad-input GEMM of {which} with an overlay needs the transposed 4-bit copy "
                                  f"(E <= {_T_MAX_E}, rows % 64 == 0 and the GEMM's N, K multiples of 128)")


def _dense_weight_grad(out: torch.Tensor, dy: torch.Tensor, x: torch.Tensor, x_rows: Optional[torch.Tensor],
                       b: "Buckets") -> None:
    """out[e] = dy_e^T @ x_e for every expert with slots (fp32 products, stored in
    out's dtype): the dense expert-weight gradient autograd gives the reference's
    trainable experts (olmoe_dml.py:22-31, olmoe_streaming.py:91-97)."""
    offs = b.offsets.tolist()
    for ei in range(len(offs) - 1):
        s0, s1 = offs[ei], offs[ei + 1]
        if s0 == s1:
            continue
        xe = x.index_select(0, x_rows[s0:s1].long()) if x_rows is not None else x[s0:s1]
        out[ei] = torch.mm(dy[s0:s1].t().float(), xe.float()).to(out.dtype)


@dataclass
class BlockedSlots:
    """Per-expert blocked slot-major operand (usaf_hip_gather_transpose_blocked):
    expert e's slots form a contiguous block of `cols` rows of round_up(S_e, 16)
    elements, zero-padded, at element offset cols * sum of the padded counts of
    the experts before e."""
    data: torch.Tensor       # flat, 16-bit
    cols: int                # C: rows per expert block (features of the operand)
    offsets: torch.Tensor    # int32 [E+1] the blocks were built with
    table: torch.Tensor      # int32 layout table of those offsets (blocked_layout)


def blocked_layout(offsets: torch.Tensor, n_slots: int) -> torch.Tensor:
    """Layout table (usaf_hip_blocked_layout) of one bucketing of n_slots slots."""
    E = offsets.numel() - 1
    lib = N.load()
    table = torch.empty(int(lib.usaf_hip_blocked_table_elems(n_slots, E)), dtype=torch.int32, device=offsets.device)
    N.call("usaf_hip_blocked_layout", offsets.data_ptr(), E, n_slots, table.data_ptr(), N.stream_ptr(offsets.device))
    return table


def slot_blocked(x: torch.Tensor, offsets: torch.Tensor, n_slots: int,
                 rows: Optional[torch.Tensor] = None, table: Optional[torch.Tensor] = None) -> BlockedSlots:
    """[S or T, C] -> BlockedSlots (rows gathered by `rows` when given)."""
    C = x.shape[1]
    E = offsets.numel() - 1
    if table is None:
        table = blocked_layout(offsets, n_slots)
    elif table.numel() < int(N.load().usaf_hip_blocked_table_elems(n_slots, E)):
        raise ValueError("slot_blocked: layout table built for fewer slots")
    lib = N.load()
    out = torch.empty(max(1, int(lib.usaf_hip_blocked_elems(n_slots, E, C))), dtype=x.dtype, device=x.device)
    N.call("usaf_hip_gather_transpose_blocked", x.data_ptr(), x.stride(0), N.ptr(rows), offsets.data_ptr(),
           table.data_ptr(), n_slots, E, C, out.data_ptr(), N.stream_ptr(x.device))
    return BlockedSlots(out, C, offsets, table)


def _blocked_ok(x: torch.Tensor) -> bool:
    return x.shape[1] % 8 == 0 and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0


def slot_major(x: torch.Tensor, rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[S or T, C] -> [C, S] (rows gathered by `rows` when given), as a view of a
    [C, round_up(S, 8)] buffer: the sampled-gradient kernel reads 16-byte
    vectors along the slots."""
    C = x.shape[1]
    S = rows.numel() if rows is not None else x.shape[0]
    ld = (S + 7) // 8 * 8
    out = torch.empty(C, ld, dtype=x.dtype, device=x.device)
    N.call("usaf_hip_gather_transpose", x.data_ptr(), x.stride(0), N.ptr(rows), S, C, out.data_ptr(), ld,
           N.stream_ptr(x.device))
    return out[:, :S]


class HsGradLink:
    """Hands the experts' hidden-state gradient from RoutedExpertsFn.backward to
    RouterFn.backward of the same block (moe_block), which adds the router's
    grad-input to it in one kernel (usaf_hip_router_dx) with autograd's
    roundings; the experts' backward then returns no gradient for the hidden
    states, the router's returns the sum."""

    def __init__(self) -> None:
        self.dx: Optional[torch.Tensor] = None


def routed_experts(hs: torch.Tensor, weights: torch.Tensor, experts: ExpertWeights, capture=None,
                   weight_params: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                   slot_capacity: Optional[int] = None, overflow: Optional[torch.Tensor] = None,
                   link: Optional[HsGradLink] = None) -> torch.Tensor:
    """Experts forward with the reference signature's data: hs [T, H], weights [T, E].

    weight_params: optional (gate_up, down) dense Parameters that ``experts``
    holds (possibly as converted copies); when they require grad they receive
    dense gradients, as the reference's autograd through the expert loop.
    slot_capacity / overflow: bucket without reading the slot count back to the
    host (graph capture, no stall before the GEMMs); see bucket_by_expert.
    link: set by moe_block when the router's backward takes the hidden-state
    gradient of both branches (HsGradLink)."""
    wg, wd = weight_params if weight_params is not None else (None, None)
    slots = None if slot_capacity is None and overflow is None else (slot_capacity, overflow)
    return RoutedExpertsFn.apply(hs, weights, experts, capture, wg, wd, slots, link)


class RouteTopKFn(torch.autograd.Function):
    """Router softmax + threshold mask (+ renorm) with the kernel backward."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, top_k: int, norm: bool, out_dtype: torch.dtype):
        weights, probs = route_topk(logits, top_k, norm, out_dtype)
        ctx.top_k, ctx.norm, ctx.ldt = top_k, norm, logits.dtype
        ctx.save_for_backward(probs)
        return weights

    @staticmethod
    def backward(ctx, dweights: torch.Tensor):
        (probs,) = ctx.saved_tensors
        T, E = probs.shape
        dweights = dweights.contiguous()
        dlogits = torch.empty(T, E, dtype=ctx.ldt, device=probs.device)
        N.call("usaf_hip_route_topk_bwd", dweights.data_ptr(), N.dtype_code(dweights.dtype), probs.data_ptr(), T, E,
               ctx.top_k, 1 if ctx.norm else 0, dlogits.data_ptr(), N.dtype_code(ctx.ldt), N.stream_ptr(probs.device))
        return dlogits, None, None, None


class RouterLinearFn(torch.autograd.Function):
    """router_logits = F.linear(hs, W) (qwen3moe_dml.py:72): forward and grad-input
    by the library GEMM, the weight gradient (a contraction over the tokens) by
    usaf_hip_router_dw."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor):
        ctx.save_for_backward(x, w)
        return torch.nn.functional.linear(x, w)

    @staticmethod
    def backward(ctx, dlogits: torch.Tensor):
        x, w = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = torch.mm(dlogits, w)
        if ctx.needs_input_grad[1]:
            dw = _router_dw(x, dlogits, w.dtype)
        return dx, dw


def _router_dw(x: torch.Tensor, dlogits: torch.Tensor, w_dtype: torch.dtype) -> torch.Tensor:
    dlogits = dlogits.contiguous()
    T, E = dlogits.shape
    H = x.shape[1]
    lib = N.load()
    ws = torch.empty(max(1, int(lib.usaf_hip_router_dw_ws_floats(T, E, H))), dtype=torch.float32, device=x.device)
    dw = torch.empty(E, H, dtype=w_dtype, device=x.device)
    N.call("usaf_hip_router_dw", dlogits.data_ptr(), x.data_ptr(), T, E, H, N.dtype_code(x.dtype), dw.data_ptr(),
           ws.data_ptr(), N.stream_ptr(x.device))
    return dw


class RouterFn(torch.autograd.Function):
    """The router of qwen3moe_dml.py:72-83 from one call (usaf_hip_router_fwd):
    logits = F.linear(hs, W) in the activation dtype, fp32 softmax, top-k
    threshold mask, optional renormalisation.  Backward: usaf_hip_route_topk_bwd to
    dlogits, usaf_hip_router_dx for dhs (with the experts' dhs added in the same
    kernel when moe_block links the two), usaf_hip_router_dw for dW."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, top_k: int, norm: bool, out_dtype: torch.dtype,
                link: Optional[HsGradLink] = None):
        T, H = x.shape
        E = w.shape[0]
        logits = torch.empty(T, E, dtype=x.dtype, device=x.device)
        weights = torch.empty(T, E, dtype=out_dtype, device=x.device)
        probs = torch.empty(T, E, dtype=torch.float32, device=x.device)
        N.call("usaf_hip_router_fwd", x.data_ptr(), w.data_ptr(), T, E, H, N.dtype_code(x.dtype), int(top_k),
               1 if norm else 0, logits.data_ptr(), weights.data_ptr(), N.dtype_code(out_dtype), probs.data_ptr(),
               N.stream_ptr(x.device))
        ctx.top_k, ctx.norm, ctx.link = top_k, norm, link
        ctx.save_for_backward(x, w, probs)
        return weights

    @staticmethod
    def backward(ctx, dweights: torch.Tensor):
        x, w, probs = ctx.saved_tensors
        T, E = probs.shape
        dweights = dweights.contiguous()
        dlogits = torch.empty(T, E, dtype=x.dtype, device=x.device)
        N.call("usaf_hip_route_topk_bwd", dweights.data_ptr(), N.dtype_code(dweights.dtype), probs.data_ptr(), T, E,
               ctx.top_k, 1 if ctx.norm else 0, dlogits.data_ptr(), N.dtype_code(x.dtype), N.stream_ptr(x.device))
        dx = None
        if ctx.needs_input_grad[0]:
            # dx = dtype(dlogits @ W), plus (link) the experts' gradient of the same
            # hidden states with autograd's accumulation rounding
            link = ctx.link
            acc = link is not None and link.dx is not None
            if acc:
                dx, link.dx = link.dx, None
            elif E % 16 == 0:
                dx = torch.empty(T, x.shape[1], dtype=x.dtype, device=x.device)
            else:  # shapes the kernel does not take (moe_block links only E % 16 == 0)
                dx = torch.mm(dlogits, w)
            if acc or E % 16 == 0:
                N.call("usaf_hip_router_dx", dlogits.data_ptr(), w.data_ptr(), T, E, x.shape[1],
                       N.dtype_code(x.dtype), dx.data_ptr(), 1 if acc else 0, N.stream_ptr(x.device))
        dw = _router_dw(x, dlogits, w.dtype) if ctx.needs_input_grad[1] else None
        return dx, dw, None, None, None, None


def _router_fused_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    return (x.dtype in (torch.float16, torch.bfloat16) and w.dtype == x.dtype and x.is_contiguous()
            and w.is_contiguous() and w.shape[0] <= 1024 and x.shape[1] % 256 == 0 and x.data_ptr() % 16 == 0
            and w.data_ptr() % 16 == 0)


def _router_dw_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    return (x.dtype in (torch.float16, torch.bfloat16) and w.dtype == x.dtype and x.is_contiguous()
            and w.shape[0] % 8 == 0 and x.shape[1] % 8 == 0 and x.data_ptr() % 16 == 0)


def moe_block(hs: torch.Tensor, router_weight: torch.Tensor, top_k: int, norm_topk_prob: bool,
              experts: ExpertWeights, capture=None, overflow: Optional[torch.Tensor] = None) -> torch.Tensor:
    """qwen3moe_dml.py:67-86: the router (RouterFn: logits MFMA kernel and
    routing kernel; RouterLinearFn + RouteTopKFn for shapes it does not take),
    the routed experts; hs [B, S, H] or [T, H].  The two branches' gradients of
    the hidden states are summed by the router's grad-input kernel (HsGradLink).

    overflow: optional int32 device tensor.  Given, the experts are bucketed
    into T * (top_k + 1) slots with no host read of the slot count, and
    overflow[0] is set to 1 if the routing selected more pairs: the caller
    checks it and recomputes without `overflow`.  The threshold mask selects
    more than top_k experts for a token whose k-th and (k+1)-th probabilities
    tie, which 16-bit logits make common; the spare T slots absorb that, and
    slots past the routed pairs cost no GEMM work."""
    shape = hs.shape
    x = hs.reshape(-1, shape[-1])
    link = None
    if _router_fused_ok(x, router_weight):
        # the router's backward sums both branches' hidden-state gradients (HsGradLink)
        link = HsGradLink() if (x.requires_grad and router_weight.shape[0] % 16 == 0) else None
        weights = RouterFn.apply(x, router_weight, top_k, norm_topk_prob, x.dtype, link)
    else:
        if _router_dw_ok(x, router_weight):
            logits = RouterLinearFn.apply(x, router_weight)
        else:
            logits = torch.nn.functional.linear(x, router_weight)
        weights = RouteTopKFn.apply(logits, top_k, norm_topk_prob, x.dtype)
    cap = None if overflow is None else x.shape[0] * min(top_k + 1, router_weight.shape[0])
    out = routed_experts(x, weights, experts, capture, slot_capacity=cap, overflow=overflow, link=link)
    return out.view(shape)
