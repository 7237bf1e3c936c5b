"""SparseAdam over the active elements, with state in HBM.

Drop-in for usaf/sparse_optim.py (same constructor, step/refresh/reselect/
state_dict surface).  The update itself is one HIP kernel per parameter
(``usaf_hip_sparse_adam_step``) over the compact fp32 vectors; the m/v state
lives on the parameter's device instead of the CPU.
"""
from __future__ import annotations

import torch

from . import _native as N


class SparseAdam:
    """Adam (L2 weight decay folded into the gradient) on flat active indices.

    ``compact_params=True``: each named parameter is itself the compact fp32
    vector aligned with ``active_idx`` (the training script's masters).
    ``compact_params=False``: parameters are full tensors; the active elements
    are gathered, updated and scattered back.
    """

    def __init__(
        self,
        named_params: dict[str, torch.nn.Parameter],
        active_mask: dict[str, torch.Tensor] | None = None,
        active_idx: dict[str, torch.Tensor] | None = None,
        lr: float = 1e-4,
        betas: tuple = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.01,
        compact_params: bool = False,
    ):
        self.compact_params = compact_params
        self.lr = lr
        self.betas = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self._named: dict[str, torch.nn.Parameter] = dict(named_params)
        self._step = 0
        # device-gated steps (step(finite=..., halt=...)): the applied-step count
        # lives on the GPU, with a table of the bias corrections of steps 1..cap
        self._count: torch.Tensor | None = None
        self._bias: torch.Tensor | None = None
        self._launched = 0  # gated launches so far: an upper bound of the device count
        self.bad = None
        self._active_ids: list[str] = []
        self._idx: dict[str, torch.Tensor] = {}
        self._m: dict[str, torch.Tensor] = {}
        self._v: dict[str, torch.Tensor] = {}
        if active_idx is not None:
            self._build_state_from_idx(active_idx)
        else:
            self._build_state(active_mask or {})

    def _device_of(self, name: str) -> torch.device:
        p = self._named[name]
        return p.device if p.is_cuda else N.default_device()

    def _init_slot(self, name: str, idx: torch.Tensor) -> None:
        dev = self._device_of(name)
        self._active_ids.append(name)
        self._idx[name] = idx.to(dev)
        self._m[name] = torch.zeros(idx.numel(), device=dev, dtype=torch.float32)
        self._v[name] = torch.zeros(idx.numel(), device=dev, dtype=torch.float32)

    def _pack_moments(self) -> None:
        """m and v of all active tensors as consecutive slices of one buffer each
        (when they share a device), so that a step over masters and gradients laid
        out the same way is one launch."""
        names = self._active_ids
        if len(names) < 2 or len({self._m[n].device for n in names}) != 1:
            return
        for state in (self._m, self._v):
            flat = torch.cat([state[n] for n in names])
            start = 0
            for n in names:
                k = state[n].numel()
                state[n] = flat[start:start + k]
                start += k

    def _build_state_from_idx(self, active_idx: dict[str, torch.Tensor]):
        """sparse_optim.py:43-53."""
        self._active_ids, self._idx, self._m, self._v = [], {}, {}, {}
        for name, idx in active_idx.items():
            if name not in self._named or idx is None or idx.numel() == 0:
                continue
            self._init_slot(name, idx.reshape(-1).to(dtype=torch.long))
        self._pack_moments()

    def _build_state(self, active_mask: dict[str, torch.Tensor]):
        """sparse_optim.py:55-68."""
        self._active_ids, self._idx, self._m, self._v = [], {}, {}, {}
        for name in self._named:
            mask = active_mask.get(name)
            if mask is None:
                continue
            idx = mask.reshape(-1).to(dtype=torch.bool).nonzero(as_tuple=False).reshape(-1)
            if idx.numel() == 0:
                continue
            self._init_slot(name, idx)
        self._pack_moments()

    def zero_grad(self, set_to_none: bool = False):
        for name in self._active_ids:
            param = self._named[name]
            if param.grad is not None:
                if set_to_none:
                    param.grad = None
                else:
                    param.grad.zero_()

    def _gate_state(self, dev: torch.device) -> None:
        """Device step count and a bias-correction table covering every step a
        gated launch can reach (grown by doubling; the growth copies from the host)."""
        if self._count is None:
            self._count = torch.full((1,), self._step, dtype=torch.int32, device=dev)
            self._launched = self._step
            self.bad = torch.zeros(1, dtype=torch.int32, device=dev)
        need = self._launched + 1
        cap = 0 if self._bias is None else self._bias.numel() // 2
        if need > cap:
            cap = max(4096, 2 * cap)
            while cap < need:
                cap *= 2
            beta1, beta2 = self.betas
            # the reference's Python-float scalars, used by fp32 tensor ops as fp32
            tab = [x for t in range(1, cap + 1) for x in (1 - beta1 ** t, 1 - beta2 ** t)]
            self._bias = torch.tensor(tab, dtype=torch.float32).to(dev)

    @property
    def step_count(self) -> int:
        """Steps applied so far (reads the device count after gated steps)."""
        return int(self._count.item()) if self._count is not None else self._step

    def step(self, compact_grads: dict[str, torch.Tensor] | None = None, finite: torch.Tensor | None = None,
             halt: torch.Tensor | None = None):
        """One Adam step over the active elements (sparse_optim.py:86-134).

        compact_grads: optional name -> 1-D gradient aligned with ``active_idx``
        (e.g. ``SparseGradStore.compact``), used instead of ``param.grad``.
        finite / halt: optional int32 GPU flags; given (or after the first such
        call), the step is decided on the device -- applied only if finite[0] != 0
        and halt[0] == 0, the trainer's finite gate (train.py:649-672) -- and the
        step count and bias corrections live on the GPU, so the update can be
        launched before the host has read the flags.
        """
        for t, what in ((finite, "finite"), (halt, "halt")):
            if t is not None and (not t.is_cuda or t.dtype != torch.int32 or t.numel() < 1):
                raise TypeError(f"SparseAdam: {what} must be an int32 GPU tensor")
        gated = finite is not None or halt is not None or self._count is not None
        if not gated:
            self._step += 1
        beta1, beta2 = self.betas
        jobs = []  # (name, target, grad) per active tensor with a gradient
        for name in self._active_ids:
            param = self._named[name]
            if compact_grads is None and param.grad is None:
                continue
            dev = param.device
            if not param.is_cuda:
                raise RuntimeError(f"SparseAdam: parameter {name} must live on the GPU")
            if compact_grads is not None:
                g = compact_grads.get(name)
                if g is None:
                    continue
                grad = g.detach().to(device=dev, dtype=torch.float32).contiguous()
            else:
                grad = param.grad.detach().reshape(-1).index_select(0, self._idx[name]).float().contiguous()
            if self.compact_params:
                if param.dtype != torch.float32 or not param.is_contiguous():
                    raise TypeError("compact_params=True needs contiguous fp32 parameters (the masters)")
                target = param.data
            else:
                target = param.data.reshape(-1).index_select(0, self._idx[name]).float().contiguous()
            if grad.numel() != target.numel():
                raise ValueError(f"SparseAdam: gradient for {name} has {grad.numel()} entries, expected "
                                 f"{target.numel()}")
            jobs.append((name, target, grad))
        # the update is elementwise with one set of hyperparameters: tensors whose
        # masters, gradients, m and v are each consecutive slices of one buffer
        # (in the same order) take one launch over the whole span
        runs = []
        for job in jobs:
            if runs and self.compact_params and self._follows(runs[-1][-1], job):
                runs[-1].append(job)
            else:
                runs.append([job])
        for run in runs:
            name, target, grad = run[0]
            dev = target.device
            n = sum(t.numel() for _, t, _ in run)
            if gated:
                self._gate_state(dev)
                N.call("usaf_hip_sparse_adam_step_gated", target.data_ptr(), grad.data_ptr(),
                       self._m[name].data_ptr(), self._v[name].data_ptr(), n, float(self.lr),
                       float(beta1), float(beta2), float(self.eps), float(self.weight_decay), N.ptr(finite),
                       N.ptr(halt), self._count.data_ptr(), self._bias.data_ptr(), self._bias.numel() // 2,
                       self.bad.data_ptr(), N.stream_ptr(dev))
            else:
                N.call("usaf_hip_sparse_adam_step", target.data_ptr(), grad.data_ptr(), self._m[name].data_ptr(),
                       self._v[name].data_ptr(), n, float(self.lr), float(beta1), float(beta2),
                       float(self.eps), float(self.weight_decay), self._step, N.stream_ptr(dev))
            if not self.compact_params:
                param = self._named[name]
                flat = param.data.reshape(-1)
                flat.scatter_(0, self._idx[name], target.to(param.dtype))
        if gated and self._count is not None:
            N.call("usaf_hip_count_step", N.ptr(finite), N.ptr(halt), self._count.data_ptr(),
                   N.stream_ptr(self._count.device))
            self._launched += 1

    def _follows(self, prev, job) -> bool:
        """Whether job's master, gradient, m and v start right where prev's end."""
        (pn, pt, pg), (n, t, g) = prev, job
        k = 4 * pt.numel()
        return (t.device == pt.device and t.data_ptr() == pt.data_ptr() + k and g.data_ptr() == pg.data_ptr() + k
                and self._m[n].data_ptr() == self._m[pn].data_ptr() + k
                and self._v[n].data_ptr() == self._v[pn].data_ptr() + k)

    def refresh(self, model):
        """Re-bind current model Parameters by name (sparse_optim.py:136-150)."""
        current = dict(model.named_parameters())
        for name in self._active_ids:
            if name not in current:
                continue
            if current[name].numel() != self._named[name].numel():
                continue
            self._named[name] = current[name]

    def reselect(self, named_params: dict[str, torch.nn.Parameter], new_active_mask: dict[str, torch.Tensor]):
        self._named = dict(named_params)
        self._build_state(new_active_mask)

    def state_dict(self) -> dict:
        """m/v/step for checkpoints (CPU copies, as the reference stores them)."""
        return {
            "step": self.step_count,
            "m": {n: t.detach().cpu().clone() for n, t in self._m.items()},
            "v": {n: t.detach().cpu().clone() for n, t in self._v.items()},
        }

    def load_state_dict(self, sd: dict) -> None:
        self._step = int(sd["step"])
        if self._count is not None:
            self._count.fill_(self._step)
            self._launched = self._step
        # copied into the existing moment slices, so that tensors packed into one
        # buffer (_pack_moments) keep their one-launch step after a resume
        for n, t in sd["m"].items():
            if n in self._m and t.numel() == self._m[n].numel():
                self._m[n].copy_(t.detach().reshape(-1).to(self._m[n].device, torch.float32))
        for n, t in sd["v"].items():
            if n in self._v and t.numel() == self._v[n].numel():
                self._v[n].copy_(t.detach().reshape(-1).to(self._v[n].device, torch.float32))

    @property
    def num_active_params(self) -> int:
        return sum(idx.numel() for idx in self._idx.values())

    @property
    def optimizer_memory_mb(self) -> float:
        total = 0
        for name in self._active_ids:
            total += self._m[name].numel() * 4 + self._v[name].numel() * 4
        return total / (1024 * 1024)


class MomentumSGD:
    """torch.optim.SGD(params, lr, momentum, weight_decay) -- dampening 0, no
    Nesterov -- as the reference trainer steps the router (train.py:493-498,
    667-672), one fused kernel per tensor (usaf_hip_sgd_momentum_step) with the
    single-tensor path's per-op rounding.  Parameters without a gradient are
    skipped, as torch does."""

    def __init__(self, params, lr: float, momentum: float = 0.0, weight_decay: float = 0.0):
        self.params = [p for p in params]
        if lr < 0 or momentum < 0 or weight_decay < 0:
            raise ValueError("MomentumSGD: lr, momentum and weight_decay must be >= 0")
        self.lr, self.momentum, self.weight_decay = float(lr), float(momentum), float(weight_decay)
        self._buf: dict[int, torch.Tensor] = {}

    def zero_grad(self, set_to_none: bool = True) -> None:
        for p in self.params:
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    @torch.no_grad()
    def step(self, finite: torch.Tensor | None = None, halt: torch.Tensor | None = None,
             loss_scale: "DeviceLossScale | None" = None) -> None:
        """One step.  ``finite`` / ``halt``: optional int32 GPU flags read by the
        kernel, which skips the update unless finite[0] != 0 and halt[0] == 0 --
        the trainer's finite gate (train.py:649-672) decided on the device, so
        the step can be launched before the host has read the flag.  A tensor's
        first step (which creates its momentum buffer, as torch does) reads the
        gate on the host instead.  ``loss_scale``: the gradients carry that
        device loss scale and are divided by loss_scale * ACCUM (rounded to the
        dtype) before the update, as train.py:669-670 does on the host."""
        for t, what in ((finite, "finite"), (halt, "halt")):
            if t is not None and (not t.is_cuda or t.dtype != torch.int32 or t.numel() < 1):
                raise TypeError(f"MomentumSGD: {what} must be an int32 GPU tensor")
        scale_ptr = None if loss_scale is None else loss_scale.state.data_ptr()
        accum = 1.0 if loss_scale is None else float(loss_scale.accum)
        for i, p in enumerate(self.params):
            g = p.grad
            if g is None:
                continue
            if not p.is_cuda or not p.is_contiguous() or not g.is_contiguous() or g.dtype != p.dtype:
                raise RuntimeError("MomentumSGD: parameters and gradients must be contiguous GPU tensors of one dtype")
            if self.momentum == 0.0:
                raise NotImplementedError("MomentumSGD: momentum 0 (plain SGD) is not on the fused path")
            buf = self._buf.get(i)
            first = buf is None
            gate_f = gate_h = None
            if first:
                if (finite is not None and int(finite[0]) == 0) or (halt is not None and int(halt[0]) != 0):
                    continue
                buf = torch.empty_like(p)
                self._buf[i] = buf
            else:
                gate_f = finite.data_ptr() if finite is not None else None
                gate_h = halt.data_ptr() if halt is not None else None
            N.call("usaf_hip_sgd_momentum_step", p.data_ptr(), g.data_ptr(), buf.data_ptr(), p.numel(),
                   N.dtype_code(p.dtype), self.lr, self.momentum, self.weight_decay, 1 if first else 0,
                   gate_f, gate_h, scale_ptr, accum, N.stream_ptr(p.device))


class DeviceLossScale:
    """The trainer's dynamic loss scale with its state on the GPU.

    train.py keeps ``loss_scale`` (LOSS_SCALE_INIT = 4096, :31), ``good_streak``
    and ``n_skipped`` as host variables: the backward runs on ``loss *
    loss_scale`` (:351-353); the compact gradients and the router gradient are
    divided by ``loss_scale * ACCUM`` (:661, :669-670); a finite step counts as
    good and every SCALE_UP_EVERY-th (200) good step doubles the scale, capped at
    65536 (:673-674); a skipped step halves it, floored at 64 (:676).  Here the
    three live in one int32[4] device buffer (``state``: scale as fp32 bits,
    good steps, skipped steps), so a loop that launches step n + 1 before it
    reads step n's finite flag keeps the same schedule:

    * ``scale_grad(g)``: g * loss_scale in g's dtype (the scaled loss's gradient
      seed, usaf_hip_loss_scale_apply);
    * ``unscale_check(flat, out, finite)``: out = flat / (loss_scale * ACCUM) and
      finite[0] = 0 if any result is not finite (usaf_hip_scale_check_state);
    * ``MomentumSGD.step(..., loss_scale=self)``: the router gradient divided the same way;
    * ``update(finite, halt)``: the schedule for that step, launched after the
      step's gated updates (usaf_hip_loss_scale_update).
    """

    def __init__(self, init_scale: float = 4096.0, scale_up_every: int = 200, min_scale: float = 64.0,
                 max_scale: float = 65536.0, accum: int = 1, device=None):
        dev = torch.device(device) if device is not None else N.default_device()
        if scale_up_every < 1 or not (0 < min_scale <= max_scale) or accum < 1:
            raise ValueError("DeviceLossScale: need scale_up_every >= 1, 0 < min_scale <= max_scale, accum >= 1")
        self.scale_up_every, self.min_scale, self.max_scale = int(scale_up_every), float(min_scale), float(max_scale)
        self.accum = int(accum)
        self.state = torch.zeros(4, dtype=torch.int32, device=dev)
        self.state[:1].view(torch.float32).fill_(float(init_scale))

    @property
    def device(self) -> torch.device:
        return self.state.device

    def scale_grad(self, g: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """g * loss_scale in g's dtype (fp16 / bf16); ``out`` may be g itself."""
        if g.dtype not in (torch.float16, torch.bfloat16) or not g.is_contiguous() or g.device != self.device:
            raise TypeError("DeviceLossScale.scale_grad: contiguous fp16/bf16 tensor on the scale's device")
        out = torch.empty_like(g) if out is None else out
        if out.shape != g.shape or out.dtype != g.dtype or not out.is_contiguous():
            raise ValueError("DeviceLossScale.scale_grad: out must match g")
        N.call("usaf_hip_loss_scale_apply", g.data_ptr(), out.data_ptr(), g.numel(), N.dtype_code(g.dtype),
               self.state.data_ptr(), N.stream_ptr(self.device))
        return out

    def unscale_check(self, flat: torch.Tensor, out: torch.Tensor, finite: torch.Tensor) -> None:
        """out = flat / (loss_scale * ACCUM); finite[0] = 0 if any result is inf/NaN
        (the caller sets finite[0] = 1 beforehand)."""
        for t in (flat, out):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device != self.device:
                raise TypeError("DeviceLossScale.unscale_check: contiguous fp32 tensors on the scale's device")
        if out.numel() != flat.numel() or finite.dtype != torch.int32 or not finite.is_cuda:
            raise ValueError("DeviceLossScale.unscale_check: out must match flat; finite is an int32 GPU flag")
        N.call("usaf_hip_scale_check_state", flat.data_ptr(), out.data_ptr(), flat.numel(), self.state.data_ptr(),
               float(self.accum), finite.data_ptr(), N.stream_ptr(self.device))

    def update(self, finite: torch.Tensor | None = None, halt: torch.Tensor | None = None) -> None:
        """The schedule for the step whose flag is finite[0] (None = finite); a
        halted step (halt[0] != 0) leaves the state unchanged."""
        N.call("usaf_hip_loss_scale_update", self.state.data_ptr(), N.ptr(finite), N.ptr(halt),
               self.scale_up_every, self.min_scale, self.max_scale, N.stream_ptr(self.device))

    @property
    def loss_scale(self) -> float:
        """The current scale (a host read)."""
        return float(self.state[:1].view(torch.float32).item())

    @property
    def good_streak(self) -> int:
        return int(self.state[1].item())

    @property
    def n_skipped(self) -> int:
        return int(self.state[2].item())

    def state_dict(self) -> dict:
        return {"loss_scale": self.loss_scale, "good_streak": self.good_streak, "n_skipped": self.n_skipped}

    def load_state_dict(self, sd: dict) -> None:
        host = torch.tensor([0, int(sd["good_streak"]), int(sd["n_skipped"]), 0], dtype=torch.int32)
        host[:1].view(torch.float32).fill_(float(sd["loss_scale"]))
        self.state.copy_(host)
