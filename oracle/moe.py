"""TEST INFRASTRUCTURE ONLY: the reference's routed-expert path restated in
torch CPU ops (the parity checker and bench.py's CPU baseline; never shipped).

Each function follows the cited reference lines op for op, in the same dtypes.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def route(logits: torch.Tensor, top_k: int, norm_topk_prob: bool, act_dtype: torch.dtype):
    """usaf/qwen3moe_dml.py:73-83 -> (weights [T,E] act_dtype, probs fp32, mask fp32)."""
    probs = F.softmax(logits, dtype=torch.float, dim=-1)                 # :74
    top_val, _ = torch.topk(probs, top_k, dim=-1)                       # :77
    thresh = top_val[:, -1:].clone()                                     # :78
    mask = (probs >= thresh).to(probs.dtype)                             # :79
    weights = probs * mask                                               # :80
    if norm_topk_prob:                                                   # :81
        weights = weights / weights.sum(dim=-1, keepdim=True).clamp_min(1e-9)  # :82
    return weights.to(act_dtype), probs, mask                            # :83


def bucket(weights: torch.Tensor):
    """benchmarks/kaggle_t4_bench.py:293-306: nonzero pairs, bincount, stable
    argsort by expert.  Returns (counts [E], offsets [E+1], token_idx [S], slot
    weight (fp32 of the act-dtype weight) [S])."""
    E = weights.shape[1]
    tok_idx, exp_idx = torch.nonzero(weights, as_tuple=True)            # :293
    counts = torch.bincount(exp_idx, minlength=E)                        # :296
    order = torch.argsort(exp_idx, stable=True)                          # :298
    exp_s, tok_s = exp_idx[order], tok_idx[order]                        # :299
    offsets = torch.zeros(E + 1, dtype=torch.long)
    offsets[1:] = torch.cumsum(counts, 0)                                # :300-301
    return counts, offsets, tok_s, weights[tok_s, exp_s].float()


def experts_dense_masked(hs, weights, w_gate_up, w_down):
    """usaf/qwen3moe_dml.py:24-64 without grad capture: every expert on every
    token, scaled by a router weight that is zero outside the top-k."""
    final = torch.zeros(hs.shape, dtype=torch.float32)                  # :26
    weights_t = weights.t().contiguous()                                 # :27
    for ei in range(w_gate_up.shape[0]):                                 # :49
        gu = F.linear(hs, w_gate_up[ei])                                 # :58
        gate, up = gu.chunk(2, dim=-1)                                   # :59
        cur = F.silu(gate) * up                                          # :60
        cur = F.linear(cur, w_down[ei])                                  # :61
        final = final + cur.float() * weights_t[ei].float().unsqueeze(-1)  # :62
    return final.to(hs.dtype)                                            # :64


def experts_routed(hs, weights, w_gate_up, w_down, return_slots: bool = False):
    """benchmarks/kaggle_t4_bench.py:253-282: the same products restricted to
    each expert's routed tokens; fp32 accumulation in expert order (equal to
    the dense-masked sum: non-routed experts add exact zeros)."""
    N, H = hs.shape
    final = torch.zeros(N, H, dtype=torch.float32)
    slots = {}
    for ei in range(w_gate_up.shape[0]):
        w_col = weights[:, ei]
        idx = torch.nonzero(w_col, as_tuple=False).reshape(-1)          # :266
        if idx.numel() == 0:
            continue
        x_e = hs.index_select(0, idx)                                    # :268
        gu = F.linear(x_e, w_gate_up[ei])                                # :276
        gate, up = gu.chunk(2, dim=-1)
        act = F.silu(gate) * up
        cur = F.linear(act, w_down[ei])                                  # :279
        if return_slots:
            slots[ei] = dict(idx=idx, gu=gu, act=act, y=cur)
        cur = cur.float() * w_col.index_select(0, idx).float().unsqueeze(-1)  # :280
        final = final.index_add(0, idx, cur)                             # :281
    out = final.to(hs.dtype)
    return (out, slots) if return_slots else out


def experts_routed_autograd(hs, weights, w_gate_up, w_down, dout):
    """Backward of the routed expert forward by torch autograd in the act
    dtype (the reference obtains its gradients the same way, through
    F.linear/silu/mul backward).  Returns (dhs, dweights, dW_gate_up, dW_down)
    with dense per-expert weight gradients in the weight dtype."""
    hs = hs.detach().clone().requires_grad_(True)
    w = weights.detach().clone().requires_grad_(True)
    wg = w_gate_up.detach().clone().requires_grad_(True)
    wd = w_down.detach().clone().requires_grad_(True)
    out = experts_routed(hs, w, wg, wd)
    out.backward(dout)
    return hs.grad, w.grad, wg.grad, wd.grad


def gather_compact(dense_grad: torch.Tensor, active_idx: torch.Tensor) -> torch.Tensor:
    """SparseGradStore.add (usaf/moe_loader.py:564-578) for one microbatch:
    the active flat positions of the dense grad, as fp32."""
    return dense_grad.reshape(-1).gather(0, active_idx.reshape(-1).long()).float()


def sparse_adam_step(p, g, m, v, step, lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
    """usaf/sparse_optim.py:94-130 (compact_params=True) on fp32 CPU vectors, in place."""
    beta1, beta2 = betas
    bias1 = 1 - beta1 ** step                                            # :96
    bias2 = 1 - beta2 ** step                                            # :97
    grad = g.clone()
    if weight_decay > 0:                                                 # :113
        grad = grad + weight_decay * p                                   # :119
    m.mul_(beta1).add_(grad, alpha=1 - beta1)                            # :123
    v.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)                  # :124
    update = (m / bias1) / ((v / bias2).sqrt() + eps)                    # :126
    p.add_(-lr * update)                                                 # :127-130
    return p, m, v


def combine_slots(y_slots: torch.Tensor, offsets, token_idx: torch.Tensor, weights: torch.Tensor):
    """usaf/qwen3moe_dml.py:62-64 given each routed slot's expert output
    (slots grouped by expert in `offsets`): fp32 accumulation over experts in
    ascending order, each product cur.float() * w.float() rounded before the add."""
    T, E = weights.shape
    final = torch.zeros(T, y_slots.shape[1], dtype=torch.float32)
    offs = [int(o) for o in offsets]
    for e in range(E):
        s0, s1 = offs[e], offs[e + 1]
        if s0 == s1:
            continue
        idx = token_idx[s0:s1].long()
        final = final.index_add(0, idx, y_slots[s0:s1].float() * weights[idx, e].float().unsqueeze(-1))
    return final.to(weights.dtype)


def _rd(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round an fp32 tensor to `dtype` and back: the output of one torch op in
    that dtype (torch computes 16-bit ops in fp32 and rounds the result once)."""
    return x.to(dtype).float()


def experts_routed_manual(hs, weights, w_gate_up, w_down, dout, active=None):
    """The forward and backward of experts_routed_autograd (the routed expert
    loop of benchmarks/kaggle_t4_bench.py:253-282 and qwen3moe_dml.py:58-64,
    differentiated as torch autograd does), written out op by op.

    Every op computes in fp32 and rounds its output to the activation dtype
    where the reference's dtype op does: F.linear outputs (forward, grad-input
    and grad-weight), F.silu and the SwiGLU product, silu_backward, the mul
    backwards, the expert output's cast of its gradient; the combine and its
    backward stay in fp32 (qwen3moe_dml.py:62-64).  Gradients reaching the same
    token from several experts are summed in fp32 and rounded once.  Instead of
    the dense per-expert weight gradients, ``active`` {"gate_up_proj": flat
    idx, "down_proj": flat idx} asks for their values at those positions only,
    as SparseGradStore.add gathers them (usaf/moe_loader.py:564-578): fp32 of
    the dtype-rounded dot product over the expert's routed tokens.

    Returns (out, dhs, dweights, compact) with compact {name: fp32 [n]}.
    Large shapes run in seconds on CPU threads, where the dtype autograd of the
    same loop (experts_routed_autograd) takes minutes; tests pin one against
    the other on small shapes."""
    dt = hs.dtype
    T, H = hs.shape
    E, I2, _ = w_gate_up.shape
    I = I2 // 2
    hs32 = hs.float()
    dout32 = dout.float()
    final = torch.zeros(T, H, dtype=torch.float32)
    dhs = torch.zeros(T, H, dtype=torch.float32)
    dweights = torch.zeros(T, E, dtype=torch.float32)
    per_expert = {}
    if active is not None:
        for name, rows, cols in (("gate_up_proj", I2, H), ("down_proj", H, I)):
            idx = active[name].reshape(-1).long()
            e_of = torch.div(idx, rows * cols, rounding_mode="floor")
            per_expert[name] = (idx, e_of, rows, cols)
    compact = {name: torch.zeros(v[0].numel(), dtype=torch.float32) for name, v in per_expert.items()}

    def sampled(name, ei, dy, x):
        if name not in per_expert:
            return
        idx, e_of, rows, cols = per_expert[name]
        sel = (e_of == ei).nonzero(as_tuple=False).reshape(-1)
        if sel.numel() == 0:
            return
        local = idx[sel] - ei * rows * cols
        o = torch.div(local, cols, rounding_mode="floor")
        i = local - o * cols
        for c0 in range(0, sel.numel(), 65536):  # bounded temporaries
            oc, ic = o[c0:c0 + 65536], i[c0:c0 + 65536]
            dots = (dy[:, oc] * x[:, ic]).sum(0)
            compact[name][sel[c0:c0 + 65536]] = _rd(dots, dt)

    for ei in range(E):
        w_col = weights[:, ei]
        idx = torch.nonzero(w_col, as_tuple=False).reshape(-1)
        if idx.numel() == 0:
            continue
        x = hs32.index_select(0, idx)
        wg = w_gate_up[ei].float()
        wd = w_down[ei].float()
        w_e = w_col.index_select(0, idx).float().unsqueeze(-1)
        # forward (qwen3moe_dml.py:58-62)
        gu = _rd(x @ wg.t(), dt)
        g, u = gu[:, :I], gu[:, I:]
        sig = torch.sigmoid(g)
        sg = _rd(g * sig, dt)
        act = _rd(sg * u, dt)
        y = _rd(act @ wd.t(), dt)
        final.index_add_(0, idx, y * w_e)
        # backward of final + y.float() * w (fp32), then of each dtype op
        d_fin = dout32.index_select(0, idx)
        dweights[idx, ei] = (d_fin * y).sum(-1)
        dy = _rd(d_fin * w_e, dt)
        dact = _rd(dy @ wd, dt)
        sampled("down_proj", ei, dy, act)
        dsg = _rd(dact * u, dt)
        du = _rd(dact * sg, dt)
        dg = _rd(dsg * (sig * (1.0 + g * (1.0 - sig))), dt)
        dgu = torch.cat([dg, du], dim=1)
        dx = _rd(dgu @ wg, dt)
        sampled("gate_up_proj", ei, dgu, x)
        dhs.index_add_(0, idx, dx)
    return final.to(dt), dhs.to(dt), dweights.to(dt), compact


def topk_store_candidates(g: torch.Tensor, ei: int, frac: float, cand_mult: float = 2.0):
    """TopKImportanceStore.add (usaf/moe_loader.py:605-611): expert ei's top
    |g| candidates as (fp32 magnitudes, global flat indices)."""
    flat = g.detach().float().reshape(-1).abs()
    k = max(1, int(flat.numel() * frac * cand_mult))
    v, i = torch.topk(flat, min(k, flat.numel()))
    return v, i.to(torch.long) + int(ei) * flat.numel()


def topk_store_select(cands, numel: int, frac: float) -> torch.Tensor:
    """TopKImportanceStore.select (usaf/moe_loader.py:613-627) for one tensor:
    ``cands`` = [(vals, idx) per expert in insertion order]."""
    vals = torch.cat([c[0] for c in cands])
    idxs = torch.cat([c[1] for c in cands])
    k = min(max(1, int(numel * frac)), vals.numel())
    return idxs[torch.topk(vals, k).indices]


def reselect_merge(old_idx: torch.Tensor, old_masters: torch.Tensor, new_idx, dequant_flat: torch.Tensor):
    """The reselect merge of train.py:556-597 for one tensor, with Python sets
    as there: (final flat indices, fp32 masters).  ``dequant_flat`` is the
    tensor's fp16 dequantized weights, flattened (:589-595)."""
    if new_idx is None or new_idx.numel() == 0:                         # :560-563
        return old_idx.clone(), old_masters.clone()
    old_set = set(old_idx.reshape(-1).tolist())                          # :559
    nw_set = set(new_idx.reshape(-1).tolist())                           # :564
    kept = sorted(old_set & nw_set)                                      # :565
    candidates = sorted(nw_set - old_set)                                # :566
    fill = max(0, len(old_set) - len(kept))                              # :568
    grown = candidates[:fill]                                            # :569
    final = torch.tensor(kept + grown, dtype=torch.long)                 # :570
    old_flat = old_idx.reshape(-1).to(torch.long)
    keep_mask = torch.isin(final, old_flat)                              # :575
    new_vals = torch.zeros(final.numel(), dtype=torch.float32)
    kept_pos = keep_mask.nonzero(as_tuple=False).reshape(-1)
    if kept_pos.numel() > 0:                                             # :582-588
        all_idx = torch.zeros(int(old_flat.max().item()) + 1, dtype=torch.long)
        all_idx[old_flat] = torch.arange(old_flat.numel(), dtype=torch.long)
        new_vals[kept_pos] = old_masters.float()[all_idx[final[kept_pos]]]
    grow_pos = (~keep_mask).nonzero(as_tuple=False).reshape(-1)
    if grow_pos.numel() > 0:                                             # :590-596
        new_vals[grow_pos] = dequant_flat.reshape(-1)[final[grow_pos]].float()
    return final, new_vals
