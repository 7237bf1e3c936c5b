"""The routed expert layer at seeded random shapes against the oracle.

Each case draws experts, hidden and intermediate sizes, tokens, top-k, the
renormalisation flag and the dtype, and runs on the GPU the routing backward
(RouteTopKFn from the oracle's logits: routing is bit-exact given the same
logits), the fused 4-bit GEMMs with trained-value overlays at 0.5 % of the
positions, the combine and the sampled weight gradients at the same positions,
forward and backward.  The oracle (oracle/moe.py) runs the reference's routing
and routed expert loop op by op on the CPU on the same dequantized weights
with the trained values scattered in.  Shapes include ragged n-tiles (hidden
sizes not a multiple of 256, intermediate sizes not a multiple of 256),
experts that receive no token and single-token batches.
"""
import pytest
import torch

from oracle import moe as M
from oracle.codec_torch import dequant_opseq
from usaf_amd import moe as G
from usaf_amd.moe_loader import SparseGradStore

from parity import check

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _cases(n=8, seed=2026):
    g = torch.Generator().manual_seed(seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    out = []
    for i in range(n):
        E = int(torch.randint(2, 49, (1,), generator=g))
        H = pick([128, 256, 384, 640])
        I = pick([128, 256, 384])
        T = pick([1, 7, 64, 200, 517])
        k = int(torch.randint(1, min(E, 8) + 1, (1,), generator=g))
        out.append((i, E, H, I, T, k, bool(i % 2), (torch.bfloat16, torch.float16)[i % 2 == 0]))
    # the widest ragged tiles: hidden 640 (2.5 down n-tiles), intermediate 384 (3 SwiGLU n-tiles)
    out.append((n, 24, 640, 384, 517, 8, True, torch.bfloat16))
    out.append((n + 1, 64, 384, 128, 300, 8, False, torch.float16))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"E{c[1]}-H{c[2]}-I{c[3]}-T{c[4]}-k{c[5]}")
def test_routed_layer_random_shape(gpu_device, case):
    i, E, H, I, T, k, norm, dt = case
    _say(f"random shape {i}: E={E} H={H} I={I} T={T} k={k} norm={norm} {dt}")
    dev = gpu_device
    g = torch.Generator().manual_seed(100 + i)
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(dev))
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(dev))
    ew = G.ExpertWeights(qg, qd)
    active, w_eff = {}, {}
    for which, q in (("gate_up", qg), ("down", qd)):
        n = q.numel()
        idx = torch.randperm(n, generator=g)[: max(1, n // 200)].sort().values
        base = dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape).reshape(-1)
        masters = base[idx].float() + torch.randn(idx.numel(), generator=g) * 0.03
        ew.set_overlay(which, idx.to(dev), masters.to(dev), dt)
        eff = base.clone()
        eff[idx] = masters.half()            # the reference's fp16 weights after its scatter
        w_eff[which] = eff.to(dt).reshape(q.shape)
        active[f"{which}_proj"] = idx
    hs = torch.randn(T, H, generator=g).to(dt)
    logits = torch.randn(T, E, generator=g).to(dt)
    dout = torch.randn(T, H, generator=g).to(dt)
    store = SparseGradStore({f"L.{n}": v for n, v in active.items()},
                            {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}, device=dev)
    # GPU: routing backward from the same logits, fused experts with overlays and capture
    x = hs.to(dev).requires_grad_(True)
    lg = logits.to(dev).requires_grad_(True)
    weights = G.RouteTopKFn.apply(lg, k, norm, dt)
    out = G.routed_experts(x, weights, ew, capture=(store, "L"))
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    # oracle
    lo = logits.clone().requires_grad_(True)
    w_ref, _, _ = M.route(lo, k, norm, dt)
    out_r, dhs_r, dw_r, comp = M.experts_routed_manual(hs, w_ref.detach(), w_eff["gate_up"], w_eff["down"], dout,
                                                       active)
    (dlogits_r,) = torch.autograd.grad(w_ref, lo, dw_r.to(w_ref.dtype))
    assert torch.equal(weights.detach().cpu(), w_ref.detach()), "routing weights differ from the oracle's"
    for name, got, ref in (("out", out, out_r), ("dhs", x.grad, dhs_r), ("dlogits", lg.grad, dlogits_r),
                           ("sampled dW gate_up", store.compact["L.gate_up_proj"], comp["gate_up_proj"]),
                           ("sampled dW down", store.compact["L.down_proj"], comp["down_proj"])):
        if float(ref.float().abs().max()) == 0.0:
            assert float(got.float().abs().max()) == 0.0, name
            continue
        check(name, got, ref, dt, say=_say)
