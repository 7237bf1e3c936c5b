"""GPU parity at the benchmark's own sizes, against the CPU oracle.

* one Qwen3-30B-A3B MoE layer step at full size (T=4096, H=2048,
  I=768, E=128, top-8, 4-bit experts) in bf16 and in fp16 -- router forward
  (fused logits kernel), routing, fused 4-bit forward, grad-input through the
  transposed 4-bit copies, router backward and weight gradient, and the
  sampled weight gradients at a 0.5 % mask of each expert tensor.
* the fp16 GEMM leg X [512, 2048] . W^T, W [768, 2048] from the
  4-bit codes, through usaf_hip_moe_down_fwd with one expert.
* the Mixtral-8x7B-shaped layer forward + backward at reduced T.

The oracle is oracle/moe.py's experts_routed_manual (the reference's expert
loop with every op rounded where the reference's dtype op rounds, sampled
gradients only), pinned against the dtype autograd oracle in
tests/test_oracle_moe.py; routing and the router's F.linear backward use the
reference's own torch ops (oracle/moe.py route, autograd) on the same logits.

Bars: normwise rel = max|got - ref| / max|ref| <= 1e-2 (bf16) / 2e-3 (fp16),
as every GPU test here.  Beside it each check reports the elementwise
relative error |got - ref| / max(|ref|, 0.01 rms(ref)) at its 99th
percentile, bounded loosely (5e-2 bf16, 1e-2 fp16) so that a few wrong
elements cannot hide under the normwise bar.
"""
import numpy as np
import pytest
import torch

from oracle import moe as M
from oracle.codec_torch import dequant_opseq
from usaf_amd import _native as N
from usaf_amd import moe as G
from usaf_amd.moe_loader import SparseGradStore

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}
P99 = {torch.bfloat16: 5e-2, torch.float16: 1e-2}


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def errs(got, ref):
    """(normwise rel, elementwise p99 rel) of got against ref."""
    got = got.detach().float().cpu().reshape(-1)
    ref = ref.detach().float().cpu().reshape(-1)
    scale = float(ref.abs().max())
    assert scale > 0, "reference is all zeros"
    norm = float((got - ref).abs().max()) / scale
    floor = 0.01 * float(ref.pow(2).mean().sqrt())
    r = ((got - ref).abs() / ref.abs().clamp_min(max(floor, 1e-30))).numpy()
    return norm, float(np.percentile(r, 99))


def check(name, got, ref, dtype, report):
    norm, p99 = errs(got, ref)
    report[name] = (norm, p99)
    _say(f"  {name}: normwise {norm:.2e} (bar {TOL[dtype]:.0e}), p99 elementwise {p99:.2e} (bar {P99[dtype]:.0e})")
    assert norm <= TOL[dtype], f"{name}: normwise {norm:.3e} > {TOL[dtype]}"
    assert p99 <= P99[dtype], f"{name}: p99 elementwise {p99:.3e} > {P99[dtype]}"


def _quantized(dev, shape, g):
    w = (torch.randn(shape, generator=g) * 0.02).half()
    q = G.Q4Tensor.quantize(w.to(dev))
    deq = dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape)  # the reference's CPU dequant of the same codes
    return q, deq


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_cfg2_full_step_vs_oracle(gpu_device, dtype):
    E, H, I, T, k = 128, 2048, 768, 4096, 8
    _say(f"cfg2 full step T={T} H={H} I={I} E={E} k={k} {dtype}: build")
    torch.set_num_threads(16)
    dev = gpu_device
    g = torch.Generator().manual_seed(2024)
    qg, deq_g = _quantized(dev, (E, 2 * I, H), g)
    qd, deq_d = _quantized(dev, (E, H, I), g)
    hs = torch.randn(T, H, generator=g).to(dtype)
    wr = (torch.randn(E, H, generator=g) / H ** 0.5).to(dtype)
    dout = torch.randn(T, H, generator=g).to(dtype)
    nG, nD = E * 2 * I * H, E * H * I
    active = {"gate_up_proj": torch.randperm(nG, generator=g)[: int(0.005 * nG)].sort().values,
              "down_proj": torch.randperm(nD, generator=g)[: int(0.005 * nD)].sort().values}
    prefix = "model.layers.0.mlp.experts"
    store = SparseGradStore({f"{prefix}.{n}": v for n, v in active.items()},
                            {f"{prefix}.gate_up_proj": (E, 2 * I, H), f"{prefix}.down_proj": (E, H, I)},
                            device=dev)
    _say("  GPU step")
    x = hs.to(dev).requires_grad_(True)
    w_r = wr.to(dev).requires_grad_(True)
    ew = G.ExpertWeights(qg, qd)
    out = G.moe_block(x, w_r, k, False, ew, capture=(store, prefix))
    out.backward(dout.to(dev))
    # the step's router logits (the fused logits kernel is deterministic): the
    # oracle routes from the same logits, so routing is compared bit for bit
    logits = torch.empty(T, E, dtype=dtype, device=dev)
    wts = torch.empty(T, E, dtype=dtype, device=dev)
    N.call("usaf_hip_router_fwd", x.data_ptr(), w_r.data_ptr(), T, E, H, N.dtype_code(dtype), k, 0, logits.data_ptr(),
           wts.data_ptr(), N.dtype_code(dtype), None, N.stream_ptr(dev))
    torch.cuda.synchronize()
    _say("  oracle")
    lg = logits.cpu().requires_grad_(True)
    w_ref, _, mask = M.route(lg, k, False, dtype)
    assert torch.equal(wts.cpu() != 0, mask != 0), "routing mask differs from the oracle's on the same logits"
    out_r, dhs_e, dw_r, comp = M.experts_routed_manual(hs, w_ref.detach(), deq_g.to(dtype), deq_d.to(dtype), dout,
                                                      active)
    w_ref.backward(dw_r)  # the routing's softmax / mask backward (reference ops), to dlogits
    dlogits = lg.grad
    dwr_ref = (dlogits.double().t() @ hs.double()).to(dtype)           # F.linear weight grad
    dhs_ref = (dhs_e.float() + (dlogits.double() @ wr.double()).to(dtype).float()).to(dtype)
    rep = {}
    check("out", out, out_r, dtype, rep)
    check("dhs", x.grad, dhs_ref, dtype, rep)
    check("router dW", w_r.grad, dwr_ref, dtype, rep)
    check("sampled dW gate_up", store.compact[f"{prefix}.gate_up_proj"], comp["gate_up_proj"], dtype, rep)
    check("sampled dW down", store.compact[f"{prefix}.down_proj"], comp["down_proj"], dtype, rep)


def test_cfg0_fp16_gemm_leg(gpu_device):
    _say("cfg0 GEMM leg: X fp16 [512,2048] . W^T, W [768,2048] 4-bit, via usaf_hip_moe_down_fwd (E=1)")
    dev = gpu_device
    g = torch.Generator().manual_seed(1234)
    q, deq = _quantized(dev, (1, 768, 2048), g)
    X = torch.randn(512, 2048, generator=g).half()
    offsets = torch.tensor([0, 512], dtype=torch.int32, device=dev)
    y = torch.empty(512, 768, dtype=torch.float16, device=dev)
    Xd = X.to(dev)
    N.call("usaf_hip_moe_down_fwd", Xd.data_ptr(), 2048, offsets.data_ptr(), 512, 1, 768, q.q.data_ptr(),
           q.scale_zero().data_ptr(), None, N.F16, y.data_ptr(), None, 0, N.stream_ptr(dev))
    torch.cuda.synchronize()
    ref = (X.float() @ deq[0].float().t()).half()  # F.linear in fp16: fp32 products, one rounding
    rep = {}
    check("Y", y, ref, torch.float16, rep)


def test_cfg3_mixtral_backward_reduced_tokens(gpu_device):
    E, H, I, T, k = 8, 4096, 14336, 384, 2
    dtype = torch.bfloat16
    _say(f"cfg3 Mixtral fwd+bwd E={E} H={H} I={I} k={k} T={T} {dtype}")
    torch.set_num_threads(16)
    dev = gpu_device
    g = torch.Generator().manual_seed(77)
    qg, deq_g = _quantized(dev, (E, 2 * I, H), g)
    qd, deq_d = _quantized(dev, (E, H, I), g)
    hs = torch.randn(T, H, generator=g).to(dtype)
    w_ref, _, _ = M.route(torch.randn(T, E, generator=g), k, False, dtype)
    dout = torch.randn(T, H, generator=g).to(dtype)
    nG, nD = E * 2 * I * H, E * H * I
    active = {"gate_up_proj": torch.randperm(nG, generator=g)[: int(0.005 * nG)].sort().values,
              "down_proj": torch.randperm(nD, generator=g)[: int(0.005 * nD)].sort().values}
    store = SparseGradStore({f"L.{n}": v for n, v in active.items()},
                            {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}, device=dev)
    x = hs.to(dev).requires_grad_(True)
    w = w_ref.to(dev).requires_grad_(True)
    out = G.routed_experts(x, w, G.ExpertWeights(qg, qd), capture=(store, "L"))
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    _say("  oracle")
    out_r, dhs_r, dw_r, comp = M.experts_routed_manual(hs, w_ref, deq_g.to(dtype), deq_d.to(dtype), dout, active)
    routed = w_ref != 0
    rep = {}
    check("out", out, out_r, dtype, rep)
    check("dhs", x.grad, dhs_r, dtype, rep)
    check("dweights", w.grad.cpu()[routed], dw_r[routed], dtype, rep)
    assert torch.all(w.grad.cpu()[~routed] == 0)
    check("sampled dW gate_up", store.compact["L.gate_up_proj"], comp["gate_up_proj"], dtype, rep)
    check("sampled dW down", store.compact["L.down_proj"], comp["down_proj"], dtype, rep)
