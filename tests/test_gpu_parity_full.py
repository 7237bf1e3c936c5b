"""GPU parity at the benchmark's own sizes, against the CPU oracle.

* one Qwen3-30B-A3B MoE layer step at full size (T=4096, H=2048,
  I=768, E=128, top-8, 4-bit experts) in bf16 and in fp16 -- router forward
  (fused logits kernel), routing, fused 4-bit forward, grad-input through the
  transposed 4-bit copies, router backward and weight gradient, and the
  sampled weight gradients at a 0.5 % mask of each expert tensor.
* the fp16 GEMM leg X [512, 2048] . W^T, W [768, 2048] from the
  4-bit codes, through usaf_hip_moe_down_fwd with one expert.
* configs[2], the benchmark's own measured step: bench.build_moe's layer with
  the trained masters (perturbed off the 4-bit values) in every GEMM through
  the overlay tables, capacity-mode bucketing (no host read of the slot
  count), the device loss scale, then the device-gated SparseAdam + router
  SGD + overlay refresh + loss-scale update, and a second step on the
  updated weights -- each step's outputs and gradients against the oracle on
  the scattered weights, the SparseAdam update against the oracle's.
* the Mixtral-8x7B-shaped layer forward + backward at T=384 and at
  T=2048 (512 slots per expert: full 256-slot m-tiles).

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
import pytest
import torch

from oracle import moe as M
from oracle.codec_torch import dequant_opseq
from usaf_amd import _native as N
from usaf_amd import moe as G
from usaf_amd.moe_loader import SparseGradStore

from parity import check

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


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


def _scattered(base16, idx, vals, dtype):
    """The reference's fp16 expert weight after its scatter of the masters
    (moe_loader.py:218-221), in the activation dtype."""
    w = base16.clone()
    w.reshape(-1)[idx.long()] = vals.half()
    return w.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_cfg2_bench_step_two_steps_vs_oracle(gpu_device, dtype):
    import bench
    E, H, I, T, k = 128, 2048, 768, 4096, 8
    _say(f"cfg2 measured step (overlays, capacity bucketing, loss scale, gated updates) x2, {dtype}: build")
    torch.set_num_threads(16)
    dev = gpu_device
    L = bench.build_moe(dev, dtype=dtype)
    L["keep_out"] = True
    ew = L["experts"]
    deq = {"gate_up_proj": dequant_opseq(ew.gate_up.q.cpu(), ew.gate_up.s.cpu(), ew.gate_up.z.cpu(), ew.gate_up.shape),
           "down_proj": dequant_opseq(ew.down.q.cpu(), ew.down.s.cpu(), ew.down.z.cpu(), ew.down.shape)}
    short = {n: n.rsplit(".", 1)[1] for n in L["active"]}
    # trained values differ from the 4-bit base: the masters move off the dequantized values
    g = torch.Generator(device=dev).manual_seed(99)
    with torch.no_grad():
        for p in L["masters"].values():
            p.add_(torch.randn(p.numel(), device=dev, generator=g) * 0.01)
    bench.sync_overlays(L)
    if dtype == torch.float16:
        # the regime loss scaling serves: a loss gradient of small per-element size,
        # which the initial scale of 4096 brings to N(0, 1) (dY ~ N(0, 1) itself
        # would overflow fp16 in the scaled grad-input sums, as it does in the oracle)
        L["dy"].div_(bench.LOSS_SCALE_INIT)
    active = {short[n]: idx.cpu() for n, idx in L["active"].items()}
    flags = torch.tensor([1, 0], dtype=torch.int32, device=dev)
    finite, halt = flags[:1], flags[1:]
    opt = L["opt"]
    for step in range(2):
        scale = L["scaler"].loss_scale
        masters = {short[n]: p.detach().cpu().clone() for n, p in L["masters"].items()}
        wr = L["router_w"].detach().cpu()
        _say(f"  step {step}: GPU (loss scale {scale:.0f})")
        cg = bench._fwd_bwd_check(L, finite, halt, slot=step % 2)
        logits = torch.empty(T, E, dtype=dtype, device=dev)
        wts = torch.empty(T, E, dtype=dtype, device=dev)
        N.call("usaf_hip_router_fwd", L["hs"].data_ptr(), L["router_w"].data_ptr(), T, E, H, N.dtype_code(dtype), k,
               0, logits.data_ptr(), wts.data_ptr(), N.dtype_code(dtype), None, N.stream_ptr(dev))
        torch.cuda.synchronize()
        assert int(halt.item()) == 0, "the routing overflowed the static slots"
        assert int(finite.item()) == 1, "non-finite gradients"
        _say(f"  step {step}: oracle")
        hs = L["hs"].detach().cpu()
        dy_s = L["dy"].cpu() * scale  # the scaled loss's gradient, exact (power of two)
        lg = logits.cpu().requires_grad_(True)
        w_ref, _, mask = M.route(lg, k, False, dtype)
        assert torch.equal(wts.cpu() != 0, mask != 0), "routing mask differs from the oracle's on the same logits"
        wg = _scattered(deq["gate_up_proj"], active["gate_up_proj"], masters["gate_up_proj"], dtype)
        wd = _scattered(deq["down_proj"], active["down_proj"], masters["down_proj"], dtype)
        out_r, dhs_e, dw_r, comp = M.experts_routed_manual(hs, w_ref.detach(), wg, wd, dy_s, active)
        del wg, wd
        w_ref.backward(dw_r)
        dlogits = lg.grad
        dwr_ref = (dlogits.double().t() @ hs.double()).to(dtype)
        dhs_ref = (dhs_e.float() + (dlogits.double() @ wr.double()).to(dtype).float()).to(dtype)
        check(f"step {step} out", L["out"], out_r, dtype)
        check(f"step {step} dhs", L["hs"].grad, dhs_ref, dtype)
        check(f"step {step} router dW", L["router_w"].grad, dwr_ref, dtype)
        for n, name in short.items():
            # the unscaled compact gradient: the oracle's (scaled) values / loss scale, exact
            check(f"step {step} sampled dW {name}", cg[n], comp[name] / scale, dtype)
        # the bench loop's update of the step, gated on the device
        before = {n: (L["masters"][n].detach().cpu().clone(), opt._m[n].cpu().clone(), opt._v[n].cpu().clone(),
                      cg[n].cpu().clone()) for n in short}
        L["sgd"].step(finite=finite, halt=halt, loss_scale=L["scaler"])
        opt.step(compact_grads=cg, finite=finite, halt=halt)
        bench.sync_overlays(L)
        L["scaler"].update(finite, halt)
        torch.cuda.synchronize()
        for n, (p0, m0, v0, g0) in before.items():
            p_ref, _, _ = M.sparse_adam_step(p0, g0, m0, v0, step + 1, 2e-4, weight_decay=0.005)
            got = L["masters"][n].detach().cpu()
            rel = float((got - p_ref).abs().max() / p_ref.abs().max())
            _say(f"  step {step} SparseAdam {short[n]}: normwise {rel:.2e} (bar 1e-06)")
            assert rel <= 1e-6
    assert opt.step_count == 2


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


@pytest.mark.parametrize("T", [384, 2048])
def test_cfg3_mixtral_backward(gpu_device, T):
    E, H, I, k = 8, 4096, 14336, 2
    dtype = torch.bfloat16
    _say(f"cfg3 Mixtral fwd+bwd E={E} H={H} I={I} k={k} T={T} {dtype}")
    torch.set_num_threads(16)
    dev = gpu_device
    g = torch.Generator().manual_seed(77 + T)
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
    if T >= 2048:
        S_e = routed.sum(0)
        assert int(S_e.min()) >= 256, "every expert should fill at least one 256-slot m-tile"
    rep = {}
    check("out", out, out_r, dtype, rep)
    check("dhs", x.grad, dhs_r, dtype, rep)
    check("dweights", w.grad.cpu()[routed], dw_r[routed], dtype, rep)
    assert torch.all(w.grad.cpu()[~routed] == 0)
    check("sampled dW gate_up", store.compact["L.gate_up_proj"], comp["gate_up_proj"], dtype, rep)
    check("sampled dW down", store.compact["L.down_proj"], comp["down_proj"], dtype, rep)
