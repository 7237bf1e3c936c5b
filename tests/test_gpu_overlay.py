"""Trained-value overlays on the fused 4-bit GEMMs (usaf_amd/moe.py Q4Overlay).

The reference scatters the optimizer's fp32 masters into its fp16 expert
weights every step (usaf/moe_loader.py:218-221, 425-443; train.py:666), and the
next forward and backward run on those weights.  Here the four fused GEMMs read
the masters through overlay entry tables instead.

* Effective weights, bit-exact: with one-hot activation rows every output of a
  GEMM is a single product 1 * w, exact in fp32 and in the 16-bit output, so
  each GEMM's output is the weight matrix it multiplied by.  It must equal the
  oracle's dequant (oracle/codec_torch.py) -> fp16 scatter of the masters ->
  activation dtype, before and after a refresh with new values.
* A routed expert layer forward + backward with overlays against the oracle's
  expert loop (oracle/moe.py experts_routed_manual) on the scattered weights,
  within the usual bars (normwise 1e-2 bf16, 2e-3 fp16).
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
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bits(t):
    """16-bit patterns, -0 read as +0: a one-hot row's product 1 * (-0) is summed
    with the +0 products of the row's zeros, so a GEMM returns +0 for it."""
    t = t.detach().cpu().contiguous()
    t = torch.where(t == 0, torch.zeros_like(t), t)
    return t.view(torch.int16)


def _scattered(q: G.Q4Tensor, idx, masters, dtype):
    """The reference's weights after the overlay scatter, in the activation dtype."""
    w16 = dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape).clone()
    w16.reshape(-1)[idx.cpu()] = masters.cpu().to(torch.float16)
    return w16.to(dtype)


def _one_hot(n, dtype, dev, reps):
    return torch.eye(n, dtype=dtype, device=dev).repeat(reps, 1).contiguous()


def _gemm_weights(ew, dtype):
    """Each fused GEMM's weight matrix, read back through one-hot activation rows:
    gate_up fwd -> W_gu^T per expert, down fwd -> W_dn^T, down grad-input -> W_dn
    (through the SwiGLU backward with g = 0, u = 2: dgate = DT(2 dact) / 2 = dact), gate_up
    grad-input -> W_gu."""
    dev = ew.gate_up.device
    E, H, I = ew.E, ew.H, ew.I
    st = N.stream_ptr(dev)
    code = N.dtype_code(dtype)
    out = {}
    # gate_up forward: slot e*H + t of expert e reads token t = one-hot row t
    x = torch.eye(H, dtype=dtype, device=dev)
    tok = torch.arange(H, dtype=torch.int32, device=dev).repeat(E)
    offs = torch.arange(E + 1, dtype=torch.int32, device=dev) * H
    gu = torch.empty(E * H, 2 * I, dtype=dtype, device=dev)
    act = torch.empty(E * H, I, dtype=dtype, device=dev)
    q, sz, _ = ew._ptrs("gate_up", dtype)
    N.call("usaf_hip_moe_gate_up_fwd", x.data_ptr(), H, H, tok.data_ptr(), offs.data_ptr(), E * H, E, I, q, sz, None,
           code, gu.data_ptr(), act.data_ptr(), None, None, *ew._ovl("gate_up_fwd", dtype), st)
    out["gate_up_fwd"] = gu.view(E, H, 2 * I).transpose(1, 2)
    # down forward: slot e*I + i = one-hot row i
    a = _one_hot(I, dtype, dev, E)
    offs = torch.arange(E + 1, dtype=torch.int32, device=dev) * I
    y = torch.empty(E * I, H, dtype=dtype, device=dev)
    q, sz, _ = ew._ptrs("down", dtype)
    N.call("usaf_hip_moe_down_fwd", a.data_ptr(), I, offs.data_ptr(), E * I, E, H, q, sz, None, code, y.data_ptr(),
           *ew._ovl("down_fwd", dtype), st)
    out["down_fwd"] = y.view(E, I, H).transpose(1, 2)
    # down grad-input (transposed copy): slot e*H + h = one-hot row h; saved gu: gate 0, up 2
    dcur = _one_hot(H, dtype, dev, E)
    gsv = torch.cat([torch.zeros(E * H, I, dtype=dtype, device=dev),
                     torch.full((E * H, I), 2.0, dtype=dtype, device=dev)], 1)
    offs = torch.arange(E + 1, dtype=torch.int32, device=dev) * H
    dgu = torch.empty(E * H, 2 * I, dtype=dtype, device=dev)
    N.call("usaf_hip_moe_down_bwd_t", dcur.data_ptr(), H, gsv.data_ptr(), offs.data_ptr(), E * H, E, I,
           *ew._ptrs_t("down"), code, dgu.data_ptr(), *ew._ovl("down_bwd", dtype), st)
    out["down_bwd"] = dgu[:, :I].reshape(E, H, I)
    out["down_bwd_up"] = dgu[:, I:]
    # gate_up grad-input (transposed copy): slot e*2I + n = one-hot row n
    dg = _one_hot(2 * I, dtype, dev, E)
    offs = torch.arange(E + 1, dtype=torch.int32, device=dev) * 2 * I
    dx = torch.empty(E * 2 * I, H, dtype=dtype, device=dev)
    N.call("usaf_hip_moe_gate_up_bwd_t", dg.data_ptr(), I, offs.data_ptr(), E * 2 * I, E, H, *ew._ptrs_t("gate_up"),
           code, dx.data_ptr(), *ew._ovl("gate_up_bwd", dtype), st)
    out["gate_up_bwd"] = dx.view(E, 2 * I, H)
    torch.cuda.synchronize()
    return out


def _check_weights(ew, want_gu, want_dn, dtype, what):
    got = _gemm_weights(ew, dtype)
    for kind, want in (("gate_up_fwd", want_gu), ("down_fwd", want_dn), ("down_bwd", want_dn),
                       ("gate_up_bwd", want_gu)):
        g, w = _bits(got[kind]), _bits(want)
        n_bad = int((g != w).sum())
        _say(f"  {what} {kind}: {n_bad} of {w.numel()} weights differ")
        assert n_bad == 0, f"{what}: {kind} multiplies {n_bad} weights that differ from the scattered oracle"
    assert torch.all(got["down_bwd_up"].float().cpu() == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_overlay_effective_weights_bit_exact(gpu_device, dtype):
    E, H, I = 3, 256, 128
    _say(f"overlay effective weights E={E} H={H} I={I} {dtype}")
    dev = gpu_device
    g = torch.Generator().manual_seed(11)
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(dev))
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(dev))
    ew = G.ExpertWeights(qg, qd)
    base_g = dequant_opseq(qg.q.cpu(), qg.s.cpu(), qg.z.cpu(), qg.shape).to(dtype)
    base_d = dequant_opseq(qd.q.cpu(), qd.s.cpu(), qd.z.cpu(), qd.shape).to(dtype)
    _check_weights(ew, base_g, base_d, dtype, "no overlay")
    idx, masters = {}, {}
    for which, q in (("gate_up", qg), ("down", qd)):
        n = q.numel()
        idx[which] = torch.randperm(n, generator=g)[: n // 100].sort().values
        # trained values: the dequantized weight plus an update, some far from it
        deq = dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape).reshape(-1)[idx[which]].float()
        masters[which] = deq + torch.randn(idx[which].numel(), generator=g) * 0.01
        masters[which][:5] = torch.tensor([0.0, -0.0, 1e-6, 3.0, -1000.0])  # zero, fp16 subnormal, large
        ew.set_overlay(which, idx[which].to(dev), masters[which].to(dev), dtype)
    _check_weights(ew, _scattered(qg, idx["gate_up"], masters["gate_up"], dtype),
                   _scattered(qd, idx["down"], masters["down"], dtype), dtype, "overlay")
    # a refresh with new values (as after an optimizer step) is seen by the next GEMMs
    for which in ("gate_up", "down"):
        masters[which] = masters[which] * 0.5 - 0.003
        ew.overlays[which].refresh(masters[which].to(dev))
    _check_weights(ew, _scattered(qg, idx["gate_up"], masters["gate_up"], dtype),
                   _scattered(qd, idx["down"], masters["down"], dtype), dtype, "refreshed")
    assert int(ew.overlays["gate_up"].bad.item()) == 0 and int(ew.overlays["down"].bad.item()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_overlay_routed_layer_vs_oracle(gpu_device, dtype):
    E, H, I, T, k = 8, 256, 128, 300, 2
    _say(f"overlay routed layer fwd+bwd E={E} H={H} I={I} T={T} k={k} {dtype}")
    dev = gpu_device
    g = torch.Generator().manual_seed(23)
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(dev))
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(dev))
    ew = G.ExpertWeights(qg, qd)
    idx, masters, w_eff = {}, {}, {}
    for which, q in (("gate_up", qg), ("down", qd)):
        n = q.numel()
        idx[which] = torch.randperm(n, generator=g)[: n // 200].sort().values
        deq = dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape).reshape(-1)[idx[which]].float()
        masters[which] = deq + torch.randn(idx[which].numel(), generator=g) * 0.05  # large updates: visible
        ew.set_overlay(which, idx[which].to(dev), masters[which].to(dev), dtype)
        w_eff[which] = _scattered(q, idx[which], masters[which], dtype)
    hs = torch.randn(T, H, generator=g).to(dtype)
    w_ref, _, _ = M.route(torch.randn(T, E, generator=g), k, False, dtype)
    dout = torch.randn(T, H, generator=g).to(dtype)
    active = {"gate_up_proj": idx["gate_up"], "down_proj": idx["down"]}
    store = SparseGradStore({f"L.{n}": v for n, v in active.items()},
                            {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}, device=dev)
    x = hs.to(dev).requires_grad_(True)
    w = w_ref.to(dev).requires_grad_(True)
    out = G.routed_experts(x, w, ew, capture=(store, "L"))
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    out_r, dhs_r, dw_r, comp = M.experts_routed_manual(hs, w_ref, w_eff["gate_up"], w_eff["down"], dout, active)
    # the same layer without the overlay differs from the oracle on the trained weights by far more than the bar
    out_plain = M.experts_routed(hs, w_ref, dequant_opseq(qg.q.cpu(), qg.s.cpu(), qg.z.cpu(), qg.shape).to(dtype),
                                 dequant_opseq(qd.q.cpu(), qd.s.cpu(), qd.z.cpu(), qd.shape).to(dtype))
    routed = w_ref != 0
    for name, got, ref in (("out", out, out_r), ("dhs", x.grad, dhs_r),
                           ("dweights", w.grad.cpu()[routed], dw_r[routed]),
                           ("sampled dW gate_up", store.compact["L.gate_up_proj"], comp["gate_up_proj"]),
                           ("sampled dW down", store.compact["L.down_proj"], comp["down_proj"])):
        check(name, got, ref, dtype, say=_say)
    sep = float((out_plain.float() - out_r.float()).abs().max() / out_r.float().abs().max())
    _say(f"  without the overlay the output would be off by rel {sep:.2e}")
    assert sep > 4 * TOL[dtype]
