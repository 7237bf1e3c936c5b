"""GPU parity of routing, bucketing, the fused expert GEMMs, the backward and
the sparse optimizer path against the CPU oracle (oracle/moe.py).

Bars: routing masks, bucket order and slot maps bit-exact; the combine
bit-exact given identical inputs; floating-point outputs within
rel = max|got - ref| / max|ref| <= 1e-2 (bf16) or 2e-3 (fp16).
"""
import numpy as np
import pytest
import torch

from oracle import moe as M
from oracle.codec_torch import dequant_opseq
from usaf_amd import _native as N
from usaf_amd import moe as G
from usaf_amd.moe_loader import SparseGradStore, overlay_scatter
from usaf_amd.sparse_optim import SparseAdam

from parity import check

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def rel_err(got, ref):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def make_layer(dev, E, H, I, T, k, dtype, seed=0, norm=False, dense=False):
    g = torch.Generator().manual_seed(seed)
    w_gu = (torch.randn(E, 2 * I, H, generator=g) * 0.02).half()
    w_dn = (torch.randn(E, H, I, generator=g) * 0.02).half()
    qg = G.Q4Tensor.quantize(w_gu.to(dev))
    qd = G.Q4Tensor.quantize(w_dn.to(dev))
    # oracle weights: the reference's CPU dequant of the same codes, in the activation dtype
    deq_g = dequant_opseq(qg.q.cpu(), qg.s.cpu(), qg.z.cpu(), qg.shape).to(dtype)
    deq_d = dequant_opseq(qd.q.cpu(), qd.s.cpu(), qd.z.cpu(), qd.shape).to(dtype)
    hs = torch.randn(T, H, generator=g).to(dtype)
    logits = torch.randn(T, E, generator=g)
    w_ref, _, _ = M.route(logits, k, norm, dtype)
    if dense:
        ew = G.ExpertWeights(deq_g.to(dev), deq_d.to(dev))
    else:
        ew = G.ExpertWeights(qg, qd)
    return dict(hs=hs, logits=logits, w=w_ref, deq_g=deq_g, deq_d=deq_d, ew=ew)


# ---- routing -----------------------------------------------------------------------

@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("ldt", [torch.float32, torch.bfloat16])
def test_route_cfg1(gpu_device, norm, ldt):
    _say(f"route T=4096 E=128 k=8 norm={norm} logits={ldt}")
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(4096, 128, generator=g).to(ldt)
    w_ref, p_ref, mask_ref = M.route(logits, 8, norm, torch.bfloat16)
    w, p = G.route_topk(logits.to(gpu_device), 8, norm, torch.bfloat16)
    torch.cuda.synchronize()
    w, p = w.cpu(), p.cpu()
    assert torch.equal(w != 0, mask_ref != 0), "routing mask differs"
    assert torch.allclose(p, p_ref, rtol=2e-6, atol=1e-9)
    # bf16 weights: equal except for rare one-ulp rounding differences of the fp32 probs
    diff = (w.float() - w_ref.float()).abs()
    assert float(diff.max()) <= 2.0 ** -8 * float(w_ref.float().abs().max())
    if ldt == torch.bfloat16:  # bf16 logits tie often: more than k selected on some tokens
        assert int((mask_ref != 0).sum(-1).max()) >= 8


def test_route_ties_brute(gpu_device):
    _say("route with forced ties")
    logits = torch.zeros(8, 16)
    logits[0, :6] = 3.0
    logits[1] = torch.arange(16.0)
    logits[2, [1, 5, 9]] = 2.0
    w_ref, _, mask_ref = M.route(logits, 4, False, torch.float32)
    w, _ = G.route_topk(logits.to(gpu_device), 4, False, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(w.cpu() != 0, mask_ref != 0)
    assert int((w.cpu()[0] != 0).sum()) == 6


def test_bucket_cfg1(gpu_device):
    _say("bucket T=4096 E=128")
    g = torch.Generator().manual_seed(8)
    w_ref, _, _ = M.route(torch.randn(4096, 128, generator=g), 8, False, torch.bfloat16)
    counts, offsets, tok, sw = M.bucket(w_ref)
    b = G.bucket_by_expert(w_ref.to(gpu_device))
    torch.cuda.synchronize()
    assert b.n_slots == int(offsets[-1])
    assert torch.equal(b.counts.cpu().long(), counts)
    assert torch.equal(b.offsets.cpu().long(), offsets)
    assert torch.equal(b.token_idx.cpu().long(), tok)
    assert torch.equal(b.slot_w.cpu(), sw)
    ps = b.pair_slot.cpu()
    assert torch.equal(ps >= 0, w_ref != 0)
    sel = ps[ps >= 0].long()
    assert torch.equal(torch.sort(sel).values, torch.arange(b.n_slots))


def test_bucket_empty_and_ragged(gpu_device):
    _say("bucket: empty experts, single token, no routed pairs")
    w = torch.zeros(5, 12, dtype=torch.bfloat16)
    w[0, 3] = 0.5
    w[4, 3] = 0.25
    w[2, 11] = 1.0
    b = G.bucket_by_expert(w.to(gpu_device))
    torch.cuda.synchronize()
    assert b.n_slots == 3 and b.token_idx.cpu().tolist() == [0, 4, 2]
    assert b.offsets.cpu().tolist() == [0, 0, 0, 0, 2, 2, 2, 2, 2, 2, 2, 2, 3]
    b0 = G.bucket_by_expert(torch.zeros(3, 4, dtype=torch.bfloat16, device=gpu_device))
    assert b0.n_slots == 0


@pytest.mark.parametrize("T,E,k", [(4096, 128, 8), (37, 12, 3), (1000, 1000, 1)])
def test_bucket_capacity_mode(gpu_device, T, E, k):
    _say(f"bucket capacity mode T={T} E={E} k={k}")
    g = torch.Generator().manual_seed(T + E)
    w_ref, _, _ = M.route(torch.randn(T, E, generator=g), k, False, torch.bfloat16)
    counts, offsets, tok, sw = M.bucket(w_ref)
    S = int(offsets[-1])
    w = w_ref.to(gpu_device)
    # capacity above the routed pairs: same buckets, zero padding, no overflow
    ovf = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    cap = S + 77
    b = G.bucket_by_expert(w, cap, ovf)
    torch.cuda.synchronize()
    assert b.n_slots == cap and int(ovf) == 0
    assert torch.equal(b.counts.cpu().long(), counts) and torch.equal(b.offsets.cpu().long(), offsets)
    assert torch.equal(b.token_idx.cpu()[:S].long(), tok) and torch.equal(b.slot_w.cpu()[:S], sw)
    assert torch.all(b.token_idx.cpu()[S:] == 0) and torch.all(b.slot_w.cpu()[S:] == 0)
    assert torch.equal(b.pair_slot.cpu(), G.bucket_by_expert(w).pair_slot.cpu())
    # capacity below: offsets clamped, later pairs dropped, overflow raised
    cap = S - S // 3 - 1
    b = G.bucket_by_expert(w, cap, ovf)
    torch.cuda.synchronize()
    assert int(ovf) == 1
    assert torch.equal(b.counts.cpu().long(), counts)
    assert torch.equal(b.offsets.cpu().long(), offsets.clamp(max=cap))
    assert torch.equal(b.token_idx.cpu().long(), tok[:cap]) and torch.equal(b.slot_w.cpu(), sw[:cap])
    ps = b.pair_slot.cpu()
    assert torch.equal(torch.sort(ps[ps >= 0]).values, torch.arange(cap, dtype=torch.int32))
    assert int((ps >= 0).sum()) == cap


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_combine_bit_exact(gpu_device, dtype):
    _say(f"combine bit-exact {dtype}")
    g = torch.Generator().manual_seed(9)
    T, E, H = 512, 32, 384
    w_ref, _, _ = M.route(torch.randn(T, E, generator=g), 4, False, dtype)
    counts, offsets, tok, sw = M.bucket(w_ref)
    y = torch.randn(int(offsets[-1]), H, generator=g).to(dtype)
    ref = M.combine_slots(y, offsets, tok, w_ref)
    b = G.bucket_by_expert(w_ref.to(gpu_device))
    out = G.combine(y.to(gpu_device), w_ref.to(gpu_device), b.pair_slot, dtype)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), ref.view(torch.int16))


# ---- forward ------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dense", [False, True])
def test_experts_forward_small(gpu_device, dtype, dense):
    _say(f"experts fwd E=8 H=256 I=128 T=300 k=2 {dtype} dense={dense}")
    L = make_layer(gpu_device, 8, 256, 128, 300, 2, dtype, seed=1, dense=dense)
    ref = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"])
    out = G.routed_experts(L["hs"].to(gpu_device), L["w"].to(gpu_device), L["ew"])
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("E,T,k", [(4, 1, 1), (2, 700, 2), (16, 37, 3), (3, 333, 3)])
def test_experts_edge_shapes(gpu_device, E, T, k):
    # one token; experts with more slots than one m-tile (700 x 2 over 2 experts);
    # experts with no tokens; every expert selected (k == E)
    _say(f"experts fwd+bwd edge E={E} T={T} k={k} bf16")
    dt = torch.bfloat16
    L = make_layer(gpu_device, E, 256, 128, T, k, dt, seed=13)
    g = torch.Generator().manual_seed(31)
    dout = torch.randn(T, 256, generator=g).to(dt)
    dhs_r, dw_r, _, _ = M.experts_routed_autograd(L["hs"], L["w"], L["deq_g"], L["deq_d"], dout)
    ref = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"])
    hs = L["hs"].to(gpu_device).requires_grad_(True)
    w = L["w"].to(gpu_device).requires_grad_(True)
    out = G.routed_experts(hs, w, L["ew"])
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= 1e-2
    assert rel_err(hs.grad, dhs_r) <= 1e-2
    routed = L["w"] != 0
    assert rel_err(w.grad.cpu()[routed], dw_r[routed]) <= 1e-2


@pytest.mark.parametrize("T", [300, 1500])
def test_experts_forward_intermediates(gpu_device, T):
    # per-slot gate_up / SwiGLU / down outputs against the oracle's per-expert tensors;
    # the blocked act^T written by the gate_up epilogue against the blocked transpose of act
    _say(f"experts fwd intermediates E=8 H=256 I=128 T={T} bf16")
    dt = torch.bfloat16
    L = make_layer(gpu_device, 8, 256, 128, T, 2, dt, seed=2)
    _, slots = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"], return_slots=True)
    b = G.bucket_by_expert(L["w"].to(gpu_device))
    ew = L["ew"]
    S, I, H = b.n_slots, ew.I, ew.H
    gu = torch.empty(S, 2 * I, dtype=dt, device=gpu_device)
    act = torch.empty(S, I, dtype=dt, device=gpu_device)
    y = torch.empty(S, H, dtype=dt, device=gpu_device)
    from usaf_amd import _native as N
    st = N.stream_ptr(gpu_device)
    q, sz, w16 = ew._ptrs("gate_up", dt)
    tb = G.blocked_layout(b.offsets, S)
    lib = N.load()
    act_blk = torch.full((int(lib.usaf_hip_blocked_elems(S, ew.E, I)),), float("nan"), dtype=dt, device=gpu_device)
    N.call("usaf_hip_moe_gate_up_fwd", L["hs"].to(gpu_device).data_ptr(), L["hs"].shape[0], H, b.token_idx.data_ptr(),
           b.offsets.data_ptr(), S, ew.E, I, q, sz, w16, N.BF16, gu.data_ptr(), act.data_ptr(), act_blk.data_ptr(),
           tb.data_ptr(), None, 0, st)
    q, sz, w16 = ew._ptrs("down", dt)
    N.call("usaf_hip_moe_down_fwd", act.data_ptr(), I, b.offsets.data_ptr(), S, ew.E, H, q, sz, w16, N.BF16,
           y.data_ptr(), None, 0, st)
    want_blk = G.slot_blocked(act, b.offsets, S, table=tb)
    torch.cuda.synchronize()
    n_used = int(want_blk.table[ew.E]) * I  # elements of the layout (the rest of the buffer is never written)
    assert n_used > 0
    assert torch.equal(act_blk[:n_used].view(torch.int16), want_blk.data[:n_used].view(torch.int16))
    offs = b.offsets.cpu().tolist()
    for e, sl in slots.items():
        s0, s1 = offs[e], offs[e + 1]
        assert torch.equal(b.token_idx[s0:s1].cpu().long(), sl["idx"])
        assert rel_err(gu[s0:s1], sl["gu"]) <= 1e-2
        assert rel_err(act[s0:s1], sl["act"]) <= 1e-2
        assert rel_err(y[s0:s1], sl["y"]) <= 1e-2


def test_experts_forward_cfg1(gpu_device):
    _say("experts fwd cfg1 Qwen3-30B-A3B: T=4096 H=2048 I=768 E=128 k=8 bf16 q4")
    dt = torch.bfloat16
    L = make_layer(gpu_device, 128, 2048, 768, 4096, 8, dt, seed=11)
    out = G.routed_experts(L["hs"].to(gpu_device), L["w"].to(gpu_device), L["ew"])
    torch.cuda.synchronize()
    torch.set_num_threads(16)
    ref = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"])
    check("cfg1 out", out, ref, dt, say=_say)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_experts_forward_dense_weights_cfg1(gpu_device, dt):
    """Dense 16-bit expert weights (the copies of the per-expert cache, the dense
    fallback of over-dense overlays) on the LDS-DMA kernel's dense-weight
    variant, at the full Qwen3 layer shape against the oracle's routed loop on
    the same weights."""
    _say(f"experts fwd cfg1 with dense {dt} weights: T=4096 H=2048 I=768 E=128 k=8")
    L = make_layer(gpu_device, 128, 2048, 768, 4096, 8, dt, seed=13, dense=True)
    out = G.routed_experts(L["hs"].to(gpu_device), L["w"].to(gpu_device), L["ew"])
    torch.cuda.synchronize()
    torch.set_num_threads(16)
    ref = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"])
    check("cfg1 out, dense weights", out, ref, dt, say=_say)


def test_experts_forward_mixtral_shape(gpu_device):
    _say("experts fwd cfg3 Mixtral shapes E=8 H=4096 I=14336 k=2 (T=192) bf16 q4")
    dt = torch.bfloat16
    L = make_layer(gpu_device, 8, 4096, 14336, 192, 2, dt, seed=12)
    out = G.routed_experts(L["hs"].to(gpu_device), L["w"].to(gpu_device), L["ew"])
    torch.cuda.synchronize()
    torch.set_num_threads(16)
    ref = M.experts_routed(L["hs"], L["w"], L["deq_g"], L["deq_d"])
    check("mixtral out", out, ref, dt, say=_say)


# ---- backward -----------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dense", [False, True])
def test_experts_backward_small(gpu_device, dtype, dense):
    _say(f"experts bwd E=8 H=256 I=128 T=300 k=2 {dtype} dense={dense}")
    E, H, I, T = 8, 256, 128, 300
    L = make_layer(gpu_device, E, H, I, T, 2, dtype, seed=3, dense=dense)
    g = torch.Generator().manual_seed(30)
    dout = torch.randn(T, H, generator=g).to(dtype)
    dhs_r, dw_r, dwg_r, dwd_r = M.experts_routed_autograd(L["hs"], L["w"], L["deq_g"], L["deq_d"], dout)
    # random 0.5 % active positions per tensor, as the bench's cfg2 mask
    nG, nD = E * 2 * I * H, E * H * I
    act_g = torch.randperm(nG, generator=g)[: max(1, nG // 200)].sort().values
    act_d = torch.randperm(nD, generator=g)[: max(1, nD // 200)]          # unsorted: exercises pos_map
    store = SparseGradStore({"L.gate_up_proj": act_g, "L.down_proj": act_d},
                            {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}, device=gpu_device)
    hs = L["hs"].to(gpu_device).requires_grad_(True)
    w = L["w"].to(gpu_device).requires_grad_(True)
    out = G.routed_experts(hs, w, L["ew"], capture=(store, "L"))
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    tol = TOL[dtype]
    assert rel_err(hs.grad, dhs_r) <= tol
    routed = L["w"] != 0
    assert torch.all(w.grad.cpu()[~routed] == 0)
    assert rel_err(w.grad.cpu()[routed], dw_r[routed]) <= tol
    cg = M.gather_compact(dwg_r, act_g)
    cd = M.gather_compact(dwd_r, act_d)
    assert rel_err(store.compact["L.gate_up_proj"], cg) <= tol
    assert rel_err(store.compact["L.down_proj"], cd) <= tol


def test_dict_capture_dense_grads(gpu_device):
    _say("experts bwd with dict grad store (dense per-expert grads)")
    E, H, I, T = 4, 256, 128, 96
    dt = torch.bfloat16
    L = make_layer(gpu_device, E, H, I, T, 2, dt, seed=4)
    dout = torch.randn(T, H, generator=torch.Generator().manual_seed(40)).to(dt)
    _, _, dwg_r, dwd_r = M.experts_routed_autograd(L["hs"], L["w"], L["deq_g"], L["deq_d"], dout)
    store = {}
    out = G.routed_experts(L["hs"].to(gpu_device).requires_grad_(True), L["w"].to(gpu_device), L["ew"],
                           capture=(store, "L"))
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    assert store["L.gate_up_proj"].dtype == torch.float16 and store["L.gate_up_proj"].shape == (E, 2 * I, H)
    assert rel_err(store["L.gate_up_proj"], dwg_r) <= 1e-2
    assert rel_err(store["L.down_proj"], dwd_r) <= 1e-2


def test_moe_block_router_backward(gpu_device):
    _say("moe block fwd+bwd incl. router softmax/top-k backward, bf16")
    E, H, I, T, k = 16, 256, 128, 200, 4
    dt = torch.bfloat16
    L = make_layer(gpu_device, E, H, I, T, k, dt, seed=5)
    g = torch.Generator().manual_seed(50)
    wr = (torch.randn(E, H, generator=g) / H ** 0.5).to(dt)
    dout = torch.randn(T, H, generator=g).to(dt)
    # oracle: the reference block on CPU with autograd
    x = L["hs"].clone().requires_grad_(True)
    wr_c = wr.clone().requires_grad_(True)
    logits = torch.nn.functional.linear(x, wr_c)
    weights, _, _ = M.route(logits, k, True, dt)
    ref = M.experts_routed(x, weights, L["deq_g"], L["deq_d"])
    ref.backward(dout)
    # GPU
    xg = L["hs"].to(gpu_device).requires_grad_(True)
    wg = wr.to(gpu_device).requires_grad_(True)
    out = G.moe_block(xg, wg, k, True, L["ew"])
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= 1e-2
    assert rel_err(xg.grad, x.grad) <= 1e-2
    assert rel_err(wg.grad, wr_c.grad) <= 1e-2


def test_moe_block_capacity_mode_matches_exact(gpu_device):
    _say("moe block with capacity-mode bucketing (no host read) == exact bucketing, bit for bit")
    E, H, I, T, k = 16, 256, 128, 200, 4
    dt = torch.bfloat16
    L = make_layer(gpu_device, E, H, I, T, k, dt, seed=7)
    g = torch.Generator().manual_seed(70)
    wr = (torch.randn(E, H, generator=g) / H ** 0.5).to(dt).to(gpu_device)
    dout = torch.randn(T, H, generator=g).to(dt).to(gpu_device)
    nG, nD = E * 2 * I * H, E * H * I
    act = {"L.gate_up_proj": torch.randperm(nG, generator=g)[: nG // 200].sort().values,
           "L.down_proj": torch.randperm(nD, generator=g)[: nD // 200].sort().values}
    shapes = {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}
    res = []
    for mode in ("exact", "capacity"):
        store = SparseGradStore(act, shapes, device=gpu_device)
        xg = L["hs"].to(gpu_device).requires_grad_(True)
        wg = wr.clone().requires_grad_(True)
        ovf = torch.zeros(1, dtype=torch.int32, device=gpu_device) if mode == "capacity" else None
        out = G.moe_block(xg, wg, k, False, L["ew"], capture=(store, "L"), overflow=ovf)
        out.backward(dout)
        torch.cuda.synchronize()
        if ovf is not None:
            assert int(ovf) == 0
        res.append([out, xg.grad, wg.grad] + [store.compact[n] for n in sorted(act)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


# ---- optimizer path ------------------------------------------------------------------

def test_sparse_adam_vs_oracle(gpu_device):
    _say("SparseAdam 3 steps, 3,019,897 elements")
    n = 3_019_897
    g = torch.Generator().manual_seed(6)
    p0 = torch.randn(n, generator=g) * 0.02
    p_ref, m_ref, v_ref = p0.clone(), torch.zeros(n), torch.zeros(n)
    master = torch.nn.Parameter(p0.clone().to(gpu_device), requires_grad=False)
    opt = SparseAdam({"w": master}, active_idx={"w": torch.arange(n)}, lr=2e-4, weight_decay=0.005,
                     compact_params=True)
    for step in range(1, 4):
        grad = torch.randn(n, generator=g) * 1e-3
        M.sparse_adam_step(p_ref, grad, m_ref, v_ref, step, 2e-4, weight_decay=0.005)
        opt.step(compact_grads={"w": grad.to(gpu_device)})
    torch.cuda.synchronize()
    # fp32 elementwise: a few ulps at most (torch's scalar tail may round differently)
    assert rel_err(master, p_ref) <= 1e-6
    assert rel_err(opt._m["w"], m_ref) <= 1e-6
    assert rel_err(opt._v["w"], v_ref) <= 1e-6


def test_sparse_adam_device_gate(gpu_device):
    """Gated on the device (finite / halt flags, GPU step count and bias table):
    the same parameters and moments as the host-stepped optimizer that skips the
    same steps, and the count of applied steps."""
    _say("SparseAdam gated on the device: 5 launches, one non-finite, one halted")
    n = 100_003
    g = torch.Generator().manual_seed(8)
    p0 = torch.randn(n, generator=g) * 0.02
    grads = [torch.randn(n, generator=g).to(gpu_device) * 1e-3 for _ in range(5)]
    gates = [(1, 0), (1, 0), (0, 0), (1, 1), (1, 0)]  # (finite, halt) per launch
    host = torch.nn.Parameter(p0.clone().to(gpu_device), requires_grad=False)
    dev_p = torch.nn.Parameter(p0.clone().to(gpu_device), requires_grad=False)
    kw = dict(lr=2e-4, weight_decay=0.005, compact_params=True)
    A = SparseAdam({"w": host}, active_idx={"w": torch.arange(n)}, **kw)
    B = SparseAdam({"w": dev_p}, active_idx={"w": torch.arange(n)}, **kw)
    for grad, (fin, halt) in zip(grads, gates):
        if fin and not halt:
            A.step(compact_grads={"w": grad})
        f = torch.tensor([fin], dtype=torch.int32, device=gpu_device)
        h = torch.tensor([halt], dtype=torch.int32, device=gpu_device)
        B.step(compact_grads={"w": grad}, finite=f, halt=h)
    torch.cuda.synchronize()
    assert B.step_count == A.step_count == 3
    assert int(B.bad.item()) == 0
    assert torch.equal(dev_p, host) and torch.equal(B._m["w"], A._m["w"]) and torch.equal(B._v["w"], A._v["w"])
    # an ungated call after gated ones keeps using (and advancing) the device count
    B.step(compact_grads={"w": grads[0]})
    A.step(compact_grads={"w": grads[0]})
    torch.cuda.synchronize()
    assert B.step_count == 4 and torch.equal(dev_p, host)


def test_sparse_adam_one_launch_for_adjacent_tensors(gpu_device):
    """Masters and gradients laid out as consecutive slices of one buffer (the
    bench's layout): the step updates them in one launch, bit-equal to separate
    tensors updated one by one, gated and ungated; a layout that breaks the
    adjacency falls back to one launch per tensor with the same result."""
    _say("SparseAdam over adjacent tensors: one launch, bit-equal to per-tensor launches")
    sizes = {"a": 70_001, "b": 30_011}
    g = torch.Generator().manual_seed(12)
    p0 = {n: torch.randn(k, generator=g) * 0.02 for n, k in sizes.items()}
    grads = [{n: torch.randn(k, generator=g) * 1e-3 for n, k in sizes.items()} for _ in range(3)]
    kw = dict(lr=2e-4, weight_decay=0.005, compact_params=True)
    idx = {n: torch.arange(k) for n, k in sizes.items()}
    flat_p = torch.cat([p0["a"], p0["b"]]).to(gpu_device)
    fused = {"a": torch.nn.Parameter(flat_p[:sizes["a"]], requires_grad=False),
             "b": torch.nn.Parameter(flat_p[sizes["a"]:], requires_grad=False)}
    single = {n: torch.nn.Parameter(p0[n].clone().to(gpu_device), requires_grad=False) for n in sizes}
    A = SparseAdam(fused, active_idx=idx, **kw)
    B = SparseAdam(single, active_idx=idx, **kw)
    assert A._m["b"].data_ptr() == A._m["a"].data_ptr() + 4 * sizes["a"]
    calls = []
    real_call = N.call

    def counting_call(fn, *args):
        calls.append(fn)
        return real_call(fn, *args)

    one = torch.ones(1, dtype=torch.int32, device=gpu_device)
    zero = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    for step, gr in enumerate(grads):
        flat_g = torch.cat([gr["a"], gr["b"]]).to(gpu_device)
        ga = {"a": flat_g[:sizes["a"]], "b": flat_g[sizes["a"]:]}
        gb = {n: gr[n].to(gpu_device) for n in sizes}
        gate = {} if step == 0 else {"finite": one, "halt": zero}
        calls.clear()
        N.call = counting_call
        try:
            A.step(compact_grads=ga, **gate)
        finally:
            N.call = real_call
        assert sum(c.startswith("usaf_hip_sparse_adam_step") for c in calls) == 1
        B.step(compact_grads=gb, **gate)
    torch.cuda.synchronize()
    for n in sizes:
        assert torch.equal(fused[n], single[n]), n
        assert torch.equal(A._m[n], B._m[n]) and torch.equal(A._v[n], B._v[n]), n
    # gradients in separate buffers: one launch per tensor, same update
    gsep = {n: grads[0][n].to(gpu_device) for n in sizes}
    calls.clear()
    N.call = counting_call
    try:
        A.step(compact_grads=gsep, finite=one, halt=zero)
    finally:
        N.call = real_call
    B.step(compact_grads=gsep, finite=one, halt=zero)
    torch.cuda.synchronize()
    assert sum(c.startswith("usaf_hip_sparse_adam_step") for c in calls) == 2
    for n in sizes:
        assert torch.equal(fused[n], single[n]), n


def test_sparse_adam_full_params(gpu_device):
    _say("SparseAdam compact_params=False")
    p = torch.nn.Parameter(torch.ones(10, device=gpu_device))
    opt = SparseAdam({"w": p}, active_idx={"w": torch.tensor([0, 1, 2, 3, 4])}, lr=1.0)
    p.grad = torch.ones(10, device=gpu_device)
    opt.step()
    torch.cuda.synchronize()
    assert float(p[0]) < 1.0 and float(p[5]) == 1.0


def test_overlay_scatter_bit_exact(gpu_device):
    _say("overlay scatter fp16")
    g = torch.Generator().manual_seed(7)
    base = torch.randn(100_000, generator=g).half()
    idx = torch.randperm(100_000, generator=g)[:500]
    vals = torch.randn(500, generator=g)
    ref = base.clone()
    ref.reshape(-1).scatter_(0, idx, vals.to(torch.float16))
    b = base.to(gpu_device)
    overlay_scatter(b, idx, vals)
    torch.cuda.synchronize()
    assert torch.equal(b.cpu().view(torch.int16), ref.view(torch.int16))
    with pytest.raises(IndexError):
        overlay_scatter(b, torch.tensor([100_000]), torch.tensor([1.0]))


def test_scale_check(gpu_device):
    _say("scale + finite check")
    from usaf_amd import _native as N
    x = torch.randn(10000, device=gpu_device)
    out = torch.empty_like(x)
    flag = torch.ones(1, dtype=torch.int32, device=gpu_device)
    N.call("usaf_hip_scale_check", x.data_ptr(), out.data_ptr(), x.numel(), 4096.0, flag.data_ptr(),
           N.stream_ptr(gpu_device))
    assert int(flag.item()) == 1 and torch.equal(out, x / 4096.0)
    x[123] = float("inf")
    N.call("usaf_hip_scale_check", x.data_ptr(), out.data_ptr(), x.numel(), 4096.0, flag.data_ptr(),
           N.stream_ptr(gpu_device))
    assert int(flag.item()) == 0


def _host_schedule(seq, init, every, lo=64.0, hi=65536.0):
    """train.py:673-677 as the reference's host code runs it, over a sequence of
    (finite, halted) steps; a halted step is not a step of the reference loop."""
    scale, good, skipped, out = init, 0, 0, []
    for finite, halted in seq:
        if not halted:
            if finite:
                good += 1
                if good % every == 0:
                    scale = min(scale * 2, hi)
            else:
                skipped += 1
                scale = max(scale / 2, lo)
        out.append((scale, good, skipped))
    return out


def test_loss_scale_schedule_on_device(gpu_device):
    _say("DeviceLossScale.update against the reference's host schedule (halve floor 64, double every 3 cap 65536)")
    from usaf_amd.sparse_optim import DeviceLossScale
    g = torch.Generator().manual_seed(5)
    # long enough to hit both the cap (from 16384 with doublings) and the floor (runs of skips)
    seq = [(bool(f), bool(h)) for f, h in zip((torch.rand(400, generator=g) < 0.8).tolist(),
                                                (torch.rand(400, generator=g) < 0.05).tolist())]
    seq[40:55] = [(False, False)] * 15  # 15 skips in a row: down to the floor
    ls = DeviceLossScale(16384.0, 3, device=gpu_device)
    one = torch.ones(1, dtype=torch.int32, device=gpu_device)
    zero = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    got = []
    for finite, halted in seq:
        ls.update(one if finite else zero, one if halted else zero)
        got.append(tuple(ls.state_dict().values()))
    want = _host_schedule(seq, 16384.0, 3)
    assert got == want
    scales = [w[0] for w in want]
    assert 64.0 in scales and 65536.0 in scales
    ls.update()  # no flags: a finite step
    assert ls.good_streak == want[-1][1] + 1


@pytest.mark.parametrize("dtype,n", [(torch.bfloat16, 4096 * 2048), (torch.float16, 4096), (torch.float16, 1003),
                                     (torch.bfloat16, 13)])
def test_loss_scale_apply_and_unscale(gpu_device, dtype, n):
    _say(f"loss_scale_apply / scale_check_state {dtype} n={n}")
    from usaf_amd.sparse_optim import DeviceLossScale
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g).to(dtype).to(gpu_device)
    x[:5] = torch.tensor([0.0, -0.0, 1e-30, 3.0e38, float("nan")]).to(dtype)
    ls = DeviceLossScale(4096.0, device=gpu_device)
    y = ls.scale_grad(x)
    ref = x * 4096.0  # torch's tensor * Python float in the dtype
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    m = ~torch.isnan(ref)
    assert torch.equal(y[m].view(torch.int16), ref[m].view(torch.int16))
    ls.scale_grad(y, out=y)  # in place
    assert torch.equal(y[m].view(torch.int16), (ref * 4096.0)[m].view(torch.int16))
    ls2 = DeviceLossScale(128.0, accum=4, device=gpu_device)
    c = torch.randn(10007, generator=g).to(gpu_device)
    out = torch.empty_like(c)
    flag = torch.ones(1, dtype=torch.int32, device=gpu_device)
    ls2.unscale_check(c, out, flag)
    assert int(flag.item()) == 1 and torch.equal(out, c / (128.0 * 4))
    c[77] = float("-inf")
    ls2.unscale_check(c, out, flag)
    assert int(flag.item()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_momentum_sgd_loss_scaled(gpu_device, dtype):
    _say(f"MomentumSGD with the device loss scale: grad.div_(scale * ACCUM) then torch's SGD step, {dtype}")
    from usaf_amd.sparse_optim import DeviceLossScale, MomentumSGD
    g = torch.Generator().manual_seed(79)
    p0 = (torch.randn(128, 2048, generator=g) * 0.05).to(dtype).to(gpu_device)
    a = p0.clone().requires_grad_(True)
    b = p0.clone().requires_grad_(True)
    ls = DeviceLossScale(1024.0, accum=2, device=gpu_device)
    ours = MomentumSGD([a], lr=2e-4, momentum=0.9, weight_decay=0.005)
    plain = MomentumSGD([b], lr=2e-4, momentum=0.9, weight_decay=0.005)
    one = torch.ones(1, dtype=torch.int32, device=gpu_device)
    for step in range(3):
        grad = (torch.randn(128, 2048, generator=g) * 2048.0).to(dtype).to(gpu_device)
        a.grad = grad.clone()
        b.grad = grad.clone()
        if step == 0:
            ours.step(loss_scale=ls)
        else:
            ours.step(finite=one, loss_scale=ls)
        b.grad.div_(1024.0 * 2)  # train.py:669-670, on the host's float
        plain.step()
        torch.cuda.synchronize()
        assert torch.equal(a.grad, grad), "the gradient buffer is left unchanged"
        assert torch.equal(a.detach(), b.detach()) and torch.equal(ours._buf[0], plain._buf[0])


# ---- slot-major operands and the sampled gradient ------------------------------------

@pytest.mark.parametrize("C,S,gathered", [(64, 333, True), (2048, 4096, False), (36, 77, True), (8, 1, False)])
def test_gather_transpose_bit_exact(gpu_device, C, S, gathered):
    _say(f"gather_transpose C={C} S={S} gathered={gathered}")
    g = torch.Generator().manual_seed(C + S)
    T = S + 5 if gathered else S
    x = torch.randn(T, C, generator=g).bfloat16()
    rows = torch.randint(0, T, (S,), generator=g, dtype=torch.int32) if gathered else None
    out = G.slot_major(x.to(gpu_device), None if rows is None else rows.to(gpu_device))
    torch.cuda.synchronize()
    ref = (x[rows.long()] if gathered else x[:S]).t()
    assert out.shape == (C, S) and out.stride(0) % 8 == 0
    assert torch.equal(out.cpu().view(torch.int16), ref.contiguous().view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sddmm_ragged_experts(gpu_device, dtype):
    _say(f"sddmm ragged experts {dtype}")
    g = torch.Generator().manual_seed(11)
    counts = [0, 3, 700, 129, 8, 1, 256]
    E, R, C = len(counts), 40, 48
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    S = offs[-1]
    dy = torch.randn(S, R, generator=g).to(dtype)
    x = torch.randn(S, C, generator=g).to(dtype)
    numel = E * R * C
    act = torch.randperm(numel, generator=g)[: numel // 5]                 # unsorted: pos_map path
    store = SparseGradStore({"L.w": act}, {"L.w": (E, R, C)}, device=gpu_device)
    init = torch.randn(act.numel(), generator=g)
    store.compact["L.w"].copy_(init)
    rowT = G.slot_major(dy.to(gpu_device))
    colT = G.slot_major(x.to(gpu_device))
    # poison the row padding: the kernel must select it out, never multiply it in
    rowT.as_strided((R, rowT.stride(0) - S), (rowT.stride(0), 1), S).fill_(float("nan"))
    offsets = torch.tensor(offs, dtype=torch.int32, device=gpu_device)
    store.add_sampled("L.w", rowT, colT, offsets, dtype)
    torch.cuda.synchronize()
    dw = torch.zeros(E, R, C, dtype=torch.float64)
    for e in range(E):
        s0, s1 = offs[e], offs[e + 1]
        dw[e] = dy[s0:s1].double().t() @ x[s0:s1].double()
    ref = init.double() + dw.reshape(-1)[act].to(dtype).double()
    got = store.compact["L.w"].cpu().double()
    assert torch.isfinite(got).all()
    assert rel_err(got - init.double(), ref - init.double()) <= TOL[dtype]
    # experts without slots contribute exact zeros
    e0 = (act // (R * C)) == 0
    assert torch.equal(got[e0], init.double()[e0])


# ---- transposed 4-bit copies for the grad-input GEMMs -----------------------------

def test_q4_transpose_bit_exact(gpu_device):
    _say("q4 transpose E=3 rows=128 cols=256")
    E, R, C = 3, 128, 256
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(E, R, C, generator=g) * 0.02).half()
    qt = G.Q4Tensor.quantize(w.to(gpu_device))
    codes_t, sz_t = qt.transposed()
    torch.cuda.synchronize()
    q = qt.q.cpu().numpy().view(np.uint8).reshape(E, R, C // 2)
    codes = np.stack([q & 15, q >> 4], axis=-1).reshape(E, R, C)           # element (r, c)
    got = codes_t.cpu().numpy().view(np.uint8).reshape(E, C, R // 2)
    got_codes = np.stack([got & 15, got >> 4], axis=-1).reshape(E, C, R)   # element (c, r)
    assert np.array_equal(got_codes, codes.transpose(0, 2, 1))
    s = qt.s.cpu().numpy().view(np.uint16).reshape(E, R, C // 128).astype(np.uint32)
    z = qt.z.cpu().numpy().view(np.uint16).reshape(E, R, C // 128).astype(np.uint32)
    words = sz_t.cpu().numpy().view(np.uint32).reshape(E, C // 128, R // 2, 2)
    exp_s = (s[:, 0::2, :] | (s[:, 1::2, :] << 16)).transpose(0, 2, 1)
    exp_z = (z[:, 0::2, :] | (z[:, 1::2, :] << 16)).transpose(0, 2, 1)
    assert np.array_equal(words[..., 0], exp_s)
    assert np.array_equal(words[..., 1], exp_z)


@pytest.mark.parametrize("E,H,I,T,k", [(128, 2048, 768, 4096, 8), (3, 384, 384, 333, 2)])
def test_backward_transposed_vs_direct(gpu_device, E, H, I, T, k):
    """The grad-input GEMMs on the transposed copies against the kernels that read
    the original layout (same dequantized weights; fp32 summation order differs)."""
    _say(f"bwd transposed vs direct E={E} H={H} I={I} T={T} k={k}")
    from usaf_amd import _native as N
    dev, dt = gpu_device, torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(5)
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, device=dev, generator=g) * 0.02).half())
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, device=dev, generator=g) * 0.02).half())
    ew = G.ExpertWeights(qg, qd)
    w, _ = G.route_topk(torch.randn(T, E, device=dev, generator=g), k, False, dt, with_probs=False)
    b = G.bucket_by_expert(w)
    S = b.n_slots
    dcur = torch.randn(S, H, device=dev, generator=g).to(dt)
    gu = torch.randn(S, 2 * I, device=dev, generator=g).to(dt)
    st, code = N.stream_ptr(dev), N.dtype_code(dt)
    dgu_a, dgu_b = torch.empty(S, 2 * I, dtype=dt, device=dev), torch.empty(S, 2 * I, dtype=dt, device=dev)
    N.call("usaf_hip_moe_down_bwd", dcur.data_ptr(), H, gu.data_ptr(), b.offsets.data_ptr(), S, E, I,
           *ew._ptrs("down", dt), code, dgu_a.data_ptr(), st)
    tq = ew._ptrs_t("down")
    assert tq is not None
    N.call("usaf_hip_moe_down_bwd_t", dcur.data_ptr(), H, gu.data_ptr(), b.offsets.data_ptr(), S, E, I, *tq,
           code, dgu_b.data_ptr(), None, 0, st)
    dx_a, dx_b = torch.empty(S, H, dtype=dt, device=dev), torch.empty(S, H, dtype=dt, device=dev)
    N.call("usaf_hip_moe_gate_up_bwd", dgu_a.data_ptr(), I, b.offsets.data_ptr(), S, E, H,
           *ew._ptrs("gate_up", dt), code, dx_a.data_ptr(), st)
    tq = ew._ptrs_t("gate_up")
    assert tq is not None
    N.call("usaf_hip_moe_gate_up_bwd_t", dgu_a.data_ptr(), I, b.offsets.data_ptr(), S, E, H, *tq, code,
           dx_b.data_ptr(), None, 0, st)
    torch.cuda.synchronize()
    assert rel_err(dgu_b, dgu_a) <= 1e-2
    assert rel_err(dx_b, dx_a) <= 1e-2
    # most elements agree exactly after the bf16 rounding
    assert float((dx_b == dx_a).float().mean()) > 0.9


# ---- per-expert blocked operands for the sampled gradient ---------------------------

def test_q4_gemm_long_mtile_list(gpu_device):
    """More m-tiles than the fused kernel's m-tile -> expert table holds (1,024):
    the kernel then searches the prefix tables per tile.  down_fwd on synthetic
    slot offsets (≈ 1,150 m-tiles, ragged experts) against an fp32 product of
    the dequantized weights on the GPU (bf16 output: rel <= 1e-2)."""
    _say("q4 down_fwd with > 1024 m-tiles (prefix-search path)")
    from usaf_amd import _native as N
    dev, dt = gpu_device, torch.bfloat16
    E, H, I = 16, 128, 128
    g = torch.Generator().manual_seed(21)
    counts = (torch.randint(15000, 21000, (E,), generator=g) + torch.arange(E) * 7).tolist()
    counts[3] = 0  # an empty expert in the list
    S = sum(counts)
    n_mt = sum((c + 255) // 256 for c in counts)
    assert n_mt > 1024
    offsets = torch.tensor([0] + list(torch.tensor(counts).cumsum(0).tolist()), dtype=torch.int32, device=dev)
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.05).half().to(dev))
    ew = G.ExpertWeights(G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.05).half().to(dev)), qd)
    act = torch.randn(S, I, generator=g).to(dt).to(dev)
    y = torch.empty(S, H, dtype=dt, device=dev)
    q, sz, w16 = ew._ptrs("down", dt)
    N.call("usaf_hip_moe_down_fwd", act.data_ptr(), I, offsets.data_ptr(), S, E, H, q, sz, w16, N.BF16, y.data_ptr(),
           None, 0, N.stream_ptr(dev))
    wd = qd.dequantize(torch.float16).to(dt).float()  # the GEMM's weight: DT(fp16 dequant)
    ref = torch.empty(S, H, dtype=torch.float32, device=dev)
    offs = offsets.tolist()
    for e in range(E):
        s0, s1 = offs[e], offs[e + 1]
        if s1 > s0:
            ref[s0:s1] = act[s0:s1].float() @ wd[e].t()
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= 1e-2


@pytest.mark.parametrize("gathered", [False, True])
def test_gather_transpose_blocked_bit_exact(gpu_device, gathered):
    _say(f"gather_transpose_blocked gathered={gathered}")
    g = torch.Generator().manual_seed(21)
    counts = [0, 3, 700, 129, 8, 1, 256, 0]
    E, C = len(counts), 136
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    S = offs[-1]
    T = S + 9 if gathered else S
    x = torch.randn(T, C, generator=g).bfloat16()
    rows = torch.randint(0, T, (S,), generator=g, dtype=torch.int32) if gathered else None
    offsets = torch.tensor(offs, dtype=torch.int32, device=gpu_device)
    blk = G.slot_blocked(x.to(gpu_device), offsets, S, None if rows is None else rows.to(gpu_device))
    torch.cuda.synchronize()
    # layout table: padded-slot prefix, 64-slot chunk prefix, chunk -> expert map
    lds = [(offs[e + 1] - offs[e] + 15) // 16 * 16 for e in range(E)]
    pre, cpre, owner = [0], [0], []
    for e in range(E):
        pre.append(pre[-1] + lds[e])
        cpre.append(cpre[-1] + (lds[e] + 63) // 64)
        owner += [e] * ((lds[e] + 63) // 64)
    table = blk.table.cpu().tolist()
    assert table[: 2 * (E + 1)] == pre + cpre
    n_map = len(table) - 2 * (E + 1)
    assert table[2 * (E + 1):] == owner + [-1] * (n_map - len(owner))
    got = blk.data.cpu().view(torch.int16)
    src = x[rows.long()] if gathered else x[:S]
    pos = 0
    for e in range(E):
        s0, s1 = offs[e], offs[e + 1]
        ld = (s1 - s0 + 15) // 16 * 16
        block = got[pos: pos + C * ld].reshape(C, ld)
        assert torch.equal(block[:, : s1 - s0], src[s0:s1].t().contiguous().view(torch.int16))
        assert torch.all(block[:, s1 - s0:] == 0)
        pos += C * ld
    assert pos <= got.numel()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,E,k,H", [(300, 12, 3, 1032), (64, 5, 2, 8), (2048, 128, 8, 2048)])
def test_combine_bwd_blocked_matches_plain(gpu_device, dtype, T, E, k, H):
    _say(f"fused combine backward + blocked transpose T={T} E={E} k={k} H={H} {dtype}")
    from usaf_amd import _native as N
    g = torch.Generator().manual_seed(T + H)
    w_ref, _, _ = M.route(torch.randn(T, E, generator=g), k, False, dtype)
    w = w_ref.to(gpu_device)
    b = G.bucket_by_expert(w, T * (k + 1), torch.zeros(1, dtype=torch.int32, device=gpu_device))
    S = b.n_slots
    dout = torch.randn(T, H, generator=g).to(dtype).to(gpu_device)
    y = torch.randn(S, H, generator=g).to(dtype).to(gpu_device)
    code, st = N.dtype_code(dtype), N.stream_ptr(gpu_device)
    # plain: combine_bwd, then the blocked gather-transpose of dcur
    dcur0 = torch.empty(S, H, dtype=dtype, device=gpu_device)
    dw0 = torch.zeros(T, E, dtype=dtype, device=gpu_device)
    N.call("usaf_hip_moe_combine_bwd", dout.data_ptr(), y.data_ptr(), b.token_idx.data_ptr(), b.slot_w.data_ptr(),
           b.offsets.data_ptr(), S, E, H, code, dcur0.data_ptr(), dw0.data_ptr(), st)
    table = G.blocked_layout(b.offsets, S)
    blk0 = G.slot_blocked(dcur0, b.offsets, S, table=table)
    # fused
    lib = N.load()
    dcur1 = torch.empty(S, H, dtype=dtype, device=gpu_device)
    dw1 = torch.zeros(T, E, dtype=dtype, device=gpu_device)
    blk1 = torch.full((int(lib.usaf_hip_blocked_elems(S, E, H)),), 7, dtype=torch.int16, device=gpu_device)
    ws = torch.empty(int(lib.usaf_hip_combine_bwd_blocked_ws_floats(S, H)), dtype=torch.float32, device=gpu_device)
    N.call("usaf_hip_moe_combine_bwd_blocked", dout.data_ptr(), y.data_ptr(), b.token_idx.data_ptr(),
           b.slot_w.data_ptr(), b.offsets.data_ptr(), table.data_ptr(), S, E, H, code, dcur1.data_ptr(),
           blk1.data_ptr(), dw1.data_ptr(), ws.data_ptr(), st)
    torch.cuda.synchronize()
    n_real = int(b.offsets[-1])
    assert torch.equal(dcur1[:n_real].view(torch.int16), dcur0[:n_real].view(torch.int16))
    used = int(table[E]) * H  # padded slots of all experts x H rows
    assert torch.equal(blk1[:used], blk0.data[:used].view(torch.int16))
    # dweights: same products, another fp32 summation order -> within one ulp of the dtype
    routed = w != 0
    assert torch.all(dw1[~routed] == 0)
    ref = torch.zeros(T, E, dtype=torch.float64)
    mag = torch.zeros(T, E, dtype=torch.float64)
    tok = b.token_idx.cpu().long()[:n_real]
    offs = b.offsets.cpu().long()
    for e in range(E):
        s0, s1 = int(offs[e]), int(offs[e + 1])
        if s1 > s0:
            p = dout.cpu().double()[tok[s0:s1]] * y.cpu().double()[s0:s1]
            ref[tok[s0:s1], e] = p.sum(1)
            mag[tok[s0:s1], e] = p.abs().sum(1)
    got = dw1.cpu().double()
    # rounding to the dtype (one ulp) plus the fp32 summation error bound
    tol = torch.finfo(dtype).eps * ref.abs() + H * 2.0 ** -23 * mag
    r = routed.cpu()
    assert torch.all((got - ref).abs()[r] <= tol[r])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sddmm_blocked_ragged_experts(gpu_device, dtype):
    _say(f"sddmm blocked ragged experts {dtype}")
    g = torch.Generator().manual_seed(12)
    counts = [0, 3, 700, 129, 8, 1, 256]
    E, R, C = len(counts), 40, 48
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    S = offs[-1]
    dy = torch.randn(S, R, generator=g).to(dtype)
    x = torch.randn(S + 4, C, generator=g).to(dtype)
    rows = torch.randperm(S + 4, generator=g)[:S].to(torch.int32)          # gathered column operand
    numel = E * R * C
    act = torch.randperm(numel, generator=g)[: numel // 5]                 # unsorted: pos_map path
    store = SparseGradStore({"L.w": act}, {"L.w": (E, R, C)}, device=gpu_device)
    init = torch.randn(act.numel(), generator=g)
    store.compact["L.w"].copy_(init)
    offsets = torch.tensor(offs, dtype=torch.int32, device=gpu_device)
    tb = G.blocked_layout(offsets, S)
    rb = G.slot_blocked(dy.to(gpu_device), offsets, S, table=tb)
    cb = G.slot_blocked(x.to(gpu_device), offsets, S, rows.to(gpu_device), table=tb)
    store.add_sampled("L.w", rb, cb, offsets, dtype)
    torch.cuda.synchronize()
    xs = x[rows.long()]
    dw = torch.zeros(E, R, C, dtype=torch.float64)
    for e in range(E):
        s0, s1 = offs[e], offs[e + 1]
        dw[e] = dy[s0:s1].double().t() @ xs[s0:s1].double()
    ref = init.double() + dw.reshape(-1)[act].to(dtype).double()
    got = store.compact["L.w"].cpu().double()
    assert torch.isfinite(got).all()
    assert rel_err(got - init.double(), ref - init.double()) <= TOL[dtype]
    e0 = (act // (R * C)) == 0
    assert torch.equal(got[e0], init.double()[e0])


def test_store_deferred_zero(gpu_device):
    _say("SparseGradStore.zero_ deferred to the first sampled add: same values as zero-then-accumulate")
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(13)
    counts = [5, 0, 300, 64]
    E, R, C = len(counts), 24, 32
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    S = offs[-1]
    numel = E * R * C
    act = torch.randperm(numel, generator=g)[: numel // 4]
    offsets = torch.tensor(offs, dtype=torch.int32, device=gpu_device)
    tb = G.blocked_layout(offsets, S)
    ops = []
    for _ in range(2):
        rb = G.slot_blocked(torch.randn(S, R, generator=g).to(dtype).to(gpu_device), offsets, S, table=tb)
        cb = G.slot_blocked(torch.randn(S, C, generator=g).to(dtype).to(gpu_device), offsets, S, table=tb)
        ops.append((rb, cb))
    fresh = SparseGradStore({"L.w": act}, {"L.w": (E, R, C)}, device=gpu_device)  # zeros, accumulating adds
    for rb, cb in ops:
        fresh.add_sampled("L.w", rb, cb, offsets, dtype)
    lazy = SparseGradStore({"L.w": act}, {"L.w": (E, R, C)}, device=gpu_device)
    lazy.compact["L.w"].fill_(123.0)
    lazy.zero_()
    assert torch.equal(lazy.compact["L.w"], torch.zeros_like(lazy.compact["L.w"]))  # reading materializes
    lazy.compact["L.w"].fill_(7.0)
    lazy.zero_()
    for rb, cb in ops:  # first add overwrites the stale 7.0 values, the second accumulates
        lazy.add_sampled("L.w", rb, cb, offsets, dtype)
    torch.cuda.synchronize()
    assert torch.equal(lazy.compact["L.w"], fresh.compact["L.w"])
    assert bool((fresh.compact["L.w"] != 0).any())


@pytest.mark.parametrize("T,E,H", [(4096, 128, 2048), (100, 16, 264), (1, 8, 8), (1000, 256, 136), (0, 8, 16)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_router_dw_vs_fp64(gpu_device, T, E, H, dtype):
    _say(f"router weight gradient T={T} E={E} H={H} {dtype}")
    from usaf_amd import _native as N
    g = torch.Generator().manual_seed(T + E + H)
    dl = torch.randn(T, E, generator=g).to(dtype)
    x = torch.randn(T, H, generator=g).to(dtype)
    lib = N.load()
    ws = torch.empty(max(1, int(lib.usaf_hip_router_dw_ws_floats(T, E, H))), dtype=torch.float32, device=gpu_device)
    dw = torch.full((E, H), 3.0, dtype=dtype, device=gpu_device)
    dl_d, x_d = dl.to(gpu_device), x.to(gpu_device)  # held until the kernel has run
    N.call("usaf_hip_router_dw", dl_d.data_ptr(), x_d.data_ptr(), T, E, H, N.dtype_code(dtype), dw.data_ptr(),
           ws.data_ptr(), N.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    ref = dl.double().t() @ x.double()
    mag = dl.double().abs().t() @ x.double().abs()
    got = dw.cpu().double()
    # one rounding to the dtype plus the fp32 summation bound
    tol = torch.finfo(dtype).eps * ref.abs() + max(T, 1) * 2.0 ** -23 * mag
    assert torch.all((got - ref).abs() <= tol)


@pytest.mark.parametrize("T,E,H", [(4096, 128, 2048), (300, 48, 136), (1, 16, 8), (129, 1024, 264)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("accumulate", [False, True])
def test_router_dx_vs_fp64(gpu_device, T, E, H, dtype, accumulate):
    """usaf_hip_router_dx: dtype(dlogits @ W), or dtype(dtype(dlogits @ W) + dx)
    (autograd's matmul rounding, then its accumulation with the experts' branch),
    against the fp64 product: one rounding per step plus the fp32 summation bound."""
    _say(f"router grad-input T={T} E={E} H={H} {dtype} accumulate={accumulate}")
    from usaf_amd import _native as N
    g = torch.Generator().manual_seed(T + 3 * E + H)
    dl = torch.randn(T, E, generator=g).to(dtype)
    w = (torch.randn(E, H, generator=g) / E ** 0.5).to(dtype)
    dx0 = torch.randn(T, H, generator=g).to(dtype)
    dl_d, w_d = dl.to(gpu_device), w.to(gpu_device)
    dx = dx0.to(gpu_device) if accumulate else torch.full((T, H), 7.0, dtype=dtype, device=gpu_device)
    N.call("usaf_hip_router_dx", dl_d.data_ptr(), w_d.data_ptr(), T, E, H, N.dtype_code(dtype), dx.data_ptr(),
           1 if accumulate else 0, N.stream_ptr(gpu_device))
    torch.cuda.synchronize()
    exact = dl.double() @ w.double()
    mag = dl.double().abs() @ w.double().abs()
    eps = torch.finfo(dtype).eps
    ref = exact + dx0.double() if accumulate else exact
    tol = eps * (exact.abs() + ref.abs()) + E * 2.0 ** -23 * mag + 1e-30
    got = dx.cpu().double()
    assert torch.all((got - ref).abs() <= tol)
    if accumulate:
        # the two roundings: the fp64 product rounded to the dtype, plus dx, rounded
        two = (exact.to(dtype).float() + dx0.float()).to(dtype)
        assert (dx.cpu() != two).float().mean() < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_momentum_sgd_matches_torch(gpu_device, dtype):
    _say(f"MomentumSGD vs torch.optim.SGD single-tensor, 3 steps from equal states, {dtype}")
    from usaf_amd.sparse_optim import MomentumSGD
    g = torch.Generator().manual_seed(77)
    p0 = (torch.randn(128, 2048, generator=g) * 0.05).to(dtype).to(gpu_device)
    a = p0.clone().requires_grad_(True)
    b = p0.clone().requires_grad_(True)
    ours = MomentumSGD([a], lr=2e-4, momentum=0.9, weight_decay=0.005)
    ref = torch.optim.SGD([b], lr=2e-4, momentum=0.9, weight_decay=0.005, foreach=False)
    for step in range(3):
        # every step starts from torch's state, so each step's arithmetic is compared alone
        with torch.no_grad():
            a.copy_(b)
            if step > 0:
                ours._buf[0].copy_(ref.state[b]["momentum_buffer"])
        grad = torch.randn(128, 2048, generator=g).to(dtype).to(gpu_device)
        a.grad = grad.clone()
        b.grad = grad.clone()
        p_prev = b.detach().clone()
        buf_prev = ref.state[b]["momentum_buffer"].clone() if step > 0 else None
        ours.step()
        ref.step()
        torch.cuda.synchronize()
        for what, x, y in (("p", a.detach(), b.detach()), ("buf", ours._buf[0], ref.state[b]["momentum_buffer"])):
            diff = (x.float() - y.float()).abs()
            # equal except where an fp32 multiply-add rounds one way fused and the other
            # unfused and the 16-bit result flips by one ulp
            ulp = torch.finfo(dtype).eps * y.float().abs() + 2.0 ** -24
            k = int(torch.argmax(diff - ulp))
            assert torch.all(diff <= ulp), (
                f"step {step} {what}[{k}]: ours {float(x.flatten()[k])!r} torch {float(y.flatten()[k])!r}, "
                f"grad {float(grad.flatten()[k])!r} p_prev {float(p_prev.flatten()[k])!r} buf_prev "
                f"{None if buf_prev is None else float(buf_prev.flatten()[k])!r} buf ours "
                f"{float(ours._buf[0].flatten()[k])!r} torch {float(ref.state[b]['momentum_buffer'].flatten()[k])!r}")
            assert float((diff > 0).float().mean()) < 1e-3


def test_momentum_sgd_device_gate(gpu_device):
    _say("MomentumSGD gated on device flags: closed gates leave p and buf untouched, open = ungated step")
    from usaf_amd.sparse_optim import MomentumSGD
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(78)
    p0 = (torch.randn(64, 512, generator=g) * 0.05).to(dt).to(gpu_device)
    grads = [torch.randn(64, 512, generator=g).to(dt).to(gpu_device) for _ in range(3)]
    one = torch.ones(1, dtype=torch.int32, device=gpu_device)
    zero = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    a = p0.clone().requires_grad_(True)
    b = p0.clone().requires_grad_(True)
    ours = MomentumSGD([a], lr=2e-4, momentum=0.9, weight_decay=0.005)
    plain = MomentumSGD([b], lr=2e-4, momentum=0.9, weight_decay=0.005)
    # first step of the buffer: the gate is read on the host; a closed one creates nothing
    a.grad = grads[0].clone()
    ours.step(finite=zero, halt=zero)
    assert not ours._buf and torch.equal(a.detach(), p0)
    ours.step(finite=one, halt=zero)
    b.grad = grads[0].clone()
    plain.step()
    torch.cuda.synchronize()
    assert torch.equal(a.detach(), b.detach()) and torch.equal(ours._buf[0], plain._buf[0])
    for closed in ((zero, zero), (one, one), (zero, one)):
        p_before, buf_before = a.detach().clone(), ours._buf[0].clone()
        a.grad = grads[1].clone()
        ours.step(finite=closed[0], halt=closed[1])
        torch.cuda.synchronize()
        assert torch.equal(a.detach(), p_before) and torch.equal(ours._buf[0], buf_before)
    for gr in grads[1:]:
        a.grad = gr.clone()
        b.grad = gr.clone()
        ours.step(finite=one, halt=zero)
        plain.step()
        torch.cuda.synchronize()
        assert torch.equal(a.detach(), b.detach()) and torch.equal(ours._buf[0], plain._buf[0])


@pytest.mark.parametrize("T,E,H,k,norm", [(4096, 128, 2048, 8, False), (333, 60, 768, 4, True), (5, 8, 256, 2, False),
                                          (77, 200, 512, 6, False)])
def test_router_fwd_exact_logits(gpu_device, T, E, H, k, norm):
    _say(f"fused router forward T={T} E={E} H={H} k={k} norm={norm}")
    from usaf_amd import _native as N
    g = torch.Generator().manual_seed(T + E)
    # few-bit operands: every fp32 partial sum is exact, so the logits are the
    # fp64 result rounded once to bf16 whatever the summation order
    x = (torch.randint(-4, 5, (T, H), generator=g).float() / 8).to(torch.bfloat16)
    w = (torch.randint(-4, 5, (E, H), generator=g).float() / 16).to(torch.bfloat16)
    logits = (x.double() @ w.double().t()).to(torch.bfloat16)
    w_ref, p_ref, _ = M.route(logits, k, norm, torch.bfloat16)
    xd, wd = x.to(gpu_device), w.to(gpu_device)
    weights = torch.empty(T, E, dtype=torch.bfloat16, device=gpu_device)
    probs = torch.empty(T, E, dtype=torch.float32, device=gpu_device)
    lg = torch.empty(T, E, dtype=torch.bfloat16, device=gpu_device)
    N.call("usaf_hip_router_fwd", xd.data_ptr(), wd.data_ptr(), T, E, H, N.BF16, k, 1 if norm else 0,
           lg.data_ptr(), weights.data_ptr(), N.BF16, probs.data_ptr(), N.stream_ptr(gpu_device))
    # the same logits through the unfused routing kernel
    w2, p2 = G.route_topk(logits.to(gpu_device), k, norm, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(lg.cpu().view(torch.int16), logits.view(torch.int16))
    assert torch.equal(weights.cpu() != 0, w_ref != 0), "routing mask differs from the oracle"
    assert torch.equal(weights.cpu().view(torch.int16), w2.cpu().view(torch.int16))
    assert torch.equal(probs.cpu(), p2.cpu())
