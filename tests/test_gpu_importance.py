"""GPU importance selection and RigL reselect (usaf/moe_loader.py:584-631,
train.py:536-613) against the oracle's restatements (oracle/moe.py
topk_store_candidates / topk_store_select / reselect_merge, which use the
reference's torch.topk and Python sets).

Bars: selections are equal as index sets where magnitudes are distinct; with
ties at the k-th magnitude the sets may differ only in positions carrying that
magnitude, and the kernel must take the tied ones from the lowest positions;
merged active sets and masters bit-exact; gathered dequant values bit-exact
against the C oracle's dequant.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import moe as M
from usaf_amd import moe as G
from usaf_amd.importance import TopKImportanceStore, dequant_at, reselect_active, topk_abs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _distinct(n, g, dtype=torch.float32):
    """n values of `dtype` with pairwise distinct, finite, nonzero magnitudes, random signs."""
    sign = torch.randint(0, 2, (n,), generator=g)
    if dtype == torch.float32:
        return (torch.randperm(n, generator=g).float() + 1.0) * (sign * 2 - 1)
    top = 0x7F7F if dtype == torch.bfloat16 else 0x7BFF  # largest finite magnitude pattern
    pats = torch.randperm(top, generator=g)[:n] + 1
    return (pats | (sign << 15)).to(torch.int16).view(dtype)


def _check_tie_aware(pos, x, k):
    """pos: the kernel's selection of the k largest |x| (CPU tensors)."""
    mag = x.float().abs()
    mag = torch.where(torch.isnan(mag), torch.full_like(mag, float("inf")), mag)  # NaN ranks first
    assert pos.numel() == k
    assert torch.all(pos[1:] > pos[:-1]), "positions must ascend"
    sel = torch.zeros(x.numel(), dtype=torch.bool)
    sel[pos] = True
    thr = mag[sel].min()
    assert torch.all(mag[~sel] <= thr) and torch.all(mag[sel] >= thr)
    tied = (mag == thr).nonzero().reshape(-1)
    taken = sel[tied]
    # the tied positions taken are a prefix of the tied positions
    assert not torch.any(taken[1:] & ~taken[:-1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_topk_abs_distinct_matches_torch(gpu_device, dtype):
    # one Qwen3 gate_up expert slice (1536 x 2048) at the reference's candidate count
    n = 1536 * 2048 if dtype == torch.float32 else 20000
    k = max(1, int(n * 0.005 * 2.0))
    _say(f"topk_abs distinct n={n} k={k} {dtype}")
    g = torch.Generator().manual_seed(n)
    x = _distinct(n, g, dtype)
    pos, vals = topk_abs(x.to(gpu_device), k)
    torch.cuda.synchronize()
    ref_v, ref_i = torch.topk(x.float().abs(), k)
    assert set(pos.cpu().tolist()) == set(ref_i.tolist())
    assert torch.equal(vals.cpu(), x.float().abs()[pos.cpu()])


@pytest.mark.parametrize("n,k", [(1536 * 2048, 31457), (4097, 100), (5000, 5000), (7, 50), (1, 1), (70000, 1)])
def test_topk_abs_ties_bf16(gpu_device, n, k):
    _say(f"topk_abs bf16 with ties n={n} k={k}")
    g = torch.Generator().manual_seed(7 + n)
    x = (torch.randn(n, generator=g) * 1e-3).bfloat16()  # bf16: many equal magnitudes
    pos, _ = topk_abs(x.to(gpu_device), k)
    torch.cuda.synchronize()
    _check_tie_aware(pos.cpu(), x, min(k, n))


def test_topk_abs_nan_inf(gpu_device):
    _say("topk_abs: NaN ranks above inf, inf above finite")
    x = torch.randn(10000, generator=torch.Generator().manual_seed(3))
    x[[17, 4000]] = float("nan")
    x[[5, 9000, 9001]] = float("-inf")
    pos, vals = topk_abs(x.to(gpu_device), 6)
    torch.cuda.synchronize()
    assert set(pos.cpu().tolist()) >= {17, 4000, 5, 9000, 9001}
    assert torch.isinf(vals.cpu()).sum() == 3 and torch.isnan(vals.cpu()).sum() == 2


def test_importance_store_matches_reference_store(gpu_device):
    # fp32 dense gradients (distinct magnitudes): per-expert candidates and the
    # global selection equal the reference store's as sets
    E, R, C, frac = 8, 512, 768, 0.005
    _say(f"TopKImportanceStore E={E} [{R},{C}] frac={frac}")
    g = torch.Generator().manual_seed(11)
    grads = [_distinct(R * C, g).reshape(R, C) * 1e-6 for _ in range(E)]
    store = TopKImportanceStore({"L.w": (E, R, C)}, frac=frac)
    cands = []
    for ei in range(E):
        store.add("L.w", ei, grads[ei].to(gpu_device))
        cands.append(M.topk_store_candidates(grads[ei], ei, frac))
    assert store.n_captured() == E
    sel = store.select()["L.w"].cpu()
    ref = M.topk_store_select(cands, E * R * C, frac)
    assert set(sel.tolist()) == set(ref.tolist())


def test_importance_pass_through_moe_backward(gpu_device):
    # the reference's reselect pass: dense per-expert gradients from the expert
    # backward go to the store through the capture protocol (bf16: tied
    # magnitudes are common, so the sets are compared tie-aware)
    E, H, I, T, k, frac = 8, 256, 128, 300, 2, 0.005
    _say("importance pass through routed_experts backward (capture protocol)")
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(12)
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(gpu_device))
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(gpu_device))
    hs = torch.randn(T, H, generator=g).to(dt).to(gpu_device)
    w, _, _ = M.route(torch.randn(T, E, generator=g), k, False, dt)
    dout = torch.randn(T, H, generator=g).to(dt).to(gpu_device)

    class Recorder:
        def __init__(self):
            self.grads = {}

        def add(self, name, ei, gr):
            self.grads[(name, ei)] = gr.detach().clone()

    rec = Recorder()
    out = G.routed_experts(hs.requires_grad_(True), w.to(gpu_device), G.ExpertWeights(qg, qd), capture=(rec, "L"))
    out.backward(dout)
    shapes = {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}
    store = TopKImportanceStore(shapes, frac=frac)
    out = G.routed_experts(hs, w.to(gpu_device), G.ExpertWeights(qg, qd), capture=(store, "L"))
    out.backward(dout)
    sel = store.select()
    torch.cuda.synchronize()
    for name, shape in shapes.items():
        numel = int(np.prod(shape))
        per = numel // E
        dense = torch.zeros(numel)
        cands = []
        for ei in range(E):
            gr = rec.grads.get((name, ei))
            if gr is None:
                continue
            dense[ei * per:(ei + 1) * per] = gr.float().cpu().reshape(-1)
            cands.append(M.topk_store_candidates(gr.cpu(), ei, frac))
        ref = M.topk_store_select(cands, numel, frac)
        got = sel[name].cpu()
        assert got.numel() == ref.numel()
        mag = dense.abs()
        thr = float(mag[ref].min())
        # a tie can be broken differently at the global threshold, and at an
        # expert's own candidate threshold when that lies above the global one
        # (then every candidate of the expert is selected)
        t_e = {int(c[1][0]) // per: float(c[0].min()) for c in cands}
        diff = set(got.tolist()) ^ set(ref.tolist())
        bad = [i for i in diff if float(mag[i]) not in (thr, t_e.get(i // per))]
        assert not bad, f"{name}: {len(bad)} positions differ beyond tied magnitudes"


def test_dequant_at_bit_exact(gpu_device):
    _say("dequant_q4_at vs the C oracle's dequant")
    g = torch.Generator().manual_seed(13)
    for shape, gs in (((64, 384), 128), ((5, 7), 3), ((1000,), 64)):
        w = torch.randn(shape, generator=g) * 0.05
        q = G.Q4Tensor.quantize(w.to(gpu_device), group_size=gs)
        full = oracle.dequant(q.q.cpu().numpy(), q.s.cpu().numpy(), q.z.cpu().numpy(), q.numel(), gs)
        idx = torch.randint(0, q.numel(), (333,), generator=g)
        got = dequant_at(q, idx.to(gpu_device)).cpu()
        want = torch.from_numpy(full.view(np.float16)[idx.numpy()].astype(np.float32))
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    with pytest.raises(IndexError):
        dequant_at(q, torch.tensor([q.numel()], device=gpu_device))


@pytest.mark.parametrize("case", ["overlap", "duplicates", "short_new", "empty_new"])
def test_reselect_active_matches_reference_merge(gpu_device, case):
    _say(f"reselect_active vs the reference merge: {case}")
    g = torch.Generator().manual_seed({"overlap": 1, "duplicates": 2, "short_new": 3, "empty_new": 4}[case])
    E, R, C = 4, 128, 256
    q = G.Q4Tensor.quantize((torch.randn(E, R, C, generator=g) * 0.02).half().to(gpu_device))
    numel = q.numel()
    old = torch.randperm(numel, generator=g)[:2000]
    if case == "duplicates":
        old = torch.cat([old, old[:50]])
    masters = torch.randn(old.numel(), generator=g)
    if case == "empty_new":
        new = torch.tensor([], dtype=torch.long)
    elif case == "short_new":
        new = torch.cat([old[:1500], torch.randperm(numel, generator=g)[:100]])
    else:
        new = torch.cat([old[:1000], torch.randperm(numel, generator=g)[:3000]])
    deq = torch.from_numpy(oracle.dequant(q.q.cpu().numpy(), q.s.cpu().numpy(), q.z.cpu().numpy(), numel)
                           .view(np.float16).copy())
    ref_f, ref_v = M.reselect_merge(old, masters, new, deq)
    got_f, got_v, counts = reselect_active(old.to(gpu_device), masters.to(gpu_device),
                                           new.to(gpu_device) if new.numel() else None, q)
    torch.cuda.synchronize()
    assert torch.equal(got_f.cpu(), ref_f)
    assert torch.equal(got_v.cpu().view(torch.int32), ref_v.view(torch.int32))
    assert counts["kept"] + counts["grown"] == ref_f.numel()
