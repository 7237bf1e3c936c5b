"""Pins the MoE part of the oracle (oracle/moe.py) on the CPU.

Checks: brute force on tiny inputs (routing threshold with ties, stable
bucketing), the reference's claim that the routed and dense-masked forwards
agree (benchmarks/kaggle_t4_bench.py:245-250), the float64 closed form of the
expert layer, closed-form Adam steps, and the reference's own qualitative
SparseAdam tests (tests/test_sparse_optim.py:21-49).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as M


def test_route_threshold_brute_force_with_ties():
    g = torch.Generator().manual_seed(0)
    T, E, k = 64, 16, 4
    logits = torch.randn(T, E, generator=g)
    logits[0, :6] = 2.5          # six-way tie at the top: all six selected
    logits[1, 3] = logits[1, 7] = logits[1].max() + 1  # tie among the top two
    logits = logits.bfloat16().float()  # bf16-valued logits produce more ties
    w, probs, mask = M.route(logits, k, False, torch.float32)
    for t in range(T):
        p = probs[t].tolist()
        thr = sorted(p, reverse=True)[k - 1]
        sel = [e for e in range(E) if p[e] >= thr]
        assert mask[t].nonzero().reshape(-1).tolist() == sel
        assert len(sel) >= k
    assert int(mask[0].sum()) == 6
    # softmax against float64 closed form
    ref = torch.softmax(logits.double(), -1)
    assert torch.allclose(probs.double(), ref, rtol=1e-6, atol=1e-9)


def test_route_renorm_sums_to_one():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(32, 128, generator=g)
    w, _, mask = M.route(logits, 8, True, torch.float32)
    assert torch.allclose(w.sum(-1), torch.ones(32), atol=1e-6)
    assert torch.all((w != 0) == (mask != 0))


def test_bucket_brute_force():
    g = torch.Generator().manual_seed(2)
    T, E = 50, 7
    w = (torch.rand(T, E, generator=g) < 0.3).float() * torch.rand(T, E, generator=g)
    counts, offsets, tok, sw = M.bucket(w)
    exp_tok = []
    exp_w = []
    for e in range(E):
        for t in range(T):
            if w[t, e] != 0:
                exp_tok.append(t)
                exp_w.append(float(w[t, e]))
        assert int(counts[e]) == sum(1 for t in range(T) if w[t, e] != 0)
    assert tok.tolist() == exp_tok
    assert sw.tolist() == pytest.approx(exp_w)
    assert offsets[-1] == len(exp_tok) and offsets[0] == 0


def _layer(E=8, H=128, I=64, T=40, k=2, dtype=torch.bfloat16, seed=3):
    g = torch.Generator().manual_seed(seed)
    hs = torch.randn(T, H, generator=g).to(dtype)
    wg = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(dtype)
    wd = (torch.randn(E, H, I, generator=g) * 0.05).to(dtype)
    logits = torch.randn(T, E, generator=g)
    w, _, _ = M.route(logits, k, False, dtype)
    return hs, w, wg, wd


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_routed_equals_dense_masked(dtype):
    hs, w, wg, wd = _layer(dtype=dtype)
    a = M.experts_dense_masked(hs, w, wg, wd)
    b = M.experts_routed(hs, w, wg, wd)
    rel = (a.float() - b.float()).abs().max() / a.float().abs().max()
    assert rel <= (1e-2 if dtype == torch.bfloat16 else 2e-3)


def test_expert_layer_vs_float64_closed_form():
    hs, w, wg, wd = _layer(dtype=torch.float32)
    out = M.experts_routed(hs, w, wg, wd).double()
    x, W, G, D = hs.double(), w.double(), wg.double(), wd.double()
    ref = torch.zeros_like(x)
    for e in range(G.shape[0]):
        gu = x @ G[e].t()
        I = D.shape[2]
        a = F.silu(gu[:, :I]) * gu[:, I:]
        ref += (a @ D[e].t()) * W[:, e:e + 1]
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_backward_dweights_closed_form():
    hs, w, wg, wd = _layer(dtype=torch.float32)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(hs.shape, generator=g)
    dhs, dw, dwg, dwd = M.experts_routed_autograd(hs, w, wg, wd, dout)
    _, slots = M.experts_routed(hs, w, wg, wd, return_slots=True)
    for e, s in slots.items():
        exp = (dout[s["idx"]] * s["y"]).sum(-1)
        assert torch.allclose(dw[s["idx"], e], exp, rtol=1e-5, atol=1e-6)
        # dW_down = dcur^T act, dcur = dout * w
        dcur = dout[s["idx"]] * w[s["idx"], e:e + 1]
        assert torch.allclose(dwd[e], dcur.t() @ s["act"], rtol=1e-4, atol=1e-6)


def test_gather_compact_brute_force():
    g = torch.Generator().manual_seed(4)
    dense = torch.randn(3, 5, 7, generator=g).half()
    idx = torch.tensor([0, 9, 50, 104])
    out = M.gather_compact(dense, idx)
    flat = dense.reshape(-1)
    assert out.tolist() == [float(flat[i]) for i in idx.tolist()]


def test_sparse_adam_closed_form_first_steps():
    g = torch.Generator().manual_seed(5)
    p = torch.randn(1000, generator=g)
    grad = torch.randn(1000, generator=g)
    m = torch.zeros(1000)
    v = torch.zeros(1000)
    lr, wd, eps = 1e-2, 0.005, 1e-8
    p0 = p.clone()
    M.sparse_adam_step(p, grad, m, v, 1, lr, weight_decay=wd, eps=eps)
    gg = grad.double() + wd * p0.double()
    # step 1: m_hat = g, v_hat = g^2 -> update = g / (|g| + eps)
    exp = p0.double() - lr * gg / (gg.abs() + eps)
    assert torch.allclose(p.double(), exp, rtol=0, atol=1e-6)
    # step 2 closed form
    p1 = p.clone()
    grad2 = torch.randn(1000, generator=g)
    M.sparse_adam_step(p, grad2, m, v, 2, lr, weight_decay=wd, eps=eps)
    g2 = grad2.double() + wd * p1.double()
    m2 = 0.9 * 0.1 * gg + 0.1 * g2
    v2 = 0.999 * 0.001 * gg ** 2 + 0.001 * g2 ** 2
    upd = (m2 / (1 - 0.9 ** 2)) / ((v2 / (1 - 0.999 ** 2)).sqrt() + eps)
    assert torch.allclose(p.double(), p1.double() - lr * upd, rtol=0, atol=2e-6)


def test_sparse_adam_reference_qualitative():
    # tests/test_sparse_optim.py:41-49 pattern: active params decrease under positive grads
    p = torch.ones(3)
    m, v = torch.zeros(3), torch.zeros(3)
    M.sparse_adam_step(p, torch.ones(3), m, v, 1, 1.0)
    assert bool((p < 1.0).all())
    assert math.isclose(float(p[0]), 0.0, abs_tol=1e-6)  # 1 - 1.0 * 1/(1+1e-8)


def test_backward_dhs_dwgate_closed_form():
    # float64 closed form of the SwiGLU expert backward: dact = (dout * w) Wd,
    # dgate = dact * up * silu'(gate), dup = dact * silu(gate), dgu = [dgate, dup],
    # dhs = sum_e dgu_e Wgu_e, dWgu_e = dgu_e^T x_e
    hs, w, wg, wd = _layer(dtype=torch.float32)
    g = torch.Generator().manual_seed(10)
    dout = torch.randn(hs.shape, generator=g)
    dhs, _, dwg, _ = M.experts_routed_autograd(hs, w, wg, wd, dout)
    x, W, G, D, dO = hs.double(), w.double(), wg.double(), wd.double(), dout.double()
    I = D.shape[2]
    dhs_ref = torch.zeros_like(x)
    for e in range(G.shape[0]):
        idx = torch.nonzero(W[:, e]).reshape(-1)
        if idx.numel() == 0:
            assert torch.all(dwg[e] == 0)
            continue
        xe = x[idx]
        gu = xe @ G[e].t()
        gate, up = gu[:, :I], gu[:, I:]
        sig = torch.sigmoid(gate)
        dact = (dO[idx] * W[idx, e:e + 1]) @ D[e]
        dgate = dact * up * (sig * (1 + gate * (1 - sig)))
        dup = dact * gate * sig
        dgu = torch.cat([dgate, dup], 1)
        dhs_ref.index_add_(0, idx, dgu @ G[e])
        assert torch.allclose(dwg[e].double(), dgu.t() @ xe, rtol=1e-4, atol=1e-6)
    assert torch.allclose(dhs.double(), dhs_ref, rtol=1e-4, atol=1e-6)


def test_combine_slots_brute_force():
    g = torch.Generator().manual_seed(12)
    T, E, H = 30, 5, 16
    w = (torch.rand(T, E, generator=g) < 0.4).float() * torch.rand(T, E, generator=g)
    counts, offsets, tok, _ = M.bucket(w)
    y = torch.randn(int(offsets[-1]), H, generator=g)
    out = M.combine_slots(y, offsets, tok, w)
    ref = torch.zeros(T, H, dtype=torch.float64)
    for e in range(E):
        for s in range(int(offsets[e]), int(offsets[e + 1])):
            t = int(tok[s])
            ref[t] += y[s].double() * float(w[t, e])
    assert torch.allclose(out.double(), ref, rtol=1e-6, atol=1e-6)
    assert torch.all(out[(w != 0).sum(1) == 0] == 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_manual_backward_matches_autograd(dtype):
    # experts_routed_manual (fp32 ops rounded at the reference's dtype op
    # outputs, sampled weight gradient only) against the dtype autograd oracle;
    # the two differ only in fp32 summation order and in where several
    # experts' token gradients are added
    g = torch.Generator().manual_seed(21)
    E, H, I, T, k = 8, 256, 128, 300, 2
    wg = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(dtype)
    wd = (torch.randn(E, H, I, generator=g) * 0.02).to(dtype)
    hs = torch.randn(T, H, generator=g).to(dtype)
    w, _, _ = M.route(torch.randn(T, E, generator=g), k, False, dtype)
    dout = torch.randn(T, H, generator=g).to(dtype)
    nG, nD = wg.numel(), wd.numel()
    active = {"gate_up_proj": torch.randperm(nG, generator=g)[: nG // 200],
              "down_proj": torch.randperm(nD, generator=g)[: nD // 200]}
    out_m, dhs_m, dw_m, comp = M.experts_routed_manual(hs, w, wg, wd, dout, active)
    out_a = M.experts_routed(hs, w, wg, wd)
    dhs_a, dw_a, dwg_a, dwd_a = M.experts_routed_autograd(hs, w, wg, wd, dout)
    tol = 1e-2 if dtype == torch.bfloat16 else 2e-3

    def rel(a, b):
        return float((a.float() - b.float()).abs().max() / b.float().abs().max())

    assert rel(out_m, out_a) <= tol / 4
    assert rel(dhs_m, dhs_a) <= tol / 4
    routed = w != 0
    assert torch.all(dw_m[~routed] == 0)
    assert rel(dw_m[routed], dw_a[routed]) <= tol / 4
    assert rel(comp["gate_up_proj"], M.gather_compact(dwg_a, active["gate_up_proj"])) <= tol / 4
    assert rel(comp["down_proj"], M.gather_compact(dwd_a, active["down_proj"])) <= tol / 4


def test_topk_store_oracle_against_full_sort():
    # distinct magnitudes: the reference's topk selection equals a full sort's head
    g = torch.Generator().manual_seed(5)
    E, R, C, frac, cand = 3, 40, 50, 0.01, 2.0
    grads = [((torch.randperm(R * C, generator=g).float() + 1) * (torch.randint(0, 2, (R * C,), generator=g) * 2 - 1))
             .reshape(R, C) for _ in range(E)]
    cands = []
    for ei, gr in enumerate(grads):
        v, i = M.topk_store_candidates(gr, ei, frac, cand)
        k = max(1, int(R * C * frac * cand))
        flat = gr.reshape(-1).abs()
        order = torch.argsort(flat, descending=True)[:k]
        assert set(i.tolist()) == set((order + ei * R * C).tolist())
        assert torch.equal(v, flat[order])
        cands.append((v, i))
    sel = M.topk_store_select(cands, E * R * C, frac)
    allv = torch.cat([c[0] for c in cands])
    alli = torch.cat([c[1] for c in cands])
    k = max(1, int(E * R * C * frac))
    assert set(sel.tolist()) == set(alli[torch.argsort(allv, descending=True)[:k]].tolist())


def test_reselect_merge_oracle_hand_example():
    # old {5, 2, 9, 7}, new {9, 3, 1, 5, 8}: kept [5, 9]; newcomers [1, 3, 8];
    # fill 4 - 2 = 2 -> grown [1, 3]; kept masters carried, grown from the weights
    old = torch.tensor([5, 2, 9, 7])
    masters = torch.tensor([0.5, 0.2, 0.9, 0.7])
    new = torch.tensor([9, 3, 1, 5, 8])
    deq = (torch.arange(12) * 10).half()
    final, vals = M.reselect_merge(old, masters, new, deq)
    assert final.tolist() == [5, 9, 1, 3]
    assert vals.tolist() == [0.5, pytest.approx(0.9), 10.0, 30.0]
    # an empty selection keeps the old set and masters
    f2, v2 = M.reselect_merge(old, masters, torch.tensor([], dtype=torch.long), deq)
    assert torch.equal(f2, old) and torch.equal(v2, masters)
    # fewer newcomers than free slots: the set shrinks
    f3, _ = M.reselect_merge(old, masters, torch.tensor([9, 11]), deq)
    assert f3.tolist() == [9, 11]


def test_lru_model_hand_sequence():
    from oracle.cache import LRUModel
    m = LRUModel(3)
    trace = [m.access(k) for k in "abcabdaeb"]
    # a b c miss; a b hit (order c a b); d misses and evicts c; a hits (b d a);
    # e misses and evicts b (d a e); b misses and evicts d (a e b)
    assert [h for h, _ in trace] == [False, False, False, True, True, False, True, False, False]
    assert [ev for _, ev in trace] == [[], [], [], [], [], ["c"], [], ["b"], ["d"]]
    assert m.keys() == ["a", "e", "b"]
