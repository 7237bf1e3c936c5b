"""The routed-expert step captured as one HIP graph (usaf_amd.graphs) against
the same step launched eagerly: bit-identical on every replay, with eager work,
host reads and in-place input updates between the replays."""
import pytest
import torch

from usaf_amd import moe as G
from usaf_amd import _native as N
from usaf_amd import graphs
from usaf_amd.graphs import CapturedStep
from usaf_amd.moe_loader import SparseGradStore

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(bool(graphs.DISABLED), reason="HIP-graph capture of the MoE step is switched off: "
                                 "its first run segfaulted in torch.cuda.graph capture_end (cause not identified)")]


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _layer(dev, E=16, H=256, I=128, T=200, k=4, seed=11):
    g = torch.Generator().manual_seed(seed)
    dt = torch.bfloat16
    qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(dev))
    qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(dev))
    nG, nD = E * 2 * I * H, E * H * I
    act = {"L.gate_up_proj": torch.randperm(nG, generator=g)[: nG // 200].sort().values,
           "L.down_proj": torch.randperm(nD, generator=g)[: nD // 200].sort().values}
    shapes = {"L.gate_up_proj": (E, 2 * I, H), "L.down_proj": (E, H, I)}
    return dict(ew=G.ExpertWeights(qg, qd), k=k,
                store=SparseGradStore(act, shapes, device=dev),
                hs=torch.randn(T, H, generator=g).to(dt).to(dev).requires_grad_(True),
                wr=(torch.randn(E, H, generator=g) / H ** 0.5).to(dt).to(dev).requires_grad_(True),
                dy=torch.randn(T, H, generator=g).to(dt).to(dev),
                flag=torch.ones(2, dtype=torch.int32, device=dev))


def _step(L):
    """Forward + backward + finite check, as bench.py's captured step."""
    store, flag = L["store"], L["flag"]
    store.zero_()
    L["hs"].grad = None
    L["wr"].grad = None
    flag.fill_(1)
    flag[1:].fill_(0)
    out = G.moe_block(L["hs"], L["wr"], L["k"], False, L["ew"], capture=(store, "L"), overflow=flag[1:])
    out.backward(L["dy"])
    dev = L["hs"].device
    cg = {}
    for name, v in store.compact.items():
        o = L.setdefault(f"cg:{name}", torch.empty_like(v))
        N.call("usaf_hip_scale_check", v.data_ptr(), o.data_ptr(), v.numel(), 1.0, flag.data_ptr(),
               N.stream_ptr(dev))
        cg[name] = o
    return out, cg


def _snapshot(L, out, cg):
    return [out.clone(), L["hs"].grad.clone(), L["wr"].grad.clone(), L["flag"].clone()] + \
           [cg[n].clone() for n in sorted(cg)]


def test_captured_step_replays_match_eager(gpu_device):
    _say("moe step captured as a HIP graph: 3 replays vs eager, router weight updated in place between")
    L = _layer(gpu_device)
    ref_eager = _snapshot(L, *_step(L))
    cap = CapturedStep(lambda: _step(L), warmup=2, device=gpu_device)
    graph_grads = (L["hs"].grad, L["wr"].grad)
    with torch.no_grad():
        wr0 = L["wr"].detach().clone()
    for r in range(3):
        # in-place input update between replays (as an optimizer step would do)
        with torch.no_grad():
            L["wr"].copy_(wr0 * (1.0 + 0.25 * r))
        torch.cuda.synchronize()
        out, cg = cap.replay()
        got = [out.clone(), graph_grads[0].clone(), graph_grads[1].clone(), L["flag"].clone()] + \
              [cg[n].clone() for n in sorted(cg)]
        torch.cuda.synchronize()
        assert L["flag"].tolist() == [1, 0]
        # the same step launched eagerly (it rebinds .grad; the graph keeps writing graph_grads)
        want = _snapshot(L, *_step(L))
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {r} differs from the eager step"
        if r == 0:
            for a, b in zip(got, ref_eager):
                assert torch.equal(a, b)
