"""configs[4] at reduced size: stacked 4-bit MoE layers resident in HBM, a
per-expert LRU of dequantized copies smaller than the working set, Zipf(1.1)
expert popularity (usaf_amd/expert_cache.py; reference semantics
usaf/moe_loader.py:130-181).

Checks, after every layer forward of every microbatch:
* the cached keys and their LRU order equal the reference policy's
  (oracle/cache.py LRUModel) fed the same accesses: the experts the routing
  selected, in ascending order (copies are made on demand);
* sampled cached copies are bit-exact with the C oracle's dequant of that
  expert's 4-bit slices;
* the layer's output from the arena GEMMs is within the bf16 bar of the
  oracle's routed forward on the same dequantized weights.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import moe as M
from oracle.cache import LRUModel
from usaf_amd import moe as G
from usaf_amd.expert_cache import ExpertSlotCache

from parity import check

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _zipf_logits(T, E, perm, s, g):
    """Router logits whose top-k draws experts without replacement with
    probability proportional to Zipf(s) popularity (Gumbel top-k)."""
    rank = torch.empty(E)
    rank[perm] = torch.arange(1, E + 1, dtype=torch.float32)
    logp = -s * torch.log(rank)
    u = torch.rand(T, E, generator=g).clamp_(1e-12, 1 - 1e-7)
    return logp + (-torch.log(-torch.log(u)))


def test_slot_cache_lru_copies_and_forward(gpu_device):
    L, E, H, I, T, k = 6, 16, 256, 128, 256, 4
    dt = torch.bfloat16
    _say(f"slot cache: {L} layers x {E} experts (H={H}, I={I}), 40 slots, Zipf(1.1), T={T} k={k}")
    g = torch.Generator().manual_seed(99)
    layers, deq, perms = {}, {}, {}
    for li in range(L):
        name = f"model.layers.{li}.mlp.experts"
        qg = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H, generator=g) * 0.02).half().to(gpu_device))
        qd = G.Q4Tensor.quantize((torch.randn(E, H, I, generator=g) * 0.02).half().to(gpu_device))
        layers[name] = G.ExpertWeights(qg, qd)
        deq[name] = tuple(torch.from_numpy(oracle.dequant(q.q.cpu().numpy(), q.s.cpu().numpy(), q.z.cpu().numpy(),
                                                          q.numel(), out_dtype="bf16").view(np.int16).copy())
                          .view(torch.bfloat16).reshape(tuple(q.shape)) for q in (qg, qd))
        perms[name] = torch.randperm(E, generator=g)
    slot_bytes = (2 * I * H + H * I) * 2
    cache = ExpertSlotCache(layers, gpu_device, max_bytes=40 * slot_bytes, dtype=dt)
    assert cache.n_slots == 40
    model = LRUModel(40)
    hs0 = torch.randn(T, H, generator=g).to(dt)
    # layers 1 and 3 come back two layers later (32 keys < 40 slots: hits), the
    # rest only once per microbatch (a cyclic walk an LRU this small never hits)
    walk = [0, 1, 2, 1, 3, 4, 3, 5]
    for mb in range(3):
        x = hs0.clone()
        for li in walk:
            name = f"model.layers.{li}.mlp.experts"
            w, _, _ = M.route(_zipf_logits(T, E, perms[name], 1.1, g), k, False, dt)
            out = cache.forward(name, x.to(gpu_device), w.to(gpu_device), k)
            torch.cuda.synchronize()
            for e in (w != 0).any(0).nonzero().reshape(-1).tolist():
                model.access((name, e))
            assert cache.cached_keys == model.keys(), f"LRU order differs after mb {mb} layer {li}"
            ref = M.experts_routed(x, w, deq[name][0], deq[name][1])
            check(f"mb {mb} layer {li} out", out, ref, dt, say=_say)
            # sampled copies, bit for bit
            keys = cache.cached_keys
            for j in torch.randint(0, len(keys), (3,), generator=g).tolist():
                lname, e = keys[j]
                s = cache.slot_of(lname, e)
                assert torch.equal(cache.copy_of(s, "gate_up").cpu().view(torch.int16),
                                   deq[lname][0][e].view(torch.int16))
                assert torch.equal(cache.copy_of(s, "down").cpu().view(torch.int16), deq[lname][1][e].view(torch.int16))
            x = (x.float() + ref.float()).to(dt)
    assert cache.evictions > 0 and cache.hits > 0
    _say(f"  hits {cache.hits}, misses {cache.misses}, evictions {cache.evictions}")


def test_slot_cache_refuses_arena_below_one_layer(gpu_device):
    E, H, I = 16, 256, 128
    q = G.Q4Tensor.quantize((torch.randn(E, 2 * I, H) * 0.02).half().to(gpu_device))
    d = G.Q4Tensor.quantize((torch.randn(E, H, I) * 0.02).half().to(gpu_device))
    with pytest.raises(ValueError):
        ExpertSlotCache({"l0": G.ExpertWeights(q, d)}, gpu_device, max_bytes=(2 * I * H + H * I) * 2 * (E - 1))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_slot_cache_qwen3_layer_shape(gpu_device, dt):
    """configs[4] at the Qwen3-30B-A3B layer shape (E=128, H=2048, I=768): two
    layers, an arena of 200 expert slots against a working set of up to 256,
    Zipf(1.1) routing (T=512 tokens still select every expert of a layer), the
    layers visited in an order with repeats -- hits and evictions -- with the
    LRU order, sampled copies and each layer output checked."""
    L, E, H, I, T, k = 2, 128, 2048, 768, 512, 8
    _say(f"slot cache at the Qwen3 layer shape: {L} layers x {E} experts, 200 slots, T={T} k={k}, {dt}")
    torch.set_num_threads(16)
    from oracle.codec_torch import dequant_opseq
    g = torch.Generator().manual_seed(4848)
    layers, deq, perms = {}, {}, {}
    for li in range(L):
        name = f"model.layers.{li}.mlp.experts"
        qs = [G.Q4Tensor.quantize((torch.randn(shp, generator=g) * 0.02).half().to(gpu_device))
              for shp in ((E, 2 * I, H), (E, H, I))]
        layers[name] = G.ExpertWeights(*qs)
        # the reference's CPU dequant of the same codes (fp16), in the cache dtype
        deq[name] = tuple(dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape).to(dt) for q in qs)
        perms[name] = torch.randperm(E, generator=g)
    slot_bytes = (2 * I * H + H * I) * 2
    cache = ExpertSlotCache(layers, gpu_device, max_bytes=200 * slot_bytes, dtype=dt)
    assert cache.n_slots == 200
    model = LRUModel(200)
    x = torch.randn(T, H, generator=g).to(dt)
    for mb, li in enumerate((0, 0, 1, 0, 1, 1)):
        if True:
            name = f"model.layers.{li}.mlp.experts"
            w, _, _ = M.route(_zipf_logits(T, E, perms[name], 1.1, g), k, False, dt)
            out = cache.forward(name, x.to(gpu_device), w.to(gpu_device), k)
            torch.cuda.synchronize()
            used = (w != 0).any(0).nonzero().reshape(-1).tolist()
            for e in used:
                model.access((name, e))
            assert cache.cached_keys == model.keys(), f"LRU order differs after mb {mb} layer {li}"
            ref = M.experts_routed(x, w, deq[name][0], deq[name][1])
            check(f"mb {mb} layer {li} out ({len(used)} experts used)", out, ref, dt, say=_say)
            keys = cache.cached_keys
            for j in torch.randint(0, len(keys), (4,), generator=g).tolist():
                lname, e = keys[j]
                s = cache.slot_of(lname, e)
                assert torch.equal(cache.copy_of(s, "gate_up").cpu().view(torch.int16),
                                   deq[lname][0][e].view(torch.int16))
                assert torch.equal(cache.copy_of(s, "down").cpu().view(torch.int16), deq[lname][1][e].view(torch.int16))
    assert cache.evictions > 0 and cache.hits > 0
    _say(f"  hits {cache.hits}, misses {cache.misses}, evictions {cache.evictions}")


def test_slot_cache_slots_beyond_4gib(gpu_device):
    """The arena addressing at the configs[4] scale: 700 Qwen3-shape slots
    (a gate_up arena of 2.2e9 elements, 4.4 GB, past 2^31 elements and 4 GiB),
    the free list taken from the top so a layer's experts land in the highest
    slots; the forward and sampled copies checked against the reference's
    dequant."""
    E, H, I, T, k = 128, 2048, 768, 512, 8
    dt = torch.float16
    _say("slot cache: 700 Qwen3-shape slots, a layer placed in slots 572..699 (offsets past 4 GiB)")
    torch.set_num_threads(16)
    from oracle.codec_torch import dequant_opseq
    g = torch.Generator().manual_seed(4949)
    qs = [G.Q4Tensor.quantize((torch.randn(shp, generator=g) * 0.02).half().to(gpu_device))
          for shp in ((E, 2 * I, H), (E, H, I))]
    ew = G.ExpertWeights(*qs)
    deq = tuple(dequant_opseq(q.q.cpu(), q.s.cpu(), q.z.cpu(), q.shape) for q in qs)
    # six names over one set of weights: room for 768 keys, the arena caps it at 700
    layers = {f"model.layers.{li}.mlp.experts": ew for li in range(6)}
    cache = ExpertSlotCache(layers, gpu_device, max_bytes=700 * cache_slot_bytes(H, I, dt), dtype=dt)
    assert cache.n_slots == 700 and cache.gu_arena.numel() > 2 ** 31
    cache._free.reverse()  # pop() now hands out 699, 698, ...
    name = "model.layers.3.mlp.experts"
    w, _, _ = M.route(_zipf_logits(T, E, torch.randperm(E, generator=g), 1.1, g), k, False, dt)
    x = torch.randn(T, H, generator=g).to(dt)
    out = cache.forward(name, x.to(gpu_device), w.to(gpu_device), k)
    torch.cuda.synchronize()
    used = (w != 0).any(0).nonzero().reshape(-1).tolist()
    slots = [cache.slot_of(name, e) for e in used]
    assert min(slots) >= 700 - len(used) and max(slots) == 699
    assert max(slots) * cache.gu_elems * 2 > 2 ** 32
    check(f"out ({len(used)} experts in slots {min(slots)}..{max(slots)})", out,
          M.experts_routed(x, w, deq[0].to(dt), deq[1].to(dt)), dt, say=_say)
    for e in (used[0], used[-1]):
        s = cache.slot_of(name, e)
        assert torch.equal(cache.copy_of(s, "gate_up").cpu().view(torch.int16), deq[0][e].view(torch.int16))
        assert torch.equal(cache.copy_of(s, "down").cpu().view(torch.int16), deq[1][e].view(torch.int16))


def cache_slot_bytes(H, I, dt):
    return 3 * H * I * torch.empty(0, dtype=dt).element_size()
