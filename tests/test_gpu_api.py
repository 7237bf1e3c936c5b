"""GPU tests of the drop-in Python surface: the HBM expert cache
(usaf/moe_loader.py:60-524), the patched Qwen3-MoE forwards
(usaf/qwen3moe_dml.py:24-94) and quantized streaming setup
(usaf/moe_loader.py:650-769), each against the CPU oracle.

Bars: dequantized cache copies and overlay scatters bit-exact; block outputs
within rel <= 1e-2 (bf16) of the oracle's dense-masked reference forward.
"""
import pytest
import torch
import torch.nn as nn

from oracle import moe as M
from oracle.codec_torch import dequant_opseq
from usaf_amd.moe_loader import QuantizedExpertCache, get_quantized_cache, setup_quantized_streaming
from usaf_amd.quantization import quantize_state_dict

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def rel_err(got, ref):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def _expert_state(n_layers, E=4, H=256, I=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for li in range(n_layers):
        p = f"model.layers.{li}.mlp.experts"
        sd[f"{p}.gate_up_proj"] = (torch.randn(E, 2 * I, H, generator=g) * 0.02).half()
        sd[f"{p}.down_proj"] = (torch.randn(E, H, I, generator=g) * 0.02).half()
    return sd


def _oracle_dequant(entry):
    return dequant_opseq(entry["q"].cpu(), entry["s"].cpu(), entry["z"].cpu(), entry["shape"])


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def test_expert_cache_lru_overlays_prefetch(gpu_device):
    _say("QuantizedExpertCache: LRU, overlays, prefetch, resident, estimates")
    sd = _expert_state(3)
    qd = quantize_state_dict(sd, device=gpu_device)
    cache = QuantizedExpertCache(qd, gpu_device, max_cached=2)
    names = [f"model.layers.{li}.mlp.experts" for li in range(3)]
    # bit-exact dequantized copies (fp16, as the reference)
    w0 = cache.get_expert_weights(names[0])
    assert set(w0) == {"gate_up_proj", "down_proj"}
    for local in w0:
        assert isinstance(w0[local], nn.Parameter) and w0[local].dtype == torch.float16
        assert torch.equal(_bits(w0[local]), _bits(_oracle_dequant(qd[f"{names[0]}.{local}"])))
    # LRU order and eviction (moe_loader.py:149-172)
    cache.get_expert_weights(names[1])
    cache.get_expert_weights(names[2])
    assert cache.cached_experts == [names[2], names[1]]
    cache.get_expert_weights(names[1])
    assert cache.cached_experts == [names[1], names[2]]
    per_module = sum(t.numel() * 2 for k, t in sd.items() if k.startswith(names[0]))
    assert cache.estimate_vram_mb() == pytest.approx(2 * per_module / 2 ** 20)
    q_bytes = sum(e["q"].numel() + 2 * e["s"].numel() + 2 * e["z"].numel() for e in qd.values())
    assert cache.estimate_cpu_mb() == pytest.approx(q_bytes / 2 ** 20)
    # overlays: fp16(vals) at the indices, everything else unchanged (moe_loader.py:218-221)
    full = f"{names[0]}.down_proj"
    g = torch.Generator().manual_seed(1)
    idx = torch.randperm(sd[full].numel(), generator=g)[:777]
    vals = torch.randn(777, generator=g)
    cache.overlays[full] = (idx.to(gpu_device), vals.to(gpu_device))
    cache.evict_all()
    assert cache.cached_experts == []
    w0b = cache.get_expert_weights(names[0])["down_proj"]
    ref = _oracle_dequant(qd[full]).reshape(-1).clone()
    ref[idx] = vals.half()
    assert torch.equal(_bits(w0b.reshape(-1)), _bits(ref))
    # prefetch on the side stream gives the same copy
    cache.prefetch(names[2])
    cache.evict(names[2])
    w2 = cache.get_expert_weights(names[2])
    torch.cuda.synchronize()
    assert torch.equal(_bits(w2["gate_up_proj"]), _bits(_oracle_dequant(qd[f"{names[2]}.gate_up_proj"])))
    cache.clear_prefetch()
    # resident layer + master sync (moe_loader.py:263-299, 411-443)
    cache.make_resident([1])
    full1 = f"{names[1]}.gate_up_proj"
    aidx = torch.randperm(sd[full1].numel(), generator=g)[:500]
    masters = {full1: nn.Parameter(torch.randn(500, generator=g).to(gpu_device))}
    cache.apply_resident_overlays({full1: aidx.to(gpu_device)}, masters)
    cache.evict_all()
    # a resident module dequantizes nothing its resident copy holds
    assert cache._dequant(names[1], skip=cache._resident[names[1]].keys()) == {}
    w1 = cache.get_expert_weights(names[1])["gate_up_proj"]
    ref1 = _oracle_dequant(qd[full1]).reshape(-1).clone()
    ref1[aidx] = masters[full1].detach().cpu().half()
    assert torch.equal(_bits(w1.reshape(-1)), _bits(ref1))
    masters[full1].data.add_(1.0)
    cache.sync_resident({full1: aidx.to(gpu_device)}, masters)
    cache.evict_all()
    w1b = cache.get_expert_weights(names[1])["gate_up_proj"]
    ref1[aidx] = masters[full1].detach().cpu().half()
    assert torch.equal(_bits(w1b.reshape(-1)), _bits(ref1))
    # frozen layers leave the store
    cache.free_frozen(0)
    assert cache.get_q4(names[0]) == {}
    torch.cuda.synchronize()


def _tiny_qwen3_moe(E=8, H=256, I=128, k=2, norm=True, seed=0):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_tok=k,
                         norm_topk_prob=norm, hidden_act="silu", intermediate_size=4 * H,
                         num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2, vocab_size=64)
    block = Qwen3MoeSparseMoeBlock(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        block.experts.gate_up_proj.copy_(torch.randn(E, 2 * I, H, generator=g) * 0.02)
        block.experts.down_proj.copy_(torch.randn(E, H, I, generator=g) * 0.02)
        block.gate.weight.copy_(torch.randn(E, H, generator=g) / H ** 0.5)
    return block


def _reference_block(hs, wr, wg, wd, k, norm):
    """qwen3moe_dml.py:67-86 on the CPU oracle (dense-masked expert loop)."""
    B, S, H = hs.shape
    x = hs.reshape(-1, H)
    logits = torch.nn.functional.linear(x, wr)
    w, _, _ = M.route(logits, k, norm, x.dtype)
    return M.experts_dense_masked(x, w, wg, wd).reshape(B, S, H)


@pytest.mark.parametrize("norm", [True, False])
def test_patched_qwen3moe_block_dense(gpu_device, norm):
    _say(f"patch_qwen3moe_for_dml: dense bf16 block, norm_topk_prob={norm}")
    from usaf_amd.qwen3moe_dml import patch_qwen3moe_for_dml
    patch_qwen3moe_for_dml()
    dt = torch.bfloat16
    block = _tiny_qwen3_moe(norm=norm).to(dt)
    hs = torch.randn(2, 96, 256, generator=torch.Generator().manual_seed(3)).to(dt)
    ref = _reference_block(hs, block.gate.weight.detach(), block.experts.gate_up_proj.detach(),
                           block.experts.down_proj.detach(), 2, norm)
    block = block.to(gpu_device)
    out = block(hs.to(gpu_device))
    torch.cuda.synchronize()
    assert out.shape == hs.shape and out.dtype == dt
    assert rel_err(out, ref) <= 1e-2
    # the experts forward with the reference's signature (hidden [N, H], weights [N, E])
    x = hs.reshape(-1, 256)
    w, _, _ = M.route(torch.nn.functional.linear(x, block.gate.weight.detach().cpu()), 2, norm, dt)
    y = block.experts(x.to(gpu_device), w.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(y, M.experts_dense_masked(x, w, block.experts.gate_up_proj.detach().cpu(),
                                             block.experts.down_proj.detach().cpu())) <= 1e-2


def test_quantized_streaming_fused_block(gpu_device):
    _say("setup_quantized_streaming (fused 4-bit) + patched block, bf16")
    from usaf_amd.qwen3moe_dml import patch_qwen3moe_for_dml
    patch_qwen3moe_for_dml()
    dt = torch.bfloat16
    block = _tiny_qwen3_moe(seed=5)
    layer = nn.Module()
    layer.mlp = block
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([layer])
    model = model.to(dt)
    experts_sd = {k: v.detach().half() for k, v in model.state_dict().items() if ".mlp.experts." in k}
    qd = quantize_state_dict(experts_sd, device=gpu_device)
    setup_quantized_streaming(model, qd, gpu_device, verbose=False)
    hs = torch.randn(1, 128, 256, generator=torch.Generator().manual_seed(6)).to(dt)
    wg = _oracle_dequant(qd["model.layers.0.mlp.experts.gate_up_proj"]).to(dt)
    wd = _oracle_dequant(qd["model.layers.0.mlp.experts.down_proj"]).to(dt)
    ref = _reference_block(hs, block.gate.weight.detach().cpu(), wg, wd, 2, True)
    out = model.model.layers[0].mlp(hs.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= 1e-2
    assert getattr(block.experts, "_usaf_q4", None) is None   # detached again by the post-hook


def test_quantized_streaming_fused_sync_resident(gpu_device):
    """The reference's training loop scatters the optimizer masters into the expert
    weights after each step (train.py:666 cache.sync_resident); the fused streaming
    block must then multiply the trained values: bit-exact weights through the
    overlay tables, the block output against the oracle on the scattered weights."""
    _say("setup_quantized_streaming (fused) + sync_resident(masters) -> block on the trained weights, bf16")
    from usaf_amd.qwen3moe_dml import patch_qwen3moe_for_dml
    patch_qwen3moe_for_dml()
    dt = torch.bfloat16
    block = _tiny_qwen3_moe(seed=9)
    layer = nn.Module()
    layer.mlp = block
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([layer])
    model = model.to(dt)
    experts_sd = {k: v.detach().half() for k, v in model.state_dict().items() if ".mlp.experts." in k}
    qd = quantize_state_dict(experts_sd, device=gpu_device)
    setup_quantized_streaming(model, qd, gpu_device, verbose=False)
    cache = get_quantized_cache(model)
    g = torch.Generator().manual_seed(10)
    active, masters, w_eff = {}, {}, {}
    for local in ("gate_up_proj", "down_proj"):
        name = f"model.layers.0.mlp.experts.{local}"
        w16 = _oracle_dequant(qd[name])
        n = w16.numel()
        idx = torch.randperm(n, generator=g)[: n // 200].sort().values
        vals = w16.reshape(-1)[idx].float() + torch.randn(idx.numel(), generator=g) * 0.05
        active[name] = idx.to(gpu_device)
        masters[name] = torch.nn.Parameter(vals.to(gpu_device), requires_grad=False)
        w = w16.clone()
        w.reshape(-1)[idx] = vals.half()  # the reference's scatter into its fp16 weights
        w_eff[local] = w.to(dt)
    cache.sync_resident(active, masters)
    hs = torch.randn(1, 128, 256, generator=g).to(dt)
    ref = _reference_block(hs, block.gate.weight.detach().cpu(), w_eff["gate_up_proj"], w_eff["down_proj"], 2, True)
    out = model.model.layers[0].mlp(hs.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= 1e-2
    # a second sync (the next optimizer step) refreshes the same tables
    for name in masters:
        masters[name].data.mul_(0.5)
    cache.sync_resident(active, masters)
    for local in ("gate_up_proj", "down_proj"):
        name = f"model.layers.0.mlp.experts.{local}"
        w = _oracle_dequant(qd[name]).clone()
        w.reshape(-1)[active[name].cpu()] = masters[name].detach().cpu().half()
        w_eff[local] = w.to(dt)
    ref = _reference_block(hs, block.gate.weight.detach().cpu(), w_eff["gate_up_proj"], w_eff["down_proj"], 2, True)
    out = model.model.layers[0].mlp(hs.to(gpu_device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) <= 1e-2
    assert len(cache.fused_overlays) == 2


def _streaming_model(seed, dt=torch.bfloat16):
    from usaf_amd.qwen3moe_dml import patch_qwen3moe_for_dml
    patch_qwen3moe_for_dml()
    block = _tiny_qwen3_moe(seed=seed)
    layer = nn.Module()
    layer.mlp = block
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([layer])
    model = model.to(dt)
    experts_sd = {k: v.detach().half() for k, v in model.state_dict().items() if ".mlp.experts." in k}
    return model, block, experts_sd


def _scattered(base16, positions, values):
    """The reference's fp16 weight after its scatter of the masters (moe_loader.py:218-221)."""
    w = base16.clone()
    w.reshape(-1)[positions.cpu().long()] = values.detach().cpu().half()
    return w


@pytest.mark.parametrize("resident", [False, True])
def test_fused_overlays_follow_reselect(gpu_device, resident):
    """train.py's overlay life cycle on the fused streaming path: cache.overlays
    set at start-up reach the first forward (train.py:467); a RigL reselect keeps
    the count (kept + grown = old size, train.py:560-565) and installs new
    overlays (:603-608) followed by sync_resident: the fused view is rebuilt on
    the new positions.  Dropped positions read the 4-bit base for a streamed
    tensor (dequant + overlays, moe_loader.py:183-224) and keep their last
    trained value for a resident one (in-place scatter, moe_loader.py:411-443).
    Masters changed without a sync reach the forward after evict_all, as the
    reference's re-dequant with the current overlay values does."""
    _say(f"fused overlays through start-up, sync and a same-size reselect, resident={resident}")
    from parity import check
    from usaf_amd.importance import reselect_active
    dt = torch.bfloat16
    model, block, experts_sd = _streaming_model(seed=21)
    qd = quantize_state_dict(experts_sd, device=gpu_device)
    setup_quantized_streaming(model, qd, gpu_device, verbose=False)
    cache = get_quantized_cache(model)
    g = torch.Generator().manual_seed(22)
    names = [f"model.layers.0.mlp.experts.{l}" for l in ("gate_up_proj", "down_proj")]
    base = {n: _oracle_dequant(qd[n]) for n in names}
    active, masters = {}, {}
    for n in names:
        numel = base[n].numel()
        idx = torch.randperm(numel, generator=g)[: numel // 200].sort().values
        active[n] = idx.to(gpu_device)
        masters[n] = torch.nn.Parameter((base[n].reshape(-1)[idx].float()
                                         + torch.randn(idx.numel(), generator=g) * 0.05).to(gpu_device),
                                        requires_grad=False)
        cache.overlays[n] = (active[n], masters[n])  # train.py:467
    if resident:
        cache.make_resident([0])
        cache.apply_resident_overlays(active, masters)
    hs = torch.randn(1, 128, 256, generator=g).to(dt)
    wr = block.gate.weight.detach().cpu()

    def run_and_check(w_eff, what):
        ref = _reference_block(hs, wr, w_eff[names[0]].to(dt), w_eff[names[1]].to(dt), 2, True)
        out = model.model.layers[0].mlp(hs.to(gpu_device))
        torch.cuda.synchronize()
        check(what, out, ref, dt)

    # start-up: no sync_resident yet, the overlays alone carry the masters
    run_and_check({n: _scattered(base[n], active[n], masters[n]) for n in names}, "start-up")
    # an optimizer step and its sync
    for n in names:
        masters[n].data.add_(0.01)
    cache.sync_resident(active, masters)
    w_prev = {n: _scattered(base[n], active[n], masters[n]) for n in names}
    run_and_check(w_prev, "after sync")
    # reselect: a new selection of the same size overlapping half of the old one
    new_active, new_masters = {}, {}
    for n in names:
        numel = base[n].numel()
        old = active[n].cpu()
        keep = old[torch.randperm(old.numel(), generator=g)[: old.numel() // 2]]
        fresh = torch.randperm(numel, generator=g)[: old.numel()]
        sel = torch.unique(torch.cat([keep, fresh]))[: old.numel() + old.numel() // 4]
        final, vals, counts = reselect_active(active[n], masters[n], sel.to(gpu_device), qd[n])
        assert final.numel() == old.numel() and counts["grown"] > 0 and counts["dropped"] > 0
        new_active[n] = final
        new_masters[n] = torch.nn.Parameter(vals + 0.02, requires_grad=False)  # one step after the reselect
    cache.overlays.clear()
    for n in names:
        cache.overlays[n] = (new_active[n].reshape(-1).long(), new_masters[n])  # train.py:603-608
    if resident:
        cache.apply_resident_overlays(new_active, new_masters)
    cache.sync_resident(new_active, new_masters)
    if resident:
        w_new = {n: _scattered(w_prev[n], new_active[n], new_masters[n]) for n in names}
    else:
        w_new = {n: _scattered(base[n], new_active[n], new_masters[n]) for n in names}
    run_and_check(w_new, "after reselect")
    for n in names:
        assert cache.fused_overlays[n].ov is not None
        if resident:
            # the resident copy the reference would multiply holds the same weights
            res = cache._resident["model.layers.0.mlp.experts"][n.rsplit(".", 1)[1]]
            assert torch.equal(_bits(res), _bits(w_new[n]))
    # masters changed in place with no sync: the reference's cache keeps a module's
    # dequantized copy until it is evicted, then dequantizes it again with the
    # overlays' current values (moe_loader.py:183-247)
    for n in names:
        new_masters[n].data.add_(0.03)
    run_and_check(w_new, "changed masters, not evicted")
    cache.evict_all()
    run_and_check({n: _scattered(w_new[n], new_active[n], new_masters[n]) for n in names},
                  "changed masters after evict_all")


def test_fused_overlay_dense_fallback_for_clustered_masks(gpu_device):
    """Importance-selected positions concentrate on a few hidden channels (the
    gradients are low-rank outer products): whole columns of 32 gate/up rows
    are selected, more than the overlay tables hold per 32 x 16 block.  The
    fused view then falls back to a dense copy of the trained weights for that
    tensor, and the block still matches the oracle on the scattered weights."""
    _say("TopKImportanceStore on column-clustered gradients -> over-dense overlay -> dense fallback")
    from parity import check
    from usaf_amd.importance import TopKImportanceStore
    dt = torch.bfloat16
    model, block, experts_sd = _streaming_model(seed=23)
    qd = quantize_state_dict(experts_sd, device=gpu_device)
    setup_quantized_streaming(model, qd, gpu_device, verbose=False)
    cache = get_quantized_cache(model)
    g = torch.Generator().manual_seed(24)
    names = [f"model.layers.0.mlp.experts.{l}" for l in ("gate_up_proj", "down_proj")]
    shapes = {n: tuple(qd[n]["shape"]) for n in names}
    store = TopKImportanceStore(shapes, frac=0.005)
    for n in names:
        E, R, C = shapes[n]
        hot = torch.zeros(C)
        hot[torch.randperm(C, generator=g)[:3]] = 50.0  # three outlier input channels
        for e in range(E):
            u = torch.randn(R, generator=g)
            v = torch.randn(C, generator=g) * 0.1 + hot
            store.add(n, e, torch.outer(u, v).to(gpu_device))
    active = store.select()
    base = {n: _oracle_dequant(qd[n]) for n in names}
    masters = {n: torch.nn.Parameter((base[n].reshape(-1)[active[n].cpu()].float() + 0.05).to(gpu_device),
                                     requires_grad=False) for n in names}
    for n in names:
        cache.overlays[n] = (active[n], masters[n])
    cache.sync_resident(active, masters)
    assert cache.fused_overlays[names[0]].dense is not None, "expected the clustered gate_up mask to be over-dense"
    hs = torch.randn(1, 128, 256, generator=g).to(dt)
    wr = block.gate.weight.detach().cpu()
    w_eff = {n: _scattered(base[n], active[n], masters[n]) for n in names}
    ref = _reference_block(hs, wr, w_eff[names[0]].to(dt), w_eff[names[1]].to(dt), 2, True)
    x = hs.to(gpu_device).requires_grad_(True)
    out = model.model.layers[0].mlp(x)
    out.float().square().sum().backward()
    torch.cuda.synchronize()
    check("clustered mask forward", out, ref, dt)
    assert torch.isfinite(x.grad).all()
    # the dense copy holds dtype(fp16(master)) at the active positions, bit for bit
    dense = cache.fused_overlays[names[0]].dense
    assert torch.equal(_bits(dense), _bits(w_eff[names[0]].to(dt)))
    # a refresh rewrites the trained values in the dense copy
    for n in names:
        masters[n].data.mul_(0.5)
    cache.sync_resident(active, masters)
    assert torch.equal(_bits(cache.fused_overlays[names[0]].dense),
                       _bits(_scattered(base[names[0]], active[names[0]], masters[names[0]]).to(dt)))


def test_streaming_slot_cache_serves_no_grad_forwards(gpu_device):
    """setup_quantized_streaming(expert_cache_bytes=...): forwards that need no
    gradients run on per-expert dequantized copies made on demand (the
    reference's dequant-on-access cache, usaf/moe_loader.py:130-181); a forward
    with gradients, or of a module with trained values, runs on the fused 4-bit
    GEMMs.  Every path matches the oracle."""
    _say("streaming with a per-expert copy cache: no-grad forwards on copies, grad / trained on the fused path")
    from parity import check
    dt = torch.bfloat16
    model, block, experts_sd = _streaming_model(seed=31)
    qd = quantize_state_dict(experts_sd, device=gpu_device)
    E, H, I = 8, 256, 128
    setup_quantized_streaming(model, qd, gpu_device, verbose=False, expert_cache_bytes=E * (3 * H * I) * 2)
    cache = get_quantized_cache(model)
    sc = cache.slot_cache
    assert sc is not None and sc.n_slots == E and sc.dtype == dt
    names = [f"model.layers.0.mlp.experts.{l}" for l in ("gate_up_proj", "down_proj")]
    base = {n: _oracle_dequant(qd[n]) for n in names}
    g = torch.Generator().manual_seed(32)
    hs = torch.randn(1, 96, H, generator=g).to(dt)
    wr = block.gate.weight.detach().cpu()
    ref = _reference_block(hs, wr, base[names[0]].to(dt), base[names[1]].to(dt), 2, True)
    with torch.no_grad():
        out = model.model.layers[0].mlp(hs.to(gpu_device))
    torch.cuda.synchronize()
    check("no-grad forward on the copies", out, ref, dt)
    used = int(sc.misses)
    assert used > 0 and sc.hits == 0
    with torch.no_grad():
        model.model.layers[0].mlp(hs.to(gpu_device))
    assert sc.hits == used and sc.misses == used  # the same experts again: hits only
    x = hs.to(gpu_device).requires_grad_(True)
    out_g = model.model.layers[0].mlp(x)
    torch.cuda.synchronize()
    assert sc.hits == used and sc.misses == used, "a forward with gradients must not use the copies"
    check("grad forward on the fused path", out_g, ref, dt)
    # trained values: the module leaves the copies for the fused path with overlays
    active, masters = {}, {}
    for n in names:
        numel = base[n].numel()
        idx = torch.randperm(numel, generator=g)[: numel // 200].sort().values
        active[n] = idx.to(gpu_device)
        masters[n] = torch.nn.Parameter((base[n].reshape(-1)[idx].float() + 0.05).to(gpu_device),
                                        requires_grad=False)
        cache.overlays[n] = (active[n], masters[n])
    w_eff = {}
    for n in names:
        w = base[n].clone()
        w.reshape(-1)[active[n].cpu()] = masters[n].detach().cpu().half()
        w_eff[n] = w.to(dt)
    ref_t = _reference_block(hs, wr, w_eff[names[0]], w_eff[names[1]], 2, True)
    with torch.no_grad():
        out_t = model.model.layers[0].mlp(hs.to(gpu_device))
    torch.cuda.synchronize()
    assert sc.hits == used and sc.misses == used
    check("no-grad forward with trained values (fused)", out_t, ref_t, dt)
    cache.free_frozen(0)
    assert not sc.layers and not sc.cached_keys


def _tiny_olmoe(E=8, H=256, I=128, k=2, seed=0, norm=False):
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeSparseMoeBlock
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k,
                      norm_topk_prob=norm, hidden_act="silu", num_hidden_layers=1, num_attention_heads=4,
                      num_key_value_heads=4, vocab_size=64)
    block = OlmoeSparseMoeBlock(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        block.experts.gate_up_proj.copy_(torch.randn(E, 2 * I, H, generator=g) * 0.02)
        block.experts.down_proj.copy_(torch.randn(E, H, I, generator=g) * 0.02)
        block.gate.weight.copy_(torch.randn(E, H, generator=g) / H ** 0.5)
    return block


def test_patched_olmoe_block_fp16_with_dense_weight_grads(gpu_device):
    # the reference runs this variant's expert math in fp32 (olmoe_dml.py:10-33): the oracle
    # is its fp32 dense-masked loop with autograd; the GPU computes it in bf16 on MFMA
    _say("patch_olmoe_for_dml: fp16 block, fp32 oracle, dense expert-weight grads")
    from usaf_amd.olmoe_dml import patch_olmoe_for_dml
    patch_olmoe_for_dml()
    block = _tiny_olmoe(seed=7)
    block.gate.half()  # the router in the activations' dtype, fp32 expert Parameters
    hs = torch.randn(2, 64, 256, generator=torch.Generator().manual_seed(8)).half()
    dout = torch.randn(2, 64, 256, generator=torch.Generator().manual_seed(9)).half()
    wg = block.experts.gate_up_proj.detach().clone().requires_grad_(True)
    wd = block.experts.down_proj.detach().clone().requires_grad_(True)
    x = hs.float().reshape(-1, 256)
    logits = torch.nn.functional.linear(hs.reshape(-1, 256), block.gate.weight.detach()).float()
    w, _, _ = M.route(logits, 2, False, torch.float16)
    w = w.float()
    ref = M.experts_dense_masked(x, w, wg, wd)
    ref.backward(dout.float().reshape(-1, 256))
    block = block.to(gpu_device)
    out = block(hs.to(gpu_device))
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == hs.shape
    assert rel_err(out.reshape(-1, 256), ref) <= 1e-2
    assert block.experts.gate_up_proj.grad.dtype == torch.float32
    assert rel_err(block.experts.gate_up_proj.grad, wg.grad) <= 1e-2
    assert rel_err(block.experts.down_proj.grad, wd.grad) <= 1e-2


def test_olmoe_streaming_capture(gpu_device):
    _say("olmoe setup_streaming + apply_captured_expert_grads")
    from usaf_amd.olmoe_dml import patch_olmoe_for_dml
    from usaf_amd.olmoe_streaming import apply_captured_expert_grads, setup_streaming
    patch_olmoe_for_dml()
    block = _tiny_olmoe(seed=11)
    layer = nn.Module()
    layer.mlp = block
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = nn.ModuleList([layer])
    setup_streaming(model, gpu_device, verbose=False)
    assert all(p.device.type == "cuda" for p in model.parameters())
    hs = torch.randn(1, 32, 256, generator=torch.Generator().manual_seed(12)).to(gpu_device)
    out = model.model.layers[0].mlp(hs)
    out.sum().backward()
    torch.cuda.synchronize()
    names = set(model._expert_grads)
    assert names == {"model.layers.0.mlp.experts.gate_up_proj", "model.layers.0.mlp.experts.down_proj"}
    g_before = model._expert_grads["model.layers.0.mlp.experts.down_proj"].clone()
    assert apply_captured_expert_grads(model, scale=0.5) == 2
    assert model._expert_grads == {}
    p = dict(model.named_parameters())["model.layers.0.mlp.experts.down_proj"]
    assert torch.allclose(p.grad, g_before * 0.5)
    assert model._stream_state["max"] == 1 and model._stream_state["resident"] == 0


def test_patched_olmoe_block_real_shape(gpu_device):
    """The OLMoE-1B-7B MoE layer shape (hidden 2048, intermediate 1024, 64
    experts, top-8): the patched block (dense fp32 expert Parameters, bf16 MFMA,
    fp32 accumulation): the output against the routed loop at the same rounding
    points (normwise and elementwise bars), and the output and the dense
    expert-weight gradients against the reference's fp32 loop with autograd
    (normwise bar)."""
    _say("patch_olmoe_for_dml at the OLMoE layer shape: E=64 H=2048 I=1024 k=8, T=256, bf16")
    from parity import check
    from usaf_amd.olmoe_dml import patch_olmoe_for_dml
    patch_olmoe_for_dml()
    torch.set_num_threads(16)
    E, H, I, k = 64, 2048, 1024, 8
    block = _tiny_olmoe(E=E, H=H, I=I, k=k, seed=21)
    block.gate.to(torch.bfloat16)
    g = torch.Generator().manual_seed(22)
    hs = torch.randn(2, 128, H, generator=g).to(torch.bfloat16)
    dout = torch.randn(2, 128, H, generator=g).to(torch.bfloat16)
    wg = block.experts.gate_up_proj.detach().clone().requires_grad_(True)
    wd = block.experts.down_proj.detach().clone().requires_grad_(True)
    x = hs.float().reshape(-1, H)
    block = block.to(gpu_device)
    xg = hs.to(gpu_device).requires_grad_(True)
    # the oracle routes from the block's own logits (the GPU's F.linear): routing is
    # bit-exact given the logits, and a near-tie flipped by the summation order of a
    # CPU product would change whole tokens
    with torch.no_grad():
        logits = torch.nn.functional.linear(xg.reshape(-1, H), block.gate.weight).float().cpu()
    w, _, _ = M.route(logits, k, False, torch.bfloat16)
    ref = M.experts_routed(x, w.float(), wg, wd)
    ref.backward(dout.float().reshape(-1, H))
    out = block(xg)
    out.backward(dout.to(gpu_device))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == hs.shape
    # the same computation at the GPU's rounding points (bf16 operands and
    # intermediates, fp32 accumulation): both bars
    with torch.no_grad():
        ref16 = M.experts_routed(hs.reshape(-1, H), w, wg.detach().to(torch.bfloat16), wd.detach().to(torch.bfloat16))
    check("out vs the bf16 routed loop", out.reshape(-1, H), ref16, torch.bfloat16, say=_say)
    # the reference's fp32 expert math (olmoe_dml.py:10-33): within the bf16 normwise bar
    for name, got, r in (("out", out.reshape(-1, H), ref), ("dW gate_up", block.experts.gate_up_proj.grad, wg.grad),
                         ("dW down", block.experts.down_proj.grad, wd.grad)):
        e = rel_err(got, r)
        _say(f"  {name} vs the fp32 loop: normwise {e:.2e} (bar 1e-2)")
        assert e <= 1e-2, name
