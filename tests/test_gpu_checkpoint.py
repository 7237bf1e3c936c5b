"""export_merged_weights on the GPU (usaf/checkpoint.py:58-92) against the
reference's CPU op sequence restated in oracle/codec_torch.py: dequant to fp16,
masters scattered as fp16, re-quantized; codes, scales and zeros bit-exact."""
import pytest
import torch

from oracle.codec_torch import dequant_opseq, quantize_opseq
from usaf_amd.checkpoint import export_merged_weights
from usaf_amd.quantization import quantize_state_dict

pytestmark = pytest.mark.gpu


def test_export_merged_weights_bit_exact(gpu_device, tmp_path):
    print("[gpu-case] export_merged_weights round trip", flush=True)
    g = torch.Generator().manual_seed(31)
    sd = {"model.layers.1.mlp.experts.gate_up_proj": (torch.randn(4, 256, 384, generator=g) * 0.02).half(),
          "model.layers.1.mlp.experts.down_proj": (torch.randn(4, 384, 128, generator=g) * 0.02).half(),
          "model.layers.1.mlp.gate.weight": (torch.randn(4, 16, generator=g) * 0.1).half()}  # < min_size: fp16
    q = quantize_state_dict(sd, device=gpu_device)
    q = {k: ({kk: (vv.cpu() if isinstance(vv, torch.Tensor) else vv) for kk, vv in v.items()}
             if isinstance(v, dict) else v.cpu()) for k, v in q.items()}
    src = tmp_path / "experts_q4.pt"
    torch.save(q, src)
    name = "model.layers.1.mlp.experts.gate_up_proj"
    numel = 4 * 256 * 384
    idx = torch.randperm(numel, generator=g)[: numel // 200]
    masters = {name: torch.randn(idx.numel(), generator=g) * 0.05}
    out = tmp_path / "merged_q4.pt"
    export_merged_weights(str(src), masters, {name: idx}, str(out), device=gpu_device)
    got = torch.load(out, map_location="cpu", weights_only=True)
    assert set(got) == set(q)
    for k, entry in q.items():
        if isinstance(entry, dict):
            t = dequant_opseq(entry["q"], entry["s"], entry["z"], entry["shape"])
            if k == name:
                flat = t.reshape(-1).clone()
                flat.scatter_(0, idx, masters[name].to(torch.float16))
                t = flat.reshape(t.shape)
            rq, rs, rz = quantize_opseq(t)
            assert torch.equal(got[k]["q"], rq), k
            assert torch.equal(got[k]["s"].view(torch.int16), rs.view(torch.int16)), k
            assert torch.equal(got[k]["z"].view(torch.int16), rz.view(torch.int16)), k
            assert tuple(got[k]["shape"]) == tuple(entry["shape"])
        else:
            assert torch.equal(got[k].view(torch.int16), entry.view(torch.int16))


def test_merge_masters_one_tensor_at_a_time(gpu_device):
    """merge_masters re-quantizes each tensor before it dequantizes the next: the
    HBM peak is one fp16 tensor and its 4-bit codes, not the whole model in fp16."""
    print("[gpu-case] merge_masters HBM peak (4 tensors of 8 Mi elements)", flush=True)
    from usaf_amd.checkpoint import merge_masters
    g = torch.Generator().manual_seed(32)
    n = 8 * 2 ** 20
    sd = {f"model.layers.{i}.mlp.experts.gate_up_proj": (torch.randn(8, 1024, 1024, generator=g) * 0.02).half()
          for i in range(4)}
    q = quantize_state_dict(sd, device=gpu_device)
    q = {k: {kk: (vv.cpu() if isinstance(vv, torch.Tensor) else vv) for kk, vv in v.items()} for k, v in q.items()}
    masters = {k: torch.randn(n // 200, generator=g) * 0.05 for k in q}
    active = {k: torch.randperm(n, generator=g)[: n // 200] for k in q}
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(gpu_device)
    torch.cuda.reset_peak_memory_stats(gpu_device)
    out = merge_masters(q, masters, active, device=gpu_device)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(gpu_device) - base
    fp16_one = 2 * n
    assert set(out) == set(q)
    # one fp16 tensor + its codes, scales, zeros, the CPU entry's device copies and the
    # master/index copies: well under two fp16 tensors (all four would be 64 MiB)
    assert peak < 2 * fp16_one, f"merge peak {peak / 2 ** 20:.1f} MiB for {fp16_one / 2 ** 20:.0f} MiB tensors"
