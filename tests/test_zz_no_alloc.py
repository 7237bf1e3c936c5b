"""usaf_hip_bucket_by_expert_noalloc (static device scratch, no allocation)
against usaf_hip_bucket_by_expert (caller workspace), through the C-ABI.

Two calls in a row on one GPU, the second smaller, so the second runs on the
scratch the first left behind; every output bit-exact, in exact and in
capacity mode.  Sizes beyond the scratch are refused on the host.
"""
import pytest
import torch

from oracle import moe as M
from usaf_amd import _native as N

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _outputs(dev, T, E, cap):
    fill = -7
    return dict(counts=torch.full((E,), fill, dtype=torch.int32, device=dev),
                offsets=torch.full((E + 1,), fill, dtype=torch.int32, device=dev),
                token_idx=torch.full((max(cap, 1),), fill, dtype=torch.int32, device=dev),
                slot_w=torch.full((max(cap, 1),), float(fill), dtype=torch.float32, device=dev),
                pair_slot=torch.full((T, E), fill, dtype=torch.int32, device=dev),
                overflow=torch.zeros(1, dtype=torch.int32, device=dev))


def _bucket(weights, cap, capacity_mode, noalloc):
    T, E = weights.shape
    dev = weights.device
    o = _outputs(dev, T, E, cap)
    st = N.stream_ptr(dev)
    ovf = o["overflow"].data_ptr() if capacity_mode else None
    args = (o["counts"].data_ptr(), o["offsets"].data_ptr(), o["token_idx"].data_ptr(), o["slot_w"].data_ptr(),
            o["pair_slot"].data_ptr(), cap, ovf, st)
    if noalloc:
        N.call("usaf_hip_bucket_by_expert_noalloc", weights.data_ptr(), N.dtype_code(weights.dtype), T, E, *args)
    else:
        ws = torch.empty(max(1, int(N.load().usaf_hip_bucket_workspace_ints(T, E))), dtype=torch.int32, device=dev)
        N.call("usaf_hip_bucket_by_expert", weights.data_ptr(), N.dtype_code(weights.dtype), T, E, ws.data_ptr(),
               *args)
    return o


def _compare(a, b, n_slots):
    assert torch.equal(a["counts"], b["counts"])
    assert torch.equal(a["offsets"], b["offsets"])
    assert torch.equal(a["pair_slot"], b["pair_slot"])
    assert torch.equal(a["overflow"], b["overflow"])
    assert torch.equal(a["token_idx"][:n_slots], b["token_idx"][:n_slots])
    assert torch.equal(a["slot_w"][:n_slots].view(torch.int32), b["slot_w"][:n_slots].view(torch.int32))


@pytest.mark.parametrize("capacity_mode", [False, True])
def test_noalloc_bucketing_matches_workspace_entry(gpu_device, capacity_mode):
    # the second call is smaller: it must not see the first call's scratch contents
    for T, E, k, seed in ((4096, 128, 8, 1), (300, 60, 4, 2)):
        _say(f"bucket noalloc vs workspace T={T} E={E} k={k} capacity_mode={capacity_mode}")
        g = torch.Generator().manual_seed(seed)
        w, _, _ = M.route(torch.randn(T, E, generator=g).bfloat16(), k, False, torch.bfloat16)
        w = w.to(gpu_device)
        S = int((w != 0).sum())
        cap = T * (k + 1) if capacity_mode else T * E
        ref = _bucket(w, cap, capacity_mode, noalloc=False)
        got = _bucket(w, cap, capacity_mode, noalloc=True)
        torch.cuda.synchronize()
        n = cap if capacity_mode else S
        _compare(got, ref, min(n, cap))
        assert int(got["offsets"][E]) == min(S, cap)


def test_noalloc_bucketing_refuses_oversized_calls(gpu_device):
    lib = N.load()
    limit = int(lib.usaf_hip_bucket_noalloc_max_ints())
    E = 1024
    T = (limit // E + 1) * 16  # one chunk of 16 tokens beyond the scratch
    assert int(lib.usaf_hip_bucket_workspace_ints(T, E)) > limit
    # host-side refusal: no pointer is touched and no kernel launched
    rc = lib.usaf_hip_bucket_by_expert_noalloc(None, N.BF16, T, E, None, None, None, None, None, T * E, None, None)
    assert rc == N.USAF_ERR_UNSUPPORTED
    assert "static scratch" in N.last_error()
