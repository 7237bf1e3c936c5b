"""Host-side activation caches (usaf/cache.py, usaf/frozen_cache.py): interface
behaviour on the CPU."""
import json

import numpy as np
import torch
import torch.nn as nn

from usaf_amd.cache import ActivationCache
from usaf_amd.frozen_cache import build_frozen_cache, dataset_fingerprint, get_hidden, load_frozen_cache


class TinyDecoderLayer(nn.Module):
    def __init__(self, h):
        super().__init__()
        self.lin = nn.Linear(h, h)

    def forward(self, x):
        return self.lin(x), None


class TinyModel(nn.Module):
    def __init__(self, h=8, n=3):
        super().__init__()
        self.layers = nn.ModuleList([TinyDecoderLayer(h) for _ in range(n)])
        self.head = nn.Linear(h, 2)

    def forward(self, x):
        for layer in self.layers:
            x, _ = layer(x)
        return self.head(x)


def test_activation_cache_records_invalidates_and_resets():
    torch.manual_seed(0)
    m = TinyModel()
    cache = ActivationCache()
    cache.register_hooks(m)
    assert cache.cached_modules == {"layers.0", "layers.1", "layers.2"}
    x0, x1 = torch.randn(4, 8), torch.randn(4, 8)
    m(x0)
    m(x1)
    out0 = cache.get_cached("layers.0", 0)
    assert isinstance(out0, tuple) and out0[1] is None
    assert torch.equal(out0[0], m.layers[0](x0)[0].detach())
    assert torch.equal(cache.get_cached("layers.0", 1)[0], m.layers[0](x1)[0].detach())
    assert cache.get_cached("layers.0", 5) is None and cache.get_cached("nope", 0) is None
    assert cache.memory_estimate_mb() > 0
    cache.invalidate({"layers.1"})
    assert "layers.1" not in cache.cached_modules
    m(x0)
    assert cache.get_cached("layers.1", 0) is None  # invalidated blocks record nothing
    cache.remove_hooks()
    n = len(cache._cache["layers.0"])
    m(x0)
    assert len(cache._cache["layers.0"]) == n
    cache.reset()
    assert cache.cached_modules == set()


def _samples(n, seq, seed):
    g = torch.Generator().manual_seed(seed)
    return [{"input_ids": torch.randint(0, 100, (seq,), generator=g)} for _ in range(n)]


def test_frozen_cache_build_reuse_and_invalidation(tmp_path):
    seq, hidden = 6, 4
    samples = _samples(5, seq, 1)
    path = str(tmp_path / "frozen.npy")
    calls = []

    def compute_hidden(s):
        calls.append(1)
        return s["input_ids"].float().unsqueeze(-1).repeat(1, hidden) / 7.0

    arr = build_frozen_cache(samples, seq, hidden, 3, "src", compute_hidden, path, verbose=False)
    assert arr.shape == (5, seq, hidden) and arr.dtype == np.float16 and len(calls) == 5
    meta = json.load(open(path + ".json"))
    assert meta["fingerprint"] == dataset_fingerprint(samples, 3, "src") and meta["N"] == 5
    # a second build reuses the file
    again = build_frozen_cache(samples, seq, hidden, 3, "src", compute_hidden, path, verbose=False)
    assert len(calls) == 5 and np.array_equal(np.asarray(again), np.asarray(arr))
    # fingerprint covers the layer, the source and the ids; shape mismatches invalidate
    assert load_frozen_cache(samples, seq, hidden, 4, "src", path) is None
    assert load_frozen_cache(samples, seq, hidden, 3, "other", path) is None
    assert load_frozen_cache(_samples(5, seq, 2), seq, hidden, 3, "src", path) is None
    assert load_frozen_cache(samples, seq, hidden + 1, 3, "src", path) is None
    h = get_hidden(arr, 2, "cpu", torch.float32)
    exp = (samples[2]["input_ids"].float().unsqueeze(-1).repeat(1, hidden) / 7.0).half().float()
    assert h.shape == (1, seq, hidden) and torch.equal(h[0], exp)


def _natural_chunk(w_rows, K, inter, nt, w, ks, j, lane):
    """Row and column of the 8 elements lane `lane` of wave `w` loads into
    register `j` at k-step `ks` of n-tile `nt` (the dense-weight GEMM's
    fragment: row 32 w + (lane & 31) of the tile, or the gate/up pair of
    SwiGLU row 16 w + (lane & 15); columns 64 ks + 32 (lane >> 5) + 8 j)."""
    if inter > 0:
        n = 128 * nt + 16 * w + lane % 16
        row = n + (inter if lane % 32 >= 16 else 0)
        ok = n < inter
    else:
        row = 256 * nt + 32 * w + lane % 32
        ok = row < w_rows
    return (row, 64 * ks + 32 * (lane // 32) + 8 * j) if ok else None


def test_fragment_order_slot_layout():
    from usaf_amd.expert_cache import frag_chunk_index
    for w_rows, K, inter in ((256, 128, 128), (384, 256, 0), (256, 128, 0), (768, 384, 384)):
        idx = frag_chunk_index(w_rows, K, inter)
        n_nt = (inter + 127) // 128 if inter else (w_rows + 255) // 256
        assert idx.numel() == n_nt * 256 * K // 8
        valid = idx[idx >= 0]
        # every natural chunk exactly once; the rest is padding
        assert torch.equal(valid.sort().values, torch.arange(w_rows * K // 8))
        # spot checks against the per-lane load pattern, walked chunk by chunk
        nk = K // 64
        for c in (0, 1, 63, 64, 255, 256, 4 * 64 * nk, idx.numel() - 1, idx.numel() // 2 + 17):
            lane, t = c % 64, c // 64
            j, t = t % 4, t // 4
            ks, t = t % nk, t // nk
            w, nt = t % 8, t // 8
            nat = _natural_chunk(w_rows, K, inter, nt, w, ks, j, lane)
            want = -1 if nat is None else nat[0] * (K // 8) + nat[1] // 8
            assert int(idx[c]) == want, (w_rows, K, inter, c)
