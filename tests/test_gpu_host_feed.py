"""The frozen-cache feed into HBM (usaf/frozen_cache.py:70-74 get_hidden):
samples staged from the on-disk memory map through the pinned two-buffer ring
into device memory, and the whole cache held resident in HBM.

Bar: every staged sample bit-exact with the memory map's row (fp16), and
equal to the reference's host-side conversion for another dtype.
"""
import numpy as np
import pytest
import torch

from usaf_amd.frozen_cache import HBMHiddenStore, build_frozen_cache, get_hidden

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _cache(tmp_path, n=9, seq=64, hidden=256):
    g = torch.Generator().manual_seed(5)
    samples = [{"input_ids": torch.randint(0, 1000, (seq,), generator=g)} for _ in range(n)]
    table = torch.randn(1000, hidden, generator=g)

    def compute_hidden(s):
        return table[s["input_ids"]]

    return build_frozen_cache(samples, seq, hidden, 3, "synthetic", compute_hidden, str(tmp_path / "f.npy"),
                              verbose=False)


def test_get_hidden_pinned_staging_into_hbm(gpu_device, tmp_path):
    _say("get_hidden: memmap -> pinned ring -> HBM, many samples in flight")
    arr = _cache(tmp_path)
    order = [0, 1, 2, 3, 8, 7, 0, 5, 5, 6, 4, 2]
    # launch every copy before reading any: each ring buffer is reused while
    # earlier copies may still be in flight
    outs = [get_hidden(arr, i, gpu_device) for i in order]
    outs_bf16 = [get_hidden(arr, i, gpu_device, torch.bfloat16) for i in order[:4]]
    torch.cuda.synchronize()
    for i, t in zip(order, outs):
        assert t.shape == (1,) + arr.shape[1:] and t.dtype == torch.float16 and t.is_cuda
        assert np.array_equal(t[0].cpu().numpy().view(np.uint16), np.asarray(arr[i]).view(np.uint16))
    for i, t in zip(order, outs_bf16):
        assert torch.equal(t[0].cpu(), torch.from_numpy(np.array(arr[i])).to(torch.bfloat16))


def test_hbm_resident_store(gpu_device, tmp_path):
    _say("HBMHiddenStore: whole cache resident in HBM, ragged last slab")
    arr = _cache(tmp_path, n=11)
    row_bytes = int(np.prod(arr.shape[1:])) * 2
    store = HBMHiddenStore(arr, gpu_device, slab_bytes=4 * row_bytes)  # slabs of 4, 4, 3 rows
    torch.cuda.synchronize()
    assert len(store) == 11 and store.nbytes() == arr.nbytes
    assert np.array_equal(store.data.cpu().numpy().view(np.uint16), np.asarray(arr).view(np.uint16))
    t = get_hidden(store, 9, gpu_device)
    assert t.shape == (1,) + arr.shape[1:]
    assert np.array_equal(t[0].cpu().numpy().view(np.uint16), np.asarray(arr[9]).view(np.uint16))


class _ToyDecoderLayer(torch.nn.Module):
    """A block whose class name the activation cache hooks (…DecoderLayer); it
    returns a tuple, as transformers' decoder layers do."""

    def __init__(self, h):
        super().__init__()
        self.lin = torch.nn.Linear(h, h)

    def forward(self, x):
        return (torch.tanh(self.lin(x)) * 3.0 + x,)


@pytest.mark.parametrize("cache_on", ["cpu", "cuda"])
def test_activation_cache_on_gpu_model(gpu_device, cache_on):
    _say(f"ActivationCache of a GPU model, cache on {cache_on}: values read right after each forward")
    from usaf_amd.cache import ActivationCache
    torch.manual_seed(3)
    h = 1024
    model = torch.nn.Sequential(_ToyDecoderLayer(h), _ToyDecoderLayer(h)).to(gpu_device)
    blocks = [model[0], model[1]]

    def run(x):
        for b in blocks:
            x = b(x)[0]
        return x

    dev = gpu_device if cache_on == "cuda" else torch.device("cpu")
    cache = ActivationCache(dev)
    cache.register_hooks(model)
    assert cache.cached_modules == {"0", "1"}
    for step in range(3):
        x = torch.randn(64, 512, h, device=gpu_device)  # 128 MiB per block output
        with torch.no_grad():
            y0 = blocks[0](x)[0]
            # the cached copy is read before any synchronisation of the GPU model's
            # stream (a host-side clone of a CPU copy does not wait for the GPU)
            got = cache.get_cached("0", step)[0]
            assert got.device.type == dev.type
            snap = got.clone()
            assert torch.equal(snap.cpu(), y0.cpu()), f"step {step}: cached block output differs"
            y1 = blocks[1](y0)[0]
            assert torch.equal(cache.get_cached("1", step)[0].cpu(), y1.cpu())
        cache.advance_step()
    assert cache.get_cached("0", 3) is None
    assert cache.memory_estimate_mb() == pytest.approx(3 * 2 * 64 * 512 * h * 4 / 2 ** 20)
    cache.invalidate({"1"})
    with torch.no_grad():
        blocks[1](y0)
    assert "1" not in cache.cached_modules and cache.get_cached("1", 0) is None
    cache.remove_hooks()
    cache.reset()
    assert not cache.cached_modules
