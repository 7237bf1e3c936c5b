"""Compact gradient store (usaf_amd/moe_loader.py SparseGradStore, the
reference's moe_loader.py:527-581 protocol): the compact gradients of all
tensors are consecutive slices of one buffer, so that a whole-store pass (the
finite check and copy of the bench step) is one launch.  CPU only."""
import torch

from usaf_amd.moe_loader import SparseGradStore


def _store():
    g = torch.Generator().manual_seed(3)
    shapes = {"L.gate_up_proj": (3, 8, 6), "L.down_proj": (3, 6, 4)}
    active = {}
    for name, (E, R, C) in shapes.items():
        n = E * R * C
        active[name] = torch.randperm(n, generator=g)[: n // 5]  # unsorted on purpose
    return SparseGradStore(active, shapes, device="cpu"), active, shapes


def test_compact_views_tile_one_buffer():
    store, active, _ = _store()
    flat = store.flat
    start = 0
    for name, idx in active.items():
        s, n = store.spans[name]
        assert (s, n) == (start, idx.numel())
        view = store.compact[name]
        assert view.numel() == n and view.data_ptr() == flat.data_ptr() + 4 * s
        start += n
    assert flat.numel() == start and flat.dtype == torch.float32


def test_dense_add_lands_in_the_flat_buffer_and_zero_is_deferred():
    store, active, shapes = _store()
    g = torch.Generator().manual_seed(4)
    dense = {name: torch.randn(*shapes[name], generator=g) for name in shapes}
    for name, (E, _, _) in shapes.items():
        for ei in range(E):
            store.add(name, ei, dense[name][ei])
    # each compact entry is the dense gradient at its flat position (in active-index order)
    for name, idx in active.items():
        want = dense[name].reshape(-1)[idx]
        assert torch.equal(store.compact[name], want)
        s, n = store.spans[name]
        assert torch.equal(store.flat[s:s + n], want)
    # zero_ defers; reading flat zeroes every slice, and a later add starts from zero
    store.zero_()
    assert torch.count_nonzero(store.flat) == 0
    name = "L.down_proj"
    store.add(name, 1, dense[name][1])
    idx = active[name]
    E, R, C = shapes[name]
    in_e1 = (idx // (R * C)) == 1
    want = torch.where(in_e1, dense[name].reshape(-1)[idx], torch.zeros(()))
    assert torch.equal(store.compact[name], want)
    other = "L.gate_up_proj"
    assert torch.count_nonzero(store.compact[other]) == 0
