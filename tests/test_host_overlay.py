"""CPU checks of the overlay entry tables (usaf_amd/moe.py overlay_entries):
every trained position must land on the lane, fragment register and half that
the fused 4-bit GEMM kernel gives that weight.

The brute force walks the kernel's own assignment forward -- tile unit
(expert, n-tile, wave) and lane -> weight row (wrow of moe_gemm_q4_kernel:
tile row 32 w + l32) and k-step -> fragment register j, dword q, half b -> byte
(l32 + 32 h) * 16 + 4 q + 2 b of register j's image -- and the table builder,
which inverts it, must agree position by position."""
import itertools

import pytest
import torch

from usaf_amd.moe import _OVL_CAP, overlay_entries


def kernel_assignment(kind, E, R, C, inter):
    """{(e, row, col) of W: (unit group key, fragment register, image byte offset)}
    enumerated the way the kernel fills its fragments."""
    if kind == "gate_up_fwd":
        N, K, n_nt = inter, C, (inter + 127) // 128
    elif kind == "down_fwd":
        N, K, n_nt = R, C, (R + 255) // 256
    else:  # transposed copies: the GEMM's rows are W's columns
        N, K, n_nt = C, R, (C + 255) // 256
    nk = K // 64
    out = {}
    for e, nt, w, l32 in itertools.product(range(E), range(n_nt), range(8), range(32)):
        b = 32 * w + l32  # tile row
        if kind == "gate_up_fwd":
            n = nt * 128 + (b >> 5) * 16 + (b & 15)
            if n >= inter:
                continue
            n_row = (inter if b & 16 else 0) + n
        else:
            n_row = nt * 256 + b
            if n_row >= N:
                continue
        for ks, h, j, q, hb in itertools.product(range(nk), range(2), range(4), range(4), range(2)):
            k = ks * 64 + 32 * h + 8 * j + 2 * q + hb
            lane = l32 + 32 * h
            off = lane * 16 + 4 * q + 2 * hb
            r, c = (n_row, k) if kind in ("gate_up_fwd", "down_fwd") else (k, n_row)
            unit = (e * n_nt + nt) * 8 + w
            out[(e, r, c)] = (unit * nk + ks, j, off)
    return out


@pytest.mark.parametrize("kind,shape,inter", [
    ("gate_up_fwd", (2, 2 * 160, 256), 160),   # I = 160: a partial 128-column n-tile
    ("down_fwd", (2, 320, 128), 128),          # N = 320: a partial 256-row n-tile
    ("down_bwd", (2, 256, 384), 384),          # W = down [E, H, I]; GEMM rows = I = 384
    ("gate_up_bwd", (1, 256, 320), 128),       # W = gate_up [E, 2I, H]; GEMM rows = H = 320
])
def test_entries_match_kernel_fragments(kind, shape, inter):
    E, R, C = shape
    ref = kernel_assignment(kind, E, R, C, inter)
    assert len(ref) == E * R * C  # every weight is held exactly once
    g = torch.Generator().manual_seed(5)
    numel = E * R * C
    idx = torch.randperm(numel, generator=g)[: numel // 100].sort().values
    word, off, n_words = overlay_entries(kind, idx, shape, inter)
    assert word.min() >= 0 and word.max() < n_words
    assert len(set(word.tolist())) == idx.numel()  # one word per position
    for f, wd, o in zip(idx.tolist(), word.tolist(), off.tolist()):
        e, rem = divmod(f, R * C)
        r, c = divmod(rem, C)
        group, j, want_off = ref[(e, r, c)]
        assert wd // 64 == group and (wd % 64) // 16 == j and o == want_off, (kind, e, r, c)
    # ranks: the positions of one (group, register) take words 16 j + 0, 1, ... in position order
    prev = {}
    for f, wd in zip(idx.tolist(), word.tolist()):
        key = (wd // 64, (wd % 64) // 16)
        assert wd % 16 == prev.get(key, -1) + 1
        prev[key] = wd % 16


def test_entries_reject_dense_blocks():
    # fragment register 0 of a wave covers k = 0..7 and 32..39 of its 32 rows (512
    # weights); 17 trained positions in it overflow, 16 fit
    shape = (1, 256, 128)
    idx = torch.tensor(sorted(r * 128 + k for r in range(32) for k in (0, 33)))[: _OVL_CAP + 1]
    with pytest.raises(ValueError, match="more than"):
        overlay_entries("down_fwd", idx, shape, 128)
    overlay_entries("down_fwd", idx[:_OVL_CAP], shape, 128)
