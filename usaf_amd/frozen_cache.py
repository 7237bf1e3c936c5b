"""Frozen-layer activation cache on disk (usaf/frozen_cache.py:14-74).

hidden@DETACH_AT is computed once per sample and kept as an fp16 ``.npy``
memory map with a JSON fingerprint; training then starts at layer
DETACH_AT + 1.  ``get_hidden`` stages a sample through pinned host memory into
the device (HBM) asynchronously.
"""
from __future__ import annotations

import hashlib
import json
import os
from typing import Callable, Optional

import numpy as np
import torch


def dataset_fingerprint(samples, detach_at: int, src: str) -> str:
    """frozen_cache.py:14-22: sha256 over (detach_at, src, int32 input ids), 16 hex digits."""
    h = hashlib.sha256()
    h.update(f"{detach_at}|{src}".encode())
    for s in samples:
        ids = s["input_ids"]
        arr = ids.numpy() if hasattr(ids, "numpy") else np.asarray(ids)
        h.update(np.asarray(arr, dtype=np.int32).tobytes())
    return h.hexdigest()[:16]


def load_frozen_cache(samples, seq: int, hidden: int, detach_at: int, src: str, path: str) -> Optional[np.ndarray]:
    """frozen_cache.py:25-39: read-only memmap when the fingerprint and shape match, else None."""
    meta_path = path + ".json"
    if not (os.path.exists(path) and os.path.exists(meta_path)):
        return None
    try:
        with open(meta_path) as f:
            meta = json.load(f)
    except (OSError, ValueError):
        return None
    if (meta.get("fingerprint") != dataset_fingerprint(samples, detach_at, src) or meta.get("seq") != seq
            or meta.get("hidden") != hidden or meta.get("N") != len(samples)):
        return None
    return np.lib.format.open_memmap(path, mode="r")


def build_frozen_cache(samples, seq: int, hidden: int, detach_at: int, src: str,
                       compute_hidden: Callable[[dict], torch.Tensor], path: str, verbose: bool = True) -> np.ndarray:
    """frozen_cache.py:42-67: build (or reuse) the [N, seq, hidden] fp16 cache."""
    existing = load_frozen_cache(samples, seq, hidden, detach_at, src, path)
    if existing is not None:
        if verbose:
            print(f"  frozen cache: reusing {path} {existing.shape}")
        return existing
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    n = len(samples)
    arr = np.lib.format.open_memmap(path, mode="w+", dtype=np.float16, shape=(n, seq, hidden))
    for i, s in enumerate(samples):
        with torch.no_grad():
            h = compute_hidden(s)
        arr[i] = h.reshape(seq, hidden).detach().to("cpu", torch.float16).numpy()
        if verbose and (i % 25 == 0 or i == n - 1):
            print(f"  frozen cache build {i + 1}/{n}")
    arr.flush()
    with open(path + ".json", "w") as f:
        json.dump({"fingerprint": dataset_fingerprint(samples, detach_at, src), "N": n, "seq": seq,
                   "hidden": hidden, "detach_at": detach_at}, f)
    if verbose:
        print(f"  frozen cache: saved {path} {arr.shape} ({arr.nbytes / 1e9:.2f}GB)")
    return arr


def get_hidden(cache: np.ndarray, idx: int, device, dtype=torch.float16) -> torch.Tensor:
    """frozen_cache.py:70-74: sample ``idx`` as [1, seq, hidden] on ``device``."""
    host = torch.from_numpy(np.array(cache[idx], copy=True))
    dev = torch.device(device)
    if dev.type == "cuda":
        host = host.pin_memory()
    return host.to(device=dev, dtype=dtype, non_blocking=dev.type == "cuda").unsqueeze(0)
