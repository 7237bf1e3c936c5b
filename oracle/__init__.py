"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

CPU restatement of the reference's quantized-expert path.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package, and only as the checker (or the timed CPU baseline); the product
(``usaf_amd``) never calls it.

* ``q4_oracle.c`` (built here with gcc into ``_build/libq4oracle.so``) is the
  scalar restatement of usaf/quantization.py:21-132 (quantize / dequantize).
* ``moe.py`` restates routing, bucketing, the expert forward/backward, the
  sparse gradient gather and SparseAdam with torch CPU ops
  (usaf/qwen3moe_dml.py:24-86, benchmarks/kaggle_t4_bench.py:284-328,
  usaf/moe_loader.py:527-581, usaf/sparse_optim.py:86-134).

Pinning: tests/test_oracle_codec.py and tests/test_oracle_moe.py check every
function here against closed forms, numpy's IEEE fp16 arithmetic, brute force
on tiny inputs and hand-derived known-answer vectors (tests/golden/).
"""
from __future__ import annotations

import ctypes
import subprocess
import threading
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
_BUILD = ORACLE_DIR / "_build"
_SO = _BUILD / "libq4oracle.so"
_SRC = ORACLE_DIR / "q4_oracle.c"
_lock = threading.Lock()
_lib = None


def build(force: bool = True) -> Path:
    """Compile q4_oracle.c with gcc (no GPU, no reference sources needed)."""
    _BUILD.mkdir(exist_ok=True)
    if force or not _SO.exists() or _SO.stat().st_mtime < _SRC.stat().st_mtime:
        tmp = _SO.with_suffix(".so.tmp")
        cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-fPIC", "-shared", "-fno-fast-math",
               "-ffp-contract=off", str(_SRC), "-o", str(tmp), "-lm"]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        tmp.replace(_SO)
    return _SO


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not _SO.exists() or _SO.stat().st_mtime < _SRC.stat().st_mtime:
                    build(force=True)
                L = ctypes.CDLL(str(_SO))
                P = ctypes.c_void_p
                I64 = ctypes.c_int64
                U16 = ctypes.c_uint16
                L.q4o_half_to_float.restype = ctypes.c_float
                L.q4o_half_to_float.argtypes = [U16]
                L.q4o_float_to_half.restype = U16
                L.q4o_float_to_half.argtypes = [ctypes.c_float]
                L.q4o_half_to_bf16.restype = U16
                L.q4o_half_to_bf16.argtypes = [U16]
                L.q4o_half_mul.restype = U16
                L.q4o_half_mul.argtypes = [U16, U16]
                L.q4o_half_add.restype = U16
                L.q4o_half_add.argtypes = [U16, U16]
                L.q4o_num_groups.restype = I64
                L.q4o_num_groups.argtypes = [I64, I64]
                L.q4o_quantize.restype = None
                L.q4o_quantize.argtypes = [P, I64, I64, P, P, P]
                L.q4o_dequant.restype = ctypes.c_int
                L.q4o_dequant.argtypes = [P, P, P, I64, I64, I64, I64, P]
                L.q4o_dequant_bf16.restype = None
                L.q4o_dequant_bf16.argtypes = [P, P, P, I64, I64, I64, I64, P]
                _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def quantize(x: np.ndarray, group_size: int = 128):
    """quantization.py:21-85 on a flat fp32 array.

    Returns (packed int8 [G, ceil(egs/2)], scale fp16-bits uint16 [G], zero uint16 [G]).
    """
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
    numel = x.size
    if numel == 0:
        raise ValueError("empty")
    egs = min(group_size, numel)
    G = (numel + egs - 1) // egs
    packed = np.zeros((G, (egs + 1) // 2), dtype=np.int8)
    scale = np.zeros(G, dtype=np.uint16)
    zero = np.zeros(G, dtype=np.uint16)
    lib().q4o_quantize(_p(x), numel, group_size, _p(packed), _p(scale), _p(zero))
    return packed, scale, zero


def dequant(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray, numel: int, group_size: int = 128,
            out_dtype: str = "f16") -> np.ndarray:
    """quantization.py:88-132.  Returns uint16 bit patterns (fp16, or bf16 when
    out_dtype == "bf16") of the flat dequantized tensor."""
    packed = np.ascontiguousarray(np.asarray(packed, dtype=np.int8))
    scale = np.ascontiguousarray(np.asarray(scale).view(np.uint16) if np.asarray(scale).dtype == np.float16
                                 else np.asarray(scale, dtype=np.uint16))
    zero = np.ascontiguousarray(np.asarray(zero).view(np.uint16) if np.asarray(zero).dtype == np.float16
                                else np.asarray(zero, dtype=np.uint16))
    G, pb = packed.shape
    out = np.zeros(numel, dtype=np.uint16)
    if out_dtype == "bf16":
        lib().q4o_dequant_bf16(_p(packed), _p(scale), _p(zero), G, pb, group_size, numel, _p(out))
    else:
        rc = lib().q4o_dequant(_p(packed), _p(scale), _p(zero), G, pb, group_size, numel, _p(out))
        if rc != 0:
            raise RuntimeError("shape is invalid for the code array (reference view would fail)")
    return out


def half_mul(a: int, b: int) -> int:
    return lib().q4o_half_mul(a, b)


def half_add(a: int, b: int) -> int:
    return lib().q4o_half_add(a, b)


def float_to_half(f: float) -> int:
    return lib().q4o_float_to_half(f)


def half_to_float(h: int) -> float:
    return lib().q4o_half_to_float(h)


def half_to_bf16(h: int) -> int:
    return lib().q4o_half_to_bf16(h)
