"""ctypes binding of ``libusaf_hip.so`` (the C-ABI in ``include/usaf_hip.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already mapped (one runtime per
process).  There is no CPU fallback: if the library is missing or no GPU is
visible, every product entry point raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libusaf_hip.so"

USAF_OK = 0
USAF_ERR_INVALID = 1
USAF_ERR_UNSUPPORTED = 2
USAF_ERR_RUNTIME = 3

F32, F16, BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_c_p = ctypes.c_void_p

# name -> argument types (all return int status)
_c_d = ctypes.c_double

_SIGNATURES: dict[str, list] = {
    "usaf_hip_init": [],
    "usaf_hip_dequant_q4": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i32, _c_p],
    "usaf_hip_dequant_q4_at": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p],
    "usaf_hip_topk_abs": [_c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p],
    "usaf_hip_dequant_q4_slices": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i32, _c_p],
    "usaf_hip_router_dx": [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i32, _c_p],
    "usaf_hip_dequant_q4_slices_frag": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64,
                                        _c_p, _c_i32, _c_p],
    "usaf_hip_moe_gate_up_fwd_slots": [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64,
                                       _c_i32, _c_p, _c_p, _c_p],
    "usaf_hip_moe_down_fwd_slots": [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i32, _c_p,
                                    _c_p],
    "usaf_hip_quantize_q4": [_c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p],
    "usaf_hip_pack_scale_zero": [_c_p, _c_p, _c_i64, _c_p, _c_p],
    "usaf_hip_q4_transpose": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p],
    "usaf_hip_route_topk": [_c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i32, _c_p, _c_p],
    "usaf_hip_route_topk_bwd": [_c_p, _c_i32, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i32, _c_p],
    "usaf_hip_bucket_by_expert": [_c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p,
                                  _c_p],
    "usaf_hip_bucket_by_expert_noalloc": [_c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p,
                                          _c_p],
    "usaf_hip_moe_combine": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_p],
    "usaf_hip_moe_combine_bwd": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_p],
    "usaf_hip_moe_gate_up_fwd": [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
                                 _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p],
    "usaf_hip_moe_down_fwd": [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_i64,
                              _c_p],
    "usaf_hip_moe_down_bwd": [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p,
                              _c_p],
    "usaf_hip_moe_gate_up_bwd": [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p,
                                 _c_p],
    "usaf_hip_moe_down_bwd_t": [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i32, _c_p, _c_p,
                                _c_i64, _c_p],
    "usaf_hip_moe_gate_up_bwd_t": [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_i64,
                                   _c_p],
    "usaf_hip_gather_transpose": [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    "usaf_hip_blocked_layout": [_c_p, _c_i64, _c_i64, _c_p, _c_p],
    "usaf_hip_gather_transpose_blocked": [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p],
    "usaf_hip_sddmm_blocked": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_i32,
                               _c_p],
    "usaf_hip_sgd_momentum_step": [_c_p, _c_p, _c_p, _c_i64, _c_i32, _c_d, _c_d, _c_d, _c_i32, _c_p, _c_p, _c_p,
                                   _c_d, _c_p],
    "usaf_hip_loss_scale_apply": [_c_p, _c_p, _c_i64, _c_i32, _c_p, _c_p],
    "usaf_hip_scale_check_state": [_c_p, _c_p, _c_i64, _c_p, _c_d, _c_p, _c_p],
    "usaf_hip_loss_scale_update": [_c_p, _c_p, _c_p, _c_i32, _c_d, _c_d, _c_p],
    "usaf_hip_router_fwd": [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32, _c_p, _c_p, _c_i32, _c_p,
                            _c_p],
    "usaf_hip_router_dw": [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_p],
    "usaf_hip_moe_combine_bwd_blocked": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_p,
                                         _c_p, _c_p, _c_p],
    "usaf_hip_sddmm_masked": [_c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p,
                              _c_p],
    "usaf_hip_sparse_adam_step": [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_d, _c_d, _c_d, _c_d, _c_i64, _c_p],
    "usaf_hip_sparse_adam_step_gated": [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_d, _c_d, _c_d, _c_d, _c_d, _c_p, _c_p, _c_p,
                                        _c_p, _c_i64, _c_p, _c_p],
    "usaf_hip_count_step": [_c_p, _c_p, _c_p, _c_p],
    "usaf_hip_scale_check": [_c_p, _c_p, _c_i64, _c_f32, _c_p, _c_p],
    "usaf_hip_overlay_scatter": [_c_p, _c_i32, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p],
    "usaf_hip_overlay_refresh": [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_p, _c_p],
}
# entry points that return a value instead of a status
_VALUE_FUNCS: dict[str, tuple] = {
    "usaf_hip_bucket_workspace_ints": (_c_i64, [_c_i64, _c_i64]),
    "usaf_hip_bucket_noalloc_max_ints": (_c_i64, []),
    "usaf_hip_blocked_elems": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "usaf_hip_blocked_table_elems": (_c_i64, [_c_i64, _c_i64]),
    "usaf_hip_combine_bwd_blocked_ws_floats": (_c_i64, [_c_i64, _c_i64]),
    "usaf_hip_router_dw_ws_floats": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "usaf_hip_topk_abs_ws_ints": (_c_i64, [_c_i64]),
    "usaf_hip_frag_slot_elems": (_c_i64, [_c_i64, _c_i64, _c_i64]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def exported_symbols() -> list[str]:
    """Names of the status-returning entry points this binding declares."""
    return list(_SIGNATURES) + list(_VALUE_FUNCS) + ["usaf_hip_abi_version", "usaf_hip_last_error"]


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built ({LIB_PATH}); run `python -m usaf_amd.build` "
                "(or __graft_entry__.build()). usaf_amd has no CPU fallback.")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.usaf_hip_abi_version.restype = ctypes.c_int
        lib.usaf_hip_abi_version.argtypes = []
        lib.usaf_hip_last_error.restype = ctypes.c_char_p
        lib.usaf_hip_last_error.argtypes = []
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        for name, (restype, argtypes) in _VALUE_FUNCS.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        check(lib.usaf_hip_init(), "usaf_hip_init") if torch.cuda.is_available() else None
        _lib = lib
    return _lib


def last_error() -> str:
    msg = load().usaf_hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Raise the Python exception matching a C-ABI status code."""
    if rc == USAF_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == USAF_ERR_INVALID:
        raise ValueError(msg)
    if rc == USAF_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    """Call entry point `name` and raise on a non-zero status."""
    check(getattr(load(), name)(*args), name)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def require_gpu() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("usaf_amd runs its hot path on a ROCm GPU only (no CPU fallback); no GPU is visible")


def default_device() -> torch.device:
    require_gpu()
    return torch.device("cuda", torch.cuda.current_device())


def stream_ptr(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def on_device(t: torch.Tensor, device: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    """`t` as a contiguous tensor on `device` (copying only if needed)."""
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if t.device != device:
        t = t.to(device, non_blocking=False)
    return t.contiguous()
