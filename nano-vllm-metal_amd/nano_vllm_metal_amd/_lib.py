"""ctypes binding of libnvm_moe.so (the C ABI in include/nvm_moe.h).

There is no fallback: if the shared library is missing or fails to load, every
entry point raises.  Errors returned by the library become ``ValueError``
(invalid or unsupported arguments) or ``RuntimeError`` (workspace, HIP).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libnvm_moe.so"

NVM_OK = 0
NVM_ERR_INVALID = -1
NVM_ERR_UNSUPPORTED = -2
NVM_ERR_WORKSPACE = -3
NVM_ERR_HIP = -4

REGIME_AUTO, REGIME_DECODE, REGIME_PREFILL = 0, 1, 2

ABI_VERSION = 2  # NVM_ABI_VERSION of include/nvm_moe.h

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}
# nvm_kv_dtype of include/nvm_attention.h
KV_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2, torch.int8: 3}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> argtypes; every function returns int status except the two getters
SIGNATURES = {
    "nvm_quantized_matmul": [_P, _P, _I, _I, _P, _P, _I, _P, _I64, _I64, _I64, _I, _P],
    "nvm_route_workspace_size": [_I64, _I64, _I64, ctypes.POINTER(_SZ)],
    "nvm_moe_route": [_P, _I64, _I64, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P],
    "nvm_dispatch_workspace_size": [_I64, _I64, ctypes.POINTER(_SZ)],
    "nvm_moe_dispatch": [_P, _I64, _I64, _P, _P, _P, _SZ, _P],
    "nvm_route_dispatch_workspace_size": [_I64, _I64, _I64, _I, ctypes.POINTER(_SZ)],
    "nvm_moe_route_dispatch": [_P, _I64, _I64, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _P, _P,
                               _P, _P, _P, _SZ, _P],
    "nvm_grouped_linear_workspace_size": [_I64, _I64, _I64, _I64, ctypes.POINTER(_SZ)],
    "nvm_grouped_expert_linear": [_P, _I64, _I64, _P, _P, _P, _I64, _I64, _I, _I, _P, _I, _P, _I, _P, _SZ, _P],
    "nvm_moe_workspace_size": [_I64, _I64, _I64, _I64, _I, ctypes.POINTER(_SZ)],
    "nvm_moe_expert_gateup": [_P, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P,
                              _P, _P, _P, _I, _P],
    "nvm_moe_expert_down": [_P, _I64, _I64, _I64, _I64, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P],
    "nvm_moe_combine": [_P, _P, _I64, _I, _I64, _I, _P, _P],
    "nvm_paged_attention_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I, _I, _I,
                                           ctypes.POINTER(_SZ)],
    "nvm_paged_attention": [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I, _P, _P, _P, _I64, _I64,
                            _P, ctypes.c_float, _I, _I, _I, _I, _P, _P, _SZ, _P],
    "nvm_causal_attention": [_P, _P, _P, _I64, _I64, _I, _I, _I64, ctypes.c_float, _I, _I, _P, _P],
    "nvm_residual_rms_norm": [_P, _P, _P, _I64, _I64, ctypes.c_float, _I, _P, _P, _P],
    "nvm_embedding": [_P, _I64, _P, _P, _P, _I64, _I64, _I, _I, _I, _P, _P],
    "nvm_qk_norm_rope_store": [_P, _I64, _I, _I, _I64, _P, _P, ctypes.c_float, _P, _P, _P, _I64,
                               _P, _P, _P, _P, _I64, _I64, _I, _P, _P, _P, _P],
    "nvm_moe_forward_residual_norm": [_P, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I,
                                      _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _P, _P, ctypes.c_float, _P, _P, _I, _P, _SZ, _P],
    "nvm_moe_forward": [_P, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I,
                        _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                        _P, _P, _P, _I, _P, _SZ, _P],
    "nvm_moe_forward_stage": [_I, _P, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I,
                              _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                              _P, _P, _P, _I, _P, _SZ, _P],
    "nvm_moe_forward_plan": [_I64, _I64, _I64, _I64, _I, _I, _I, ctypes.POINTER(_I)],
    "nvm_moe_scratch_bytes": [ctypes.POINTER(_SZ)],
    "nvm_moe_forward_noalloc": [_P, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I,
                                _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                _P, _P, _P, _I, _P],
}

_lib = None


def library_path() -> Path:
    return Path(os.environ.get("NVM_MOE_LIB", LIB_PATH))


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"nano_vllm_metal_amd: HIP library {path} is missing; build it with "
            "`python -m nano_vllm_metal_amd._build` (there is no CPU fallback)")
    lib = ctypes.CDLL(str(path))
    lib.nvm_abi_version.restype = _I
    lib.nvm_abi_version.argtypes = []
    lib.nvm_last_error.restype = ctypes.c_char_p
    lib.nvm_last_error.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = _I
        fn.argtypes = args
    if lib.nvm_abi_version() != ABI_VERSION:
        raise RuntimeError(f"unexpected ABI version {lib.nvm_abi_version()}")
    _lib = lib
    return lib


def check(status: int) -> None:
    if status == NVM_OK:
        return
    msg = _lib.nvm_last_error().decode(errors="replace")
    if status in (NVM_ERR_INVALID, NVM_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"activations must be float16 or bfloat16, got {dtype}") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one GPU; the HIP kernels are the only path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("nano_vllm_metal_amd runs on the GPU only; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev
