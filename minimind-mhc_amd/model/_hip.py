"""ctypes binding of libmhc_amd.so, the C ABI declared in include/mhc_amd.h.

PyTorch supplies device memory and the current HIP stream; every kernel call
goes through the C ABI with raw pointers.  There is no CPU or PyTorch
fallback: a missing library, a CPU tensor or an unsupported dtype raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

# The library built next to this package, unless MHC_AMD_LIB names another path
# (for a checkout that copies these modules into its own package).
LIB_PATH = Path(os.environ.get("MHC_AMD_LIB") or
                Path(__file__).resolve().parent.parent / "libmhc_amd.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
MODE_FULL, MODE_NOHRES, MODE_HEAD, MODE_RMS = 0, 1, 2, 3
_DTYPE_TAG = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/mhc_amd.h
_SIGNATURES = {
    "mhc_abi_version": (_I, []),
    "mhc_last_error": (ctypes.c_char_p, []),
    "mhc_init": (_I, []),
    "mhc_phi_packed_bytes": (_I64, [_I, _I, _I]),
    "mhc_phi_pack": (_I, [_P, _I, _P, _I, _I, _I, _P]),
    "mhc_phi_split_bytes": (_I64, [_I, _I, _I]),
    "mhc_phi_pack_split": (_I, [_P, _I, _P, _I, _I, _I, _P]),
    "mhc_pre_fwd": (_I, [_P, _I, _P, _I, _P,              # x, x_dt, phi, phi_dt, packed
                         _P, _P, _P, _P, _P, _P, _I,      # alphas/biases, param_dt
                         _P, _P, _P, _P, _P, _P, _P,      # sub_in, h_pre, h_post, raw, h_res, inv, mixes
                         _I64, _I, _I, _F, _F, _F, _I, _F,
                         _P, _P]),                        # x_ssq, stream
    "mhc_pre_nohres_fwd": (_I, [_P, _I, _P, _I, _P,
                                _P, _P, _P, _P, _I,
                                _P, _P, _P, _P, _P,
                                _I64, _I, _I, _F, _F, _F, _P, _P]),
    "mhc_post_fwd": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _I64, _I, _I, _P, _P]),
    "mhc_post_nohres_fwd": (_I, [_P, _I, _P, _I, _P, _I, _P, _I64, _I, _I, _P, _P]),
    "mhc_head_fwd": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I64, _I, _I, _F, _F,
                          _P, _P]),
    "mhc_pre_norm_fwd": (_I, [_P, _I, _P, _I, _P,
                              _P, _P, _P, _P, _P, _P, _I,
                              _P, _P, _P, _P, _P, _P, _P,
                              _I64, _I, _I, _F, _F, _F, _I, _F,
                              _P, _I, _F, _P, _P]),            # norm weight, dtype, eps, x_ssq, stream
    "mhc_pre_nohres_norm_fwd": (_I, [_P, _I, _P, _I, _P,
                                     _P, _P, _P, _P, _I,
                                     _P, _P, _P, _P, _P,
                                     _I64, _I, _I, _F, _F, _F,
                                     _P, _I, _F, _P, _P]),
    "mhc_head_norm_fwd": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I64, _I, _I, _F, _F,
                               _P, _I, _F, _P, _P]),
    "mhc_expand_norm_fwd": (_I, [_P, _I, _P, _I, _P, _I64, _I, _I, _F, _P, _P]),
    "mhc_pre_token_threshold": (_I64, [_I64]),
    "mhc_pre_row_staging": (_I, [_I]),
    "mhc_pre_group_split_tokens": (_I64, [_I64]),
    "mhc_sinkhorn_fwd": (_I, [_P, _P, _I, _I64, _I, _I, _F, _P]),
    "mhc_stream_expand_fwd": (_I, [_P, _P, _I, _I64, _I, _I, _P]),
    "mhc_post_bwd": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _P, _P, _P, _P, _I64, _I, _I, _P]),
    "mhc_post_nohres_bwd": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _I64, _I, _I, _P]),
    "mhc_pre_bwd": (_I, [_P, _I, _P, _I,                  # x, x_dt, phi, phi_dt
                         _P, _P, _P, _P, _P, _I,          # a_pre, b_pre, a_post, b_post, a_res, param_dt
                         _P, _P,                          # inv_rms, mixes_raw
                         _P, _P, _P, _P, _I,              # g_sub, g_h_pre, g_h_post, g_h_res_raw, grad_dt
                         _P, _P,                          # g_x, g_raw
                         _I64, _I, _I, _I, _F, _F, _P]),
    "mhc_pre_bwd_weights_workspace_bytes": (_I64, [_I64, _I, _I, _I]),
    "mhc_pre_bwd_weights": (_I, [_P, _I, _P, _P, _P,      # x, x_dt, inv, mixes, g_raw
                                 _P, _P, _P, _I,          # alphas, param_dt
                                 _P, _I,                  # g_phi, phi_dt
                                 _P, _P, _P, _P, _P, _P,  # g_alpha/bias pre, post, res
                                 _P, _I64,                # workspace, bytes
                                 _I64, _I, _I, _I, _P]),
    "mhc_pre_bwd_weights_noalloc": (_I, [_P, _I, _P, _P, _P,   # x, x_dt, inv, mixes, g_raw
                                         _P, _P, _P, _I,       # alphas, param_dt
                                         _P, _I,               # g_phi, phi_dt
                                         _P, _P, _P, _P, _P, _P,
                                         _I64, _I, _I, _I, _P]),
    "mhc_sinkhorn_bwd": (_I, [_P, _I, _P, _I, _P, _I, _I64, _I, _I, _F, _P]),
    "mhc_sinkhorn_bwd_max_iters": (_I, [_I]),
}

ABI_VERSION = 8
_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libmhc_amd.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"mhc_amd: {LIB_PATH} is missing; build it with "
            "`python minimind-mhc_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mhc_abi_version() != ABI_VERSION:
        raise RuntimeError(f"mhc_amd: ABI version {lib.mhc_abi_version()} != {ABI_VERSION}")
    _lib = lib
    if torch.cuda.is_available():
        # per-device set-up (the noalloc entry point's scratch addresses), done
        # here so that no later call needs it inside a graph capture
        check(lib.mhc_init(), "mhc_init")
    return lib


def dtype_tag(t: torch.Tensor) -> int:
    try:
        return _DTYPE_TAG[t.dtype]
    except KeyError:
        raise TypeError(f"mhc_amd: unsupported dtype {t.dtype} (fp32, bf16, fp16 only)") from None


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "mhc_amd: tensors must be on a ROCm GPU; the mHC kernels have no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"mhc_amd: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError("mhc_amd: no device tensor given")
    return dev


def stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def check(rc: int, fn: str) -> None:
    if rc != 0:
        msg = load().mhc_last_error().decode(errors="replace")
        raise RuntimeError(f"mhc_amd: {fn} failed (status {rc}): {msg}")


def params_like(ref: torch.Tensor, *ps: torch.Tensor):
    """alpha/bias tensors as contiguous device tensors of one dtype (the first's)."""
    dt = ps[0].dtype
    out = []
    for p in ps:
        p = p.detach()
        if p.dtype != dt:
            p = p.to(dt)
        out.append(p.contiguous())
    dtype_tag(out[0])
    return out
