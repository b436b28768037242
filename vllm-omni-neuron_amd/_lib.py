"""ctypes binding of libwanmi.so, the gfx950 kernel library.

There is no CPU fallback: every op in this package runs the HIP kernels or raises. A missing
library, a CPU tensor, or a non-zero status from the C ABI is an error.
"""

from __future__ import annotations

import ctypes
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libwanmi.so"

WANMI_OK = 0
WANMI_ERR_ARG = -1
WANMI_ERR_UNSUPPORTED = -2
WANMI_ERR_HIP = -3

NORM = {"none": 0, "layer_norm": 1, "rms_norm": 2}
QUANT = {"none": 0, "mx": 1, "row": 2}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes, mirroring include/wanmi.h
_SIGNATURES = {
    "wanmi_abi_version": [],
    "wanmi_last_error": [],
    "wanmi_adaln_quant": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _i32, _vp, _vp, _vp, _vp],
    "wanmi_e4m3_encode": [_vp, _vp, _i64, _vp],
    "wanmi_mxfp8_gemm": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp, _i64, _vp, _vp, _vp, _vp],
    "wanmi_qk_rmsnorm_rope": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _f32, _vp, _vp],
    "wanmi_qk_rmsnorm_rope_to": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _f32, _vp, _i64, _i64, _vp],
    "wanmi_rope_tables": [_i64, _i64, _i64, _i32, _i64, ctypes.c_double, _i32, _vp, _vp, _vp],
    "wanmi_transpose_heads": [_vp, _i64, _i64, _i64, _i32, _vp, _i64, _vp],
    "wanmi_head_max_norm": [_vp, _i64, _i64, _i64, _i32, _vp, _vp],
    "wanmi_mxfp8_gemm_rowsumsq": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp],
    "wanmi_mxfp8_gemm_qkv": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                             _i64, _vp],
    "wanmi_attention_const_max": [
        _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _f32, _i32,
        _vp, _i64, _i64, _i64, _vp, _i64, _vp,
    ],
    "wanmi_attention_exact": [
        _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _f32, _i32,
        _vp, _i64, _i64, _i64, _vp, _vp,
    ],
    "wanmi_attention_exact_noalloc": [
        _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _f32, _i32,
        _vp, _i64, _i64, _i64, _vp,
    ],
    "wanmi_hbm_stream_copy": [_vp, _vp, _i64, _vp],
    "wanmi_hbm_stream_fold": [_vp, _vp, _i64, _vp],
    "wanmi_dmajor_to_mx": [_vp, _i64, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp],
    "wanmi_qk_rmsnorm_rope_qrr": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _i32, _f32, _vp, _vp, _i64, _i32, _f32, _vp, _vp],
    "wanmi_attention_const_max_qrr": [
        _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _f32, _i32,
        _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
    ],
    "wanmi_attention_const_max_qprep": [
        _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _f32, _i32,
        _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _f32, _vp,
    ],
}

_LIB = None


class WanmiError(RuntimeError):
    """A HIP launch or runtime failure reported by libwanmi."""


def load() -> ctypes.CDLL:
    """Load libwanmi.so once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the gfx950 kernels first (__graft_entry__.build()); "
            "this package has no CPU fallback"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _i32
    lib.wanmi_last_error.restype = ctypes.c_char_p
    _LIB = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def hbm_stream_copy(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """Copy ``src`` into ``dst`` (same number of bytes, a multiple of 16; contiguous, on one GPU)
    with the library's streaming copy kernel, on the current stream. Measurement helper: the
    practical HBM streaming rate the memory-bound kernels are compared against."""
    lib = load()
    if src.device.type != "cuda" or dst.device != src.device:
        raise RuntimeError("hbm_stream_copy: src and dst must be on the same GPU; no CPU fallback")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("hbm_stream_copy: src and dst must be contiguous")
    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != n:
        raise ValueError("hbm_stream_copy: src and dst must hold the same number of bytes")
    check(lib.wanmi_hbm_stream_copy(ptr(src), ptr(dst), n, stream_of(src)), "wanmi_hbm_stream_copy")
    return dst


def hbm_stream_fold(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """Read ``src`` (a multiple of 32768 bytes) and write half as many bytes to ``dst`` with the
    library's read-2-write-1 streaming kernel (``wanmi_hbm_stream_fold``: each output 16-byte word
    is the xor of two input words), on the current stream. Measurement helper: the HBM ceiling for
    a pass that reads two bytes per byte it writes, as the adaLN + MX pass does."""
    lib = load()
    if src.device.type != "cuda" or dst.device != src.device:
        raise RuntimeError("hbm_stream_fold: src and dst must be on the same GPU; no CPU fallback")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("hbm_stream_fold: src and dst must be contiguous")
    n = src.numel() * src.element_size()
    if n % 32768:
        raise ValueError("hbm_stream_fold: src must hold a multiple of 32768 bytes")
    if dst.numel() * dst.element_size() != n // 2:
        raise ValueError("hbm_stream_fold: dst must hold half as many bytes as src")
    check(lib.wanmi_hbm_stream_fold(ptr(src), ptr(dst), n, stream_of(src)), "wanmi_hbm_stream_fold")
    return dst


def check(status: int, what: str) -> None:
    if status == WANMI_OK:
        return
    msg = load().wanmi_last_error().decode(errors="replace")
    if status == WANMI_ERR_ARG:
        raise ValueError(f"{what}: {msg}")
    if status == WANMI_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise WanmiError(f"{what}: status {status}: {msg}")


def ptr(t: torch.Tensor | None):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current HIP stream of ``t``'s device, as the void* the C ABI takes."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def expect(t: torch.Tensor | None, what: str, *, dtype: torch.dtype, shape: tuple | None = None,
           contiguous: bool = True, optional: bool = False, row_contiguous: bool = False) -> None:
    """Host-side check of one tensor whose pointer goes to the C ABI: dtype, exact shape (None
    entries match any size) and memory layout. Raises ValueError before anything is launched."""
    if t is None:
        if optional:
            return
        raise ValueError(f"{what} is required")
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{what} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise ValueError(f"{what} must be {dtype}, got {t.dtype}")
    if shape is not None:
        if t.dim() != len(shape) or any(want is not None and have != want for have, want in zip(t.shape, shape)):
            want = "[" + ", ".join("*" if w is None else str(w) for w in shape) + "]"
            raise ValueError(f"{what} must have shape {want}, got {list(t.shape)}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if row_contiguous and t.dim() >= 1 and t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{what} must have unit stride along its last dimension")


def require_gpu(*tensors: torch.Tensor | None, what: str) -> torch.device:
    """Every tensor must live on the same GPU; the kernels never run on the host."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{what}: tensors must be on a ROCm GPU (got {t.device}); no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{what}: no tensor given")
    return dev
