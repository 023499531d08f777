"""ctypes binding of ``libgptq2d.so``, the C-ABI of the GPTQ-2D HIP kernels.

Every entry point takes raw device pointers, int64 sizes, host arrays describing batch
broadcasting (shape of the broadcast batch, and each operand's batch strides, 0 where it
broadcasts), and the HIP stream to launch on; it returns 0 or an error code.  The library is
loaded lazily and never replaced by a fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libgptq2d.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F64 = ctypes.c_double
_AP = ctypes.POINTER(ctypes.c_int64)

# name -> argument types, for both the _f32 and _f64 variants
_SIGNATURES = {
    "push_plain": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _AP, _P],
    "add_own_errors": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "push_down_se": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _P],
    "push_right_se": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _P],
    "gather_antidiagonal": [_P, _P, _I64, _I64, _I64, _I64, _P],
    "fill": [_P, _F64, _I64, _P],
    "flush": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _AP, _P],
    "sweep_fused": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _AP, _AP, _AP, _I32, _P, _AP, _P, _AP, _F64, _F64, _P,
                    _I64, _I64, _I64, _P],
    "sweep_fused_se": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _AP, _I32, _P, _AP, _P, _AP, _F64,
                       _F64, _I32, _P, _P, _I64, _I64, _I64, _P],
    "sweep_fused_noalloc": [_P, _P, _P, _I64, _I64, _I32, _AP, _AP, _AP, _I32, _P, _AP, _P, _AP, _F64, _F64, _P, _I64,
                            _P],
    "affine_quantize": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _AP, _F64, _F64, _P],
    "round_quantize": [_P, _P, _I64, _I64, _I64, _I64, _I32, _AP, _P],
    "affine_quantize_se": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _AP, _AP, _AP, _F64,
                           _F64, _P],
    "round_quantize_se": [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _AP, _P],
    "absmax_scale": [_P, _P, _I64, _I64, _I64, _I64, _F64, _F64, _I32, _P],
    "absmax_quantize_se": [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F64, _F64, _I32, _P, _P],
    "ldl_of_inverse": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "ldl": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "ldl_of_inverse_part": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P],
    "ldl_of_inverse_pair": [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P, _P],
    "gemm": [_I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _F64, _F64,
             _I32, _I32, _I32, _P],
    "viterbi": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _I32, _P],
    "pack_int": [_P, _I64, _I64, _I64, _P, _AP, _P, _AP, _F64, _F64, _I32, _P, _I64, _P, _P],
    "unpack_int": [_P, _I64, _I64, _I64, _I64, _P, _AP, _P, _AP, _F64, _I32, _P, _P],
    "trellis_unpack": [_P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _I64, _P, _P, _P],
}

_lib = None


class GPTQ2DError(RuntimeError):
    """A C-ABI call of the GPTQ-2D library returned an error code."""


def lib() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise GPTQ2DError(f"{LIB_PATH} is missing: build it with `python gptq-2d_amd/build_lib.py`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in _SIGNATURES.items():
            for suffix in ("f32", "f64"):
                fn = getattr(handle, f"gptq2d_{name}_{suffix}")
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
        handle.gptq2d_sweep_fused_noalloc_capacity.argtypes = [_I32]
        handle.gptq2d_sweep_fused_noalloc_capacity.restype = ctypes.c_int64
        handle.gptq2d_viterbi_rows_f32.argtypes = [_P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _I64, _I64, _I32, _I32,
                                                   _I32, _I32, _P]
        handle.gptq2d_viterbi_rows_f32.restype = ctypes.c_int
        handle.gptq2d_sweep_fused_kron_f32.argtypes = [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32,
                                                       _P, _P, _F64, _F64, _I32, _P, _P, _I64, _I64, _I64, _P]
        handle.gptq2d_sweep_fused_kron_f32.restype = ctypes.c_int
        handle.gptq2d_viterbi_workspace.argtypes = [_I64, _I64, _I32, _I32, _I32]
        handle.gptq2d_viterbi_workspace.restype = ctypes.c_int64
        handle.gptq2d_int_code_bits.argtypes = [_F64, _F64]
        handle.gptq2d_int_code_bits.restype = ctypes.c_int32
        handle.gptq2d_trellis_stream_words.argtypes = [_I64, _I32, _I32, _I32, _I32]
        handle.gptq2d_trellis_stream_words.restype = ctypes.c_int64
        handle.gptq2d_trellis_pack.argtypes = [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P,
                                               _I64, _P, _P]
        handle.gptq2d_trellis_pack.restype = ctypes.c_int
        handle.gptq2d_profile_start.argtypes = [_I64, ctypes.c_uint32]
        handle.gptq2d_profile_start.restype = ctypes.c_int
        handle.gptq2d_profile_read.argtypes = [_I32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                               ctypes.POINTER(ctypes.c_int64)]
        handle.gptq2d_profile_read.restype = ctypes.c_int
        handle.gptq2d_profile_stop.argtypes = []
        handle.gptq2d_profile_stop.restype = ctypes.c_int
        _lib = handle
    return _lib


def call_untyped(name: str, *args) -> None:
    """Call ``gptq2d_<name>`` (an entry point with no element type) and raise on a non-zero return code."""
    rc = getattr(lib(), f"gptq2d_{name}")(*args)
    if rc != 0:
        raise GPTQ2DError(f"gptq2d_{name} failed with code {rc}")


def call(name: str, dtype: torch.dtype, *args) -> None:
    """Call ``gptq2d_<name>_<f32|f64>`` and raise on a non-zero return code."""
    suffix = {torch.float32: "f32", torch.float64: "f64"}.get(dtype)
    if suffix is None:
        raise GPTQ2DError(f"unsupported dtype {dtype}")
    fn = getattr(lib(), f"gptq2d_{name}_{suffix}")
    rc = fn(*args)
    if rc != 0:
        raise GPTQ2DError(f"gptq2d_{name}_{suffix} failed with code {rc}")


# Kernel classes of the launch profiler (csrc/profile.h).
PROF_FLUSH, PROF_TILE_SWEEP, PROF_LDL_GEMM = 0, 1, 2


def profile_start(capacity: int = 4096, kinds=(PROF_FLUSH, PROF_TILE_SWEEP, PROF_LDL_GEMM)) -> None:
    """Time every launch of the kernel classes ``kinds`` with HIP events until ``profile_stop``."""
    rc = lib().gptq2d_profile_start(capacity, sum(1 << k for k in kinds))
    if rc:
        raise GPTQ2DError(f"gptq2d_profile_start failed with code {rc}")


def profile_read(kind: int):
    """(summed launch ms, summed algorithmic work, launches) of one kernel class; waits for its events."""
    ms, work, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
    rc = lib().gptq2d_profile_read(kind, ctypes.byref(ms), ctypes.byref(work), ctypes.byref(n))
    if rc:
        raise GPTQ2DError(f"gptq2d_profile_read failed with code {rc}")
    return ms.value, work.value, n.value


def profile_stop() -> None:
    lib().gptq2d_profile_stop()


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def i64_array(values) -> ctypes.Array:
    values = [int(v) for v in values]
    return (ctypes.c_int64 * max(1, len(values)))(*(values or [0]))


def batch_strides(x: torch.Tensor, batch_shape: torch.Size) -> ctypes.Array:
    """Batch strides of matrix-shaped ``x`` broadcast to ``batch_shape`` (0 on broadcast dims)."""
    pad = len(batch_shape) - (x.dim() - 2)
    view = x.reshape((1,) * pad + tuple(x.shape)).expand(*batch_shape, *x.shape[-2:])
    return i64_array(view.stride()[:-2])


def require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise GPTQ2DError("the HIP engine needs GPU tensors")
