"""Integer quantizer plug-ins for GPTQ-2D (drop-in for the reference's ``quantizer_int.py``).

A quantizer is called once per antidiagonal as ``quantizer(y_flat, selection, *inputs, out=z)``:
``y_flat`` is the live matrix Y flattened to ``[*batch, m*n]`` (earlier antidiagonals already hold
their rounded values), ``selection`` a flat slice of the antidiagonal or, for super-entries, a
``select`` callable viewing any ``[..., m*n]`` tensor as ``[..., d, p, q]``; ``out`` is contiguous
and must be overwritten completely (reference gptq_2d.py:147-164, quantizer_int.py:1-134).

The ``*_hip`` plug-ins run one HIP kernel per call and never synchronise with the host, so they
can be captured in a hipGraph; the reference's ``*_triton`` names are aliases of them.  The
``*_torch`` plug-ins are the reference's PyTorch formulations.  ``gptq_2d`` recognises
``round_quantizer`` and the affine plug-ins (with full-matrix scale and zero point) and then fuses
the rounding into its tile sweep instead of calling the plug-in per antidiagonal.

The affine plug-ins write ``(clamp(round(y / scale + zero_point), qmin, qmax) - zero_point) *
scale``; ``int_abs_max_scale_*`` gives GPTQ's symmetric scales.
"""

from __future__ import annotations

from typing import Callable

import torch

import _hip

_SCALE_DTYPES = {torch.bfloat16: 1, torch.float16: 2}


def _pick(flat: torch.Tensor, selection) -> torch.Tensor:
    return selection(flat) if callable(selection) else flat[..., selection]


# ------------------------------------------------------------------------------------------------ rounding

def round_quantizer(y_flat: torch.Tensor, antidiagonal_slice: slice, *, out: torch.Tensor) -> None:
    """Round the selected antidiagonal half to even into ``out`` (quantizer_int.py:18-25)."""
    if not y_flat.is_cuda:
        torch.round(y_flat[..., antidiagonal_slice], out=out)
        return
    assert y_flat.is_contiguous() and out.is_contiguous(), "the HIP round quantizer needs contiguous Y and out"
    batch_shape = y_flat.shape[:-1]
    sl = antidiagonal_slice
    length = out.size(-1)
    _hip.call("round_quantize", y_flat.dtype, _hip.ptr(out), _hip.ptr(y_flat), y_flat.size(-1), sl.start or 0,
              sl.step or 1, length, len(batch_shape), _hip.i64_array(batch_shape), _hip.stream(y_flat.device))


def round_quantizer_super_entry(y_flat: torch.Tensor, select: Callable, *, out: torch.Tensor) -> None:
    """Round the selected super-entries half to even into ``out`` (quantizer_int.py:28-35)."""
    x = select(y_flat)
    if not y_flat.is_cuda:
        torch.round(x, out=out)
        return
    assert y_flat.is_contiguous() and out.is_contiguous(), "the HIP round quantizer needs contiguous Y and out"
    assert x.untyped_storage().data_ptr() == y_flat.untyped_storage().data_ptr(), "select must return views"
    assert out.shape == x.shape
    batch_shape = y_flat.shape[:-1]
    d, p, q = x.shape[-3:]
    sd, sp, sq = x.stride()[-3:]
    _hip.call("round_quantize_se", y_flat.dtype, _hip.ptr(out), _hip.ptr(x), y_flat.size(-1), d, p, q, sd, sp, sq,
              len(batch_shape), _hip.i64_array(batch_shape), _hip.stream(y_flat.device))


# ------------------------------------------------------------------------------------------------ affine

def _validate_affine_inputs(y_flat, scale, zero_point, out, qmin, qmax) -> torch.Size:
    """The reference's affine input contract (quantizer_int.py:38-60); returns Y's batch shape."""
    assert qmin < qmax, "expected qmin < qmax"
    assert scale.dim() >= 2 and zero_point.dim() >= 2, "scale and zero point must have matrix dimensions"
    assert scale.shape[-2:] == zero_point.shape[-2:], "scale and zero point matrix shapes must match"
    assert scale.shape[-2:].numel() == y_flat.size(-1), "scale and zero point matrix shapes must match Y"
    assert scale.dtype == zero_point.dtype == y_flat.dtype, "scale, zero point, and Y must share dtype"
    assert scale.device == zero_point.device == y_flat.device, "scale, zero point, and Y must share device"
    batch_shape = y_flat.shape[:-1]
    assert torch.broadcast_shapes(scale.shape[:-2], zero_point.shape[:-2], batch_shape) == batch_shape, (
        "scale and zero point batch dimensions must broadcast to Y"
    )
    assert out.shape[:-1] == batch_shape and out.dtype == y_flat.dtype and out.device == y_flat.device, (
        "out must match Y's batch shape, dtype, and device"
    )
    return batch_shape


def affine_quantizer_torch(y_flat, antidiagonal_slice, scale, zero_point, *, out, qmin=-torch.inf, qmax=torch.inf):
    """Affine-quantize one antidiagonal with PyTorch (quantizer_int.py:63-83)."""
    _validate_affine_inputs(y_flat, scale, zero_point, out, qmin, qmax)
    y = y_flat[..., antidiagonal_slice]
    s = scale.flatten(start_dim=-2)[..., antidiagonal_slice]
    zp = zero_point.flatten(start_dim=-2)[..., antidiagonal_slice]
    torch.div(y, s, out=out)
    out.add_(zp).round_().clamp_(qmin, qmax)
    out.sub_(zp).mul_(s)


def affine_quantizer_super_entry_torch(y_flat, select, scale, zero_point, *, out, qmin=-torch.inf, qmax=torch.inf):
    """Affine-quantize selected super-entries entry by entry with PyTorch (quantizer_int.py:86-107)."""
    _validate_affine_inputs(y_flat, scale, zero_point, out.flatten(start_dim=-3), qmin, qmax)
    y = select(y_flat)
    s = select(scale.flatten(start_dim=-2))
    zp = select(zero_point.flatten(start_dim=-2))
    torch.div(y, s, out=out)
    out.add_(zp).round_().clamp_(qmin, qmax)
    out.sub_(zp).mul_(s)


def affine_quantizer_hip(y_flat, antidiagonal_slice, scale, zero_point, *, out, qmin=-torch.inf, qmax=torch.inf):
    """Affine-quantize one antidiagonal in one HIP kernel (quantizer_int.py:208-244)."""
    batch_shape = _validate_affine_inputs(y_flat, scale, zero_point, out, qmin, qmax)
    _hip.require_device(y_flat)
    assert y_flat.is_contiguous() and scale.is_contiguous() and zero_point.is_contiguous() and out.is_contiguous(), (
        "the HIP affine quantizer requires contiguous Y, scale, zero point, and out"
    )
    assert out.shape == y_flat[..., antidiagonal_slice].shape, "out must match the selected antidiagonal"
    sl = antidiagonal_slice
    _hip.call("affine_quantize", y_flat.dtype, _hip.ptr(out), _hip.ptr(y_flat), _hip.ptr(scale), _hip.ptr(zero_point),
              y_flat.size(-1), sl.start or 0, sl.step or 1, out.size(-1), len(batch_shape),
              _hip.i64_array(batch_shape), _hip.batch_strides(scale, batch_shape),
              _hip.batch_strides(zero_point, batch_shape), float(qmin), float(qmax), _hip.stream(y_flat.device))


def affine_quantizer_super_entry_hip(y_flat, select, scale, zero_point, *, out, qmin=-torch.inf, qmax=torch.inf):
    """Affine-quantize selected super-entries in one HIP kernel, reading them through the views' strides
    (quantizer_int.py:302-351)."""
    batch_shape = _validate_affine_inputs(y_flat, scale, zero_point, out.flatten(start_dim=-3), qmin, qmax)
    _hip.require_device(y_flat)
    assert y_flat.is_contiguous() and scale.is_contiguous() and zero_point.is_contiguous() and out.is_contiguous(), (
        "the HIP affine quantizer requires contiguous Y, scale, zero point, and out"
    )
    sources = y_flat, scale.flatten(start_dim=-2), zero_point.flatten(start_dim=-2)
    views = tuple(select(src) for src in sources)
    assert all(v.untyped_storage().data_ptr() == src.untyped_storage().data_ptr() for v, src in zip(views, sources)), (
        "select must return views"
    )
    assert views[0].stride()[-3:] == views[1].stride()[-3:] == views[2].stride()[-3:], (
        "Y, scale, and zero point must share their layout"
    )
    assert out.shape == views[0].shape, "out must match the selected super-entries"
    d, p, q = views[0].shape[-3:]
    sd, sp, sq = views[0].stride()[-3:]
    _hip.call("affine_quantize_se", y_flat.dtype, _hip.ptr(out), _hip.ptr(views[0]), _hip.ptr(views[1]),
              _hip.ptr(views[2]), y_flat.size(-1), d, p, q, sd, sp, sq, len(batch_shape), _hip.i64_array(batch_shape),
              _hip.batch_strides(scale, batch_shape), _hip.batch_strides(zero_point, batch_shape), float(qmin),
              float(qmax), _hip.stream(y_flat.device))


# ------------------------------------------------------------------------------------------------ INT abs-max

def int_abs_max_scale_torch(x: torch.Tensor, *, qmin: float, qmax: float, dtype: torch.dtype) -> torch.Tensor:
    """GPTQ's symmetric scale 2 absmax / (qmax - qmin) of each last-dim row, rounded to ``dtype``, or 1 for a
    row of zeros (quantizer_int.py:110-117)."""
    divisor = x.new_full((), (qmax - qmin) / 2)
    scale = torch.linalg.vector_norm(x, ord=torch.inf, dim=-1, keepdim=True).div_(divisor).to(dtype).to(x.dtype)
    return scale.masked_fill_(scale == 0, 1.)


def int_abs_max_scale_hip(x: torch.Tensor, *, qmin: float, qmax: float, dtype: torch.dtype) -> torch.Tensor:
    """``int_abs_max_scale_torch`` for a 16-bit ``dtype`` in one HIP kernel (quantizer_int.py:388-404)."""
    _hip.require_device(x)
    assert dtype in _SCALE_DTYPES, "the HIP scale rounds to fp16 or bf16"
    assert qmin < qmax
    rows = x.reshape(-1, x.size(-1))
    out = x.new_empty(*x.shape[:-1], 1)
    _hip.call("absmax_scale", x.dtype, _hip.ptr(out), _hip.ptr(rows), rows.size(0), rows.size(1), rows.stride(0),
              rows.stride(1), float(qmin), float(qmax), _SCALE_DTYPES[dtype], _hip.stream(x.device))
    return out


def _scale_map(scales, y_flat):
    """The optional per-entry scale map of the abs-max quantizers: [*batch, m, n] like Y, flattened."""
    flat = scales.flatten(start_dim=-2)
    assert flat.shape == y_flat.shape and flat.dtype == y_flat.dtype and flat.device == y_flat.device, (
        "scales must be a [*batch, m, n] tensor of Y's batch shape, dtype and device"
    )
    return flat


def int_abs_max_quantizer_torch(y_flat, select, scales=None, *, out, qmin, qmax, dtype) -> None:
    """Round each row of the selected super-entries to qmin..qmax times its current abs-max scale, with PyTorch
    (quantizer_int.py:120-134).  ``scales`` (optional, [*batch, m, n], no reference counterpart): every entry
    receives the scale its row was rounded with -- the scales of the packed layer."""
    x = select(y_flat)
    scale = int_abs_max_scale_torch(x, qmin=qmin, qmax=qmax, dtype=dtype)
    torch.div(x, scale, out=out).round_().clamp_(qmin, qmax).mul_(scale)
    if scales is not None:
        select(_scale_map(scales, y_flat)).copy_(scale.expand_as(x))


def int_abs_max_quantizer_hip(y_flat, select, scales=None, *, out, qmin, qmax, dtype) -> None:
    """``int_abs_max_quantizer_torch`` in one HIP kernel that reads each row through the view's strides
    (quantizer_int.py:442-470); ``scales`` as there, written by the same kernel."""
    x = select(y_flat)
    _hip.require_device(y_flat)
    assert y_flat.is_contiguous() and out.is_contiguous(), "the HIP quantizer requires contiguous Y and out"
    assert x.untyped_storage().data_ptr() == y_flat.untyped_storage().data_ptr(), "select must return views"
    assert out.shape == x.shape and out.dtype == x.dtype, "out must match the selected super-entries"
    assert qmin < qmax and dtype in _SCALE_DTYPES, "expected qmin < qmax and a scale in fp16 or bf16"
    d, p, q = x.shape[-3:]
    sd, sp, sq = x.stride()[-3:]
    B = y_flat.shape[:-1].numel()
    sv = None
    if scales is not None:
        flat = _scale_map(scales, y_flat)
        assert flat.is_contiguous(), "the HIP quantizer writes a contiguous scale map"
        sv = select(flat)
        assert sv.stride() == x.stride(), "select must view the scale map as it views Y"
    _hip.call("absmax_quantize_se", y_flat.dtype, _hip.ptr(out), _hip.ptr(x), y_flat.size(-1), B, d, p, q, sd, sp, sq,
              float(qmin), float(qmax), _SCALE_DTYPES[dtype], _hip.ptr(sv), _hip.stream(y_flat.device))


# ------------------------------------------------------------------------------------------------ teacher forcing

def teacher_forced_quantizer(y_flat, selection, values, y_before, *, out) -> None:
    """Write the prescribed rounded ``values`` and record Y just before rounding into ``y_before``.

    ``values`` and ``y_before`` are ``[*batch, m, n]``.  This plug-in has no counterpart in the
    reference: it measures how close an engine's pre-rounding Y stays to another implementation's
    trajectory when both are forced to the same codes.  ``gptq_2d`` fuses it like the built-ins.
    """
    _pick(y_before.flatten(start_dim=-2), selection).copy_(_pick(y_flat, selection))
    out.copy_(_pick(values.flatten(start_dim=-2), selection))


# The reference's Triton names, kept for drop-in use: one implementation, not two.
affine_quantizer_triton = affine_quantizer_hip
affine_quantizer_super_entry_triton = affine_quantizer_super_entry_hip
int_abs_max_scale_triton = int_abs_max_scale_hip
int_abs_max_quantizer_triton = int_abs_max_quantizer_hip
