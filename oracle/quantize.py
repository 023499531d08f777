"""CPU restatement of the reference's PyTorch quantizers (test oracle only).

Restates quantizer_int.py:18-134: nearest rounding, the affine quantizer
``(clamp(round(y/s + z), qmin, qmax) - z) * s`` for antidiagonal slices and
super-entry selectors, and GPTQ's symmetric abs-max scale rounded to a 16-bit
dtype.

Pinned by: tests/test_oracle_quantize.py -- the reference's known answers
(quantizer_int.py:476-488, 532-533), the closed form checked entry by entry in
Python ``fractions`` arithmetic, round-half-to-even ties, a zero row (scale 1)
and a denormal scale, and the bf16/fp16 scale rounding checked against an
independent bit-level round-to-nearest-even restatement.
"""

from __future__ import annotations

import torch


def _pick(flat, selection):
    return selection(flat) if callable(selection) else flat[..., selection]


def round_quantizer(y_flat, selection, *, out):
    """Round half to even into ``out`` (quantizer_int.py:18-35, both variants)."""
    torch.round(_pick(y_flat, selection), out=out)


def affine_quantizer(y_flat, selection, scale, zero_point, *, out, qmin=-float("inf"), qmax=float("inf")):
    """Affine quantize with full-matrix scale and zero point (quantizer_int.py:63-107).

    ``selection`` is a flat slice or a super-entry selector; scale and zero point are
    ``[*, m, n]`` and are picked with the same selection after flattening.
    """
    assert qmin < qmax
    y = _pick(y_flat, selection)
    s = _pick(scale.flatten(-2), selection)
    zp = _pick(zero_point.flatten(-2), selection)
    torch.div(y, s, out=out)
    out.add_(zp).round_().clamp_(qmin, qmax)
    out.sub_(zp).mul_(s)


def int_abs_max_scale(x, *, qmin, qmax, dtype):
    """absmax / ((qmax - qmin)/2) per last-dim row, rounded to ``dtype``, zero -> 1 (quantizer_int.py:110-117)."""
    divisor = x.new_full((), (qmax - qmin) / 2)
    s = torch.linalg.vector_norm(x, ord=torch.inf, dim=-1, keepdim=True).div_(divisor).to(dtype).to(x.dtype)
    return s.masked_fill_(s == 0, 1.)


def int_abs_max_quantizer(y_flat, select, *, out, qmin, qmax, dtype):
    """Per-row abs-max INT quantizer of super-entries from current values (quantizer_int.py:120-134)."""
    x = select(y_flat)
    s = int_abs_max_scale(x, qmin=qmin, qmax=qmax, dtype=dtype)
    torch.div(x, s, out=out).round_().clamp_(qmin, qmax).mul_(s)
