"""CPU restatement of the reference's PyTorch quantizers (test oracle only).

Restates quantizer_int.py:18-134: nearest rounding, the affine quantizer
``(clamp(round(y/s + z), qmin, qmax) - z) * s`` for antidiagonal slices and
super-entry selectors, and GPTQ's symmetric abs-max scale rounded to a 16-bit
dtype.

Pinned by: tests/test_oracle_quantize.py -- the reference's known answers
(quantizer_int.py:476-488, 532-533), the closed form checked entry by entry in
Python float arithmetic, round-half-to-even ties, a zero row (scale 1) and a
denormal scale, the bf16/fp16 scale rounding checked against an independent
bit-level round-to-nearest-even restatement, and the abs-max quantizer against
vectors the reference's ``int_abs_max_quantizer_torch`` wrote on the cases of
its own test (quantizer_int.py:535-553, ``tests/golden/absmax.npz``) with rows
of exact ties; planted floor, trunc and half-away-from-zero rounding fail
those checks.
"""

from __future__ import annotations

import torch


def _pick(flat, selection):
    return selection(flat) if callable(selection) else flat[..., selection]


def _round_half_even(t):
    """In place, to the nearest integer, ties to even (torch.round, as every reference quantizer rounds)."""
    return t.round_()


def round_quantizer(y_flat, selection, *, out):
    """Round half to even into ``out`` (quantizer_int.py:18-35, both variants)."""
    _round_half_even(out.copy_(_pick(y_flat, selection)))


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
    _round_half_even(out.add_(zp)).clamp_(qmin, qmax)
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
    _round_half_even(torch.div(x, s, out=out)).clamp_(qmin, qmax).mul_(s)
