"""CPU restatement of the reference's PyTorch sweeps (test oracle only).

Restates gptq_2d.py:65-164 (input contract, antidiagonal geometry, the
quantizer call) and gptq_2d.py:1122-1292 (``direct_2d``, ``gptq_2d_torch``
and their super-entry variants).  ``gptq_2d_torch`` keeps the reference's
exact sequence of floating-point operations (three ``addcmul_`` per stage,
gptq_2d.py:1217-1235) so that its fp32 codes are the reference's codes; the
other functions only need to be exact in fp64.

Pinned by: tests/test_oracle_algorithms.py (every sweep equals Algorithm 1 on
vec(X) bitwise in fp64 on the reference's test shapes, with a
coordinate-dependent codebook), tests/test_oracle_golden.py (fp32 codes of
``gptq_2d_torch`` at 512x512 against vectors written from the reference) and
tests/test_oracle_sweep_state.py (``TorchSweepState`` run stage by stage
against the same golden codes and against Algorithm 1 with NaN-poisoned
triangles; ``stage_work`` against a brute-force count of the entries the
stage's ``addcmul_`` calls update).
"""

from __future__ import annotations

import functools
from typing import Callable

import torch


def stage_geometry(m: int, n: int, s: int, p: int = 1, q: int = 1):
    """Coarse row range, coarse column range and flat slice of antidiagonal s.

    Follows gptq_2d.py:112-130: super-entry (ib, jb) starts at flat offset
    ib*p*n + jb*q; consecutive super-entries of one antidiagonal start
    max(p*n - q, (p-1)*n + q) apart.
    """
    lo = max(0, s - n // q + 1)
    hi = min(s + 1, m // p)
    step = max(p * n - q, (p - 1) * n + q)
    start = lo * p * n + (s - lo) * q
    return slice(lo, hi), slice(s - hi + 1, s - lo + 1), slice(start, start + (hi - lo) * step, step)


def select_super_entries(flat: torch.Tensor, sl: slice, n: int, p: int, q: int) -> torch.Tensor:
    """View ``[..., m*n]`` as the ``[..., d, p, q]`` super-entries of one antidiagonal (gptq_2d.py:133-144)."""
    window = (p - 1) * n + q
    return flat[..., sl.start:sl.stop].unfold(-1, window, sl.step).unfold(-1, q, n)


def check_inputs(x, l, u, inplace, p=1, q=1):
    """The reference's input contract (gptq_2d.py:65-84); returns m, n, batch shape."""
    assert x.dim() >= 2 and l.dim() >= 2 and u.dim() >= 2, "X, L, and U must have at least two dimensions"
    m, n = x.shape[-2:]
    assert l.shape[-2:] == (m, m) and u.shape[-2:] == (n, n), "expected X=[...,m,n], L=[...,m,m], and U=[...,n,n]"
    assert p > 0 and q > 0 and m % p == 0 and n % q == 0, "the super-entry shape must divide the matrix shape"
    assert x.dtype in (torch.float32, torch.float64) and x.dtype == l.dtype == u.dtype
    assert x.device == l.device == u.device
    batch = torch.broadcast_shapes(x.shape[:-2], l.shape[:-2], u.shape[:-2])
    assert not inplace or (x.is_contiguous() and x.shape[:-2] == batch)
    return m, n, batch


def _output(x, l, u, inplace, p=1, q=1):
    m, n, batch = check_inputs(x, l, u, inplace, p, q)
    y = x if inplace else x.expand(*batch, m, n).clone(memory_format=torch.contiguous_format)
    return y, m, n, batch


def unit_triangular(a: torch.Tensor, upper: bool, size: int = 1) -> torch.Tensor:
    """Zero the unused triangle and set the size x size diagonal blocks to identity (gptq_2d.py:103-109)."""
    a = a.triu() if upper else a.tril()
    k = a.shape[-1]
    blk = torch.arange(k) // size
    same = blk[:, None] == blk[None, :]
    eye = torch.eye(k, dtype=a.dtype)
    return torch.where(same, eye, a)


def _call_quantizer(zbuf, y_flat, selection, quantizer, inputs):
    ysel = selection(y_flat) if callable(selection) else y_flat[..., selection]
    z = zbuf[: ysel.numel()].view(ysel.shape)
    quantizer(y_flat, selection, *inputs, out=z)
    return ysel, z


def _round(y_flat, selection, *, out):
    sel = selection(y_flat) if callable(selection) else y_flat[..., selection]
    torch.round(sel, out=out)


class TorchSweepState:
    """The loop of the reference's ``gptq_2d_torch`` (gptq_2d.py:1197-1236), one stage at a time.

    ``run_stage(s)`` is the body of the loop of gptq_2d.py:1217-1235 for stage s; ``gptq_2d_torch``
    below runs it over every stage, so this class is the only copy of that body.  The CPU baseline
    times a sample of stages on full-size tensors and weights them by ``stage_work`` (a stage's
    cost depends only on the shapes).
    """

    def __init__(self, x, l, u, quantizer: Callable = _round, quantizer_inputs=(), inplace=False):
        self.y, self.m, self.n, batch = _output(x, l, u, inplace)
        self.stages = self.m + self.n - 1
        self.c = torch.zeros_like(self.y)
        self.yf, self.cf = self.y.flatten(-2), self.c.flatten(-2)
        self.lf = unit_triangular(l, upper=False).flip(-1)
        self.uf = unit_triangular(u, upper=True).flip(-2)
        self.zbuf = self.y.new_empty(batch.numel() * min(self.m, self.n))
        self.quantizer, self.inputs = quantizer, quantizer_inputs

    @torch.no_grad()
    def run_stage(self, s: int) -> None:
        m, n, y, c = self.m, self.n, self.y, self.c
        isl, jsl, asl = stage_geometry(m, n, s)
        ysel, z = _call_quantizer(self.zbuf, self.yf, asl, self.quantizer, self.inputs)
        e = z - ysel
        lcols = self.lf[..., isl.start:, m - isl.stop:m - isl.start]
        erow = e.flip(-1)[..., None, :]
        c[..., isl.start:, jsl].addcmul_(lcols, erow)
        y[..., isl.start:, jsl].addcmul_(lcols, erow)
        urows = self.uf[..., n - jsl.stop:n - jsl.start, jsl.start:]
        y[..., isl, jsl.start:].addcmul_(self.cf[..., asl, None], urows)
        self.yf[..., asl] = z


@torch.no_grad()
def gptq_2d_torch(x, l, u, *, quantizer: Callable = _round, inplace=False, quantizer_inputs=()):
    """Algorithm 3 with three ``addcmul_`` per stage, same operation order as gptq_2d.py:1197-1236."""
    st = TorchSweepState(x, l, u, quantizer=quantizer, quantizer_inputs=quantizer_inputs, inplace=inplace)
    if st.y.numel() == 0:
        return st.y
    for s in range(st.stages):
        st.run_stage(s)
    return st.y


def stage_work(m: int, n: int, s: int) -> int:
    """Entries the three ``addcmul_`` of stage s update: 2 (m - i_lo) d + d (n - j_lo), d = |I_s|."""
    isl, jsl, _ = stage_geometry(m, n, s)
    d = isl.stop - isl.start
    return 2 * (m - isl.start) * d + d * (n - jsl.start)


@torch.no_grad()
def gptq_2d_super_entry_torch(x, l, u, *, quantizer: Callable = None, super_entry_shape=(1, 1), inplace=False,
                              quantizer_inputs=()):
    """Super-entry Algorithm 3, same operation order as gptq_2d.py:1239-1292."""
    p, q = super_entry_shape
    if quantizer is None:
        quantizer = _round
    y, m, n, batch = _output(x, l, u, inplace, p, q)
    if y.numel() == 0:
        return y
    mb, nb = m // p, n // q
    B = batch.numel()
    c = torch.zeros_like(y)
    yf, cf = y.flatten(-2), c.flatten(-2)
    lb = unit_triangular(l, upper=False, size=p).unflatten(-1, (mb, p)).flip(-2).movedim(-2, -3).contiguous()
    ub = unit_triangular(u, upper=True, size=q).unflatten(-2, (nb, q)).flip(-3).contiguous()
    zbuf = y.new_empty(B * min(mb, nb) * p * q)
    for s in range(mb + nb - 1):
        isl, jsl, asl = stage_geometry(m, n, s, p, q)
        sel = functools.partial(select_super_entries, sl=asl, n=n, p=p, q=q)
        ysel, z = _call_quantizer(zbuf, yf, sel, quantizer, quantizer_inputs)
        e = z - ysel
        upd = lb[..., mb - isl.stop:mb - isl.start, isl.start * p:, :] @ e.flip(-3)
        c.unflatten(-1, (nb, q))[..., isl.start * p:, jsl, :] += upd.transpose(-3, -2)
        y.unflatten(-1, (nb, q))[..., isl.start * p:, jsl, :] += upd.transpose(-3, -2)
        y.unflatten(-2, (mb, p))[..., isl, :, jsl.start * q:] += sel(cf) @ ub[..., nb - jsl.stop:nb - jsl.start, :, jsl.start * q:]
        ysel.copy_(z)
    return y


@torch.no_grad()
def direct_2d(x, l, u, *, quantizer: Callable = _round, inplace=False, quantizer_inputs=()):
    """Algorithm 2 (quartic dense updates), gptq_2d.py:1122-1151."""
    y, m, n, batch = _output(x, l, u, inplace)
    if y.numel() == 0:
        return y
    B = batch.numel()
    yf = y.flatten(-2)
    lt = unit_triangular(l, upper=False)
    uf = unit_triangular(u, upper=True).flip(-2)
    zbuf = y.new_empty(B * min(m, n))
    for s in range(m + n - 1):
        isl, jsl, asl = stage_geometry(m, n, s)
        ysel, z = _call_quantizer(zbuf, yf, asl, quantizer, quantizer_inputs)
        e = z - ysel
        y[..., isl.start:, jsl.start:] += (lt[..., isl.start:, isl] * e[..., None, :]) @ uf[..., n - jsl.stop:n - jsl.start, jsl.start:]
        yf[..., asl] = z
    return y


@torch.no_grad()
def direct_2d_super_entry(x, l, u, *, quantizer: Callable = None, super_entry_shape=(1, 1), inplace=False,
                          quantizer_inputs=()):
    """Super-entry Algorithm 2, gptq_2d.py:1154-1193."""
    p, q = super_entry_shape
    if quantizer is None:
        quantizer = _round
    y, m, n, batch = _output(x, l, u, inplace, p, q)
    if y.numel() == 0:
        return y
    mb, nb = m // p, n // q
    B = batch.numel()
    yf = y.flatten(-2)
    lt = unit_triangular(l, upper=False, size=p)
    ub = unit_triangular(u, upper=True, size=q).unflatten(-2, (nb, q)).flip(-3)
    zbuf = y.new_empty(B * min(mb, nb) * p * q)
    for s in range(mb + nb - 1):
        isl, jsl, asl = stage_geometry(m, n, s, p, q)
        sel = functools.partial(select_super_entries, sl=asl, n=n, p=p, q=q)
        ysel, z = _call_quantizer(zbuf, yf, sel, quantizer, quantizer_inputs)
        i0, j0 = isl.start * p, jsl.start * q
        right = ((z - ysel) @ ub[..., nb - jsl.stop:nb - jsl.start, :, j0:]).flatten(-3, -2)
        y[..., i0:, j0:] += lt[..., i0:, i0:isl.stop * p] @ right
        ysel.copy_(z)
    return y
