"""GPTQ-2D on MI355X: drop-in for the reference's ``gptq_2d.py`` entry points.

GPTQ-2D rounds X [..., m, n] under the two-sided objective tr((Z-X)^T G (Z-X) H) given the
unit triangular feedback factors L (G^{-1} = L Lambda L^T) and U (H^{-1} = U^T Lambda U).  Stages
are antidiagonals s = i + j; each rounds its entries at once and feeds the errors forward.

Two engines sit behind the same API:

* the fused tile sweep (built-in quantizers: ``round_quantizer``, the affine plug-ins,
  ``teacher_forced_quantizer``, and for 1 x 32 super-entries also the abs-max plug-ins; plain entries
  or 1 x 32 super-entries): one C-ABI call runs the whole sweep as a stream of HIP kernels --
  LDS-resident tile sweeps with the rounding fused in, and masked band GEMMs for the feedback
  between tiles (``csrc/sweep_tiles.hip``, ``csrc/flush_mfma.hip``, ``csrc/flush.hip``);
* the plug-in path (any Python quantizer, any super-entry shape): the host calls the quantizer
  once per antidiagonal and HIP kernels push the errors inside the current block and flush whole
  blocks, with the reference's two-level blocking (``csrc/sweep_generic.hip``).

Both give the reference's rounding in exact arithmetic; fp32 results differ from it only by
floating-point summation order.  ``capture_gptq_2d`` records either engine as a hipGraph
(``torch.cuda.graph`` on ROCm).  ``gptq_2d_torch``, ``direct_2d`` and their super-entry variants
are the reference's device-agnostic PyTorch formulations.

Reference: IST-DASLab/GPTQ-2D gptq_2d.py (entry points :1378-1564, PyTorch sweeps :1122-1292).
"""

from __future__ import annotations

import functools
import math
from typing import Callable

import torch

import _hip
import quantizer_int as _qi
from quantizer_int import round_quantizer, round_quantizer_super_entry

# Coarse stages (tile antidiagonals) per outer block of the fused sweep when the caller asks for
# the default outer block; tiles are TILE x TILE entries.
TILE = 32


# ------------------------------------------------------------------------------------------------ contract

class KroneckerU:
    """U = outer (x) inner given by its two factors ([k, k] each, one dtype and device), for the sweeps' ``u``
    argument in place of the (k_outer k_inner)^2 entries of the explicit product (Algorithm 4's per-mode form,
    gptq_2d_reference.py:270-294, whose factors the reference never multiplies out).  Entries are read as
    torch.kron(outer, inner) forms them -- every entry of both factors, the product's zeros and diagonal
    included -- so results equal those with ``dense()`` bit for bit.  The fused fp32 engine reads the factors
    directly (one matrix, no batch; inner size a multiple of 16, sizes multiples of 4); every other path forms
    ``dense()`` first."""

    def __init__(self, outer: torch.Tensor, inner: torch.Tensor):
        assert outer.dim() == 2 and inner.dim() == 2, "the Kronecker factors must be matrices"
        assert outer.size(0) == outer.size(1) and inner.size(0) == inner.size(1), "the Kronecker factors must be square"
        assert outer.dtype == inner.dtype and outer.device == inner.device, (
            "the Kronecker factors must share dtype and device")
        self.outer, self.inner = outer, inner

    @property
    def shape(self) -> torch.Size:
        k = self.outer.size(0) * self.inner.size(0)
        return torch.Size((k, k))

    @property
    def dtype(self) -> torch.dtype:
        return self.outer.dtype

    @property
    def device(self) -> torch.device:
        return self.outer.device

    def dim(self) -> int:
        return 2

    def numel(self) -> int:
        return self.shape.numel()

    def contiguous(self) -> "KroneckerU":
        return KroneckerU(self.outer.contiguous(), self.inner.contiguous())

    def dense(self) -> torch.Tensor:
        return torch.kron(self.outer, self.inner)


def _validate_inputs(x, l, u, inplace, require_cuda=False, super_entry_shape=(1, 1)):
    """The shared input contract (gptq_2d.py:65-84); returns m, n and the broadcast batch shape."""
    assert x.dim() >= 2 and l.dim() >= 2 and u.dim() >= 2, "X, L, and U must have at least two dimensions"
    m, n = x.shape[-2:]
    assert l.shape[-2:] == (m, m) and u.shape[-2:] == (n, n), "expected X=[...,m,n], L=[...,m,m], and U=[...,n,n]"
    p, q = super_entry_shape
    assert p > 0 and q > 0 and m % p == 0 and n % q == 0, "the super-entry shape must divide the matrix shape"
    assert x.dtype in (torch.float32, torch.float64) and x.dtype == l.dtype == u.dtype, (
        "X, L, and U must share dtype float32 or float64"
    )
    assert x.device == l.device == u.device, "X, L, and U must be on the same device"
    assert not require_cuda or x.is_cuda, "X, L, and U must be GPU tensors"
    batch_shape = torch.broadcast_shapes(x.shape[:-2], l.shape[:-2], u.shape[:-2])
    assert not inplace or (x.is_contiguous() and x.shape[:-2] == batch_shape), (
        "inplace=True requires contiguous X with the exact broadcast batch shape"
    )
    return m, n, batch_shape


def _dense_u(u):
    """U as a tensor: a KroneckerU's product (the PyTorch variants multiply U's entries directly)."""
    return u.dense() if isinstance(u, KroneckerU) else u


def _prepare_output(x, l, u, inplace, require_cuda=False, super_entry_shape=(1, 1)):
    """Validate and create the work matrix Y (a clone, or x itself in place) (gptq_2d.py:87-100)."""
    m, n, batch_shape = _validate_inputs(x, l, u, inplace, require_cuda, super_entry_shape)
    y = x if inplace else x.expand(*batch_shape, m, n).clone(memory_format=torch.contiguous_format)
    return y, m, n, batch_shape


def _antidiagonal_slices(*, m, n, s, super_entry_shape=(1, 1)):
    """Coarse row slice, coarse column slice and flat slice of stage s (gptq_2d.py:112-130).

    Super-entry (ib, jb) starts at flat offset ib*p*n + jb*q; along a coarse antidiagonal the starts
    are max(p*n - q, (p-1)*n + q) apart.
    """
    p, q = super_entry_shape
    lo, hi = max(0, s - n // q + 1), min(s + 1, m // p)
    step = max(p * n - q, (p - 1) * n + q)
    start = lo * p * n + (s - lo) * q
    return slice(lo, hi), slice(s - hi + 1, s - lo + 1), slice(start, start + (hi - lo) * step, step)


def _super_entries(x_flat, antidiagonal_slice, n, super_entry_shape):
    """View ``[..., m*n]`` as the ``[..., d, p, q]`` super-entries of one antidiagonal (gptq_2d.py:133-144)."""
    p, q = super_entry_shape
    window = x_flat[..., antidiagonal_slice.start:antidiagonal_slice.stop]
    return window.unfold(-1, (p - 1) * n + q, antidiagonal_slice.step).unfold(-1, q, n)


def _quantize_antidiagonal(z_scratch, y_flat, selection, quantizer, quantizer_inputs):
    """Call the plug-in on the stage; ``out`` is a contiguous view at the head of ``z_scratch``."""
    y_sel = selection(y_flat) if callable(selection) else y_flat[..., selection]
    z = z_scratch[:y_sel.numel()].view(y_sel.shape)
    quantizer(y_flat, selection, *quantizer_inputs, out=z)
    return y_sel, z


def _unit_triangular(x, upper, size=1):
    """Zero the unused triangle and set the size x size diagonal blocks to identity (gptq_2d.py:103-109)."""
    x = x.triu() if upper else x.tril()
    blocks = x.unflatten(-2, (-1, size)).unflatten(-1, (-1, size)).diagonal(dim1=-4, dim2=-2)
    blocks.copy_(torch.eye(size, dtype=x.dtype, device=x.device)[:, :, None])
    return x


# ------------------------------------------------------------------------------------------------ fused engine

def _unwrap(quantizer):
    """(function, keyword arguments) of a plain function or a keyword-only functools.partial."""
    if isinstance(quantizer, functools.partial) and not quantizer.args:
        return quantizer.func, dict(quantizer.keywords)
    return quantizer, {}


def _matrix_input(t, y, batch_shape):
    """A quantizer input usable by the fused kernels: [*, m, n], contiguous, same dtype/device, broadcastable."""
    if not isinstance(t, torch.Tensor) or t.dim() < 2 or t.shape[-2:] != y.shape[-2:]:
        return None
    if t.dtype != y.dtype or t.device != y.device:
        return None
    try:
        if torch.broadcast_shapes(t.shape[:-2], batch_shape) != batch_shape:
            return None
    except RuntimeError:
        return None
    return t.contiguous()


def _fused_spec(quantizer, quantizer_inputs, y, batch_shape, rows=False):
    """Recognise a built-in quantizer the tile sweep can fuse; None for any other plug-in.  ``rows``: super-entries
    of one tile row (1 x TILE), where the abs-max quantizer of a super-entry row is fused too."""
    fn, kw = _unwrap(quantizer)
    if fn in (round_quantizer, round_quantizer_super_entry) and not kw and not quantizer_inputs:
        return dict(kind=0, qa=None, qb=None, qmin=0.0, qmax=0.0, ypre=None)
    if rows and fn in (_qi.int_abs_max_quantizer_hip, _qi.int_abs_max_quantizer_torch) and set(kw) == {
            "qmin", "qmax", "dtype"} and len(quantizer_inputs) <= 1:
        if kw["dtype"] not in _qi._SCALE_DTYPES or not float(kw["qmin"]) < float(kw["qmax"]):
            return None
        sout = quantizer_inputs[0] if quantizer_inputs else None
        if sout is not None and (not isinstance(sout, torch.Tensor) or sout.shape != y.shape or
                                 not sout.is_contiguous() or sout.dtype != y.dtype or sout.device != y.device):
            return None
        return dict(kind=3, qa=None, qb=None, qmin=float(kw["qmin"]), qmax=float(kw["qmax"]), ypre=None,
                    dtype16=_qi._SCALE_DTYPES[kw["dtype"]], sout=sout)
    if fn in (_qi.affine_quantizer_hip, _qi.affine_quantizer_torch, _qi.affine_quantizer_super_entry_hip,
              _qi.affine_quantizer_super_entry_torch) and set(kw) <= {"qmin", "qmax"}:
        if len(quantizer_inputs) != 2:
            return None
        scale, zp = (_matrix_input(t, y, batch_shape) for t in quantizer_inputs)
        if scale is None or zp is None:
            return None
        qmin, qmax = float(kw.get("qmin", -math.inf)), float(kw.get("qmax", math.inf))
        assert qmin < qmax, "expected qmin < qmax"
        return dict(kind=1, qa=scale, qb=zp, qmin=qmin, qmax=qmax, ypre=None)
    if fn is _qi.teacher_forced_quantizer and not kw and len(quantizer_inputs) == 2:
        values = _matrix_input(quantizer_inputs[0], y, batch_shape)
        ypre = quantizer_inputs[1]
        if values is None or not isinstance(ypre, torch.Tensor) or ypre.shape != y.shape or not ypre.is_contiguous():
            return None
        if ypre.dtype != y.dtype or ypre.device != y.device:
            return None
        return dict(kind=2, qa=values, qb=None, qmin=0.0, qmax=0.0, ypre=ypre)
    return None


def _run_fused_kron(y, l, u, m, n, spec, outer_block_size, p=1, q=1):
    """The fused sweep of one matrix with U given by its Kronecker factors (gptq2d_sweep_fused_kron_f32)."""
    c = torch.empty_like(y)  # zeroed by the library
    e = torch.empty_like(y)
    qa, qb = spec["qa"], spec["qb"]
    _hip.call_untyped(
        "sweep_fused_kron_f32", _hip.ptr(y), _hip.ptr(c), _hip.ptr(e), _hip.ptr(l), _hip.ptr(u.outer),
        _hip.ptr(u.inner), m, u.outer.size(0), u.inner.size(0), p, q, spec["kind"], _hip.ptr(qa), _hip.ptr(qb),
        spec["qmin"], spec["qmax"], spec.get("dtype16", 0), _hip.ptr(spec["ypre"]), _hip.ptr(spec.get("sout")),
        _outer_tiles(outer_block_size), 0, -1, _hip.stream(y.device),
    )


def _kron_fusable(y, l, u, batch_shape, spec):
    """Whether the fused engine reads U = u.outer (x) u.inner from its factors (else the product is formed)."""
    if spec is None or len(batch_shape) != 0 or y.dtype != torch.float32 or l.dim() != 2:
        return False
    m, n = y.shape
    tensors = [y, l, u.inner] + [t for t in (spec["qa"], spec["qb"]) if t is not None]
    return (u.inner.size(0) % 16 == 0 and m % 4 == 0 and n % 4 == 0 and m < 1 << 20 and n < 1 << 20 and
            all(t.data_ptr() % 16 == 0 for t in tensors) and
            all(t.shape == y.shape for t in (spec["qa"], spec["qb"]) if t is not None))


def _outer_tiles(outer_block_size):
    return max(1, int(outer_block_size) // TILE) if outer_block_size and outer_block_size > 0 else 1


def _run_fused(y, l, u, m, n, batch_shape, spec, outer_block_size, p=1, q=1):
    B = batch_shape.numel()
    yb = y.reshape(B, m, n)
    c = torch.empty_like(yb)  # zeroed by the library
    e = torch.empty_like(yb)
    bshape = _hip.i64_array(batch_shape)
    nd = len(batch_shape)
    qa, qb = spec["qa"], spec["qb"]
    _hip.call(
        "sweep_fused_se", y.dtype, _hip.ptr(yb), _hip.ptr(c), _hip.ptr(e), _hip.ptr(l), _hip.ptr(u), m, n, p, q, nd,
        bshape, _hip.batch_strides(l, batch_shape), _hip.batch_strides(u, batch_shape), spec["kind"], _hip.ptr(qa),
        _hip.batch_strides(qa, batch_shape) if qa is not None else None, _hip.ptr(qb),
        _hip.batch_strides(qb, batch_shape) if qb is not None else None, spec["qmin"], spec["qmax"],
        spec.get("dtype16", 0), _hip.ptr(spec["ypre"]), _hip.ptr(spec.get("sout")), _outer_tiles(outer_block_size), 0,
        -1, _hip.stream(y.device),
    )


# ------------------------------------------------------------------------------------------------ plug-in engine

def _run_blocked(y, l, u, m, n, batch_shape, p, q, super_entry, quantizer, quantizer_inputs, inner, outer):
    """Two-level blocked sweep with a per-antidiagonal Python quantizer (gptq_2d.py:1295-1375)."""
    B = batch_shape.numel()
    lanes = min(m // p, n // q)
    y_flat = y.flatten(start_dim=-2)
    yb = y.reshape(B, m, n)
    dt, dev = y.dtype, y.device
    c = torch.empty_like(yb)
    _hip.call("fill", dt, _hip.ptr(c), 0.0, c.numel(), _hip.stream(dev))
    e = torch.empty_like(yb)
    z_scratch = y.new_empty(B * lanes * p * q)
    old = y.new_empty(2, B * lanes)
    stages = m // p + n // q - 1
    inner = inner if 0 < inner <= stages else stages
    outer = outer if inner < outer < stages else inner
    nd = len(batch_shape)
    bshape = _hip.i64_array(batch_shape)
    lstr, ustr = _hip.batch_strides(l, batch_shape), _hip.batch_strides(u, batch_shape)
    plain = p == q == 1

    def flush(s0, s1, s_end):
        _hip.call("flush", dt, _hip.ptr(yb), _hip.ptr(c), _hip.ptr(e), _hip.ptr(l), _hip.ptr(u), m, n, p, q, s0, s1,
                  s_end, nd, bshape, lstr, ustr, _hip.stream(dev))

    for outer_start in range(0, stages, outer):
        outer_stop = min(outer_start + outer, stages)
        for s0 in range(outer_start, outer_stop, inner):
            s1 = min(s0 + inner, outer_stop)
            if plain:  # Y on the block's first antidiagonal is final after the flushes
                _hip.call("gather_antidiagonal", dt, _hip.ptr(yb), _hip.ptr(old[s0 % 2]), B, m, n, s0,
                          _hip.stream(dev))
            for s in range(s0, s1):
                sl = _antidiagonal_slices(m=m, n=n, s=s, super_entry_shape=(p, q))[2]
                selection = functools.partial(_super_entries, antidiagonal_slice=sl, n=n,
                                              super_entry_shape=(p, q)) if super_entry else sl
                _, z = _quantize_antidiagonal(z_scratch, y_flat, selection, quantizer, quantizer_inputs)
                if plain:
                    _hip.call("push_plain", dt, _hip.ptr(yb), _hip.ptr(c), _hip.ptr(e), _hip.ptr(z),
                              _hip.ptr(old[s % 2]), _hip.ptr(old[(s + 1) % 2]), _hip.ptr(l), _hip.ptr(u), m, n, s,
                              s1, nd, bshape, lstr, ustr, _hip.stream(dev))
                else:
                    _hip.call("push_down_se", dt, _hip.ptr(yb), _hip.ptr(c), _hip.ptr(e), _hip.ptr(z), _hip.ptr(l),
                              m, n, p, q, s, s1, nd, bshape, lstr, _hip.stream(dev))
                    _hip.call("push_right_se", dt, _hip.ptr(yb), _hip.ptr(c), _hip.ptr(z), _hip.ptr(u), m, n, p, q,
                              s, s1, nd, bshape, ustr, _hip.stream(dev))
            if plain and s1 < stages:
                _hip.call("add_own_errors", dt, _hip.ptr(c), _hip.ptr(e), B, m, n, s0, s1, _hip.stream(dev))
            if s1 < outer_stop:
                flush(s0, s1, outer_stop)
        if outer_stop < stages:
            flush(outer_start, outer_stop, stages)


def _sweep(x, l, u, quantizer, super_entry_shape, inner_block_size, outer_block_size, inplace, quantizer_inputs,
           fused):
    p, q = super_entry_shape or (1, 1)
    y, m, n, batch_shape = _prepare_output(x, l, u, inplace, require_cuda=True, super_entry_shape=(p, q))
    if y.numel() == 0:
        return y
    l, u = l.contiguous(), u.contiguous()
    spec = None
    if fused is not False and (p, q) in ((1, 1), (1, TILE)):
        spec = _fused_spec(quantizer, quantizer_inputs, y, batch_shape, rows=(p, q) == (1, TILE))
    assert not (fused is True and spec is None), (
        "fused=True needs a built-in quantizer and plain entries or 1 x 32 super-entries")
    kron = isinstance(u, KroneckerU)
    if kron and not _kron_fusable(y, l, u, batch_shape, spec):
        u, kron = u.dense(), False
    with torch.cuda.device(x.device):
        if kron:
            _run_fused_kron(y, l, u, m, n, spec, outer_block_size, p, q)
        elif spec is not None:
            _run_fused(y, l, u, m, n, batch_shape, spec, outer_block_size, p, q)
        else:
            _run_blocked(y, l, u, m, n, batch_shape, p, q, super_entry_shape is not None, quantizer,
                         quantizer_inputs, inner_block_size, outer_block_size)
    return y


# ------------------------------------------------------------------------------------------------ public API

@torch.no_grad()
def gptq_2d(x, l, u, *, quantizer: Callable = round_quantizer, inner_block_size: int = 32,
            outer_block_size: int = 512, inplace: bool = False, quantizer_inputs: tuple = (),
            fused: bool | None = None) -> torch.Tensor:
    """Blocked GPTQ-2D of x [..., m, n] with unit lower L [..., m, m] and unit upper U [..., n, n]
    (gptq_2d.py:1378-1418).

    Leading dimensions broadcast; L is read only strictly below its diagonal and U strictly above.
    The quantizer receives live Y flattened to [*batch, m*n], a slice of the current antidiagonal,
    ``quantizer_inputs`` and ``out``.  With ``inplace`` x must be contiguous with the full batch shape.
    Built-in per-entry quantizers run fused in the tile sweep (``fused=None`` decides, ``False``
    forces the per-antidiagonal plug-in path); block sizes count antidiagonals as in the reference,
    and the fused sweep uses ``outer_block_size // 32`` tile stages per outer block.
    """
    return _sweep(x, l, u, quantizer, None, inner_block_size, outer_block_size, inplace, quantizer_inputs, fused)


@torch.no_grad()
def gptq_2d_super_entry(x, l, u, *, quantizer: Callable = round_quantizer_super_entry, super_entry_shape=(1, 1),
                        inner_block_size: int = 8, outer_block_size: int = 64, inplace: bool = False,
                        quantizer_inputs: tuple = (), fused: bool | None = None) -> torch.Tensor:
    """Blocked GPTQ-2D over p x q super-entries rounded jointly (gptq_2d.py:1421-1447).

    The quantizer receives a ``select`` callable viewing any [..., m*n] tensor as the [..., d, p, q]
    super-entries of the current coarse antidiagonal.  L and U have implicit identity p x p and
    q x q diagonal blocks.  1 x 1 super-entries with a built-in per-entry quantizer, and 1 x 32
    super-entries with a built-in per-entry or abs-max quantizer, run fused (``outer_block_size``
    then counts entry antidiagonals of 32-wide tiles, as for ``gptq_2d``).
    """
    return _sweep(x, l, u, quantizer, tuple(super_entry_shape), inner_block_size, outer_block_size, inplace,
                  quantizer_inputs, fused)


@torch.no_grad()
def capture_gptq_2d(x, l, u, *, quantizer: Callable | None = None, super_entry_shape=None,
                    inner_block_size: int | None = None, outer_block_size: int | None = None, inplace: bool = False,
                    quantizer_inputs: tuple = ()) -> Callable[..., torch.Tensor]:
    """Capture GPTQ-2D as a hipGraph and return ``replay(x, l, u, *quantizer_inputs)`` (gptq_2d.py:1450-1564).

    Replay inputs must match the examples' shapes, dtypes and devices; they are copied into private
    static buffers.  Out of place a replay returns a clone; in place it copies into x and returns it.
    One replay callable owns its static buffers and must be used sequentially.
    """
    _validate_inputs(x, l, u, inplace, require_cuda=True, super_entry_shape=super_entry_shape or (1, 1))
    assert all(t.is_cuda and t.device == x.device for t in quantizer_inputs), (
        "quantizer inputs must be GPU tensors on the same device as X"
    )
    options = dict(quantizer=quantizer, super_entry_shape=super_entry_shape, inner_block_size=inner_block_size,
                   outer_block_size=outer_block_size)
    run = functools.partial(gptq_2d if super_entry_shape is None else gptq_2d_super_entry, inplace=inplace,
                            **{k: v for k, v in options.items() if v is not None})
    names = ("X", "L", "U", *(f"quantizer input {i}" for i in range(len(quantizer_inputs))))
    inputs = (x, l, u, *quantizer_inputs)
    # a KroneckerU is captured as its two factors (static copies of both; replays take a pair of the same sizes)
    factors = lambda t: (t.outer.shape, t.inner.shape) if isinstance(t, KroneckerU) else None
    expected = tuple((t.shape, t.dtype, t.device, factors(t)) for t in inputs)

    def validate_replay(*replay_inputs):
        assert len(replay_inputs) == len(expected), f"expected {len(expected) - 3} quantizer inputs"
        for name, t, (shape, dtype, device, fs) in zip(names, replay_inputs, expected):
            assert t.shape == shape, f"{name} shape must match its capture example"
            assert t.dtype == dtype, f"{name} dtype must match its capture example"
            assert t.device == device, f"{name} device must match its capture example"
            assert factors(t) == fs, f"{name} must be given as its capture example was (tensor or Kronecker pair)"
        if inplace:
            assert replay_inputs[0].is_contiguous(), "inplace=True requires contiguous X"

    if x.numel() == 0 or l.numel() == 0 or u.numel() == 0:
        run(x=x, l=l, u=u, quantizer_inputs=quantizer_inputs)

        @torch.no_grad()
        def replay_empty(x, l, u, *qi):
            validate_replay(x, l, u, *qi)
            return run(x=x, l=l, u=u, quantizer_inputs=qi)

        return replay_empty

    def static(t):
        if isinstance(t, KroneckerU):
            return KroneckerU(static(t.outer), static(t.inner))
        return t.detach().clone(memory_format=torch.contiguous_format)

    def refill(dst, src):
        if isinstance(dst, KroneckerU):
            dst.outer.copy_(src.outer)
            dst.inner.copy_(src.inner)
        else:
            dst.copy_(src)

    statics = tuple(static(t) for t in inputs)
    sx, sl, su = statics[:3]
    sq = statics[3:]
    with torch.cuda.device(x.device):
        side = torch.cuda.Stream(device=x.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                run(x=sx, l=sl, u=su, quantizer_inputs=sq)
            sx.copy_(x)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(cuda_graph=graph, stream=side):
            static_y = run(x=sx, l=sl, u=su, quantizer_inputs=sq)

    @torch.no_grad()
    def replay(x, l, u, *qi):
        validate_replay(x, l, u, *qi)
        sx.copy_(x)
        sl.copy_(l)
        refill(su, u)
        for s, t in zip(sq, qi):
            s.copy_(t)
        graph.replay()
        if inplace:
            x.copy_(static_y)
            return x
        return static_y.clone()

    return replay


# ------------------------------------------------------------------------------------------------ PyTorch variants

@torch.no_grad()
def gptq_2d_torch(x, l, u, *, quantizer: Callable = round_quantizer, inplace: bool = False,
                  quantizer_inputs: tuple = ()) -> torch.Tensor:
    """Algorithm 3 in PyTorch on any device: three ``addcmul_`` per stage (gptq_2d.py:1196-1236)."""
    u = _dense_u(u)
    y, m, n, batch_shape = _prepare_output(x, l, u, inplace)
    if y.numel() == 0:
        return y
    c = y.new_zeros(y.shape)
    y_flat, c_flat = y.flatten(start_dim=-2), c.flatten(start_dim=-2)
    l_rev = _unit_triangular(l, upper=False).flip(dims=(-1,))
    u_rev = _unit_triangular(u, upper=True).flip(dims=(-2,))
    z_scratch = y.new_empty(batch_shape.numel() * min(m, n))
    for s in range(m + n - 1):
        isl, jsl, asl = _antidiagonal_slices(m=m, n=n, s=s)
        y_sel, z = _quantize_antidiagonal(z_scratch, y_flat, asl, quantizer, quantizer_inputs)
        e = z - y_sel
        cols = l_rev[..., isl.start:, m - isl.stop:m - isl.start]
        e_row = e.flip(dims=(-1,))[..., None, :]
        c[..., isl.start:, jsl].addcmul_(cols, e_row)
        y[..., isl.start:, jsl].addcmul_(cols, e_row)
        rows = u_rev[..., n - jsl.stop:n - jsl.start, jsl.start:]
        y[..., isl, jsl.start:].addcmul_(c_flat[..., asl, None], rows)
        y_flat[..., asl] = z
    return y


@torch.no_grad()
def gptq_2d_super_entry_torch(x, l, u, *, quantizer: Callable = round_quantizer_super_entry, super_entry_shape=(1, 1),
                              inplace: bool = False, quantizer_inputs: tuple = ()) -> torch.Tensor:
    """Super-entry Algorithm 3 in PyTorch on any device (gptq_2d.py:1239-1292)."""
    u = _dense_u(u)
    p, q = super_entry_shape
    y, m, n, batch_shape = _prepare_output(x, l, u, inplace, super_entry_shape=(p, q))
    if y.numel() == 0:
        return y
    mb, nb = m // p, n // q
    c = y.new_zeros(y.shape)
    y_flat, c_flat = y.flatten(start_dim=-2), c.flatten(start_dim=-2)
    l_bands = _unit_triangular(l, upper=False, size=p).unflatten(-1, (mb, p)).flip(dims=(-2,)).movedim(-2, -3)
    l_bands = l_bands.contiguous()
    u_bands = _unit_triangular(u, upper=True, size=q).unflatten(-2, (nb, q)).flip(dims=(-3,)).contiguous()
    z_scratch = y.new_empty(batch_shape.numel() * min(mb, nb) * p * q)
    for s in range(mb + nb - 1):
        isl, jsl, asl = _antidiagonal_slices(m=m, n=n, s=s, super_entry_shape=(p, q))
        select = functools.partial(_super_entries, antidiagonal_slice=asl, n=n, super_entry_shape=(p, q))
        y_sel, z = _quantize_antidiagonal(z_scratch, y_flat, select, quantizer, quantizer_inputs)
        e = z - y_sel
        upd = l_bands[..., mb - isl.stop:mb - isl.start, isl.start * p:, :] @ e.flip(dims=(-3,))
        c.unflatten(-1, (nb, q))[..., isl.start * p:, jsl, :] += upd.transpose(-3, -2)
        y.unflatten(-1, (nb, q))[..., isl.start * p:, jsl, :] += upd.transpose(-3, -2)
        y.unflatten(-2, (mb, p))[..., isl, :, jsl.start * q:] += (
            select(c_flat) @ u_bands[..., nb - jsl.stop:nb - jsl.start, :, jsl.start * q:]
        )
        y_sel.copy_(z)
    return y


@torch.no_grad()
def direct_2d(x, l, u, *, quantizer: Callable = round_quantizer, inplace: bool = False,
              quantizer_inputs: tuple = ()) -> torch.Tensor:
    """Direct quartic Algorithm 2 in PyTorch (gptq_2d.py:1122-1151)."""
    u = _dense_u(u)
    y, m, n, batch_shape = _prepare_output(x, l, u, inplace)
    if y.numel() == 0:
        return y
    y_flat = y.flatten(start_dim=-2)
    lt = _unit_triangular(l, upper=False)
    u_rev = _unit_triangular(u, upper=True).flip(dims=(-2,))
    z_scratch = y.new_empty(batch_shape.numel() * min(m, n))
    for s in range(m + n - 1):
        isl, jsl, asl = _antidiagonal_slices(m=m, n=n, s=s)
        y_sel, z = _quantize_antidiagonal(z_scratch, y_flat, asl, quantizer, quantizer_inputs)
        e = z - y_sel
        y[..., isl.start:, jsl.start:] += (lt[..., isl.start:, isl] * e[..., None, :]) @ (
            u_rev[..., n - jsl.stop:n - jsl.start, jsl.start:])
        y_flat[..., asl] = z
    return y


@torch.no_grad()
def direct_2d_super_entry(x, l, u, *, quantizer: Callable = round_quantizer_super_entry, super_entry_shape=(1, 1),
                          inplace: bool = False, quantizer_inputs: tuple = ()) -> torch.Tensor:
    """Direct quartic Algorithm 2 over super-entries in PyTorch (gptq_2d.py:1154-1193)."""
    u = _dense_u(u)
    p, q = super_entry_shape
    y, m, n, batch_shape = _prepare_output(x, l, u, inplace, super_entry_shape=(p, q))
    if y.numel() == 0:
        return y
    mb, nb = m // p, n // q
    y_flat = y.flatten(start_dim=-2)
    lt = _unit_triangular(l, upper=False, size=p)
    u_bands = _unit_triangular(u, upper=True, size=q).unflatten(-2, (nb, q)).flip(dims=(-3,))
    z_scratch = y.new_empty(batch_shape.numel() * min(mb, nb) * p * q)
    for s in range(mb + nb - 1):
        isl, jsl, asl = _antidiagonal_slices(m=m, n=n, s=s, super_entry_shape=(p, q))
        select = functools.partial(_super_entries, antidiagonal_slice=asl, n=n, super_entry_shape=(p, q))
        y_sel, z = _quantize_antidiagonal(z_scratch, y_flat, select, quantizer, quantizer_inputs)
        i0, j0 = isl.start * p, jsl.start * q
        right = ((z - y_sel) @ u_bands[..., nb - jsl.stop:nb - jsl.start, :, j0:]).flatten(start_dim=-3, end_dim=-2)
        y[..., i0:, j0:] += lt[..., i0:, i0:isl.stop * p] @ right
        y_sel.copy_(z)
    return y
