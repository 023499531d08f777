"""Packed output formats of a quantized layer, on the GPU.

The reference returns dequantized values only (gptq_2d.py:1378-1447); its trellis docstring notes that the
T*K-bit code of a sequence is recoverable (quantizer_trellis.py:11-16) and its search returns the states
(quantizer_trellis.py:121-143).  These functions turn a sweep's output into the codes a deployment stores
and back, each in one HIP launch (csrc/pack.hip):

* INT codes (affine quantizer, quantizer_int.py:63-83, and the abs-max quantizer, :120-134): code
  u = q - qmin of value z = (q - zp) * s in ceil(log2(qmax - qmin + 1)) bits, little-endian bit fields per
  row of the layer (4 bits: 8 codes per 32-bit word, low nibble first).  The scales of the abs-max
  quantizer are the per-entry map its ``scales`` input records during the sweep.
* Trellis streams (bitshift trellis, quantizer_trellis.py:82-143): per super-entry sequence, the top K*V
  bits of each state in order, MSB first -- exactly T*K bits with tail-biting -- from the per-entry state
  map the trellis quantizers' ``states`` input records; decoding reads state t as the L-bit window at bit
  t*K*V and writes table[state] * scale, the quantizer's values.

Words are returned as int32 tensors holding the uint32 bit patterns.
"""

from __future__ import annotations

import torch

import _hip


def int_code_bits(qmin: float, qmax: float) -> int:
    """Bits of a packed code for integer bounds qmin <= qmax (at most 16)."""
    bits = int(_hip.lib().gptq2d_int_code_bits(float(qmin), float(qmax)))
    if bits < 0:
        raise ValueError(f"packed INT codes need integer bounds qmin <= qmax spanning at most 2^16 codes, "
                         f"got [{qmin}, {qmax}]")
    return bits


def _operand(t, z, B, m, n):
    """t broadcast to z [*, m, n] as [B, m, n] with its (batch, row, column) element strides."""
    v = torch.as_tensor(t, dtype=z.dtype, device=z.device).expand(z.shape).reshape(B, m, n)
    return v, _hip.i64_array(v.stride())


def _check_bad(bad: torch.Tensor, what: str) -> None:
    count = int(bad.sum())
    if count:
        rows = torch.nonzero(bad).flatten()[:8].tolist()
        raise ValueError(f"{count} {what} (first rows {rows})")


@torch.no_grad()
def pack_int(z: torch.Tensor, scale, zero_point=None, *, qmin: float, qmax: float, check: bool = True,
             return_bad: bool = False):
    """Codes of z [*, m, n] (values of the affine quantizer with ``scale`` and ``zero_point``, each
    broadcastable to z) packed into int32 words [*, m, ceil(n * bits / 32)].  With ``check`` (a host
    synchronisation) a value that is not (q - zp) * s for an integer q in [qmin, qmax] raises; with
    ``return_bad`` the per-row count of such values [*, m] is returned too."""
    _hip.require_device(z)
    assert z.dim() >= 2 and z.dtype in (torch.float32, torch.float64), "z must be a float32/float64 [*, m, n] tensor"
    bits = int_code_bits(qmin, qmax)
    m, n = z.shape[-2:]
    B = z.shape[:-2].numel()
    zc = z.reshape(B, m, n).contiguous()
    s, ss = _operand(scale, z, B, m, n)
    zp, zs = (None, None) if zero_point is None else _operand(zero_point, z, B, m, n)
    row_words = -(-n * bits // 32)
    words = torch.empty(*z.shape[:-1], row_words, dtype=torch.int32, device=z.device)
    bad = torch.empty(*z.shape[:-1], dtype=torch.int32, device=z.device)
    with torch.cuda.device(z.device):
        _hip.call("pack_int", z.dtype, _hip.ptr(zc), B, m, n, _hip.ptr(s), ss, _hip.ptr(zp), zs, float(qmin),
                  float(qmax), bits, _hip.ptr(words), row_words, _hip.ptr(bad), _hip.stream(z.device))
    if check:
        _check_bad(bad, "values are not on the quantizer's grid")
    return (words, bad) if return_bad else words


@torch.no_grad()
def unpack_int(words: torch.Tensor, scale, zero_point=None, *, n: int, qmin: float, qmax: float,
               dtype: torch.dtype | None = None) -> torch.Tensor:
    """Values (u + qmin - zp) * s [*, m, n] of packed codes [*, m, row_words] (the inverse of ``pack_int``);
    ``dtype`` defaults to the scale's (a tensor's) or float32."""
    _hip.require_device(words)
    assert words.dtype == torch.int32 and words.dim() >= 2, "words must be int32 [*, m, row_words]"
    bits = int_code_bits(qmin, qmax)
    m, row_words = words.shape[-2:]
    assert row_words >= -(-n * bits // 32), "too few words per row for n codes"
    if dtype is None:
        dtype = scale.dtype if isinstance(scale, torch.Tensor) else torch.float32
    B = words.shape[:-2].numel()
    z = torch.empty(*words.shape[:-1], n, dtype=dtype, device=words.device)
    s, ss = _operand(scale, z, B, m, n)
    zp, zs = (None, None) if zero_point is None else _operand(zero_point, z, B, m, n)
    wc = words.contiguous()
    with torch.cuda.device(words.device):
        _hip.call("unpack_int", dtype, _hip.ptr(wc), B, m, n, row_words, _hip.ptr(s), ss,
                  _hip.ptr(zp), zs, float(qmin), bits, _hip.ptr(z), _hip.stream(words.device))
    return z


def super_entry_scales(scales: torch.Tensor, super_entry_shape) -> torch.Tensor:
    """The compact scales [*, m, n / q] of a per-entry abs-max scale map [*, m, n] (one per super-entry
    row), as the 16-bit values a packed layer stores are read from."""
    q = super_entry_shape[1]
    return scales[..., ::q].contiguous()


def stream_words(steps: int, L: int, K: int, V: int, tail_biting: bool = True) -> int:
    """Words of one packed trellis stream of ``steps`` states."""
    words = int(_hip.lib().gptq2d_trellis_stream_words(steps, L, K, V, int(bool(tail_biting))))
    if words < 0:
        raise ValueError(f"invalid trellis stream: steps={steps} L={L} K={K} V={V}")
    return words


@torch.no_grad()
def pack_trellis(states: torch.Tensor, *, L: int, K: int, V: int, tail_biting: bool = True,
                 super_entry_shape=None, check: bool = True, return_bad: bool = False):
    """Trellis streams of state paths.

    ``states`` is either the per-entry state map [*, m, n] that the trellis quantizers record (each state
    repeated over the V entries it emitted, super-entries of ``super_entry_shape`` (p, q) read row by row)
    -> words [*, m / p, n / q, W]; or, with ``super_entry_shape`` None, paths [..., S] one state per step
    -> words [..., W].  W = ``stream_words``.  With ``check`` (a host synchronisation) a path that breaks
    the trellis rule (or, with tail-biting, is not circular) raises."""
    _hip.require_device(states)
    assert states.dtype == torch.int64, "states must be int64"
    if super_entry_shape is None:
        lead, S = states.shape[:-1], states.size(-1)
        R = lead.numel()
        B, m, n, p, q, copies = 1, R, S, 1, S, 1
        out_shape = (*lead,)
    else:
        p, q = super_entry_shape
        m, n = states.shape[-2:]
        assert m % p == 0 and n % q == 0 and (p * q) % V == 0, "the super-entries must tile the map, T % V == 0"
        B = states.shape[:-2].numel()
        S, copies = p * q // V, V
        out_shape = (*states.shape[:-2], m // p, n // q)
    W = stream_words(S, L, K, V, tail_biting)
    words = torch.empty(*out_shape, W, dtype=torch.int32, device=states.device)
    bad = torch.empty(out_shape, dtype=torch.int32, device=states.device)
    sc = states.contiguous()
    with torch.cuda.device(states.device):
        _hip.call_untyped("trellis_pack", _hip.ptr(sc), B, m, n, p, q, copies, L, K, V,
                          int(bool(tail_biting)), _hip.ptr(words), W, _hip.ptr(bad), _hip.stream(states.device))
    if check:
        _check_bad(bad.flatten(), "state-path violations")
    return (words, bad) if return_bad else words


@torch.no_grad()
def unpack_trellis(words: torch.Tensor, *, steps: int, L: int, K: int, V: int,
                   tail_biting: bool = True) -> torch.Tensor:
    """State paths [..., steps] of streams [..., W] (the inverse of ``pack_trellis`` on paths)."""
    _hip.require_device(words)
    assert words.dtype == torch.int32
    W = words.size(-1)
    assert W >= stream_words(steps, L, K, V, tail_biting), "too few words for the stream"
    lead = words.shape[:-1]
    R = lead.numel()
    states = torch.empty(*lead, steps, dtype=torch.int64, device=words.device)
    wc = words.contiguous()
    with torch.cuda.device(words.device):
        _hip.call("trellis_unpack", torch.float32, _hip.ptr(wc), 1, R, steps * V, 1, steps * V, W, L,
                  K, V, int(bool(tail_biting)), None, None, 0, None, _hip.ptr(states), _hip.stream(words.device))
    return states


@torch.no_grad()
def decode_trellis(words: torch.Tensor, table: torch.Tensor, scale=None, *, K: int, tail_biting: bool = True,
                   super_entry_shape=None, steps: int | None = None) -> torch.Tensor:
    """Values of packed trellis streams: table[state] * scale, the trellis quantizer's output.

    With ``super_entry_shape`` (p, q): words [*, m / p, n / q, W] decode into the layer [*, m, n], each
    super-entry read row by row, and ``scale`` broadcasts against [*, m / p, n / q].  Without: words
    [..., W] of paths of ``steps`` states decode into sequences [..., steps * V], ``scale`` broadcasting
    against [...]."""
    _hip.require_device(words)
    assert words.dtype == torch.int32, "words must be int32"
    num_states, V = table.shape
    L = num_states.bit_length() - 1
    assert num_states == 1 << L, "the table needs 2^L rows"
    dtype = table.dtype if table.dtype in (torch.float32, torch.float64) else torch.float32
    W = words.size(-1)
    if super_entry_shape is None:
        assert steps is not None, "plain sequences need their number of steps"
        lead = words.shape[:-1]
        B, m, n, p, q = 1, lead.numel(), steps * V, 1, steps * V
        seq_shape, out_shape = lead, (*lead, steps * V)
    else:
        p, q = super_entry_shape
        assert (p * q) % V == 0, "T = p q must be a multiple of V"
        steps = p * q // V
        mb, nb = words.shape[-3:-1]
        lead = words.shape[:-3]
        B, m, n = lead.numel(), mb * p, nb * q
        seq_shape, out_shape = (*lead, mb, nb), (*lead, m, n)
    assert W >= stream_words(steps, L, K, V, tail_biting), "too few words for the stream"
    tab = table.to(device=words.device, dtype=dtype).contiguous()
    values = torch.empty(out_shape, dtype=dtype, device=words.device)
    sc = None
    if scale is not None:
        sc = torch.as_tensor(scale, dtype=dtype, device=words.device).expand(seq_shape).reshape(-1).contiguous()
    wc = words.contiguous()
    with torch.cuda.device(words.device):
        _hip.call("trellis_unpack", dtype, _hip.ptr(wc), B, m, n, p, q, W, L, K, V,
                  int(bool(tail_biting)), _hip.ptr(tab), _hip.ptr(sc), 1 if sc is not None else 0, _hip.ptr(values),
                  None, _hip.stream(words.device))
    return values
