"""CPU restatement of the packed output formats (test infrastructure: only tests/, smoke() and bench's
CPU baseline use the oracle, and only as the checker).

The reference stores no packed format -- it returns dequantized values (gptq_2d.py:1378-1447) -- but its
quantizers define what a code is: the affine quantizer's integer q in [qmin, qmax] with value (q - zp) * s
(quantizer_int.py:63-83, 120-134), and the bitshift trellis's state path, whose consecutive states share
L - K*V bits so that a tail-biting path is T*K bits (quantizer_trellis.py:1-16, 82-143).  The layouts are
this engine's (csrc/pack.hip): INT codes u = q - qmin as little-endian bit fields per row; trellis streams
as the top K*V bits of each state, MSB first.  Written with numpy bit arrays, independently of the
kernels' word arithmetic.

Pinned by (tests/test_oracle_packing.py): hand-derived words for small code rows and paths; every golden
state path the reference wrote (tests/golden/trellis.npz, tail-biting or not) satisfies the shift rule,
packs to a stream whose L-bit windows give back every state, and decodes to the reference's values; INT
round trips on the reference's C1 output and on the quantizer's own grid.
"""

from __future__ import annotations

import numpy as np


def int_bits(qmin: int, qmax: int) -> int:
    """ceil(log2(qmax - qmin + 1))."""
    return max(1, int(np.ceil(np.log2(qmax - qmin + 1))))


def int_codes(z, scale, zp, qmin, qmax):
    """(u = q - qmin, ok) of values z under (scale, zp) broadcast to z; ok = (q - zp) * s == z, q in range."""
    z = np.asarray(z)
    s = np.broadcast_to(np.asarray(scale, dtype=z.dtype), z.shape)
    p = np.broadcast_to(np.asarray(0 if zp is None else zp, dtype=z.dtype), z.shape)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(z / s + p)
        ok = (q >= qmin) & (q <= qmax) & ((q - p) * s == z)
    u = np.where(ok, q - qmin, 0).astype(np.uint64)
    return u, ok


def pack_lsb(codes, bits: int):
    """Rows of codes [..., n] as little-endian bit fields in uint32 words [..., ceil(n bits / 32)]."""
    codes = np.asarray(codes, dtype=np.uint64)
    n = codes.shape[-1]
    W = -(-n * bits // 32)
    # bit k of code j is stream bit j*bits + k
    bitarr = ((codes[..., :, None] >> np.arange(bits, dtype=np.uint64)) & 1).astype(np.uint8)
    stream = bitarr.reshape(*codes.shape[:-1], n * bits)
    stream = np.concatenate([stream, np.zeros((*codes.shape[:-1], W * 32 - n * bits), np.uint8)], axis=-1)
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (stream.reshape(*codes.shape[:-1], W, 32).astype(np.uint64) * weights).sum(-1).astype(np.uint32)


def unpack_lsb(words, n: int, bits: int):
    words = np.asarray(words, dtype=np.uint32)
    stream = ((words[..., :, None].astype(np.uint64) >> np.arange(32, dtype=np.uint64)) & 1).reshape(
        *words.shape[:-1], -1)[..., :n * bits]
    weights = np.uint64(1) << np.arange(bits, dtype=np.uint64)
    return (stream.reshape(*words.shape[:-1], n, bits) * weights).sum(-1)


def dequantize(u, scale, zp, qmin, dtype):
    """(u + qmin - zp) * s in ``dtype``: the quantizer's value of code q = u + qmin."""
    q = np.asarray(u).astype(dtype) + dtype(qmin)
    p = np.asarray(0 if zp is None else zp, dtype=dtype)
    return (q - p) * np.asarray(scale, dtype=dtype)


def _msb_words(bitrows, total_bits):
    """Bit rows [..., total_bits] (0/1) as MSB-first uint32 words."""
    W = -(-total_bits // 32)
    pad = np.zeros((*bitrows.shape[:-1], W * 32 - total_bits), np.uint8)
    b = np.concatenate([bitrows.astype(np.uint8), pad], axis=-1).reshape(*bitrows.shape[:-1], W, 32)
    weights = np.uint64(1) << np.arange(31, -1, -1, dtype=np.uint64)
    return (b.astype(np.uint64) * weights).sum(-1).astype(np.uint32)


def _bits_msb(values, k):
    """The k low bits of each value, MSB first: [..., k]."""
    v = np.asarray(values, dtype=np.int64)[..., None]
    return ((v >> np.arange(k - 1, -1, -1)) & 1).astype(np.uint8)


def path_violations(states, L: int, KV: int, tail_biting: bool):
    """Per path [..., S]: states outside [0, 2^L) plus breaks of s_{t+1} >> KV == s_t mod 2^(L-KV) (and
    between the last state and the first with tail-biting)."""
    s = np.asarray(states, dtype=np.int64)
    low = (1 << (L - KV)) - 1
    bad = ((s < 0) | (s >= 1 << L)).sum(-1)
    bad = bad + ((s[..., 1:] >> KV) != (s[..., :-1] & low)).sum(-1)
    if tail_biting:
        bad = bad + ((s[..., 0] >> KV) != (s[..., -1] & low))
    return bad


def trellis_stream(states, L: int, KV: int, tail_biting: bool):
    """MSB-first streams [..., W] of paths [..., S]: the top KV bits of each state, then (without
    tail-biting) the low L - KV bits of the last state."""
    s = np.asarray(states, dtype=np.int64)
    S = s.shape[-1]
    top = _bits_msb(s >> (L - KV), KV).reshape(*s.shape[:-1], S * KV)
    if not tail_biting and L > KV:
        top = np.concatenate([top, _bits_msb(s[..., -1] & ((1 << (L - KV)) - 1), L - KV)], axis=-1)
    return _msb_words(top, top.shape[-1])


def stream_states(words, S: int, L: int, KV: int, tail_biting: bool):
    """State t = the L-bit window at stream bit t*KV (modulo the stream length with tail-biting)."""
    words = np.asarray(words, dtype=np.uint32)
    total = S * KV if tail_biting else S * KV + L - KV
    bits = ((words[..., :, None].astype(np.uint64) >> np.arange(31, -1, -1, dtype=np.uint64)) & 1).reshape(
        *words.shape[:-1], -1)[..., :total]
    pos = (np.arange(S)[:, None] * KV + np.arange(L)[None, :]) % total
    win = bits[..., pos]  # [..., S, L]
    weights = np.int64(1) << np.arange(L - 1, -1, -1, dtype=np.int64)
    return (win.astype(np.int64) * weights).sum(-1)
