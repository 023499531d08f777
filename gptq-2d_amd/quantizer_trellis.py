"""Trellis (QTIP bitshift) quantizer plug-ins for super-entry GPTQ-2D (drop-in for the reference's
``quantizer_trellis.py``).

A trellis state is an L-bit window of a bitstream; each step shifts K*V new bits in and emits the V
values ``table[state]``, so T values cost T*K bits.  The Viterbi search finds the bitstream whose
values are closest to the input; tail-biting makes it circular (exactly T*K bits) with two passes.
The codes ``one_mad``, ``three_inst`` and ``hyb`` map states to roughly Gaussian values (QTIP).

``trellis_quantizer_super_entry_hip`` quantizes each super-entry of an antidiagonal, read row by
row, as one sequence and writes ``scale`` times its values; the whole two-pass search of all the
stage's sequences is one HIP launch (``csrc/viterbi.hip``), never synchronises with the host, and
is graph-capturable.  Tables with at most 1024 distinct rows or row pairs (HYB: 512 look-up rows, each
with both signs; 1MAD: 908 values at L = 16) are searched from a per-step cost table of those entries; the entries
and each state's entry are found once per table (one host synchronisation, outside graph capture) and
cached.  ``trellis_quantizer_super_entry_torch`` is the PyTorch formulation on any
device; the reference's ``*_triton`` name is an alias of the HIP plug-in.

Reference: IST-DASLab/GPTQ-2D quantizer_trellis.py (codes :28-79, Viterbi :82-143, plug-ins
:344-391).
"""

from __future__ import annotations

import weakref
from typing import Callable

import numpy as np
import torch

import _hip

# Distinct rows of a code table (bitwise): at most this many make the search use per-step cost tables.
ROWS_MAX = 1024
_rows_cache: dict = {}


# ------------------------------------------------------------------------------------------------ codes

def one_mad(L: int = 16, device=None, dtype=None) -> torch.Tensor:
    """1MAD code [2^L, 1]: x = (s * 34038481 + 76625530) mod 2^32, the sum of its four bytes, then
    (sum - 510) / 147.800537109375 in float32 (quantizer_trellis.py:28-33)."""
    x = (torch.arange(1 << L, dtype=torch.int64, device=device) * 34038481 + 76625530) & 0xFFFFFFFF
    x = (x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255) + ((x >> 24) & 255)
    divisor = x.new_tensor(147.800537109375, dtype=torch.float32)  # a tensor divisor: a true division everywhere
    return ((x - 510).float() / divisor)[:, None].to(dtype=dtype)


def three_inst(L: int = 16, device=None, dtype=None) -> torch.Tensor:
    """3INST code [2^L, 1]: ((s * 89226354 + 64248484) & 0x8FFF8FFF) ^ 0x3B603B60 read as two fp16
    halves, summed in fp16 (quantizer_trellis.py:36-41)."""
    x = ((torch.arange(1 << L, dtype=torch.int64, device=device) * 89226354 + 64248484) & 0x8FFF8FFF) ^ 0x3B603B60
    halves = torch.stack((x >> 16, x & 0xFFFF), dim=-1)
    halves = torch.where(halves >= 1 << 15, halves - (1 << 16), halves).to(torch.int16).view(torch.float16)
    return (halves[:, 0] + halves[:, 1]).float()[:, None].to(dtype=dtype)


def _gaussian_codebook(size: int, seed: int = 0, samples: int = 1 << 16, iters: int = 25, device=None) -> torch.Tensor:
    """Seeded k-means codebook [size, 2] of the 2-D standard Gaussian, rescaled to population std
    sqrt(15/16) (quantizer_trellis.py:44-60).  The points and the initial centres come from a seeded
    CPU generator; each cluster sums its points in order, so the result is deterministic."""
    gen = torch.Generator().manual_seed(seed)
    data = torch.randn(samples, 2, generator=gen).to(device)
    centers = torch.randn(size, 2, generator=gen).to(device)
    for _ in range(iters):
        nearest = torch.cdist(data, centers).argmin(dim=1)
        counts = nearest.bincount(minlength=size)
        sums = torch.segment_reduce(data[nearest.argsort(stable=True), :], "sum", lengths=counts, axis=0)
        centers = torch.where(counts[:, None] > 0, sums / counts[:, None].clamp_min(1), centers)
    return centers / centers.std(correction=0) * (15 / 16) ** .5


def hyb(L: int = 16, tlut: torch.Tensor | None = None, seed: int = 0, device=None, dtype=None) -> torch.Tensor:
    """HYB code [2^L, 2]: the hash x = s (s + 1) picks row (x >> (15 - b)) & (2^b - 1) of the 2^b-row
    look-up table ``tlut`` (default: the seeded 512-row k-means codebook), and bit 15 of x flips the
    sign of the first value (quantizer_trellis.py:63-79)."""
    tlut = _gaussian_codebook(1 << 9, seed=seed, device=device) if tlut is None else tlut
    bits = tlut.size(0).bit_length() - 1
    x = torch.arange(1 << L, dtype=torch.int64, device=tlut.device)
    x = x * (x + 1)
    table = tlut[(x >> (15 - bits)) & ((1 << bits) - 1), :]
    table[:, 0] *= 1 - 2 * ((x >> 15) & 1)
    return table.to(dtype=dtype)


# ------------------------------------------------------------------------------------------------ search

def _check(table: torch.Tensor, K: int, T: int):
    num_states, V = table.shape
    L = num_states.bit_length() - 1
    assert num_states == 1 << L, "the table needs 2^L rows"
    assert V in (1, 2) and K * V <= 8 and K * V <= L and T % V == 0, (
        "the same sums need V <= 2, a walk back holds 2^(K*V) <= 256 candidates, and T must be a multiple of V"
    )
    return L, V


def distinct_rows(table: torch.Tensor):
    """The table as at most ROWS_MAX entries of its distinct rows, or None: (urows [E, W, V], index [2^L / W]
    int32, W) with ``table[s + w 2^L / W] == urows[index[s], w]`` bit for bit.  W = 2 (pairs of the states s and
    s + 2^(L-1): for HYB the same look-up row with both signs, 1024 ordered pairs) where at most ROWS_MAX distinct pairs
    occur, else W = 1 (the distinct rows).  Only for an fp32 GPU table; computed once per table object and
    version (one host synchronisation, never inside graph capture) and cached while the table lives."""
    if table.dtype != torch.float32 or not table.is_cuda or not table.is_contiguous() or table.dim() != 2:
        return None
    key = id(table)
    hit = _rows_cache.get(key)
    if hit is not None and hit[0]() is table and hit[1] == table._version:
        return hit[2]
    if torch.cuda.is_current_stream_capturing():
        return None
    bits, index = torch.unique(table.view(torch.int32), dim=0, return_inverse=True)
    R, S = bits.size(0), table.size(0)
    found = None
    if S >= 2:
        pairs, pindex = torch.unique(index[:S // 2] * R + index[S // 2:], return_inverse=True)
        if pairs.size(0) <= ROWS_MAX:
            urows = torch.stack((bits[pairs // R], bits[pairs % R]), dim=1)
            found = (urows.view(torch.float32).contiguous(), pindex.to(torch.int32).contiguous(), 2)
    if found is None and R <= ROWS_MAX:
        found = (bits.view(torch.float32)[:, None, :].contiguous(), index.to(torch.int32).contiguous(), 1)
    _rows_cache[key] = (weakref.ref(table, lambda _, k=key: _rows_cache.pop(k, None)), table._version, found, {})
    return found


def bank_copies(index: torch.Tensor, W: int, kv: int, sweeps: int = 2) -> torch.Tensor:
    """``index`` with bit 16 set for the states whose cost the distinct-row search reads from the second copy
    of its per-step cost table (``csrc/viterbi.hip``, ``second_slot``).

    The search's thread t reads, at (h, e), the entry of state h G + 4 t + e (G = 2^(L - kv), h < 2^kv / W,
    e < 4); 64 / W neighbouring threads read together (32 lanes of 8 bytes, or 64 of 4) and wait for the busiest
    of the 64 four-byte banks.  Entry x lies at bank x mod NB of the first copy and (x + x div NB) mod NB of the
    second (NB = 64 / W entries a bank row).  Per read, each distinct entry in turn takes the copy whose bank is
    less loaded, then ``sweeps`` passes move each to the other copy where that is less loaded: the busiest bank
    of HYB's pair reads drops from 3.4 to 2.0 on average.  Lanes that read one entry read one copy (a broadcast).
    Either copy holds the same values, so any choice gives the same search."""
    idx = index.cpu().numpy().astype(np.int64)
    he = (1 << kv) // W
    G = idx.size // he
    nl = nb = 64 // W
    T = min(G // 4, 1024)  # threads that own groups
    tp = -(-T // nl) * nl
    tid = np.arange(tp)
    st = np.stack([h * G + 4 * tid + e for h in range(he) for e in range(4)])  # [he 4, tp] states
    st = np.where(tid[None, :] < T, st, -1).reshape(-1, nl)  # [reads, lanes]
    ent = np.where(st >= 0, idx[np.maximum(st, 0)], -1)
    valid = ent >= 0
    e0 = np.maximum(ent, 0)
    banks = np.stack((e0 % nb, (e0 + e0 // nb) % nb))  # [2, reads, lanes]
    n = ent.shape[0]
    first = np.argmax((ent[:, :, None] == ent[:, None, :]) & valid[:, :, None], axis=2)
    lead = (first == np.arange(nl)[None, :]) & valid
    rows = np.arange(n)
    load = np.zeros((n, nb), np.int64)
    pick = np.zeros((n, nl), np.int64)
    for sweep in range(sweeps + 1):
        for i in range(nl):
            m = lead[:, i]
            if sweep:  # take the lane's entry off its bank, then place it again
                np.add.at(load, (rows[m], banks[pick[m, i], rows[m], i]), -1)
            l0, l1 = load[rows, banks[0, :, i]], load[rows, banks[1, :, i]]
            pick[:, i] = np.where(l1 == l0, pick[:, i], l1 < l0)
            np.add.at(load, (rows[m], banks[pick[m, i], rows[m], i]), 1)
    pick = np.take_along_axis(pick, first, 1)
    out = idx.copy()
    ok = st >= 0
    out[st[ok]] |= pick[ok] << 16
    return torch.from_numpy(out.astype(np.int32)).to(index.device)


def rows_index(table: torch.Tensor, kv: int):
    """``distinct_rows(table)`` with its index as the search reads it for K V = kv: (urows, index | copy << 16,
    W) with the copies of ``bank_copies``, or None.  Cached beside the rows; None under graph capture when not
    yet computed."""
    found = distinct_rows(table)
    if found is None:
        return None
    per_kv = _rows_cache[id(table)][3]
    ridx = per_kv.get(kv)
    if ridx is None:
        urows, index, W = found
        he = (1 << kv) // W
        if torch.cuda.is_current_stream_capturing() or he < 1 or index.numel() % he:
            return None
        ridx = per_kv[kv] = bank_copies(index, W, kv)
    return found[0], ridx, found[2]


def trellis_quantize_hip(x: torch.Tensor, table: torch.Tensor, K: int, tail_biting: bool = True, *,
                         out: torch.Tensor | None = None, scale: torch.Tensor | None = None,
                         states: torch.Tensor | None = None):
    """Quantize the sequences x [..., T] on the GPU: values [..., T] (times ``scale`` [...] if given) and
    states [..., T/V] of the closest (tail-biting) trellis paths.  Writes into ``out`` / ``states`` when
    given, else returns (values, states).  One HIP launch; no host synchronisation.

    The same search as the reference's _trellis_quantize_torch / _trellis_quantize_triton
    (quantizer_trellis.py:118-143, 271-341)."""
    _hip.require_device(x)
    assert x.dtype in (torch.float32, torch.float64)
    T = x.size(-1)
    L, V = _check(table, K, T)
    steps = T // V
    seq = x.reshape(-1, T).contiguous()
    rows = seq.size(0)
    tab = table.to(device=x.device, dtype=x.dtype).contiguous()
    ret = out is None
    if out is None:
        out = torch.empty_like(seq)
    if states is None and ret:
        states = torch.empty(rows, steps, dtype=torch.int64, device=x.device)
    if rows == 0:
        return (out.view(x.shape), states.view(*x.shape[:-1], steps)) if ret else None
    sc = None if scale is None else scale.to(x.dtype).reshape(rows).contiguous()
    # The history is sized for a power of two of rows: under graph capture, freed buffers of the graph's
    # pool serve later requests that fit, so growing antidiagonals reserve less than twice the largest.
    cap = 1 << (rows - 1).bit_length()
    size = int(_hip.lib().gptq2d_viterbi_workspace(cap, steps, L, K, V))
    hist = x.new_empty(size)
    with torch.cuda.device(x.device):
        urows = rows_index(tab, K * V) if tab is table else None
        if urows is not None:
            _hip.call_untyped("viterbi_rows_f32", _hip.ptr(seq), _hip.ptr(tab), _hip.ptr(urows[0]), _hip.ptr(urows[1]),
                              urows[0].size(0), urows[2], _hip.ptr(hist), _hip.ptr(sc), _hip.ptr(out),
                              _hip.ptr(states), rows, steps, L, K, V, int(bool(tail_biting)), _hip.stream(x.device))
        else:
            _hip.call("viterbi", x.dtype, _hip.ptr(seq), _hip.ptr(tab), _hip.ptr(hist), _hip.ptr(sc),
                      _hip.ptr(out), _hip.ptr(states), rows, steps, L, K, V, int(bool(tail_biting)),
                      _hip.stream(x.device))
    if ret:
        return out.view(x.shape), states.view(*x.shape[:-1], steps)
    return None


def _viterbi_torch(x, table, K, init=None, final=None):
    """States [..., T/V] of the closest path, first-index ties, optional first/last-state masks
    (quantizer_trellis.py:82-115)."""
    num_states, V = table.shape
    shift = K * V
    G = num_states >> shift
    tab = table.to(x)
    xs = x.unflatten(-1, (-1, V))

    def local(t):
        return (tab - xs[..., t, None, :]).square().sum(dim=-1)

    cost = local(0)
    if init is not None:
        cost = cost.masked_fill(~init, torch.inf)
    choices = []
    for t in range(1, xs.size(-2)):
        best, h = cost.unflatten(-1, (1 << shift, G)).min(dim=-2)
        choices.append(h)
        cost = best.repeat_interleave(1 << shift, dim=-1) + local(t)
    if final is not None:
        cost = cost.masked_fill(~final, torch.inf)
    path = [cost.argmin(dim=-1)]
    for h in reversed(choices):
        low = path[-1] >> shift
        path.append(low + h.gather(-1, low[..., None])[..., 0] * G)
    return torch.stack(path[::-1], dim=-1)


def trellis_quantize_torch(x: torch.Tensor, table: torch.Tensor, K: int, tail_biting: bool = True):
    """(values [..., T], states [..., T/V]) of the closest tail-biting trellis paths, with PyTorch on any
    device (quantizer_trellis.py:118-143)."""
    num_states, V = table.shape
    shift = K * V
    init = final = None
    if tail_biting:
        half = x.size(-1) // V // 2
        overlap = _viterbi_torch(x.roll(half * V, dims=-1), table, K)[..., half, None] >> shift
        st = torch.arange(num_states, device=x.device)
        init = (st >> shift) == overlap
        final = (st % (num_states >> shift)) == overlap
    states = _viterbi_torch(x, table, K, init, final)
    return table.to(x)[states, :].flatten(start_dim=-2), states


# ------------------------------------------------------------------------------------------------ plug-ins

def _record_states(states, y_flat, select, st, V):
    """Write each super-entry's states into the per-entry state map ``states`` [*batch, m, n] (int64): the
    entries t*V .. t*V + V - 1 of a super-entry, read row by row, hold its state t (the state that emitted
    them) -- the input of packing.pack_trellis."""
    flat = states.flatten(start_dim=-2)
    assert flat.shape == y_flat.shape and flat.dtype == torch.int64 and flat.device == y_flat.device, (
        "states must be an int64 [*batch, m, n] tensor of Y's batch shape on Y's device"
    )
    view = select(flat)
    view.copy_(st.repeat_interleave(V, dim=-1).view(view.shape))


def trellis_quantizer_super_entry_torch(y_flat: torch.Tensor, select: Callable, scale: torch.Tensor,
                                        states: torch.Tensor | None = None, *, out: torch.Tensor,
                                        table: torch.Tensor, K: int, tail_biting: bool = True) -> None:
    """Each super-entry of ``select(y_flat) / scale``, read row by row, is one sequence; ``out`` gets
    ``scale`` times its trellis values (quantizer_trellis.py:344-369).  Rows are padded with zero
    sequences to a power of two, as the reference does, so that graph memory pools stay small.
    ``states`` (optional, no reference counterpart): the per-entry state map of ``_record_states``."""
    x = select(y_flat) / scale
    seqs = x.reshape(-1, x.size(-2) * x.size(-1))
    rows, T = seqs.shape
    padded = torch.cat((seqs, seqs.new_zeros((1 << (rows - 1).bit_length()) - rows, T)))
    values, st = trellis_quantize_torch(padded, table, K, tail_biting)
    torch.mul(values[:rows, :].view_as(x), scale, out=out)
    if states is not None:
        _record_states(states, y_flat, select, st[:rows], table.size(1))


def trellis_quantizer_super_entry_hip(y_flat: torch.Tensor, select: Callable, scale: torch.Tensor,
                                      states: torch.Tensor | None = None, *, out: torch.Tensor,
                                      table: torch.Tensor, K: int, tail_biting: bool = True) -> None:
    """``trellis_quantizer_super_entry_torch`` with the search in one HIP launch per call
    (quantizer_trellis.py:372-391).  ``y_flat``, ``scale`` and ``table`` must be on one GPU; ``scale``
    broadcasts against the super-entries and is constant within each.  ``states`` as there."""
    _hip.require_device(y_flat)
    assert table.device == y_flat.device and (not isinstance(scale, torch.Tensor) or scale.device == y_flat.device), (
        "the HIP trellis quantizer requires Y, scale, and table on one GPU"
    )
    x = select(y_flat) / scale
    seqs = x.flatten(start_dim=-2)
    sc = torch.as_tensor(scale, dtype=x.dtype, device=x.device).broadcast_to(x.shape)[..., 0, 0]
    st = None if states is None else torch.empty(seqs.shape[:-1].numel(), seqs.size(-1) // table.size(1),
                                                 dtype=torch.int64, device=x.device)
    trellis_quantize_hip(seqs, table, K, tail_biting, out=out.view(seqs.shape), scale=sc, states=st)
    if states is not None:
        _record_states(states, y_flat, select, st.view(*seqs.shape[:-1], -1), table.size(1))


# The reference's Triton name, kept for drop-in use: one implementation, not two.
trellis_quantizer_super_entry_triton = trellis_quantizer_super_entry_hip
