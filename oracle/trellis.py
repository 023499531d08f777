"""CPU restatement of the reference's trellis (QTIP bitshift) quantizer (test oracle only).

Restates quantizer_trellis.py:28-143 and 344-369: the 1MAD, 3INST and HYB
state->value codes, the seeded k-means HYB look-up table, the Viterbi search
with first-index ties and optional first/last-state masks, the two-pass
tail-biting quantizer, and the super-entry plug-in.

Pinned by: tests/test_oracle_trellis.py -- Viterbi against brute force over
all paths on tiny trellises (with and without masks), path validity and
circularity of tail-biting, the code statistics of quantizer_trellis.py:429-438,
bit-level recomputation of 1MAD/3INST/HYB from their integer definitions, and
tests/test_oracle_golden.py (default HYB table, Viterbi states at L=16)
against vectors written from the reference.
"""

from __future__ import annotations

import itertools

import torch


def one_mad(L: int = 16, dtype=None) -> torch.Tensor:
    """1MAD: x = (s*34038481 + 76625530) mod 2^32, byte sum, (sum - 510)/147.800537109375 in fp32 (quantizer_trellis.py:28-33)."""
    x = (torch.arange(1 << L, dtype=torch.int64) * 34038481 + 76625530) & 0xFFFFFFFF
    x = (x & 255) + ((x >> 8) & 255) + ((x >> 16) & 255) + ((x >> 24) & 255)
    div = x.new_tensor(147.800537109375, dtype=torch.float32)
    return ((x - 510).float() / div)[:, None].to(dtype=dtype)


def three_inst(L: int = 16, dtype=None) -> torch.Tensor:
    """3INST: masked hash, two fp16 halves summed in fp16 (quantizer_trellis.py:36-41)."""
    x = ((torch.arange(1 << L, dtype=torch.int64) * 89226354 + 64248484) & 0x8FFF8FFF) ^ 0x3B603B60
    halves = torch.stack((x >> 16, x & 0xFFFF), dim=-1)
    halves = torch.where(halves >= 1 << 15, halves - (1 << 16), halves).to(torch.int16).view(torch.float16)
    return (halves[:, 0] + halves[:, 1]).float()[:, None].to(dtype=dtype)


def gaussian_codebook(size: int, seed: int = 0, samples: int = 1 << 16, iters: int = 25) -> torch.Tensor:
    """Seeded k-means codebook of the 2-D standard Gaussian, std sqrt(15/16) (quantizer_trellis.py:44-60)."""
    gen = torch.Generator().manual_seed(seed)
    data = torch.randn(samples, 2, generator=gen)
    centers = torch.randn(size, 2, generator=gen)
    for _ in range(iters):
        nearest = torch.cdist(data, centers).argmin(dim=1)
        counts = nearest.bincount(minlength=size)
        sums = torch.segment_reduce(data[nearest.argsort(stable=True), :], "sum", lengths=counts, axis=0)
        centers = torch.where(counts[:, None] > 0, sums / counts[:, None].clamp_min(1), centers)
    return centers / centers.std(correction=0) * (15 / 16) ** .5


def hyb(L: int = 16, tlut: torch.Tensor | None = None, seed: int = 0, dtype=None) -> torch.Tensor:
    """HYB: x = s(s+1); row (x >> (15 - b)) & (2^b - 1) of tlut, sign of col 0 from bit 15 (quantizer_trellis.py:63-79)."""
    tlut = gaussian_codebook(1 << 9, seed=seed) if tlut is None else tlut
    bits = tlut.size(0).bit_length() - 1
    x = torch.arange(1 << L, dtype=torch.int64)
    x = x * (x + 1)
    table = tlut[(x >> (15 - bits)) & ((1 << bits) - 1), :]
    table[:, 0] *= 1 - 2 * ((x >> 15) & 1)
    return table.to(dtype=dtype)


def viterbi(x, table, K, init=None, final=None):
    """States [..., T/V] of the closest trellis path, first-index ties (quantizer_trellis.py:82-115)."""
    nstates, V = table.shape
    shift = K * V
    table = table.to(x)
    xs = x.unflatten(-1, (-1, V))

    def local(t):
        return (table - xs[..., t, None, :]).square().sum(dim=-1)

    cost = local(0)
    if init is not None:
        cost = cost.masked_fill(~init, torch.inf)
    choices = []
    for t in range(1, xs.size(-2)):
        best, h = cost.unflatten(-1, (1 << shift, nstates >> shift)).min(dim=-2)
        choices.append(h)
        cost = best.repeat_interleave(1 << shift, dim=-1) + local(t)
    if final is not None:
        cost = cost.masked_fill(~final, torch.inf)
    states = [cost.argmin(dim=-1)]
    for h in reversed(choices):
        low = states[-1] >> shift
        states.append(low + h.gather(-1, low[..., None])[..., 0] * (nstates >> shift))
    return torch.stack(states[::-1], dim=-1)


def trellis_quantize(x, table, K, tail_biting=True):
    """Values [..., T] and states [..., T/V]; tail-biting by a first pass on x rolled by half (quantizer_trellis.py:118-143)."""
    nstates, V = table.shape
    shift = K * V
    init = final = None
    if tail_biting:
        half = x.size(-1) // V // 2
        overlap = viterbi(x.roll(half * V, dims=-1), table, K)[..., half, None] >> shift
        st = torch.arange(nstates)
        init = (st >> shift) == overlap
        final = (st % (nstates >> shift)) == overlap
    states = viterbi(x, table, K, init, final)
    return table.to(x)[states, :].flatten(start_dim=-2), states


def trellis_quantizer_super_entry(y_flat, select, scale, *, out, table, K, tail_biting=True):
    """Super-entry plug-in: each super-entry read row by row is one sequence (quantizer_trellis.py:344-369)."""
    x = select(y_flat) / scale
    seqs = x.reshape(-1, x.size(-2) * x.size(-1))
    rows, T = seqs.shape
    padded = torch.cat((seqs, seqs.new_zeros((1 << (rows - 1).bit_length()) - rows, T)))
    values, _ = trellis_quantize(padded, table, K, tail_biting)
    torch.mul(values[:rows, :].view_as(x), scale, out=out)


def brute_force(x, table, K, init=None, final=None):
    """Least squared distance from x [T] over all allowed paths (quantizer_trellis.py:394-403)."""
    nstates, V = table.shape
    best = float("inf")
    for first in range(nstates):
        for bits in itertools.product(range(1 << K * V), repeat=x.numel() // V - 1):
            st = list(itertools.accumulate(bits, lambda s, b: ((s << K * V) | b) % nstates, initial=first))
            if (init is None or init[first]) and (final is None or final[st[-1]]):
                best = min(best, (table[st, :].flatten() - x).square().sum().item())
    return best
