"""Pin the oracle's trellis quantizer (CPU only).

Viterbi against brute force over all paths (quantizer_trellis.py:407-417), tail-biting path validity
and circularity (:419-427), code statistics (:429-438), and the codes recomputed bit by bit from
their integer definitions in plain Python (numpy for the fp16 halves).
"""

import struct

import numpy as np
import torch

from oracle import trellis as Tr


def test_viterbi_brute_force():
    g = torch.Generator().manual_seed(0)
    for L, K, V, T in (5, 1, 1, 7), (4, 1, 2, 8):
        table = torch.randn(1 << L, V, generator=g, dtype=torch.float64)
        x = torch.randn(3, T, generator=g, dtype=torch.float64)
        init, final = torch.rand(2, 3, 1 << L, generator=g) < .5
        for masks in ((None, None), (init, final)):
            st = Tr.viterbi(x, table, K, *masks)
            values = table[st, :].flatten(start_dim=-2)
            for b in range(3):
                expected = Tr.brute_force(x[b], table, K, *(None if mk is None else mk[b] for mk in masks))
                assert abs((values[b] - x[b]).square().sum().item() - expected) < 1e-9


def test_tail_biting_paths():
    g = torch.Generator().manual_seed(1)
    L, K, V = 10, 2, 2
    table = torch.randn(1 << L, V, generator=g)
    values, states = Tr.trellis_quantize(torch.randn(4, 32, generator=g), table, K)
    shared = (1 << (L - K * V)) - 1
    assert ((states[:, 1:] >> K * V) == (states[:, :-1] & shared)).all()
    assert ((states[:, 0] >> K * V) == (states[:, -1] & shared)).all()
    assert values.equal(table[states, :].flatten(start_dim=-2))


def test_first_index_ties():
    """With an all-equal table every path costs the same: the search must pick the all-zero bitstream."""
    table = torch.zeros(1 << 6, 2)
    st = Tr.viterbi(torch.zeros(2, 16), table, 2)
    assert (st == 0).all()


def test_code_statistics():
    for code in Tr.one_mad(), Tr.three_inst():
        assert code.mean().abs().item() < .01
    assert abs(Tr.one_mad().std().item() - 1.) < .01
    tlut = torch.randn(1 << 9, 2, generator=torch.Generator().manual_seed(2))
    table = Tr.hyb(tlut=tlut)
    rows = (table[:, 1, None] == tlut[:, 1]).int().argmax(dim=-1)
    assert table[:, 0].abs().equal(tlut[rows, 0].abs())
    assert rows.bincount(minlength=1 << 9).eq(1 << 7).all()
    assert abs((table[:, 0] != tlut[rows, 0]).float().mean().item() - .5) < .01


def _f32(v):
    return struct.unpack("<f", struct.pack("<f", v))[0]


def test_codes_bitwise():
    """1MAD, 3INST and HYB recomputed from their integer definitions, state by state."""
    om, ti = Tr.one_mad(), Tr.three_inst()
    tlut = torch.randn(1 << 9, 2, generator=torch.Generator().manual_seed(7))
    hy = Tr.hyb(tlut=tlut)
    for s in list(range(0, 1 << 16, 997)) + [0, 1, 65535]:
        x = (s * 34038481 + 76625530) & 0xFFFFFFFF
        bsum = sum((x >> sh) & 255 for sh in (0, 8, 16, 24))
        assert om[s, 0].item() == float(np.float32(bsum - 510) / np.float32(147.800537109375))
        x = ((s * 89226354 + 64248484) & 0x8FFF8FFF) ^ 0x3B603B60
        h0 = np.array([x >> 16], dtype=np.uint16).view(np.float16)[0]
        h1 = np.array([x & 0xFFFF], dtype=np.uint16).view(np.float16)[0]
        assert ti[s, 0].item() == float(np.float16(h0 + h1))
        xh = s * (s + 1)
        row = (xh >> 6) & 511
        sign = -1. if (xh >> 15) & 1 else 1.
        assert hy[s, 0].item() == _f32(sign * tlut[row, 0].item())
        assert hy[s, 1].item() == tlut[row, 1].item()


def test_super_entry_plugin_matches_sequences():
    """The super-entry plug-in quantizes each super-entry read row by row as one sequence, times scale."""
    g = torch.Generator().manual_seed(5)
    table = torch.randn(1 << 8, 2, generator=g)
    y = torch.randn(2, 6 * 4 * 4, generator=g)
    sel = lambda t: t.unflatten(-1, (6, 4, 4))
    out = torch.empty(2, 6, 4, 4)
    Tr.trellis_quantizer_super_entry(y, sel, torch.tensor(1.3), out=out, table=table, K=2)
    vals, _ = Tr.trellis_quantize(sel(y).reshape(12, 16) / 1.3, table, 2)
    assert torch.allclose(out.reshape(12, 16), vals * 1.3)
