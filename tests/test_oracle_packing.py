"""Pin the CPU restatement of the packed formats (oracle/packing.py) -- CPU only.

INT codes: hand-derived words for small rows (nibbles, a 3-bit field that straddles a word), and the
reference's own C1 output (tests/golden/c1_int4.npz: its codes and per-row scales) packed and unpacked
back bit for bit.  Trellis streams: hand-derived words for a 4-bit path with and without tail-biting, and
every state path the reference's search wrote (tests/golden/trellis.npz) obeys the shift rule, packs into
exactly T*K bits with tail-biting, gives back every state as the L-bit window at t*K*V, and decodes to
the reference's values.
"""

import pathlib

import numpy as np
import pytest
import torch

import quantizer_trellis as QT
from oracle import packing as P

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("codes,bits,words", [
    ([1, 2, 3, 4, 5, 6, 7, 8], 4, [0x87654321]),
    ([15, 0, 15, 0, 15, 0, 15, 0, 9], 4, [0x0F0F0F0F, 0x00000009]),
    ([7, 1, 2], 3, [0x0000008F]),
    ([7] * 11, 3, [0xFFFFFFFF, 0x00000001]),
    ([0] * 10 + [5], 3, [0x40000000, 0x00000001]),
    ([255, 1, 128, 0], 8, [0x008001FF]),
    ([1, 0, 1, 1] + [0] * 28 + [1], 1, [0x0000000D, 0x00000001]),
])
def test_int_known_words(codes, bits, words):
    got = P.pack_lsb(np.array([codes]), bits)
    assert got.tolist() == [words]
    assert P.unpack_lsb(got, len(codes), bits).tolist() == [codes]


def test_int_bits():
    assert [P.int_bits(*r) for r in ((-8, 7), (-4, 3), (0, 15), (-128, 127), (-2, 1), (0, 1), (-3, 2))] == [
        4, 3, 4, 8, 2, 1, 3]


def test_int_reference_c1_round_trip():
    """The reference's C1 values (codes times per-row bf16 scales, zero point 0) pack to their codes + 8
    and unpack to the same values."""
    d = np.load(GOLDEN / "c1_int4.npz")
    codes = d["codes"].astype(np.float32)
    s = d["row_scale"]
    z = (codes - np.float32(0)) * s  # the affine quantizer's (q - zp) * s in fp32
    u, ok = P.int_codes(z, s, 0., -8, 7)
    assert ok.all() and (u.astype(np.int64) == d["codes"].astype(np.int64) + 8).all()
    words = P.pack_lsb(u, 4)
    assert words.shape == (512, 64)
    back = P.dequantize(P.unpack_lsb(words, 512, 4), s, 0., -8, np.float32)
    assert np.array_equal(back.view(np.uint32), z.view(np.uint32))


def test_int_codes_flags_off_grid():
    s = np.float32(0.25)
    z = np.array([0.5, 0.26, -2.0, 1.75, 2.0, np.nan], dtype=np.float32)
    u, ok = P.int_codes(z, s, None, -8, 7)
    assert ok.tolist() == [True, False, True, True, False, False]  # 0.26 off the grid; 2.0 = code 8 > 7
    assert u[ok].tolist() == [10, 0, 15]
    # an affine grid with a zero point: z = (q - 3) * 0.5
    z2 = (np.arange(16, dtype=np.float64) - 3.) * 0.5
    u2, ok2 = P.int_codes(z2, 0.5, 3., 0, 15)
    assert ok2.all() and u2.tolist() == list(range(16))


def test_trellis_known_words():
    # stream 10 11 01 00 (circular): windows of 4 bits at 0, 2, 4, 6 are 1011, 1101, 0100, 0010
    st = np.array([[11, 13, 4, 2]])
    assert P.path_violations(st, 4, 2, True).tolist() == [0]
    assert P.trellis_stream(st, 4, 2, True).tolist() == [[0xB4000000]]
    # without tail-biting the low 2 bits of the last state follow: 10 11 01 00 10
    assert P.trellis_stream(st, 4, 2, False).tolist() == [[0xB4800000]]
    assert P.stream_states(np.array([[0xB4000000]]), 4, 4, 2, True).tolist() == st.tolist()
    assert P.stream_states(np.array([[0xB4800000]]), 4, 4, 2, False).tolist() == st.tolist()
    assert P.path_violations(np.array([[11, 1]]), 4, 2, False).tolist() == [1]
    # 14 -> 4 (4 >> 2 = 1, 14 mod 4 = 2) and, circularly, 3 -> 11 (11 >> 2 = 2, 3 mod 4 = 3) break the rule
    assert P.path_violations(np.array([[11, 14, 4, 3]]), 4, 2, True).tolist() == [2]
    assert P.path_violations(np.array([[11, 14, 4, 3]]), 4, 2, False).tolist() == [1]


# (L, K, V, T) of tests/golden/make_golden.py's trellis shapes s0..s6
GOLDEN_SHAPES = [(5, 1, 1, 7), (4, 1, 2, 8), (6, 1, 2, 14), (10, 2, 2, 64), (9, 3, 1, 21), (12, 4, 2, 40),
                 (7, 1, 1, 1)]


def _golden_paths():
    d = np.load(GOLDEN / "trellis.npz")
    for idx, (L, K, V, T) in enumerate(GOLDEN_SHAPES):
        for dt in ("float32", "float64"):
            for tb in (0, 1):
                key = f"s{idx}_{dt}_{tb}"
                yield key, L, K, V, T, bool(tb), d[key + "_states"], d[key + "_table"], d[key + "_values"]
    hyb = QT.hyb().numpy()
    for tb in (0, 1):
        yield f"hyb16_{tb}", 16, 2, 2, 256, bool(tb), d[f"hyb16_states_{tb}"], hyb, d[f"hyb16_values_{tb}"]
    yield "ties", 8, 2, 2, 64, True, d["ties_states"], d["ties_table"], None


@pytest.mark.parametrize("case", list(_golden_paths()), ids=lambda c: c[0])
def test_trellis_reference_paths(case):
    key, L, K, V, T, tb, states, table, values = case
    KV = K * V
    assert P.path_violations(states, L, KV, tb).tolist() == [0] * states.shape[0]
    words = P.trellis_stream(states, L, KV, tb)
    bits = T * K if tb else T * K + L - KV
    assert words.shape[-1] == -(-bits // 32)
    assert np.array_equal(P.stream_states(words, T // V, L, KV, tb), states)
    if values is not None:
        dec = table[states].reshape(states.shape[0], T)
        assert np.array_equal(dec.view(np.uint8), values.view(np.uint8)), key
