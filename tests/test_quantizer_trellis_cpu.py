"""CPU tests of the trellis module of the package (codes and its PyTorch search) against the golden vectors
written from the reference (tests/golden/trellis.npz); the HIP search is tested in test_trellis_gpu.py."""

import hashlib
import pathlib

import numpy as np
import torch

import quantizer_trellis as QT

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
SHAPES = (5, 1, 1, 7), (4, 1, 2, 8), (6, 1, 2, 14), (10, 2, 2, 64), (9, 3, 1, 21), (12, 4, 2, 40), (7, 1, 1, 1)


def _sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def test_codes_match_reference():
    data = np.load(GOLDEN / "trellis.npz")
    assert _sha(QT.one_mad()) == str(data["sha_one_mad"])
    assert _sha(QT.three_inst()) == str(data["sha_three_inst"])
    assert np.array_equal(QT._gaussian_codebook(1 << 9).numpy(), data["hyb_tlut"])
    assert _sha(QT.hyb()) == str(data["sha_hyb"])
    assert QT.hyb(dtype=torch.float64).equal(QT.hyb().double())


def test_torch_search_matches_reference():
    data = np.load(GOLDEN / "trellis.npz")
    for idx, (L, K, V, T) in enumerate(SHAPES):
        for dname in ("float32", "float64"):
            for tb in (0, 1):
                key = f"s{idx}_{dname[-7:]}_{tb}"
                vals, st = QT.trellis_quantize_torch(torch.from_numpy(data[key + "_x"]),
                                                     torch.from_numpy(data[key + "_table"]), K, bool(tb))
                assert np.array_equal(st.numpy(), data[key + "_states"]), key
                assert np.array_equal(vals.numpy(), data[key + "_values"]), key


def _reads(index, W, kv):
    """The entries the distinct-row search reads together: thread t reads, at (h, e), the entry of state
    h 2^(L - kv) + 4 t + e, and 64 / W neighbouring threads read at once (csrc/viterbi.hip, forward_rows)."""
    he = (1 << kv) // W
    G = index.numel() // he
    T = min(G // 4, 1024)
    nl = 64 // W
    idx = index.numpy().astype(np.int64)
    for h in range(he):
        for e in range(4):
            for t0 in range(0, T, nl):
                yield idx[h * G + 4 * np.arange(t0, min(t0 + nl, T)) + e]


def _busiest(reads, W, second=lambda x, nb: (x + x // nb) % nb):
    """Mean over the reads of the busiest bank: entry x of copy c at bank x mod NB (c = 0) or second(x, NB)
    (c = 1; the kernel's rotation by default), NB = 64 / W; one read per distinct (copy, entry)."""
    nb = 64 // W
    out = []
    for r in reads:
        x, c = r & 0xffff, r >> 16
        slots = np.unique(np.stack([c, x], 1), axis=0)
        bank = np.where(slots[:, 0] == 1, second(slots[:, 1], nb), slots[:, 1] % nb)
        out.append(np.bincount(bank, minlength=nb).max())
    return float(np.mean(out))


def _rows(table):
    bits, index = torch.unique(table.view(torch.int32), dim=0, return_inverse=True)
    R, S = bits.size(0), table.size(0)
    pairs, pindex = torch.unique(index[:S // 2] * R + index[S // 2:], return_inverse=True)
    return (pindex.int(), 2) if pairs.numel() <= QT.ROWS_MAX else (index.int(), 1)


def test_bank_copies():
    """The copy choice keeps every state's entry, sends the lanes that read one entry in one read to one copy,
    and spreads the reads of HYB's 1024 pairs (W = 2) and 1MAD's 908 values (W = 1) so that the busiest bank of
    a read carries about 2 of them, against about 3.4 and 3.1 with one copy.  Mutants: all states on the first
    copy, or the choice ignored by a rotation that does not move the bank, lose the spread."""
    for table, kv, W_expect in ((QT.hyb(), 4, 2), (QT.one_mad(), 4, 1), (QT.hyb(), 2, 2)):
        index, W = _rows(table)
        assert W == W_expect
        r = QT.bank_copies(index, W, kv)
        assert r.dtype == torch.int32 and torch.equal(r & 0xffff, index) and bool(((r >> 16) <= 1).all())
        for read in _reads(r, W, kv):
            x, c = read & 0xffff, read >> 16
            for v in np.unique(x):
                assert len(np.unique(c[x == v])) == 1
        one, two = _busiest(_reads(index, W, kv), W), _busiest(_reads(r, W, kv), W)
        assert one > 2.8 and two < 2.1, (one, two)
        # the same choice with a second copy that is not rotated, or with every choice flipped
        assert _busiest(_reads(r, W, kv), W, second=lambda x, nb: x % nb) == one
        assert _busiest(_reads(r ^ (1 << 16), W, kv), W) > 2.5
