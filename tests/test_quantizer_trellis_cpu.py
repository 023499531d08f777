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
