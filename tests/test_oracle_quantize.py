"""Pin the oracle's integer quantizers (CPU only).

Known answers from the reference (quantizer_int.py:476-488, 532-533), the affine closed form
re-derived entry by entry in Python float arithmetic, ties to even, the 16-bit scale rounding
against an independent bit-level round-to-nearest-even on the fp32 pattern, and the abs-max
quantizer against vectors the reference wrote on its own test's cases (quantizer_int.py:535-553)
plus a nearest-integer / ties-to-even property; floor, trunc and half-away-from-zero rounding
planted in the oracle fail both.
"""

import pathlib
import struct

import numpy as np
import pytest
import torch

from oracle import quantize as Qz


def test_affine_known_answers():
    y = torch.zeros(3, 3, dtype=torch.float64)
    scale, zp = torch.ones_like(y), torch.zeros_like(y)
    y[0, 2], y[1, 1], y[2, 0] = .5, 1.75, -9.
    scale[1, 1], scale[2, 0], zp[2, 0] = .5, 2., 1.
    sl = slice(2, 8, 2)
    for kw, expected in (({}, [0., 2., -10.]), (dict(qmin=-2, qmax=2), [0., 1., -6.])):
        out = torch.empty(3, dtype=torch.float64)
        Qz.affine_quantizer(y.flatten(), sl, scale, zp, out=out, **kw)
        assert out.tolist() == expected


def test_affine_closed_form_fp64():
    """Entry by entry in Python float arithmetic (IEEE fp64, round() ties to even): the reference's chain
    fl(fl(y / s) + z) -> round -> clamp -> fl(fl(code - z) * s), with batch-broadcast scales."""
    g = torch.Generator().manual_seed(0)
    y = 4 * torch.randn(2, 35, generator=g, dtype=torch.float64)
    s = .1 + torch.rand(1, 5, 7, generator=g, dtype=torch.float64)
    z = torch.randint(-2, 3, (2, 5, 7), generator=g).double()
    sl = slice(6, 36, 6)
    out = torch.empty(2, 5, dtype=torch.float64)
    Qz.affine_quantizer(y, sl, s, z, out=out, qmin=-3, qmax=4)
    for b in range(2):
        for k, pos in enumerate(range(6, 36, 6)):
            sv, zv, yv = s.flatten(-2)[0, pos].item(), z.flatten(-2)[b, pos].item(), y[b, pos].item()
            code = min(max(float(round(yv / sv + zv)), -3.), 4.)
            assert out[b, k].item() == (code - zv) * sv


def test_round_half_even():
    y = torch.tensor([.5, 1.5, 2.5, -.5, -1.5, 2.4999995, 2.5000005])
    out = torch.empty_like(y)
    Qz.round_quantizer(y, slice(0, 7, 1), out=out)
    assert out.tolist() == [0., 2., 2., -0., -2., 2., 3.]


def _bf16_rne_bits(f):
    u = struct.unpack("<I", struct.pack("<f", f))[0]
    low = u & 0xFFFF
    hi = u >> 16
    if low > 0x8000 or (low == 0x8000 and hi & 1):
        hi += 1
    return struct.unpack("<f", struct.pack("<I", (hi & 0xFFFF) << 16))[0]


def test_int_abs_max_scale():
    s = Qz.int_abs_max_scale(torch.tensor([[0., 0.], [3., -1.5]]), qmin=-8, qmax=7, dtype=torch.float16)
    assert s.equal(torch.tensor([[1.], [.4]]).half().float())
    g = torch.Generator().manual_seed(3)
    x = 4 * torch.randn(64, 32, generator=g)
    x[5] = 0.
    x[7] *= 1e-38
    s = Qz.int_abs_max_scale(x, qmin=-8, qmax=7, dtype=torch.bfloat16)
    for r in range(64):
        amax = x[r].abs().max().item()
        # fp32 division of the fp32 absmax by 7.5, then RNE to bf16
        quot = (torch.tensor(amax, dtype=torch.float32) / torch.tensor(7.5, dtype=torch.float32)).item()
        exp = _bf16_rne_bits(quot) if quot != 0 else 1.
        assert s[r, 0].item() == exp, r


def test_int_abs_max_quantizer_rows():
    g = torch.Generator().manual_seed(5)
    y = 4 * torch.randn(2, 64 * 96, generator=g)
    y[1, 128:168] = 0.
    sel = lambda t: t[..., 64:224].unfold(-1, 32, 64).unflatten(-1, (1, 32))
    x = sel(y)
    for qmin, qmax in (-2, 1), (-4, 3), (-8, 7), (-128, 127):
        out = torch.empty_like(x)
        Qz.int_abs_max_quantizer(y, sel, out=out, qmin=qmin, qmax=qmax, dtype=torch.bfloat16)
        s = Qz.int_abs_max_scale(x, qmin=qmin, qmax=qmax, dtype=torch.bfloat16)
        codes = out / s
        assert torch.equal(codes, codes.round()) and codes.min() >= qmin and codes.max() <= qmax
        # the largest magnitude of each row maps to (close to) the extreme code
        assert ((codes.abs().amax(-1) >= (qmax - qmin) / 2 - 1) | (x.abs().amax(-1) == 0)).all()


# ------------------------------------------------------------------------------------------------ abs-max golden

GOLD = np.load(pathlib.Path(__file__).with_name("golden") / "absmax.npz")
PAIRS = ((-2, 1), (-4, 3), (-8, 7), (-128, 127))
SELECTORS = {  # quantizer_int.py:545-548
    "r1x32": lambda t: t[..., 64:224].unfold(-1, 32, 64).unflatten(-1, (1, 32)),
    "r2x24": lambda t: t[..., 48:552].unfold(-1, 120, 168).unfold(-1, 24, 96),
}
DTYPES = {"float32": torch.float32, "float64": torch.float64}
SCALES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _golden_cases():
    """(key, y_flat, select, qmin, qmax, scale dtype, expected) for every vector of absmax.npz."""
    for xd in DTYPES:
        y = torch.from_numpy(GOLD[f"{xd}_y"])
        for name, sel in SELECTORS.items():
            for qmin, qmax in PAIRS:
                for sd, sdt in SCALES.items():
                    key = f"{xd}_{name}_{sd}_{qmin}_{qmax}"
                    yield key, y, sel, qmin, qmax, sdt, torch.from_numpy(GOLD[key])
        mat = torch.from_numpy(GOLD[f"{xd}_mat"])
        sel = lambda t: t.unflatten(-1, (mat.numel() // 32, 1, 32))
        for qmin, qmax in PAIRS:
            for sd, sdt in SCALES.items():
                key = f"{xd}_mat_{sd}_{qmin}_{qmax}"
                yield key, mat.flatten(), sel, qmin, qmax, sdt, torch.from_numpy(GOLD[key]).reshape(-1, 1, 32)


def _golden_mismatches():
    bad = []
    for key, y, sel, qmin, qmax, sdt, expected in _golden_cases():
        out = torch.empty_like(sel(y))
        Qz.int_abs_max_quantizer(y, sel, out=out, qmin=qmin, qmax=qmax, dtype=sdt)
        if not torch.equal(out, expected):
            bad.append(key)
    return bad


def test_int_abs_max_quantizer_golden():
    """Bit for bit the reference's int_abs_max_quantizer_torch output on its own test's cases."""
    assert len(list(_golden_cases())) == 2 * (2 * 4 * 2 + 4 * 2)
    assert _golden_mismatches() == []


def test_golden_absmax_holds_exact_ties():
    """The vectors exercise exact ties k + 1/2 (with even and odd k), clamped codes, zero and 1e-38 rows."""
    ties = odd = even = clamped = 0
    for key, y, sel, qmin, qmax, sdt, expected in _golden_cases():
        x = sel(y)
        s = Qz.int_abs_max_scale(x, qmin=qmin, qmax=qmax, dtype=sdt)
        q = x / s
        t = (q - q.floor()) == .5
        ties += int(t.sum())
        odd += int((t & (q.floor().remainder(2) == 1)).sum())
        even += int((t & (q.floor().remainder(2) == 0)).sum())
        clamped += int(((q.round() > qmax) | (q.round() < qmin)).sum())
    assert ties > 10000 and odd > 1000 and even > 1000 and clamped > 0


def _check_nearest_integer(y, sel, qmin, qmax, sdt, out):
    """Nearest-integer property of abs-max codes, independent of how the oracle rounds: each code k = out / s
    is an integer in [qmin, qmax]; where the IEEE quotient q = y / s lies inside [qmin, qmax], |q - k| <= 1/2 and
    |q - k| == 1/2 only for even k; outside it, k is the bound on q's side."""
    x = sel(y)
    s = Qz.int_abs_max_scale(x, qmin=qmin, qmax=qmax, dtype=sdt)
    q = (x / s).double()
    k = (out / s).double()
    ok = torch.equal(k, k.round()) and bool((k >= qmin).all()) and bool((k <= qmax).all())
    inside = (q >= qmin) & (q <= qmax)
    d = (q - k).abs()
    ok &= bool((d[inside] <= .5).all())
    tie = inside & (d == .5)
    ok &= bool((k[tie].remainder(2) == 0).all())
    ok &= bool((k[q > qmax] == qmax).all()) and bool((k[q < qmin] == qmin).all())
    return ok


def test_int_abs_max_quantizer_nearest_integer():
    for key, y, sel, qmin, qmax, sdt, expected in _golden_cases():
        out = torch.empty_like(sel(y))
        Qz.int_abs_max_quantizer(y, sel, out=out, qmin=qmin, qmax=qmax, dtype=sdt)
        assert _check_nearest_integer(y, sel, qmin, qmax, sdt, out), key
        assert _check_nearest_integer(y, sel, qmin, qmax, sdt, expected), key


@pytest.mark.parametrize("mutant", ["floor", "trunc", "half_away"])
def test_rounding_mutants_fail(monkeypatch, mutant):
    """A mistake planted in the oracle's rounding fails both the golden vectors and the nearest-integer check."""
    planted = {
        "floor": lambda t: t.floor_(),
        "trunc": lambda t: t.trunc_(),
        "half_away": lambda t: t.copy_(torch.sign(t) * torch.floor(t.abs() + .5)),
    }[mutant]
    monkeypatch.setattr(Qz, "_round_half_even", planted)
    assert len(_golden_mismatches()) >= 16
    failed = 0
    for key, y, sel, qmin, qmax, sdt, expected in _golden_cases():
        out = torch.empty_like(sel(y))
        Qz.int_abs_max_quantizer(y, sel, out=out, qmin=qmin, qmax=qmax, dtype=sdt)
        failed += not _check_nearest_integer(y, sel, qmin, qmax, sdt, out)
    assert failed >= 16
