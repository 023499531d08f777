"""Pin the oracle's integer quantizers (CPU only).

Known answers from the reference (quantizer_int.py:476-488, 532-533), the affine closed form
re-derived entry by entry in Python float arithmetic, ties to even, and the 16-bit scale
rounding against an independent bit-level round-to-nearest-even on the fp32 pattern.
"""

import struct

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
