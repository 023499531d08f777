"""GPU tests of the HIP integer quantizer plug-ins, following quantizer_int.py:473-553 of the reference,
checked against the CPU oracle and the golden scale vectors."""

import pathlib

import numpy as np
import pytest
import torch

import quantizer_int as QI
from oracle import quantize as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def test_affine_known_answers():
    y = torch.zeros(3, 3, dtype=torch.float64, device=DEV)
    scale, zp = torch.ones_like(y), torch.zeros_like(y)
    y[0, 2], y[1, 1], y[2, 0] = .5, 1.75, -9.
    scale[1, 1], scale[2, 0], zp[2, 0] = .5, 2., 1.
    for kw, expected in (({}, [0., 2., -10.]), (dict(qmin=-2, qmax=2), [0., 1., -6.])):
        for fn in (QI.affine_quantizer_hip, QI.affine_quantizer_torch):
            out = torch.empty(3, dtype=torch.float64, device=DEV)
            fn(y.flatten(), slice(2, 8, 2), scale, zp, out=out, **kw)
            assert out.tolist() == expected


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_affine_broadcasting(dtype):
    g = torch.Generator().manual_seed(0)
    y = 4. * torch.randn(2, 3, 35, generator=g, dtype=dtype)
    scale = .1 + torch.rand(1, 5, 7, generator=g, dtype=dtype)
    zp = torch.randint(-2, 3, (2, 1, 5, 7), generator=g).to(dtype)
    sl = slice(6, 36, 6)
    expected = torch.empty(2, 3, 5, dtype=dtype)
    OQ.affine_quantizer(y, sl, scale, zp, out=expected, qmin=-3, qmax=4)
    out = torch.empty(2, 3, 5, dtype=dtype, device=DEV)
    QI.affine_quantizer_hip(y.to(DEV), sl, scale.to(DEV), zp.to(DEV), out=out, qmin=-3, qmax=4)
    assert out.cpu().equal(expected)


def test_affine_super_entry():
    g = torch.Generator().manual_seed(0)
    y = 4. * torch.randn(2, 3, 24, generator=g, dtype=torch.float64)
    scale = .1 + torch.rand(1, 4, 6, generator=g, dtype=torch.float64)
    zp = torch.randint(-2, 3, (2, 1, 4, 6), generator=g).double()
    select = lambda x: x[..., 3:21].unfold(-1, 9, 9).unfold(-1, 3, 6)
    expected = torch.empty_like(y)
    OQ.affine_quantizer(y, slice(0, 24, 1), scale, zp, out=expected, qmin=-3, qmax=4)
    out = torch.empty(2, 3, 2, 2, 3, dtype=torch.float64, device=DEV)
    QI.affine_quantizer_super_entry_hip(y.to(DEV), select, scale.to(DEV), zp.to(DEV), out=out, qmin=-3, qmax=4)
    assert out.cpu().equal(select(expected))


def test_round_plugins():
    g = torch.Generator().manual_seed(1)
    y = 4 * torch.randn(3, 64 * 96, generator=g)
    y[0, :8] = torch.tensor([.5, 1.5, 2.5, -.5, -1.5, 2.4999995, 2.5000005, 0.])
    out = torch.empty(3, 64, device=DEV)
    QI.round_quantizer(y.to(DEV), slice(0, 64 * 97, 97), out=out)
    assert out.cpu().equal(torch.round(y[..., 0:64 * 97:97]))
    sel = lambda t: t[..., 48:552].unfold(-1, 120, 168).unfold(-1, 24, 96)
    out = torch.empty(3, 3, 2, 24, device=DEV)
    QI.round_quantizer_super_entry(y.to(DEV), sel, out=out)
    assert out.cpu().equal(torch.round(sel(y)))


def test_int_abs_max_scale_golden():
    data = np.load(GOLDEN / "scales.npz")
    keys = sorted(k[:-2] for k in data.files if k.endswith("_x"))
    for key in keys:
        _, sd, qmin, qmax = key.split("_")
        dtype = torch.bfloat16 if "bfloat16" in sd else torch.float16
        x = torch.from_numpy(data[key + "_x"]).to(DEV)
        s = QI.int_abs_max_scale_hip(x, qmin=int(qmin), qmax=int(qmax), dtype=dtype)
        assert np.array_equal(s.cpu().numpy(), data[key + "_s"]), key


def test_int_abs_max_quantizer():
    g = torch.Generator().manual_seed(5)
    y = 4. * torch.randn(2, 64 * 96, generator=g)
    y[1, 128:168] = 0.
    y[0, 192:224] *= 1e-38
    for select in (lambda x: x[..., 64:224].unfold(-1, 32, 64).unflatten(-1, (1, 32)),
                   lambda x: x[..., 48:552].unfold(-1, 120, 168).unfold(-1, 24, 96)):
        x = select(y)
        for qmin, qmax in (-2, 1), (-4, 3), (-8, 7), (-128, 127):
            for dtype in torch.float16, torch.bfloat16:
                expected = torch.empty_like(x)
                OQ.int_abs_max_quantizer(y, select, out=expected, qmin=qmin, qmax=qmax, dtype=dtype)
                out = torch.empty(x.shape, device=DEV)
                QI.int_abs_max_quantizer_hip(y.to(DEV), select, out=out, qmin=qmin, qmax=qmax, dtype=dtype)
                assert out.cpu().equal(expected), (qmin, qmax, dtype)
