"""GPU tests of the abs-max INT quantizer against vectors the reference wrote (tests/golden/absmax.npz).

The vectors are ``int_abs_max_quantizer_torch`` (quantizer_int.py:120-134) on the cases of the reference's
own test (quantizer_int.py:535-553): 1 x 32 and 2 x 24 selectors, four (qmin, qmax) pairs, fp16 and bf16
scales, a zero row, a 1e-38 row, and rows of exact ties k + 1/2.  The HIP plug-in must equal them bit for
bit, and so must the fused 1 x 32 row sweep (``gptq_2d_super_entry`` with ``fused=True``) and the plug-in
engine on a 48 x 96 matrix whose feedback factors are zero where they are read (L strictly below its
diagonal, U strictly above its 32 x 32 block diagonal; NaN everywhere else), so that the sweep's output
is the quantizer of the input.  With zero feedback the fused sweep's errors and column errors are also
exactly the rounded differences z - y of the quantizer's rounded output: the affine quantizer's
dequantized value is rounded on its own before the subtraction, as the plug-in rounds it.
"""

import functools
import pathlib
from fractions import Fraction

import numpy as np
import pytest
import torch

import _hip
import gptq_2d as G
import quantizer_int as QI

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "absmax.npz")
PAIRS = ((-2, 1), (-4, 3), (-8, 7), (-128, 127))
SELECTORS = {
    "r1x32": lambda t: t[..., 64:224].unfold(-1, 32, 64).unflatten(-1, (1, 32)),
    "r2x24": lambda t: t[..., 48:552].unfold(-1, 120, 168).unfold(-1, 24, 96),
}
DTYPES = {"float32": torch.float32, "float64": torch.float64}
SCALES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def _zero_feedback(m, n, dtype):
    """L, U with zeros wherever the sweep reads them and NaN everywhere else."""
    l = torch.full((m, m), float("nan"), dtype=dtype)
    l[torch.ones(m, m, dtype=torch.bool).tril(-1)] = 0.
    blk = torch.arange(n) // 32
    u = torch.full((n, n), float("nan"), dtype=dtype)
    u[blk[None, :] > blk[:, None]] = 0.
    return l.to(DEV), u.to(DEV)


@pytest.mark.parametrize("xd", list(DTYPES))
def test_plugin_equals_reference_vectors(xd):
    y = torch.from_numpy(GOLD[f"{xd}_y"]).to(DEV)
    for name, sel in SELECTORS.items():
        x = sel(y)
        for qmin, qmax in PAIRS:
            for sd, sdt in SCALES.items():
                key = f"{xd}_{name}_{sd}_{qmin}_{qmax}"
                out = torch.empty(x.shape, dtype=x.dtype, device=DEV)
                QI.int_abs_max_quantizer_hip(y, sel, out=out, qmin=qmin, qmax=qmax, dtype=sdt)
                assert np.array_equal(out.cpu().numpy(), GOLD[key]), key


@pytest.mark.parametrize("xd", list(DTYPES))
@pytest.mark.parametrize("fused", [True, False])
def test_row_sweeps_equal_reference_vectors(xd, fused):
    mat = torch.from_numpy(GOLD[f"{xd}_mat"]).to(DEV)
    m, n = mat.shape
    l, u = _zero_feedback(m, n, mat.dtype)
    for qmin, qmax in PAIRS:
        for sd, sdt in SCALES.items():
            key = f"{xd}_mat_{sd}_{qmin}_{qmax}"
            q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=qmin, qmax=qmax, dtype=sdt)
            got = G.gptq_2d_super_entry(mat, l, u, super_entry_shape=(1, 32), quantizer=q, fused=fused,
                                        outer_block_size=64)
            assert np.array_equal(got.cpu().numpy(), GOLD[key]), key


def _fused_rows_c_e(x, l, u, kind, qa=None, qb=None, qmin=0., qmax=0., dtype16=0):
    """Run the fused 1 x 32 row sweep through the C ABI and return (Y, C, E, Y before rounding)."""
    m, n = x.shape
    y = x.clone()
    c = torch.empty_like(y)
    e = torch.empty_like(y)
    ypre = torch.full_like(y, float("nan"))
    bs = torch.Size([])
    _hip.call("sweep_fused_se", y.dtype, _hip.ptr(y), _hip.ptr(c), _hip.ptr(e), _hip.ptr(l), _hip.ptr(u), m, n, 1,
              32, 0, _hip.i64_array(bs), _hip.batch_strides(l, bs), _hip.batch_strides(u, bs), kind, _hip.ptr(qa),
              _hip.batch_strides(qa, bs) if qa is not None else None, _hip.ptr(qb),
              _hip.batch_strides(qb, bs) if qb is not None else None, qmin, qmax, dtype16, _hip.ptr(ypre), None, 2,
              0, -1, _hip.stream(y.device))
    torch.cuda.synchronize()
    return y, c, e, ypre


@pytest.mark.parametrize("kind", ["affine", "absmax"])
def test_fused_rows_errors_are_rounded_differences(kind):
    """fp64, zero feedback: E = C = RN(z - y) with z the plug-in's output, bit for bit (no contraction of the
    dequantization into the error), and Y before rounding is the input."""
    m, n = 64, 128
    g = torch.Generator().manual_seed(21)
    x = (4. * torch.randn(m, n, generator=g, dtype=torch.float64)).to(DEV)
    l, u = _zero_feedback(m, n, torch.float64)
    if kind == "affine":
        scale = (.3 + torch.rand(m, n, generator=g, dtype=torch.float64)).to(DEV)
        zp = torch.randint(-3, 4, (m, n), generator=g).double().to(DEV)
        y, c, e, ypre = _fused_rows_c_e(x, l, u, 1, scale, zp, -8., 7.)
        z = torch.empty_like(x)
        QI.affine_quantizer_hip(x.flatten(), slice(0, m * n, 1), scale, zp, out=z.view(-1), qmin=-8, qmax=7)
        # the check can see a contraction only where (code - zp) s is inexact: count the entries where
        # fma(code - zp, s, -y) (exact in fractions, rounded once) differs from RN(RN((code - zp) s) - y)
        zc, xc, sc = z.cpu().flatten()[:512], x.cpu().flatten()[:512], scale.cpu().flatten()[:512]
        visible = 0
        for zi, xi, si in zip(zc.tolist(), xc.tolist(), sc.tolist()):
            code_zp = round(zi / si)  # z = (code - zp) s with a small integer code - zp
            fused = float(Fraction(code_zp) * Fraction(si) - Fraction(xi))
            visible += fused != zi - xi
        assert visible > 10
    else:
        y, c, e, ypre = _fused_rows_c_e(x, l, u, 3, qmin=-8., qmax=7., dtype16=1)
        z = torch.empty(m * n // 32, 1, 32, dtype=x.dtype, device=DEV)
        QI.int_abs_max_quantizer_hip(x.flatten(), lambda t: t.unflatten(-1, (m * n // 32, 1, 32)), out=z, qmin=-8,
                                     qmax=7, dtype=torch.bfloat16)
        z = z.reshape(m, n)
    assert y.equal(z)
    assert ypre.equal(x)
    diff = (z.cpu() - x.cpu())  # IEEE subtraction on the host
    assert e.cpu().equal(diff)
    assert c.cpu().equal(diff)
