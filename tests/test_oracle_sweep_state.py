"""Pin the stage-by-stage form of the oracle (``TorchSweepState``) and its work count (CPU only).

``TorchSweepState.run_stage`` is the oracle of the full-size GPU parity tests and of the CPU baseline;
``stage_work`` weights the baseline's sampled stages.  Pins:
  * run stage by stage over a whole sweep, it reproduces the codes the reference itself wrote at C1
    (tests/golden/c1_int4.npz, fp32) and equals Algorithm 3 / Algorithm 1 bitwise in fp64 with NaN in the
    triangles it must not read;
  * ``stage_work`` equals a brute-force count of the entries that the stage's ``addcmul_`` calls update,
    taken by intercepting every ``addcmul_`` the stage issues (a torch function mode), and its sum over
    all stages equals the closed form of the per-stage loop.
"""

import functools

import numpy as np
import pytest
import torch
from torch.overrides import TorchFunctionMode

from oracle import algorithms as A
from oracle import quantize as Qz
from oracle import sweep as S
from test_oracle_golden import c1_inputs


def test_run_stage_reproduces_reference_c1_codes():
    """Stage by stage at C1 (512 x 512 fp32, INT4 per-row): the reference's own codes, up to near-ties on a
    CPU with other vector units (<= 0.01%, |frac - 0.5| < 1e-3)."""
    cfg, data, x, l, u, scale, zp = c1_inputs()
    q = functools.partial(Qz.affine_quantizer, qmin=cfg.qmin, qmax=cfg.qmax)
    st = S.TorchSweepState(x, l, u, quantizer=q, quantizer_inputs=(scale, zp))
    assert st.stages == 1023
    for s in range(st.stages):
        st.run_stage(s)
    codes = torch.round(st.y / scale).to(torch.int8).numpy()
    mism = codes != data["codes"]
    assert mism.mean() <= 1e-4, mism.sum()
    if mism.any():
        frac = np.abs(np.abs(data["ypre_codes"] - np.floor(data["ypre_codes"])) - .5)
        assert (frac[mism] < 1e-3).all()


@pytest.mark.parametrize("m,n", [(1, 1), (1, 9), (9, 1), (13, 5), (5, 13), (24, 40)])
def test_run_stage_equals_alg1_fp64(m, n):
    """Stage by stage in fp64 with a coordinate-dependent codebook: equal to Algorithm 1 on vec(X) (Theorem 1)
    and to Algorithm 3, with NaN in the triangles of L and U that must not be read."""
    Am, Bm, X = A.random_instance((m, n), 7 * m + n)
    L, U = A.feedback_factors(Am, Bm)
    zref = A.vectorized_alg1(X, Am, Bm, Q=A.coordinate_round)
    ln, un = L.clone(), U.clone()
    ln[torch.ones(m, m, dtype=torch.bool).triu()] = torch.nan
    un[torch.ones(n, n, dtype=torch.bool).tril()] = torch.nan

    def coord(y_flat, sl, *, out):
        idx = torch.arange(sl.start, sl.stop, sl.step)
        out.copy_(A.coordinate_round(y_flat[sl], idx // n, idx % n))

    st = S.TorchSweepState(X, ln, un, quantizer=coord)
    for s in range(st.stages):
        st.run_stage(s)
    assert st.y.equal(zref)
    assert st.y.equal(A.alg3(X, L, U, Q=A.coordinate_round))


class _AddcmulCount(TorchFunctionMode):
    """Counts the entries every in-place ``addcmul_`` updates (the size of the tensor it writes)."""

    def __init__(self):
        super().__init__()
        self.entries = 0
        self.calls = 0

    def __torch_function__(self, func, types, args=(), kwargs=None):
        if getattr(func, "__name__", "") == "addcmul_":
            self.entries += args[0].numel()
            self.calls += 1
        return func(*args, **(kwargs or {}))


@pytest.mark.parametrize("m,n", [(1, 1), (1, 6), (6, 1), (7, 7), (5, 11), (11, 5), (32, 20)])
def test_stage_work_brute_force(m, n):
    g = torch.Generator().manual_seed(m * 31 + n)
    x = torch.randn(m, n, generator=g)
    l = torch.randn(m, m, generator=g).tril(-1)
    u = torch.randn(n, n, generator=g).triu(1)
    st = S.TorchSweepState(x, l, u)
    total = 0
    for s in range(st.stages):
        with _AddcmulCount() as cnt:
            st.run_stage(s)
        assert cnt.calls == 3
        assert cnt.entries == S.stage_work(m, n, s), s
        total += cnt.entries
    # closed form: stage s has d_s entries with rows i_lo.. and columns j_lo..; summed over the antidiagonals
    # every entry (i, j) is a source once, pushing to the m - i_lo(i + j) rows below its stage's first row
    # twice (C and Y) and to the n - j_lo(i + j) columns right of its stage's first column once
    closed = 0
    for i in range(m):
        for j in range(n):
            s = i + j
            i_lo, j_lo = max(0, s - n + 1), max(0, s - m + 1)
            closed += 2 * (m - i_lo) + (n - j_lo)
    assert total == closed


@pytest.mark.parametrize("m,n", [(13, 5), (9, 16), (24, 40)])
def test_transposed_layer_is_the_same_rounding(m, n):
    """The yardstick of the full-size free-running comparison: the sweep of X^T with L' = U^T and U' = L^T (rows
    and columns exchanged) rounds exactly as the sweep of X, transposed, in fp64 with a coordinate-dependent
    codebook; in fp32 only the summation order differs."""
    Am, Bm, X = A.random_instance((m, n), 3 * m + n)
    L, U = A.feedback_factors(Am, Bm)

    def coord(transposed):
        def q(y_flat, sl, *, out):
            idx = torch.arange(sl.start, sl.stop, sl.step)
            i, j = (idx % m, idx // m) if transposed else (idx // n, idx % n)
            out.copy_(A.coordinate_round(y_flat[sl], i, j))
        return q

    z = S.gptq_2d_torch(X, L, U, quantizer=coord(False))
    zt = S.gptq_2d_torch(X.t().contiguous(), U.t().contiguous(), L.t().contiguous(), quantizer=coord(True))
    assert zt.t().equal(z)
