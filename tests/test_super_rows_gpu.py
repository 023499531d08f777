"""GPU tests of the fused sweep over 1 x 32 super-entries (one super-entry per tile row).

fp64: the fused engine equals the CPU oracle's super-entry Algorithm 3 (gptq_2d_reference.py:360-382,
restated in oracle/algorithms.py) exactly, with NaN in every entry of L and U the reference must not read
(L on and above its diagonal, U on and below its 32 x 32 block diagonal), for the abs-max INT quantizer of
quantizer_int.py:120-134 with bf16 and fp16 scales and for the per-entry quantizers; and it equals the
per-stage plug-in engine bit for bit.  fp32: with every stage forced to the fp64 run's values, each entry's
Y before rounding stays within 1e-4 of the fp64 trajectory (values are O(10)).
"""

import functools

import pytest
import torch

import gptq_2d as G
import quantizer_int as QI
from oracle import algorithms as A
from oracle import quantize as OQ
from oracle import sweep as S

pytestmark = pytest.mark.gpu
DEV = "cuda"
SE = (1, 32)


def _instance(m, n, seed, batch=()):
    g = torch.Generator().manual_seed(seed)
    x = 4. * torch.randn(*batch, m, n, generator=g, dtype=torch.float64)
    l = .3 / m ** .5 * torch.randn(m, m, generator=g, dtype=torch.float64)
    u = .3 / n ** .5 * torch.randn(n, n, generator=g, dtype=torch.float64)
    blk = torch.arange(n) // 32
    l[torch.ones(m, m, dtype=torch.bool).triu()] = torch.nan
    u[blk[None, :] <= blk[:, None]] = torch.nan
    return x, l, u


def _oracle(x, l, u, q):
    lu = S.unit_triangular(l, False, 1)
    uu = S.unit_triangular(u, True, 32)
    return A.alg3_super_entry(x, lu, uu, Q=q, super_entry_shape=SE)


def _absmax_q(dtype):
    def q(y, i, j):
        out = torch.empty_like(y)
        OQ.int_abs_max_quantizer(y, lambda t: t, out=out, qmin=-8, qmax=7, dtype=dtype)
        return out
    return q


@pytest.mark.parametrize("m,n", [(32, 32), (64, 96), (70, 64), (33, 160), (100, 128)])
@pytest.mark.parametrize("dtype16", [torch.bfloat16, torch.float16])
def test_absmax_rows_fp64_exact(m, n, dtype16):
    print(f"rows abs-max {m}x{n} scale {dtype16}", flush=True)
    x, l, u = _instance(m, n, 7 * m + n)
    expected = _oracle(x, l, u, _absmax_q(dtype16))
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=-8, qmax=7, dtype=dtype16)
    for outer in (32, 64, 1024):
        got = G.gptq_2d_super_entry(x.to(DEV), l.to(DEV), u.to(DEV), super_entry_shape=SE, quantizer=q,
                                    outer_block_size=outer, fused=True)
        assert got.cpu().equal(expected), outer
    plug = G.gptq_2d_super_entry(x.to(DEV), l.to(DEV), u.to(DEV), super_entry_shape=SE, quantizer=q, fused=False)
    assert plug.cpu().equal(expected)


@pytest.mark.parametrize("kind", ["round", "affine"])
def test_per_entry_rows_fp64_exact(kind):
    m, n = 70, 128
    x, l, u = _instance(m, n, 3)
    g = torch.Generator().manual_seed(4)
    if kind == "round":
        q, qi = QI.round_quantizer_super_entry, ()
        oq = lambda y, i, j: torch.round(y)
    else:
        scale = (0.5 + torch.rand(m, n, generator=g, dtype=torch.float64))
        zp = torch.randint(-2, 3, (m, n), generator=g).double()
        q, qi = functools.partial(QI.affine_quantizer_super_entry_hip, qmin=-8, qmax=7), (scale.to(DEV), zp.to(DEV))
        s4, z4 = scale.reshape(m, 1, n // 32, 32), zp.reshape(m, 1, n // 32, 32)

        def oq(y, i, j):
            sc, zz = s4[i[:, 0, 0], :, j[:, 0, 0], :], z4[i[:, 0, 0], :, j[:, 0, 0], :]
            return (torch.clamp(torch.round(y / sc + zz), -8, 7) - zz) * sc
    expected = _oracle(x, l, u, oq)
    got = G.gptq_2d_super_entry(x.to(DEV), l.to(DEV), u.to(DEV), super_entry_shape=SE, quantizer=q,
                                quantizer_inputs=qi, outer_block_size=64, fused=True)
    assert got.cpu().equal(expected)


def test_absmax_rows_batched():
    """Broadcast batch: every batch entry equals its own call."""
    x, l, u = _instance(40, 96, 11, batch=(3,))
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=-4, qmax=3, dtype=torch.bfloat16)
    both = G.gptq_2d_super_entry(x.to(DEV), l.to(DEV), u.to(DEV), super_entry_shape=SE, quantizer=q, fused=True)
    for b in range(3):
        one = G.gptq_2d_super_entry(x[b].to(DEV), l.to(DEV), u.to(DEV), super_entry_shape=SE, quantizer=q,
                                    fused=True)
        assert both[b].equal(one)


@pytest.mark.parametrize("m,n", [(300, 640), (1024, 1024)])
def test_absmax_rows_fp32_trajectory(m, n):
    print(f"rows fp32 trajectory {m}x{n}", flush=True)
    g = torch.Generator().manual_seed(m + n)
    x = (4. * torch.randn(m, n, generator=g, dtype=torch.float64)).to(DEV)
    lo = S.unit_triangular(.3 / m ** .5 * torch.randn(m, m, generator=g, dtype=torch.float64), False).to(DEV)
    up = S.unit_triangular(.3 / n ** .5 * torch.randn(n, n, generator=g, dtype=torch.float64), True, 32).to(DEV)
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=-8, qmax=7, dtype=torch.bfloat16)
    run = functools.partial(G.gptq_2d_super_entry, super_entry_shape=SE, outer_block_size=256, fused=True)
    z64 = run(x, lo, up, quantizer=q)
    pre64 = torch.full_like(x, float("nan"))
    assert run(x, lo, up, quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z64, pre64)).equal(z64)
    pre32 = torch.full_like(x, float("nan"), dtype=torch.float32)
    z32 = run(x.float(), lo.float(), up.float(), quantizer=QI.teacher_forced_quantizer,
              quantizer_inputs=(z64.float(), pre32))
    assert z32.equal(z64.float())
    err = (pre32.double() - pre64).abs()
    assert not err.isnan().any()
    print(f"  max |dY| {err.max().item():.2e}", flush=True)
    assert err.max().item() < 1e-4
