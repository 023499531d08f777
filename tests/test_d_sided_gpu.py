"""GPU tests of the D-sided sweep (gptq_d_sided): the rounding of X [n_1, ..., n_D] under a Kronecker
Hessian, whose reference is the CPU listing of Algorithm 4 (gptq_2d_reference.py:270-294).

fp64: equal bit for bit to the oracle's alg4 (itself pinned against Algorithm 1 on vec(X) in the CPU
suite) for D = 3 shapes that cross the engine's 32 x 32 tiles, D = 2 and D = 4, with NaN above every
factor's diagonal, on the fused engine (round-to-nearest and a per-entry affine codebook whose scales
depend on every coordinate) and on the per-stage plug-in engine.

fp32 at full size: C5a's three-factor layer as the 8192 x 112 x 256 tensor X[i, b1, b2] under
ldl_of_inverse of A, B1, B2 with static INT4 abs-max scales per 32 consecutive b2 (bf16): deterministic, codes
on the grid, each output the affine quantizer of its own pre-rounding value, objective below rounding
without feedback, the first hyper-antidiagonals (a crop holding every entry they depend on) in
agreement with the oracle's alg4, and 24 whole rows of the two-sided view whose pre-rounding values equal
Algorithm 3's recomputed in fp64 from the engine's own errors.
"""

import functools
import time

import pytest
import torch

import gptq_2d_ldl as LDL
import gptq_d_sided as DS
import instances
import quantizer_int as QI
from oracle import algorithms as A
from oracle import sweep as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _instance(shape, seed):
    *bases, x = A.random_instance(shape, seed)
    ls = [A.ldl_of_inverse(b.t() @ b) for b in bases]
    g = torch.Generator().manual_seed(seed + 1)
    scale = 2. ** torch.randint(-1, 2, shape, generator=g).double()
    return x, ls, scale


def _poisoned(ls):
    return [f.masked_fill(torch.ones_like(f, dtype=torch.bool).triu(), torch.nan) for f in ls]


SHAPES = [(3, 4, 5), (6, 2, 3), (1, 5, 4), (4, 1, 1), (33, 40, 7), (40, 3, 50), (70, 5, 13), (64, 32, 2),
          (5, 7), (2, 3, 2, 3), (9, 4, 3, 5)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("kind", ["round", "affine"])
def test_d_sided_fp64_equals_alg4(shape, kind):
    print(f"d-sided {shape} {kind}", flush=True)
    x, ls, scale = _instance(shape, sum(shape) + len(shape))
    if kind == "round":
        expected = A.alg4(x, ls)
        q, qi = QI.round_quantizer, ()
    else:
        def oq(y, *idx):
            s = scale[idx]
            return torch.clamp(torch.round(y / s), -3., 2.) * s
        expected = A.alg4(x, ls, Q=oq)
        q = functools.partial(QI.affine_quantizer_hip, qmin=-3., qmax=2.)
        qi = (scale.to(DEV), torch.zeros(shape, dtype=torch.float64, device=DEV))
    lg = [f.to(DEV) for f in _poisoned(ls)]
    for fused, outer in ((None, 32), (None, 1024), (False, 64)):
        got = DS.gptq_d_sided(x.to(DEV), lg, quantizer=q, quantizer_inputs=qi, outer_block_size=outer, fused=fused)
        assert got.shape == x.shape and got.is_contiguous()
        assert got.cpu().equal(expected), (fused, outer)


def test_d_sided_inplace():
    """inplace writes the result into x, both when x's memory is in the flattened order (the sweep runs on it
    directly) and when it is not; quantizer inputs in that order are read without a copy."""
    shape = (20, 9, 6)
    x, ls, _ = _instance(shape, 3)
    expected = A.alg4(x, ls)
    lg = [f.to(DEV) for f in _poisoned(ls)]
    xa = x.to(DEV)
    assert DS.gptq_d_sided(xa, lg, inplace=True) is xa and xa.cpu().equal(expected)
    xb = x.permute(0, 2, 1).contiguous().to(DEV).permute(0, 2, 1)  # memory order [n1, n3, n2]
    ptr = xb.data_ptr()
    assert DS.gptq_d_sided(xb, lg, inplace=True) is xb and xb.data_ptr() == ptr and xb.cpu().equal(expected)
    xc = x.to(DEV)
    DS.gptq_d_sided(xc, lg)
    assert xc.cpu().equal(x), "x changed without inplace"


def test_d_sided_empty():
    x = torch.empty(0, 3, 4, dtype=torch.float64, device=DEV)
    ls = [torch.eye(k, dtype=torch.float64, device=DEV) for k in x.shape]
    assert DS.gptq_d_sided(x, ls).shape == x.shape


def _gpu_factor(k, alpha, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    s = torch.arange(1, 4 * k + 1, device=DEV, dtype=torch.float64) ** (-alpha)
    g = torch.randn(k, 4 * k, generator=gen, device=DEV, dtype=torch.float64)
    f = (g * s) @ g.t() / (4 * k)
    f.diagonal().add_(1e-2)
    return f


def test_c5a_three_sided_full_size():
    cfg = instances.THREE_FACTOR["C5a"]
    m, n1, n2, grp = cfg.m, cfg.n1, cfg.n2, cfg.group
    print(f"C5a three-sided: {m}x{n1}x{n2}, static INT4 abs-max scale per {grp} b2 (bf16)", flush=True)
    x = instances.weights(m, n1 * n2, cfg.seeds[0], True, False).float().view(m, n1, n2).to(DEV)
    a, b1, b2 = _gpu_factor(m, cfg.alpha, 21), _gpu_factor(n1, cfg.alpha, 23), _gpu_factor(n2, cfg.alpha, 24)
    ls = [LDL.ldl_of_inverse(f.float()) for f in (a, b1, b2)]
    scale = instances.abs_max_group_scale(x, grp, cfg.qmin, cfg.qmax)
    zero = torch.zeros_like(x)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    run = functools.partial(DS.gptq_d_sided, x, ls, outer_block_size=1024)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    z = run(quantizer=q, quantizer_inputs=(scale, zero))
    torch.cuda.synchronize()
    print(f"  sweep {1e3 * (time.perf_counter() - t0):.1f} ms (first call)", flush=True)
    assert run(quantizer=q, quantizer_inputs=(scale, zero)).equal(z), "not deterministic"
    codes = z / scale
    assert torch.equal(codes, codes.round()) and codes.min() >= cfg.qmin and codes.max() <= cfg.qmax

    def affine(v):
        return torch.clamp(torch.round(v / scale), cfg.qmin, cfg.qmax) * scale

    # pre-rounding values captured in the flattened memory order [m, n2, n1], so the quantizer writes them
    pre = torch.full((m, n2, n1), float("nan"), device=DEV).permute(0, 2, 1)
    assert run(quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre)).equal(z)
    assert not pre.isnan().any()
    assert torch.equal(affine(pre), z), "outputs are not the quantizer of their own pre-rounding values"
    # every entry of 24 rows spread over the layer, on the two-sided view the sweep runs (columns b1 + n1 b2, U =
    # (L_B2 (x) L_B1)^T): the pre-rounding values equal Algorithm 3's, recomputed in fp64 by torch from the
    # engine's own errors, and their rounding gives the engine's codes
    flat = lambda t: t.permute(0, 2, 1).reshape(m, -1)
    rows = torch.linspace(0, m - 1, 24, device=DEV).round().long()
    y64 = A.alg3_pre_rounding(flat(x), ls[0], DS.column_factor(ls), flat(z), flat(pre), (1, 1), rows)
    dy = (y64 - flat(pre)[rows].double()).abs()
    rel = float(dy.max() / y64.abs().max())
    sr = flat(scale)[rows]
    agree = float((torch.clamp(torch.round(y64.float() / sr), cfg.qmin, cfg.qmax) * sr == flat(z)[rows]).double().mean())
    print(f"  {rows.numel()} rows ({rows.numel() * n1 * n2} entries): max |Y_pre - Y_alg3(fp64)| {dy.max():.2e} "
          f"({rel:.2e} of max |Y|), codes of the fp64 values agree in {agree:.6%}", flush=True)
    assert rel < 5e-6 and agree >= 0.9999
    del pre, codes, y64, dy

    def objective(zz):
        r = (zz - x).double()
        rb = torch.matmul(b1.t(), torch.matmul(r, b2))
        return float(((a @ r.view(m, -1)) * rb.view(m, -1)).sum())

    ratio = objective(z) / objective(affine(x))
    print(f"  objective / no-feedback rounding = {ratio:.4f}", flush=True)
    assert ratio < 1.

    K = (48, 8, 32)
    crop = tuple(slice(0, k) for k in K)
    lc = [f[:k, :k].cpu() for f, k in zip(ls, K)]
    sc = scale[crop].cpu()

    def oq(y, *idx):
        s = sc[idx]
        return torch.clamp(torch.round(y / s), cfg.qmin, cfg.qmax) * s

    zo = A.alg4(x[crop].cpu(), [S.unit_triangular(f, False) for f in lc], Q=oq)
    agree = float((z[crop].cpu() == zo).double().mean())
    print(f"  crop {K} ({zo.numel()} entries, {sum(K) - 2} hyper-antidiagonals): agreement with alg4 "
          f"{agree:.6%}", flush=True)
    assert agree >= 0.999
