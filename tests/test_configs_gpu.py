"""Parity of the benchmark configurations on the GPU (the layer shapes and quantizers of C2-C5 and H).

At full size the CPU oracle cannot run the whole sweep in a test, so the full-size tests use the
oracle where it is cheap -- the first antidiagonals, which span the first outer block and the
first outer flush (only the first rows of U and columns of L are touched there) -- and
size-independent properties everywhere: valid codes, bitwise determinism, and an objective below
round-to-nearest.  The reduced-size tests run the reference's whole algorithm in fp64, where the
codes must be equal.

Factors here are Wishart-like as in the benchmark definition, F = G diag(i^-alpha) G^T / (4k) +
1e-2 I, but G is drawn with torch's GPU generator (the numpy PCG64 draws of the benchmark's
generator take seconds at these sizes); both sides of every comparison use the same L and U.
"""

import functools

import pytest
import torch

import gptq_2d as G
import gptq_2d_ldl as LDL
import instances
import quantizer_int as QI
import quantizer_trellis as QT
from oracle import algorithms as A
from oracle import quantize as OQ
from oracle import sweep as S
from oracle import trellis as OT

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gpu_factor(k, alpha, seed, dtype=torch.float64):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    s = torch.arange(1, 4 * k + 1, device=DEV, dtype=torch.float64) ** (-alpha)
    f = torch.zeros(k, k, device=DEV, dtype=torch.float64)
    for c0 in range(0, 4 * k, 4096):
        g = torch.randn(k, min(4096, 4 * k - c0), generator=gen, device=DEV, dtype=torch.float64)
        f.addmm_(g * s[c0:c0 + g.size(1)], g.t())
        del g
    f /= 4 * k
    f.diagonal().add_(1e-2)
    return f.to(dtype)


def _objective(z, x, a, b):
    r = (z - x).double()
    return float(((a.double() @ r) * (r @ b.double())).sum())


# ------------------------------------------------------------------------------------------------ full size

@pytest.mark.parametrize("name", ["C2", "C3", "H"])
def test_full_size_layer(name):
    """C2 (4096^2 INT4 asymmetric g128), C3 (14336 x 4096 INT3 per-row), H (8192^2 INT4 per-row), fp32 fused
    engine.  Oracle check on the first 640 antidiagonals (first outer block, its flush into the next block,
    and in-block pulls): with those stages teacher-forced to the oracle's codes, the engine's Y before
    rounding agrees with the oracle's to 1e-4 code units and its own rounding reproduces the oracle's codes
    except at near-ties |frac - 0.5| < 1e-5.  Whole layer: codes in range and on the grid, bitwise identical
    on a second run, objective tr(R^T A R B) below round-to-nearest's."""
    cfg = instances.CONFIGS[name]
    m, n = cfg.m, cfg.n
    print(f"{name}: {m}x{n} qmin={cfg.qmin} qmax={cfg.qmax}", flush=True)
    x = instances.weights(m, n, cfg.seeds[0], cfg.outliers, cfg.bf16).float().to(DEV)
    a = _gpu_factor(m, cfg.alpha, 11)
    b = _gpu_factor(n, cfg.alpha, 12)
    lo, up = LDL.feedback_factors_of_grams(a.float(), b.float())
    scale, zp = instances.quantizer_inputs(cfg, x)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    z = G.gptq_2d(x, lo, up, quantizer=q, quantizer_inputs=(scale, zp))
    z2 = G.gptq_2d(x, lo, up, quantizer=q, quantizer_inputs=(scale, zp))
    torch.cuda.synchronize()
    assert z.equal(z2), "not deterministic"
    codes = torch.round(z / scale + zp)
    assert codes.min() >= cfg.qmin and codes.max() <= cfg.qmax
    assert torch.equal(z, (codes - zp) * scale), "values off the quantization grid"
    rtn = (torch.clamp(torch.round(x / scale + zp), cfg.qmin, cfg.qmax) - zp) * scale
    ratio = _objective(z, x, a, b) / _objective(rtn, x, a, b)
    print(f"  objective / RTN = {ratio:.4f}", flush=True)
    assert ratio < 1.

    # oracle on the first antidiagonals (CPU, fp32, the reference's own operation sequence)
    stages = 640
    pre_o = torch.full((m, n), float("nan"))

    def spy(y_flat, sl, sc, zz, *, out):
        pre_o.view(-1)[sl] = y_flat[sl]
        OQ.affine_quantizer(y_flat, sl, sc, zz, out=out, qmin=cfg.qmin, qmax=cfg.qmax)

    st = S.TorchSweepState(x.cpu(), lo.cpu(), up.cpu(), quantizer=spy, quantizer_inputs=(scale.cpu(), zp.cpu()))
    for s in range(stages):
        st.run_stage(s)
    early = (torch.arange(m)[:, None] + torch.arange(n)[None, :]) < stages
    values = torch.where(early.to(DEV), st.y.to(DEV), z)
    pre_e = torch.full_like(x, float("nan"))
    zf = G.gptq_2d(x, lo, up, quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(values, pre_e))
    assert zf.equal(values)
    sc = scale.cpu()[early]
    ye, yo = (pre_e.cpu()[early] / sc + zp.cpu()[early]), (pre_o[early] / sc + zp.cpu()[early])
    assert not ye.isnan().any() and not yo.isnan().any()
    dev = (ye - yo).abs()
    own = ye.round().clamp(cfg.qmin, cfg.qmax)
    ref = (st.y[early] / sc + zp.cpu()[early]).round()
    mism = own != ref
    frac = (ye - ye.floor() - .5).abs()
    print(f"  first {stages} antidiagonals ({int(early.sum())} entries): max |dY| {dev.max():.2e} code units, "
          f"own-rounding mismatches {int(mism.sum())}", flush=True)
    assert dev.max() < 1e-4
    assert (frac[mism] < 1e-5).all()


def test_c5b_batch_capture():
    """C5b: a batch of 8 independent 2048 x 2048 INT4 layers in one hipGraph-captured call: every replay equals
    the eager batched call, which equals the eight layers quantized one at a time (bitwise)."""
    B, k = 8, 2048
    x = torch.stack([instances.weights(k, k, 100 + i, True, False) for i in range(B)]).float().to(DEV)
    grams_a = torch.stack([_gpu_factor(k, .5, 200 + i) for i in range(B)]).float()
    grams_b = torch.stack([_gpu_factor(k, .5, 300 + i) for i in range(B)]).float()
    lo = LDL.ldl_of_inverse(grams_a)
    up = LDL.ldl_of_inverse(grams_b).transpose(-1, -2).contiguous()
    scale = instances.abs_max_row_scale(x, -8, 7).expand_as(x).contiguous()
    zp = torch.zeros_like(x)
    q = functools.partial(QI.affine_quantizer_hip, qmin=-8, qmax=7)
    eager = G.gptq_2d(x, lo, up, quantizer=q, quantizer_inputs=(scale, zp))
    replay = G.capture_gptq_2d(x, lo, up, quantizer=q, quantizer_inputs=(scale, zp))
    for _ in range(2):
        got = replay(x, lo, up, scale, zp)
        torch.cuda.synchronize()
        assert got.equal(eager)
    for i in (0, 5):
        one = G.gptq_2d(x[i], lo[i], up[i], quantizer=q, quantizer_inputs=(scale[i], zp[i]))
        assert one.equal(eager[i]), i


# ------------------------------------------------------------------------------------------------ reduced size, fp64

def test_c4_trellis_reduced():
    """C4's quantizer at reduced size: 128 x 128 weights in 16 x 16 super-entries, HYB code L=16 K=2 V=2,
    tail-biting, scale RMS(W) / (0.9 RMS(table)) (demo.ipynb:541-545), fp64: the HIP trellis plug-in inside the
    GPU super-entry sweep equals super-entry Algorithm 3 with the oracle's trellis quantizer exactly."""
    gen = torch.Generator().manual_seed(4)
    m = n = 128
    x = 0.02 * torch.randn(m, n, generator=gen, dtype=torch.float64)
    a = instances.wishart_factor(m, .5, 1)
    b = instances.wishart_factor(n, .5, 2)
    lo, up = A.ldl_of_inverse(a, size=16), A.ldl_of_inverse(b, size=16).t()
    table = OT.hyb(L=16, dtype=torch.float64)
    scale = x.pow(2).mean().sqrt() / (0.9 * table.pow(2).mean().sqrt())

    def trellis(y, i, j):
        out = torch.empty_like(y)
        OT.trellis_quantizer_super_entry(y, lambda t: t, scale, out=out, table=table, K=2)
        return out

    expected = A.alg3_super_entry(x, lo, up, Q=trellis, super_entry_shape=(16, 16))
    got = G.gptq_2d_super_entry(
        x.to(DEV), lo.to(DEV), up.to(DEV), super_entry_shape=(16, 16), quantizer_inputs=(scale.to(DEV),),
        quantizer=functools.partial(QT.trellis_quantizer_super_entry_hip, table=table.to(DEV), K=2))
    assert got.cpu().equal(expected)


def test_c5a_three_factor_reduced():
    """C5a at reduced size: W 64 x (7 x 64) under A (64) x B1 (7) x B2 (64), super-entries 1 x 32, INT4 abs-max
    per super-entry row with bf16 scales, fp64.  U = ldl_of_inverse(B1 (x) B2, 32)^T equals
    U_B1 (x) U_B2^(32) (Cholesky of a Kronecker product), on the GPU LDL too; and the GPU super-entry sweep with
    the HIP quantizer equals super-entry Algorithm 3 with the oracle's quantizer exactly."""
    m, n1, n2 = 64, 7, 64
    gen = torch.Generator().manual_seed(5)
    x = 0.02 * torch.randn(m, n1 * n2, generator=gen, dtype=torch.float64)
    a = instances.wishart_factor(m, .5, 1)
    b1 = instances.wishart_factor(n1, .5, 3)
    b2 = instances.wishart_factor(n2, .5, 4)
    u_kron = torch.kron(A.ldl_of_inverse(b1).contiguous(), A.ldl_of_inverse(b2, size=32).contiguous()).t()
    u_dev = LDL.ldl_of_inverse(torch.kron(b1, b2).to(DEV), size=32).t().cpu()
    assert (u_dev - u_kron).abs().max() < 1e-9
    lo = A.ldl_of_inverse(a)
    qk = dict(qmin=-8, qmax=7, dtype=torch.bfloat16)

    def absmax(y, i, j):
        out = torch.empty_like(y)
        OQ.int_abs_max_quantizer(y, lambda t: t, out=out, **qk)
        return out

    expected = A.alg3_super_entry(x, lo, u_kron, Q=absmax, super_entry_shape=(1, 32))
    got = G.gptq_2d_super_entry(x.to(DEV), lo.to(DEV), u_kron.to(DEV), super_entry_shape=(1, 32),
                                quantizer=functools.partial(QI.int_abs_max_quantizer_hip, **qk))
    assert got.cpu().equal(expected)
