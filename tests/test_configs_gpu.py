"""Parity of the benchmark configurations on the GPU (the layer shapes and quantizers of C2-C5 and H).

Full-size layers (C2, C3, H) run in the benchmark's configuration (fp32 fused engine, 768-antidiagonal
outer blocks) and are checked against the CPU oracle run over the whole sweep.  Teacher-forced (every stage
given the oracle's codes), the engine's own Y before rounding gives the oracle's code in >= 99.99% of the
entries and every mismatch is a near-tie |frac - 0.5| < 1e-5 (code units) or an entry where the engine
rounds as the fp64 trajectory of the same forced codes does (the reference path's fp32 sums, not the
engine's, crossed the rounding boundary; at most 1e-6 of the entries); free running, the objective
tr(R^T A R B) is within 1e-4 relative of the oracle's and of its fp64 run's, and the engine's codes agree
with the oracle's fp64 trajectory at least as well as the oracle's fp32 codes do (see
test_full_size_layer).  The reduced-size tests run the reference's whole algorithm in fp64, where the
codes must be equal.

Factors here are Wishart-like as in the benchmark definition, F = G diag(i^-alpha) G^T / (4k) +
1e-2 I, but G is drawn with torch's GPU generator (the numpy PCG64 draws of the benchmark's
generator take seconds at these sizes); both sides of every comparison use the same L and U.
"""

import functools
import time

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


def _pre_rounding_rows(x, lo, up, z, pre, p, q, rows):
    """The rows' pre-rounding values as Algorithm 3 fixes them from the engine's own errors (fp64 torch GEMMs on
    the GPU, independent of the engine's kernels; the identity is pinned on the CPU)."""
    return A.alg3_pre_rounding(x, lo, up, z, pre, (p, q), rows)


def _say(capsys, *parts, **kw):
    """A progress line straight to the terminal, past pytest's output capture: the full-size tests run CPU
    oracles for minutes between their results, and the lines show that they are running."""
    with capsys.disabled():
        print(*parts, flush=True)


# ------------------------------------------------------------------------------------------------ full size

# outer blocks of the benchmark: bench.py OUTER_BLOCK (24 tile stages) and, for the 8192 x 28672 C5a layers,
# OUTER_BLOCK_WIDE (32 tile stages)
BENCH_OUTER = 768
BENCH_OUTER_WIDE = 1024


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["C2", "H", "C3"])
def test_full_size_layer(name, capsys):
    """C2 (4096^2 INT4 asymmetric g128), H (8192^2 INT4 per-row), C3 (14336 x 4096 INT3 per-row), fp32 fused
    engine with the benchmark's outer blocks, against the CPU oracle over every stage (see the module
    docstring for the tolerances).  Also: codes in range and on the grid, bitwise identical on a second run,
    objective below round-to-nearest's."""
    cfg = instances.CONFIGS[name]
    m, n = cfg.m, cfg.n
    _say(capsys, f"{name}: {m}x{n} qmin={cfg.qmin} qmax={cfg.qmax} outer={BENCH_OUTER}", flush=True)
    x = instances.weights(m, n, cfg.seeds[0], cfg.outliers, cfg.bf16).float().to(DEV)
    a = _gpu_factor(m, cfg.alpha, 11)
    b = _gpu_factor(n, cfg.alpha, 12)
    lo, up = LDL.feedback_factors_of_grams(a.float(), b.float())
    scale, zp = instances.quantizer_inputs(cfg, x)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    run = functools.partial(G.gptq_2d, x, lo, up, outer_block_size=BENCH_OUTER)
    z = run(quantizer=q, quantizer_inputs=(scale, zp))
    z2 = run(quantizer=q, quantizer_inputs=(scale, zp))
    torch.cuda.synchronize()
    assert z.equal(z2), "not deterministic"
    codes = torch.round(z / scale + zp)
    assert codes.min() >= cfg.qmin and codes.max() <= cfg.qmax
    assert torch.equal(z, (codes - zp) * scale), "values off the quantization grid"
    rtn = (torch.clamp(torch.round(x / scale + zp), cfg.qmin, cfg.qmax) - zp) * scale
    obj = _objective(z, x, a, b)
    ratio = obj / _objective(rtn, x, a, b)
    _say(capsys, f"  objective / RTN = {ratio:.4f}", flush=True)
    assert ratio < 1.

    # the CPU oracle over the whole sweep (fp32, the reference's own operation sequence), recording every
    # entry's Y just before it is rounded
    xc, sc, zc = x.cpu(), scale.cpu(), zp.cpu()
    pre_o = torch.full((m, n), float("nan"))

    def spy(y_flat, sl, s_, z_, *, out):
        pre_o.view(-1)[sl] = y_flat[sl]
        OQ.affine_quantizer(y_flat, sl, s_, z_, out=out, qmin=cfg.qmin, qmax=cfg.qmax)

    st = S.TorchSweepState(xc, lo.cpu(), up.cpu(), quantizer=spy, quantizer_inputs=(sc, zc))
    t0 = time.perf_counter()
    for s in range(st.stages):
        st.run_stage(s)
        if s % 1024 == 1023:
            _say(capsys, f"  oracle: {s + 1} / {st.stages} stages, {time.perf_counter() - t0:.0f} s", flush=True)
    assert not pre_o.isnan().any()
    ref_codes = torch.round(st.y / sc + zc)

    # teacher forced: every stage takes the oracle's codes; the engine's own Y before rounding must round to
    # the oracle's code in >= 99.99% of the entries, every mismatch a near-tie (|frac - 0.5| < 1e-5 code
    # units) or decided by the engine as the fp64 trajectory decides it
    pre_e = torch.full_like(x, float("nan"))
    zf = run(quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(st.y.to(DEV), pre_e))
    assert zf.equal(st.y.to(DEV))
    ye = (pre_e / scale + zp).cpu()
    yo = pre_o / sc + zc
    assert not ye.isnan().any()
    own = ye.round().clamp(cfg.qmin, cfg.qmax)
    mism = own != ref_codes
    frac = (ye - ye.floor() - .5).abs()
    dev = (ye - yo).abs()
    tf_agree = 1. - float(mism.double().mean())
    far = mism & (frac >= 1e-5)
    _say(capsys, f"  teacher forced: code agreement {tf_agree:.6%} ({int(mism.sum())} mismatches, {int(far.sum())} with "
          f"|frac - 0.5| >= 1e-5), max |dY| {dev.max():.2e} code units (median {dev.median():.2e}), largest "
          f"mismatch |frac - 0.5| {float(frac[mism].max()) if mism.any() else 0.:.2e}", flush=True)
    assert tf_agree >= 0.9999
    # far mismatches are rare: at most 1e-6 of the entries
    assert int(far.sum()) <= 1e-6 * m * n
    if far.any():
        # a mismatch farther from the rounding boundary than 1e-5 code units: the two fp32 trajectories (the
        # engine's and the reference path's) lie on either side of it.  The engine's fp64 run on the same forced
        # codes gives the trajectory both approximate; at every such entry the engine's code must be the fp64
        # trajectory's (the reference path's fp32 sums crossed the boundary, not the engine's), and the entry
        # must lie within the reference path's own largest deviation from that trajectory of the boundary
        pre64 = torch.full(x.shape, float("nan"), dtype=torch.float64, device=DEV)
        G.gptq_2d(x.double(), lo.double(), up.double(), quantizer=QI.teacher_forced_quantizer,
                  quantizer_inputs=(st.y.to(DEV, torch.float64), pre64), outer_block_size=BENCH_OUTER)
        y64 = (pre64 / scale.double() + zp.double()).cpu()
        code64 = y64.round().clamp(cfg.qmin, cfg.qmax)
        err_e, err_o = (ye.double() - y64).abs(), (yo.double() - y64).abs()
        _say(capsys, f"  fp64 trajectory: max |Y_engine - Y_fp64| {err_e.max():.2e}, max |Y_oracle - Y_fp64| "
              f"{err_o.max():.2e} code units; at the {int(far.sum())} far mismatches the engine's code is the fp64 "
              f"code at {int((own[far] == code64[far]).sum())}, the oracle's at "
              f"{int((ref_codes[far] == code64[far]).sum())}; their largest |frac - 0.5| {frac[far].max():.2e}",
              flush=True)
        assert (own[far] == code64[far]).all()
        assert (frac[far].double() <= err_o.max()).all()
        del pre64, y64, code64, err_e, err_o
    del pre_e, pre_o, ye, yo, own, frac, dev

    # free running.  A rounding sweep is chaotic in floating point: one near-tie decided the other way changes
    # that entry's error by a whole step, which moves every later entry, so two summation orders of the same
    # algorithm part ways over a large layer (the reference's own path run on the transposed layer -- the same
    # rounding in exact arithmetic, other fp32 sums -- agrees with itself in 95.3% / 98.6% / 99.998% of the
    # codes at C2 / H / C3).  The yardstick is the trajectory both fp32 runs approximate: the CPU oracle in
    # fp64 on the same inputs.  The engine's free-running codes must agree with it at least as well as the
    # reference path's fp32 codes (the oracle) do, and its objective must be within 1e-4 relative of the
    # oracle's and of the fp64 trajectory's.
    st64 = S.TorchSweepState(xc.double(), lo.cpu().double(), up.cpu().double(),
                             quantizer=functools.partial(OQ.affine_quantizer, qmin=cfg.qmin, qmax=cfg.qmax),
                             quantizer_inputs=(sc.double(), zc.double()))
    t0 = time.perf_counter()
    for s in range(st64.stages):
        st64.run_stage(s)
        if s % 1024 == 1023:
            _say(capsys, f"  fp64 oracle: {s + 1} / {st64.stages} stages, {time.perf_counter() - t0:.0f} s", flush=True)
    codes64 = torch.round(st64.y / sc.double() + zc.double()).float()
    ce = codes.cpu()
    agree = float((ce == ref_codes).double().mean())
    agree_e64 = float((ce == codes64).double().mean())
    agree_o64 = float((ref_codes == codes64).double().mean())
    obj_o = _objective(st.y.to(DEV), x, a, b)
    obj_64 = _objective(st64.y.to(DEV), x, a, b)
    rel, rel_64, rel_o64 = abs(obj - obj_o) / obj_o, abs(obj - obj_64) / obj_64, abs(obj_o - obj_64) / obj_64
    _say(capsys, f"  free running: codes agreeing with the fp64 trajectory: engine {agree_e64:.6%}, oracle {agree_o64:.6%}; "
          f"engine vs oracle {agree:.6%}; objective rel engine-oracle {rel:.2e}, engine-fp64 {rel_64:.2e}, "
          f"oracle-fp64 {rel_o64:.2e}", flush=True)
    assert agree_e64 >= agree_o64
    assert rel <= 1e-4 and rel_64 <= 1e-4


@pytest.mark.timeout(900)
def test_c5a_full_size(capsys):
    """C5a: W 8192 x 28672 = 8192 x (112 x 256) under A (x) B1 (x) B2, INT4 abs-max per 1 x 32 super-entry row
    with bf16 scales, fp32 fused engine with the benchmark's outer blocks.  U = ldl_of_inverse(B1 (x) B2, 32)^T
    is formed as U_B1 (x) U_B2^(32) (28672^2 entries: the MFMA flush's staging is based per panel).  Checks:
    bitwise determinism; teacher-forced with its own codes, the abs-max quantizer applied to the captured
    pre-rounding values reproduces every output bit for bit; the objective tr(R^T A R (B1 (x) B2)) is below
    rounding each super-entry row of W on its own; on the first 96 coarse antidiagonals the codes agree
    with the CPU oracle (super-entry Algorithm 3 in fp32 on the cropped layer, which holds every entry those
    antidiagonals depend on) in >= 99.9% of the entries; and on 24 whole rows spread over the layer the
    pre-rounding values equal super-entry Algorithm 3's, recomputed in fp64 by torch from the engine's own
    errors, and the codes of those values agree with the engine's in >= 99.99% of the entries."""
    cfg = instances.THREE_FACTOR["C5a"]
    m, n1, n2 = cfg.m, cfg.n1, cfg.n2
    n = n1 * n2
    _say(capsys, f"C5a: {m}x{n} = {m}x({n1}x{n2}), 1x{cfg.group} abs-max INT4 bf16", flush=True)
    x = instances.weights(m, n, cfg.seeds[0], True, False).float().to(DEV)
    a = _gpu_factor(m, cfg.alpha, 21)
    b1 = _gpu_factor(n1, cfg.alpha, 23)
    b2 = _gpu_factor(n2, cfg.alpha, 24)
    lo = LDL.ldl_of_inverse(a.float())
    up = torch.kron(LDL.ldl_of_inverse(b1.float()).t().contiguous(),
                    LDL.ldl_of_inverse(b2.float(), size=cfg.group).t().contiguous())
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax, dtype=torch.bfloat16)
    run = functools.partial(G.gptq_2d_super_entry, x, lo, up, super_entry_shape=(1, cfg.group),
                            outer_block_size=BENCH_OUTER_WIDE, fused=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    z = run(quantizer=q)
    torch.cuda.synchronize()
    _say(capsys, f"  sweep {1e3 * (time.perf_counter() - t0):.1f} ms (first call)", flush=True)
    assert run(quantizer=q).equal(z), "not deterministic"

    half = torch.full((), (cfg.qmax - cfg.qmin) / 2, device=DEV)

    def absmax_rows_of(v, r):
        rows = v.view(r, n // cfg.group, cfg.group)
        sc = (rows.abs().amax(-1, keepdim=True) / half).to(torch.bfloat16).float()
        sc = torch.where(sc == 0, torch.ones_like(sc), sc)
        return (torch.clamp(torch.round(rows / sc), cfg.qmin, cfg.qmax) * sc).view(r, n)

    absmax_rows = functools.partial(absmax_rows_of, r=m)

    pre = torch.full_like(x, float("nan"))
    assert run(quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre)).equal(z)
    assert not pre.isnan().any()
    assert torch.equal(absmax_rows(pre), z), "outputs are not the abs-max quantizer of their own pre-rounding values"
    # every entry of 24 rows spread over the layer: the pre-rounding values equal Algorithm 3's, recomputed in fp64
    # from the engine's own errors, within fp32 summation error, and their quantizer gives the engine's codes
    rows = torch.linspace(0, m - 1, 24, device=DEV).round().long()
    y64 = _pre_rounding_rows(x, lo, up, z, pre, 1, cfg.group, rows)
    dy = (y64 - pre[rows].double()).abs()
    rel = float(dy.max() / y64.abs().max())
    zr = absmax_rows_of(y64.float(), rows.numel())
    agree = float((zr == z[rows]).double().mean())
    _say(capsys, f"  {rows.numel()} rows ({rows.numel() * n} entries): max |Y_pre - Y_alg3(fp64)| {dy.max():.2e} "
          f"({rel:.2e} of max |Y|), codes of the fp64 values agree in {agree:.6%}", flush=True)
    assert rel < 5e-6 and agree >= 0.9999
    del pre, y64, dy

    def objective(zz):
        r = (zz - x).double()
        rb = torch.matmul(b1.t(), torch.matmul(r.view(m, n1, n2), b2)).view(m, n)
        return float(((a @ r) * rb).sum())

    ratio = objective(z) / objective(absmax_rows(x))
    _say(capsys, f"  objective / no-feedback rounding = {ratio:.4f}", flush=True)
    assert ratio < 1.

    K = 96
    xc, lc, uc = x[:K, :K * cfg.group].cpu(), lo[:K, :K].cpu(), up[:K * cfg.group, :K * cfg.group].cpu()

    def oq(y, i, j):
        out = torch.empty_like(y)
        OQ.int_abs_max_quantizer(y, lambda t: t, out=out, qmin=cfg.qmin, qmax=cfg.qmax, dtype=torch.bfloat16)
        return out

    zo = A.alg3_super_entry(xc, S.unit_triangular(lc, False), S.unit_triangular(uc, True, cfg.group), Q=oq,
                            super_entry_shape=(1, cfg.group))
    stage = torch.arange(K)[:, None] + (torch.arange(K * cfg.group) // cfg.group)[None, :]
    win = stage < K
    agree = float((z[:K, :K * cfg.group].cpu()[win] == zo[win]).double().mean())
    _say(capsys, f"  first {K} coarse antidiagonals ({int(win.sum())} entries): agreement with the oracle {agree:.6%}",
          flush=True)
    assert agree >= 0.999


def _trellis_rows(v, table, scale, K, rows_per_call=512):
    """Trellis quantization of every 16 x 16 block of v (read row by row) on its own, in calls of
    ``rows_per_call`` sequences (the search's history workspace is 2 MB per sequence at L = 16)."""
    m, n = v.shape
    seqs = (v.view(m // 16, 16, n // 16, 16).permute(0, 2, 1, 3).reshape(-1, 256) / scale).contiguous()
    out = torch.empty_like(seqs)
    sc = torch.full((seqs.size(0),), float(scale), device=v.device, dtype=v.dtype)
    for r0 in range(0, seqs.size(0), rows_per_call):
        QT.trellis_quantize_hip(seqs[r0:r0 + rows_per_call], table, K, True, out=out[r0:r0 + rows_per_call],
                                scale=sc[r0:r0 + rows_per_call])
    return out.view(m // 16, n // 16, 16, 16).permute(0, 2, 1, 3).reshape(m, n)


@pytest.mark.timeout(900)
def test_c4_full_size(capsys):
    """C4: 8192^2 weights (the headline layer's distribution) in 16 x 16 super-entries under the HYB trellis code,
    L = 16, K = 2, V = 2, tail-biting, scale RMS(W) / (0.9 RMS(table)) (demo.ipynb:541-545), fp32 plug-in engine
    with the one-launch HIP search per stage.  Checks: bitwise determinism; every output pair is a row of the
    code table times the scale; the objective is below quantizing each super-entry of W on its own; on the
    first 4 coarse antidiagonals the values agree with the CPU oracle (super-entry Algorithm 3 with the PyTorch
    search on the cropped layer, which holds every entry they depend on) in >= 99% of the entries; and at 8
    coarse antidiagonals sampled over the whole sweep (the longest, 512 super-entries, among them) the oracle's
    trellis quantizer applied to the super-entries the engine's quantizer received writes the engine's values
    bit for bit; and on 24 whole rows spread over the layer the pre-rounding values equal super-entry Algorithm
    3's, recomputed in fp64 by torch from the engine's own errors."""
    m = n = 8192
    _say(capsys, f"C4: {m}x{n}, 16x16 super-entries, HYB L=16 K=2 V=2", flush=True)
    x = instances.weights(m, n, 0, True, False).float().to(DEV)
    a = _gpu_factor(m, .5, 31)
    b = _gpu_factor(n, .5, 32)
    lo = LDL.ldl_of_inverse(a.float(), size=16)
    up = LDL.ldl_of_inverse(b.float(), size=16).t().contiguous()
    table_cpu = OT.hyb(L=16)  # the pinned CPU table (golden fixture), on both sides
    table = table_cpu.to(DEV)
    scale = x.pow(2).mean().sqrt() / (0.9 * table.pow(2).mean().sqrt())
    q = functools.partial(QT.trellis_quantizer_super_entry_hip, table=table, K=2)
    run = functools.partial(G.gptq_2d_super_entry, x, lo, up, super_entry_shape=(16, 16), quantizer=q,
                            quantizer_inputs=(scale,))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    z = run()
    torch.cuda.synchronize()
    _say(capsys, f"  layer sweep {time.perf_counter() - t0:.2f} s", flush=True)
    # a second run records, at sampled coarse antidiagonals, the super-entries the quantizer receives (the
    # engine's own pre-rounding values) and what it writes
    sampled = {0: None, 1: None, 100: None, 255: None, 511: None, 700: None, 1000: None, 1022: None}
    calls = [0]

    def spy(y_flat, select, sc_, *, out):
        s = calls[0]
        calls[0] += 1
        y_in = select(y_flat).clone() if s in sampled else None
        q(y_flat, select, sc_, out=out)
        if s in sampled:
            sampled[s] = (y_in, out.clone())

    z_spy = G.gptq_2d_super_entry(x, lo, up, super_entry_shape=(16, 16), quantizer=spy, quantizer_inputs=(scale,))
    assert calls[0] == 1023
    assert z_spy.equal(z), "not deterministic"

    def keys(pairs):
        bits = pairs.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        return (bits[..., 0] << 32) | bits[..., 1]

    grid = keys(table * scale)
    assert torch.isin(keys(z.view(m, n // 2, 2)), grid).all(), "values off the code grid"

    def objective(zz):
        r = (zz - x).double()
        return float(((a @ r) * (r @ b)).sum())

    ratio = objective(z) / objective(_trellis_rows(x, table, scale, 2))
    _say(capsys, f"  objective / no-feedback trellis = {ratio:.4f}", flush=True)
    assert ratio < 1.

    K = 4
    W = 16 * K
    xc, lc, uc = x[:W, :W].cpu(), lo[:W, :W].cpu(), up[:W, :W].cpu()
    sc = scale.cpu()

    def oq(y, i, j):
        out = torch.empty_like(y)
        OT.trellis_quantizer_super_entry(y, lambda t: t, sc, out=out, table=table_cpu, K=2)
        return out

    zo = A.alg3_super_entry(xc, S.unit_triangular(lc, False, 16), S.unit_triangular(uc, True, 16), Q=oq,
                            super_entry_shape=(16, 16))
    win = (torch.arange(W)[:, None] // 16 + torch.arange(W)[None, :] // 16) < K
    agree = float((z[:W, :W].cpu()[win] == zo[win]).double().mean())
    _say(capsys, f"  first {K} coarse antidiagonals ({int(win.sum())} entries): agreement with the oracle {agree:.4%}",
          flush=True)
    assert agree >= 0.99

    # at the sampled antidiagonals across the whole layer, the CPU oracle's quantizer on the engine's own
    # pre-rounding super-entries (up to 24 of each, spread over the antidiagonal) writes what the engine wrote
    checked = 0
    for s_, (y_in, y_out) in sampled.items():
        d = y_in.size(0)
        pick = torch.unique(torch.linspace(0, d - 1, min(d, 24)).round().long())
        yc = y_in[pick].cpu()
        ref = torch.empty_like(yc)
        OT.trellis_quantizer_super_entry(yc.flatten(), lambda t: t.unflatten(-1, yc.shape), sc, out=ref,
                                         table=table_cpu, K=2)
        assert ref.equal(y_out[pick].cpu()), s_
        checked += pick.numel()
    _say(capsys, f"  {checked} super-entries at {len(sampled)} sampled antidiagonals: the oracle's quantizer on the engine's "
          f"inputs equals the engine's output", flush=True)

    # every entry of 24 rows spread over the layer: the pre-rounding values (teacher-forced with the engine's own
    # values) equal Algorithm 3's, recomputed in fp64 from the engine's own errors, within fp32 summation error
    pre = torch.full_like(x, float("nan"))
    zf = G.gptq_2d_super_entry(x, lo, up, super_entry_shape=(16, 16), quantizer=QI.teacher_forced_quantizer,
                               quantizer_inputs=(z, pre))
    assert zf.equal(z) and not pre.isnan().any()
    rows = torch.linspace(0, m - 1, 24, device=DEV).round().long()
    y64 = _pre_rounding_rows(x, lo, up, z, pre, 16, 16, rows)
    dy = (y64 - pre[rows].double()).abs()
    rel = float(dy.max() / y64.abs().max())
    _say(capsys, f"  {rows.numel()} rows ({rows.numel() * n} entries): max |Y_pre - Y_alg3(fp64)| {dy.max():.2e} "
          f"({rel:.2e} of max |Y|)", flush=True)
    assert rel < 5e-6


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
