"""GPU tests of the fused sweep with U given by its Kronecker factors (gptq_2d.KroneckerU,
gptq2d_sweep_fused_kron_f32): U = P (x) Q read as P[i / nq, j / nq] * Q[i % nq, j % nq] by the tile stages and the
flushes, against the same sweep with the explicit product torch.kron(P, Q) -- the entries Algorithm 4 forms from
its per-mode factors (gptq_2d_reference.py:270-294) -- bit for bit: outputs, and for the teacher-forced quantizer
every pre-rounding value.  Cases cross the tile and workgroup edges of both factors (nq = 16 and 48, where
blocks of P change inside a 32-row k-tile and inside a tile's columns; nq = 32, where the two tile columns of a
flush workgroup lie in different blocks; nq = 96 and 112; m and n not multiples of 32), plain entries and 1 x 32
super-entry rows, several outer block sizes, a resumed call, the D-sided sweep (D = 3, 4) and the full-size
three-factor layer in both forms (C5a, C5a three-sided).  Shapes the fused reader does not take (fp64, a batch,
nq % 16 != 0) form the product and give the same result.
"""

import functools

import pytest
import torch

import _hip
import gptq_2d as G
import gptq_2d_ldl as LDL
import gptq_d_sided as DS
import instances
import quantizer_int as QI

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _unit_upper(k, seed, dtype=torch.float32, scale=.3, diag=1.):
    g = torch.Generator().manual_seed(seed)
    f = scale / k ** .5 * torch.randn(k, k, generator=g, dtype=torch.float64)
    return (f.triu(1) + diag * torch.eye(k, dtype=torch.float64)).to(dtype).to(DEV)


def _unit_lower(k, seed, dtype=torch.float32):
    return _unit_upper(k, seed, dtype).t().contiguous()


def _instance(m, np_, nq, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = (4. * torch.randn(m, np_ * nq, generator=g, dtype=torch.float64)).to(dtype).to(DEV)
    return x, _unit_lower(m, seed + 1, dtype), _unit_upper(np_, seed + 2, dtype), _unit_upper(nq, seed + 3, dtype)


def _quantizer(kind, x, seed):
    """(quantizer, quantizer inputs) of a built-in quantizer the fused engine takes."""
    if kind == "round":
        return QI.round_quantizer, ()
    g = torch.Generator().manual_seed(seed)
    if kind == "affine":
        scale = (2. ** torch.randint(-2, 2, x.shape, generator=g).double() * .37).to(x.dtype).to(DEV)
        zero = torch.randint(-2, 3, x.shape, generator=g).to(x.dtype).to(DEV)
        return functools.partial(QI.affine_quantizer_hip, qmin=-8, qmax=7), (scale, zero)
    assert kind == "absmax"
    return functools.partial(QI.int_abs_max_quantizer_hip, qmin=-8, qmax=7, dtype=torch.bfloat16), ()


CASES = [  # m, np, nq, quantizer, 1 x 32 rows, outer block (antidiagonals)
    (64, 3, 32, "round", False, 64),
    (64, 5, 16, "round", False, 64),
    (68, 3, 48, "affine", False, 96),
    (96, 3, 112, "affine", False, 128),
    (40, 2, 80, "round", False, 64),
    (64, 4, 48, "absmax", True, 96),
    (32, 2, 112, "affine", True, 64),
    (100, 5, 32, "affine", False, 128),
    (96, 2, 64, "affine", False, 96),
    (128, 3, 96, "round", False, 256),
    (200, 7, 64, "affine", False, 512),
    (64, 3, 64, "absmax", True, 128),
    (96, 4, 32, "affine", True, 64),
    (36, 9, 32, "round", True, 96),
]


@pytest.mark.parametrize("m,np_,nq,kind,rows,outer", CASES)
def test_kron_equals_explicit(m, np_, nq, kind, rows, outer):
    print(f"kron {m}x({np_}x{nq}) {kind} rows={rows} outer={outer}", flush=True)
    x, lo, p, q = _instance(m, np_, nq, m + np_ + nq)
    quant, qin = _quantizer(kind, x, m)
    if rows:
        run = functools.partial(G.gptq_2d_super_entry, x, lo, super_entry_shape=(1, 32), quantizer=quant,
                                quantizer_inputs=qin, outer_block_size=outer, fused=True)
    else:
        run = functools.partial(G.gptq_2d, x, lo, quantizer=quant, quantizer_inputs=qin, outer_block_size=outer,
                                fused=True)
    z_kron = run(G.KroneckerU(p, q))
    z_dense = run(torch.kron(p, q))
    assert torch.equal(z_kron, z_dense)
    assert z_kron.isfinite().all()


def test_kron_factor_diagonals_enter():
    """Factors whose diagonals are not 1 (the engine reads U strictly above its diagonal, which then holds P's
    diagonal entries times Q's upper entries, and Q's diagonal times P's upper ones) and a 1 x 1 outer factor:
    equal to the explicit product's sweep, values before rounding included."""
    for m, np_, nq, rows in ((64, 3, 48, False), (96, 1, 64, False), (64, 2, 32, True), (40, 4, 16, False)):
        print(f"kron diagonals {m}x({np_}x{nq}) rows={rows}", flush=True)
        x, lo, _, _ = _instance(m, np_, nq, 3 * m + nq)
        p = _unit_upper(np_, m + 1, diag=1.25)
        q = _unit_upper(nq, m + 2, diag=0.75)
        se = dict(super_entry_shape=(1, 32)) if rows else {}
        run = functools.partial(G.gptq_2d_super_entry, **se) if rows else G.gptq_2d
        z = run(x, lo, torch.kron(p, q), outer_block_size=64, fused=True)
        pre_k, pre_d = torch.full_like(x, float("nan")), torch.full_like(x, float("nan"))
        zk = run(x, lo, G.KroneckerU(p, q), quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre_k),
                 outer_block_size=64, fused=True)
        zd = run(x, lo, torch.kron(p, q), quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre_d),
                 outer_block_size=64, fused=True)
        assert torch.equal(zk, z) and torch.equal(zd, z)
        assert torch.equal(run(x, lo, G.KroneckerU(p, q), outer_block_size=64, fused=True), z)
        assert not pre_k.isnan().any() and torch.equal(pre_k, pre_d)


@pytest.mark.parametrize("m,np_,nq,outer", [(96, 3, 32, 64), (100, 4, 64, 128), (64, 2, 96, 96), (72, 3, 112, 96),
                                             (64, 7, 16, 64)])
def test_kron_teacher_forced_values(m, np_, nq, outer):
    """Teacher-forced with the dense run's codes: every pre-rounding value of the Kronecker run equals the
    explicit run's bit for bit (the feedback sums, not only the codes)."""
    print(f"kron forced {m}x({np_}x{nq}) outer={outer}", flush=True)
    x, lo, p, q = _instance(m, np_, nq, 7 * m + nq)
    z = G.gptq_2d(x, lo, torch.kron(p, q), outer_block_size=outer, fused=True)
    pre_k, pre_d = torch.full_like(x, float("nan")), torch.full_like(x, float("nan"))
    zk = G.gptq_2d(x, lo, G.KroneckerU(p, q), quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre_k),
                   outer_block_size=outer, fused=True)
    zd = G.gptq_2d(x, lo, torch.kron(p, q), quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z, pre_d),
                   outer_block_size=outer, fused=True)
    assert torch.equal(zk, z) and torch.equal(zd, z)
    assert not pre_k.isnan().any()
    assert torch.equal(pre_k, pre_d)


def test_kron_resumed_call():
    """Two calls of the C entry point over consecutive outer blocks (stage_begin / stage_end on a block boundary,
    C and E kept between them) equal one call over the whole sweep."""
    m, np_, nq, ot = 96, 3, 64, 2
    x, lo, p, q = _instance(m, np_, nq, 31)
    n = np_ * nq
    stages = (m + 31) // 32 + (n + 31) // 32 - 1

    def run(ranges):
        y = x.clone()
        c, e = torch.empty_like(y), torch.empty_like(y)
        for sb, se in ranges:
            _hip.call_untyped("sweep_fused_kron_f32", _hip.ptr(y), _hip.ptr(c), _hip.ptr(e), _hip.ptr(lo), _hip.ptr(p),
                              _hip.ptr(q), m, np_, nq, 1, 1, 0, None, None, 0.0, 0.0, 0, None, None, ot, sb, se,
                              _hip.stream(y.device))
        torch.cuda.synchronize()
        return y

    whole = run([(0, -1)])
    assert torch.equal(run([(0, 2 * ot), (2 * ot, stages)]), whole)
    assert torch.equal(whole, G.gptq_2d(x, lo, torch.kron(p, q), outer_block_size=32 * ot, fused=True))


def test_kron_other_paths_form_the_product():
    """fp64, a batch of matrices and an inner factor whose size is not a multiple of 16 take the explicit product:
    the same result as passing it."""
    x, lo, p, q = _instance(64, 3, 32, 5, torch.float64)
    assert torch.equal(G.gptq_2d(x, lo, G.KroneckerU(p, q)), G.gptq_2d(x, lo, torch.kron(p, q)))
    x, lo, p, q = _instance(64, 4, 24, 6)
    assert torch.equal(G.gptq_2d(x, lo, G.KroneckerU(p, q)), G.gptq_2d(x, lo, torch.kron(p, q)))
    x, lo, p, q = _instance(64, 2, 32, 8)
    xb = torch.stack([x, -x])
    assert torch.equal(G.gptq_2d(xb, lo, G.KroneckerU(p, q)), G.gptq_2d(xb, lo, torch.kron(p, q)))
    assert torch.equal(G.gptq_2d(x, lo, G.KroneckerU(p, q), fused=False),
                       G.gptq_2d(x, lo, torch.kron(p, q), fused=False))


@pytest.mark.parametrize("shape", [(40, 64, 3), (36, 32, 2, 3), (64, 96, 2), (40, 112, 3), (32, 16, 3, 2)])
def test_d_sided_kron(shape):
    """The D-sided sweep passes U as the pair (L_D^T (x) ... (x) L_3^T, L_2^T); with n_2 a multiple of 16 the
    fused engine reads it from the factors: equal to the sweep with U = column_factor(ls) formed."""
    print(f"d-sided kron {shape}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    x = (4. * torch.randn(*shape, generator=g, dtype=torch.float64)).float().to(DEV)
    ls = [_unit_lower(k, 100 + i) for i, k in enumerate(shape)]
    pair = DS.column_factor_pair(ls)
    assert isinstance(pair, G.KroneckerU) and torch.equal(pair.dense(), DS.column_factor(ls))
    perm = DS.mode_permutation(len(shape))
    w = x.permute(*perm).reshape(shape[0], -1)
    z = G.gptq_2d(w, ls[0], DS.column_factor(ls), outer_block_size=1024, fused=True)
    expected = z.reshape(shape[0], *(shape[d] for d in perm[1:])).permute(*[perm.index(d) for d in range(len(shape))])
    assert torch.equal(DS.gptq_d_sided(x, ls, fused=True), expected)


@pytest.mark.timeout(600)
def test_kron_c5a_full_size():
    """C5a's 8192 x (112 x 256) layer, 1 x 32 abs-max INT4 rows, the benchmark's outer blocks: U_B1 (x) U_B2 read
    from its factors gives the outputs of the explicit 28672^2 U bit for bit."""
    cfg = instances.THREE_FACTOR["C5a"]
    m, n1, n2 = cfg.m, cfg.n1, cfg.n2
    print(f"C5a kron: {m}x({n1}x{n2})", flush=True)
    x = instances.weights(m, n1 * n2, cfg.seeds[0], True, False).float().to(DEV)
    fac = [instances.wishart_factor(k, cfg.alpha, s, device=DEV).float() for k, s in zip((m, n1, n2), cfg.seeds[1:])]
    lo = LDL.ldl_of_inverse(fac[0])
    u1 = LDL.ldl_of_inverse(fac[1]).t().contiguous()
    u2 = LDL.ldl_of_inverse(fac[2], size=cfg.group).t().contiguous()
    del fac
    q = functools.partial(QI.int_abs_max_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax, dtype=torch.bfloat16)
    run = functools.partial(G.gptq_2d_super_entry, x, lo, super_entry_shape=(1, cfg.group), quantizer=q,
                            outer_block_size=1024, fused=True)
    z_kron = run(G.KroneckerU(u1, u2))
    up = torch.kron(u1, u2)
    z_dense = run(up)
    del up
    assert torch.equal(z_kron, z_dense)
    print(f"  equal ({z_kron.numel()} entries)", flush=True)


@pytest.mark.timeout(600)
def test_kron_c5a_three_sided_full_size():
    """C5a's layer as the three-sided tensor X[i, b1, b2] (8192 x 112 x 256, D-sided sweep, static abs-max INT4
    scales per 32 consecutive b2): U = (L_B2 (x) L_B1)^T read from its factors (the inner one 112 x 112) gives the
    outputs of the sweep with the explicit 28672^2 U bit for bit."""
    cfg = instances.THREE_FACTOR["C5a"]
    m, n1, n2 = cfg.m, cfg.n1, cfg.n2
    print(f"C5a three-sided kron: {m}x{n1}x{n2}", flush=True)
    x = instances.weights(m, n1 * n2, cfg.seeds[0], True, False).float().view(m, n1, n2).to(DEV)
    ls = [LDL.ldl_of_inverse(instances.wishart_factor(k, cfg.alpha, s, device=DEV).float())
          for k, s in zip((m, n1, n2), cfg.seeds[1:])]
    scale = instances.abs_max_group_scale(x, cfg.group, cfg.qmin, cfg.qmax)
    q = functools.partial(QI.affine_quantizer_hip, qmin=cfg.qmin, qmax=cfg.qmax)
    z_kron = DS.gptq_d_sided(x, ls, quantizer=q, quantizer_inputs=(scale, torch.zeros_like(x)), outer_block_size=1024,
                             fused=True)
    perm = DS.mode_permutation(3)
    flat = lambda t: t.permute(*perm).reshape(m, -1).contiguous()
    up = DS.column_factor(ls)
    z = G.gptq_2d(flat(x), ls[0], up, quantizer=q, quantizer_inputs=(flat(scale), torch.zeros(m, n1 * n2, device=DEV)),
                  outer_block_size=1024, fused=True)
    del up
    assert torch.equal(flat(z_kron), z)
    print(f"  equal ({z.numel()} entries)", flush=True)


def test_kron_graph_replay():
    """capture_gptq_2d with U given as a Kronecker pair: every replay -- new inputs each time, with eager work and
    synchronisations between replays -- equals the eager sweep with the explicit product."""
    m, np_, nq = 64, 3, 48
    x, lo, p, q = _instance(m, np_, nq, 77)
    eye = torch.eye(np_, device=DEV)
    replay = G.capture_gptq_2d(x, lo, G.KroneckerU(p, q), outer_block_size=64)
    for r in range(3):
        print(f"kron graph replay {r}", flush=True)
        xr = x * (1. + .25 * r)
        pr = (p - eye) * (1. + .1 * r) + eye
        got = replay(xr, lo, G.KroneckerU(pr, q))
        torch.cuda.synchronize()
        want = G.gptq_2d(xr, lo, torch.kron(pr, q), outer_block_size=64, fused=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    with pytest.raises(AssertionError):
        replay(x, lo, torch.kron(p, q))  # captured as a pair: replays take a pair
