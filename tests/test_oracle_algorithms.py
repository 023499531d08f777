"""Pin the CPU oracle's sweeps and paper algorithms (CPU only).

Follows the reference's exactness suites (gptq_2d_reference.py:386-478, test_gptq_2d.py:70-89)
and adds an independent pin of Algorithm 1: every decision equals the rounding of the
conditional minimiser of the quadratic objective given the earlier decisions, computed by a
linear solve -- the definition of sequential (GPTQ/OBQ) rounding, not a restatement of the loop.
"""

import functools

import pytest
import torch

import gptq_d_sided as DS
from oracle import algorithms as A
from oracle import sweep as S

SHAPES = (8, 8), (5, 13), (13, 5), (1, 7), (7, 1), (32, 32), (24, 40), (40, 24)


@pytest.mark.parametrize("shape", SHAPES)
def test_theorem1_all_algorithms(shape):
    """Algorithms 2, 3, 5 (several block widths), 6, 7 equal Algorithm 1 on vec(X) bitwise in fp64."""
    m, n = shape
    blocked = {f"alg5{w}": functools.partial(A.alg5, w=w) for w in ((), (2,), (2, 4), (3, 5), (2, 3, 8))}
    algs = {"alg2": A.alg2, "alg3": A.alg3, **blocked, "alg6": A.alg6, "alg7": A.alg7}
    for seed in range(3):
        Am, Bm, X = A.random_instance((m, n), 1000 * m + 10 * n + seed)
        L, U = A.feedback_factors(Am, Bm)
        Zref = A.vectorized_alg1(X, Am, Bm, Q=A.coordinate_round)
        for name, fn in algs.items():
            assert fn(X, L, U, Q=A.coordinate_round).equal(Zref), (name, seed)


@pytest.mark.parametrize("case", [(8, 12, (2, 4)), (6, 6, (3, 2)), (4, 64, (1, 32)), (12, 8, (4, 4)),
                                  (16, 16, (16, 16)), (13, 5, (1, 1))])
def test_super_entry_and_yaqa(case):
    """Super-entry Algorithm 3 equals super-entry Algorithm 1; YAQA_iterative equals the rotated sweep."""
    m, n, (p, q) = case
    mb, nb = m // p, n // q
    for seed in range(2):
        Am, Bm, X = A.random_instance((m, n), 1000 * m + 10 * n + seed)
        L, U = A.feedback_factors(Am, Bm, (p, q))
        Zref = A.vectorized_alg1(X, Am, Bm, Q=A.coordinate_round, super_entry_shape=(p, q))
        assert A.alg3_super_entry(X, L, U, Q=A.coordinate_round, super_entry_shape=(p, q)).equal(Zref)
        Lr, Ur = A.feedback_factors(Am.flip(dims=(1,)), Bm.flip(dims=(0,)), (p, q))
        Qr = lambda x, i, j: A.coordinate_round(x, mb - 1 - i, nb - 1 - j)
        Zr = A.alg3_super_entry(X.flip(dims=(0, 1)), Lr, Ur, Q=Qr, super_entry_shape=(p, q)).flip(dims=(0, 1))
        Lin, Lout = A.yaqa_factors(Am, Bm, (p, q))
        assert A.yaqa_iterative(X, Lin, Lout, p, q, Q=A.coordinate_round).equal(Zr)


@pytest.mark.parametrize("shape", [(1,), (7,), (4, 6), (1, 1, 1), (1, 4, 3), (3, 4, 5), (3, 1, 1, 2), (2, 3, 2, 3)])
def test_d_sided(shape):
    """Direct and buffered D-sided rounding equal Algorithm 1 on the column-major vec (gptq_2d_reference.py:450-478)."""
    D = len(shape)
    for seed in range(2):
        *bases, X = A.random_instance(shape, seed)
        grams = [b.t() @ b for b in bases]
        F = A.ldl_of_inverse(A.kron_reduce(list(reversed(grams))))
        z = A.alg1(X.permute(*reversed(range(D))).flatten(), F)
        Zref = z.reshape(shape[::-1]).permute(*reversed(range(D)))
        Ls = [A.ldl_of_inverse(g) for g in grams]
        assert A.alg2_d_sided(X, Ls).equal(Zref)
        assert A.alg4(X, Ls).equal(Zref)


def test_alg1_is_sequential_conditional_rounding():
    """Independent pin of Algorithm 1: z_k = round(y_k) where y_k is the k-th coordinate of the minimiser
    of (z - x)^T H (z - x) over the free coordinates k.. given z_{<k}; F comes from the LDL of H^{-1}."""
    g = torch.Generator().manual_seed(11)
    for N in (1, 2, 5, 9):
        a = torch.randn(N, N, generator=g, dtype=torch.float64) + 2 * torch.eye(N, dtype=torch.float64)
        H = a.t() @ a
        x = 3 * torch.randn(N, generator=g, dtype=torch.float64)
        F = A.ldl_of_inverse(H)
        z = A.alg1(x, F)
        for k in range(N):
            d_fixed = z[:k] - x[:k]
            rhs = -H[k:, :k] @ d_fixed
            d_free = torch.linalg.solve(H[k:, k:], rhs)
            y_k = x[k] + d_free[0]
            assert torch.round(y_k) == z[k], (N, k)
    # a dropped feedback term would be caught: with F = I the decisions are plain rounding, and differ here
    assert not A.alg1(x, torch.eye(N, dtype=torch.float64)).equal(z)


def _instance(m, n, seed, se=(1, 1)):
    """X, L, U with NaN in the unused triangles (test_gptq_2d.py:32-40), CPU generator."""
    g = torch.Generator().manual_seed(seed)
    x = 4. * torch.randn(m, n, generator=g, dtype=torch.float64)
    l, u = (.05 * torch.randn(k, k, generator=g, dtype=torch.float64) for k in (m, n))
    for f, size, unused in ((l, se[0], torch.ge), (u, se[1], torch.le)):
        blk = torch.arange(f.size(0)) // size
        f[unused(blk[None, :], blk[:, None])] = torch.nan
    return x, l, u


def _unit(l, u, se=(1, 1)):
    return S.unit_triangular(l, False, se[0]), S.unit_triangular(u, True, se[1])


@pytest.mark.parametrize("m,n,se", [(1, 1, (1, 1)), (1, 7, (1, 1)), (7, 1, (1, 1)), (13, 5, (1, 1)),
                                    (9, 13, (1, 1)), (8, 12, (2, 4)), (6, 6, (3, 2)), (4, 64, (1, 32)),
                                    (12, 8, (4, 4)), (16, 16, (16, 16)), (24, 8, (1, 8)), (32, 64, (16, 16))])
def test_oracle_sweeps_match_alg3(m, n, se):
    """The oracle's torch sweeps equal super-entry Algorithm 3 in fp64 (test_gptq_2d.py:70-89, on the CPU)."""
    x, l, u = _instance(m, n, 100 * m + n, se)
    lu, uu = _unit(l, u, se)
    expected = A.alg3_super_entry(x, lu, uu, super_entry_shape=se)
    assert S.gptq_2d_super_entry_torch(x, l, u, super_entry_shape=se).equal(expected)
    assert S.direct_2d_super_entry(x, l, u, super_entry_shape=se).equal(expected)
    if se == (1, 1):
        assert S.gptq_2d_torch(x, lu, uu).equal(expected)
        assert S.direct_2d(x, lu, uu).equal(expected)


def test_oracle_sweep_batches():
    """Broadcast batches: every logical batch equals its own unbatched sweep."""
    x, l, u = _instance(9, 15, 3)
    lu, uu = _unit(l, u)
    xb = torch.stack((x, x + .25))[:, None]
    lb = torch.stack((lu, .5 * lu, 2 * lu))[None]
    out = S.gptq_2d_torch(xb, lb, uu)
    assert out.shape == (2, 3, 9, 15)
    for i in range(2):
        for j in range(3):
            assert out[i, j].equal(S.gptq_2d_torch(xb[i, 0], lb[0, j], uu))


def test_ldl_invariants():
    """ldl_of_inverse: unit (block) lower triangular, identity diagonal blocks, L^T M L block diagonal
    (so that M^{-1} = L Lambda L^T), and agreement with an LDL computed from an explicit inverse."""
    g = torch.Generator().manual_seed(5)
    k = 24
    a = torch.randn(k, 3 * k, generator=g, dtype=torch.float64)
    M = a @ a.t() / (3 * k) + 1e-2 * torch.eye(k, dtype=torch.float64)
    for size in (1, 2, 3, 4, 8):
        L = A.ldl_of_inverse(M, size)
        blk = torch.arange(k) // size
        same = blk[:, None] == blk[None, :]
        assert torch.equal(L.masked_select(same), torch.eye(k, dtype=torch.float64).masked_select(same))
        assert (L.masked_select(blk[:, None] < blk[None, :]) == 0).all()
        D = L.t() @ M @ L  # = Lambda^{-1}, block diagonal
        assert D.masked_select(~same).abs().max() < 1e-10 * D.abs().max()
    # size 1 against an independent LDL of the explicit inverse: M^{-1} = C C^T, L = C diag(C)^{-1}
    C = torch.linalg.cholesky(torch.linalg.inv(M))
    assert torch.allclose(A.ldl_of_inverse(M), C / C.diagonal(), atol=1e-9)
    # Kronecker identity used by the three-factor configuration
    k1, k2 = 4, 6
    a1 = torch.randn(k1, k1, generator=g, dtype=torch.float64)
    a2 = torch.randn(k2, k2, generator=g, dtype=torch.float64)
    M1 = a1 @ a1.t() + torch.eye(k1, dtype=torch.float64)
    M2 = a2 @ a2.t() + torch.eye(k2, dtype=torch.float64)
    assert torch.allclose(A.ldl_of_inverse(torch.kron(M1, M2)),
                          torch.kron(A.ldl_of_inverse(M1), A.ldl_of_inverse(M2)), atol=1e-10)


@pytest.mark.parametrize("shape", [(3, 4, 5), (6, 2, 3), (1, 5, 4), (4, 1, 1), (2, 3, 2, 3), (5, 7)])
def test_d_sided_is_a_2d_sweep(shape):
    """The map the GPU D-sided entry point (gptq_d_sided) uses: for X [n_1, ..., n_D] and unit lower L_1..L_D, Algorithm 4
    equals the two-sided sweep (Algorithm 3) of the [n_1, n_2 ... n_D] matrix whose column index is
    i_2 + n_2 (i_3 + n_3 (...)) -- mode 2 fastest, i.e. X permuted to (1, D, ..., 2) -- under L = L_1 and
    U = (L_D (x) ... (x) L_2)^T; bitwise in fp64 with a codebook that depends on every coordinate."""
    D = len(shape)
    for seed in range(2):
        *bases, X = A.random_instance(shape, 50 + seed)
        Ls = [A.ldl_of_inverse(b.t() @ b) for b in bases]

        def Qd(x, *idx):
            return A.coordinate_round(x, idx[0], sum(int(k) * i for k, i in enumerate(idx[1:], 1)))

        expected = A.alg4(X, Ls, Q=Qd)
        n1, rest = shape[0], shape[1:]
        perm = DS.mode_permutation(D)
        assert perm == (0, *range(D - 1, 0, -1))
        W = X.permute(*perm).reshape(n1, -1)
        U = Ls[-1]
        for f in reversed(Ls[1:-1]):
            U = torch.kron(U, f)
        U = U.t()
        # the product's factor reads each L_d strictly below its diagonal only
        poisoned = [f.masked_fill(torch.ones_like(f, dtype=torch.bool).triu(), torch.nan) for f in Ls]
        assert DS.column_factor(poisoned).equal(U)
        strides = [1]
        for k in rest[:-1]:
            strides.append(strides[-1] * k)

        def Q2(x, i, c):
            coords = [(c // s_) % k for s_, k in zip(strides, rest)]
            return Qd(x, i, *coords)

        got = A.alg3(W, Ls[0], U, Q=Q2)
        got = got.reshape(n1, *reversed(rest)).permute(*[perm.index(d) for d in range(D)])
        assert got.equal(expected), seed


@pytest.mark.parametrize("m,n,p,q", [(12, 10, 1, 1), (16, 24, 4, 8), (8, 64, 1, 32), (32, 32, 16, 16)])
def test_alg3_pre_rounding_identity(m, n, p, q):
    """The closed form of the values Algorithm 3 rounds, from its own errors, equals the values its quantizer
    receives (fp64, within summation order); a dropped transpose or sign fails it."""
    g = torch.Generator().manual_seed(m * n + p)
    x = 3 * torch.randn(m, n, generator=g, dtype=torch.float64)
    lo = A.unit_diagonal_blocks(torch.randn(m, m, generator=g, dtype=torch.float64).tril(), p) if p > 1 else \
        torch.randn(m, m, generator=g, dtype=torch.float64).tril(-1) * .3 + torch.eye(m, dtype=torch.float64)
    up = (A.unit_diagonal_blocks(torch.randn(n, n, generator=g, dtype=torch.float64).tril(), q) if q > 1 else
          torch.randn(n, n, generator=g, dtype=torch.float64).tril(-1) * .3 + torch.eye(n, dtype=torch.float64)).t()
    pre = torch.full_like(x, float("nan"))

    def spy(y, i, j):  # y [d, p, q] of the super-entries (i, j) of one antidiagonal
        pre.view(m // p, p, n // q, q)[i.flatten(), :, j.flatten(), :] = y
        return y.round()

    z = A.alg3_super_entry(x, lo, up, Q=spy, super_entry_shape=(p, q))
    assert not pre.isnan().any()
    got = A.alg3_pre_rounding(x, lo, up, z, pre, (p, q))
    assert torch.allclose(got, pre, rtol=0, atol=1e-9 * float(pre.abs().max()))
    bad = A.alg3_pre_rounding(x, lo, up.t().contiguous(), z, pre, (p, q))  # transposed U
    assert not torch.allclose(bad, pre, rtol=0, atol=1e-6 * float(pre.abs().max()))
    bad = A.alg3_pre_rounding(x, lo, up, 2 * pre - z, pre, (p, q))  # errors with the wrong sign
    assert not torch.allclose(bad, pre, rtol=0, atol=1e-6 * float(pre.abs().max()))
