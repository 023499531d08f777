"""CPU restatement of the paper's algorithms and the LDL helpers (test oracle only).

Restates gptq_2d_reference.py:24-382.  That file cannot be imported on
Python 3.10 (it uses the PEP 646 star subscript ``Z[*i]``), so every function
is written again here; star subscripts become tuple indexing.

Pinned by: tests/test_oracle_algorithms.py -- Theorem 1 (Algorithms 2, 3,
5, 6, 7 equal Algorithm 1 on vec(X) bitwise in fp64 with F from the LDL of the
explicit Kronecker Gram), the super-entry and D-sided exactness checks, the
YAQA rotation identity, Algorithm 1 against a brute-force least-squares
statement on tiny inputs, and the LDL invariants (unit block triangular,
L^T M L block diagonal, agreement with a numpy LDL of M^{-1}).
``alg3_pre_rounding``: equal to the values super-entry Algorithm 3 rounds,
recorded by its quantizer, on plain and super-entry shapes (fp64, within
summation order), and a transposed or sign-flipped term fails it.
"""

from __future__ import annotations

import functools

import torch


def nearest(x, *coords):
    """Default quantizer Q of the paper listings: round half to even (gptq_2d_reference.py:24-26)."""
    return x.round()


# ----------------------------------------------------------------------------------------------- LDL helpers

def unit_diagonal_blocks(lo: torch.Tensor, size: int) -> torch.Tensor:
    """(L - D) D^{-1} + I for lower triangular L and D its block diagonal (gptq_2d_reference.py:29-38)."""
    if size == 1:
        return lo / lo.diagonal()
    k = lo.size(0) // size
    blocks = lo.reshape(k, size, k, size).diagonal(dim1=0, dim2=2).permute(2, 0, 1)
    d = torch.block_diag(*blocks)
    eye = torch.eye(lo.size(0), dtype=lo.dtype, device=lo.device)
    return torch.linalg.solve_triangular(d, lo - d, upper=False, left=False) + eye


def ldl_of_inverse(mat: torch.Tensor, size: int = 1) -> torch.Tensor:
    """Unit lower (block) triangular L with M^{-1} = L Lambda L^T (gptq_2d_reference.py:41-49).

    Reverse-order Cholesky M = Um Um^T (Um upper), then L = Um^{-T} normalised by
    its diagonal blocks.
    """
    um = torch.linalg.cholesky(mat.flip(0, 1)).flip(0, 1)
    eye = torch.eye(mat.size(0), dtype=mat.dtype, device=mat.device)
    lo = torch.linalg.solve_triangular(um, eye, upper=True).t()
    return unit_diagonal_blocks(lo, size)


def ldl(mat: torch.Tensor, size: int = 1) -> torch.Tensor:
    """Unit lower (block) triangular L with M = L Lambda L^T (gptq_2d_reference.py:52-55)."""
    return unit_diagonal_blocks(torch.linalg.cholesky(mat), size)


def feedback_factors(a: torch.Tensor, b: torch.Tensor, super_entry_shape=(1, 1)):
    """L and U from G = A^T A and H = B B^T (gptq_2d_reference.py:58-66)."""
    p, q = super_entry_shape
    lo = ldl_of_inverse(a.t() @ a, size=p)
    up = ldl_of_inverse(b @ b.t(), size=q).t()
    return lo, up


# ----------------------------------------------------------------------------------------------- geometry

def antidiagonal(s: int, m: int, n: int):
    """Entries (i, j) with i + j = s in ascending i (gptq_2d_reference.py:69-74)."""
    i = torch.arange(max(0, s - n + 1), min(s, m - 1) + 1)
    return i, s - i


def hyper_antidiagonal(s: int, shape):
    """Multi-indices with i_1 + ... + i_D = s, lexicographic (gptq_2d_reference.py:77-82)."""
    grids = torch.meshgrid(*(torch.arange(k) for k in shape), indexing="ij")
    return (sum(grids) == s).nonzero(as_tuple=True)


# ----------------------------------------------------------------------------------------------- Algorithms 1-7

@torch.no_grad()
def alg1(x, f, Q=nearest):
    """One-dimensional adaptive rounding under unit lower triangular F (gptq_2d_reference.py:85-96)."""
    z = torch.empty_like(x)
    y = x.clone()
    for k in range(x.size(0)):
        z[k] = Q(y[k], k)
        e = z[k] - y[k]
        y[k:] += f[k:, k] * e
    return z


@torch.no_grad()
def alg2(X, L, U, Q=nearest):
    """Direct antidiagonal rank-|I_s| updates (gptq_2d_reference.py:99-111)."""
    m, n = X.shape
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = X.clone()
    for s in range(m + n - 1):
        i, j = antidiagonal(s, m, n)
        Z[i, j] = Q(Y[i, j], i, j)
        E[i, j] = Z[i, j] - Y[i, j]
        Y += (L[:, i] * E[i, j]) @ U[j, :]
    return Z


@torch.no_grad()
def alg3(X, L, U, Q=nearest):
    """Buffered antidiagonal sweep, C = L E (gptq_2d_reference.py:114-130)."""
    m, n = X.shape
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = X.clone()
    C = torch.zeros_like(X)
    for s in range(m + n - 1):
        i, j = antidiagonal(s, m, n)
        Z[i, j] = Q(Y[i, j], i, j)
        E[i, j] = Z[i, j] - Y[i, j]
        M = L[:, i] * E[i, j]
        C[:, j] += M
        Y[:, j] += M
        Y[i, :] += C[i, j, None] * U[j, :]
    return Z


@torch.no_grad()
def alg5(X, L, U, w=(), Q=nearest):
    """Blocked GPTQ-2D with block widths w = (w_1..w_h) (gptq_2d_reference.py:133-163)."""
    m, n = X.shape
    h = len(w)
    w = (1, *w, m + n - 1)
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = X.clone()
    C = torch.zeros_like(X)
    stage = torch.arange(m)[:, None] + torch.arange(n)
    for s in range(m + n - 1):
        i, j = antidiagonal(s, m, n)
        Z[i, j] = Q(Y[i, j], i, j)
        E[i, j] = Z[i, j] - Y[i, j]
        C[i, j] += E[i, j]
        lev = max(v for v in range(h + 1) if (s + 1) % w[v] == 0)
        s0 = max(s // w[v] * w[v] for v in range(lev, h + 2))
        s1 = min(-(-(s + 1) // w[v]) * w[v] - 1 for v in range(lev + 1, h + 2))
        src = (s0 <= stage) & (stage <= s)
        tgt = (s < stage) & (stage <= s1)
        M = L @ E.where(src, 0.)
        C += M.where(tgt, 0.)
        Y += (M + C.where(src, 0.) @ U).where(tgt, 0.)
    return Z


@torch.no_grad()
def alg6(X, L, U, Q=nearest):
    """Column-major nested form (gptq_2d_reference.py:166-180)."""
    m, n = X.shape
    Z = torch.empty_like(X)
    Y = X.clone()
    for j in range(n):
        y = Y[:, j].clone()
        for i in range(m):
            Z[i, j] = Q(y[i], i, j)
            e = Z[i, j] - y[i]
            y[i:] += L[i:, i] * e
        Y += (y - Y[:, j])[:, None] * U[j, :]
    return Z


@torch.no_grad()
def alg7(X, L, U, Q=nearest):
    """Implicit-Y antidiagonal form (gptq_2d_reference.py:183-200)."""
    m, n = X.shape
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = torch.empty_like(X)
    C = torch.zeros_like(X)
    for s in range(m + n - 1):
        i, j = antidiagonal(s, m, n)
        Y[i, j] = X[i, j] + (C[i, :] * U[:, j].t()).sum(dim=1)
        Z[i, j] = Q(Y[i, j], i, j)
        E[i, j] = Z[i, j] - Y[i, j]
        C[:, j] += L[:, i] * E[i, j]
    return Z


# ----------------------------------------------------------------------------------------------- super-entries

@torch.no_grad()
def alg1_super_entry(x, f, Q=nearest, super_entry_shape=(1, 1)):
    """Algorithm 1 over column-major p x q super-entries (gptq_2d_reference.py:203-218)."""
    p, q = super_entry_shape
    z = torch.empty_like(x)
    y = x.clone()
    for k in range(x.size(0) // (p * q)):
        sl = slice(k * p * q, (k + 1) * p * q)
        z[sl] = Q(y[sl].reshape(q, p).t(), k).t().flatten()
        e = z[sl] - y[sl]
        y[sl.start:] += f[sl.start:, sl] @ e
    return z


@torch.no_grad()
def alg3_super_entry(X, L, U, Q=nearest, super_entry_shape=(1, 1)):
    """Algorithm 3 on the coarse matrix of super-entries (gptq_2d_reference.py:221-245)."""
    m, n = X.shape
    p, q = super_entry_shape
    mb, nb = m // p, n // q
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = X.clone()
    C = torch.zeros_like(X)
    Z4, E4, Y4, C4 = (t.reshape(mb, p, nb, q) for t in (Z, E, Y, C))
    for s in range(mb + nb - 1):
        i, j = antidiagonal(s, mb, nb)
        Z4[i, :, j, :] = Q(Y4[i, :, j, :], i[:, None, None], j[:, None, None])
        E4[i, :, j, :] = Z4[i, :, j, :] - Y4[i, :, j, :]
        M = (L.reshape(m, mb, 1, p)[:, i, :, :] @ E4[i, :, j, :])[:, :, 0, :]
        C.reshape(m, nb, q)[:, j, :] += M
        Y.reshape(m, nb, q)[:, j, :] += M
        Y.reshape(mb, p, n)[i, :, :] += C4[i, :, j, :] @ U.reshape(nb, q, n)[j, :, :]
    return Z


# ----------------------------------------------------------------------------------------------- D-sided

@torch.no_grad()
def alg3_pre_rounding(X, L, U, Z, Ypre, super_entry_shape=(1, 1), rows=None, slab=4096):
    """The values super-entry Algorithm 3 rounds, from the errors E = Z - Ypre of the whole matrix (no
    counterpart in the reference; the closed form of gptq_2d_reference.py:360-382 and gptq_2d.py:1239-1292):
    Ypre = X + L' E + C U' with C = E + L' E, where L' is L below its p x p block diagonal and U' is U above its
    q x q block diagonal.  Evaluated in fp64 for the given rows (all by default), in column slabs of U'.
    Identity of the sweep, not a sweep: it checks a trajectory against its own errors."""
    p, q = super_entry_shape
    m, n = X.shape[-2:]
    dev = X.device
    rows = torch.arange(m, device=dev) if rows is None else rows
    e = Z.double() - Ypre.double()
    ib, jb = torch.arange(m, device=dev) // p, torch.arange(n, device=dev) // q
    down = (L[rows].double() * (ib[None, :] < ib[rows][:, None])) @ e
    c = e[rows] + down
    right = torch.zeros_like(down)
    for c0 in range(0, n, slab):
        right[:, c0:c0 + slab] = c @ (U[:, c0:c0 + slab].double() * (jb[:, None] < jb[None, c0:c0 + slab]))
    return X[rows].double() + down + right


def alg2_d_sided(X, Ls, Q=nearest):
    """Algorithm 2 on an n_1 x ... x n_D tensor (gptq_2d_reference.py:248-267)."""
    D = X.dim()
    Z = torch.empty_like(X)
    E = torch.empty_like(X)
    Y = X.clone()
    for s in range(sum(X.shape) - D + 1):
        i = hyper_antidiagonal(s, X.shape)
        Z[i] = Q(Y[i], *i)
        E[i] = Z[i] - Y[i]
        upd = E[i]
        for d in range(D):
            upd = upd[..., None, :] * Ls[d][:, i[d]]
        Y += upd.sum(dim=-1)
    return Z


@torch.no_grad()
def alg4(X, Ls, Q=nearest):
    """Buffered D-sided rounding (gptq_2d_reference.py:270-294)."""
    D = X.dim()
    Z = torch.empty_like(X)
    C = [torch.zeros_like(X) for _ in range(D + 1)]
    Y = torch.empty_like(X)
    for s in range(sum(X.shape) - D + 1):
        i = hyper_antidiagonal(s, X.shape)
        Y[i] = X[i] + sum(C[d][i] for d in range(1, D + 1))
        Z[i] = Q(Y[i], *i)
        C[0][i] = Z[i] - Y[i]
        for d in range(D):
            fiber = torch.arange(X.size(d))[:, None]
            idx = (*i[:d], fiber, *i[d + 1:])
            C[d + 1][idx] += Ls[d][:, i[d]] * C[d][i]
    return Z


# ----------------------------------------------------------------------------------------------- YAQA

def yaqa_factors(A, B, super_entry_shape=(1, 1)):
    """Lin = L_I - I and Lout = L_O - I from the block LDL of the Grams (gptq_2d_reference.py:297-305)."""
    p, q = super_entry_shape
    lin = ldl(B @ B.t(), size=q) - torch.eye(B.size(0), dtype=B.dtype)
    lout = ldl(A.t() @ A, size=p) - torch.eye(A.size(1), dtype=A.dtype)
    return lin, lout


@torch.no_grad()
def yaqa_iterative(W, Lin, Lout, td_x, td_y, Q=nearest):
    """YAQA_iterative, bottom-right to top-left (gptq_2d_reference.py:308-334)."""
    m, n = W.shape
    hat = torch.zeros_like(W)
    for s in reversed(range(m // td_x + n // td_y - 1)):
        ii, jj = antidiagonal(s, m // td_x, n // td_y)
        idx = list(zip(ii.tolist(), jj.tolist()))
        targets = []
        for a, b in idx:
            rows, cols = slice(a * td_x, (a + 1) * td_x), slice(b * td_y, (b + 1) * td_y)
            down, right = slice(a * td_x, m), slice(b * td_y, n)
            targets.append(W[rows, cols] + (
                Lout[down, rows].t() @ (W[down, right] - hat[down, right]) @ Lin[right, cols]
                + Lout[down, rows].t() @ (W[down, cols] - hat[down, cols])
                + (W[rows, right] - hat[rows, right]) @ Lin[right, cols]
            ))
        qt = Q(torch.stack(targets), ii[:, None, None], jj[:, None, None])
        for k, (a, b) in enumerate(idx):
            hat[a * td_x:(a + 1) * td_x, b * td_y:(b + 1) * td_y] = qt[k]
    return hat


# ----------------------------------------------------------------------------------------------- instances

def random_instance(shape, seed, dtype=torch.float64, cond=10.):
    """Bases with condition number <= cond and X = 4 randn (gptq_2d_reference.py:337-351), CPU generator."""
    g = torch.Generator().manual_seed(seed)

    def basis(k):
        q1, _ = torch.linalg.qr(torch.randn(k, k, generator=g, dtype=dtype))
        q2, _ = torch.linalg.qr(torch.randn(k, k, generator=g, dtype=dtype))
        sv = cond ** torch.rand(k, generator=g, dtype=dtype)
        return (q1 * sv) @ q2.t()

    bases = [basis(k) for k in shape]
    X = 4. * torch.randn(shape, generator=g, dtype=dtype)
    return (*bases, X)


def coordinate_round(x, i, j):
    """Clipped coordinate-dependent codebook (gptq_2d_reference.py:354-357)."""
    scale = 2. ** ((i + 2 * j) % 3 - 1)
    return (x / scale).round().clamp(-3., 2.) * scale


def vectorized_alg1(X, A, B, Q=nearest, super_entry_shape=None):
    """Algorithm 1 on vec(X) with F factored on the explicit Kronecker Gram (gptq_2d_reference.py:360-382)."""
    m, n = X.shape
    p, q = super_entry_shape or (1, 1)
    mb = m // p
    rows = torch.arange(m).reshape(1, mb, 1, p)
    cols = torch.arange(n).reshape(n // q, 1, q, 1)
    perm = (cols * m + rows).flatten()
    F = ldl_of_inverse(torch.kron(B @ B.t(), A.t() @ A)[perm, :][:, perm], size=p * q)
    x = X.t().flatten()[perm]
    Qk = lambda y, k: Q(y, k % mb, k // mb)
    if super_entry_shape is None:
        z = alg1(x, F, Q=Qk)
    else:
        z = alg1_super_entry(x, F, Q=Qk, super_entry_shape=super_entry_shape)
    Z = torch.empty_like(z)
    Z[perm] = z
    return Z.reshape(n, m).t()


def kron_reduce(mats):
    """Kronecker product of a list, last factor fastest."""
    return functools.reduce(torch.kron, mats)
