"""GPU tests of the feedback-factor preprocessing (gptq_2d_ldl) and of the strided GEMM beneath it.

The LDL factors are checked against the CPU oracle's restatement of ldl_of_inverse / ldl
(gptq_2d_reference.py:29-55, computed in fp64 with torch.linalg), and against what fixes them
independently of any implementation: unit (block) lower triangular with exactly identity diagonal
blocks, and L^{-1} M^{-1} L^{-T} block diagonal, which with the uniqueness of the LDL pins L.  Tolerances: fp64 1e-9, fp32 2e-4 relative to max |L| (well-conditioned Wishart-like
factors, condition number < 1e3).
"""

import ctypes
import time

import numpy as np

import pytest
import torch

import _hip
import gptq_2d_ldl as LDL
import instances
from oracle import algorithms as A

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gemm(M, N, K, batch, a, b, d, alpha, beta, a_tri=0, b_tri=0, d_tri=0, a_t=False, b_t=False):
    """Call gptq2d_gemm with a/b given as [batch, M, K] / [batch, K, N] tensors (possibly as transposed views)."""
    ars, acs = (a.stride(-2), a.stride(-1))
    brs, bcs = (b.stride(-2), b.stride(-1))
    _hip.call("gemm", d.dtype, M, N, K, batch, _hip.ptr(a), ars, acs, a.stride(0), _hip.ptr(b), brs, bcs, b.stride(0),
              _hip.ptr(d), d.stride(-2), d.stride(-1), d.stride(0), float(alpha), float(beta), a_tri, b_tri, d_tri,
              _hip.stream(d.device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("M,N,K", [(200, 300, 77), (128, 128, 16), (257, 129, 33), (64, 64, 1000), (5, 700, 9),
                                   (1000, 6, 64), (320, 256, 96), (130, 260, 36)])
@pytest.mark.parametrize("tri", [(0, 0, 0), (1, 0, 0), (0, 1, 0), (0, 0, 1), (2, 0, 0), (0, 2, 0), (2, 2, 0),
                                 (1, 1, 1)])
@pytest.mark.parametrize("b_layout", ["nk", "kn"])
def test_gemm(dtype, M, N, K, tri, b_layout):
    """Strided GEMM with triangular operand structure against a host fp64 product; the structurally zero
    parts hold NaN, which must not reach the result.  B is either a transposed view (contiguous along k)
    or contiguous along j, which selects the two layouts of the vectorised MFMA path.  The structures cover
    every fp64 tile order (rows, rows from the last, columns from the first or the last, a square lower D's
    triangle of tiles)."""
    print(f"gemm {M}x{N}x{K} {dtype} tri={tri} B {b_layout}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    batch = 2
    a = torch.randn(batch, M, K, generator=g, dtype=torch.float64)
    if b_layout == "nk":
        b = torch.randn(batch, N, K, generator=g, dtype=torch.float64).transpose(-1, -2)  # a transposed view
    else:
        b = torch.randn(batch, K, N, generator=g, dtype=torch.float64)
    d0 = torch.randn(batch, M, N, generator=g, dtype=torch.float64)
    a_tri, b_tri, d_tri = tri
    i = torch.arange(M)[:, None]
    k_a = torch.arange(K)[None, :]
    k_b = torch.arange(K)[:, None]
    j = torch.arange(N)[None, :]
    am = torch.ones(M, K, dtype=torch.bool) if a_tri == 0 else (k_a <= i if a_tri == 1 else k_a >= i)
    bm = torch.ones(K, N, dtype=torch.bool) if b_tri == 0 else (k_b >= j if b_tri == 1 else k_b <= j)
    dm = torch.ones(M, N, dtype=torch.bool) if d_tri == 0 else (i >= j)
    expected = d0 * .5 + 1.5 * (a * am) @ (b * bm)
    expected = torch.where(dm, expected, d0)
    a_dev = a.masked_fill(~am, torch.nan).to(dtype).to(DEV)
    b_dev = b.masked_fill(~bm, torch.nan).to(dtype)
    b_dev = (b_dev.transpose(-1, -2).contiguous().to(DEV).transpose(-1, -2) if b_layout == "nk"
             else b_dev.contiguous().to(DEV))
    d_dev = d0.to(dtype).to(DEV)
    _gemm(M, N, K, batch, a_dev, b_dev, d_dev, 1.5, .5, a_tri, b_tri, d_tri)
    got = d_dev.double().cpu()
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    err = ((got - expected).abs() / (1 + expected.abs())).max().item()
    assert err < tol * max(1, K ** .5), err


def _check_factor(got, m, size, inverse, tol):
    k = m.size(-1)
    expected = (A.ldl_of_inverse if inverse else A.ldl)(m.cpu().double(), size=size)
    g = got.double().cpu()
    blk = torch.arange(k) // size
    same = blk[:, None] == blk[None, :]
    above = blk[None, :] > blk[:, None]
    # exact structure: identity diagonal blocks, zero above
    assert torch.equal(g[same], torch.eye(k, dtype=torch.float64)[same])
    assert (g[above] == 0).all()
    err = ((g - expected).abs().max() / expected.abs().max()).item()
    assert err < tol, err
    # L^{-1} M^{-1} L^{-T} (inverse) or L^{-1} M L^{-T} (ldl) is block diagonal
    mm = m.cpu().double()
    target = torch.linalg.inv(mm) if inverse else mm
    li = torch.linalg.inv(g)
    lam = li @ target @ li.T
    off = lam.masked_fill(same, 0).abs().max() / lam.abs().max()
    assert off.item() < 50 * tol, off.item()


@pytest.mark.parametrize("k", [1, 5, 64, 65, 100, 257, 600, 777, 1000, 1536, 2052])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_ldl_of_inverse(k, dtype):
    """fp32 from k = 512 on: the inverse's level products on the triangular MFMA kernel (600, 1000:
    short last pairs and ragged 128-blocks; 1536: three full levels and a short one; 2052: the inverse
    split at its top level), or on the library's strided GEMM where rows are not 16-byte aligned (777)."""
    print(f"ldl_of_inverse k={k} {dtype}", flush=True)
    m = instances.wishart_factor(k, .5, 10 + k).to(dtype).to(DEV)
    got = LDL.ldl_of_inverse(m)
    _check_factor(got, m, 1, True, 1e-9 if dtype == torch.float64 else 2e-4)


@pytest.mark.parametrize("k,size", [(64, 2), (96, 4), (256, 16), (128, 32), (192, 64), (240, 48), (384, 96),
                                    (256, 128)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_ldl_of_inverse_blocks(k, size, dtype):
    """Diagonal blocks up to the one-wave register inverse (64 fp32, 32 fp64) and, above it, the LDS solve
    (up to 128 fp32, 64 fp64; larger blocks are refused)."""
    if size > LDL.MAX_BLOCK[dtype]:
        with pytest.raises(AssertionError):
            LDL.ldl_of_inverse(torch.eye(k, dtype=dtype, device=DEV), size=size)
        return
    print(f"ldl_of_inverse k={k} size={size} {dtype}", flush=True)
    m = instances.wishart_factor(k, 1., 20 + k).to(dtype).to(DEV)
    got = LDL.ldl_of_inverse(m, size=size)
    _check_factor(got, m, size, True, 1e-9 if dtype == torch.float64 else 2e-4)


@pytest.mark.parametrize("k,size", [(70, 1), (128, 8)])
def test_ldl(k, size):
    m = instances.wishart_factor(k, .5, 30 + k).to(DEV)
    got = LDL.ldl(m, size=size)
    _check_factor(got, m, size, False, 1e-9)


def test_batch_and_feedback_factors():
    ms = torch.stack([instances.wishart_factor(48, .5, s) for s in range(6)]).reshape(2, 3, 48, 48).to(DEV)
    got = LDL.ldl_of_inverse(ms, size=4)
    for idx in np.ndindex(2, 3):
        expected = A.ldl_of_inverse(ms[idx].cpu(), size=4)
        assert (got[idx].cpu() - expected).abs().max() < 1e-9
    g = torch.Generator().manual_seed(3)
    a = torch.randn(40, 24, generator=g, dtype=torch.float64)
    b = torch.randn(30, 50, generator=g, dtype=torch.float64)
    lo, up = LDL.feedback_factors(a.to(DEV), b.to(DEV), (2, 5))
    elo, eup = A.feedback_factors(a, b, (2, 5))
    assert (lo.cpu() - elo).abs().max() < 1e-9 and (up.cpu() - eup).abs().max() < 1e-9


@pytest.mark.parametrize("k", [256, 2048])
def test_grouped_batch_fp32(k):
    """fp32 batches factored in groups that share every Cholesky launch (16 at a time, here 16 + 2 or 3 + 0):
    each matrix equals its own call bitwise, for ldl_of_inverse and ldl, and so do batched factor pairs;
    a matrix that is not positive definite inside a group is reported as that batch entry."""
    nb = 18 if k == 256 else 3
    print(f"grouped batch k={k} nb={nb}", flush=True)
    ms = torch.stack([instances.wishart_factor(k, .5, 90 + s) for s in range(nb)]).float().to(DEV)
    for fn in (LDL.ldl_of_inverse, LDL.ldl):
        got = fn(ms)
        for b in range(nb):
            assert got[b].equal(fn(ms[b])), (fn.__name__, b)
    hs = torch.stack([instances.wishart_factor(k // 2, .5, 120 + s) for s in range(nb)]).float().to(DEV)
    lo, up = LDL.feedback_factors_of_grams(ms, hs, check=False)
    for b in range(nb):
        assert lo[b].equal(LDL.ldl_of_inverse(ms[b])) and up[b].equal(LDL.ldl_of_inverse(hs[b]).t()), b
    bad = ms.clone()
    bad[nb - 2, k // 2, k // 2] = -1.
    with pytest.raises(torch.linalg.LinAlgError, match=f"batch {nb - 2}"):
        LDL.ldl_of_inverse(bad)


def test_not_positive_definite():
    m = instances.wishart_factor(80, .5, 1).to(DEV)
    m[70, 70] = -1.
    with pytest.raises(torch.linalg.LinAlgError):
        LDL.ldl_of_inverse(m)
    with pytest.raises(torch.linalg.LinAlgError):
        LDL.ldl(m)


def test_concurrent_factors_deterministic():
    """Regression: the two factorisations of feedback_factors_of_grams run concurrently on two streams, so a
    panel launch's workgroups may start late, behind the other stream's work.  They must still read the
    unfactored diagonal block (the factored one is staged and copied into place by a later launch): every
    run equals the single-stream ldl_of_inverse of each factor, bitwise."""
    a = instances.wishart_factor(8192, .5, 1, device=DEV).float()
    b = instances.wishart_factor(8192, .5, 2, device=DEV).float()
    ref_l = LDL.ldl_of_inverse(a, check=False)
    ref_u = LDL.ldl_of_inverse(b, check=False).t()
    for rep in range(24):
        lo, up = LDL.feedback_factors_of_grams(a, b, check=False)
        assert lo.equal(ref_l) and up.equal(ref_u), rep


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("ka,kb", [(777, 600), (100, 257), (65, 64), (600, 600), (2052, 2052)])
def test_feedback_factors_of_grams_ragged(ka, kb, dtype):
    """Sizes that are not multiples of the panel width: the factor pair equals the single-stream factors
    bitwise (the inverse-only part starts at column k, past the last panel).  Equal fp32 sizes share
    every Cholesky launch (the second matrix as blockIdx.y = 1); 2052 also splits the inverse."""
    print(f"feedback_factors_of_grams {ka} {kb} {dtype}", flush=True)
    a = instances.wishart_factor(ka, .5, 40 + ka).to(dtype).to(DEV)
    b = instances.wishart_factor(kb, .5, 50 + kb).to(dtype).to(DEV)
    lo, up = LDL.feedback_factors_of_grams(a, b, (1, 1))
    assert lo.equal(LDL.ldl_of_inverse(a)) and up.equal(LDL.ldl_of_inverse(b).t())
    _check_factor(lo, a, 1, True, 1e-9 if dtype == torch.float64 else 2e-4)


@pytest.mark.parametrize("k,cuts,dtype", [(601, (64, 320), torch.float32), (600, (64, 320), torch.float64),
                                          (1536, (192, 640), torch.float64)])
def test_cholesky_in_parts_plain(k, cuts, dtype):
    """The one-panel-per-launch Cholesky (fp64, and fp32 with k % 4 != 0) split over calls that end inside a
    256-column strip: a part leaves its strip's trailing update pending, and the next part's left-looking
    panel updates and the strip-end update read the strip's factored columns from W, so the parts issue
    the one call's launches in the same order and give its factor bit for bit."""
    print(f"cholesky in parts (plain path) k={k} cuts={cuts} {dtype}", flush=True)
    m = instances.wishart_factor(k, .5, 70 + k).to(dtype).to(DEV)
    out, work = torch.empty_like(m), torch.empty_like(m)
    info = torch.zeros(1, dtype=torch.int32, device=DEV)
    bounds = (0,) + cuts + (-1,)
    for c0, c1 in zip(bounds[:-1], bounds[1:]):
        LDL._part(m, out, work, info, k, 1, c0, c1, 0)
    LDL._part(m, out, work, info, k, 1, k, -1, 1)
    torch.cuda.synchronize()
    assert info.item() == 0
    assert out.equal(LDL.ldl_of_inverse(m))
    _check_factor(out, m, 1, True, 1e-9 if dtype == torch.float64 else 2e-4)


@pytest.mark.parametrize("k,cuts", [(1536, (192, 640)), (600, (64, 320, 512)), (8192, (4160,))])
def test_cholesky_in_parts(k, cuts):
    """The Cholesky split over calls at panel boundaries that cut the strips of the fp32 path (512 columns,
    1024 from k = 8192): each call ends with the update of everything right of its range, so the parts make
    the same factor (up to rounding: the strips' updates are grouped differently)."""
    print(f"cholesky in parts k={k} cuts={cuts}", flush=True)
    m = instances.wishart_factor(k, .5, 60 + k).float().to(DEV)
    out, work = torch.empty_like(m), torch.empty_like(m)
    info = torch.zeros(1, dtype=torch.int32, device=DEV)
    bounds = (0,) + cuts + (-1,)
    for c0, c1 in zip(bounds[:-1], bounds[1:]):
        LDL._part(m, out, work, info, k, 1, c0, c1, 0)
    LDL._part(m, out, work, info, k, 1, k, -1, 1)
    torch.cuda.synchronize()
    assert info.item() == 0
    ref = LDL.ldl_of_inverse(m)
    err = ((out - ref).abs().max() / ref.abs().max()).item()
    print(f"  parts vs one call: max rel diff {err:.2e}", flush=True)
    assert err < 1e-4
    if k <= 2048:
        _check_factor(out, m, 1, True, 2e-4)


def test_headline_size_fp32():
    """8192 x 8192 fp32 factor of the headline layer: structure, and agreement with the fp64 oracle on a
    sampled set of rows (the full fp64 CPU reference takes too long here)."""
    k = 8192
    m64 = instances.wishart_factor(k, .5, 1, device=DEV)
    got = LDL.ldl_of_inverse(m64.float())
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert (got.diagonal() == 1).all() and (got.triu(1) == 0).all()
    ref = LDL.ldl_of_inverse(m64)  # the GPU fp64 path, pinned against the oracle above
    err = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    print(f"8192 fp32 vs fp64: max rel err {err:.2e}", flush=True)
    assert err < 1e-3


@pytest.mark.timeout(600)
def test_beyond_2_29_elements_fp32():
    """A 24576 x 24576 fp32 factor (6.0e8 elements, past 2^29: the 28672-column Grams of a 70B MLP are larger
    still) on the two-level Cholesky and the MFMA inverse levels, whose buffer offsets are relative to their
    blocks' rows: structure, agreement with the fp64 path, and faster than the one-panel-per-launch sequence
    (forced by a size that is not a multiple of 4)."""
    k = 24576
    gen = torch.Generator(device=DEV).manual_seed(5)
    g = torch.randn(k, k // 2, generator=gen, device=DEV, dtype=torch.float64)
    m64 = g @ g.t() / (k // 2)
    m64.diagonal().add_(.1)
    del g
    m32 = m64.float()
    LDL.ldl_of_inverse(m32[:512, :512])  # load and warm up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    got = LDL.ldl_of_inverse(m32)
    torch.cuda.synchronize()
    t_two = time.perf_counter() - t0
    assert torch.isfinite(got).all()
    assert (got.diagonal() == 1).all() and (got.triu(1) == 0).all()
    ref = LDL.ldl_of_inverse(m64)
    err = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    del ref
    m_odd = m32[:k - 2, :k - 2].contiguous()  # k % 4 != 0: the one-panel-per-launch sequence
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    LDL.ldl_of_inverse(m_odd)
    torch.cuda.synchronize()
    t_plain = time.perf_counter() - t0
    print(f"{k} fp32 vs fp64: max rel err {err:.2e}; {1e3 * t_two:.0f} ms (two-level) against {1e3 * t_plain:.0f} ms "
          f"(plain sequence, k = {k - 2})", flush=True)
    assert err < 1e-3
    assert t_two < t_plain


@pytest.mark.parametrize("k", [3584, 7168])
def test_split_inverse_fp32(k):
    """fp32 factors whose triangular inverse splits at 2048 / 4096 with a trailing block that is not a power of
    two (1536, 3072: short pairs at the top of its recursive doubling): against the fp64 path (not split), and
    the factor pair (part 1 of each inverse on a side stream beside the shared Cholesky chain) against single
    calls bitwise."""
    print(f"split inverse k={k}", flush=True)
    m64 = instances.wishart_factor(k, .5, 70 + k, device=DEV)
    m = m64.float()
    got = LDL.ldl_of_inverse(m)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    assert (got.diagonal() == 1).all() and (got.triu(1) == 0).all()
    ref = LDL.ldl_of_inverse(m64)
    err = ((got.double() - ref).abs().max() / ref.abs().max()).item()
    print(f"  fp32 vs fp64: max rel err {err:.2e}", flush=True)
    assert err < 1e-3
    b = instances.wishart_factor(k, .5, 80 + k, device=DEV).float()
    lo, up = LDL.feedback_factors_of_grams(m, b, check=False)
    assert lo.equal(got) and up.equal(LDL.ldl_of_inverse(b, check=False).t())
    assert up.is_contiguous()  # U written by the library, not a transposed view


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("k", [0, 96, 640])
def test_info_zeroed_by_library(dtype, k):
    """The C ABI reports the pivot status in info itself: info pre-filled with garbage (a stale failure) reads 0
    after a successful factorisation, on two calls in a row, through all three LDL entry points."""
    print(f"info k={k} {dtype}", flush=True)
    m = instances.wishart_factor(max(k, 1), .5, 3)[:k, :k].to(DEV, dtype).contiguous()
    out, work = torch.empty_like(m), torch.empty_like(m)
    st = _hip.stream(m.device)
    for _ in range(2):
        info = torch.full((1,), 12345, dtype=torch.int32, device=DEV)
        _hip.call("ldl_of_inverse", dtype, _hip.ptr(m), _hip.ptr(out), _hip.ptr(work), _hip.ptr(info), 1, k, 1, st)
        torch.cuda.synchronize()
        assert int(info.item()) == 0
        info.fill_(-7)
        _hip.call("ldl_of_inverse_part", dtype, _hip.ptr(m), _hip.ptr(out), _hip.ptr(work), _hip.ptr(info), k, 1, 0,
                  -1, 1, st)
        torch.cuda.synchronize()
        assert int(info.item()) == 0
    m1 = m.clone()
    out1, work1 = torch.empty_like(m), torch.empty_like(m)
    infos = torch.full((2,), 99, dtype=torch.int32, device=DEV)
    streams = [torch.cuda.Stream() for _ in range(3)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    _hip.call("ldl_of_inverse_pair", dtype, _hip.ptr(m), _hip.ptr(out), _hip.ptr(work), _hip.ptr(infos[0:1]), k, 1,
              _hip.ptr(m1), _hip.ptr(out1), _hip.ptr(work1), _hip.ptr(infos[1:2]), k, 1, 0,
              *(ctypes.c_void_p(s.cuda_stream) for s in streams))
    torch.cuda.synchronize()
    assert infos.tolist() == [0, 0]
    if k:  # U = L^T only for unit diagonal blocks: a block size with upper1 is refused before any launch
        with pytest.raises(_hip.GPTQ2DError):
            _hip.call("ldl_of_inverse_pair", dtype, _hip.ptr(m), _hip.ptr(out), _hip.ptr(work), _hip.ptr(infos[0:1]),
                      k, 1, _hip.ptr(m1), _hip.ptr(out1), _hip.ptr(work1), _hip.ptr(infos[1:2]), k, 2, 1,
                      *(ctypes.c_void_p(s.cuda_stream) for s in streams))
