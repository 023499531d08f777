"""Feedback factors of GPTQ-2D on the GPU: the LDL helpers of the reference, HIP-backed.

``ldl_of_inverse(M, size)`` gives the unit lower (block) triangular L with M^{-1} = L Lambda L^T
without forming M^{-1}; ``ldl(M, size)`` the same for M itself; ``feedback_factors(A, B, shape)``
the pair (L, U) that ``gptq_2d`` takes for the Grams G = A^T A and H = B B^T.  Same names,
arguments and results as the reference (gptq_2d_reference.py:29-66); leading batch dimensions of
M are supported.  Everything runs on the current stream of M's device in blocked HIP kernels
(reverse-order Cholesky, recursive-doubling triangular inverse, normalisation; the GEMM-shaped
parts on fp32 MFMA).  A matrix that is not positive definite raises
``torch.linalg.LinAlgError`` as ``torch.linalg.cholesky`` does; ``check=False`` skips that test
(it is the only host synchronisation) so that ``ldl_of_inverse`` and ``ldl`` can be captured in a graph.
``feedback_factors_of_grams``, which spreads the two factors over three side streams, refuses to run
under stream capture: capture the two ``ldl_of_inverse`` calls instead.
"""

from __future__ import annotations

import ctypes

import torch

import _hip

# p x p diagonal blocks up to this size are normalised on the GPU (one wave's register inverse up to 64 /
# 32, a triangular solve against the block in LDS above that).
MAX_BLOCK = {torch.float32: 128, torch.float64: 64}

# Three side streams per device for feedback_factors_of_grams (created once: a new stream per call
# would cost a stream creation and defeat the caching allocator's reuse of its blocks).
_SIDE_STREAMS: dict = {}


def _side_streams(device: torch.device):
    key = torch.device(device).index if torch.device(device).index is not None else torch.cuda.current_device()
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = tuple(torch.cuda.Stream(device=key) for _ in range(3))
    return _SIDE_STREAMS[key]


def _factor(name: str, m: torch.Tensor, size: int, check: bool) -> torch.Tensor:
    assert m.dim() >= 2 and m.size(-1) == m.size(-2), "expected square matrices [..., k, k]"
    assert m.dtype in (torch.float32, torch.float64), "expected float32 or float64"
    _hip.require_device(m)
    k = m.size(-1)
    assert size > 0 and k % size == 0, "the block size must divide the matrix size"
    assert size <= MAX_BLOCK[m.dtype], f"diagonal blocks up to {MAX_BLOCK[m.dtype]} are supported for {m.dtype}"
    batch = m.shape[:-2]
    src = m.reshape(-1, k, k).contiguous()
    nb = src.size(0)
    out = torch.empty_like(src)
    work = torch.empty_like(src)
    info = torch.zeros(nb, dtype=torch.int32, device=m.device)
    with torch.cuda.device(m.device):
        _hip.call(name, m.dtype, _hip.ptr(src), _hip.ptr(out), _hip.ptr(work), _hip.ptr(info), nb, k, size,
                  _hip.stream(m.device))
    if check and nb and k:
        bad = info.cpu()
        if bool((bad != 0).any()):
            b = int((bad != 0).nonzero()[0, 0])
            raise torch.linalg.LinAlgError(
                f"the leading minor of order {int(bad[b])} of batch {b} is not positive-definite")
    return out.reshape(*batch, k, k)


def ldl_of_inverse(M: torch.Tensor, size: int = 1, *, check: bool = True) -> torch.Tensor:
    """Unit lower (block) triangular L with M^{-1} = L Lambda L^T, Lambda block diagonal with size x size
    blocks, via the reverse-order Cholesky M = Um Um^T and L = Um^{-T} normalised by its diagonal blocks
    (gptq_2d_reference.py:41-49)."""
    return _factor("ldl_of_inverse", M, size, check)


def ldl(M: torch.Tensor, size: int = 1, *, check: bool = True) -> torch.Tensor:
    """Unit lower (block) triangular L with M = L Lambda L^T (gptq_2d_reference.py:52-55)."""
    return _factor("ldl", M, size, check)


def _part(m, out, work, info, k, size, col_begin, col_end, finish):
    """One part of ldl_of_inverse of the k x k matrix m on the current stream (see the C ABI)."""
    _hip.call("ldl_of_inverse_part", m.dtype, _hip.ptr(m), _hip.ptr(out), _hip.ptr(work), _hip.ptr(info), k, size,
              col_begin, col_end, finish, _hip.stream(m.device))


def feedback_factors_of_grams(G: torch.Tensor, H: torch.Tensor, super_entry_shape=(1, 1), *, check: bool = True):
    """(L, U) = (ldl_of_inverse(G, p), ldl_of_inverse(H, q)^T) from the Grams themselves, both at once on
    three side streams of the current device (gptq2d_ldl_of_inverse_pair): the two Cholesky
    factorisations -- chains of latency-bound panel launches -- share every launch when the factors are
    fp32 of one size (else they run together on two streams), and the first part of each triangular
    inverse runs beside the rest of the factorisations.  Batched Grams: each factor's batch in one call on
    its own stream, its matrices sharing the Cholesky launches in groups of up to 16.  Bitwise equal to the
    two ldl_of_inverse calls.  No counterpart in the reference, whose callers compute the two factors one
    after the other (demo.ipynb cell 5)."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("feedback_factors_of_grams runs on three side streams and cannot be captured in a graph; "
                           "capture ldl_of_inverse(G, p) and ldl_of_inverse(H, q).T instead")
    p, q = super_entry_shape
    main = torch.cuda.current_stream(G.device)
    streams = _side_streams(G.device)
    for s in streams:
        s.wait_stream(main)
    jobs = []
    for m, size in ((G, p), (H, q)):
        assert m.dim() >= 2 and m.size(-1) == m.size(-2), "expected square matrices [..., k, k]"
        assert m.dtype in (torch.float32, torch.float64), "expected float32 or float64"
        _hip.require_device(m)
        k = m.size(-1)
        assert size > 0 and k % size == 0, "the block size must divide the matrix size"
        assert size <= MAX_BLOCK[m.dtype], f"diagonal blocks up to {MAX_BLOCK[m.dtype]} are supported for {m.dtype}"
        jobs.append((m, size, k))
    out = []
    upper = False  # whether out[1] holds U itself (else the second factor, U its transpose)
    with torch.cuda.device(G.device):
        # each factor's buffers on its stream's pool
        bufs = []
        for s, (m, size, k) in zip(streams, jobs):
            with torch.cuda.stream(s):
                src = m.reshape(-1, k, k).contiguous()
                bufs.append((src, torch.empty_like(src), torch.empty_like(src),
                             torch.zeros(src.size(0), dtype=torch.int32, device=m.device)))
        (sa, oa, wa, ia), (sb, ob, wb, ib) = bufs
        (_, pa, ka), (_, pb, kb) = jobs
        if max(sa.size(0), sb.size(0)) > 1:
            # batches: each factor's matrices in one batched call on its own stream, whose matrices of the
            # fp32 two-level path share every Cholesky launch (up to 16 at a time)
            for s, (m, size, k), (src, o, w, info) in zip(streams, jobs, bufs):
                with torch.cuda.stream(s):
                    _hip.call("ldl_of_inverse", src.dtype, _hip.ptr(src), _hip.ptr(o), _hip.ptr(w), _hip.ptr(info),
                              src.size(0), k, size, _hip.stream(m.device))
        elif sa.dtype == sb.dtype and sa.size(0) == sb.size(0):
            # U = ldl_of_inverse(H)^T written by the library (unit diagonal): no transposed copy in the sweep
            upper = pb == 1
            sp = [ctypes.c_void_p(s.cuda_stream) for s in streams]
            for b in range(sa.size(0)):
                _hip.call("ldl_of_inverse_pair", sa.dtype, _hip.ptr(sa[b]), _hip.ptr(oa[b]), _hip.ptr(wa[b]),
                          _hip.ptr(ia[b:b + 1]), ka, pa, _hip.ptr(sb[b]), _hip.ptr(ob[b]), _hip.ptr(wb[b]),
                          _hip.ptr(ib[b:b + 1]), kb, pb, int(upper), *sp)
        else:  # one matrix each, of different dtypes: each factor on its own stream
            for s, (m, size, k), (src, o, w, info) in zip(streams, jobs, bufs):
                with torch.cuda.stream(s):
                    for b in range(src.size(0)):
                        _part(src[b], o[b], w[b], info[b:b + 1], k, size, 0, -1, 1)
        out = [oa.reshape(G.shape), ob.reshape(H.shape)]
    # streams[2]'s work is ordered before the last launches of streams[0] and [1] (events)
    for s, t in zip(streams, out):
        main.wait_stream(s)
        t.record_stream(main)
    if check:
        for t, m in zip(out, (G, H)):
            if not bool(torch.isfinite(t).all()):
                ldl_of_inverse(m, size=1)  # raises the LinAlgError with the failing minor
    return out[0], out[1] if upper else out[1].transpose(-1, -2)


def feedback_factors(A: torch.Tensor, B: torch.Tensor, super_entry_shape=(1, 1)):
    """L and U for the Grams G = A^T A and H = B B^T, with p x p and q x q identity diagonal blocks
    (gptq_2d_reference.py:58-66)."""
    p, q = super_entry_shape
    L = ldl_of_inverse(A.t() @ A, size=p)
    U = ldl_of_inverse(B @ B.t(), size=q).t()
    return L, U
