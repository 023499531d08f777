"""D-sided GPTQ-2D on MI355X: the rounding of an n_1 x ... x n_D tensor under a Kronecker Hessian
H_1 (x) ... (x) H_D (one Gram per mode), which the reference runs only as its CPU listing of
Algorithm 4 (``alg4``, gptq_2d_reference.py:270-294; with the direct form ``alg2_d_sided`` :248-267).

Algorithm 4 equals Algorithm 1 on the column-major vec(X) with the feedback factor
F = L_D (x) ... (x) L_1 (L_d = ldl_of_inverse(H_d)), and so does the two-sided sweep of the
n_1 x (n_2 ... n_D) matrix whose column index is i_2 + n_2 (i_3 + n_3 (...)) under L = L_1 and
U = (L_D (x) ... (x) L_2)^T -- the same vec order and the same factor.  The GPU path therefore runs
the tensor on the two-sided engine: X permuted to modes (1, D, ..., 2) and flattened, U passed as the
Kronecker pair (L_D^T (x) ... (x) L_3^T, L_2^T) -- read from its factors by the fused fp32 engine where n_2 is
a multiple of 16, formed once as the product (n_2 ... n_D squared entries) elsewhere --, the fused tile sweep
(built-in quantizers) or the per-stage plug-in path, and the result permuted back.  The rounding decisions are those of
Algorithm 4 in exact arithmetic (bitwise in fp64 on the test instances); the schedule is the two-sided
engine's tiles rather than Algorithm 4's 1 + sum_d (n_d - 1) hyper-antidiagonals.
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch

import gptq_2d as _g2
from quantizer_int import round_quantizer


def _unit_lower(f: torch.Tensor) -> torch.Tensor:
    """The unit lower triangular factor that f's strict lower triangle defines (the rest of f is not read)."""
    k = f.size(-1)
    return f.tril(-1) + torch.eye(k, dtype=f.dtype, device=f.device)


def mode_permutation(D: int) -> tuple:
    """Modes (1, D, D-1, ..., 2) (0-based: (0, D-1, ..., 1)): flattening the permuted tensor's trailing modes
    gives the column index i_2 + n_2 (i_3 + n_3 (...))."""
    return (0, *range(D - 1, 0, -1))


def column_factor(ls: Sequence[torch.Tensor]) -> torch.Tensor:
    """U = (L_D (x) ... (x) L_2)^T = L_D^T (x) ... (x) L_2^T, unit upper triangular of size n_2 ... n_D, formed
    from the transposed mode factors: every entry is the same product of the same factor entries as in the
    transposed product (equal bits), without a transposed copy of the n_2 ... n_D squared result."""
    f = _unit_lower(ls[-1]).t()
    for fd in reversed(ls[1:-1]):
        f = torch.kron(f, _unit_lower(fd).t())
    return f.contiguous()


def column_factor_pair(ls: Sequence[torch.Tensor]):
    """column_factor(ls) as the Kronecker pair of its last product, (L_D^T (x) ... (x) L_3^T) (x) L_2^T
    (gptq_2d.KroneckerU; D >= 3): the outer factor is the product column_factor forms before its last step, so
    the pair's entries are column_factor's bit for bit.  D = 2: the single factor L_2^T."""
    if len(ls) == 2:
        return column_factor(ls)
    return _g2.KroneckerU(column_factor([ls[0], *ls[2:]]), _unit_lower(ls[1]).t().contiguous())


@torch.no_grad()
def gptq_d_sided(x: torch.Tensor, ls: Sequence[torch.Tensor], *, quantizer: Callable = round_quantizer,
                 quantizer_inputs: tuple = (), inplace: bool = False, outer_block_size: int = 1024,
                 fused: bool | None = None) -> torch.Tensor:
    """Round x [n_1, ..., n_D] (D >= 2) under unit lower triangular factors ls[d] [n_d, n_d]
    (ls[d] = ldl_of_inverse(H_d), the paper's L^(d+1); read strictly below the diagonal).

    ``quantizer`` follows the two-sided plug-in protocol (gptq_2d.py:147-164) on the flattened
    [n_1, n_2 ... n_D] matrix (mode 2 fastest along its columns); ``quantizer_inputs`` are tensors shaped
    like x and are flattened the same way -- without a copy when their memory is already in that order
    (a tensor allocated as [n_1, n_D, ..., n_2] and permuted to x's modes), so a quantizer that writes
    into an input writes into the caller's tensor only then.  With ``inplace`` the result is written back
    into x.
    """
    D = x.dim()
    assert D >= 2, "the D-sided sweep needs a tensor of at least two modes"
    assert len(ls) == D, "one factor per mode"
    assert all(f.shape == (k, k) for f, k in zip(ls, x.shape)), "factor d must be [n_d, n_d]"
    assert all(f.dtype == x.dtype and f.device == x.device for f in ls), "factors must match x's dtype and device"
    assert all(t.shape == x.shape for t in quantizer_inputs), "quantizer inputs must be shaped like x"
    if x.numel() == 0:
        return x if inplace else x.clone()
    perm = mode_permutation(D)
    n1 = x.size(0)
    w = x.permute(*perm).reshape(n1, -1)
    # x already in the flattened order: the sweep runs on its memory when it may write there
    in_place_2d = inplace and w.is_contiguous() and w.data_ptr() == x.data_ptr()
    # otherwise the flattening copied x, and the sweep may run on that copy instead of a clone of it
    fresh = w.untyped_storage().data_ptr() != x.untyped_storage().data_ptr()
    z = _g2.gptq_2d(w, ls[0].contiguous(), column_factor_pair(ls), quantizer=quantizer,
                    quantizer_inputs=tuple(t.permute(*perm).reshape(n1, -1).contiguous() for t in quantizer_inputs),
                    outer_block_size=outer_block_size, inplace=in_place_2d or fresh, fused=fused)
    out = z.reshape(n1, *(x.size(d) for d in perm[1:])).permute(*[perm.index(d) for d in range(D)])
    if inplace:
        if not in_place_2d:
            x.copy_(out)
        return x
    return out.contiguous()
