"""Model-level driver: Kronecker-factor (Hessian) collection over calibration data, then every linear layer
quantized by GPTQ-2D on the GPU.

The reference quantizes one layer given its factors; its README (`README.md:19`) describes quantizing a
70B model, a pipeline it does not ship.  Here, for a linear layer y = W x (W [m, n]) the Hessian of the
loss is taken in the Kronecker form of K-FAC / YAQA: H ~ A (x) B with B = E[x x^T] over the layer's inputs
(n x n, the column side) and A = E[g g^T] over the gradients of the loss with respect to its outputs (m x m,
the row side; the identity when no backward pass is run, which is GPTQ's one-sided Hessian).  The objective
tr((Z - W)^T A (Z - W) B) is then the second-order change of the loss, and GPTQ-2D rounds W under
L = ldl_of_inverse(A), U = ldl_of_inverse(B)^T.

The Grams are accumulated with plain GEMMs (torch's addmm) in float64 by default; quantization runs the fused
HIP engine and the packed INT codes come from `packing`.
"""

from __future__ import annotations

import dataclasses
import functools
import time
from typing import Callable, Iterable

import torch

import gptq_2d as G
import gptq_2d_ldl as LDL
import packing
import quantizer_int as QI


class HessianCollector:
    """Running Kronecker factors of the linear layers of `model`: forward hooks add x^T x of every input batch
    (flattened to [tokens, n]) to B and (``output_side``) hook the output tensor, so that a backward pass adds
    g^T g of its gradient to A.
    Use it as a context manager or call ``remove()``; run forward (and backward) passes on calibration data
    in between."""

    def __init__(self, model: torch.nn.Module, layers: Iterable[str] | None = None, *, output_side: bool = True,
                 dtype: torch.dtype = torch.float64):
        self.dtype = dtype
        self.output_side = output_side
        names = set(layers) if layers is not None else None
        self.modules = {n: mod for n, mod in model.named_modules()
                        if isinstance(mod, torch.nn.Linear) and (names is None or n in names)}
        if names is not None and names - set(self.modules):
            raise ValueError(f"not linear layers of the model: {sorted(names - set(self.modules))}")
        self.B: dict[str, torch.Tensor] = {}
        self.A: dict[str, torch.Tensor] = {}
        self.tokens: dict[str, int] = {n: 0 for n in self.modules}
        self.grad_tokens: dict[str, int] = {n: 0 for n in self.modules}
        self._handles = []
        for name, mod in self.modules.items():
            self._handles.append(mod.register_forward_hook(functools.partial(self._forward, name)))

    @staticmethod
    def _gram(acc: dict, name: str, v: torch.Tensor, dtype) -> int:
        rows = v.detach().reshape(-1, v.size(-1)).to(dtype)
        if name not in acc:
            acc[name] = torch.zeros(rows.size(1), rows.size(1), dtype=dtype, device=rows.device)
        acc[name].addmm_(rows.t(), rows)
        return rows.size(0)

    def _forward(self, name, module, inputs, output):
        if not self._handles:
            return
        self.tokens[name] += self._gram(self.B, name, inputs[0], self.dtype)
        if self.output_side and output.requires_grad:
            # the gradient of the loss with respect to this output, when a backward pass reaches it
            output.register_hook(functools.partial(self._backward, name))

    def _backward(self, name, grad):
        if self._handles:
            self.grad_tokens[name] += self._gram(self.A, name, grad, self.dtype)

    def remove(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.remove()

    def factors(self, name: str, damping: float = 1e-2) -> tuple[torch.Tensor, torch.Tensor]:
        """(A, B) of layer `name`: the Grams averaged over their tokens, each with `damping` times its mean
        diagonal added to the diagonal (A is the identity without output-side statistics)."""
        if name not in self.B:
            raise KeyError(f"no inputs were seen by layer {name}")
        b = self.B[name] / max(1, self.tokens[name])
        m = self.modules[name].out_features
        if name in self.A and self.grad_tokens[name]:
            a = self.A[name] / self.grad_tokens[name]
        else:
            a = torch.eye(m, dtype=self.dtype, device=b.device)

        def damp(f):
            f = f.clone()
            f.diagonal().add_(damping * f.diagonal().mean().clamp_min(torch.finfo(f.dtype).tiny))
            return f
        return damp(a), damp(b)


@dataclasses.dataclass
class QuantSpec:
    """What ``quantize_model`` needs from a quantizer factory: the plug-in and its inputs for ``gptq_2d``, and
    -- for an affine INT quantizer -- the scale and zero point (broadcastable to the weight) and the code range
    its values are packed with (``pack_scale`` None: not packed)."""
    quantizer: Callable
    inputs: tuple = ()
    pack_scale: torch.Tensor | None = None
    pack_zero: torch.Tensor | None = None
    qmin: int = 0
    qmax: int = 0


def int_row_quantizer(weight: torch.Tensor, qmin: int = -8, qmax: int = 7) -> QuantSpec:
    """Symmetric INT quantizer with a static per-row scale (the abs-max of the row over (qmax - qmin) / 2,
    bf16-rounded, 0 -> 1), zero point 0 -- the headline configuration's quantizer."""
    divisor = weight.new_full((), (qmax - qmin) / 2)
    s = weight.abs().amax(dim=-1, keepdim=True).div_(divisor).to(torch.bfloat16).to(weight.dtype)
    s.masked_fill_(s == 0, 1.)
    full = s.expand_as(weight).contiguous()
    q = functools.partial(QI.affine_quantizer_hip, qmin=qmin, qmax=qmax)
    return QuantSpec(q, (full, torch.zeros_like(weight)), pack_scale=s, qmin=qmin, qmax=qmax)


@dataclasses.dataclass
class LayerResult:
    name: str
    shape: tuple
    objective: float        # tr(R^T A R B) of the GPTQ-2D rounding
    objective_rtn: float    # the same of rounding every entry on its own
    factors_ms: float
    sweep_ms: float
    words: torch.Tensor | None = None   # packed INT codes [m, ceil(n bits / 32)] (int32 bit patterns)
    scale: torch.Tensor | None = None   # the scale the codes were packed with (e.g. per row, [m, 1])
    zero_point: torch.Tensor | None = None


def _objective(r: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> float:
    r = r.double()
    return float(((a.double() @ r) * (r @ b.double())).sum())


@torch.no_grad()
def quantize_model(model: torch.nn.Module, collector: HessianCollector, *,
                   make_quantizer: Callable = int_row_quantizer, damping: float = 1e-2,
                   outer_block_size: int = 1024, pack: bool = True, layers: Iterable[str] | None = None,
                   dtype: torch.dtype = torch.float32) -> list[LayerResult]:
    """Quantize the collected linear layers of `model` in place, one after the other: factors
    L = ldl_of_inverse(A), U = ldl_of_inverse(B)^T (both in one call), the GPTQ-2D sweep of the weight in
    `dtype` with the `QuantSpec` that ``make_quantizer(weight)`` returns (built-in quantizers run fused),
    the result written back into the layer and (``pack``, for a spec with a pack scale) its INT codes packed.
    Each result carries the objective of the rounding and of rounding without feedback (the same quantizer
    under zero L and U).  Returns one `LayerResult` per layer."""
    results = []
    names = list(layers) if layers is not None else list(collector.modules)
    for name in names:
        lin = collector.modules[name]
        w = lin.weight.detach()
        assert w.is_cuda, "quantize_model runs on the GPU: move the model to a ROCm device"
        a, b = collector.factors(name, damping)
        a, b = a.to(dtype).to(w.device), b.to(dtype).to(w.device)
        torch.cuda.synchronize(w.device)
        t0 = time.perf_counter()
        lo, up = LDL.feedback_factors_of_grams(a, b)
        torch.cuda.synchronize(w.device)
        t1 = time.perf_counter()
        x = w.to(dtype).contiguous()
        spec = make_quantizer(x)
        z = G.gptq_2d(x, lo, up, quantizer=spec.quantizer, quantizer_inputs=spec.inputs,
                      outer_block_size=outer_block_size)
        torch.cuda.synchronize(w.device)
        t2 = time.perf_counter()
        zl, zu = torch.zeros_like(lo), torch.zeros_like(up)  # no feedback: each entry rounded on its own
        rtn = G.gptq_2d(x, zl, zu, quantizer=spec.quantizer, quantizer_inputs=spec.inputs)
        res = LayerResult(name, tuple(w.shape), _objective(z - x, a, b), _objective(rtn - x, a, b),
                          1e3 * (t1 - t0), 1e3 * (t2 - t1))
        if pack and spec.pack_scale is not None:
            res.words = packing.pack_int(z, spec.pack_scale, spec.pack_zero, qmin=spec.qmin, qmax=spec.qmax)
            res.scale, res.zero_point = spec.pack_scale, spec.pack_zero
        lin.weight.copy_(z.to(w.dtype))
        results.append(res)
    return results
