"""Seeded synthetic layers for the benchmark configurations (inputs only; no algorithm here).

Every generator draws fp64 numbers from ``numpy.random.Generator(PCG64(seed))``, which is
platform-deterministic, before any cast.  Kronecker factors are "Wishart-like":

    F(k, alpha, seed) = G diag(s) G^T / (4k) + 1e-2 I,   G ~ N(0,1)^{k x 4k},  s_i = i^-alpha,

and weights are N(0, 0.02^2), optionally with 0.5% of the entries (chosen without replacement)
replaced by 0.1 * Student-t(3) outliers and optionally rounded to bf16.  The configurations follow
the benchmark definitions; the factors are the Grams A (rows) and B (columns), so the feedback
factors are L = ldl_of_inverse(A) and U = ldl_of_inverse(B)^T, and the objective is
tr(R^T A R B) with R = Z - X.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch


def wishart_factor(k: int, alpha: float, seed: int, device: str | torch.device = "cpu") -> torch.Tensor:
    """F(k, alpha, seed) in fp64 on ``device`` (the product is formed there, in column chunks)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    g = rng.standard_normal((k, 4 * k))
    s = np.arange(1, 4 * k + 1, dtype=np.float64) ** (-alpha)
    gt = torch.from_numpy(g).to(device)
    st = torch.from_numpy(s).to(device)
    out = torch.zeros(k, k, dtype=torch.float64, device=device)
    step = 8192
    for c0 in range(0, 4 * k, step):
        blk = gt[:, c0:c0 + step]
        out.addmm_(blk * st[c0:c0 + step], blk.t())
    out /= 4 * k
    out.diagonal().add_(1e-2)
    return out


def weights(m: int, n: int, seed: int, outliers: bool = True, bf16: bool = False) -> torch.Tensor:
    """W [m, n] in fp64 (CPU)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    w = 0.02 * rng.standard_normal((m, n))
    if outliers:
        count = int(round(0.005 * m * n))
        idx = rng.choice(m * n, size=count, replace=False)
        w.reshape(-1)[idx] = 0.1 * rng.standard_t(3, size=count)
    t = torch.from_numpy(w)
    if bf16:
        t = t.to(torch.bfloat16).to(torch.float64)
    return t


def abs_max_row_scale(w: torch.Tensor, qmin: int, qmax: int, dtype=torch.bfloat16) -> torch.Tensor:
    """Static symmetric scale of each row of w: absmax / ((qmax - qmin)/2) rounded to ``dtype``, 0 -> 1,
    as ``int_abs_max_scale_torch`` computes it, returned as [m, 1] in w's dtype."""
    divisor = w.new_full((), (qmax - qmin) / 2)
    s = w.abs().amax(dim=-1, keepdim=True).div_(divisor).to(dtype).to(w.dtype)
    return s.masked_fill_(s == 0, 1.)


def abs_max_group_scale(w: torch.Tensor, group: int, qmin: int, qmax: int, dtype=torch.bfloat16) -> torch.Tensor:
    """Static symmetric scale of each run of ``group`` consecutive entries along w's last mode (the abs-max
    scale of ``abs_max_row_scale`` per run), as a full tensor shaped like w."""
    runs = w.reshape(*w.shape[:-1], w.size(-1) // group, group)
    return abs_max_row_scale(runs, qmin, qmax, dtype).expand_as(runs).reshape(w.shape).contiguous()


def group_affine(w: torch.Tensor, group: int, qmax: int = 15):
    """Asymmetric scale (max-min)/qmax and zero point round(-min/s) per (row, group of columns), as full
    [m, n] tensors; min/max include 0 so the grid holds zero."""
    m, n = w.shape
    g = w.reshape(m, n // group, group)
    lo = g.amin(-1, keepdim=True).clamp(max=0)
    hi = g.amax(-1, keepdim=True).clamp(min=0)
    s = (hi - lo) / qmax
    s = torch.where(s == 0, torch.ones_like(s), s)
    z = torch.round(-lo / s)
    return s.expand_as(g).reshape(m, n).contiguous(), z.expand_as(g).reshape(m, n).contiguous()


@dataclasses.dataclass
class Config:
    name: str
    m: int
    n: int
    alpha: float
    outliers: bool
    bf16: bool
    quantizer: str  # "int_row" (symmetric per-row, static), "int_g128" (asymmetric per group)
    qmin: int
    qmax: int
    seeds: tuple = (0, 1, 2)


CONFIGS = {
    "C1": Config("C1", 512, 512, 0.5, False, False, "int_row", -8, 7),
    "C2": Config("C2", 4096, 4096, 0.5, True, True, "int_g128", 0, 15),
    "C3": Config("C3", 14336, 4096, 1.0, True, False, "int_row", -4, 3),
    "H": Config("H", 8192, 8192, 0.5, True, False, "int_row", -8, 7),
}


def quantizer_inputs(cfg: Config, w: torch.Tensor):
    """(scale, zero_point) full [m, n] tensors in w's dtype for the affine plug-in."""
    if cfg.quantizer == "int_row":
        s = abs_max_row_scale(w, cfg.qmin, cfg.qmax).expand_as(w).contiguous()
        return s, torch.zeros_like(w)
    if cfg.quantizer == "int_g128":
        return group_affine(w, 128, cfg.qmax)
    raise ValueError(cfg.quantizer)


def layer(cfg: Config, device="cpu", factor_device=None):
    """(W, A, B) in fp64: weights on ``device``, Grams formed on ``factor_device`` (default ``device``)."""
    sw, sa, sb = cfg.seeds
    fd = factor_device or device
    w = weights(cfg.m, cfg.n, sw, cfg.outliers, cfg.bf16).to(device)
    a = wishart_factor(cfg.m, cfg.alpha, sa, fd).to(device)
    b = wishart_factor(cfg.n, cfg.alpha, sb, fd).to(device)
    return w, a, b


@dataclasses.dataclass
class ThreeFactorConfig:
    """W [m, n1 n2] (columns c = b1 n2 + b2) under the Hessian A (m) (x) B1 (n1) (x) B2 (n2), quantized in
    1 x ``group`` super-entries with the abs-max INT quantizer (qmin..qmax, bf16 scales)."""
    name: str
    m: int
    n1: int
    n2: int
    alpha: float
    qmin: int
    qmax: int
    group: int
    seeds: tuple  # W, A, B1, B2


THREE_FACTOR = {
    "C5a": ThreeFactorConfig("C5a", 8192, 112, 256, 0.5, -8, 7, 32, (0, 1, 3, 4)),
}


def three_factor_layer(cfg: ThreeFactorConfig, device="cpu"):
    """(W, A, B1, B2) in fp64 on ``device``: W with 0.5% outliers, Wishart-like factors (s_i = i^-alpha)."""
    sw, sa, sb1, sb2 = cfg.seeds
    w = weights(cfg.m, cfg.n1 * cfg.n2, sw, True, False).to(device)
    a = wishart_factor(cfg.m, cfg.alpha, sa, device)
    b1 = wishart_factor(cfg.n1, cfg.alpha, sb1, device)
    b2 = wishart_factor(cfg.n2, cfg.alpha, sb2, device)
    return w, a, b1, b2
