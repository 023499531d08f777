"""Write golden vectors from the reference implementation (build container only).

Imports the reference's PyTorch code from /root/reference (gptq_2d.py, quantizer_int.py,
quantizer_trellis.py) on the CPU, only for the results that no closed form, invariant or brute
force pins:

* c1_int4.npz   -- fp32 ``gptq_2d_torch`` codes of configuration C1 (512 x 512, INT4 symmetric
                   per-row static bf16 scale through ``affine_quantizer_torch``), with the L and U it
                   ran on (stored, since LAPACK bits may differ between machines), each entry's Y just
                   before rounding in code units, and the objective tr(R^T A R B).
* trellis.npz   -- the default HYB look-up table (seeded k-means), SHA-256 digests of the 1MAD/3INST/HYB
                   tables, and Viterbi states/values of ``_trellis_quantize_torch`` on seeded sequences,
                   including HYB L=16 K=2 V=2 T=256 with and without tail-biting.
* scales.npz    -- ``int_abs_max_scale_torch`` on rows with zeros and denormal scales, bf16 and fp16.
* absmax.npz    -- ``int_abs_max_quantizer_torch`` on the cases of the reference's own test
                   (quantizer_int.py:535-553): the 1 x 32 and 2 x 24 selectors, (qmin, qmax) in
                   {(-2, 1), (-4, 3), (-8, 7), (-128, 127)}, fp16 and bf16 scales, a zero row and a
                   1e-38 row (denormal or vanishing scale), in fp32 and fp64, with a CPU generator;
                   plus rows built so that every entry is an exact tie k + 1/2 of its scale for each
                   (qmin, qmax), and a 48 x 96 matrix quantized as 1 x 32 super-entries (the input of
                   the fused row sweep's check).

Run from the repository root: ``python tests/golden/make_golden.py``.  The reference never
travels to the GPU box; only these data files do.
"""

from __future__ import annotations

import functools
import hashlib
import pathlib
import sys

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
OUT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gptq-2d_amd"))
sys.path.insert(0, str(ROOT))
sys.path.insert(0, "/root/reference")

import gptq_2d as ref_sweep  # noqa: E402  (the reference's module of this name)
import quantizer_int as ref_qi  # noqa: E402
import quantizer_trellis as ref_tr  # noqa: E402

assert pathlib.Path(ref_sweep.__file__).parent == pathlib.Path("/root/reference"), ref_sweep.__file__

import instances  # noqa: E402  (this repository's seeded generators)
from oracle import algorithms as alg  # noqa: E402


def c1():
    cfg = instances.CONFIGS["C1"]
    w, a, b = instances.layer(cfg)
    lo = alg.ldl_of_inverse(a)
    up = alg.ldl_of_inverse(b).t()
    x, l, u = w.float(), lo.float().contiguous(), up.float().contiguous()
    scale, zp = instances.quantizer_inputs(cfg, x)
    ypre = torch.full_like(x, float("nan"))
    base = functools.partial(ref_qi.affine_quantizer_torch, qmin=cfg.qmin, qmax=cfg.qmax)

    def spy(y_flat, sl, s, z, *, out):
        ypre.view(-1)[sl] = y_flat[sl]
        base(y_flat, sl, s, z, out=out)

    zq = ref_sweep.gptq_2d_torch(x, l, u, quantizer=spy, quantizer_inputs=(scale, zp))
    codes = torch.round(zq / scale)
    assert torch.equal(codes * scale, zq)
    r = (zq - x).double()
    obj = float(((a @ r) * (r @ b)).sum())
    rtn = torch.clamp(torch.round(x / scale), cfg.qmin, cfg.qmax) * scale
    r0 = (rtn - x).double()
    obj_rtn = float(((a @ r0) * (r0 @ b)).sum())
    np.savez_compressed(OUT / "c1_int4.npz", l=l.numpy(), u=u.numpy(), codes=codes.to(torch.int8).numpy(),
                        ypre_codes=(ypre / scale).numpy(), row_scale=scale[:, :1].numpy(),
                        objective=np.float64(obj), objective_rtn=np.float64(obj_rtn))
    print(f"C1: objective {obj:.6e} (RTN {obj_rtn:.6e})")


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def trellis():
    data = {}
    data["hyb_tlut"] = ref_tr._gaussian_codebook(1 << 9).numpy()
    data["sha_one_mad"] = np.array(_sha(ref_tr.one_mad()))
    data["sha_three_inst"] = np.array(_sha(ref_tr.three_inst()))
    data["sha_hyb"] = np.array(_sha(ref_tr.hyb()))
    g = torch.Generator().manual_seed(4)
    shapes = (5, 1, 1, 7), (4, 1, 2, 8), (6, 1, 2, 14), (10, 2, 2, 64), (9, 3, 1, 21), (12, 4, 2, 40), (7, 1, 1, 1)
    for idx, (L, K, V, T) in enumerate(shapes):
        for dtype in (torch.float32, torch.float64):
            table = torch.randn(1 << L, V, generator=g, dtype=dtype)
            x = torch.randn(13, T, generator=g, dtype=dtype)
            for tb in (False, True):
                vals, st = ref_tr._trellis_quantize_torch(x, table, K, tb)
                key = f"s{idx}_{str(dtype)[-7:]}_{int(tb)}"
                data[key + "_table"] = table.numpy()
                data[key + "_x"] = x.numpy()
                data[key + "_states"] = st.numpy().astype(np.int32)
                data[key + "_values"] = vals.numpy()
    table = torch.randint(-3, 4, (1 << 8, 2), generator=g).float()  # many equal costs
    x = torch.randint(-3, 4, (20, 64), generator=g).float()
    vals, st = ref_tr._trellis_quantize_torch(x, table, 2, True)
    data.update(ties_table=table.numpy(), ties_x=x.numpy(), ties_states=st.numpy().astype(np.int32))
    hyb = ref_tr.hyb()
    x = torch.randn(6, 256, generator=g)
    for tb in (False, True):
        vals, st = ref_tr._trellis_quantize_torch(x, hyb, 2, tb)
        data[f"hyb16_x_{int(tb)}"] = x.numpy()
        data[f"hyb16_states_{int(tb)}"] = st.numpy().astype(np.int32)
        data[f"hyb16_values_{int(tb)}"] = vals.numpy()
    np.savez_compressed(OUT / "trellis.npz", **data)
    print(f"trellis: {len(data)} arrays")


def scales():
    g = torch.Generator().manual_seed(3)
    data = {}
    for xd in (torch.float32, torch.float64):
        x = 4 * torch.randn(6, 32, generator=g, dtype=xd)
        x[1] = 0.
        x[2] *= 1e-38
        x[3] *= 1e-6
        x[4, 0] = 65504. * 8
        for sd in (torch.float16, torch.bfloat16):
            for qmin, qmax in ((-8, 7), (-4, 3), (-128, 127), (-2, 1)):
                s = ref_qi.int_abs_max_scale_torch(x, qmin=qmin, qmax=qmax, dtype=sd)
                key = f"{str(xd)[-7:]}_{str(sd)[-8:]}_{qmin}_{qmax}"
                data[key + "_x"] = x.numpy()
                data[key + "_s"] = s.numpy()
    np.savez_compressed(OUT / "scales.npz", **data)
    print(f"scales: {len(data)} arrays")


ABSMAX_PAIRS = ((-2, 1), (-4, 3), (-8, 7), (-128, 127))
# the two selectors of quantizer_int.py:545-548 on a [*, 64 * 96] flat matrix: the 1 x 32 super-entries
# (i, j), i + j = 2, and the 2 x 24 super-entries (i, j), i + j = 2
ABSMAX_SELECTORS = {
    "r1x32": lambda t: t[..., 64:224].unfold(-1, 32, 64).unflatten(-1, (1, 32)),
    "r2x24": lambda t: t[..., 48:552].unfold(-1, 120, 168).unfold(-1, 24, 96),
}


def _name(dtype):
    return str(dtype).split(".")[-1]


def _tie_rows(g, count, width, dtype):
    """Rows of exact ties for each (qmin, qmax): entries (k + 1/2) / 4 with k in [qmin, qmax - 1], one
    entry per row set to +-(qmax - qmin) / 8, so that the abs-max scale is exactly 1/4 (in fp16 and bf16)
    and every quotient y / scale is k + 1/2."""
    rows = []
    for qmin, qmax in ABSMAX_PAIRS:
        k = torch.randint(qmin, qmax, (count, width), generator=g).to(dtype)
        r = (k + .5) / 4
        r[:, 0] = (qmax - qmin) / 8 * torch.where(torch.rand(count, generator=g) < .5, -1., 1.).to(dtype)
        rows.append(r)
    return rows


def absmax():
    """int_abs_max_quantizer_torch on the reference test's cases (quantizer_int.py:535-553)."""
    g = torch.Generator().manual_seed(5)
    data = {}
    for xd in (torch.float32, torch.float64):
        y = 4. * torch.randn(2 + len(ABSMAX_PAIRS), 64 * 96, generator=g, dtype=xd)
        y[1, 128:168] = 0.
        y[0, 192:224] *= 1e-38  # a scale so small that it is denormal (bf16) or vanishes (fp16)
        # batch rows 2.. : exact ties in every super-entry row either selector reads
        ties = _tie_rows(g, 1, 64 * 96, xd)
        for i, r in enumerate(ties):
            for lo in (64, 128, 192, 48, 144, 216, 312, 384, 480):
                r[0, lo] = r[0, 0]  # the abs-max entry at the head of each selected row
            y[2 + i] = r[0]
        data[f"{_name(xd)}_y"] = y.numpy()
        for name, select in ABSMAX_SELECTORS.items():
            x = select(y)
            for qmin, qmax in ABSMAX_PAIRS:
                for sd in (torch.float16, torch.bfloat16):
                    out = torch.empty_like(x)
                    ref_qi.int_abs_max_quantizer_torch(y, select, out=out, qmin=qmin, qmax=qmax, dtype=sd)
                    data[f"{_name(xd)}_{name}_{_name(sd)}_{qmin}_{qmax}"] = out.numpy()
        # a 48 x 96 matrix as 1 x 32 super-entries: random rows, a zero row, a 1e-38 row, tie rows
        mat = 4. * torch.randn(48, 96, generator=g, dtype=xd)
        mat[3] = 0.
        mat[5] *= 1e-38
        for i, r in enumerate(_tie_rows(g, 6, 96, xd)):
            r[:, 32] = r[:, 0]
            r[:, 64] = r[:, 0]
            mat[8 + 6 * i: 14 + 6 * i] = r
        data[f"{_name(xd)}_mat"] = mat.numpy()
        select = lambda t: t.unflatten(-1, (48 * 3, 1, 32))
        for qmin, qmax in ABSMAX_PAIRS:
            for sd in (torch.float16, torch.bfloat16):
                out = torch.empty(48 * 3, 1, 32, dtype=xd)
                ref_qi.int_abs_max_quantizer_torch(mat.flatten(), select, out=out, qmin=qmin, qmax=qmax, dtype=sd)
                data[f"{_name(xd)}_mat_{_name(sd)}_{qmin}_{qmax}"] = out.reshape(48, 96).numpy()
    np.savez_compressed(OUT / "absmax.npz", **data)
    print(f"absmax: {len(data)} arrays")


if __name__ == "__main__":
    torch.set_num_threads(8)
    if sys.argv[1:]:  # only the named sets
        for name in sys.argv[1:]:
            globals()[name]()
        sys.exit(0)
    absmax()
    scales()
    trellis()
    c1()
