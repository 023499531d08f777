"""GPU tests of the block flush (gptq2d_flush_*), both the cell-masked MFMA kernel (any cell shape, fp32 and
fp64) and the tuned tile-aligned one (32 x 32 coarse cells: fp32, and fp64 with even m and n), against a dense
CPU statement of the flush:

  stage(i, j) = i // P + j // Q;  band = [s0, s1);  targets = [s1, s_end)
  D = (L masked to k//P < i//P) @ (E masked to the band);  R = (C masked to the band) @ (U masked to k//Q < j//Q)
  on targets: C += D, Y = (Y + D) + R;  elsewhere unchanged

(the block flush of gptq_2d.py:1090-1119: _repack_errors, _flush_down, _flush_right).  Every entry the
flush must not read -- L on and above its diagonal blocks, U on and below, E and C off the band -- holds NaN.
"""

import pytest
import torch

import _hip

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _reference(y, c, e, l, u, P, Q, s0, s1, s_end):
    m, n = y.shape
    i = torch.arange(m)[:, None]
    j = torch.arange(n)[None, :]
    st = i // P + j // Q
    band = (st >= s0) & (st < s1)
    tgt = (st >= s1) & (st < s_end)
    lm = torch.where((torch.arange(m)[None, :] // P) < (torch.arange(m)[:, None] // P), l, torch.zeros_like(l))
    um = torch.where((torch.arange(n)[:, None] // Q) < (torch.arange(n)[None, :] // Q), u, torch.zeros_like(u))
    eb = torch.where(band, e, torch.zeros_like(e))
    cb = torch.where(band, c, torch.zeros_like(c))
    d = lm @ eb
    r = cb @ um
    return torch.where(tgt, (y + d) + r, y), torch.where(tgt, c + d, c), band, tgt


CASES = [  # m, n, P, Q, s0, s1, s_end
    (70, 45, 32, 32, 0, 1, 2), (70, 45, 32, 32, 0, 2, 3), (256, 512, 32, 32, 0, 4, 23),
    (300, 200, 32, 32, 2, 3, 9), (300, 200, 32, 32, 4, 8, 20), (1000, 1000, 32, 32, 0, 16, 63),
    (1000, 1000, 32, 32, 16, 32, 63), (1000, 1000, 32, 32, 40, 41, 48), (520, 1030, 32, 32, 10, 14, 50),
    (64, 96, 1, 1, 10, 20, 150), (48, 40, 4, 8, 2, 5, 17), (90, 75, 3, 5, 3, 9, 34),
    # 16 x 16 cells (the trellis configuration's super-entries), 1 x 32 rows, cells taller than an output tile
    (256, 320, 16, 16, 3, 9, 40), (520, 130, 16, 16, 0, 4, 30), (1000, 600, 16, 16, 20, 30, 90),
    (96, 256, 1, 32, 4, 12, 30), (300, 200, 100, 40, 0, 1, 5),
    # a 24-stage band over many 2 x 2-tile workgroups (interior k-tiles, the XCD order's full runs)
    (2048, 1536, 32, 32, 20, 44, 110),
]


@pytest.mark.parametrize("m,n,P,Q,s0,s1,s_end", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_flush(m, n, P, Q, s0, s1, s_end, dtype):
    print(f"flush {m}x{n} P={P} Q={Q} [{s0},{s1})->[{s1},{s_end}) {dtype}", flush=True)
    g = torch.Generator().manual_seed(m + 3 * n + s0)
    y, c, e = (torch.randn(m, n, generator=g, dtype=torch.float64) for _ in range(3))
    l = torch.randn(m, m, generator=g, dtype=torch.float64) / m ** .5
    u = torch.randn(n, n, generator=g, dtype=torch.float64) / n ** .5
    ey, ec, band, tgt = _reference(y, c, e, l, u, P, Q, s0, s1, s_end)
    # poison what must not be read
    ar_m, ar_n = torch.arange(m), torch.arange(n)
    l = l.masked_fill((ar_m[None, :] // P) >= (ar_m[:, None] // P), torch.nan)
    u = u.masked_fill((ar_n[:, None] // Q) >= (ar_n[None, :] // Q), torch.nan)
    e = e.masked_fill(~band, torch.nan)
    c = c.masked_fill(~band & ~tgt, torch.nan)
    ec = ec.masked_fill(~band & ~tgt, torch.nan)
    yd, cd, ed, ld, ud = (t.to(dtype).to(DEV) for t in (y, c, e, l, u))
    one = _hip.i64_array([])
    _hip.call("flush", dtype, _hip.ptr(yd), _hip.ptr(cd), _hip.ptr(ed), _hip.ptr(ld), _hip.ptr(ud), m, n, P, Q, s0, s1,
              s_end, 0, one, one, one, _hip.stream(yd.device))
    gy, gc = yd.double().cpu(), cd.double().cpu()
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    assert torch.equal(gy[~tgt], ey.to(dtype).double()[~tgt])
    keep = ~band & ~tgt
    assert torch.equal(gc[band], ec.to(dtype).double()[band]) and gc[keep].isnan().all()
    for got, exp in ((gy, ey), (gc, ec)):
        err = ((got[tgt] - exp[tgt]).abs() / (1 + exp[tgt].abs())).max().item() if tgt.any() else 0.
        assert err < tol * max(1., (m + n) ** .5), err


def test_flush_mfma_large_operand():
    """The MFMA flush on a layer whose U has more than 2^29 entries (n = 24576): the staging resources are
    based at each panel, so the 32-bit offsets hold and the result matches the dense statement (computed on
    the GPU in fp64), with NaN everywhere the flush must not read."""
    m, n, P, Q, s0, s1, s_end = 96, 24576, 32, 32, 100, 110, 400
    print(f"flush {m}x{n} [{s0},{s1})->[{s1},{s_end}) fp32, U with {n * n} entries", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    y, c, e = (torch.randn(m, n, generator=g, device=DEV, dtype=torch.float64) for _ in range(3))
    l = torch.randn(m, m, generator=g, device=DEV, dtype=torch.float64) / m ** .5
    i = torch.arange(m, device=DEV)[:, None]
    j = torch.arange(n, device=DEV)[None, :]
    st = i // P + j // Q
    band = (st >= s0) & (st < s1)
    tgt = (st >= s1) & (st < s_end)
    lm = torch.where(i.t() // P < i // P, l, 0.)
    d = lm @ torch.where(band, e, 0.)
    u = torch.randn(n, n, generator=g, device=DEV, dtype=torch.float32) / n ** .5
    ar = torch.arange(n, device=DEV)
    upper = (ar[:, None] // Q) < (ar[None, :] // Q)
    r = torch.where(band, c.float().double(), 0.) @ torch.where(upper, u, 0.).double()
    ey = torch.where(tgt, (y.float().double() + d) + r, y)
    u.masked_fill_(~upper, torch.nan)
    del upper
    yd, cd = y.float().contiguous(), c.float().masked_fill(~band & ~tgt, torch.nan).contiguous()
    ed = e.float().masked_fill(~band, torch.nan).contiguous()
    ld = l.float().masked_fill(i.t() // P >= i // P, torch.nan).contiguous()
    one = _hip.i64_array([])
    _hip.call("flush", torch.float32, _hip.ptr(yd), _hip.ptr(cd), _hip.ptr(ed), _hip.ptr(ld), _hip.ptr(u), m, n, P, Q,
              s0, s1, s_end, 0, one, one, one, _hip.stream(yd.device))
    torch.cuda.synchronize()
    assert torch.equal(yd[~tgt], y.float()[~tgt])
    err = ((yd.double()[tgt] - ey[tgt]).abs() / (1 + ey[tgt].abs())).max().item()
    print(f"  max rel err {err:.2e}", flush=True)
    assert err < 2e-5 * (m + n) ** .5
