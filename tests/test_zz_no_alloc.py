"""The allocation-free fused sweep (gptq2d_sweep_fused_noalloc_*), called through the C ABI, against the fused
sweep with caller-owned scratch (gptq2d_sweep_fused_*): bitwise equal on two calls in a row, the second on a
smaller input (the fixed scratch keeps the first call's contents), and sizes beyond the scratch rejected
before anything runs."""

import ctypes

import pytest
import torch

import _hip
from oracle import sweep as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(batch, m, n, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = (4. * torch.randn(*batch, m, n, generator=g, dtype=torch.float64)).to(DEV, dtype)
    lo = S.unit_triangular(.3 / m ** .5 * torch.randn(m, m, generator=g, dtype=torch.float64), upper=False)
    up = S.unit_triangular(.3 / n ** .5 * torch.randn(n, n, generator=g, dtype=torch.float64), upper=True)
    scale = (0.5 + torch.rand(m, n, generator=g, dtype=torch.float64)).to(DEV, dtype)
    zp = torch.randint(-2, 3, (m, n), generator=g).to(DEV, dtype)
    return x, lo.to(DEV, dtype), up.to(DEV, dtype), scale, zp


def _args(x, lo, up, qkind, scale, zp):
    batch = x.shape[:-2]
    m, n = x.shape[-2:]
    bs = torch.Size(batch)
    common = (m, n, len(batch), _hip.i64_array(batch), _hip.batch_strides(lo, bs), _hip.batch_strides(up, bs), qkind,
              _hip.ptr(scale), _hip.batch_strides(scale, bs) if scale is not None else None, _hip.ptr(zp),
              _hip.batch_strides(zp, bs) if zp is not None else None, -8., 7.)
    return common


def _both(x, lo, up, qkind, scale=None, zp=None, outer_tiles=4):
    dt = x.dtype
    y_ref, y_new = x.clone(), x.clone()
    c, e = torch.empty_like(x), torch.empty_like(x)
    st = _hip.stream(x.device)
    m, n, *rest = _args(x, lo, up, qkind, scale, zp)
    _hip.call("sweep_fused", dt, _hip.ptr(y_ref), _hip.ptr(c), _hip.ptr(e), _hip.ptr(lo), _hip.ptr(up), m, n, *rest,
              None, outer_tiles, 0, -1, st)
    _hip.call("sweep_fused_noalloc", dt, _hip.ptr(y_new), _hip.ptr(lo), _hip.ptr(up), m, n, *rest, None, outer_tiles,
              st)
    torch.cuda.synchronize()
    return y_ref, y_new


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_equals_fused_twice(dtype):
    print(f"no-alloc sweep {dtype}", flush=True)
    x, lo, up, scale, zp = _layer((2,), 700, 520, 1, dtype)
    y_ref, y_new = _both(x, lo, up, 1, scale, zp)
    assert y_new.equal(y_ref)
    x2, lo2, up2, _, _ = _layer((), 300, 257, 2, dtype)  # smaller, round quantizer, one matrix
    y_ref2, y_new2 = _both(x2, lo2, up2, 0, outer_tiles=2)
    assert y_new2.equal(y_ref2)
    assert not y_new2.isnan().any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_rejects_oversize(dtype):
    cap = _hip.lib().gptq2d_sweep_fused_noalloc_capacity(torch.finfo(dtype).bits // 8)
    assert cap == (1 << 24 if dtype == torch.float32 else 1 << 23)
    m, n = 4096, cap // 4096 + 1  # one row more than fits; nothing is launched, so no memory is read
    bshape = _hip.i64_array([])
    fn = getattr(_hip.lib(), f"gptq2d_sweep_fused_noalloc_{'f32' if dtype == torch.float32 else 'f64'}")
    rc = fn(None, None, None, m, n, 0, bshape, bshape, bshape, 0, None, None, None, None, 0., 0., None, 1,
            _hip.stream(torch.device(DEV)))
    assert rc == -3
