"""GPU tests of the GPTQ-2D engine, following the reference's test_gptq_2d.py (:70-204).

Every engine path (fused tile sweep, plug-in path with plain entries and super-entries, capture,
PyTorch variants on the GPU) must equal the CPU oracle's super-entry Algorithm 3 exactly in fp64
on the reference's shapes and block configurations, with NaN in the unused triangles of L and U.
"""

import functools
import warnings

import pytest
import torch

import gptq_2d as G
import quantizer_int as QI
from oracle import algorithms as A
from oracle import quantize as OQ
from oracle import sweep as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _instance(m, n, seed, se=(1, 1)):
    """X, L, U on the GPU with NaN in the unused triangles and diagonal blocks (test_gptq_2d.py:32-40)."""
    g = torch.Generator().manual_seed(seed)
    x = 4. * torch.randn(m, n, generator=g, dtype=torch.float64)
    l, u = (.05 * torch.randn(k, k, generator=g, dtype=torch.float64) for k in (m, n))
    for f, size, unused in ((l, se[0], torch.ge), (u, se[1], torch.le)):
        blk = torch.arange(f.size(0)) // size
        f[unused(blk[None, :], blk[:, None])] = torch.nan
    return x.to(DEV), l.to(DEV), u.to(DEV)


def _unit(l, u, se=(1, 1)):
    return S.unit_triangular(l.cpu(), False, se[0]).to(DEV), S.unit_triangular(u.cpu(), True, se[1]).to(DEV)


def _expected(x, l, u, se):
    lu, uu = _unit(l, u, se)
    return A.alg3_super_entry(x.cpu(), lu.cpu(), uu.cpu(), super_entry_shape=se).to(DEV)


CASES = [(1, 1, (1, 1)), (1, 7, (1, 1)), (7, 1, (1, 1)), (13, 5, (1, 1)), (9, 13, (1, 1)), (65, 97, (1, 1)),
         (8, 12, (2, 4)), (6, 6, (3, 2)), (4, 64, (1, 32)), (12, 8, (4, 4)), (16, 16, (16, 16)), (24, 8, (1, 8)),
         (32, 64, (16, 16)), (96, 160, (16, 16)), (90, 75, (3, 5))]


@pytest.mark.parametrize("m,n,se", CASES)
def test_reference(m, n, se):
    """Every implementation equals super-entry Algorithm 3 in fp64, with one block, one level, two levels."""
    print(f"case m={m} n={n} se={se}", flush=True)
    x, l, u = _instance(m, n, 100 * m + n, se)
    expected = _expected(x, l, u, se)
    lu, uu = _unit(l, u, se)
    runs = []
    for inner, outer in ((0, 0), (1, 0), (2, 8), (3, 11)):
        runs.append((f"super {inner},{outer}", functools.partial(G.gptq_2d_super_entry, super_entry_shape=se,
                                                                 inner_block_size=inner, outer_block_size=outer)))
        if se == (1, 1):
            runs.append((f"plugin {inner},{outer}", functools.partial(G.gptq_2d, inner_block_size=inner,
                                                                      outer_block_size=outer, fused=False)))
            runs.append((f"fused {inner},{outer}", functools.partial(G.gptq_2d, inner_block_size=inner,
                                                                     outer_block_size=outer, fused=True)))
    runs.append(("super torch", functools.partial(G.gptq_2d_super_entry_torch, super_entry_shape=se)))
    runs.append(("super direct", functools.partial(G.direct_2d_super_entry, super_entry_shape=se)))
    for name, run in runs:
        assert run(x, l, u).equal(expected), name
    if se == (1, 1):
        assert G.gptq_2d_torch(x, lu, uu).equal(expected)
        assert G.direct_2d(x, lu, uu).equal(expected)
        # the fused sweep with outer blocks of 1, 2 and many tile stages on a matrix of several tiles
        for outer in (32, 64, 4096):
            assert G.gptq_2d(x, l, u, outer_block_size=outer, fused=True).equal(expected), outer


@pytest.mark.parametrize("m,n", [(70, 45), (100, 130), (33, 65)])
def test_fused_multi_tile(m, n):
    """The fused tile sweep across several tile stages, ragged edges, and both flush levels, in fp64."""
    x, l, u = _instance(m, n, 7 * m + n)
    expected = _expected(x, l, u, (1, 1))
    for outer in (0, 32, 64, 96, 10_000):
        assert G.gptq_2d(x, l, u, outer_block_size=outer).equal(expected), outer


@pytest.mark.parametrize("outer", [256, 384, 10_000])
def test_fused_fp64_bands(outer):
    """The fp64 fused sweep's bands inside an outer block: each tile pulls the tiles of its band's earlier stages
    itself, and a band flush delivers a finished band to the rest of the block.  300 x 420 has 23 tile stages:
    blocks of 8, 12 and all 23 stages, so several bands per block, with a partial band where the block's length
    is not a multiple of the band's (4 stages: the last block of 384 and the single block of 23)."""
    print(f"fp64 fused bands 300x420 outer={outer}", flush=True)
    x, l, u = _instance(300, 420, 11)
    expected = _expected(x, l, u, (1, 1))
    assert G.gptq_2d(x, l, u, outer_block_size=outer).equal(expected)


def test_fused_fp64_bands_batched():
    """A batch of layers with a factor pair each through the fp64 fused sweep (bands with pulls and band flushes
    inside one outer block) equals the layers swept one by one, bit for bit: the pulls read each layer's own
    E, C, L and U."""
    print("fp64 fused bands, batch of 2, 300x420", flush=True)
    xs, ls, us = zip(*(_instance(300, 420, 20 + b) for b in range(2)))
    x, l, u = torch.stack(xs), torch.stack(ls), torch.stack(us)
    got = G.gptq_2d(x, l, u, outer_block_size=10_000)
    for b in range(2):
        assert got[b].equal(G.gptq_2d(xs[b], ls[b], us[b], outer_block_size=10_000)), b


def test_quantizer_sees_quantized_values():
    """Live Y holds the quantized values of all earlier antidiagonals (test_gptq_2d.py:113-127)."""
    x, l, u = _instance(12, 8, 7, (2, 2))
    lu, uu = _unit(l, u, (2, 2))
    runs = [("plugin", functools.partial(G.gptq_2d, inner_block_size=3, outer_block_size=7), lu, uu),
            ("super", functools.partial(G.gptq_2d_super_entry, super_entry_shape=(2, 2), inner_block_size=2,
                                        outer_block_size=5), l, u)]
    for name, run, lr, ur in runs:
        earlier = []

        def quantizer(y_flat, selection, *, out):
            select = selection if callable(selection) else (lambda t: t[..., selection])
            for es, ez in earlier:
                assert es(y_flat).equal(ez), name
            torch.round(select(y_flat), out=out)
            earlier.append((select, out.clone()))

        run(x, lr, ur, quantizer=quantizer)
        assert earlier


def _round_to_scale(y_flat, selection, scale, *, out):
    select = selection if callable(selection) else (lambda t: t[..., selection])
    torch.div(select(y_flat), select(scale), out=out).round_().mul_(select(scale))


@pytest.mark.parametrize("m,n,se", [(12, 8, (4, 2)), (9, 15, (3, 5)), (8, 24, (1, 8))])
def test_batches_inplace_and_quantizer_inputs(m, n, se):
    """Broadcast batches and quantizer inputs, in and out of place (test_gptq_2d.py:129-147)."""
    x, l, u = _instance(m, n, 10 * m + n, se)
    x = torch.stack((x, x + .25))[:, None]
    l = torch.stack((l, .5 * l, 2. * l))[None]
    scale = x.abs().flatten(start_dim=-2) * .05 + .2
    x_before = x.clone()
    lu, uu = _unit(l, u, se)
    expected = S.gptq_2d_torch(x.cpu(), lu.cpu(), uu.cpu(), quantizer=_round_to_scale,
                               quantizer_inputs=(scale.cpu(),)).to(DEV)
    assert expected.shape == (2, 3, m, n)
    runs = [(functools.partial(G.gptq_2d, inner_block_size=3, outer_block_size=7), lu, uu),
            (functools.partial(G.gptq_2d_super_entry, super_entry_shape=se, inner_block_size=2,
                               outer_block_size=5), l, u),
            (functools.partial(G.gptq_2d_super_entry_torch, super_entry_shape=se), l, u),
            (G.gptq_2d_torch, lu, uu)]
    for run, lr, ur in runs:
        assert run(x, lr, ur, quantizer=_round_to_scale, quantizer_inputs=(scale,)).equal(expected)
        target = x.expand(2, 3, m, n).clone()
        res = run(target, lr, ur, quantizer=_round_to_scale, quantizer_inputs=(scale,), inplace=True)
        assert res.data_ptr() == target.data_ptr() and res.equal(expected)
    assert x.equal(x_before)
    # the fused engine with the affine plug-in: batch-broadcast full-matrix scales, zero point 0
    sc = scale.unflatten(-1, (m, n))
    zp = torch.zeros_like(sc)
    q = functools.partial(QI.affine_quantizer_hip)
    exp2 = S.gptq_2d_torch(x.cpu(), lu.cpu(), uu.cpu(), quantizer=OQ.affine_quantizer,
                           quantizer_inputs=(sc.cpu(), zp.cpu())).to(DEV)
    got = G.gptq_2d(x, lu, uu, quantizer=q, quantizer_inputs=(sc, zp))
    assert got.equal(exp2)
    target = x.expand(2, 3, m, n).clone()
    res = G.gptq_2d(target, lu, uu, quantizer=q, quantizer_inputs=(sc, zp), inplace=True)
    assert res.data_ptr() == target.data_ptr() and res.equal(exp2)


def test_empty_inputs():
    """Empty batches and matrices give empty results without calling the quantizer (test_gptq_2d.py:149-163)."""
    calls = []
    quantizer = lambda *args, **kwargs: calls.append(args)
    x, l, u = _instance(6, 10, 0, (3, 5))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        for empty, le, ue in ((x.new_empty(0, 6, 10), l, u), (x.new_empty(0, 10), l[:0, :0], u),
                              (x.new_empty(6, 0), l, u[:0, :0])):
            for run in (G.gptq_2d, G.gptq_2d_torch, G.direct_2d,
                        functools.partial(G.gptq_2d_super_entry, super_entry_shape=(3, 5)),
                        functools.partial(G.gptq_2d_super_entry_torch, super_entry_shape=(3, 5))):
                assert run(empty, le, ue, quantizer=quantizer).shape == empty.shape
            replay = G.capture_gptq_2d(empty, le, ue, quantizer=quantizer)
            assert replay(empty, le, ue).shape == empty.shape
    assert calls == []


def test_large_batch():
    """A batch of 70000 exceeds the 65535 grid limit of the y/z axes (test_gptq_2d.py:165-172)."""
    x, l, u = _instance(4, 6, 9, (2, 2))
    x = x + torch.arange(70_000, dtype=torch.float64, device=DEV)[:, None, None] / 7
    expected = S.gptq_2d_super_entry_torch(x.cpu(), l.cpu(), u.cpu(), super_entry_shape=(2, 2)).to(DEV)
    assert G.gptq_2d_super_entry(x, l, u, super_entry_shape=(2, 2), inner_block_size=1).equal(expected)
    lu, uu = _unit(l, u, (2, 2))
    exp_plain = S.gptq_2d_torch(x.cpu(), lu.cpu(), uu.cpu()).to(DEV)
    assert G.gptq_2d(x, lu, uu, inner_block_size=2, fused=False).equal(exp_plain)
    assert G.gptq_2d(x, lu, uu).equal(exp_plain)


@pytest.mark.parametrize("shape", [None, (3, 4)])
def test_graph_capture(shape):
    """Replays equal direct runs on new inputs, in and out of place (test_gptq_2d.py:174-194)."""
    x, l, u = _instance(12, 20, 4321, shape or (1, 1))
    x = torch.stack((x, x + .25))
    scale = x.abs().flatten(start_dim=-2) * .05 + .2
    options = dict(quantizer=_round_to_scale, inner_block_size=2, outer_block_size=4)
    if shape is not None:
        options["super_entry_shape"] = shape
    run = functools.partial(G.gptq_2d if shape is None else G.gptq_2d_super_entry, **options)
    replay = G.capture_gptq_2d(x, l, u, quantizer_inputs=(scale,), **options)
    first = replay(x, l, u, scale)
    assert first.equal(run(x, l, u, quantizer_inputs=(scale,)))
    second = replay(x + .375, 1.5 * l, .5 * u, 1.5 * scale)
    assert second.equal(run(x + .375, 1.5 * l, .5 * u, quantizer_inputs=(1.5 * scale,)))
    assert first.equal(run(x, l, u, quantizer_inputs=(scale,)))
    replay = G.capture_gptq_2d(x, l, u, quantizer_inputs=(scale,), inplace=True, **options)
    target = x + .25
    assert replay(target, l, u, scale).data_ptr() == target.data_ptr()
    assert target.equal(run(x + .25, l, u, quantizer_inputs=(scale,)))


def test_graph_capture_fused():
    """The fused sweep (one C-ABI call issuing every launch) captured and replayed several times, with
    eager work in between; every replay equals the eager result."""
    x, l, u = _instance(70, 90, 99)
    lu, uu = _unit(l, u)
    x = x.float()
    lu, uu = lu.float(), uu.float()
    sc = (x.abs() * .05 + .2)
    zp = torch.zeros_like(sc)
    opts = dict(quantizer=functools.partial(QI.affine_quantizer_hip, qmin=-8, qmax=7), outer_block_size=64)
    replay = G.capture_gptq_2d(x, lu, uu, quantizer_inputs=(sc, zp), **opts)
    for k in range(3):
        xs = x + .1 * k
        eager = G.gptq_2d(xs, lu, uu, quantizer_inputs=(sc, zp), **opts)
        torch.cuda.synchronize()
        assert replay(xs, lu, uu, sc, zp).equal(eager), k


@pytest.mark.parametrize("m,n", [(100, 70), (300, 260), (520, 1030), (1024, 512)])
@pytest.mark.parametrize("outer", [32, 64, 512])
def test_fused_fp32_trajectory(m, n, outer):
    """The fp32 fused engine (MFMA pulls inside an outer block, MFMA flushes between blocks) follows the fp64
    engine's trajectory: with every stage forced to the fp64 run's codes, each entry's Y just before rounding
    agrees with the fp64 value to 1e-4 absolute (values are O(10); fp32 summation error is O(1e-5)).
    The fp64 engine itself equals the oracle's Algorithm 3 exactly (test_reference, test_fused_multi_tile)."""
    print(f"fp32 trajectory {m}x{n} outer={outer}", flush=True)
    g = torch.Generator().manual_seed(m * 3 + n)
    x = 4. * torch.randn(m, n, generator=g, dtype=torch.float64)
    lo = S.unit_triangular(.3 / m ** .5 * torch.randn(m, m, generator=g, dtype=torch.float64), upper=False)
    up = S.unit_triangular(.3 / n ** .5 * torch.randn(n, n, generator=g, dtype=torch.float64), upper=True)
    x, lo, up = x.to(DEV), lo.to(DEV), up.to(DEV)
    z64 = G.gptq_2d(x, lo, up, outer_block_size=outer)
    pre64 = torch.full_like(x, float("nan"))
    assert G.gptq_2d(x, lo, up, quantizer=QI.teacher_forced_quantizer, quantizer_inputs=(z64, pre64),
                     outer_block_size=outer).equal(z64)
    pre32 = torch.full_like(x, float("nan"), dtype=torch.float32)
    z32 = G.gptq_2d(x.float(), lo.float(), up.float(), quantizer=QI.teacher_forced_quantizer,
                    quantizer_inputs=(z64.float(), pre32), outer_block_size=outer)
    assert z32.equal(z64.float())
    err = (pre32.double() - pre64).abs()
    assert not err.isnan().any()
    print(f"  max |dY| {err.max().item():.2e}, mean {err.mean().item():.2e}", flush=True)
    assert err.max().item() < 1e-4
    # free-running fp32 codes agree except at near-ties of the fp32 trajectory
    z32f = G.gptq_2d(x.float(), lo.float(), up.float(), outer_block_size=outer)
    assert (z32f.double() != z64).float().mean().item() < 1e-3


@pytest.mark.parametrize("last_zp", [0., float("nan"), float("inf"), float("-inf")])
@pytest.mark.parametrize("qmin,qmax", [(-8., 7.), (0., 15.)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_fused_quantizer_special_values(qmin, qmax, last_zp, dtype):
    """The fused sweep's affine quantizer on entries that leave its fast path (scales outside
    [2^-60, 2^60] in fp32, [2^-500, 2^500] in fp64, or negative; |y| outside the range where the reciprocal
    gives the IEEE quotient; a NaN or infinite zero point; qmin > qmax is rejected by the API, as in the
    reference): with identity factors there is no feedback, so every entry is quantized once, and the result
    must equal (clamp(round(y / s + z), qmin, qmax) - z) * s in the sweep's dtype bit for bit.  A NaN or
    infinite zero point makes its entry's error NaN, which 0 x NaN would carry to every later entry (as the
    reference's products would), so it sits on the last entry."""
    print(f"{dtype} quantizer special values qmin={qmin} qmax={qmax} last zp={last_zp}", flush=True)
    m, n = 40, 70
    g = torch.Generator().manual_seed(5)
    x = (3. * torch.randn(m, n, generator=g)).to(dtype)
    s = (0.1 + torch.rand(m, n, generator=g)).to(dtype)
    z = torch.randint(-2, 3, (m, n), generator=g).to(dtype)
    big, tiny = (1e30, 1e-30) if dtype == torch.float32 else (1e200, 1e-200)
    s[0, :10] = tiny
    s[1, :10] = big
    s[2, :10] = -0.5
    x[5, :10] = 1e25 if dtype == torch.float32 else 1e180
    x[6, :10] = 1e-25 if dtype == torch.float32 else 1e-180
    x[7, :10] = 0.
    z[m - 1, n - 1] = last_zp
    eye_m, eye_n = torch.eye(m, dtype=dtype), torch.eye(n, dtype=dtype)
    quant = functools.partial(QI.affine_quantizer_hip, qmin=qmin, qmax=qmax)
    got = G.gptq_2d(x.to(DEV), eye_m.to(DEV), eye_n.to(DEV), quantizer=quant,
                    quantizer_inputs=(s.to(DEV), z.to(DEV))).cpu()
    expected = (torch.clamp(torch.round(x / s + z), qmin, qmax) - z) * s
    assert torch.equal(got.isnan(), expected.isnan())
    ok = ~expected.isnan()
    assert torch.equal(got[ok], expected[ok])


@pytest.mark.parametrize("outer_tiles", [2, 6])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_fused_resume_at_block_boundary(dtype, outer_tiles):
    """gptq2d_sweep_fused over [0, S) then [S, end) with S on an outer-block boundary equals one call over the
    whole sweep bit for bit (the C scratch carries the state); an end inside an outer block is rejected.  Blocks
    of 6 tile stages hold a band flush of the fp64 sweep (bands of 4) as well as its pulls."""
    import _hip

    print(f"fused resume {dtype} outer_tiles={outer_tiles}", flush=True)
    m, n = 200, 330
    g = torch.Generator().manual_seed(9)
    x = (4. * torch.randn(m, n, generator=g, dtype=torch.float64)).to(DEV, dtype)
    lo = S.unit_triangular(.3 / m ** .5 * torch.randn(m, m, generator=g, dtype=torch.float64), upper=False)
    up = S.unit_triangular(.3 / n ** .5 * torch.randn(n, n, generator=g, dtype=torch.float64), upper=True)
    lo, up = lo.to(DEV, dtype), up.to(DEV, dtype)
    stages = -(-m // 32) + -(-n // 32) - 1
    bshape, strides = _hip.i64_array([]), _hip.i64_array([])
    st = _hip.stream(x.device)

    def run(y, c, e, begin, end):
        _hip.call("sweep_fused", dtype, _hip.ptr(y), _hip.ptr(c), _hip.ptr(e), _hip.ptr(lo), _hip.ptr(up), m, n, 0,
                  bshape, strides, strides, 0, None, None, None, None, 0., 0., None, outer_tiles, begin, end, st)

    whole = x.clone()
    c, e = torch.empty_like(x), torch.empty_like(x)
    run(whole, c, e, 0, -1)
    split = x.clone()
    c, e = torch.empty_like(x), torch.empty_like(x)
    run(split, c, e, 0, 2 * outer_tiles)
    run(split, c, e, 2 * outer_tiles, stages)
    torch.cuda.synchronize()
    assert split.equal(whole)
    with pytest.raises(_hip.GPTQ2DError):
        run(x.clone(), c, e, 0, 3)
    with pytest.raises(_hip.GPTQ2DError):
        run(x.clone(), c, e, 1, stages)
