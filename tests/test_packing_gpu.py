"""GPU tests of the packed output formats (packing.py over csrc/pack.hip) against the CPU restatement
(oracle/packing.py, pinned on the reference's fixtures in test_oracle_packing.py).

INT codes: the HIP words equal the oracle's bit for bit for code widths 1-16 (power-of-two and straddling
fields), per-row / per-group / full scales, zero points, batches and ragged rows; off-grid values are
counted per row as the oracle counts them; unpacking gives the values back.  End to end, the fused
sweep's INT4 output packs with no off-grid entry and unpacks to itself, and the abs-max super-entry
quantizers record the scale map the packed layer needs (the HIP and PyTorch plug-ins agree, and the
fused sweep agrees with them in fp64).

Trellis: the streams of Viterbi paths (the reference's fixtures and fresh HYB L=16 searches) equal the
oracle's, unpack to the states and decode to the quantizer's values bit for bit; the trellis plug-ins
record the per-entry state map during a 16 x 16 super-entry sweep, and its packed streams decode to the
sweep's output.
"""

import functools
import pathlib

import numpy as np
import pytest
import torch

import gptq_2d as G
import packing as PK
import quantizer_int as QI
import quantizer_trellis as QT
from oracle import packing as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _u32(words: torch.Tensor) -> np.ndarray:
    return words.cpu().numpy().view(np.uint32)


def _grid_values(shape, qmin, qmax, scale, zp, g, dtype):
    q = torch.randint(qmin, qmax + 1, shape, generator=g).to(dtype)
    return (q - zp) * scale


@pytest.mark.parametrize("qmin,qmax", [(-8, 7), (0, 15), (-4, 3), (0, 1), (-2, 1), (-16, 15), (0, 63), (-64, 63),
                                       (-128, 127), (0, 1023), (-32768, 32767)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_pack_int_matches_oracle(qmin, qmax, dtype):
    g = torch.Generator().manual_seed(qmax - qmin)
    m, n = 37, 203
    s = (0.5 + torch.rand(m, 1, generator=g, dtype=dtype)).to(torch.bfloat16).to(dtype)  # per-row scale
    zp = torch.randint(qmin, qmax + 1, (m, 1), generator=g).to(dtype) if qmin == 0 else torch.zeros((), dtype=dtype)
    z = _grid_values((m, n), qmin, qmax, s, zp, g, dtype)
    z[3, 5] += s[3, 0] * 0.25  # off the grid
    z[10, 0] = float("nan")
    words, bad = PK.pack_int(z.to(DEV), s.to(DEV), zp.to(DEV), qmin=qmin, qmax=qmax, check=False, return_bad=True)
    u, ok = P.int_codes(z.numpy(), s.numpy(), zp.numpy(), qmin, qmax)
    bits = P.int_bits(qmin, qmax)
    assert np.array_equal(_u32(words), P.pack_lsb(u, bits))
    assert np.array_equal(bad.cpu().numpy(), (~ok).sum(-1))
    back = PK.unpack_int(words, s.to(DEV), zp.to(DEV), n=n, qmin=qmin, qmax=qmax)
    keep = torch.from_numpy(ok)
    assert torch.equal(back.cpu()[keep], z[keep])
    with pytest.raises(ValueError):
        PK.pack_int(z.to(DEV), s.to(DEV), zp.to(DEV), qmin=qmin, qmax=qmax)


@pytest.mark.parametrize("m,n", [(1, 1), (3, 7), (64, 64), (5, 1000), (130, 33)])
def test_pack_int_layouts(m, n):
    """Full-map and per-group scales, a zero-point map, batch dimensions; INT3 (fields straddle words) and INT4."""
    g = torch.Generator().manual_seed(m * n)
    for qmin, qmax in ((-4, 3), (0, 15)):
        s = (0.1 + torch.rand(2, m, n, generator=g)).to(torch.bfloat16).float()
        zp = torch.randint(qmin, qmax + 1, (2, m, n), generator=g).float() if qmin == 0 else None
        z = _grid_values((2, m, n), qmin, qmax, s, 0. if zp is None else zp, g, torch.float32)
        words = PK.pack_int(z.to(DEV), s.to(DEV), None if zp is None else zp.to(DEV), qmin=qmin, qmax=qmax)
        assert words.shape == (2, m, -(-n * P.int_bits(qmin, qmax) // 32))
        u, ok = P.int_codes(z.numpy(), s.numpy(), None if zp is None else zp.numpy(), qmin, qmax)
        assert ok.all() and np.array_equal(_u32(words), P.pack_lsb(u, P.int_bits(qmin, qmax)))
        back = PK.unpack_int(words, s.to(DEV), None if zp is None else zp.to(DEV), n=n, qmin=qmin, qmax=qmax)
        assert torch.equal(back.cpu(), z)
    # per-group scales (7 columns each) expanded to the layer
    if n % 7 == 0:
        sg = (0.1 + torch.rand(m, n // 7, 1, generator=g)).float()
        z = _grid_values((m, n // 7, 7), -8, 7, sg, 0., g, torch.float32).reshape(m, n)
        sfull = sg.expand(m, n // 7, 7).reshape(m, n)
        words = PK.pack_int(z.to(DEV), sfull.to(DEV), qmin=-8, qmax=7)
        assert torch.equal(PK.unpack_int(words, sfull.to(DEV), n=n, qmin=-8, qmax=7).cpu(), z)


def test_pack_int_empty():
    z = torch.empty(0, 5, device=DEV)
    assert PK.pack_int(z, torch.ones(1, device=DEV), qmin=-8, qmax=7).shape == (0, 1)


def test_pack_int_fused_sweep_output():
    """The fused INT4 sweep's output is on the quantizer's grid: it packs with no off-grid entry (nibbles,
    8 per word) and unpacks to itself."""
    g = torch.Generator().manual_seed(5)
    m, n = 200, 320
    x = 0.02 * torch.randn(m, n, generator=g)
    lo = torch.eye(m) + torch.randn(m, m, generator=g).tril(-1) * 0.02
    up = torch.eye(n) + torch.randn(n, n, generator=g).triu(1) * 0.02
    s = (x.abs().amax(-1, keepdim=True) / 7.5).to(torch.bfloat16).float().expand(m, n).contiguous()
    zp = torch.zeros(m, n)
    q = functools.partial(QI.affine_quantizer_hip, qmin=-8, qmax=7)
    z = G.gptq_2d(x.to(DEV), lo.to(DEV), up.to(DEV), quantizer=q, quantizer_inputs=(s.to(DEV), zp.to(DEV)), fused=True)
    words = PK.pack_int(z, s[:, :1].to(DEV), qmin=-8, qmax=7)
    assert words.shape == (m, n // 8)
    assert torch.equal(PK.unpack_int(words, s[:, :1].to(DEV), n=n, qmin=-8, qmax=7), z)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_abs_max_scale_map(dtype):
    """The abs-max quantizer's scale map (1 x 32 super-entries, bf16 scales): the plug-in engine gives the
    same output and map with the HIP and the PyTorch quantizer, and so does the fused sweep in fp64 (fp32
    sums differ between the engines); in the fused run each super-entry row holds one scale, the abs-max
    scale of the row's values just before rounding, and the output packs onto the map."""
    g = torch.Generator().manual_seed(9)
    m, n = 70, 128
    x = (4. * torch.randn(m, n, generator=g, dtype=dtype)).to(DEV)
    lo = (torch.eye(m, dtype=dtype) + .3 / m ** .5 * torch.randn(m, m, generator=g, dtype=dtype).tril(-1)).to(DEV)
    blk = torch.arange(n) // 32
    up = torch.eye(n, dtype=dtype) + torch.where(blk[None, :] > blk[:, None],
                                                 .3 / n ** .5 * torch.randn(n, n, generator=g, dtype=dtype), 0.)
    up = up.to(DEV)
    kw = dict(qmin=-8, qmax=7, dtype=torch.bfloat16)
    runs = {}
    for name, fn, fused in (("fused", QI.int_abs_max_quantizer_hip, True), ("hip", QI.int_abs_max_quantizer_hip, False),
                            ("torch", QI.int_abs_max_quantizer_torch, False)):
        smap = torch.full_like(x, float("nan"))
        z = G.gptq_2d_super_entry(x, lo, up, super_entry_shape=(1, 32), quantizer=functools.partial(fn, **kw),
                                  quantizer_inputs=(smap,), outer_block_size=64, fused=fused)
        runs[name] = z, smap
    assert torch.equal(runs["hip"][0], runs["torch"][0]) and torch.equal(runs["hip"][1], runs["torch"][1])
    z, smap = runs["fused"]
    if dtype == torch.float64:
        assert torch.equal(runs["hip"][0], z) and torch.equal(runs["hip"][1], smap)
    assert not smap.isnan().any()
    rows = smap.view(m, n // 32, 32)
    assert torch.equal(rows, rows[..., :1].expand_as(rows))
    pre = torch.full_like(x, float("nan"))
    G.gptq_2d_super_entry(x, lo, up, super_entry_shape=(1, 32), quantizer=QI.teacher_forced_quantizer,
                          quantizer_inputs=(z, pre), outer_block_size=64, fused=True)
    expect = QI.int_abs_max_scale_torch(pre.view(m, n // 32, 32), **kw).expand(m, n // 32, 32).reshape(m, n)
    assert torch.equal(smap, expect)
    words = PK.pack_int(z, smap, qmin=-8, qmax=7)
    assert torch.equal(PK.unpack_int(words, smap, n=n, qmin=-8, qmax=7), z)
    compact = PK.super_entry_scales(smap, (1, 32))
    assert compact.shape == (m, n // 32) and torch.equal(compact, compact.to(torch.bfloat16).to(dtype))


def _golden_cases():
    d = np.load(GOLDEN / "trellis.npz")
    shapes = [(5, 1, 1, 7), (4, 1, 2, 8), (6, 1, 2, 14), (10, 2, 2, 64), (9, 3, 1, 21), (12, 4, 2, 40), (7, 1, 1, 1)]
    for idx, (L, K, V, T) in enumerate(shapes):
        for dt in ("float32", "float64"):
            for tb in (0, 1):
                key = f"s{idx}_{dt}_{tb}"
                yield key, L, K, V, T, bool(tb), d[key + "_states"], d[key + "_table"], d[key + "_values"]


@pytest.mark.parametrize("case", list(_golden_cases()), ids=lambda c: c[0])
def test_trellis_golden_paths(case):
    key, L, K, V, T, tb, states, table, values = case
    st = torch.from_numpy(states.astype(np.int64)).to(DEV)
    words = PK.pack_trellis(st, L=L, K=K, V=V, tail_biting=tb)
    assert np.array_equal(_u32(words), P.trellis_stream(states, L, K * V, tb))
    assert torch.equal(PK.unpack_trellis(words, steps=T // V, L=L, K=K, V=V, tail_biting=tb), st)
    dec = PK.decode_trellis(words, torch.from_numpy(table).to(DEV), K=K, tail_biting=tb, steps=T // V)
    assert np.array_equal(dec.cpu().numpy().view(np.uint8), values.view(np.uint8))


@pytest.mark.parametrize("tail_biting", [True, False])
def test_trellis_hyb_search_round_trip(tail_biting):
    """Fresh HYB L=16 K=2 V=2 searches of 300 sequences of 256 (C4's code): stream = oracle's, exactly
    T*K = 512 bits with tail-biting; unpack = states; decode with a per-sequence scale = the search's values."""
    table = QT.hyb().to(DEV)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(300, 256, generator=g, device=DEV)
    scale = 0.5 + torch.rand(300, generator=g, device=DEV)
    vals, st = QT.trellis_quantize_hip(x, table, 2, tail_biting, scale=scale)
    words, bad = PK.pack_trellis(st, L=16, K=2, V=2, tail_biting=tail_biting, return_bad=True)
    assert int(bad.sum()) == 0
    assert words.shape == (300, 16 if tail_biting else 17)
    assert np.array_equal(_u32(words), P.trellis_stream(st.cpu().numpy(), 16, 4, tail_biting))
    assert torch.equal(PK.unpack_trellis(words, steps=128, L=16, K=2, V=2, tail_biting=tail_biting), st)
    dec = PK.decode_trellis(words, table, scale, K=2, tail_biting=tail_biting, steps=128)
    assert torch.equal(dec, vals)


def test_trellis_pack_flags_broken_paths():
    st = torch.tensor([[11, 13, 4, 2], [11, 14, 4, 3], [11, 13, 4, 16]], device=DEV)
    _, bad = PK.pack_trellis(st, L=4, K=1, V=2, tail_biting=True, check=False, return_bad=True)
    expect = P.path_violations(np.array([[11, 13, 4, 2], [11, 14, 4, 3], [11, 13, 4, 0]]), 4, 2, True)
    expect[2] += 1  # 16 is out of [0, 2^4) and counted as state 0
    assert bad.tolist() == expect.tolist() and bad.tolist()[0] == 0
    with pytest.raises(ValueError):
        PK.pack_trellis(st, L=4, K=1, V=2, tail_biting=True)


@pytest.mark.parametrize("plugin", [QT.trellis_quantizer_super_entry_hip, QT.trellis_quantizer_super_entry_torch])
def test_trellis_state_map_in_sweep(plugin):
    """A 16 x 16 super-entry sweep (HYB L=16, K=2, V=2) records the per-entry state map; its streams
    (one per super-entry, 512 bits) decode with the sweep's scale to the sweep's output bit for bit."""
    m, n, se = 64, 96, (16, 16)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(m, n, generator=gen).to(DEV)
    l = (torch.eye(m) + .05 * torch.randn(m, m, generator=gen).tril(-16)).to(DEV)
    blk = torch.arange(n) // 16
    u = (torch.eye(n) + torch.where(blk[None, :] > blk[:, None], .05 * torch.randn(n, n, generator=gen), 0.)).to(DEV)
    table = QT.hyb().to(DEV)
    scale = torch.tensor(0.75, device=DEV)
    smap = torch.full((m, n), -1, dtype=torch.int64, device=DEV)
    q = functools.partial(plugin, table=table, K=2)
    z = G.gptq_2d_super_entry(x, l, u, super_entry_shape=se, quantizer=q, quantizer_inputs=(scale, smap))
    assert int(smap.min()) >= 0
    words = PK.pack_trellis(smap, L=16, K=2, V=2, super_entry_shape=se)
    assert words.shape == (m // 16, n // 16, 16)
    dec = PK.decode_trellis(words, table, scale, K=2, super_entry_shape=se)
    assert torch.equal(dec, z)
    z2 = G.gptq_2d_super_entry(x, l, u, super_entry_shape=se, quantizer=q, quantizer_inputs=(scale,))
    assert torch.equal(z2, z), "recording the states changed the sweep"
