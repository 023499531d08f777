"""GPU tests of the HIP trellis quantizer (one-launch Viterbi search), following the reference's
quantizer_trellis.py:406-519 and test_gptq_2d.py:91-111.

Bitwise targets: the golden values and states written from the reference's _trellis_quantize_torch
(tests/golden/trellis.npz, including L=16 HYB and a table with many equal costs); the PyTorch
formulation in this package and the CPU oracle on fresh random sequences; brute-force optimality on
tiny trellises; path validity (consecutive states share L - K V bits, circular when tail-biting).
"""

import functools
import itertools
import pathlib

import numpy as np
import pytest
import torch

import gptq_2d as G
import quantizer_trellis as QT
from oracle import algorithms as A
from oracle import sweep as S
from oracle import trellis as OT

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
SHAPES = (5, 1, 1, 7), (4, 1, 2, 8), (6, 1, 2, 14), (10, 2, 2, 64), (9, 3, 1, 21), (12, 4, 2, 40), (7, 1, 1, 1)


def _valid_path(states, table, K, tail_biting):
    shift = K * table.size(1)
    shared = (table.size(0) >> shift) - 1
    assert ((states[..., 1:] >> shift) == (states[..., :-1] & shared)).all()
    assert not tail_biting or ((states[..., 0] >> shift) == (states[..., -1] & shared)).all()


def test_golden_vectors():
    data = np.load(GOLDEN / "trellis.npz")
    for idx, (L, K, V, T) in enumerate(SHAPES):
        for dname in ("float32", "float64"):
            for tb in (0, 1):
                key = f"s{idx}_{dname[-7:]}_{tb}"
                print(key, flush=True)
                table = torch.from_numpy(data[key + "_table"]).to(DEV)
                x = torch.from_numpy(data[key + "_x"]).to(DEV)
                vals, st = QT.trellis_quantize_hip(x, table, K, bool(tb))
                assert np.array_equal(st.cpu().numpy(), data[key + "_states"]), key
                assert np.array_equal(vals.cpu().numpy(), data[key + "_values"]), key
                _valid_path(st, table, K, bool(tb))
    vals, st = QT.trellis_quantize_hip(torch.from_numpy(data["ties_x"]).to(DEV),
                                       torch.from_numpy(data["ties_table"]).to(DEV), 2, True)
    assert np.array_equal(st.cpu().numpy(), data["ties_states"])
    hyb = QT.hyb(device=DEV)
    for tb in (0, 1):
        vals, st = QT.trellis_quantize_hip(torch.from_numpy(data[f"hyb16_x_{tb}"]).to(DEV), hyb, 2, bool(tb))
        assert np.array_equal(st.cpu().numpy(), data[f"hyb16_states_{tb}"])
        assert np.array_equal(vals.cpu().numpy(), data[f"hyb16_values_{tb}"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_against_torch_and_oracle(dtype):
    """HIP search == this package's PyTorch formulation on the GPU == the CPU oracle, values and states, on fresh
    sequences of every shape (quantizer_trellis.py:450-479), with leading batch dimensions."""
    g = torch.Generator().manual_seed(11)
    for (L, K, V, T), tb in itertools.product(SHAPES, (False, True)):
        table = torch.randn(1 << L, V, generator=g, dtype=dtype)
        x = torch.randn(3, 5, T, generator=g, dtype=dtype)
        vals, st = QT.trellis_quantize_hip(x.to(DEV), table.to(DEV), K, tb)
        tv, ts = QT.trellis_quantize_torch(x.to(DEV), table.to(DEV), K, tb)
        ov, os_ = OT.trellis_quantize(x, table, K, tb)
        assert st.equal(ts) and vals.equal(tv), (L, K, V, T, tb)
        assert st.cpu().equal(os_) and vals.cpu().equal(ov), (L, K, V, T, tb)
    table = torch.randint(-3, 4, (1 << 8, 2), generator=g).to(dtype)  # many equal costs
    x = torch.randint(-3, 4, (40, 64), generator=g).to(dtype)
    vals, st = QT.trellis_quantize_hip(x.to(DEV), table.to(DEV), 2, True)
    assert st.cpu().equal(OT.trellis_quantize(x, table, 2, True)[1])


@pytest.mark.parametrize("rows", [257, 301, 517])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_many_rows(dtype, rows):
    """Calls with more rows than the device has compute units search two sequences per workgroup (one table
    load per state for both): 257, 301 and 517 rows (the last workgroup of the odd counts holds one), L = 12,
    V = 1 and 2, with and without tail-biting -- equal to the PyTorch formulation, values and states."""
    g = torch.Generator().manual_seed(13)
    for (L, K, V, T), tb in itertools.product(((12, 2, 2, 32), (12, 3, 1, 24)), (False, True)):
        table = torch.randn(1 << L, V, generator=g, dtype=dtype).to(DEV)
        x = torch.randn(rows, T, generator=g, dtype=dtype).to(DEV)
        vals, st = QT.trellis_quantize_hip(x, table, K, tb)
        tv, ts = QT.trellis_quantize_torch(x, table, K, tb)
        assert st.equal(ts) and vals.equal(tv), (L, K, V, T, tb)
        _valid_path(st, table, K, tb)


@pytest.mark.parametrize("tb", [True, False])
def test_bench_call(tb):
    """The benchmark's call (bench.py's Viterbi line: C4's longest antidiagonal, 512 sequences of 256, HYB L = 16,
    K = 2, V = 2, the same seeded input, values scaled per row, two sequences per workgroup with four groups per
    thread): states and values equal the PyTorch formulation (pinned by the reference's L = 16 golden states) on
    every row, and the CPU oracle on a sample of rows, bit for bit (quantizer_trellis.py:450-479)."""
    rows, T, K = 512, 256, 2
    table = QT.hyb(L=16, device=DEV)
    x = torch.randn(rows, T, generator=torch.Generator().manual_seed(0)).to(DEV)
    out = torch.empty_like(x)
    scale = torch.ones(rows, device=DEV)
    states = torch.empty(rows, T // 2, dtype=torch.int64, device=DEV)
    QT.trellis_quantize_hip(x, table, K, tb, out=out, scale=scale, states=states)
    tv, ts = QT.trellis_quantize_torch(x, table, K, tb)
    assert states.equal(ts) and out.equal(tv)
    _valid_path(states, table, K, tb)
    sample = torch.tensor([0, 1, 2, 255, 256, 257, 301, 510, 511])
    ov, os_ = OT.trellis_quantize(x[sample].cpu(), OT.hyb(L=16), K, tb)
    assert states[sample].cpu().equal(os_) and out[sample].cpu().equal(ov)
    scale2 = torch.linspace(.5, 2., rows, device=DEV)
    QT.trellis_quantize_hip(x, table, K, tb, out=out, scale=scale2, states=states)
    assert states.equal(ts) and out.equal(tv * scale2[:, None])


def _generic(monkeypatch):
    monkeypatch.setattr(QT, "distinct_rows", lambda table: None)


@pytest.mark.parametrize("rows", [1, 7, 256, 300, 512])
def test_distinct_rows_search_equals_plain(monkeypatch, rows):
    """Tables with few distinct rows (HYB L = 16, 1MAD L = 16, and L = 12 tables drawn from 5-300 distinct rows
    with K V = 2, 3, 4) are searched from per-step cost tables, written twice with each state's copy chosen by
    ``bank_copies``; the states and values equal the plain search's bit for bit, with and without tail-biting,
    for a row count below, at and above the compute units."""
    g = torch.Generator().manual_seed(17 + rows)
    cases = [(QT.hyb(device=DEV), 2), (QT.one_mad(device=DEV), 4), (QT.one_mad(device=DEV), 2)]
    for (L, V, K), distinct in zip(((12, 2, 1), (12, 1, 3), (12, 2, 2), (12, 1, 4)), (5, 300, 64, 1024)):
        pool = torch.randn(distinct, V, generator=g)
        cases.append((pool[torch.randint(0, distinct, (1 << L,), generator=g)].to(DEV), K))
    for table, K in cases:
        assert QT.distinct_rows(table) is not None
        V = table.size(1)
        T = 256 if V == 2 else 128
        x = torch.randn(rows, T, generator=g).to(DEV)
        for tb in (False, True):
            v_rows, s_rows = QT.trellis_quantize_hip(x, table, K, tb)
            with pytest.MonkeyPatch.context() as mp:
                _generic(mp)
                v_plain, s_plain = QT.trellis_quantize_hip(x, table, K, tb)
            assert s_rows.equal(s_plain) and v_rows.equal(v_plain), (table.size(0), V, K, tb)


def test_distinct_rows_one_copy(monkeypatch):
    """Sequences so long that two copies of the cost table leave no room for a second workgroup per CU (HYB,
    T = 4096) take one copy and ignore the copy bits; sequences whose minima and costs exceed the LDS take the
    plain search.  Both equal the plain search bit for bit."""
    g = torch.Generator().manual_seed(5)
    table = QT.hyb(device=DEV)
    for T in (4096, 16384):
        x = torch.randn(3, T, generator=g).to(DEV)
        v_rows, s_rows = QT.trellis_quantize_hip(x, table, 2, True)
        assert (QT.rows_index(table, 4)[1] >> 16).any()  # copy bits were passed
        with pytest.MonkeyPatch.context() as mp:
            _generic(mp)
            v_plain, s_plain = QT.trellis_quantize_hip(x, table, 2, True)
        assert s_rows.equal(s_plain) and v_rows.equal(v_plain), T


def test_distinct_rows_cache():
    """The distinct rows are found once per table and redone after an in-place change; tables with more than
    1024 distinct rows, fp64 tables and CPU tables take the plain search."""
    def expand(r):  # the table the entries stand for
        urows, index, W = r
        return urows[index.long()].transpose(0, 1).reshape(-1, urows.size(-1))

    table = QT.hyb(device=DEV)
    r1 = QT.distinct_rows(table)
    assert r1 is not None and r1[2] == 2 and r1[0].size(0) == 1024  # HYB: each look-up row, signs in either order
    assert QT.distinct_rows(table) is r1
    assert torch.equal(expand(r1).view(torch.int32), table.view(torch.int32))
    table[0] = table[5]  # another row's values: still at most 1024 distinct row pairs
    r2 = QT.distinct_rows(table)
    assert r2 is not r1 and torch.equal(expand(r2).view(torch.int32), table.view(torch.int32))
    one = QT.one_mad(device=DEV)  # 908 values, pairs of states beyond 1024: the distinct rows
    r3 = QT.distinct_rows(one)
    assert r3 is not None and r3[2] == 1 and torch.equal(expand(r3).view(torch.int32), one.view(torch.int32))
    assert QT.distinct_rows(torch.randn(1 << 12, 2, device=DEV)) is None
    assert QT.distinct_rows(QT.hyb(device=DEV, dtype=torch.float64)) is None
    assert QT.distinct_rows(QT.hyb()) is None


def test_codes_and_k():
    """The real codes at L = 16 with several K, against the oracle (quantizer_trellis.py:474-479)."""
    g = torch.Generator().manual_seed(12)
    for code, Ks in (QT.hyb(), (2, 3, 4)), (QT.one_mad(), (2, 4)), (QT.three_inst(), (2,)):
        for K in Ks:
            x = torch.randn(6, 256, generator=g)
            vals, st = QT.trellis_quantize_hip(x.to(DEV), code.to(DEV), K, True)
            _, os_ = OT.trellis_quantize(x, code, K, True)
            assert st.cpu().equal(os_), (code.size(1), K)
            assert vals.cpu().equal(code[os_, :].flatten(start_dim=-2))


def test_brute_force():
    """Without tail-biting the search is optimal over all paths (quantizer_trellis.py:407-417)."""
    g = torch.Generator().manual_seed(0)
    for L, K, V, T in (5, 1, 1, 7), (4, 1, 2, 8):
        table = torch.randn(1 << L, V, generator=g, dtype=torch.float64)
        x = torch.randn(3, T, generator=g, dtype=torch.float64)
        vals, _ = QT.trellis_quantize_hip(x.to(DEV), table.to(DEV), K, False)
        for b in range(3):
            best = OT.brute_force(x[b], table, K)
            assert abs((vals[b].cpu() - x[b]).square().sum().item() - best) < 1e-12


def test_plugins_equal():
    """The two plug-ins write the same values for a scale per matrix or per batch (quantizer_trellis.py:482-492)."""
    g = torch.Generator().manual_seed(5)
    table = QT.hyb(device=DEV)
    y_flat = torch.randn(2, 6 * 16 * 16, generator=g).to(DEV)
    select = lambda t: t.unflatten(-1, (6, 16, 16))
    for scale in torch.tensor(1.3, device=DEV), torch.tensor([1.3, .7], device=DEV)[:, None, None, None]:
        expected, out = torch.empty(2, 6, 16, 16, device=DEV), torch.empty(2, 6, 16, 16, device=DEV)
        QT.trellis_quantizer_super_entry_torch(y_flat, select, scale, out=expected, table=table, K=2)
        QT.trellis_quantizer_super_entry_hip(y_flat, select, scale, out=out, table=table, K=2)
        assert out.equal(expected)


def test_plugin_graph():
    """The captured HIP plug-in replays on new inputs and scales, each replay checked against an eager call
    (quantizer_trellis.py:494-519)."""
    g = torch.Generator().manual_seed(6)
    table = QT.hyb(device=DEV)
    select = lambda t: t.unflatten(-1, (6, 16, 16))
    y_flat, scale = torch.randn(6 * 16 * 16, generator=g).to(DEV), torch.tensor(1.3, device=DEV)
    out = torch.empty(6, 16, 16, device=DEV)
    run = lambda: QT.trellis_quantizer_super_entry_hip(y_flat, select, scale, out=out, table=table, K=2)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run()
    for factor in (1., 2.5, .5):
        new_y, new_scale = factor * torch.randn(6 * 16 * 16, generator=g).to(DEV), torch.tensor(.9 * factor, device=DEV)
        y_flat.copy_(new_y)
        scale.copy_(new_scale)
        graph.replay()
        torch.cuda.synchronize()
        expected = torch.empty_like(out)
        QT.trellis_quantizer_super_entry_hip(new_y, select, new_scale, out=expected, table=table, K=2)
        torch.cuda.synchronize()
        assert out.equal(expected), factor


def _instance(m, n, seed, se):
    gen = torch.Generator().manual_seed(seed)
    x = 4. * torch.randn(m, n, generator=gen, dtype=torch.float64)
    l, u = (.05 * torch.randn(k, k, generator=gen, dtype=torch.float64) for k in (m, n))
    for f, size, unused in ((l, se[0], torch.ge), (u, se[1], torch.le)):
        blk = torch.arange(f.size(0)) // size
        f[unused(blk[None, :], blk[:, None])] = torch.nan
    return x.to(DEV), l.to(DEV), u.to(DEV)


def test_joint_quantizer_in_sweep():
    """A trellis rounds each 16 x 16 super-entry as one sequence inside GPTQ-2D, also in a graph with new inputs
    (test_gptq_2d.py:91-111): the sweep equals super-entry Algorithm 3 with the oracle's trellis quantizer."""
    table = torch.randn(1 << 8, 2, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    opts = dict(quantizer=functools.partial(QT.trellis_quantizer_super_entry_hip, table=table.to(DEV), K=2),
                super_entry_shape=(16, 16))

    def reference(x, l, u, scale):
        def trellis(y, i, j):
            out = torch.empty_like(y)
            OT.trellis_quantizer_super_entry(y, lambda t: t, scale, out=out, table=table, K=2)
            return out

        lu = S.unit_triangular(l.cpu(), False, 16)
        uu = S.unit_triangular(u.cpu(), True, 16)
        return A.alg3_super_entry(x.cpu(), lu, uu, Q=trellis, super_entry_shape=(16, 16)).to(DEV)

    x, l, u = _instance(32, 64, 7, (16, 16))
    scale = torch.tensor(4., dtype=torch.float64, device=DEV)
    expected = reference(x, l, u, scale.cpu())
    for inner, outer in ((0, 0), (1, 0), (1, 2)):
        got = G.gptq_2d_super_entry(x, l, u, quantizer_inputs=(scale,), inner_block_size=inner,
                                    outer_block_size=outer, **opts)
        assert got.equal(expected), (inner, outer)
    replay = G.capture_gptq_2d(x, l, u, quantizer_inputs=(scale,), **opts)
    assert replay(x, l, u, scale).equal(expected)
    assert replay(x + .375, 1.5 * l, .5 * u, 2 * scale).equal(reference(x + .375, 1.5 * l, .5 * u, 2 * scale.cpu()))
