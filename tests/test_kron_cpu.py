"""CPU tests of U given by its Kronecker factors (gptq_2d.KroneckerU): the pair's dense form is torch.kron of
its factors, the D-sided sweep's pair equals the U it formed before bit for bit, the host decides which inputs
the fused reader takes, and the C entry point rejects bad arguments before any device work (loaded with ctypes;
no compute call, so this runs without a GPU)."""

import ctypes
import pathlib

import pytest
import torch

import gptq_2d as G
import gptq_d_sided as DS
import quantizer_int as QI

LIB = pathlib.Path(__file__).resolve().parents[1] / "gptq-2d_amd" / "libgptq2d.so"
EINVAL, EUNSUPPORTED = -1, -2


def _unit_lower(k, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(k, k, generator=g, dtype=torch.float64).tril(-1) / k + torch.eye(k, dtype=torch.float64)).to(
        dtype)


def test_kronecker_u_contract():
    p, q = _unit_lower(3, 1).t(), _unit_lower(32, 2).t()
    u = G.KroneckerU(p, q)
    assert u.shape == (96, 96) and u.dim() == 2 and u.numel() == 96 * 96 and u.dtype == torch.float32
    assert u.device == p.device
    assert torch.equal(u.dense(), torch.kron(p, q))
    assert u.contiguous().outer.is_contiguous() and torch.equal(u.contiguous().dense(), u.dense())
    with pytest.raises(AssertionError):
        G.KroneckerU(p[:, :2], q)
    with pytest.raises(AssertionError):
        G.KroneckerU(p, q.double())


@pytest.mark.parametrize("shape", [(5, 7), (4, 3, 5), (3, 2, 4, 3), (2, 32, 3, 2)])
def test_column_factor_pair_equals_formed_product(shape):
    ls = [_unit_lower(k, 10 + i) for i, k in enumerate(shape)]
    pair = DS.column_factor_pair(ls)
    dense = pair.dense() if isinstance(pair, G.KroneckerU) else pair
    assert isinstance(pair, G.KroneckerU) == (len(shape) > 2)
    assert torch.equal(dense, DS.column_factor(ls))


def test_fused_reader_selection():
    """One fp32 matrix, inner size a multiple of 16, sizes multiples of 4, 16-byte aligned operands, a built-in
    quantizer: read from the factors; anything else forms the product."""
    def fusable(m, np_, nq, dtype=torch.float32, batch=(), spec_kind="round"):
        y = torch.zeros(*batch, m, np_ * nq, dtype=dtype)
        l = torch.eye(m, dtype=dtype)
        u = G.KroneckerU(torch.eye(np_, dtype=dtype), torch.eye(nq, dtype=dtype))
        spec = G._fused_spec(QI.round_quantizer, (), y, torch.Size(batch)) if spec_kind == "round" else None
        return G._kron_fusable(y, l, u, torch.Size(batch), spec)

    assert fusable(64, 3, 32) and fusable(100, 2, 96) and fusable(64, 2, 112) and fusable(32, 5, 48)
    assert not fusable(64, 3, 24)                          # inner size not a multiple of 16
    assert not fusable(62, 3, 32)                          # m not a multiple of 4
    assert not fusable(64, 3, 32, dtype=torch.float64)     # fp64 engine
    assert not fusable(64, 3, 32, batch=(2,))              # a batch of matrices
    assert not fusable(64, 3, 32, spec_kind=None)          # a plug-in quantizer
    # m = 2^20 rows: beyond the factor-reading flush (the check reads only L's rank and alignment, so a small
    # stand-in L keeps this test's memory at the 64 MiB of y)
    y = torch.zeros(1 << 20, 16)
    u = G.KroneckerU(torch.eye(1), torch.eye(16))
    spec = G._fused_spec(QI.round_quantizer, (), y, torch.Size(()))
    assert not G._kron_fusable(y, torch.eye(4), u, torch.Size(()), spec)
    assert G._kron_fusable(y[: (1 << 20) - 4], torch.eye(4), u, torch.Size(()), spec)


def test_entry_point_rejects_bad_arguments():
    if not LIB.exists():
        pytest.skip("libgptq2d.so is not built (run __graft_entry__.build())")
    fn = ctypes.CDLL(str(LIB)).gptq2d_sweep_fused_kron_f32
    P, I64, I32, F64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_double
    fn.argtypes = [P, P, P, P, P, P, I64, I64, I64, I64, I64, I32, P, P, F64, F64, I32, P, P, I64, I64, I64, P]
    fn.restype = ctypes.c_int
    dummy = 256  # never dereferenced: every case below returns before any device call

    def call(m=64, np_=3, nq=32, p=1, q=1, qkind=0, outer=2, up=dummy, uq=dummy, ptr=dummy):
        return fn(ptr, ptr, ptr, ptr, up, uq, m, np_, nq, p, q, qkind, None, None, 0.0, 0.0, 0, None, None, outer, 0,
                  -1, None)

    assert call(up=None) == EINVAL
    assert call(np_=0) == EINVAL
    assert call(nq=40) == EUNSUPPORTED                      # inner size not a multiple of 16
    assert call(np_=1 << 20, nq=64) == EUNSUPPORTED         # n >= 2^26
    assert call(np_=1 << 15, nq=32) == EUNSUPPORTED         # n = 2^20: beyond the factor-reading flush
    assert call(m=1 << 20) == EUNSUPPORTED                  # m = 2^20: the same
    assert call(p=3) == EINVAL                              # super-entry rows must divide m
    assert call(q=16) == EUNSUPPORTED                       # only 1 x 1 and 1 x 32 super-entries
    assert call(m=0) == EINVAL
    assert call(outer=0) == EINVAL
    assert call(qkind=7) == EINVAL
    assert call(m=62) == EUNSUPPORTED                       # rows of 62 entries: no 128-bit staging
    assert call(ptr=dummy + 4) == EUNSUPPORTED              # operands not 16-byte aligned


def test_torch_variants_take_the_pair():
    """The PyTorch variants (CPU here) run a KroneckerU as its product: the same outputs as with torch.kron."""
    g = torch.Generator().manual_seed(5)
    x = 3. * torch.randn(6, 8, generator=g, dtype=torch.float64)
    lo = _unit_lower(6, 21, torch.float64)
    p, q = _unit_lower(2, 22, torch.float64).t(), _unit_lower(4, 23, torch.float64).t()
    for fn in (G.gptq_2d_torch, G.direct_2d):
        assert torch.equal(fn(x, lo, G.KroneckerU(p, q)), fn(x, lo, torch.kron(p, q)))
    for fn in (G.gptq_2d_super_entry_torch, G.direct_2d_super_entry):
        assert torch.equal(fn(x, lo, G.KroneckerU(p, q), super_entry_shape=(2, 2)),
                           fn(x, lo, torch.kron(p, q), super_entry_shape=(2, 2)))
