"""GPU test of the model-level driver (model_driver.quantize_model): on a two-layer MLP with Kronecker factors
collected from forward and backward passes, every layer's new weight is exactly what the public single-layer
path gives for the same factors and quantizer (ldl_of_inverse of both Grams, fused GPTQ-2D sweep), the rounding
beats rounding without feedback on the layer's objective tr(R^T A R B), and the packed INT4 codes unpack to the
new weight."""

import pytest
import torch

import gptq_2d as G
import gptq_2d_ldl as LDL
import model_driver as MD
import packing

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_quantize_mlp():
    g = torch.Generator().manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(128, 192), torch.nn.GELU(), torch.nn.Linear(192, 96))
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(0.1 * torch.randn(p.shape, generator=g))
    model = model.to(DEV)
    x = torch.randn(16, 8, 128, generator=g).to(DEV)
    target = torch.randn(16, 8, 96, generator=g).to(DEV)
    orig = {n: p.detach().clone() for n, p in model.named_parameters()}
    with MD.HessianCollector(model) as col:
        for k in range(0, 16, 4):
            model.zero_grad()
            ((model(x[k:k + 4]) - target[k:k + 4]) ** 2).sum().backward()
    assert set(col.modules) == {"0", "2"} and col.grad_tokens == {"0": 128, "2": 128}
    expect = {}
    for name in col.modules:
        a, b = col.factors(name)
        lo, up = LDL.feedback_factors_of_grams(a.float(), b.float())
        w = orig[name + ".weight"].float().contiguous()
        spec = MD.int_row_quantizer(w)
        expect[name] = G.gptq_2d(w, lo, up, quantizer=spec.quantizer, quantizer_inputs=spec.inputs,
                                 outer_block_size=1024)
    results = MD.quantize_model(model, col)
    mods = dict(model.named_modules())
    for r in results:
        w = mods[r.name].weight.detach()
        print(f"layer {r.name} {r.shape}: objective / no feedback {r.objective / r.objective_rtn:.4f}", flush=True)
        assert torch.equal(w, expect[r.name])
        assert r.objective < r.objective_rtn
        assert torch.equal(packing.unpack_int(r.words, r.scale, n=w.size(1), qmin=-8, qmax=7), w)
