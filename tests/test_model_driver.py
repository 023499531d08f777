"""CPU tests of the model-level driver's Kronecker-factor collection (model_driver.HessianCollector): on a small
MLP the forward hooks' B equals X^T X of each layer's inputs and the backward hooks' A equals G^T G of the
gradients of the loss with respect to each layer's outputs (both computed directly with autograd), averaged
over the tokens, with the stated damping; without output-side statistics A is the identity; removed hooks
collect nothing.  (Quantization itself runs on the GPU: test_model_driver_gpu.py.)"""

import pytest
import torch

import model_driver as MD


class _MLP(torch.nn.Module):
    def __init__(self, g):
        super().__init__()
        self.fc1 = torch.nn.Linear(12, 20, dtype=torch.float64)
        self.fc2 = torch.nn.Linear(20, 7, dtype=torch.float64)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float64) * 0.3)

    def forward(self, x):
        return self.fc2(torch.nn.functional.gelu(self.fc1(x)))


def _batches(g, n=3):
    return [torch.randn(4, 5, 12, generator=g, dtype=torch.float64) for _ in range(n)]


def test_input_and_output_grams():
    g = torch.Generator().manual_seed(0)
    model = _MLP(g)
    xs = _batches(g)
    target = [torch.randn(4, 5, 7, generator=g, dtype=torch.float64) for _ in xs]
    with MD.HessianCollector(model) as col:
        for x, t in zip(xs, target):
            model.zero_grad()
            ((model(x) - t) ** 2).sum().backward()
    # direct: inputs and output gradients of each layer
    b1 = b2 = a1 = a2 = 0
    for x, t in zip(xs, target):
        h1 = model.fc1(x)
        h1.retain_grad()
        u = torch.nn.functional.gelu(h1)
        y = model.fc2(u)
        y.retain_grad()
        ((y - t) ** 2).sum().backward()
        x2, u2 = x.reshape(-1, 12), u.detach().reshape(-1, 20)
        b1 = b1 + x2.t() @ x2
        b2 = b2 + u2.t() @ u2
        g1, g2 = h1.grad.reshape(-1, 20), y.grad.reshape(-1, 7)
        a1 = a1 + g1.t() @ g1
        a2 = a2 + g2.t() @ g2
    tokens = 3 * 4 * 5
    assert col.tokens == {"fc1": tokens, "fc2": tokens} and col.grad_tokens == {"fc1": tokens, "fc2": tokens}
    for name, a, b in (("fc1", a1, b1), ("fc2", a2, b2)):
        assert torch.allclose(col.B[name], b, rtol=1e-12, atol=1e-12)
        assert torch.allclose(col.A[name], a, rtol=1e-12, atol=1e-12)
        fa, fb = col.factors(name, damping=0.1)
        ea, eb = a / tokens, b / tokens
        assert torch.allclose(fa, ea + 0.1 * ea.diagonal().mean() * torch.eye(ea.size(0), dtype=ea.dtype))
        assert torch.allclose(fb, eb + 0.1 * eb.diagonal().mean() * torch.eye(eb.size(0), dtype=eb.dtype))


def test_one_sided_and_removal():
    g = torch.Generator().manual_seed(1)
    model = _MLP(g)
    xs = _batches(g, 2)
    col = MD.HessianCollector(model, layers=["fc2"], output_side=False)
    with torch.no_grad():
        for x in xs:
            model(x)
    col.remove()
    model(xs[0])  # after remove(): nothing more is collected
    assert set(col.B) == {"fc2"} and col.tokens["fc2"] == 2 * 4 * 5 and not col.A
    fa, fb = col.factors("fc2", damping=0.)
    assert torch.equal(fa, torch.eye(7, dtype=torch.float64))
    u = torch.cat([torch.nn.functional.gelu(model.fc1(x)).reshape(-1, 20) for x in xs]).detach()
    assert torch.allclose(fb, u.t() @ u / u.size(0), rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        MD.HessianCollector(model, layers=["nope"])
    with pytest.raises(KeyError):
        MD.HessianCollector(model).factors("fc1")
