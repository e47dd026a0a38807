"""QAT kernels (quant/dimq.py:197-296) against the float64 CPU oracle (oracle/qat.py, gradients by autograd):
softmin distortion, soft dequantization and separation loss forward and backward, the hard STE, and the
nearest-centre values with their gradient to the centres."""

import pytest
import torch

import oracle
from oracle import qat as oqat
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(n, K, seed, dt=torch.float32):
    g = _gen(seed)
    w = (torch.randn(n, generator=g) * 0.05).to(dt)
    c = (torch.randn(K, generator=g) * 0.05).sort().values
    return w, c


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _close_dtype(got, ref, dt, rel=1e-4):
    """got (rounded to dt) against the float64 ref: the dtype's rounding (half an ulp, subnormal spacing
    included) plus rel of the largest value for the fp32 arithmetic before it."""
    got, ref = got.double().cpu(), ref.double().cpu()
    fi = torch.finfo(dt)
    bound = fi.eps * ref.abs() + fi.smallest_normal * fi.eps + rel * float(ref.abs().max())
    return bool(((got - ref).abs() <= bound).all())


@pytest.mark.parametrize("n,K", [(1, 1), (1000, 2), (4099, 8), (100_003, 16), (20_000, 256), (1 << 20, 16)])
@pytest.mark.parametrize("tau", [1.0, 1e-2, 1e-4, 1e-9])
def test_softmin_loss_forward_backward(gpu, n, K, tau):
    from dimq_amd import qat
    announce(f"softmin n={n} K={K} tau={tau}")
    w, c = _case(n, K, n + K)
    wd = w.to(gpu).requires_grad_()
    cd = c.to(gpu).requires_grad_()
    loss = qat.dimq_softmin_loss(wd, cd, tau)
    assert loss.dtype == torch.float32 and loss.shape == ()
    (loss * 3.0).backward()
    wo = w.float().requires_grad_()
    co = c.float().requires_grad_()
    ref = oqat.softmin_loss(wo, co, tau)
    (ref * 3.0).backward()
    assert _rel(loss.detach(), ref.detach()) <= 2e-5
    assert _rel(wd.grad, wo.grad) <= 1e-4
    assert _rel(cd.grad, co.grad) <= 1e-4


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_softmin_loss_mean_and_dtypes(gpu, dt):
    from dimq_amd import qat
    w, c = _case(30_000, 16, 7, dt)
    wd = w.to(gpu).requires_grad_()
    cd = c.to(gpu).requires_grad_()
    loss = qat.dimq_softmin_loss(wd, cd, 5e-3, reduction="mean_per_layer")
    loss.backward()
    wo = w.float().requires_grad_()  # the fp32 values of the weights, as the reference's w.float()
    co = c.float().requires_grad_()
    ref = oqat.softmin_loss(wo, co, 5e-3, "mean_per_layer")
    ref.backward()
    assert _rel(loss.detach(), ref.detach()) <= 2e-5
    assert wd.grad.dtype == dt
    assert _close_dtype(wd.grad, wo.grad, dt)  # grad_w rounded to w's dtype (fp16: mostly subnormal here)
    assert _rel(cd.grad, co.grad) <= 1e-4
    with pytest.raises(ValueError, match="reduction"):
        qat.dimq_softmin_loss(wd, cd, 1.0, reduction="mean")


@pytest.mark.parametrize("n,K,tau", [(1, 1, 1.0), (5000, 4, 1e-3), (70_001, 16, 2e-2), (10_000, 256, 1e-5),
                                     (3000, 8, 1e-10)])
def test_soft_dequantize_forward_backward(gpu, n, K, tau):
    from dimq_amd import qat
    announce(f"soft dequantize n={n} K={K} tau={tau}")
    w, c = _case(n, K, 3 * n + K)
    wd = w.to(gpu).requires_grad_()
    cd = c.to(gpu).requires_grad_()
    y = qat.soft_dequantize_weight(wd, cd, tau)
    assert y.dtype == w.dtype and y.shape == w.shape
    up = torch.randn(n, generator=_gen(9))
    (y * up.to(gpu)).sum().backward()
    wo = w.float().requires_grad_()
    co = c.float().requires_grad_()
    ref = oqat.soft_dequantize(wo, co, tau)
    (ref * up.double()).sum().backward()
    assert _rel(y.detach(), ref.detach()) <= 1e-5
    assert _rel(wd.grad, wo.grad) <= 2e-4
    assert _rel(cd.grad, co.grad) <= 2e-4


@pytest.mark.parametrize("K,eta,spread", [(1, 1.0, 0.1), (2, 1.0, 1e-3), (16, 1.0, 0.01), (16, 3.0, 0.02),
                                          (256, 1.0, 0.05), (8, 0.5, 1.0)])
def test_separation_loss_forward_backward(gpu, K, eta, spread):
    from dimq_amd import qat
    g = _gen(K + 11)
    w = torch.randn(50_000, generator=g) * 0.05
    c = (torch.randn(K, generator=g) * spread).sort().values
    c[K // 2:] = c[K // 2:] + 0.0  # keep the layout; near pairs come from the small spreads
    wd = w.to(gpu).requires_grad_()
    cd = c.to(gpu).requires_grad_()
    loss = qat.separation_loss(wd, cd, eta)
    co = c.float().requires_grad_()
    ref = oqat.separation_loss(w, co, eta)
    if K == 1:
        assert float(loss) == 0.0
        return
    (loss * 2.0).backward()
    (ref * 2.0).backward()
    assert wd.grad is None  # the margin comes from the detached weights
    assert abs(float(loss) - float(ref)) <= 1e-5 * max(float(ref), 1e-12) + 1e-12
    assert _rel(cd.grad, co.grad) <= 1e-4 or float(co.grad.abs().max()) == 0.0


def test_hard_ste_and_values(gpu):
    """hard_ste: the forward is the hard-quantized weight, the backward the identity to w and nothing to the
    centres (quant/dimq_wrapper.py:78-80); hard_quantize_weight's values are differentiable in the centres
    through the indexing, as the reference's centers[idx]."""
    from dimq_amd import qat
    w, c = _case(10_000, 16, 21)
    wd = w.to(gpu).requires_grad_()
    cd = c.to(gpu).requires_grad_()
    y = qat.fake_quant_weight_ste(wd, cd)
    idx, vals = oracle.hard_quantize(w, c)
    assert torch.equal(y.detach().cpu(), torch.from_numpy(vals))
    up = torch.randn(10_000, generator=_gen(2)).to(gpu)
    (y * up).sum().backward()
    assert torch.equal(wd.grad, up) and cd.grad is None
    v, i = qat.hard_quantize_weight(wd.detach(), cd)
    assert torch.equal(i.cpu(), torch.from_numpy(idx).long())
    (v * up).sum().backward()
    want = torch.zeros(16, dtype=torch.float64).index_add_(0, torch.from_numpy(idx).long(), up.cpu().double())
    assert torch.allclose(cd.grad.cpu().double(), want, rtol=1e-5, atol=1e-5)
    a = qat.fake_quant_activation_ste(torch.tensor([0.5, -2.0, 7.0], device=gpu), torch.tensor([-1.0, 0.0, 1.0], device=gpu))
    assert a.cpu().tolist() == [0.0, -1.0, 1.0]  # 0.5 ties between 0 and 1: the first centre wins


def test_qat_deterministic_and_errors(gpu):
    from dimq_amd import qat
    w, c = _case(200_000, 16, 5)
    wd, cd = w.to(gpu), c.to(gpu)
    a = qat.dimq_softmin_loss(wd, cd, 1e-3)
    b = qat.dimq_softmin_loss(wd, cd, 1e-3)
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="non-empty"):
        qat.dimq_softmin_loss(wd, cd[:0], 1.0)
    with pytest.raises(RuntimeError, match="256"):
        qat.dimq_softmin_loss(wd, torch.zeros(300, device=gpu), 1.0)
