"""CPU oracle of the DIMQ QAT functions (TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker).

Float64 restatements of the reference's formulas on the CPU; gradients come from torch's autograd over
them, which is how the reference obtains its own (it defines no backward):

* ``softmin_loss``    -- quant/dimq.py:244-273 (per element ``-tau (logsumexp(-d / tau) - log K)``, summed or
  averaged over the elements);
  (the squared distances in fp32 as the reference forms them, everything after them in float64);
* ``soft_dequantize`` -- quant/dimq.py:224-241 (``softmax(-d / tau) @ c``);
* ``separation_loss`` -- quant/dimq.py:276-296 (pairs ``a < b`` of the centres, margin
  ``eta * 6 * std(w, unbiased=False) / K`` from the detached weights).

Pinned in ``tests/test_oracle.py`` by closed forms that do not retype these expressions: one centre (the loss
is the plain squared distance), two centres (the softmin term in closed form with ``log1p``), tau -> 0 (the
hard nearest-centre distortion), tau -> infinity (the uniform mean), the two-centre hinge, and finite
differences of each function.
"""

from __future__ import annotations

import math

import torch


def _d(w: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """Squared distances as the reference forms them -- from w.float() and c.float() in fp32
    (quant/dimq.py:229-236, :253-263) -- or in float64 for float64 inputs; returned as float64 for the rest."""
    dt = torch.float64 if (w.dtype == torch.float64 and c.dtype == torch.float64) else torch.float32
    return ((w.to(dt).reshape(-1)[:, None] - c.to(dt).reshape(-1)[None, :]) ** 2).double()


def softmin_loss(w: torch.Tensor, c: torch.Tensor, tau: float, reduction: str = "sum") -> torch.Tensor:
    tau = max(float(tau), 1e-12)
    K = c.numel()
    per = -tau * (torch.logsumexp(-_d(w, c) / tau, dim=1) - math.log(K))
    return per.sum() if reduction == "sum" else per.sum() / max(1, per.numel())


def soft_dequantize(w: torch.Tensor, c: torch.Tensor, tau: float) -> torch.Tensor:
    tau = max(float(tau), 1e-12)
    p = torch.softmax(-_d(w, c) / tau, dim=1)
    return (p @ c.double().reshape(-1)).reshape(w.shape)


def separation_loss(w: torch.Tensor, c: torch.Tensor, eta: float = 1.0, eps: float = 1e-12) -> torch.Tensor:
    cc = c.double().reshape(-1)
    K = cc.numel()
    if K <= 1:
        return cc.new_zeros(())
    sigma = w.detach().double().std(unbiased=False).clamp_min(1e-12)
    delta = float(eta) * 6.0 * sigma / K
    a, b = torch.triu_indices(K, K, offset=1)
    dist = torch.sqrt((cc[a] - cc[b]) ** 2 + float(eps))
    return torch.relu(delta - dist).pow(2).sum()
