"""DIMQ QAT math on the HIP kernels: the reference's quantization-aware-training functions
(quant/dimq.py:197-296, quant/dimq_wrapper.py:78-86) with the same names, arguments and
results, for CUDA (HIP) tensors.

* ``hard_quantize_weight`` -- nearest-centre assignment (the sorted-search kernel), values
  ``centers[idx].to(w.dtype)`` (differentiable in the centres through the indexing, as the
  reference's).
* ``fake_quant_weight_ste`` / ``fake_quant_activation_ste`` -- the ``hard_ste`` forward:
  ``w + (w_hard - w).detach()``: the hard values forward, the identity to ``w`` backward,
  nothing to the centres.
* ``soft_dequantize_weight`` -- ``softmax(-d / tau) @ centers`` with its backward kernel.
* ``dimq_softmin_loss`` -- the Gibbs softmin distortion, forward and backward kernels.
* ``separation_loss`` -- the hinge margin over centre pairs (margin from ``std(w)``, no
  gradient to ``w``).

``chunk_size`` is accepted for signature compatibility: the kernels stream the weights and
need no chunking.  Everything is computed in fp32 from ``w.float()`` and ``centers.float()``;
the loss values are fp32 scalars on the device.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _C


def _tau(tau: float) -> float:
    return max(float(tau), 1e-12)  # quant/dimq.py:230, :252


def hard_quantize_weight(w: Tensor, centers: Tensor, chunk_size: int | None = 262144) -> tuple[Tensor, Tensor]:
    """(values, indices) of the nearest centres (quant/dimq.py:197-221): indices int64 of w's shape, values
    ``centers[idx].to(w.dtype)``."""
    from . import ops

    c = centers.reshape(-1)
    idx, _ = ops.hard_quantize(w.detach(), c.detach().float(), False)
    idx = idx.long().reshape(w.shape)
    return c[idx].to(dtype=w.dtype), idx


class _STE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w: Tensor, centers: Tensor) -> Tensor:
        from . import ops

        _, vals = ops.hard_quantize(w.detach(), centers.detach().reshape(-1).float(), False)
        return vals.reshape(w.shape).to(w.dtype)

    @staticmethod
    def backward(ctx, grad: Tensor):
        return grad, None


def fake_quant_weight_ste(w: Tensor, centers: Tensor) -> Tensor:
    """The ``hard_ste`` forward of the QAT wrappers (quant/dimq_wrapper.py:78-80): the hard-quantized weight
    forward, the straight-through identity to ``w`` backward."""
    return _STE.apply(w, centers)


def fake_quant_activation_ste(x: Tensor, activation_centers: Tensor) -> Tensor:
    """Activations to their nearest activation centre, straight through backward (quant/dimq_wrapper.py:84-86,
    without the wrapper's running centre update)."""
    return _STE.apply(x, activation_centers)


class _SoftDequant(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w: Tensor, centers: Tensor, tau: float) -> Tensor:
        out, aux = _C.soft_dequantize_forward_impl(w, centers, tau)
        ctx.save_for_backward(w, centers, aux)
        ctx.tau = tau
        return out

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        w, centers, aux = ctx.saved_tensors
        gw, gc = _C.soft_dequantize_backward_impl(w, centers, ctx.tau, aux, grad_out)
        return gw, gc.to(centers.dtype).reshape(centers.shape), None


def soft_dequantize_weight(w: Tensor, centers: Tensor, tau: float, chunk_size: int | None = 262144) -> Tensor:
    """``softmax(-(w - c)^2 / tau) @ c`` per element, in w's dtype (quant/dimq.py:224-241)."""
    return _SoftDequant.apply(w, centers, _tau(tau))


class _Softmin(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w: Tensor, centers: Tensor, tau: float, mean: bool) -> Tensor:
        loss, aux = _C.softmin_loss_forward_impl(w, centers, tau, mean)
        ctx.save_for_backward(w, centers, aux)
        ctx.tau, ctx.mean = tau, mean
        return loss

    @staticmethod
    def backward(ctx, grad: Tensor):
        w, centers, aux = ctx.saved_tensors
        g = grad / max(1, w.numel()) if ctx.mean else grad
        gw, gc = _C.softmin_loss_backward_impl(w, centers, ctx.tau, aux, g)
        return gw, gc.to(centers.dtype).reshape(centers.shape), None, None


def dimq_softmin_loss(w: Tensor, centers: Tensor, tau: float, reduction: str = "sum",
                      chunk_size: int | None = 262144) -> Tensor:
    """Gibbs softmin distortion ``sum_i -tau (logsumexp_j(-(w_i - c_j)^2 / tau) - log K)`` (quant/dimq.py:244-273);
    ``reduction`` "sum" or "mean_per_layer"."""
    if centers.numel() == 0:
        raise ValueError("centers must be non-empty")
    if reduction not in ("sum", "mean_per_layer"):
        raise ValueError(f"Unsupported loss reduction: {reduction}")
    return _Softmin.apply(w, centers, _tau(tau), reduction == "mean_per_layer")


class _Separation(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w: Tensor, centers: Tensor, eta: float, eps: float) -> Tensor:
        loss, gc = _C.separation_loss_impl(w, centers, eta, eps)
        ctx.save_for_backward(gc)
        ctx.shape, ctx.dtype = centers.shape, centers.dtype
        return loss

    @staticmethod
    def backward(ctx, grad: Tensor):
        (gc,) = ctx.saved_tensors
        return None, (grad * gc).to(ctx.dtype).reshape(ctx.shape), None, None


def separation_loss(w: Tensor, centers: Tensor, eta: float = 1.0, eps: float = 1e-12) -> Tensor:
    """Hinge margin ``sum_{a<b} relu(delta - sqrt((c_a - c_b)^2 + eps))^2``, ``delta = eta 6 std(w) / K``
    (quant/dimq.py:276-296)."""
    if centers.numel() <= 1:
        return centers.new_zeros((), dtype=torch.float32)
    return _Separation.apply(w, centers, float(eta), float(eps))
