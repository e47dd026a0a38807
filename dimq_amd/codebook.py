"""Codebook initialisation and nearest-centre assignment.

* ``init_centers_per_channel`` / ``init_centers_1d`` build the quantile
  codebook of ``quant/dimq.py:88-137,175-194`` (the initialiser the BASELINE
  configurations use): K centres at the quantiles ``linspace(0, 1, K+2)[1:-1]``
  of a weight row, then spread so that they strictly increase and re-centred
  on the quantiles' mean.  Both share one vectorised implementation over rows
  (per output channel, or one row for a per-layer codebook).  The reference's
  other initialisers (k-means, min/max linspace) belong to its QAT training
  and are not provided.
* ``assign_indices`` / ``hard_quantize_weight`` keep the reference semantics
  of ``quant/dimq.py:197-221`` (argmin of the squared distance, first minimum)
  and run on the GPU kernel (``dimq_hard_quantize``).
"""

from __future__ import annotations

import torch

from . import ops


def _spread(centers: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """Sorted, strictly increasing, re-centred codebooks of [R, K] centres for
    their [R, n] weight rows (quant/dimq.py:175-194).

    Walking up each sorted row, a centre that does not exceed its predecessor
    is moved to predecessor + gap, gap = 1e-6 * max(span, std) of the row's
    weights (at least 1e-12); the row is then shifted so that its mean equals
    that of the sorted centres before the walk.  Rows whose centres are not
    all finite restart from the linspace over mean +- 3 std of their weights.
    """
    K = centers.shape[1]
    mu = rows.mean(dim=1, keepdim=True)
    sd = rows.std(dim=1, unbiased=False, keepdim=True)
    bad = ~torch.isfinite(centers).all(dim=1, keepdim=True)
    if bool(bad.any()):
        steps = torch.linspace(-3.0, 3.0, K, dtype=centers.dtype, device=centers.device)[None, :]
        fallback = torch.where(sd > 0, mu + sd * steps, mu.expand(-1, K))
        centers = torch.where(bad, fallback, centers)
    base = centers.float().sort(dim=1).values
    span = (rows.max(dim=1).values - rows.min(dim=1).values).abs()
    gap = torch.maximum(span, sd[:, 0].abs()).clamp_min(1e-6) * 1e-6
    walked = base.clone()
    for i in range(1, K):
        prev, cur = walked[:, i - 1], walked[:, i]
        walked[:, i] = torch.where(cur <= prev, prev + gap, cur)
    walked -= (walked.mean(dim=1) - base.mean(dim=1))[:, None]
    return walked.sort(dim=1).values


def _quantile_rows(rows: torch.Tensor, K: int) -> torch.Tensor:
    """[R, K] quantile codebooks of finite [R, n] fp32 rows."""
    if rows.shape[1] == 1:
        centers = rows.expand(-1, K).clone()
    else:
        q = torch.linspace(0.0, 1.0, K + 2, dtype=rows.dtype, device=rows.device)[1:-1]
        centers = torch.quantile(rows, q, dim=1).T.contiguous()
    return _spread(centers, rows)


@torch.no_grad()
def init_centers_1d(w: torch.Tensor, K: int, method: str = "quantile", *, sample_size: int = 200000) -> torch.Tensor:
    """One sorted K-entry codebook for a whole weight tensor (quant/dimq.py:88-130).

    Non-finite weights are left out; above ``sample_size`` weights the codebook
    is built on ``torch.randperm(n)[:sample_size]`` of them, as the reference
    does, so the same generator state gives the same codebook.
    """
    if K <= 0:
        raise ValueError("K must be positive")
    if method.lower() != "quantile":
        raise ValueError(f"Unsupported center initialization: {method} (this backend provides 'quantile')")
    flat = w.detach().float().reshape(-1)
    if flat.numel() == 0:
        raise ValueError("Cannot initialize centers from an empty tensor")
    flat = flat[torch.isfinite(flat)]
    if flat.numel() == 0:
        raise ValueError("Cannot initialize centers because all weights are non-finite")
    if flat.numel() > sample_size:
        flat = flat[torch.randperm(flat.numel(), device=flat.device)[:sample_size]]
    return _quantile_rows(flat[None, :], K)[0].to(device=w.device, dtype=w.dtype)


@torch.no_grad()
def init_centers_per_channel(w: torch.Tensor, K: int, method: str = "quantile") -> torch.Tensor:
    """[out_channels, K] codebook: the quantile codebook of every output row of w.

    Rows are ``w.reshape(out_channels, -1)``; they must be finite and are used
    whole (a row of the BASELINE layers holds at most 4,608 weights, far below
    the reference's 200,000-weight subsampling threshold)."""
    if K <= 0:
        raise ValueError("K must be positive")
    if method.lower() != "quantile":
        raise ValueError(f"Unsupported center initialization: {method} (this backend provides 'quantile')")
    rows = w.detach().float().reshape(w.shape[0], -1)
    if rows.numel() == 0:
        raise ValueError("Cannot initialize centers from an empty tensor")
    if not bool(torch.isfinite(rows).all()):
        raise ValueError("per-channel codebooks need finite weights")
    return _quantile_rows(rows, K).to(w.dtype)


def _to_gpu(t: torch.Tensor) -> torch.Tensor:
    if t.is_cuda:
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("the DIMQ HIP backend needs a GPU; no GPU is visible")
    return t.cuda()


@torch.no_grad()
def assign_indices(w: torch.Tensor, centers: torch.Tensor) -> torch.Tensor:
    """uint8 nearest-centre indices, weight-shaped; centers [K] or [out_channels, K] (per channel)."""
    per_channel = centers.dim() == 2 and centers.shape[0] == w.shape[0] and centers.shape[0] > 1
    idx, _ = ops.hard_quantize(_to_gpu(w), _to_gpu(centers), per_channel)
    return idx.to(w.device)


@torch.no_grad()
def hard_quantize_weight(w: torch.Tensor, centers: torch.Tensor, chunk_size: int | None = 262144):
    """(values, idx) as in quant/dimq.py:197-221, computed by the GPU kernel."""
    del chunk_size  # chunking only bounds the reference's host memory; results are identical
    per_channel = centers.dim() == 2 and centers.shape[0] == w.shape[0] and centers.shape[0] > 1
    idx, vals = ops.hard_quantize(_to_gpu(w), _to_gpu(centers), per_channel)
    return vals.to(device=w.device, dtype=w.dtype), idx.long().to(w.device)
