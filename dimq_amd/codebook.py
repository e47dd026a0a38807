"""Codebook initialisation and nearest-centre assignment.

* ``init_centers_1d`` restates ``quant/dimq.py:88-194`` (quantile, linspace and
  k-means initialisers, then ``_postprocess_centers``); it is host-side data
  preparation in torch, as in the reference.
* ``init_centers_per_channel`` applies the same recipe to every output row at
  once (the BASELINE configurations use per-output-channel codebooks; the
  reference only has per-layer ones).
* ``hard_quantize_weight`` keeps the reference signature
  (``quant/dimq.py:197-221``) but runs the assignment on the GPU kernel
  (``dimq_hard_quantize``); ``chunk_size`` is accepted for compatibility and
  does not change the result.
"""

from __future__ import annotations

import torch

from . import ops


@torch.no_grad()
def init_centers_1d(w: torch.Tensor, K: int, method: str = "kmeans", *, kmeans_iters: int = 50,
                    sample_size: int = 200000) -> torch.Tensor:
    """Sorted 1-D codebook of K centres from a weight tensor (quant/dimq.py:88-130)."""
    if K <= 0:
        raise ValueError("K must be positive")
    flat = w.detach().float().reshape(-1)
    if flat.numel() == 0:
        raise ValueError("Cannot initialize centers from an empty tensor")
    finite = torch.isfinite(flat)
    if not bool(finite.all()):
        flat = flat[finite]
    if flat.numel() == 0:
        raise ValueError("Cannot initialize centers because all weights are non-finite")
    if flat.numel() > sample_size:
        perm = torch.randperm(flat.numel(), device=flat.device)[:sample_size]
        sample = flat[perm]
    else:
        sample = flat
    method = method.lower()
    if method == "quantile":
        centers = _quantile_centers(sample, K)
    elif method == "linspace_std":
        centers = _linspace_std_centers(sample, K)
    elif method == "linspace_minmax":
        centers = _linspace_minmax_centers(sample, K)
    elif method == "kmeans":
        centers = _kmeans_1d(sample, K, kmeans_iters)
    else:
        raise ValueError(f"Unsupported center initialization: {method}")
    centers = _postprocess_centers(centers, sample, K)
    return centers.to(device=w.device, dtype=w.dtype)


def _quantile_centers(flat: torch.Tensor, K: int) -> torch.Tensor:
    # quant/dimq.py:133-137
    if flat.numel() == 1:
        return flat.new_full((K,), flat.item())
    q = torch.linspace(0.0, 1.0, K + 2, device=flat.device, dtype=flat.dtype)[1:-1]
    return torch.quantile(flat, q)


def _linspace_std_centers(flat: torch.Tensor, K: int) -> torch.Tensor:
    # quant/dimq.py:140-145
    mu = flat.mean()
    sigma = flat.std(unbiased=False)
    if float(sigma) <= 0.0:
        return flat.new_full((K,), float(mu))
    return torch.linspace(mu - 3.0 * sigma, mu + 3.0 * sigma, K, device=flat.device, dtype=flat.dtype)


def _linspace_minmax_centers(flat: torch.Tensor, K: int) -> torch.Tensor:
    # quant/dimq.py:148-153
    lo = flat.min()
    hi = flat.max()
    if float((hi - lo).abs()) <= 0.0:
        return flat.new_full((K,), float(lo))
    return torch.linspace(lo, hi, K, device=flat.device, dtype=flat.dtype)


def _kmeans_1d(flat: torch.Tensor, K: int, iters: int) -> torch.Tensor:
    # quant/dimq.py:156-172 (Lloyd iterations from quantile seeds)
    centers = _quantile_centers(flat, K)
    if K == 1:
        return centers
    for _ in range(max(1, int(iters))):
        assignment = ((flat[:, None] - centers[None, :]) ** 2).argmin(dim=1)
        new_centers = centers.clone()
        for k in range(K):
            mask = assignment == k
            if bool(mask.any()):
                new_centers[k] = flat[mask].mean()
        if torch.allclose(new_centers, centers):
            break
        centers = new_centers.sort().values
    return centers


def _postprocess_centers(centers: torch.Tensor, reference: torch.Tensor, K: int) -> torch.Tensor:
    """quant/dimq.py:175-194: sort, enforce a strictly increasing minimum gap, re-centre."""
    if centers.numel() != K:
        raise ValueError(f"Expected {K} centers, got {centers.numel()}")
    if not bool(torch.isfinite(centers).all()):
        centers = _linspace_std_centers(reference, K)
    centers = centers.float().sort().values
    span = (reference.max() - reference.min()).abs()
    sigma = reference.std(unbiased=False).abs()
    scale = torch.maximum(span, sigma).clamp_min(1e-6)
    min_gap = scale * 1e-6
    fixed = centers.clone()
    for i in range(1, K):
        if fixed[i] <= fixed[i - 1]:
            fixed[i] = fixed[i - 1] + min_gap
    center_shift = fixed.mean() - centers.mean()
    fixed = fixed - center_shift
    return fixed.sort().values


@torch.no_grad()
def init_centers_per_channel(w: torch.Tensor, K: int, method: str = "quantile") -> torch.Tensor:
    """[out_channels, K] codebook: the quantile recipe of init_centers_1d applied to every row.

    Rows are the flattened output channels (w.reshape(out_channels, -1)); every
    row is small enough (< 200,000 weights) that no subsampling applies.
    """
    rows = w.detach().float().reshape(w.shape[0], -1)
    if method != "quantile":
        return torch.stack([init_centers_1d(r, K, method) for r in rows]).to(w.dtype)
    if rows.shape[1] == 1:
        centers = rows.expand(-1, K).clone()
    else:
        q = torch.linspace(0.0, 1.0, K + 2, device=rows.device, dtype=rows.dtype)[1:-1]
        centers = torch.quantile(rows, q, dim=1).T.contiguous()
    # _postprocess_centers, row-wise
    centers = centers.sort(dim=1).values
    span = (rows.max(dim=1).values - rows.min(dim=1).values).abs()
    sigma = rows.std(dim=1, unbiased=False).abs()
    min_gap = (torch.maximum(span, sigma).clamp_min(1e-6) * 1e-6)
    fixed = centers.clone()
    for i in range(1, K):
        bad = fixed[:, i] <= fixed[:, i - 1]
        fixed[:, i] = torch.where(bad, fixed[:, i - 1] + min_gap, fixed[:, i])
    shift = fixed.mean(dim=1) - centers.mean(dim=1)
    fixed = fixed - shift[:, None]
    return fixed.sort(dim=1).values.to(w.dtype)


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
