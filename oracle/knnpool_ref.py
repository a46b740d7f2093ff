"""Oracle of the kNN pooling forward (test infrastructure only, see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch


def normalize(x, dim=None):
    """Min-max normalisation (reference fovi/utils/__init__.py:126-167): (x - min) / (max - min),
    min and max over ``dim`` (keepdim) or over the whole tensor."""
    if dim is not None:
        lo = x.min(dim).values.unsqueeze(dim)
        hi = x.max(dim).values.unsqueeze(dim)
    else:
        lo, hi = x.min(), x.max()
    return (x - lo) / (hi - lo)


def gaussian_weights(knn_distances, sigma):
    """KNNPoolingLayer._compute_gaussian_weights (reference knn.py:325-343): distances [k, N_out]
    min-max normalised per output point, exp(-d^2 / (2 sigma^2)), divided by (sum + 1e-8).
    Returns [k, N_out] fp32."""
    d = normalize(knn_distances, dim=0)
    w = torch.exp(-d ** 2 / (2 * sigma ** 2))
    return w / (w.sum(dim=0, keepdim=True) + 1e-8)


def knnpool_forward(x, knn_indices, n_in, mode, weights=None):
    """KNNPoolingLayer.forward restated with torch CPU ops (reference fovi/arch/knn.py:345-394).

    x [B, C, N_in]; knn_indices [k, N_out] (indices >= n_in are the pad token, whose feature
    is the appended NaN column, knn.py:357); mode 'max' | 'avg' | 'sum' | 'gaussian'
    (weights [k, N_out]). Returns [B, C, N_out].
    """
    B, C, _ = x.shape
    k, n_out = knn_indices.shape
    idx = knn_indices.clone()
    idx[idx >= n_in] = n_in
    xp = torch.cat([x, torch.nan * torch.zeros(B, C, 1, dtype=x.dtype)], dim=2)          # knn.py:357
    f = torch.gather(xp, 2, idx.reshape(1, 1, -1).expand(B, C, -1)).reshape(B, C, k, n_out)  # knn.py:362-363
    if mode == "avg":
        return torch.nanmean(f, dim=2)                                                  # knn.py:367
    if mode == "max":
        f = f.clone()
        f[torch.isnan(f)] = -float("inf")                                               # knn.py:369
        return torch.max(f, dim=2)[0]                                                   # knn.py:370
    if mode == "sum":
        return torch.nansum(f, dim=2)                                                   # knn.py:372
    if mode == "gaussian":
        nan = torch.isnan(f)                                                            # knn.py:379
        clean = torch.where(nan, torch.zeros_like(f), f)
        w = weights.unsqueeze(0).unsqueeze(0)
        w = torch.where(nan, torch.zeros_like(w), w)                                    # knn.py:384
        w = w / (w.sum(dim=2, keepdim=True) + 1e-8)                                     # knn.py:387-388
        return torch.sum(clean * w, dim=2)                                              # knn.py:391
    raise NotImplementedError(f"Pooling style {mode} not implemented")


def knnpool_bruteforce(x, knn_indices, n_in, mode, weights=None):
    """Independent float64 loop form of the four pooling modes, NaN handled per definition:
    max over the features with NaN read as -inf; mean / sum over the non-NaN features (mean
    of none = NaN); Gaussian: sum of f_j w_j / (sum of the non-NaN w_j + 1e-8)."""
    x = np.asarray(x, np.float64)
    idx = np.asarray(knn_indices)
    w = None if weights is None else np.asarray(weights, np.float64)
    B, C, _ = x.shape
    k, n_out = idx.shape
    y = np.zeros((B, C, n_out))
    for b in range(B):
        for c in range(C):
            for n in range(n_out):
                vals = [x[b, c, i] if i < n_in else np.nan for i in idx[:, n]]
                ok = [not np.isnan(v) for v in vals]
                if mode == "max":
                    y[b, c, n] = max(v if o else -np.inf for v, o in zip(vals, ok))
                elif mode == "avg":
                    good = [v for v, o in zip(vals, ok) if o]
                    y[b, c, n] = sum(good) / len(good) if good else np.nan
                elif mode == "sum":
                    y[b, c, n] = sum(v for v, o in zip(vals, ok) if o)
                else:
                    s = sum(w[j, n] for j in range(k) if ok[j])
                    y[b, c, n] = sum(vals[j] * w[j, n] / (s + 1e-8) for j in range(k) if ok[j])
    return y
