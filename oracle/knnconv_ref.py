"""Oracle of the kNN-conv forward (test infrastructure only, see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def knnconv_forward(x, knn_indices, n_in, local_rf, weight, bias=None):
    """KNNConvLayer.forward restated with torch CPU fp32 (reference fovi/arch/knn.py:484-557).

    x [B, C, N_in]; knn_indices [k, N_out] (indices >= n_in are the pad
    token, knn.py:451-453); local_rf [N_out, k, V] one-hot; weight
    [C_out, C*V] with reduction index c*V + v. Returns [B, C_out, N_out].
    """
    B, C, _ = x.shape
    k, n_out = knn_indices.shape
    V = local_rf.shape[2]
    idx = knn_indices.clone()
    idx[idx >= n_in] = n_in
    xp = torch.cat([x, torch.zeros(B, C, 1, dtype=x.dtype)], dim=2)                      # knn.py:495
    g = torch.gather(xp, 2, idx.reshape(1, 1, -1).expand(B, C, -1)).reshape(B, C, k, n_out)  # knn.py:500
    g = g.permute(0, 1, 3, 2).reshape(B * C, n_out, k)                                  # knn.py:521
    g = torch.einsum("ank,nkv->anv", g, local_rf.to(g.dtype))                          # knn.py:522
    g = g.reshape(B, C, n_out, V).permute(0, 2, 1, 3).reshape(B, n_out, C * V)          # knn.py:524
    return F.linear(g, weight, bias).transpose(1, 2)                                    # knn.py:555


def knnconv_bruteforce(x, knn_indices, slots, n_in, weight, bias=None):
    """Independent float64 loop form: y[b,o,n] = sum_j sum_c x[b,c,nbr_j] * W[o, c*V + slot_j]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    idx = np.asarray(knn_indices)
    sl = np.asarray(slots)
    B, C, _ = x.shape
    k, n_out = idx.shape
    c_out = w.shape[0]
    V = w.shape[1] // C
    y = np.zeros((B, c_out, n_out))
    for n in range(n_out):
        for j in range(k):
            src = idx[j, n]
            if src < 0 or src >= n_in:
                continue
            cols = np.arange(C) * V + sl[n, j]
            y[:, :, n] += x[:, :, src] @ w[:, cols].T
    if bias is not None:
        y += np.asarray(bias, np.float64)[None, :, None]
    return y


def quantize_e4m3(t, scale):
    """``(t / scale).to(float8_e4m3fn)`` back to fp32: the fp8 operand values."""
    return (t / scale).to(torch.float8_e4m3fn).to(torch.float32)
