"""Oracle of the kNN-conv forward (test infrastructure only, see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def knnconv_forward(x, knn_indices, n_in, local_rf, weight, bias=None):
    """KNNConvLayer.forward restated with torch CPU fp32 (reference fovi/arch/knn.py:484-557).

    x [B, C, N_in]; knn_indices [k, N_out] (indices >= n_in, and the -1 that pads a
    partitioning patch embedding's groups, are the pad token, knn.py:451-453 and
    knnvit.py:196-198); local_rf [N_out, k, V] one-hot; weight
    [C_out, C*V] with reduction index c*V + v. Returns [B, C_out, N_out].
    """
    B, C, _ = x.shape
    k, n_out = knn_indices.shape
    V = local_rf.shape[2]
    idx = knn_indices.clone()
    idx[(idx >= n_in) | (idx < 0)] = n_in
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


def e4m3_values():
    """The 254 finite OCP e4m3 values by code (bias 7, subnormals m * 2^-9, codes
    0x7f/0xff NaN): float64 array of length 256 with NaN at the two NaN codes."""
    v = np.empty(256)
    for code in range(256):
        s, e, m = code >> 7, (code >> 3) & 15, code & 7
        mag = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        v[code] = np.nan if (e == 15 and m == 7) else (-mag if s else mag)
    return v


def e4m3_round_bruteforce(x):
    """Round-to-nearest-even onto the e4m3 grid by exhaustive search, saturating at
    +-448: the nearest finite value, ties to the code with an even mantissa."""
    vals = e4m3_values()
    codes = np.array([c for c in range(256) if not np.isnan(vals[c])])
    grid = vals[codes]
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    for i, t in np.ndenumerate(x):
        if np.isnan(t):
            out[i] = np.nan
            continue
        t = min(max(t, -448.0), 448.0)
        d = np.abs(grid - t)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:     # a tie: the even mantissa (for +-0 either is 0)
            best = [b for b in best if (codes[b] & 1) == 0] or best
        out[i] = grid[best[0]]
    return out


def knnconv_fp8_forward(xq, x_scale, knn_indices, n_in, local_rf, wq, w_scale, bias=None):
    """The fp8 kNN-conv on dequantized operands (no reference counterpart; the
    structure is knn.py:484-557 with e4m3 operands).

    xq [B, C, N_in] and wq [C_out, C*V] hold e4m3 values (as fp32); the slot
    sums A[b, n, c, v] = sum of xq over the neighbours of n in slot v are exact
    in float64 and are rounded once more to e4m3 where a slot holds two or more
    neighbours (the kernel feeds e4m3 operands to the MFMA). Returns
    x_scale * w_scale[o] * sum_{c,v} A * wq[o, c*V+v] + bias[o], [B, C_out, N_out].
    """
    B, C, _ = xq.shape
    k, n_out = knn_indices.shape
    V = local_rf.shape[2]
    idx = knn_indices.clone()
    idx[(idx >= n_in) | (idx < 0)] = n_in
    xp = torch.cat([xq.double(), torch.zeros(B, C, 1, dtype=torch.float64)], dim=2)
    g = torch.gather(xp, 2, idx.reshape(1, 1, -1).expand(B, C, -1)).reshape(B, C, k, n_out)
    g = g.permute(0, 1, 3, 2)                                                   # [B, C, N, k]
    rf = local_rf.double()
    a = torch.einsum("bcnk,nkv->bncv", g, rf)                                   # slot sums
    multi = (rf.sum(1) >= 2)[None, :, None, :].expand_as(a)                     # [1, N, 1, V]
    a = torch.where(multi, a.float().to(torch.float8_e4m3fn).double(), a)
    y = torch.einsum("bncv,ocv->bon", a, wq.double().reshape(-1, C, V))
    y = y * (float(x_scale) * w_scale.double())[None, :, None]
    if bias is not None:
        y = y + bias.double()[None, :, None]
    return y
