"""Oracle of the fixation policy's draws (test infrastructure only, see oracle/__init__.py).

The reference draws from numpy's global generator; these functions take an explicit
``np.random.RandomState`` so a test can replay a seed (``np.random.seed(s)`` and
``RandomState(s)`` give the same stream).
"""
from __future__ import annotations

import numpy as np


def random_crop(rs, height, width, scale, ratio):
    """BaseSaccadePolicy.get_random_crop (reference fovi/sensing/policies.py:36-88):
    returns ((cy, cx), (h, w))."""
    area = height * width
    log_ratio = np.log(ratio)
    for _ in range(10):                                                    # policies.py:53
        if hasattr(scale, "__len__"):
            target_area = area * rs.uniform(scale[0], scale[1])           # policies.py:55
        else:
            target_area = area * scale
        if hasattr(ratio, "__len__"):
            aspect_ratio = np.exp(rs.uniform(log_ratio[0], log_ratio[1]))  # policies.py:59
        else:
            aspect_ratio = ratio
        w = int(np.round(np.sqrt(target_area * aspect_ratio)))            # policies.py:62
        h = int(np.round(np.sqrt(target_area / aspect_ratio)))
        if 0 < w <= width and 0 < h <= height:
            i = int(rs.uniform(0, height - h + 1))                        # policies.py:65
            j = int(rs.uniform(0, width - w + 1))
            return ((i + h / 2) / height, (j + w / 2) / width), (h, w)
    in_ratio = float(width) / float(height)                               # policies.py:71
    if in_ratio < min(ratio):
        w = width
        h = int(round(w / min(ratio)))
    elif in_ratio > max(ratio):
        h = height
        w = int(round(h * max(ratio)))
    else:
        w, h = width, height
    i, j = (height - h) // 2, (width - w) // 2
    return ((i + h / 2) / height, (j + w / 2) / width), (h, w)


def nearcenter_fixation(rs, height, width, scale, ratio, dist):
    """BaseSaccadePolicy.get_random_nearcenter_fixation (reference policies.py:90-129)."""
    area = height * width
    log_ratio = np.log(ratio)
    target_area = area * rs.uniform(scale[0], scale[1]) if hasattr(scale, "__len__") else area * scale
    aspect_ratio = np.exp(rs.uniform(log_ratio[0], log_ratio[1])) if hasattr(ratio, "__len__") else ratio
    w = int(round(np.sqrt(target_area * aspect_ratio)))                   # policies.py:121
    h = int(round(np.sqrt(target_area / aspect_ratio)))
    cy = rs.uniform(0.5 - dist, 0.5 + dist)                               # policies.py:127
    cx = rs.uniform(0.5 - dist, 0.5 + dist)
    return (cy, cx), (h, w)


def multi_random_fixations(rs, batch, height, width, n_fixations, training, crop_area_range=(0.08, 1),
                           add_aspect_variation=False, val_crop_size=1, nonrandom_first=False, dist=None):
    """The fixations and sizes MultiRandomSaccadePolicy.forward draws (reference
    policies.py:147-164,248-256): float64 ``[B, F, 2]`` centres, int64 ``[B, F, 2]`` sizes."""
    scale = list(crop_area_range) if training else val_crop_size
    ratio = ([3 / 4, 4 / 3] if add_aspect_variation else 1) if training else 1
    locs = np.zeros((batch, n_fixations, 2))
    sizes = np.zeros((batch, n_fixations, 2), np.int64)
    for f in range(n_fixations):
        for b in range(batch):
            if dist is not None:
                loc, size = nearcenter_fixation(rs, height, width, scale, ratio, dist)
            else:
                loc, size = random_crop(rs, height, width, scale, ratio)
            locs[b, f], sizes[b, f] = loc, size
        if f == 0 and nonrandom_first:
            locs[:, 0] = 0.5
    return locs, sizes
