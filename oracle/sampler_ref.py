"""Oracle of the foveated sampler (test infrastructure only, see oracle/__init__.py)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def grid_from_cartesian(cartesian):
    """``[1, 1, N, 2]`` grid_sample grid of ``[N, 2]`` sensor points (x, y): column = x,
    row = -y (reference ``BaseGridSampler._prep_grid_for_grid_sample``,
    fovi/sensing/samplers.py:35-47, via ``xy_to_colrow(..., do_norm=False, format='-11')``,
    fovi/sensing/coords.py:530-564)."""
    cartesian = torch.as_tensor(cartesian)
    return torch.stack((cartesian[:, 0], -cartesian[:, 1]), dim=1)[None, None]


def transform_sampling_grid(sampling_grid, fix_loc, fixation_size, image_size):
    """Fixation transform of a (1,1,N,2) (x,-y) grid (reference fovi/sensing/coords.py:590-642).

    Element-wise fp32 torch ops in the reference's order: centre *= size,
    grid *= size/2, grid += centre, grid = 2*grid/size - 1.
    """
    fix_loc = torch.as_tensor(fix_loc).clone()
    if fix_loc.ndim == 1:
        fix_loc = fix_loc.unsqueeze(0)
    fixation_size = torch.as_tensor(fixation_size).clone()
    if fixation_size.ndim == 1:
        fixation_size = fixation_size.unsqueeze(0)
    ch = fix_loc[:, 0].reshape(-1, 1, 1)
    cw = fix_loc[:, 1].reshape(-1, 1, 1)
    fh = fixation_size[:, 0].reshape(-1, 1, 1)
    fw = fixation_size[:, 1].reshape(-1, 1, 1)
    H, W = image_size
    cw *= W
    ch *= H
    g = sampling_grid.clone()
    if g.shape[0] == 1:
        g = g.repeat(ch.shape[0], 1, 1, 1)
    g[:, :, :, 0] *= (fw / 2)
    g[:, :, :, 1] *= (fh / 2)
    g[:, :, :, 0] += cw
    g[:, :, :, 1] += ch
    g[:, :, :, 0] = (2 * g[:, :, :, 0] / W) - 1
    g[:, :, :, 1] = (2 * g[:, :, :, 1] / H) - 1
    return g


def grid_sample_views(img, grid, mode="bilinear", padding_mode="zeros"):
    """``F.grid_sample(img, grid, mode, align_corners=False).squeeze(2)`` -> [B, C, N]
    (reference fovi/sensing/samplers.py:108), on CPU in fp32."""
    return F.grid_sample(img.float(), grid.float(), mode=mode, padding_mode=padding_mode,
                         align_corners=False).squeeze(2)


def sampler_forward(img, sampling_grid, fix_loc, fixation_size, mode="bilinear", padding_mode="zeros"):
    """GridSampler.forward restated (reference samplers.py:91-112). Returns (out, grid)."""
    g = transform_sampling_grid(sampling_grid, fix_loc, fixation_size, img.shape[-2:])
    return grid_sample_views(img, g, mode, padding_mode), g


def bilinear_numpy(img, gx, gy, mode="bilinear", padding_mode="zeros"):
    """Textbook grid sampling of one [C,H,W] image at normalised points (float64).

    align_corners=False: pixel i covers [i, i+1) in the unnormalised frame,
    so the sample position is ((g + 1) * size - 1) / 2.
    """
    img = np.asarray(img, dtype=np.float64)
    C, H, W = img.shape
    out = np.zeros((C, len(gx)))
    for p, (x, y) in enumerate(zip(np.asarray(gx, np.float64), np.asarray(gy, np.float64))):
        ix = ((x + 1) * W - 1) / 2
        iy = ((y + 1) * H - 1) / 2
        if padding_mode == "border":
            ix = min(max(ix, 0), W - 1)
            iy = min(max(iy, 0), H - 1)
        if mode == "nearest":
            xi, yi = int(np.rint(ix)), int(np.rint(iy))
            if 0 <= xi < W and 0 <= yi < H:
                out[:, p] = img[:, yi, xi]
            continue
        x0, y0 = int(np.floor(ix)), int(np.floor(iy))
        for yy, wy in ((y0, 1 - (iy - y0)), (y0 + 1, iy - y0)):
            for xx, wx in ((x0, 1 - (ix - x0)), (x0 + 1, ix - x0)):
                if 0 <= xx < W and 0 <= yy < H:
                    out[:, p] += wy * wx * img[:, yy, xx]
    return out
