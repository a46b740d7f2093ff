"""Retinal transform, drop-in for the reference ``fovi.sensing.retina.RetinalTransform``.

Argument handling follows the reference (``fovi/sensing/retina.py:31-237``):
``fixation_size`` normalised to a numpy ``[B, 2]`` (h, w) array and
``fix_loc`` to an fp32 ``[B, 2]`` (h, w) tensor, then the grid sampler, the
optional foveal colour decay ``x * exp(-r / sigma)`` and a cast to ``dtype``.
Only the grid samplers ('grid_nn', 'grid_bilinear') are built.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

from .coords import find_desired_res
from .samplers import GaussianKNNGridSampler, GridSampler, KNNGridSampler

__all__ = ["RetinalTransform", "GaussianColorDecay"]


class GaussianColorDecay(nn.Module):
    """``x[b, c, n] * exp(-radius[n] / sigma)``; identity for ``sigma=None`` (reference
    ``retina.py:365-404``).

    Deviation: the reference multiplies the sampled ``[B, C, N]`` by ``decay.unsqueeze(1)``,
    an ``[N, 1]`` tensor, which broadcasts as ``[1, N, 1]`` against the channel axis: it
    raises for 1 < C != N and returns ``[B, N, N]`` for C = 1. Here the decay is applied per
    sensor point, the eccentricity weighting that module describes."""

    def __init__(self, sigma):
        super().__init__()
        self.sigma = sigma

    def forward(self, x, radius):
        if self.sigma is None:
            return x
        return x * torch.exp(-radius.to(x.device) / self.sigma).unsqueeze(0).unsqueeze(0)


class RetinalTransform(nn.Module):
    def __init__(self, resolution, start_res=256, fov=16, cmf_a=0.5, style="isotropic", sampler="grid_nn",
                 fixation_size=None, device="cuda", dtype=torch.float, auto_match_cart_resources=True,
                 pre_transforms=None, post_transforms=None, sigma=None, no_color_val=False,
                 padding_mode="zeros", **kwargs):
        super().__init__()
        self.sigma = sigma
        self.cmf_a = cmf_a
        self.fov = fov
        self.fixation_size = start_res if fixation_size is None else fixation_size
        self.start_res = start_res
        self.device = device
        self.dtype = dtype
        if auto_match_cart_resources != 0 and "fixn" not in style:
            resolution, _ = find_desired_res(fov, cmf_a, resolution ** 2, style=style, force_less_than=True,
                                             quiet=True)
        self.resolution = resolution
        self.mode = f"pointcloud_{style}"
        self.out_size = resolution
        self.reshape_as_grid = "_as_grid" in self.mode
        self.no_color_val = no_color_val
        self.foveal_color = GaussianColorDecay(sigma)
        if sampler == "grid_nn":
            self.sampler = GridSampler(fov, cmf_a, resolution, device=device, mode="nearest", style=style,
                                       padding_mode=padding_mode)
        elif sampler == "grid_bilinear":
            self.sampler = GridSampler(fov, cmf_a, resolution, device=device, mode="bilinear", style=style,
                                       padding_mode=padding_mode)
        elif sampler == "gaussian_pooling":
            self.sampler = GaussianKNNGridSampler(fov, cmf_a, resolution, fixation_size=self.fixation_size,
                                                  device=device, style=style, **kwargs)
        elif sampler == "pooling":
            self.sampler = KNNGridSampler(fov, cmf_a, resolution, fixation_size=self.fixation_size, device=device,
                                          style=style, **kwargs)
        else:
            raise ValueError(f"Invalid sampler: {sampler}")
        self.pre_transforms = pre_transforms
        self.post_transforms = post_transforms
        self.scatter_sizes = self.sampler.coords.get_scatter_sizes().cpu().numpy()

    @torch.autocast(device_type="cuda", enabled=False)
    def forward(self, x, fix_loc, fixation_size=None, **kwargs):
        fixation_size = self._check_fixation_size(fixation_size, x.shape[0])
        fix_loc = self._check_fix_loc(fix_loc, x.shape[0])
        if self.pre_transforms is not None and self.training:
            x = self.pre_transforms(x.clone())
        x = self.sampler(x, fix_loc=fix_loc, fixation_size=fixation_size, **kwargs)
        if self.post_transforms is not None and self.training:
            x = self.post_transforms(x.unsqueeze(3)).clone().squeeze(3)
        return self._finish(x)

    @torch.autocast(device_type="cuda", enabled=False)
    def forward_views(self, x, fix_loc, fixation_size):
        """``forward`` for ``F`` fixations of every image in one sampler launch: ``fix_loc
        [B, F, 2]`` (h, w) in [0, 1], ``fixation_size [B, F, 2]`` (h, w) pixels -> ``[B, F, C, N]``,
        view ``(b, f)`` equal to ``forward(x, fix_loc[:, f], fixation_size[:, f])[b]``. Random
        pre/post transforms are drawn per call, so in training mode they need the per-fixation
        calls: this raises when they are set."""
        if self.training and (self.pre_transforms is not None or self.post_transforms is not None):
            raise ValueError("forward_views: pre/post transforms are drawn per call; call forward per fixation")
        bsz, n_fix = x.shape[0], fix_loc.shape[1]
        if tuple(fix_loc.shape) != (bsz, n_fix, 2):
            raise ValueError(f"fix_loc must be [{bsz}, F, 2]; got {tuple(fix_loc.shape)}")
        loc = torch.as_tensor(fix_loc).to(dtype=self.dtype, device=self.device).reshape(bsz * n_fix, 2)
        size = torch.as_tensor(fixation_size).detach().cpu()
        if tuple(size.shape) != (bsz, n_fix, 2):
            raise ValueError(f"fixation_size must be [{bsz}, {n_fix}, 2]; got {tuple(size.shape)}")
        view_image = torch.arange(bsz).repeat_interleave(n_fix)
        y = self.sampler.sample_views(x, loc, size.reshape(bsz * n_fix, 2).numpy(), view_image=view_image)
        y = self._finish(y)
        return y.reshape(bsz, n_fix, *y.shape[1:])

    def _finish(self, x):
        """Colour decay, eval-mode grayscale, grid reshape and dtype of the sampled ``[V, C, N]``."""
        if self.foveal_color is not None:
            x = self.foveal_color(x, self.sampler.polar_radius)
        if not self.training and self.no_color_val:
            # torchvision's rgb_to_grayscale(num_output_channels=3) of the reference (retina.py:150):
            # 0.2989 R + 0.587 G + 0.114 B in x's dtype, repeated over three channels
            r, g, b = x.unbind(1)
            x = (0.2989 * r + 0.587 * g + 0.114 * b).to(x.dtype).unsqueeze(1).expand(-1, 3, -1).clone()
        if self.reshape_as_grid:
            x = x.reshape(x.shape[0], x.shape[1], self.resolution, self.resolution)
        return x.to(self.dtype)

    def get_warp_params(self):
        return self.fov, self.cmf_a, self.resolution, self.fixation_size

    def _check_fixation_size(self, fixation_size, batch_size):
        """numpy ``[B, 2]`` (h, w) fixation sizes (reference ``retina.py:176-209``)."""
        if fixation_size is None or (isinstance(fixation_size, str) and fixation_size == "none"):
            if hasattr(self.fixation_size, "__len__"):
                fixation_size = np.array(self.fixation_size)
            else:
                fixation_size = np.array([self.fixation_size, self.fixation_size])
        elif isinstance(fixation_size, (int, float)):
            fixation_size = np.array([fixation_size, fixation_size])
        elif isinstance(fixation_size, torch.Tensor):
            fixation_size = fixation_size.cpu().numpy()
        elif hasattr(fixation_size, "__len__") and len(fixation_size) == 2:
            fixation_size = np.array(fixation_size)
        fixation_size = fixation_size.squeeze()
        if len(fixation_size.shape) == 1:
            if fixation_size.shape[0] == 2:
                fixation_size = np.expand_dims(np.array(fixation_size), axis=0).repeat(batch_size, axis=0)
            elif fixation_size.shape[0] == batch_size:
                fixation_size = np.expand_dims(np.array(fixation_size), axis=1).repeat(2, axis=1)
            else:
                raise ValueError(f"fixation_size shape: {fixation_size.shape}")
        else:
            assert fixation_size.shape[0] == batch_size
        return fixation_size

    def _check_fix_loc(self, fix_loc, batch_size):
        """fp32 ``[B, 2]`` (h, w) fixation centres (reference ``retina.py:211-237``)."""
        if fix_loc is None:
            fix_loc = np.array([0.5, 0.5])
        elif isinstance(fix_loc, (float, int)):
            fix_loc = np.array([fix_loc, fix_loc])
        elif isinstance(fix_loc, torch.Tensor):
            fix_loc = fix_loc.cpu().numpy()
        elif isinstance(fix_loc, (list, tuple)):
            fix_loc = np.array(fix_loc)
        if len(fix_loc.squeeze().shape) == 1:
            fix_loc = np.expand_dims(np.array(fix_loc.squeeze()), axis=0).repeat(batch_size, axis=0)
        else:
            assert fix_loc.shape[0] == batch_size
        return torch.tensor(fix_loc, dtype=self.dtype, device=self.device)
