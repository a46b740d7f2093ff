"""Foveated grid sampler, drop-in for the reference ``fovi.sensing.samplers.GridSampler``.

``GridSampler.forward(img, fix_loc, fixation_size)`` has the reference's
signature and result (``fovi/sensing/samplers.py:51-130``): the fixation
transform of ``transform_sampling_grid`` (``fovi/sensing/coords.py:590-642``)
and ``grid_sample(..., align_corners=False)`` with zeros padding, here one HIP
launch (``fovi_sampler_fwd``) for the whole batch.

``GridSampler.sample_views`` additionally samples many fixation views of the
same images in one launch (view ``v`` reads image ``view_image[v]``), the
fused form of the per-fixation loop of ``fovi/sensing/policies.py:268-270``.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

from .. import _lib
from .coords import SamplingCoords, xy_to_colrow

__all__ = ["BaseGridSampler", "GridSampler", "KNNGridSampler", "GaussianKNNGridSampler", "fixation_half_sizes"]

_MODES = {"nearest": _lib.NEAREST, "bilinear": _lib.BILINEAR}
_PADS = {"zeros": _lib.PAD_ZEROS, "border": _lib.PAD_BORDER}


def fixation_half_sizes(fixation_size, n):
    """``(half [n,2] float64, wide)`` for the kernel's ``fix_size / 2`` factor.

    The reference divides the fixation-size tensor by 2 (``coords.py:632-633``):
    an integer or fp32 size gives an fp32 half size and an fp32 multiply
    (``wide = 0``); an fp64 size gives an fp64 half size, so the multiply runs
    in fp64 before the result is stored as fp32 (``wide = 1``).
    """
    fs = fixation_size
    if isinstance(fs, (tuple, list, np.ndarray)):
        fs = torch.tensor(np.asarray(fs))
    fs = torch.as_tensor(fs).detach().cpu()
    if fs.ndim == 1:
        fs = fs.unsqueeze(0)
    if fs.shape[0] == 1 and n > 1:
        fs = fs.expand(n, 2)
    if fs.shape != (n, 2):
        raise ValueError(f"fixation_size must be [{n}, 2] (h, w); got {tuple(fs.shape)}")
    if not bool(torch.isfinite(fs.to(torch.float64)).all()):
        raise ValueError("fixation_size must be finite")
    half = fs / 2
    wide = half.dtype == torch.float64
    return half.to(torch.float64).contiguous(), int(wide)


class _Views:
    """Device-resident fixation tables of one set of views."""

    def __init__(self, fix_loc, half, wide, view_image, n_views, n_img):
        self.fix_loc, self.half, self.wide = fix_loc, half, wide
        self.view_image, self.n_views, self.n_img = view_image, n_views, n_img


class BaseGridSampler(nn.Module):
    """Grid preparation shared by samplers (reference ``samplers.py:13-47``)."""

    def _prep_grid_for_grid_sample(self, cartesian_grid):
        """(n,2) (x, y) -> (1,1,n,2) (x, -y) grid_sample order."""
        return xy_to_colrow(cartesian_grid.clone()).unsqueeze(0).unsqueeze(0)


class GridSampler(BaseGridSampler):
    """Samples images at (fixation-shifted) sensor points with one HIP launch."""

    def __init__(self, fov, cmf_a, resolution, device="cuda", dtype=torch.float, mode="nearest",
                 style="isotropic", coords=None, padding_mode="zeros"):
        super().__init__()
        if mode not in _MODES:
            raise ValueError(f"mode must be one of {list(_MODES)}; got {mode!r}")
        if padding_mode not in _PADS:
            raise ValueError(f"padding_mode must be one of {list(_PADS)}; got {padding_mode!r}")
        self.fov = fov
        self.cmf_a = cmf_a
        self.resolution = resolution
        self.ring_order = True
        self.device = device
        self.dtype = dtype
        self.mode = mode
        self.style = style
        self.padding_mode = padding_mode
        self.coords = SamplingCoords(fov, cmf_a, resolution, device=device, style=style, dtype=dtype) \
            if coords is None else coords
        self.sampling_grid = self._prep_grid_for_grid_sample(self.coords.cartesian)
        self.out_sampling_grid = self.sampling_grid
        self.polar_radius = self.coords.polar[:, 0]
        self._grid_dev = None

    def _grid(self, device):
        g = self._grid_dev
        if g is None or g.device != device:
            g = self.sampling_grid.reshape(-1, 2).to(device=device, dtype=torch.float32).contiguous()
            self._grid_dev = g
        return g

    def prepare_views(self, fix_loc, fixation_size, n_img, device, view_image=None):
        """Device tables of a set of fixation views, reusable across calls.

        ``fix_loc [V, 2]`` (h, w) in [0, 1]; ``fixation_size [V, 2]`` (h, w)
        pixels; ``view_image [V]`` image index per view (default: view v
        reads image v).
        """
        fix_loc = torch.as_tensor(fix_loc, dtype=torch.float32).reshape(-1, 2)
        # non-finite centres or sizes would put taps at undefined pixel coordinates
        if not bool(torch.isfinite(fix_loc).all()):
            raise ValueError("fix_loc must be finite")
        fix_loc = fix_loc.to(device).contiguous()
        n_views = fix_loc.shape[0]
        half, wide = fixation_half_sizes(fixation_size, n_views)
        vmap = None
        if view_image is not None:
            vi = torch.as_tensor(view_image).reshape(-1)
            if vi.numel() != n_views:
                raise ValueError("view_image must have one entry per view")
            if int(vi.min()) < 0 or int(vi.max()) >= n_img:
                raise ValueError(f"view_image entries must be in [0, {n_img})")
            vmap = vi.to(device=device, dtype=torch.int32).contiguous()
        elif n_views > n_img:
            raise ValueError(f"{n_views} views of {n_img} images need a view_image map")
        return _Views(fix_loc, half.to(device), wide, vmap, n_views, n_img)

    def sample_views(self, img, fix_loc=None, fixation_size=None, view_image=None, out=None, out_dtype=None,
                     return_grid=False, views=None):
        """Samples ``V`` views in one launch; returns ``out [V, C, N]``.

        Views come from ``views`` (see ``prepare_views``) or from
        ``fix_loc``/``fixation_size``/``view_image``. ``out`` may be any
        strided ``[V, C, N]`` tensor (e.g. a channels-last view).
        """
        _lib.require_device(img)
        if img.dim() != 4:
            raise ValueError(f"img must be [B, C, H, W]; got {tuple(img.shape)}")
        n_img, ch, hh, ww = img.shape
        dev = img.device
        if views is None:
            views = self.prepare_views(fix_loc, fixation_size, n_img, dev, view_image)
        elif views.n_img > n_img:
            raise ValueError(f"views were prepared for {views.n_img} images, got {n_img}")
        n_views = views.n_views
        grid = self._grid(dev)
        n_pts = grid.shape[0]
        odt = out_dtype or (img.dtype if img.dtype in (torch.float32, torch.bfloat16) else torch.float32)
        if out is None:
            out = torch.empty(n_views, ch, n_pts, dtype=odt, device=dev)
        if tuple(out.shape) != (n_views, ch, n_pts):
            raise ValueError(f"out must be [{n_views}, {ch}, {n_pts}]; got {tuple(out.shape)}")
        g_out = torch.empty(n_views, n_pts, 2, dtype=torch.float32, device=dev) if return_grid else None
        a = _lib.SamplerArgs()
        a.img = img.data_ptr(); a.img_dtype = _lib.dtype_code(img.dtype)
        a.n_img, a.channels, a.height, a.width = n_img, ch, hh, ww
        a.img_stride[:] = list(img.stride())
        a.grid = grid.data_ptr(); a.n_points = n_pts; a.n_views = n_views
        a.fix_loc = views.fix_loc.data_ptr(); a.fix_half = views.half.data_ptr(); a.fix_half_wide = views.wide
        a.view_image = None if views.view_image is None else views.view_image.data_ptr()
        a.mode = _MODES[self.mode]; a.padding = _PADS[self.padding_mode]
        a.out = out.data_ptr(); a.out_dtype = _lib.dtype_code(out.dtype)
        a.out_stride[:] = list(out.stride())
        a.grid_out = None if g_out is None else g_out.data_ptr()
        # ring-major grids (index = ring * res + angle) are sampled in 8-ring x 32-angle blocks;
        # the order changes no result (ring_order=False samples point by point)
        res = getattr(self.coords, "resolution", 0)
        res = int(res) if isinstance(res, (int, float)) else 0
        a.ring_len = res if self.ring_order and res > 0 and res * res == n_pts else 0
        lib = _lib.load()
        _lib.check(lib.fovi_sampler_fwd(a, _lib.stream_handle(dev)), "fovi_sampler_fwd")
        return (out, g_out) if return_grid else out

    def forward(self, img, fix_loc=None, fixation_size=None, return_coords=False):
        """``[B, C, N]`` samples (reference ``samplers.py:91-112``)."""
        n = img.shape[0]
        if fix_loc is None:
            fix_loc = torch.full((n, 2), 0.5)
        if fixation_size is None:
            fixation_size = np.array([[img.shape[-2], img.shape[-1]]] * n)
        res = self.sample_views(img, fix_loc, fixation_size, return_grid=return_coords)
        if return_coords:
            out, g = res
            return out, g.unsqueeze(1)
        return res

    def all_coords(self, device=None):
        return self.coords.cartesian.to(device or self.device)

    def __repr__(self):
        return (f"GridSampler(fov={self.fov}, cmf_a={self.cmf_a}, style={self.style}, "
                f"resolution={self.resolution}, mode={self.mode}, n={len(self.coords)})")


class KNNGridSampler(BaseGridSampler):
    """Two-layer foveated sampler (reference ``samplers.py:134-230``): nearest samples on a
    denser "photoreceptor" grid (``res_mult`` x the resolution, ``cmf_a_mult`` x a), then kNN
    average pooling onto the sensor grid. Both stages are HIP launches: the sampler kernel on
    the dense grid and ``fovi_knnpool_fwd``."""

    pool_mode = "avg"

    def __init__(self, fov, cmf_a, resolution, res_mult=3, cmf_a_mult=1, fixation_size=3000, k=None,
                 style="isotropic", sample_cortex=True, dtype=torch.float, device="cuda"):
        super().__init__()
        from ..arch.knn import KNNPoolingLayer
        self.highres_coords = SamplingCoords(fov, cmf_a_mult * cmf_a, res_mult * resolution, device=device,
                                             style=style, dtype=dtype)
        self.coords = SamplingCoords(fov, cmf_a, resolution, device=device, style=style, dtype=dtype)
        if k is None:
            # the ratio of the numbers of points of the two grids (samplers.py:164-166)
            k = int(np.round(len(self.highres_coords) / len(self.coords)))
            print(f"auto-set knngridsampler k={k}")
        self.pooler = KNNPoolingLayer(k, self.highres_coords, self.coords, mode=self.pool_mode, device=device,
                                      sample_cortex=sample_cortex)
        self.sampling_grid = self._prep_grid_for_grid_sample(self.highres_coords.cartesian)
        self.out_sampling_grid = self._prep_grid_for_grid_sample(self.coords.cartesian)
        self.polar_radius = self.coords.polar[:, 0]
        self.fov = fov
        self.cmf_a = cmf_a
        self.resolution = resolution
        self.fixation_size = fixation_size
        self.k = k
        self.dtype = dtype
        self.device = device
        self.style = style
        self.num_coords = len(self.coords)
        self.sample_cortex = sample_cortex
        self.rf_sizes = self.coords.get_scatter_sizes()
        # the dense first layer: nearest samples, zeros padding (the reference's grid_sample call)
        self._dense = GridSampler(fov, cmf_a_mult * cmf_a, res_mult * resolution, device=device, dtype=dtype,
                                  mode="nearest", style=style, coords=self.highres_coords)

    def forward(self, img, fix_loc=None, fixation_size=None):
        """``[B, C, H, W]`` images -> ``[B, C, N]`` pooled samples (reference samplers.py:187-209)."""
        img = img.to(self.device).to(self.dtype)
        dense = self._dense(img, fix_loc=fix_loc, fixation_size=fixation_size)
        return self.pooler(dense)

    def sample_views(self, img, fix_loc=None, fixation_size=None, view_image=None):
        """``[V, C, N]`` pooled samples of ``V`` views (view ``v`` reads image ``view_image[v]``):
        one dense sampler launch for all views, then the pooling."""
        img = img.to(self.device).to(self.dtype)
        return self.pooler(self._dense.sample_views(img, fix_loc, fixation_size, view_image=view_image))

    def all_coords(self, device=None):
        if device is None:
            return self.coords.cartesian, self.coords.polar, self.coords.plotting
        return self.coords.cartesian.to(device), self.coords.polar.to(device), self.coords.plotting.to(device)

    def __repr__(self):
        return (f"KNNGridSampler(fov={self.fov}, cmf_a={self.cmf_a}, resolution={self.resolution}, "
                f"num_coords={self.num_coords}, fixation_size={self.fixation_size}, k={self.k}, "
                f"dtype={self.dtype}, device={self.device}, style={self.style})")


class GaussianKNNGridSampler(KNNGridSampler):
    """``KNNGridSampler`` with Gaussian-weighted pooling (reference ``samplers.py:233-259``)."""

    pool_mode = "gaussian"
