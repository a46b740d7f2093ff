"""Sensor geometry on the host: log-polar and uniform sensor point sets.

This is the setup side of the foveated sampler and of the kNN-conv tables.
It runs once per layer on the host CPU with torch/numpy, and its results are
uploaded to HBM as small tables. Values must equal the reference's bit for
bit, so each step keeps the reference's dtype chain:

* ring radii in fp32 (``torch.linspace`` default dtype) then ``exp(w) - a``
  (reference ``fovi/sensing/coords.py:345-368``);
* cartesian points as ``float64(r_fp32) * cos/sin(angle_fp64)``, because the
  reference multiplies a 0-dim fp32 tensor by a 0-dim fp64 tensor, which
  promotes to fp64 (``coords.py:270-275``), cast to fp32 at the end
  (``coords.py:61-65``);
* log-polar cortical coords ``(log(r+a)-log a)/(log(fov/2+a)-log a)``
  computed in fp64 from the fp64 cartesian points, with the two ``log a``
  terms evaluated on a 0-dim fp32 tensor (``coords.py:46-53``), then per-column
  min-max normalisation (``fovi/utils/__init__.py:126-167``).

Only the 'logpolar' and 'uniform' styles are built (every benchmark
configuration is log-polar). 'isotropic' needs the 3-D cortical manifold and
raises ``NotImplementedError``.
"""
from __future__ import annotations

import math

import numpy as np
import torch

__all__ = [
    "SamplingCoords",
    "find_desired_res",
    "num_sampling_coords",
    "logpolar_ring_radii",
    "xy_to_colrow",
    "auto_match_num_coords",
]

_LOGPOLAR_STYLES = ("logpolar", "logpolar_as_grid")
_UNIFORM_STYLES = ("uniform", "uniform_as_grid")


def logpolar_ring_radii(fov, cmf_a, res):
    """Normalised ring radii (fp32, length ``res``) of the log(r+a) sampling.

    Rings are evenly spaced in cortical radius ``w = log(r + a)`` over
    ``[log a, log(fov/2 + a) + dw]`` with ``res + 1`` samples (the extra sample
    is dropped), mapped back with ``r = exp(w) - a`` and divided by ``fov/2``
    (reference ``coords.py:322-370``; the isotropic angle counts computed there
    are discarded by the log-polar style and are not evaluated here).
    """
    res = int(res)
    r_max = fov / 2
    w_lo = np.log(cmf_a)
    w_hi = np.log(r_max + cmf_a)
    dw = (w_hi - w_lo) / (res - 1)
    w = torch.linspace(w_lo, w_hi + dw, steps=res + 1)
    r = torch.exp(w) - cmf_a
    return 1 * (r[:-1] / (fov / 2))


def _logpolar_points(fov, cmf_a, res, max_val):
    """fp64 cartesian and polar point sets, ring-major (index = ring*res + angle)."""
    radii = logpolar_ring_radii(fov, cmf_a, res) * max_val
    angles = np.linspace(0, 2 * np.pi, res, endpoint=False)
    n = res * res
    cart = np.empty((n, 2), dtype=np.float64)
    polar = np.empty((n, 2), dtype=np.float64)
    cos_a = [math.cos(a) for a in angles]
    sin_a = [math.sin(a) for a in angles]
    for i, r32 in enumerate(radii.tolist()):
        # r32 is the exact fp32 radius widened to a Python float (IEEE double)
        row = slice(i * res, (i + 1) * res)
        cart[row, 0] = [r32 * c for c in cos_a]
        cart[row, 1] = [r32 * s for s in sin_a]
        polar[row, 0] = r32
        polar[row, 1] = angles
    return torch.from_numpy(cart), torch.from_numpy(polar)


def _minmax_columns(x):
    lo = x.min(0).values.unsqueeze(0)
    hi = x.max(0).values.unsqueeze(0)
    return (x - lo) / (hi - lo)


def _logpolar_cortical(cart64, polar64, fov, cmf_a):
    cortical = polar64.clone()
    radius = ((cart64[:, 0] ** 2 + cart64[:, 1] ** 2) ** .5) * fov / 2
    a32 = torch.tensor(cmf_a)
    cortical[:, 0] = (torch.log(radius + cmf_a) - torch.log(a32)) / (
        torch.log(fov / 2 + a32) - torch.log(a32))
    return _minmax_columns(cortical)


def _uniform_points(res, max_val):
    lin = torch.linspace(-max_val, max_val, res)
    cart = torch.stack(torch.meshgrid(lin, lin, indexing="ij"), dim=2).reshape(-1, 2)
    polar = torch.stack([torch.sqrt(cart[:, 0] ** 2 + cart[:, 1] ** 2),
                         torch.arctan2(cart[:, 1], cart[:, 0])], dim=1)
    return cart, polar


def num_sampling_coords(fov, cmf_a, res, style="logpolar", device="cpu"):
    """Number of sensor points for ``res`` (reference ``coords.py:567-586``)."""
    if style in _LOGPOLAR_STYLES + _UNIFORM_STYLES + ("isotropic_fixn",):
        return res ** 2
    if style == "isotropic":
        raise NotImplementedError("isotropic point counts need the cortical manifold")
    raise ValueError(f"Style {style} not recognized")


def find_desired_res(fov, cmf_a, n_points_desired, style, device="cpu", bounds=(1, 1000),
                     force_less_than=False, quiet=False):
    """Resolution whose point count is closest to ``n_points_desired``.

    Binary search over a monotone count, then a walk down (``force_less_than``)
    or up until the count is on the requested side (reference
    ``coords.py:393-447``).
    """
    best_res, best_diff = None, float("inf")
    lo, hi = bounds
    while lo <= hi:
        mid = (lo + hi) // 2
        n = num_sampling_coords(fov, cmf_a, mid, style=style)
        if abs(n - n_points_desired) < best_diff:
            best_diff, best_res = abs(n - n_points_desired), mid
        if n < n_points_desired:
            lo = mid + 1
        else:
            hi = mid - 1
    n = num_sampling_coords(fov, cmf_a, best_res, style=style)
    if force_less_than:
        while n > n_points_desired:
            best_res -= 1
            n = num_sampling_coords(fov, cmf_a, best_res, style=style)
    else:
        while n < n_points_desired:
            best_res += 1
            n = num_sampling_coords(fov, cmf_a, best_res, style=style)
    if not quiet:
        print(f"found resolution {best_res} giving {n} points (desired: {n_points_desired})")
    return best_res, n


def auto_match_num_coords(fov, cmf_a, cart_res, style, auto_match_cart_resources, device="cpu",
                          force_less_than=True, quiet=False):
    """(in_res, cart_res) matched to a cartesian grid (reference ``coords.py:645-670``)."""
    if "fixn" in style or auto_match_cart_resources == 0:
        return cart_res, cart_res
    in_res, _ = find_desired_res(fov, cmf_a, cart_res ** 2, style, device=device,
                                 force_less_than=force_less_than, quiet=quiet)
    return in_res, cart_res


def xy_to_colrow(xy):
    """(x, y) in [-1,1] -> grid_sample (col, row) = (x, -y) (reference ``coords.py:521-564``)."""
    return torch.stack((xy[:, 0], -xy[:, 1]), dim=1)


class SamplingCoords:
    """Sensor point set with cartesian, polar and cortical coordinates.

    Constructor and attributes follow the reference ``SamplingCoords``
    (``fovi/sensing/coords.py:10-201``): ``cartesian [N,2]`` in [-1,1],
    ``polar [N,2]`` (radius, angle), ``cortical [N,2]`` normalised to [0,1]
    per column, ``shape``, ``resolution``, ``style``. Points are ring-major:
    index ``ring * res + angle``.
    """

    def __init__(self, fov, cmf_a, res, device="cpu", style="logpolar", dtype=torch.float, max_val=1):
        if isinstance(res, float) and res.is_integer():
            res = int(res)
        self.fov = fov
        self.cmf_a = cmf_a
        self.resolution = res
        self.device = device
        self.style = style
        self.dtype = dtype
        self.max_val = max_val
        if res == 1:
            cart = torch.zeros(1, 2, dtype=torch.float64)
            polar = torch.zeros(1, 2, dtype=torch.float64)
            cortical = torch.zeros(1, 3, dtype=torch.float64)
        elif style in _LOGPOLAR_STYLES:
            cart, polar = _logpolar_points(fov, cmf_a, res, max_val)
            cortical = _logpolar_cortical(cart, polar, fov, cmf_a)
        elif style in _UNIFORM_STYLES:
            cart, polar = _uniform_points(res, max_val)
            cortical = None
        else:
            raise NotImplementedError(
                f"style {style!r}: only 'logpolar' and 'uniform' sensor geometries are built")
        self.cartesian = cart.to(device=device, dtype=dtype)
        self.polar = polar.to(device=device, dtype=dtype)
        self.cortical = None if cortical is None else cortical.to(device=device, dtype=dtype)
        self.plotting = self.cortical if self.cortical is not None else self.cartesian
        # log-polar styles add no pad points (the reference's pad ring is only
        # reachable through the isotropic/cartesian distance paths)
        self.cartesian_pad_coords = torch.zeros(0, 2, dtype=dtype, device=device)
        self.shape = self.cartesian.shape

    def get_strided_coords(self, stride, auto_match_cart_resources=0, in_cart_res=None,
                           force_less_than=True, max_val=1):
        """A new, coarser point set of the same style (reference ``coords.py:89-131``).

        The output set is regenerated at ``res // stride`` (or matched to
        ``(in_cart_res // stride)**2`` points); it is not a subset of the input.
        """
        out_cart_res = None
        if "fixn" in self.style:
            assert in_cart_res is not None, "in_cart_res must be provided if using fixn style"
            out_radii = in_cart_res // stride
            out_cart_res = in_cart_res // stride
        elif auto_match_cart_resources > 0 and in_cart_res is not None:
            out_cart_res = in_cart_res // stride
            out_radii, _ = find_desired_res(self.fov, self.cmf_a, out_cart_res ** 2, style=self.style,
                                            force_less_than=force_less_than, quiet=True)
        else:
            out_radii = self.resolution // stride
        if out_radii < 1:
            raise ValueError(f"Out radii decreased to less than 1: {out_radii}")
        out = SamplingCoords(self.fov, self.cmf_a, out_radii, self.device, self.style, self.dtype,
                             max_val=max_val)
        return out, out_radii, out_cart_res

    def to(self, device=None, dtype=None):
        dtype = self.dtype if dtype is None else dtype
        device = self.device if device is None else device
        self.device, self.dtype = device, dtype
        self.cartesian = self.cartesian.to(device=device, dtype=dtype)
        if self.cortical is not None:
            self.cortical = self.cortical.to(device=device, dtype=dtype)
        self.polar = self.polar.to(device=device, dtype=dtype)
        self.plotting = self.plotting.to(device=device, dtype=dtype)
        return self

    def get_scatter_sizes(self):
        """Plotting sizes ``radius * fov / res`` (reference ``coords.py:153-167``)."""
        return self.polar[:, 0] * self.fov / self.resolution

    def clone(self, **kw):
        args = dict(fov=self.fov, cmf_a=self.cmf_a, res=self.resolution, device=self.device,
                    style=self.style, dtype=self.dtype, max_val=self.max_val)
        args.update({("res" if k == "resolution" else k): v for k, v in kw.items() if v is not None})
        return SamplingCoords(**args)

    def __len__(self):
        return self.cartesian.shape[0]

    def __repr__(self):
        return (f"SamplingCoords(length={len(self)}, fov={self.fov}, cmf_a={self.cmf_a}, "
                f"resolution={self.resolution}, style={self.style})")
