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

The 'isotropic' style (the reference's default) keeps the same radii with
a per-ring angle count that makes neighbouring angles as far apart as
neighbouring rings (``coords.py:345-361``), maps the points onto the 3-D
cortical sensor manifold (``fovi/sensing/manifold.py:14-215,347-375``: the
cortical height is the integral of ``sqrt(M(r)^2 - (d rho/dr)^2)``, a
trapezoid rule on a 1e-4-degree mesh interpolated linearly) and adds the pad
ring beyond the last ring (``coords.py:68-87``). Both keep the reference's
numpy dtype chain: the points enter the manifold in fp64, the pad ring in
fp32, one point at a time in numpy scalars. 'isotropic_fixn' fixes the point
count to ``res**2`` by adding or removing single angles on rings drawn with
numpy's global RNG, by the same calls in the same order (``coords.py:224-258``),
so a seeded run builds the reference's sensor.
"""
from __future__ import annotations

import numpy as np
import torch

__all__ = [
    "SamplingCoords",
    "find_desired_res",
    "num_sampling_coords",
    "logpolar_ring_radii",
    "xy_to_colrow",
    "xy_to_rowcol",
    "auto_match_num_coords",
]

_LOGPOLAR_STYLES = ("logpolar", "logpolar_as_grid")
_ISOTROPIC_STYLES = ("isotropic", "isotropic_fixn")
_UNIFORM_STYLES = ("uniform", "uniform_as_grid")


def logpolar_ring_radii(fov, cmf_a, res):
    """Normalised ring radii (fp32, length ``res``) of the log(r+a) sampling.

    Rings are evenly spaced in cortical radius ``w = log(r + a)`` over
    ``[log a, log(fov/2 + a) + dw]`` with ``res + 1`` samples (the extra sample
    is dropped), mapped back with ``r = exp(w) - a`` and divided by ``fov/2``
    (reference ``coords.py:322-370``; the isotropic angle counts computed there
    are ``isotropic_ring_counts``).
    """
    res = int(res)
    r_max = fov / 2
    w_lo = np.log(cmf_a)
    w_hi = np.log(r_max + cmf_a)
    dw = (w_hi - w_lo) / (res - 1)
    w = torch.linspace(w_lo, w_hi + dw, steps=res + 1)
    r = torch.exp(w) - cmf_a
    return 1 * (r[:-1] / (fov / 2))


def isotropic_ring_counts(fov, cmf_a, res):
    """Angles per ring of the isotropic sampling (``res`` ints): 1 at the centre, then the
    number of steps of the mean neighbouring-ring spacing that fit in the ring's
    circumference, counted by the reference's own ``torch.arange`` call on the fp32 radii
    (reference ``coords.py:345-361``)."""
    res = int(res)
    r_max = fov / 2
    w_lo = np.log(cmf_a)
    w_hi = np.log(r_max + cmf_a)
    dw = (w_hi - w_lo) / (res - 1)
    w = torch.linspace(w_lo, w_hi + dw, steps=res + 1)
    r = torch.exp(w) - cmf_a
    counts = [1]
    for i in range(1, res):
        spacing = ((r[i] - r[i - 1]) + (r[i + 1] - r[i])) / 2
        counts.append(len(torch.arange(0, 2 * torch.pi * r[i], spacing)))
    return counts


def _ring_points(radii, counts):
    """fp64 cartesian and polar point sets, ring-major, ``counts[i]`` angles on ring i.

    Each point is the exact fp32 radius times torch's fp64 cosine and sine of the numpy
    angle, the reference's arithmetic (``coords.py:270-278``); libm's ``math.sin`` differs
    from torch's in the last bit of a few angles, which the fp64 ``cartesian_rowcol`` keeps."""
    rad = torch.cat([torch.full((cnt,), r32, dtype=torch.float64) for r32, cnt in zip(radii.tolist(), counts)])
    ang = torch.cat([torch.from_numpy(np.linspace(0, 2 * np.pi, cnt, endpoint=False)) for cnt in counts])
    cart = torch.stack([rad * torch.cos(ang), rad * torch.sin(ang)], dim=1)
    return cart, torch.stack([rad, ang], dim=1)


def _logpolar_points(fov, cmf_a, res, max_val):
    """fp64 cartesian and polar point sets, ring-major (index = ring*res + angle)."""
    return _ring_points(logpolar_ring_radii(fov, cmf_a, res) * max_val, [res] * res)


def fixn_ring_counts(fov, cmf_a, n_points):
    """(rings, angles per ring) of an isotropic sensor with exactly ``n_points`` points: the
    resolution whose count is nearest, then one angle added to or removed from rings drawn
    by ``np.random.choice`` over the outer 80% of rings (global numpy RNG, the reference's
    calls and order, ``coords.py:224-258``); a ring down to one angle passes its removal
    outwards."""
    res, _ = find_desired_res(fov, cmf_a, n_points, style="isotropic", quiet=True)
    counts = isotropic_ring_counts(fov, cmf_a, res)
    diff = sum(counts) - n_points
    n_rad = len(counts)
    add = -1 if diff > 0 else 1
    if diff != 0:
        rad_idx = []
        rad_min = int(0.2 * n_rad)
        while len(rad_idx) < abs(diff):
            this_diff = min(abs(diff) - len(rad_idx), n_rad - 1)
            draw = np.random.choice(np.arange(rad_min, n_rad), size=min(this_diff, n_rad - rad_min), replace=False)
            rad_idx = np.concatenate([rad_idx, draw])
        rad_idx = rad_idx.astype(int)
        for ii in range(abs(diff)):
            j = rad_idx[ii]
            while counts[j] <= 1 and add < 0:
                j += 1
            counts[j] += add
        if min(counts) <= 0:
            raise AssertionError("some radii have no angles")
    return res, counts


def _isotropic_points(fov, cmf_a, res, max_val, fixn=False):
    if fixn:
        rings, counts = fixn_ring_counts(fov, cmf_a, res ** 2)
    else:
        rings, counts = res, isotropic_ring_counts(fov, cmf_a, res)
    return _ring_points(logpolar_ring_radii(fov, cmf_a, rings) * max_val, counts)


def _isotropic_plotting(cart64, fov, cmf_a):
    """Complex-log plotting coordinates with the hemifields pulled apart (reference
    ``coords.py:281-294``)."""
    fov_xy = cart64 * (fov / 2)
    z = torch.log(torch.abs(fov_xy[:, 0]) + 1j * fov_xy[:, 1] + cmf_a)
    plot = torch.stack([z.real, -z.imag], 1)
    edge = np.log(fov / 2 + cmf_a)
    half_sd = torch.std(plot[:, 0]) * .5
    left = cart64[:, 0] < 0
    plot[left, 0] = half_sd + edge - plot[left, 0]
    plot[~left, 0] = plot[~left, 0] - (half_sd + edge)
    return plot


def _pad_ring(polar, dtype, padding_distance=0.5):
    """Points on rings beyond the last ring, spaced by the outermost ring gap in radius and in
    angle, out to ``padding_distance`` (reference ``coords.py:68-87``).

    ``torch.arange`` with a 0-d tensor step returns the default dtype (fp32 unless changed),
    whatever ``polar``'s dtype, and the reference's ``np.cos(angle)`` of such a 0-d tensor is
    numpy's cosine in that dtype; each coordinate is that cos/sin times the radius, then the
    set is rounded to ``dtype``."""
    radii = torch.sort(torch.unique(polar[:, 0])).values
    gap = radii[-1] - radii[-2]
    start = radii[-1] + gap
    angles = torch.arange(0, 2 * np.pi, gap)
    rings = torch.arange(start, start + padding_distance, gap).to(angles.dtype)
    ang = angles.numpy()
    cos_a = torch.from_numpy(np.array([np.cos(a) for a in ang], dtype=ang.dtype))
    sin_a = torch.from_numpy(np.array([np.sin(a) for a in ang], dtype=ang.dtype))
    ring_t = rings.unsqueeze(1)
    xy = torch.stack([ring_t * cos_a, ring_t * sin_a], dim=2)
    return xy.reshape(-1, 2).to(dtype=dtype)


class _CorticalManifold:
    """Cortical height of the 3-D sensor manifold as a function of eccentricity (degrees),
    for M(r) = k / (r + a) (reference ``manifold.py:32-48,117-137``): the running trapezoid
    integral of ``sqrt(M^2 - (d rho/dr)^2)`` over ``np.arange(0, 2 fov, 1e-4)``,
    interpolated linearly."""

    _cache = {}

    def __init__(self, cmf_a, fov, k=10):
        from scipy.integrate import cumulative_trapezoid
        from scipy.interpolate import interp1d
        self.cmf_a, self.fov, self.k = cmf_a, fov, k
        mesh = np.arange(0, 2 * fov, 0.0001)
        integrand = (self.mag(mesh) ** 2 - self.drho_dr(mesh) ** 2) ** 0.5
        self.height = interp1d(mesh, cumulative_trapezoid(integrand, x=mesh, initial=0), kind="linear")

    @classmethod
    def get(cls, cmf_a, fov, k=10):
        key = (cmf_a, fov, k)
        if key not in cls._cache:
            cls._cache[key] = cls(cmf_a, fov, k)
        return cls._cache[key]

    def mag(self, r):
        return self.k / (self.cmf_a + r)

    def rho(self, r):
        return self.mag(r) * np.sin(np.deg2rad(r)) * (180 / np.pi)

    def drho_dr(self, r):
        dmag = -self.k * ((self.cmf_a + r) ** (-2))
        return dmag * np.sin(np.deg2rad(r)) * (180 / np.pi) + self.mag(r) * np.cos(np.deg2rad(r))

    def to_cortex(self, xy):
        """Visual (x, y) in degrees -> cortical cartesian (x_c, y_c, z), one point at a time in
        numpy scalars of ``xy``'s dtype, z in fp64 (reference ``manifold.py:139-171,202-211``)."""
        out = []
        for x, y in xy:
            r = np.sqrt(x ** 2 + y ** 2)
            theta = np.arctan2(y, x)
            rho = self.rho(r)
            out.append((rho * np.cos(theta), rho * np.sin(theta), self.height(r)))
        return np.array(out)


def sensor_manifold_coords(cartesian, cmf_a, fov, k=10):
    """Cortical cartesian coordinates ``[n, 3]`` (fp64 tensor) of normalised visual points
    ``cartesian`` (numpy, [-1, 1]) on the 3-D sensor manifold (reference
    ``manifold.py:347-375``)."""
    return torch.tensor(_CorticalManifold.get(cmf_a, fov, k).to_cortex(cartesian * (fov / 2)))


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


def num_sampling_coords(fov, cmf_a, res, style="isotropic", device="cpu"):
    """Number of sensor points for ``res`` (reference ``coords.py:567-586``)."""
    if style in _LOGPOLAR_STYLES + _UNIFORM_STYLES + ("isotropic_fixn",):
        return res ** 2
    if style == "isotropic":
        return int(sum(isotropic_ring_counts(fov, cmf_a, res)))
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


def xy_to_rowcol(xy):
    """(x, y) in [-1,1] -> image (row, col) = (-y, x) in [-1,1], the reference's
    ``xy_to_rowcol(coords, do_norm=False, format='-11')`` (``coords.py:522-548``): no
    normalisation, the input's dtype and device."""
    return torch.stack((-xy[:, 1], xy[:, 0]), dim=1)


class SamplingCoords:
    """Sensor point set with cartesian, polar and cortical coordinates.

    Constructor (default style 'isotropic') and attributes follow the reference
    ``SamplingCoords`` (``fovi/sensing/coords.py:10-201``): ``cartesian [N,2]`` in
    [-1,1], ``polar [N,2]`` (radius, angle), ``cortical`` (log-polar: ``[N,2]``
    normalised to [0,1] per column; isotropic: ``[N,3]`` on the cortical manifold;
    uniform: None), ``plotting``, ``cartesian_pad_coords [P,2]`` (the pad ring),
    ``cortical_pad_coords [P,3]`` (isotropic), ``cartesian_rowcol [N,2]`` (image row, col
    = (-y, x) before the cast to ``dtype``), ``shape``, ``resolution``, ``style``.
    Points are ring-major: log-polar index ``ring * res + angle``; isotropic rings
    hold ``isotropic_ring_counts`` points each.
    """

    def __init__(self, fov, cmf_a, res, device="cpu", style="isotropic", dtype=torch.float, max_val=1):
        if isinstance(res, float) and res.is_integer():
            res = int(res)
        self.fov = fov
        self.cmf_a = cmf_a
        self.resolution = res
        self.device = device
        self.style = style
        self.dtype = dtype
        self.max_val = max_val
        # the points are built on the host; a tensor scale (max_out_coord_val='auto') may live
        # on the device, and its fp32 product with the radii is the same IEEE multiply there
        if isinstance(max_val, torch.Tensor):
            max_val = max_val.detach().cpu()
        plotting = None
        if res == 1:
            cart = torch.zeros(1, 2, dtype=torch.float64)
            polar = torch.zeros(1, 2, dtype=torch.float64)
            cortical = torch.zeros(1, 3, dtype=torch.float64)
        elif style in _LOGPOLAR_STYLES:
            cart, polar = _logpolar_points(fov, cmf_a, res, max_val)
            pad = _pad_ring(polar, dtype)
            cortical = _logpolar_cortical(cart, polar, fov, cmf_a)
        elif style in _UNIFORM_STYLES:
            cart, polar = _uniform_points(res, max_val)
            pad = _pad_ring(polar, dtype)
            cortical = None
        elif style in _ISOTROPIC_STYLES:
            cart, polar = _isotropic_points(fov, cmf_a, res, max_val, fixn=style == "isotropic_fixn")
            plotting = _isotropic_plotting(cart, fov, cmf_a)
            pad = _pad_ring(polar, dtype)
            cortical = sensor_manifold_coords(cart.numpy(), cmf_a, fov)
            self.cortical_pad_coords = sensor_manifold_coords(pad.numpy(), cmf_a, fov).to(
                device=device, dtype=dtype)
        else:
            raise ValueError(f"Style {style} not recognized")
        if res != 1:
            # image (row, col) of the points before the cast to ``dtype`` (fp64 for the ring
            # styles, fp32 for 'uniform'), as the reference sets it (``coords.py:41-42``); the
            # DINOv3 adapter's RoPE reads it (``dinov3.py:97``). A one-point sensor has none.
            self.cartesian_rowcol = xy_to_rowcol(cart).to(device=device)
        self.cartesian = cart.to(device=device, dtype=dtype)
        self.polar = polar.to(device=device, dtype=dtype)
        self.cortical = None if cortical is None else cortical.to(device=device, dtype=dtype)
        if plotting is not None:
            self.plotting = plotting.to(device=device, dtype=dtype)
        else:
            self.plotting = self.cortical if self.cortical is not None else self.cartesian
        # the pad ring beyond the outermost ring (none for a one-point sensor); only the
        # isotropic manifold and the visual-field neighbour searches reach it
        self.cartesian_pad_coords = (pad if res != 1 else torch.zeros(0, 2, dtype=dtype)).to(device=device)
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
