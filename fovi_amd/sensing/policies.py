"""Fixation (saccade) policies, drop-in for the reference ``fovi.sensing.policies``.

``MultiRandomSaccadePolicy`` draws ``F`` fixations per image on the host with
numpy's global generator, in the reference's draw order (``policies.py:36-164``),
so a run seeded with ``np.random.seed`` gets the reference's fixations and
fixation sizes. It then samples all ``B * F`` views in one launch of the
sampler kernel (``RetinalTransform.forward_views``: view ``b * F + f`` reads
image ``b``) instead of the reference's ``F`` calls of the retinal transform
(``policies.py:266-273``). Per-call random pre/post transforms (training mode)
keep the per-fixation calls, as their draws are per call.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn

__all__ = ["BaseSaccadePolicy", "MultiRandomSaccadePolicy", "NoSaccadePolicy", "PolicyRegistry",
           "FIXATION_POLICY_REGISTRY"]


class BaseSaccadePolicy(nn.Module):
    """Fixation sampling shared by the policies (reference ``policies.py:13-164``)."""

    def __init__(self, retinal_transform, n_fixations):
        super().__init__()
        self.retinal_transform = retinal_transform
        self.n_fixations = n_fixations
        self.fixation_size = retinal_transform.fixation_size
        self.dtype = retinal_transform.dtype
        self.device = retinal_transform.device

    def get_random_crop(self, height, width, scale, ratio):
        """A random crop of area ``scale`` x the image and aspect ``ratio`` (each a value or a
        range): up to 10 draws of (area, log-aspect) until the crop fits, then its top-left
        corner uniformly; otherwise the centred crop clamped to the ratio range
        (reference ``policies.py:36-88``). Returns ``([cy, cx] normalised, [h, w])``."""
        area = height * width
        log_ratio = np.log(ratio)
        for _ in range(10):
            target_area = area * (np.random.uniform(scale[0], scale[1]) if hasattr(scale, "__len__") else scale)
            aspect = np.exp(np.random.uniform(log_ratio[0], log_ratio[1])) if hasattr(ratio, "__len__") else ratio
            w = int(np.round(np.sqrt(target_area * aspect)))
            h = int(np.round(np.sqrt(target_area / aspect)))
            if 0 < w <= width and 0 < h <= height:
                top = int(np.random.uniform(0, height - h + 1))
                left = int(np.random.uniform(0, width - w + 1))
                return [(top + h / 2) / height, (left + w / 2) / width], [h, w]
        in_ratio = float(width) / float(height)
        if in_ratio < min(ratio):
            w = width
            h = int(round(w / min(ratio)))
        elif in_ratio > max(ratio):
            h = height
            w = int(round(h * max(ratio)))
        else:
            w, h = width, height
        top, left = (height - h) // 2, (width - w) // 2
        return [(top + h / 2) / height, (left + w / 2) / width], [h, w]

    def get_random_nearcenter_fixation(self, height, width, scale, ratio, normalized_dist_from_center):
        """Fixation size from one (area, log-aspect) draw, then a centre uniform in
        ``[0.5 - d, 0.5 + d]`` per axis, y first (reference ``policies.py:90-129``)."""
        area = height * width
        log_ratio = np.log(ratio)
        target_area = area * (np.random.uniform(scale[0], scale[1]) if hasattr(scale, "__len__") else scale)
        aspect = np.exp(np.random.uniform(log_ratio[0], log_ratio[1])) if hasattr(ratio, "__len__") else ratio
        if isinstance(target_area, torch.Tensor):
            target_area = target_area.item()
        w = int(round(np.sqrt(target_area * aspect)))
        h = int(round(np.sqrt(target_area / aspect)))
        lo, hi = 0.5 - normalized_dist_from_center, 0.5 + normalized_dist_from_center
        cy = float(np.random.uniform(lo, hi))
        cx = float(np.random.uniform(lo, hi))
        return [cy, cx], [h, w]

    def sample_fixations(self, img_size, n=1, area_range=None, ratio=None, norm_dist_from_center=None):
        """``n`` fixations: ``(fix_loc [n, 2] in the transform's dtype on its device,
        fixation_size [n, 2] int64)`` (reference ``policies.py:131-164``)."""
        if area_range is None:
            area_range = self.crop_area_range if self.training else self.val_crop_size
        if ratio is None:
            ratio = self.crop_aspect_range if self.training else 1
        if norm_dist_from_center is not None:
            return self._nearcenter_batch(img_size[0], img_size[1], n, area_range, ratio, norm_dist_from_center)
        locs, sizes = [], []
        for _ in range(n):
            loc, size = self.get_random_crop(img_size[0], img_size[1], scale=area_range, ratio=ratio)
            locs.append(loc)
            sizes.append(size)
        return torch.tensor(locs, dtype=self.dtype, device=self.device), torch.tensor(sizes)

    def _nearcenter_batch(self, height, width, n, scale, ratio, dist):
        """``n`` calls of ``get_random_nearcenter_fixation`` as one draw of the same uniforms:
        the legacy generator's ``uniform(lo, hi)`` is ``lo + (hi - lo) * u`` with ``u`` the next
        ``random_sample()``, and each call draws a fixed number of them (area and log-aspect
        when ranges are given, then y, x), so one ``random_sample((n, m))`` yields the same
        values in the same order."""
        area = height * width
        cols = []
        if hasattr(scale, "__len__"):
            cols.append((scale[0], scale[1]))
        if hasattr(ratio, "__len__"):
            lr = np.log(ratio)
            cols.append((lr[0], lr[1]))
        lo, hi = 0.5 - dist, 0.5 + dist
        cols += [(lo, hi), (lo, hi)]
        u = np.random.random_sample((n, len(cols)))
        v = np.stack([a + (b - a) * u[:, j] for j, (a, b) in enumerate(cols)], axis=1)
        j = 0
        if hasattr(scale, "__len__"):
            target_area = area * v[:, j]
            j += 1
        else:
            target_area = np.full(n, area * scale, np.float64)
        aspect = np.exp(v[:, j]) if hasattr(ratio, "__len__") else np.full(n, ratio, np.float64)
        w = np.round(np.sqrt(target_area * aspect)).astype(np.int64)
        h = np.round(np.sqrt(target_area / aspect)).astype(np.int64)
        locs = torch.from_numpy(np.ascontiguousarray(v[:, -2:])).to(dtype=self.dtype, device=self.device)
        return locs, torch.from_numpy(np.stack([h, w], axis=1))

    def _sample_views(self, x, fixations, fixation_sizes):
        """``[B, F, C, N]`` samples of the ``F`` fixations ``[B, 2]`` with sizes ``[B, 2]``."""
        rt = self.retinal_transform
        per_call = rt.training and (rt.pre_transforms is not None or rt.post_transforms is not None)
        if per_call or not hasattr(rt, "forward_views"):
            return torch.stack([rt(x, f, fixation_size=s) for f, s in zip(fixations, fixation_sizes)], dim=1)
        return rt.forward_views(x, torch.stack([torch.as_tensor(f).to(rt.device) for f in fixations], dim=1),
                                torch.stack(list(fixation_sizes), dim=1))


class MultiRandomSaccadePolicy(BaseSaccadePolicy):
    """``n_fixations`` random fixations per image (reference ``policies.py:167-292``): random
    crops of area ``crop_area_range`` (training) or ``val_crop_size`` (eval), aspect in
    [3/4, 4/3] with ``add_aspect_variation``; with ``norm_dist_from_center`` the centres are
    uniform within that distance of the image centre."""

    def __init__(self, retinal_transform, n_fixations=2, crop_area_range=(0.08, 1), add_aspect_variation=False,
                 nonrandom_val=False, val_crop_size=1, nonrandom_first=False, norm_dist_from_center=None):
        super().__init__(retinal_transform, n_fixations)
        self.crop_area_range = list(crop_area_range)
        self.add_aspect_variation = add_aspect_variation
        self.crop_aspect_range = [3 / 4, 4 / 3] if add_aspect_variation else 1
        self.val_crop_size = val_crop_size
        self.nonrandom_first = nonrandom_first
        self.multi_policy = True
        self.nonrandom_val = nonrandom_val
        self.norm_dist_from_center = norm_dist_from_center

    def forward(self, x, n_fixations=None, fixations=None, fixation_size=None, area_range=None):
        """Dict of ``x_fixs [B, F, C, N]``, ``fixations [B, F, 2]``, ``fixation_sizes [B, F, 2]``
        and ``fix_deltas [B, F, 2]`` (reference ``policies.py:221-281``). Fixations are drawn
        even when given (the reference consumes the draws either way); ``fixation_size`` is
        accepted and unused, as in the reference."""
        if n_fixations is None:
            n_fixations = self.n_fixations
        assert fixations is None or len(fixations) == n_fixations
        bsz = x.shape[0]
        sizes, drawn = [], []
        for fix_i in range(n_fixations):
            loc, size = self.sample_fixations(x.shape[2:], n=bsz, area_range=area_range,
                                              norm_dist_from_center=self.norm_dist_from_center)
            sizes.append(size)
            if fix_i == 0 and self.nonrandom_first:
                loc = torch.tensor([0.5, 0.5]).to(dtype=loc.dtype, device=loc.device).unsqueeze(0).expand(bsz, 2)
            drawn.append(loc)
        if fixations is None:
            if self.nonrandom_val and not self.training:
                # centre fixations (the reference builds a flat list of floats here, which its
                # torch.stack below rejects)
                fixations = [torch.full((bsz, 2), 0.5, dtype=self.dtype, device=self.device)
                             for _ in range(n_fixations)]
            else:
                fixations = drawn
        else:
            fixations = list(fixations)
            for ii, fixation in enumerate(fixations):
                if len(fixation) == 2:
                    fixations[ii] = torch.ones(bsz, 2) * fixation
        x_fixs = self._sample_views(x, fixations, sizes)
        deltas = [torch.zeros(bsz, 2, device=x.device)]
        deltas += [fixations[ii] - fixations[ii - 1] for ii in range(1, n_fixations)]
        return {
            "x_fixs": x_fixs,
            "fixations": torch.stack(fixations, dim=1),
            "fixation_sizes": torch.stack(sizes, dim=1),
            "fix_deltas": torch.stack(deltas, dim=1),
        }

    def __repr__(self):
        return (f"MultiRandomSaccadePolicy(\n  retinal_transform={self.retinal_transform},\n"
                f"  n_fixations={self.n_fixations},\n  nonrandom_first={self.nonrandom_first},\n"
                f"  nonrandom_val={self.nonrandom_val},\n  crop_area_range={self.crop_area_range},\n"
                f"  add_aspect_variation={self.add_aspect_variation},\n  val_crop_size={self.val_crop_size},\n"
                f"  norm_dist_from_center={self.norm_dist_from_center}\n)")


class NoSaccadePolicy(BaseSaccadePolicy):
    """One centre fixation of the transform's default size (reference ``policies.py:294-340``)."""

    def __init__(self, retinal_transform):
        super().__init__(retinal_transform, 1)
        self.multi_policy = False

    def forward(self, x, f1=None, area_range=None, n_fixations=None, fixation_size=None, fixations=None):
        assert (f1 is None and area_range is None and (n_fixations is None or n_fixations == 1)
                and fixation_size is None and fixations is None)
        x_f1 = self.retinal_transform(x, f1).unsqueeze(1)
        n = x_f1.shape[0]
        return {
            "x_fixs": x_f1,
            "fixations": 0.5 * torch.ones((n, 1, 2)),
            "fixation_sizes": self.fixation_size * torch.ones((n, 1, 2)),
            "fix_deltas": torch.zeros(n, 1, 2),
        }

    def __repr__(self):
        return f"NoSaccadePolicy(\n  retinal_transform={self.retinal_transform},\n  n_fixations={self.n_fixations}\n)"


class PolicyRegistry:
    """Name -> builder of a policy from a network object with ``retinal_transform``,
    ``n_fixations`` and ``cfg.saccades`` (reference ``policies.py:343-399``)."""

    def __init__(self):
        self._builders = {}

    def register(self, name, builder_fn):
        self._builders[name] = builder_fn

    def get(self, name):
        if name not in self._builders:
            raise ValueError(f"Policy '{name}' not found. Available policies: {list(self._builders.keys())}")
        return self._builders[name]

    def has(self, name):
        return name in self._builders

    def __repr__(self):
        if not self._builders:
            return "PolicyRegistry(no policies registered)"
        return "PolicyRegistry(\n  " + "\n  ".join(sorted(self._builders)) + "\n)"


def _multi_random(nearcenter, nonrandom_val):
    def build(sn):
        s = sn.cfg.saccades
        return MultiRandomSaccadePolicy(
            sn.retinal_transform, sn.n_fixations,
            nonrandom_first=getattr(s, "nonrandom_first", False),
            norm_dist_from_center=s.nearcenter_dist if nearcenter else None,
            nonrandom_val=nonrandom_val,
            crop_area_range=[s.fixation_size_min_frac, s.fixation_size_max_frac],
            add_aspect_variation=s.add_aspect_variation,
            val_crop_size=s.fixation_size_frac_val)
    return build


# the reference's built-in names (policies.py:405-474)
FIXATION_POLICY_REGISTRY = PolicyRegistry()
FIXATION_POLICY_REGISTRY.register("multi_random", _multi_random(False, False))
FIXATION_POLICY_REGISTRY.register("multi_random_nearcenter", _multi_random(True, False))
FIXATION_POLICY_REGISTRY.register("multi_random_nearcenter_train", _multi_random(True, True))
FIXATION_POLICY_REGISTRY.register("multi_random_train", _multi_random(False, True))
FIXATION_POLICY_REGISTRY.register("none", lambda sn: NoSaccadePolicy(sn.retinal_transform))
FIXATION_POLICY_REGISTRY.register("MultiRandomSaccadePolicy", FIXATION_POLICY_REGISTRY.get("multi_random"))
FIXATION_POLICY_REGISTRY.register("NoSaccadePolicy", FIXATION_POLICY_REGISTRY.get("none"))
