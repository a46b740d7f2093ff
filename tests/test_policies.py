"""Fixation policies (reference fovi/sensing/policies.py): the draw sequence pinned on the CPU,
the fused multi-view sampling checked on the GPU against per-fixation calls and the oracle."""
import types

import numpy as np
import pytest
import torch

from fovi_amd.sensing.policies import (FIXATION_POLICY_REGISTRY, MultiRandomSaccadePolicy, NoSaccadePolicy)
from oracle import policy_ref as R
from tests.helpers import assert_close_rel


class _StubTransform(torch.nn.Module):
    """A retinal transform stand-in for CPU tests: records the views it is asked for."""

    def __init__(self, fixation_size=64):
        super().__init__()
        self.fixation_size, self.dtype, self.device = fixation_size, torch.float32, "cpu"
        self.pre_transforms = self.post_transforms = None
        self.calls = []

    def forward_views(self, x, fix_loc, fixation_size):
        self.calls.append((fix_loc.clone(), fixation_size.clone()))
        return torch.zeros(x.shape[0], fix_loc.shape[1], 3, 5)

    def forward(self, x, fix_loc, fixation_size=None):
        return torch.zeros(x.shape[0], 3, 5)


# ------------------------------------------------------------------- CPU: oracle pinning ---
def test_nearcenter_eval_draws_closed_form():
    """Eval mode, scalar area and ratio: the only draws are the centres, y then x per image,
    images within a fixation: lo + (hi - lo) * u over one stream of uniforms."""
    rs = np.random.RandomState(11)
    locs, sizes = R.multi_random_fixations(rs, 5, 96, 128, 3, training=False, dist=0.25)
    u = np.random.RandomState(11).random_sample(5 * 3 * 2).reshape(3, 5, 2)
    want = 0.25 + 0.5 * u
    assert np.array_equal(locs, want.transpose(1, 0, 2))
    side = int(round(np.sqrt(96 * 128)))
    assert (sizes == side).all()


def test_nearcenter_training_draws_closed_form():
    """Training with area and aspect ranges: per image four draws (area, log-aspect, y, x)."""
    rs = np.random.RandomState(3)
    locs, sizes = R.multi_random_fixations(rs, 4, 200, 300, 2, training=True, crop_area_range=(0.2, 0.9),
                                           add_aspect_variation=True, dist=0.1)
    u = np.random.RandomState(3).random_sample(2 * 4 * 4).reshape(2, 4, 4)
    area = 200 * 300 * (0.2 + 0.7 * u[..., 0])
    lr = np.log([3 / 4, 4 / 3])
    aspect = np.exp(lr[0] + (lr[1] - lr[0]) * u[..., 1])
    w = np.round(np.sqrt(area * aspect)).astype(np.int64)
    h = np.round(np.sqrt(area / aspect)).astype(np.int64)
    assert np.array_equal(sizes, np.stack([h, w], -1).transpose(1, 0, 2))
    lo, hi = 0.5 - 0.1, 0.5 + 0.1
    assert np.array_equal(locs, (lo + (hi - lo) * u[..., 2:]).transpose(1, 0, 2))


def test_random_crop_invariants_and_fallback():
    rs = np.random.RandomState(5)
    for _ in range(300):
        (cy, cx), (h, w) = R.random_crop(rs, 90, 160, [0.08, 1.0], [3 / 4, 4 / 3])
        assert 0 < h <= 90 and 0 < w <= 160
        top, left = cy * 90 - h / 2, cx * 160 - w / 2
        assert abs(top - round(top)) < 1e-9 and abs(left - round(left)) < 1e-9
        assert 0 <= round(top) <= 90 - h and 0 <= round(left) <= 160 - w
        assert 0.08 * 90 * 160 * 0.9 <= h * w <= 90 * 160 * 1.02
        assert 3 / 4 * 0.9 <= w / h <= 4 / 3 * 1.1
    # an area that never fits: the centred crop clamped to the ratio range
    (cy, cx), (h, w) = R.random_crop(np.random.RandomState(0), 90, 160, [4.0, 5.0], [3 / 4, 4 / 3])
    assert (h, w) == (90, 120) and (cy, cx) == (0.5, 0.5)


# ------------------------------------------------------------------- CPU: the policy ---
@pytest.mark.parametrize("dist", [None, 0.25])
@pytest.mark.parametrize("training", [True, False])
def test_policy_draws_match_the_oracle(dist, training):
    rt = _StubTransform()
    pol = MultiRandomSaccadePolicy(rt, n_fixations=3, crop_area_range=[0.3, 1.0], add_aspect_variation=True,
                                   norm_dist_from_center=dist, nonrandom_first=True)
    pol.train(training)
    # eval-mode random crops take the whole image (val_crop_size 1, ratio 1), which fits only a
    # square image: for others the reference's fallback min(ratio) of a scalar raises
    hh, ww = (72, 100) if training or dist is not None else (80, 80)
    x = torch.zeros(4, 3, hh, ww)
    np.random.seed(21)
    out = pol(x)
    locs, sizes = R.multi_random_fixations(np.random.RandomState(21), 4, hh, ww, 3, training,
                                           crop_area_range=(0.3, 1.0), add_aspect_variation=True,
                                           nonrandom_first=True, dist=dist)
    assert out["x_fixs"].shape == (4, 3, 3, 5)
    assert torch.equal(out["fixations"], torch.tensor(locs, dtype=torch.float32))
    assert torch.equal(out["fixation_sizes"], torch.tensor(sizes))
    d = out["fixations"]
    assert torch.equal(out["fix_deltas"][:, 0], torch.zeros(4, 2))
    assert torch.equal(out["fix_deltas"][:, 1:], d[:, 1:] - d[:, :-1])
    # one fused call with all views
    (loc, size), = rt.calls
    assert torch.equal(loc, out["fixations"]) and torch.equal(size, out["fixation_sizes"])


def test_policy_given_fixations_and_nonrandom_val():
    rt = _StubTransform()
    pol = MultiRandomSaccadePolicy(rt, n_fixations=2, nonrandom_val=True).eval()
    out = pol(torch.zeros(3, 3, 40, 40))
    assert torch.equal(out["fixations"], torch.full((3, 2, 2), 0.5))
    given = [torch.tensor([0.2, 0.7]), torch.tensor([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]])]
    out = MultiRandomSaccadePolicy(rt, n_fixations=2)(torch.zeros(3, 3, 40, 40), fixations=given)
    assert torch.equal(out["fixations"][:, 0], torch.tensor([[0.2, 0.7]] * 3))
    assert torch.equal(out["fixations"][:, 1], given[1])


def test_no_saccade_policy_and_registry():
    rt = _StubTransform(fixation_size=48)
    out = NoSaccadePolicy(rt)(torch.zeros(2, 3, 48, 48))
    assert out["x_fixs"].shape == (2, 1, 3, 5)
    assert torch.equal(out["fixations"], torch.full((2, 1, 2), 0.5))
    assert torch.equal(out["fixation_sizes"], torch.full((2, 1, 2), 48.0))
    s = types.SimpleNamespace(nonrandom_first=False, nearcenter_dist=0.25, fixation_size_min_frac=0.5,
                              fixation_size_max_frac=1.0, add_aspect_variation=False, fixation_size_frac_val=1)
    sn = types.SimpleNamespace(retinal_transform=rt, n_fixations=4, cfg=types.SimpleNamespace(saccades=s))
    p = FIXATION_POLICY_REGISTRY.get("multi_random_nearcenter")(sn)
    assert p.n_fixations == 4 and p.norm_dist_from_center == 0.25 and p.crop_area_range == [0.5, 1.0]
    assert FIXATION_POLICY_REGISTRY.get("multi_random_nearcenter_train")(sn).nonrandom_val
    assert isinstance(FIXATION_POLICY_REGISTRY.get("NoSaccadePolicy")(sn), NoSaccadePolicy)
    with pytest.raises(ValueError):
        FIXATION_POLICY_REGISTRY.get("nope")


# ------------------------------------------------------------------------------ GPU ---
@pytest.mark.gpu
@pytest.mark.parametrize("sampler", ["grid_nn", "grid_bilinear", "pooling"])
def test_fused_views_equal_per_fixation_calls_and_oracle(sampler):
    from fovi_amd.sensing.retina import RetinalTransform
    from oracle import knnpool_ref, sampler_ref
    rt = RetinalTransform(16, start_res=96, fov=16, cmf_a=2.78, style="logpolar", sampler=sampler, device="cuda",
                          auto_match_cart_resources=0, res_mult=2) if sampler == "pooling" else \
        RetinalTransform(32, start_res=96, fov=16, cmf_a=2.78, style="logpolar", sampler=sampler, device="cuda",
                         auto_match_cart_resources=0)
    pol = MultiRandomSaccadePolicy(rt, n_fixations=4, crop_area_range=[0.3, 1.0], add_aspect_variation=True)
    img = torch.rand(3, 3, 96, 128, generator=torch.Generator().manual_seed(2))
    np.random.seed(7)
    with torch.no_grad():
        out = pol(img.cuda())
    y = out["x_fixs"]
    assert y.shape == (3, 4, 3, rt.sampler.coords.shape[0])
    mode = "bilinear" if sampler == "grid_bilinear" else "nearest"
    for f in range(4):
        with torch.no_grad():
            loop = rt(img.cuda(), out["fixations"][:, f], fixation_size=out["fixation_sizes"][:, f])
        assert torch.equal(y[:, f], loop), f"fixation {f}: fused views differ from the per-fixation call"
        sizes = out["fixation_sizes"][:, f].numpy()
        ref, _ = sampler_ref.sampler_forward(img, rt.sampler.sampling_grid.cpu(), out["fixations"][:, f].cpu(),
                                             sizes, mode=mode)
        if sampler == "pooling":
            ref = knnpool_ref.knnpool_forward(ref, rt.sampler.pooler.knn_indices.cpu(), ref.shape[2], "avg")
            assert_close_rel(y[:, f].cpu(), ref, 1e-5, f"pooling view {f}")
        elif mode == "nearest":
            assert torch.equal(y[:, f].cpu(), ref)
        else:
            assert_close_rel(y[:, f].cpu(), ref, 1e-5, f"bilinear view {f}")
