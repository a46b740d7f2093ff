"""GPU parity of the foveated sampler against the CPU oracle.

Bar: transformed sample coordinates bit-exact; nearest-mode values bit-exact;
bilinear fp32 values within 1e-5 relative (L2 and max-abs/max|ref|) and at
least 99.9% of them bit-identical to torch's CPU grid_sample (the kernel uses
its fused-multiply-add rounding); bf16 outputs within 1e-2 relative.
"""
import os

import numpy as np
import pytest
import torch

from fovi_amd.sensing.retina import RetinalTransform
from fovi_amd.sensing.samplers import GridSampler
from oracle import sampler_ref
from tests.helpers import assert_close_rel, assert_mostly_bit_exact

pytestmark = pytest.mark.gpu


def _run(img, res, mode, pad, fix_loc, fix_size, out_dtype=None):
    s = GridSampler(16, 2.78, res, device="cuda", mode=mode, style="logpolar", padding_mode=pad)
    out, grid = s.sample_views(img.cuda(), fix_loc, fix_size, out_dtype=out_dtype, return_grid=True)
    ref, ref_grid = sampler_ref.sampler_forward(img.float(), s.sampling_grid.cpu(), torch.as_tensor(fix_loc),
                                                fix_size, mode, pad)
    return out.cpu(), grid.cpu(), ref, ref_grid.squeeze(1)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("pad", ["zeros", "border"])
def test_c1_plumbing_centre_fixation(mode, pad):
    """C1: batch 8 of 3x256x256 fp32, 64x64 log-polar sensor, centre fixation, 256 px window."""
    g = torch.Generator().manual_seed(0)
    img = torch.rand(8, 3, 256, 256, generator=g)
    fix_loc = torch.full((8, 2), 0.5)
    fix_size = np.array([[256, 256]] * 8)
    out, grid, ref, ref_grid = _run(img, 64, mode, pad, fix_loc, fix_size)
    assert torch.equal(grid, ref_grid), "sample coordinates differ"
    if mode == "nearest":
        assert torch.equal(out, ref)
    else:
        assert_close_rel(out, ref, 1e-5, "bilinear fp32")
        assert_mostly_bit_exact(out, ref, what="bilinear fp32")


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
def test_random_fixations_non_square(mode):
    g = torch.Generator().manual_seed(2)
    img = torch.rand(5, 3, 200, 312, generator=g)
    fix_loc = 0.25 + 0.5 * torch.rand(5, 2, generator=g)
    fix_size = np.array([[150, 170], [200, 312], [96, 96], [300, 250], [64, 128]])
    out, grid, ref, ref_grid = _run(img, 32, mode, "zeros", fix_loc, fix_size)
    assert torch.equal(grid, ref_grid)
    if mode == "nearest":
        assert torch.equal(out, ref)
    else:
        assert_close_rel(out, ref, 1e-5, "bilinear fp32")
        assert_mostly_bit_exact(out, ref, what="bilinear fp32")


def test_float64_fixation_sizes_use_fp64_multiply():
    """Float fixation sizes make the reference multiply in fp64 (coords.py:632-633)."""
    g = torch.Generator().manual_seed(3)
    img = torch.rand(3, 3, 128, 128, generator=g)
    fix_loc = torch.tensor([[0.5, 0.5], [0.31, 0.62], [0.7, 0.41]])
    fix_size = np.array([[127.3, 99.9], [64.7, 64.7], [111.1, 131.13]], dtype=np.float64)
    out, grid, ref, ref_grid = _run(img, 48, "bilinear", "zeros", fix_loc, fix_size)
    assert torch.equal(grid, ref_grid)
    assert_close_rel(out, ref, 1e-5)


def test_bf16_image_and_output():
    g = torch.Generator().manual_seed(4)
    img = torch.rand(4, 3, 256, 256, generator=g).bfloat16()
    fix_loc = 0.25 + 0.5 * torch.rand(4, 2, generator=g)
    fix_size = np.array([[256, 256]] * 4)
    out, grid, ref, ref_grid = _run(img, 64, "bilinear", "zeros", fix_loc, fix_size, out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    assert torch.equal(grid, ref_grid)
    assert_close_rel(out.float(), ref, 1e-2, "bf16")
    out32, _, ref32, _ = _run(img, 64, "nearest", "zeros", fix_loc, fix_size, out_dtype=torch.float32)
    assert torch.equal(out32, ref32)


def test_fused_fixation_views_match_per_view_calls():
    """F fixations x B images in one launch, view (f, b) reads image b."""
    g = torch.Generator().manual_seed(5)
    B, Fx = 3, 4
    img = torch.rand(B, 3, 160, 160, generator=g)
    fix = 0.25 + 0.5 * torch.rand(Fx, B, 2, generator=g)
    s = GridSampler(16, 2.78, 40, device="cuda", mode="bilinear", style="logpolar")
    view_image = torch.arange(B).repeat(Fx)
    out = s.sample_views(img.cuda(), fix.reshape(-1, 2), np.array([[160, 160]] * (Fx * B)),
                         view_image=view_image).cpu()
    for f in range(Fx):
        ref, _ = sampler_ref.sampler_forward(img, s.sampling_grid.cpu(), fix[f], np.array([[160, 160]] * B))
        assert_close_rel(out[f * B:(f + 1) * B], ref, 1e-5, f"fixation {f}")


def test_strided_input_and_output_layouts():
    g = torch.Generator().manual_seed(6)
    img = torch.rand(2, 3, 96, 96, generator=g).to(memory_format=torch.channels_last)
    s = GridSampler(16, 2.78, 24, device="cuda", mode="bilinear", style="logpolar")
    out_cl = torch.empty(2, 576, 3, device="cuda").transpose(1, 2)   # [V, C, N] view of [V, N, C]
    fix_loc = torch.tensor([[0.4, 0.6], [0.5, 0.5]])
    s.sample_views(img.cuda(), fix_loc, np.array([[96, 96]] * 2), out=out_cl)
    ref, _ = sampler_ref.sampler_forward(img.contiguous(), s.sampling_grid.cpu(), fix_loc, np.array([[96, 96]] * 2))
    assert_close_rel(out_cl.cpu(), ref, 1e-5)


def test_retinal_transform_defaults():
    """RetinalTransform argument handling: scalar fixation size, tuple fix_loc, numpy sizes."""
    g = torch.Generator().manual_seed(7)
    img = torch.rand(4, 3, 224, 224, generator=g)
    rt = RetinalTransform(64, start_res=224, fov=16, cmf_a=2.78, style="logpolar", sampler="grid_bilinear",
                          device="cuda")
    out = rt(img.cuda(), (0.5, 0.5)).cpu()
    ref, _ = sampler_ref.sampler_forward(img, rt.sampler.sampling_grid.cpu(), torch.full((4, 2), 0.5),
                                         np.array([[224, 224]] * 4))
    assert out.shape == (4, 3, 4096)
    assert_close_rel(out, ref, 1e-5)


def test_full_size_c4_views_match_per_view_and_are_deterministic():
    """C4-shaped launch (512 views of 128 images, 16384 points, bf16): size-independent checks.

    Each view equals the single-view launch of the same image bit for bit,
    and a repeat launch is bit-identical.
    """
    g = torch.Generator().manual_seed(0)
    B, Fx = 128, 4
    img = torch.rand(B, 3, 512, 512, generator=g).bfloat16().cuda()
    fix = (0.25 + 0.5 * torch.rand(B * Fx, 2, generator=g))
    vmap = torch.arange(B).repeat_interleave(Fx)
    s = GridSampler(16, 2.78, 128, device="cuda", mode="nearest", style="logpolar")
    sizes = np.array([[512, 512]] * (B * Fx))
    out = s.sample_views(img, fix, sizes, view_image=vmap)
    out2 = s.sample_views(img, fix, sizes, view_image=vmap)
    assert torch.equal(out, out2)
    for v in (0, 1, 257, B * Fx - 1):
        one = s.sample_views(img[vmap[v]:vmap[v] + 1], fix[v:v + 1], sizes[:1])
        assert torch.equal(out[v:v + 1], one)
    ref, _ = sampler_ref.sampler_forward(img[vmap[5]:vmap[5] + 1].float().cpu(), s.sampling_grid.cpu(),
                                         fix[5:6], sizes[:1], mode="nearest")
    assert torch.equal(out[5:6].float().cpu(), ref)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("pad", ["zeros", "border"])
@pytest.mark.parametrize("dt,channels", [(torch.float32, 3), (torch.bfloat16, 3), (torch.bfloat16, 1),
                                         (torch.float32, 4)])
def test_ring_blocked_order_equals_point_order(mode, pad, dt, channels):
    """The 8-ring x 32-angle processing order of ring-major grids changes no result.

    Fixations near the corners put part of the sensor outside the image, and
    an odd image width sends some rows to the per-pixel bilinear loads.
    """
    g = torch.Generator().manual_seed(11)
    img = torch.rand(3, channels, 150, 173, generator=g).to(dt).cuda()
    fix = torch.tensor([[0.5, 0.5], [0.05, 0.95], [0.9, 0.1], [0.3, 0.7], [0.6, 0.4], [0.99, 0.99]])
    sizes = np.array([[150, 173]] * 6)
    vmap = torch.tensor([0, 0, 1, 1, 2, 2])
    s = GridSampler(16, 2.78, 64, device="cuda", mode=mode, style="logpolar", padding_mode=pad)
    blocked, g1 = s.sample_views(img, fix, sizes, view_image=vmap, return_grid=True)
    out_cl = torch.empty(6, 4096, channels, device="cuda", dtype=dt).transpose(1, 2)
    s.sample_views(img, fix, sizes, view_image=vmap, out=out_cl)
    s.ring_order = False
    linear, g2 = s.sample_views(img, fix, sizes, view_image=vmap, return_grid=True)
    assert torch.equal(g1, g2)
    assert torch.equal(blocked, linear)
    assert torch.equal(out_cl, linear)
    ref, _ = sampler_ref.sampler_forward(img[1:2].float().cpu(), s.sampling_grid.cpu(), fix[2:3], sizes[:1],
                                         mode, pad)
    assert_close_rel(blocked[2:3].float().cpu(), ref, 1e-5 if dt == torch.float32 else 1e-2)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("pad", ["zeros", "border"])
@pytest.mark.parametrize("channels,width", [(3, 173), (3, 174), (4, 173)])
def test_channels_last_images_equal_channel_planes(mode, pad, channels, width):
    """bf16 images in the channels-last memory format (one load per tap for all channels)
    give the channel-plane results bit for bit: odd and even widths, so taps start at odd and
    even elements, and corner fixations with border padding, so taps hit each row's last
    pixel (loaded channel by channel)."""
    g = torch.Generator().manual_seed(12)
    planar = torch.rand(3, channels, 150, width, generator=g).to(torch.bfloat16).cuda()
    cl = planar.contiguous(memory_format=torch.channels_last)
    assert cl.stride()[1] == 1 and cl.stride()[3] == channels
    fix = torch.tensor([[0.5, 0.5], [0.05, 0.95], [0.9, 0.1], [0.3, 0.7], [0.6, 0.4], [0.99, 0.99]])
    sizes = np.array([[150, width]] * 6)
    vmap = torch.tensor([0, 0, 1, 1, 2, 2])
    s = GridSampler(16, 2.78, 64, device="cuda", mode=mode, style="logpolar", padding_mode=pad)
    want = s.sample_views(planar, fix, sizes, view_image=vmap)
    got = s.sample_views(cl, fix, sizes, view_image=vmap)
    assert torch.equal(got, want)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("channels", [3, 4])
def test_channels_last_views_with_odd_row_stride(mode, channels):
    """Channels-last views whose row stride is odd (``as_strided`` over a larger buffer) put
    the pixels of odd rows at odd elements. Three-channel pixels are read there with the
    one-load-per-tap path; four-channel ones need even elements, so such a view takes the
    channel-plane kernel. Either way the samples equal those of a contiguous copy."""
    g = torch.Generator().manual_seed(13)
    H, W, B = 90, 101, 2
    rs = channels * W + (1 if channels * W % 2 == 0 else 2)    # odd
    base = torch.rand(B * H * rs + 8, generator=g).to(torch.bfloat16).cuda()
    img = base.as_strided((B, channels, H, W), (H * rs, 1, rs, channels))
    assert img.stride(2) % 2 == 1 and img.stride(0) % 2 == 0
    fix = torch.tensor([[0.5, 0.5], [0.1, 0.9], [0.8, 0.2], [0.97, 0.97]])
    sizes = np.array([[H, W]] * 4)
    vmap = torch.tensor([0, 0, 1, 1])
    s = GridSampler(16, 2.78, 64, device="cuda", mode=mode, style="logpolar", padding_mode="border")
    want = s.sample_views(img.contiguous(), fix, sizes, view_image=vmap)
    got = s.sample_views(img, fix, sizes, view_image=vmap)
    assert torch.equal(got, want)


@pytest.mark.parametrize("mode", ["bilinear", "nearest"])
@pytest.mark.parametrize("channels,layout,n_views,res", [(3, "planes", 37, 64), (3, "channels_last", 40, 64),
                                                         (4, "channels_last", 16, 64), (1, "planes", 20, 64),
                                                         (2, "planes", 19, 64), (3, "planes", 517, 128),
                                                         (3, "channels_last", 512, 128), (1, "planes", 512, 128),
                                                         (2, "planes", 520, 128), (4, "planes", 512, 128)])
def test_view_major_output_equals_the_view_planes(mode, channels, layout, n_views, res):
    """Output into a view-major buffer [N, V, 4] (the rows of one point for all views
    adjacent, as the view-major kNN-conv kernel reads them; a sampler block writes 4 or 16
    views of a point as one run, 16 at the C4 size, where nearest sampling from channel planes
    takes eight views at a time, 1 to 4 channels) holds the samples of the ordinary
    [V, C, N] output bit for bit, for partial groups of views, and leaves the row elements past
    the channels untouched."""
    g = torch.Generator().manual_seed(16)
    n_img = (n_views + 3) // 4
    img = torch.rand(n_img, channels, 120, 131, generator=g).to(torch.bfloat16).cuda()
    if layout == "channels_last":
        img = img.contiguous(memory_format=torch.channels_last)
    fix = 0.2 + 0.6 * torch.rand(n_views, 2, generator=g)
    sizes = np.array([[120, 131]] * n_views)
    vmap = torch.arange(n_views) // 4
    s = GridSampler(16, 2.78, res, device="cuda", mode=mode, style="logpolar", padding_mode="zeros")
    want = s.sample_views(img, fix, sizes, view_image=vmap, out_dtype=torch.bfloat16)
    buf = torch.full((res * res, n_views, 4), 7.0, dtype=torch.bfloat16, device="cuda")
    view = buf.permute(1, 2, 0)[:, :channels]
    s.sample_views(img, fix, sizes, view_image=vmap, out=view)
    assert torch.equal(view, want)
    assert (buf[..., channels:] == 7.0).all(), "elements past the channels were written"


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tables.npz")


@pytest.mark.parametrize("mode", ["nearest", "bilinear"])
def test_oracle_grid_from_reference_cartesian(mode):
    """The oracle's grid comes from the reference-written sensor points (64x64 log-polar,
    tests/golden/tables.npz) through the reference's (x, -y) mapping, not from the build's
    own sampling_grid."""
    import types
    cart = torch.from_numpy(np.load(GOLDEN)["c1__in_cartesian"])
    # the sampler takes the reference-written points as its coords: host-built coordinates
    # round per host CPU (MKL's vendor-dispatched kernels), the written ones do not
    coords = types.SimpleNamespace(cartesian=cart, polar=torch.zeros_like(cart), resolution=64,
                                   shape=cart.shape)
    g = torch.Generator().manual_seed(12)
    img = torch.rand(3, 3, 200, 240, generator=g)
    fix_loc = torch.tensor([[0.5, 0.5], [0.35, 0.6], [0.7, 0.3]])
    fix_size = np.array([[200, 240], [150, 150], [256, 200]])
    s = GridSampler(16, 2.78, 64, device="cuda", mode=mode, style="logpolar", coords=coords)
    out, grid = s.sample_views(img.cuda(), fix_loc, fix_size, return_grid=True)
    ref, ref_grid = sampler_ref.sampler_forward(img, sampler_ref.grid_from_cartesian(cart), fix_loc, fix_size,
                                                mode)
    assert torch.equal(grid.cpu(), ref_grid.squeeze(1))
    if mode == "nearest":
        assert torch.equal(out.cpu(), ref)
    else:
        assert_close_rel(out.cpu(), ref, 1e-5, "bilinear vs the reference-cartesian oracle")


@pytest.mark.parametrize("mode", ["nearest", "bilinear"])
@pytest.mark.parametrize("axis", ["rows", "columns"])
def test_half_lit_image_known_answer(mode, axis):
    """Known answer of the axis convention: with the top half of the image lit (rows < H/2),
    every sensor point above the fixation (y > 0, clear of the middle row) samples 1 and every
    point below samples 0; with the right half lit (columns >= W/2), points with x > 0 sample
    1. Centre fixation, window = image."""
    H = W = 256
    img = torch.zeros(2, 3, H, W)
    if axis == "rows":
        img[:, :, : H // 2, :] = 1.0
    else:
        img[:, :, :, W // 2:] = 1.0
    s = GridSampler(16, 2.78, 64, device="cuda", mode=mode, style="logpolar")
    out = s.sample_views(img.cuda(), torch.full((2, 2), 0.5), np.array([[H, W]] * 2)).cpu()
    cart = s.coords.cartesian.cpu()
    coord = cart[:, 1] if axis == "rows" else cart[:, 0]
    margin = 2.0 / H      # one pixel in normalised units: clear of the lit edge (bilinear blends 1 px)
    # and clear of the image border, where the outer ring's bilinear taps meet the zero padding
    inside = cart.norm(dim=1) < 1 - 2 * margin
    hi, lo = (coord > margin) & inside, (coord < -margin) & inside
    assert hi.sum() > 1000 and lo.sum() > 1000
    # bilinear weights (1 - dy)(1 - dx) + ... sum to 1 within fp32 rounding
    tol = 0.0 if mode == "nearest" else 1e-6
    ref, _ = sampler_ref.sampler_forward(img, s.sampling_grid.cpu(), torch.full((2, 2), 0.5),
                                         np.array([[H, W]] * 2), mode)
    for got, what in ((out, "kernel"), (ref, "oracle")):
        assert torch.all((got[:, :, hi] - 1.0).abs() <= tol), f"{what}: points on the lit side did not sample 1"
        assert torch.all(got[:, :, lo] == 0.0), f"{what}: points on the dark side did not sample 0"


def test_colour_decay_and_eval_grayscale():
    """sigma: samples x exp(-r / sigma) per sensor point (r = the sampler's polar radius);
    eval with no_color_val: 0.2989 R + 0.587 G + 0.114 B on all three channels (torchvision's
    rgb_to_grayscale, reference retina.py:148-150). The reference's own decay expression
    (x * decay.unsqueeze(1), retina.py:398-401) cannot broadcast [B, 3, N] against [N, 1]."""
    g = torch.Generator().manual_seed(13)
    img = torch.rand(3, 3, 128, 128, generator=g)
    sigma = 0.35
    rt = RetinalTransform(32, start_res=128, fov=16, cmf_a=2.78, style="logpolar", sampler="grid_bilinear",
                          device="cuda", sigma=sigma, auto_match_cart_resources=0)
    plain = RetinalTransform(32, start_res=128, fov=16, cmf_a=2.78, style="logpolar", sampler="grid_bilinear",
                             device="cuda", auto_match_cart_resources=0)
    base = plain(img.cuda(), (0.5, 0.5)).cpu()
    decay = torch.exp(-rt.sampler.polar_radius.cuda() / sigma).cpu()
    assert torch.equal(rt(img.cuda(), (0.5, 0.5)).cpu(), base * decay[None, None, :])
    with pytest.raises(RuntimeError):
        base * decay.unsqueeze(1)
    gray = RetinalTransform(32, start_res=128, fov=16, cmf_a=2.78, style="logpolar", sampler="grid_bilinear",
                            device="cuda", no_color_val=True, auto_match_cart_resources=0).eval()
    y = gray(img.cuda(), (0.5, 0.5)).cpu()
    want = 0.2989 * base[:, 0] + 0.587 * base[:, 1] + 0.114 * base[:, 2]
    for c in range(3):
        assert torch.equal(y[:, c], want)
    assert torch.equal(gray.train()(img.cuda(), (0.5, 0.5)).cpu(), base)
