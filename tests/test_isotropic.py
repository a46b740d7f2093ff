"""Isotropic sensor (the reference's default style) and visual-field neighbourhoods.

CPU: coordinates, pad rings, neighbour indices / distances and ref slots bit for bit
against ``tests/golden/isotropic.npz`` (written by the reference itself,
``tests/golden/make_golden.py --isotropic``), and closed forms of the cortical manifold.
GPU: kNN-conv forward and backward and kNN pooling on isotropic layers, whose neighbour
lists hold pad-ring tokens (indices >= N_in), against the oracle; fp32 1e-5 relative,
bf16 1e-2 relative (same bars as the log-polar tests).
"""
import os

import numpy as np
import pytest
import torch

from fovi_amd.arch.knn import KNNConvLayer, KNNPoolingLayer, get_in_out_coords
from fovi_amd.sensing.coords import SamplingCoords, isotropic_ring_counts, num_sampling_coords
from oracle import knnconv_ref, knnpool_ref
from tests.helpers import assert_close_rel

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "isotropic.npz"))
FOV, CMF_A = 16, 2.78
ISO_LAYERS = {"iso_16_8": (16, 8, 9), "iso_24_12": (24, 12, 25), "iso_16_16": (16, 16, 9)}
VIS_LAYERS = {"vis_iso_16_8": ("isotropic", 16, 8, 9), "vis_lp_16_8": ("logpolar", 16, 8, 9)}
KEYS = ("cartesian", "polar", "plotting", "cortical", "cartesian_pad_coords", "cortical_pad_coords")


def _coords(res, style="isotropic", **kw):
    return SamplingCoords(FOV, CMF_A, res, style=style, **kw)


def _equal(got, name):
    want = GOLDEN[name]
    got = got.numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    assert got.shape == want.shape, f"{name}: shape {got.shape} != {want.shape}"
    assert np.array_equal(got, want), f"{name}: {int((got != want).sum())} elements differ"


# ------------------------------------------------------------------------- CPU ---
@pytest.mark.parametrize("res", [8, 16, 24])
def test_isotropic_coords_match_reference(res):
    c = _coords(res)
    for key in KEYS:
        _equal(getattr(c, key), f"res{res}__{key}")
    assert c.shape[0] == num_sampling_coords(FOV, CMF_A, res, style="isotropic")


def test_scaled_and_auto_matched_sensors_match_reference():
    c = _coords(16, max_val=0.9)
    for key in ("cartesian", "plotting", "cortical", "cartesian_pad_coords", "cortical_pad_coords"):
        _equal(getattr(c, key), f"scaled16__{key}")
    cin, cout, out_cart_res = get_in_out_coords(None, FOV, CMF_A, 2, style="isotropic", in_cart_res=32,
                                                device="cpu", max_out_coord_val="auto")
    _equal([cin.resolution, cout.resolution, out_cart_res], "auto__resolutions")
    for key in ("cartesian", "cortical"):
        _equal(getattr(cin, key), f"auto__in_{key}")
        _equal(getattr(cout, key), f"auto__out_{key}")


@pytest.mark.parametrize("seed,res", [(0, 16), (1, 24)])
def test_fixn_sensor_matches_reference(seed, res):
    """'isotropic_fixn' moves single angles between rings drawn by numpy's global RNG: a
    seeded run builds the reference's sensor, with exactly res**2 points."""
    np.random.seed(seed)
    c = _coords(res, "isotropic_fixn")
    assert c.shape[0] == res * res == num_sampling_coords(FOV, CMF_A, res, style="isotropic_fixn")
    for key in ("cartesian", "polar", "cortical"):
        _equal(getattr(c, key), f"fixn{res}__{key}")


def test_pad_rings_of_other_styles_match_reference():
    _equal(_coords(16, "logpolar").cartesian_pad_coords, "pad_logpolar16")
    _equal(_coords(8, "uniform").cartesian_pad_coords, "pad_uniform8")


def test_isotropic_ring_counts_closed_form():
    """Ring i holds about 2 pi r_i / spacing_i angles: the count is the length of
    arange(0, 2 pi r_i, spacing_i), i.e. ceil(2 pi r_i / spacing_i); the centre is one point."""
    counts = isotropic_ring_counts(FOV, CMF_A, 24)
    assert counts[0] == 1 and len(counts) == 24
    w_lo, w_hi = np.log(CMF_A), np.log(FOV / 2 + CMF_A)
    w = np.linspace(w_lo, w_hi + (w_hi - w_lo) / 23, 25)
    r = np.exp(w) - CMF_A
    for i in range(1, 24):
        spacing = (r[i + 1] - r[i - 1]) / 2
        assert abs(counts[i] - 2 * np.pi * r[i] / spacing) <= 1.0 + 1e-3
    assert sum(counts) == len(_coords(24).cartesian)


def test_notebook_known_answers():
    """Point counts the reference's notebooks print for isotropic sensors (fov 16):
    step2_knnconv cell 12 (a=0.5, auto-matched to 64/32/16/8/4-pixel grids) lists
    4085, 964, 230, 60, 16 coords per layer; cell 10 (stride 4) prints a k=121, n_ref=484
    layer from 4085 coords (res 53) to 230 (res 13); step4_get_activations cell 1
    (a=2.785765) lists 3976 and 64."""
    from fovi_amd.sensing.coords import find_desired_res
    got = [find_desired_res(16, 0.5, c * c, "isotropic", force_less_than=True, quiet=True)[1]
           for c in (64, 32, 16, 8, 4)]
    assert got == [4085, 964, 230, 60, 16]
    got = [find_desired_res(16, 2.785765, c * c, "isotropic", force_less_than=True, quiet=True)[1] for c in (64, 8)]
    assert got == [3976, 64]
    cin, cout, _ = get_in_out_coords(None, 16, 0.5, 4, style="isotropic", in_cart_res=64, device="cpu")
    assert (cin.resolution, cin.shape[0], cout.resolution, cout.shape[0]) == (53, 4085, 13, 230)
    layer = KNNConvLayer(3, 64, 121, cin, cout, device="cpu", arch_flag="doubleres")
    assert layer._k == 121 and layer.ref_coords.shape[0] == 484


def test_cortical_manifold_closed_forms():
    """The manifold's in-plane radius is rho(r) = k/(r+a) sin(r deg) 180/pi (its projection on
    the cortical plane, exact up to fp32 rounding); the height z grows with eccentricity and
    is 0 at the fovea; the polar angle is kept."""
    c = _coords(16)
    ecc = c.polar[:, 0].double() * FOV / 2
    rho = 10 / (ecc + CMF_A) * torch.sin(torch.deg2rad(ecc)) * 180 / np.pi
    xy = c.cortical[:, :2].double()
    assert torch.allclose(xy.norm(dim=1), rho, rtol=1e-5, atol=1e-6)
    order = torch.argsort(ecc)
    z = c.cortical[order, 2].double()
    assert z[0] == 0 and torch.all(z[1:] >= z[:-1] - 1e-6)
    far = ecc > 0.5
    ang = torch.atan2(xy[far, 1], xy[far, 0])
    want = torch.atan2(c.cartesian[far, 1].double(), c.cartesian[far, 0].double())
    assert torch.allclose(torch.remainder(ang - want + np.pi, 2 * np.pi) - np.pi, torch.zeros_like(ang), atol=1e-5)


@pytest.mark.parametrize("name", list(ISO_LAYERS))
def test_isotropic_layer_tables_match_reference(name):
    r_in, r_out, k = ISO_LAYERS[name]
    cin, cout = _coords(r_in), _coords(r_out)
    layer = KNNConvLayer(1, 1, k, cin, cout, device="cpu")
    _equal(layer.knn_indices.to(torch.int32), f"{name}__idx")
    _equal(layer.knn_distances, f"{name}__dist")
    _equal(layer.slots.to(torch.uint8), f"{name}__slots")
    n_in = cin.shape[0]
    assert (layer.knn_indices >= n_in).any(), "the pad ring is reached"
    # the device tables drop pad tokens: every CSR entry is a real input point
    nbr = layer.nbr_sorted.cpu()
    assert torch.all((nbr == -1) | ((nbr >= 0) & (nbr < n_in)))
    assert int((nbr >= 0).sum()) == int((layer.knn_indices < n_in).sum())


@pytest.mark.parametrize("name", list(VIS_LAYERS))
def test_visual_field_layer_tables_match_reference(name):
    style, r_in, r_out, k = VIS_LAYERS[name]
    layer = KNNConvLayer(1, 1, k, _coords(r_in, style), _coords(r_out, style), device="cpu", sample_cortex=False)
    _equal(layer.knn_indices.to(torch.int32), f"{name}__idx")
    _equal(layer.knn_distances, f"{name}__dist")
    _equal(layer.slots.to(torch.uint8), f"{name}__slots")


def test_isotropic_pool_layer_tables():
    layer = KNNPoolingLayer(9, _coords(16), _coords(8), mode="max", device="cpu")
    _equal(layer.knn_indices.to(torch.int32), "iso_16_8__idx")
    n_in = layer.in_coords.shape[0]
    assert torch.equal(layer.knn_indices_pad_mask, layer.knn_indices >= n_in)
    assert torch.all(layer.knn_indices_pad_token[layer.knn_indices_pad_mask] == n_in)


# ------------------------------------------------------------------------- GPU ---
def _gpu_layer(r_in, r_out, k, c_in, c_out, bias, seed=3):
    layer = KNNConvLayer(c_in, c_out, k, _coords(r_in), _coords(r_out), device="cuda", bias=bias)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * (1.0 / (c_in * layer._k)) ** 0.5)
        if bias:
            layer.bias.copy_(torch.randn(c_out, generator=g) * 0.1)
    return layer


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("r_in,r_out,k,c_in,c_out,bias", [
    (24, 12, 25, 3, 64, True),       # first-layer shape, many pad neighbours
    (16, 16, 9, 64, 96, False),      # stride 1, channels-last vector loader
])
def test_isotropic_knnconv_forward_backward_vs_oracle(dt, r_in, r_out, k, c_in, c_out, bias):
    layer = _gpu_layer(r_in, r_out, k, c_in, c_out, bias)
    n_in, n_out = layer.in_coords.shape[0], layer.out_coords.shape[0]
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, c_in, n_in, generator=g).to(dt)
    dy = torch.randn(3, c_out, n_out, generator=g)
    xd = x.cuda()
    if c_in % 8 == 0:
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    xd.requires_grad_(True)
    y = layer(xd)
    assert y.dtype == dt and y.shape == (3, c_out, n_out)
    y.backward(dy.to(dt).cuda())
    w = layer.weight.detach().cpu().to(dt).float()
    b = layer.bias.detach().cpu() if bias else None
    xr = x.float().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    ref = knnconv_ref.knnconv_forward(xr, layer.knn_indices.cpu(), n_in, layer.local_rf.cpu(), wr, b)
    ref.backward(dy.to(dt).float())
    tol = 1e-5 if dt == torch.float32 else 1e-2
    assert_close_rel(y.detach().float().cpu(), ref.detach(), tol, "isotropic forward")
    assert_close_rel(xd.grad.float().cpu(), xr.grad, tol, "isotropic dx")
    assert_close_rel(layer.weight.grad.cpu(), wr.grad, tol, "isotropic dW")
    # pad-ring neighbours carry no input: inputs never gathered get no gradient
    used = torch.zeros(n_in, dtype=torch.bool)
    used[layer.knn_indices[layer.knn_indices < n_in].cpu()] = True
    assert torch.all(xd.grad.float().cpu()[:, :, ~used] == 0)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["max", "avg", "sum", "gaussian"])
def test_isotropic_knnpool_vs_oracle(mode):
    layer = KNNPoolingLayer(9, _coords(16), _coords(8), mode=mode, device="cuda", gauss_sigma=3.0)
    n_in, n_out = layer.in_coords.shape[0], layer.out_coords.shape[0]
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 32, n_in, generator=g)
    dy = torch.randn(2, 32, n_out, generator=g)
    xd = x.cuda().requires_grad_(True)
    y = layer(xd)
    w = layer.gaussian_weights.cpu() if mode == "gaussian" else None
    ref = knnpool_ref.knnpool_forward(x, layer.knn_indices.cpu(), n_in, mode, w)
    got = y.detach().float().cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert_close_rel(got[ok], ref[ok], 1e-5, f"isotropic pool {mode}")
    y.backward(dy.cuda())
    xr = x.clone().requires_grad_(True)
    knnpool_ref.knnpool_forward(xr, layer.knn_indices.cpu(), n_in, mode, w).backward(dy)
    assert_close_rel(xd.grad.cpu(), xr.grad, 1e-5, f"isotropic pool backward {mode}")


# ------------------------------------------------------- the notebook's isotropic AlexNet ---
def _notebook_alexnet(device, norm_type):
    """fovi_alexnet2023 with arch_spec base_lowres as config/fovi_alexnet.yaml builds it
    (architectures.py:73-120): 64-pixel auto-matched isotropic input, a=0.5, fov 16,
    channels 96/256/384/384/256, k = 11^2/5^2/3^2/3^2/3^2, strides 2/1/1/1/1, pooling after
    blocks 0, 1 and 4, ref_frame_mult 2, one output point."""
    from fovi_amd.arch.knnalexnet import KNNAlexNet
    return KNNAlexNet(64, 3, [96, 256, 384, 384, 256], [2, 1, 1, 1, 1], [0, 1, 4], [121, 25, 9, 9, 9], out_res=1,
                      auto_match_cart_resources=1, style="isotropic", norm_type=norm_type, fov=16.0, cmf_a=0.5,
                      device=device, ref_frame_mult=2)


def _knn_layers(net):
    return [m for m in net.modules() if isinstance(m, (KNNConvLayer, KNNPoolingLayer))]


def test_notebook_alexnet_coords_per_layer():
    """step2_knnconv cell 12 prints 'Number of coords per layer: [4085, 964, 230, 230, 60,
    60, 60, 60, 16, 1]' for this network (fovinet.py:516-528: the first layer's inputs,
    then every kNN layer's outputs)."""
    layers = _knn_layers(_notebook_alexnet("cpu", "force_batch"))
    assert [len(layers[0].in_coords)] + [len(l.out_coords) for l in layers] == [4085, 964, 230, 230, 60, 60, 60,
                                                                               60, 16, 1]
    assert layers[0]._k == 121 and layers[0].ref_coords.shape[0] == 484


@pytest.mark.gpu
def test_notebook_alexnet_forward_backward_vs_oracle():
    """The notebook network (no normalisation, so the chain is kNN-conv + ReLU and kNN
    pooling only) in fp32 on the GPU. Output: against the oracles composed layer by layer
    (1e-4 relative: nine fp32 layers, each within 1e-5). Input gradient: the chain rule over
    the oracles' vector-Jacobian products, each taken at the GPU's own layer input and ReLU
    mask (a maximum or a ReLU sign decided by the last ulp would otherwise route gradient
    differently). Every parameter gets a finite gradient."""
    from fovi_amd.arch.knnalexnet import KNNAlexNetBlock
    net = _notebook_alexnet("cuda", "none")
    g = torch.Generator().manual_seed(21)
    with torch.no_grad():
        for layer in _knn_layers(net):
            if isinstance(layer, KNNConvLayer):
                c_in = layer.in_channels
                layer.weight.copy_(torch.randn(layer.weight.shape, generator=g) * (2.0 / (c_in * layer._k)) ** 0.5)
    x = torch.rand(2, 3, 4085, generator=g)
    xd = x.cuda().requires_grad_(True)
    y = net(xd)
    assert y.shape == (2, 256, 1)
    dy = torch.randn(y.shape, generator=g)
    y.backward(dy.cuda())
    for name, prm in net.named_parameters():
        assert prm.grad is not None and torch.isfinite(prm.grad).all(), name

    def conv_ref(layer, h):
        b = None if layer.bias is None else layer.bias.detach().cpu()
        return knnconv_ref.knnconv_forward(h, layer.knn_indices.cpu(), layer.in_coords.shape[0],
                                           layer.local_rf.cpu(), layer.weight.detach().cpu(), b)

    def pool_ref(layer, h):
        w = layer.gaussian_weights.cpu() if layer.mode == "gaussian" else None
        return knnpool_ref.knnpool_forward(h, layer.knn_indices.cpu(), layer.in_coords.shape[0], layer.mode, w)

    # the GPU chain step by step: (kind, layer, input, output) of every kNN layer
    steps, h = [], xd.detach()
    with torch.no_grad():
        for mod in net.layers:
            if isinstance(mod, KNNAlexNetBlock):
                out = mod.conv.forward_fused(h, "relu")
                steps.append(("conv", mod.conv, h.cpu(), out.cpu()))
                h = out
                if mod.pool is not None:
                    out = mod.pool(h)
                    steps.append(("pool", mod.pool, h.cpu(), out.cpu()))
                    h = out
            else:
                out = mod(h)
                steps.append(("pool", mod, h.cpu(), out.cpu()))
                h = out
    assert torch.equal(h.cpu(), y.detach().cpu())
    ref = x
    for kind, layer, _, _ in steps:
        ref = torch.relu(conv_ref(layer, ref)) if kind == "conv" else pool_ref(layer, ref)
    assert_close_rel(y.detach().cpu(), ref, 1e-4, "notebook AlexNet output")
    grad = dy
    for kind, layer, inp, out in reversed(steps):
        hr = inp.clone().requires_grad_(True)
        if kind == "conv":
            conv_ref(layer, hr).backward(grad * (out > 0))
        else:
            pool_ref(layer, hr).backward(grad)
        grad = hr.grad
    assert_close_rel(xd.grad.cpu(), grad, 1e-4, "notebook AlexNet input gradient")


# -------------------------------------------------------- partitioning patch embeddings ---
PATCH_LAYERS = {"part_a05": ("PartitioningPatchEmbedding", 0.5, 16),
                "kpart_a05": ("KNNPartitioningPatchEmbedding", 0.5, 16),
                "kpart_a2786": ("KNNPartitioningPatchEmbedding", 2.785765, 8)}


def _patch_layer(name, device):
    from fovi_amd.arch import knnvit
    cls, cmf_a, patch = PATCH_LAYERS[name]
    return getattr(knnvit, cls)(3, 8, 64, 16, cmf_a, in_cart_res=64, cart_patch_size=patch, device=device,
                                sample_cortex=True)


@pytest.mark.parametrize("name", list(PATCH_LAYERS))
def test_partitioning_patch_embeddings_match_reference(name):
    """k, neighbour tables (index -1 pads a partition's groups) and ref slots of the
    partitioning patch embeddings, as the reference builds them with Euclidean distances."""
    layer = _patch_layer(name, "cpu")
    assert layer._k == int(GOLDEN[f"{name}__k"])
    _equal(layer.knn_indices.to(torch.int16), f"{name}__idx")
    _equal(layer.slots.numpy().astype(np.uint16), f"{name}__slots")


def test_partition_is_a_partition():
    """Every sensor point sits in exactly one group, the group of its nearest centre; -1 only
    pads the tail of a group's column."""
    layer = _patch_layer("part_a05", "cpu")
    idx = layer.knn_indices
    n_in = len(layer.in_coords)
    real = idx[idx >= 0]
    assert torch.equal(torch.sort(real).values, torch.arange(n_in))
    nearest = torch.argmin(layer.distances[:n_in], 1)
    cols = torch.arange(idx.shape[1]).expand_as(idx)[idx >= 0]
    assert torch.equal(nearest[real], cols)
    pad = idx < 0
    assert torch.all(pad[1:] >= pad[:-1])


def test_geodesic_partitioning_raises():
    from fovi_amd.arch.knnvit import KNNPartitioningPatchEmbedding
    with pytest.raises(NotImplementedError):
        KNNPartitioningPatchEmbedding(3, 8, 64, 16, 0.5, in_cart_res=64, cart_patch_size=16, device="cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["part_a05", "kpart_a2786"])
def test_partitioning_patch_embedding_forward_vs_oracle(name):
    layer = _patch_layer(name, "cuda")
    n_in = len(layer.in_coords)
    x = torch.rand(2, 3, n_in, generator=torch.Generator().manual_seed(31))
    with torch.no_grad():
        tokens = layer(x.cuda())
    assert tokens.shape == (2, len(layer.out_coords), 8)
    ref = knnconv_ref.knnconv_forward(x, layer.knn_indices.cpu(), n_in, layer.local_rf.cpu(),
                                      layer.weight.detach().cpu())
    assert_close_rel(tokens.transpose(1, 2).cpu(), ref, 1e-5, f"{name} tokens")


def test_oracle_pads_negative_indices_like_the_pad_token():
    """-1 entries (partition padding) and pad-ring entries contribute nothing: the oracle's
    library-call form equals its float64 loop form, which skips both."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 10, generator=g)
    idx = torch.randint(0, 10, (4, 6), generator=g)
    idx[3, ::2] = -1
    idx[2, 1] = 12
    slots = torch.randint(0, 4, (6, 4), generator=g)
    rf = torch.zeros(6, 4, 4).scatter_(2, slots.unsqueeze(2), 1)
    w = torch.randn(5, 12, generator=g)
    got = knnconv_ref.knnconv_forward(x, idx, 10, rf, w)
    want = knnconv_ref.knnconv_bruteforce(x, idx, slots, 10, w)
    assert np.allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)


def test_partitioning_keeps_an_empty_group_as_padding():
    """A token centre nearest to no input point gets an all -1 column (no input), as the
    reference's partition loop leaves it (knnvit.py:176-186); the k-nearest variant refuses."""
    import types

    import torch

    from fovi_amd.arch.knnvit import PartitioningPatchEmbedding, _partition
    from fovi_amd.sensing.coords import SamplingCoords
    cin = SamplingCoords(16, 2.78, 8, style="logpolar")
    cart = torch.tensor([[0.0, 0.0], [0.5, 0.0], [5.0, 5.0]])
    cout = types.SimpleNamespace(cartesian=cart, cortical=None, polar=torch.zeros_like(cart), shape=cart.shape,
                                 style="logpolar", dtype=torch.float32)
    pe = PartitioningPatchEmbedding(3, 8, None, 16, 2.78, in_coords=cin, out_coords=cout, sample_cortex=False,
                                    device="cpu")
    idx = pe.knn_indices.cpu()
    assert idx.shape[1] == 3 and bool((idx[:, 2] == -1).all())
    covered = torch.sort(idx[:, :2][idx[:, :2] >= 0]).values
    assert torch.equal(covered, torch.arange(cin.shape[0]))
    assert int((pe.slot_ptr.cpu()[2] & 0xFFFF).sum()) == 0          # no neighbour in any slot
    with pytest.raises(ValueError, match="nearest to no input point"):
        _partition(pe.distances, cin.shape[0], 3)
