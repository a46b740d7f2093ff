"""The drop-in boundary: the reference's registry path with its own coords objects, and the
Conv2d weight import (reference ``knn.py:649-715``) that DINOv3 uses for pretrained patch
weights (``dinov3.py:88-91``).

The registry snippet is read from the repository's integration guide (the block between its
registry-snippet markers) and executed as written, with stand-ins
for the two reference modules it imports (``fovi.arch.knn``: ``KNNBaseLayer``,
``KNN_CONV_REGISTRY``, ``get_knn_conv_layer`` as ``knn.py:1007-1030`` defines them;
``fovi.arch.knnalexnet``) and coords given as a plain namespace of the reference-written
vectors (``tests/golden/tables.npz``). Conv2d import pins are geometric known answers: a
Conv2d tap at (row r, column c) is the ref point at x = lin[c], y = -lin[r] (image rows
grow downwards, the ref grid's y upwards), and bilinear resampling with
``align_corners=True`` reproduces a kernel that is linear in (row, column) exactly.
"""
import os
import re
import sys
import types

import numpy as np
import pytest
import torch
import torch.nn as nn

from fovi_amd.arch import knn_tables as T
from fovi_amd.arch.knn import KNNConvLayer, KNNPoolingLayer
from fovi_amd.sensing.coords import SamplingCoords

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")
GOLDEN = np.load(os.path.join(ROOT, "tests", "golden", "tables.npz"))


def _registry_snippet():
    text = open(GUIDE).read()
    m = re.search(r"<!-- registry-snippet -->\s*```python\n(.*?)```\s*<!-- /registry-snippet -->", text, re.S)
    assert m, f"{GUIDE} lost its registry snippet"
    return m.group(1)


def _reference_stand_ins(monkeypatch):
    """Module objects shaped like the reference's fovi.arch.knn / fovi.arch.knnalexnet."""
    ref_knn = types.ModuleType("fovi.arch.knn")

    class KNNBaseLayer:
        # the reference's mixin defines these; the drop-in's own must take precedence
        def _compute_knns(self, batch_size=None):
            raise AssertionError("the reference's _compute_knns was called")

        def _compute_euclidean_distances_batched(self, batch_size):
            raise AssertionError("the reference's distance search was called")

    ref_knn.KNNBaseLayer = KNNBaseLayer
    ref_knn.KNN_CONV_REGISTRY = {"default": object}

    def get_knn_conv_layer(name):
        if name not in ref_knn.KNN_CONV_REGISTRY:
            raise ValueError(f"Unknown KNN conv layer: {name}")
        return ref_knn.KNN_CONV_REGISTRY[name]

    ref_knn.get_knn_conv_layer = get_knn_conv_layer
    ref_alex = types.ModuleType("fovi.arch.knnalexnet")
    ref_alex.KNNPoolingLayer = object
    fovi = types.ModuleType("fovi")
    arch = types.ModuleType("fovi.arch")
    fovi.arch, arch.knn, arch.knnalexnet = arch, ref_knn, ref_alex
    for name, mod in (("fovi", fovi), ("fovi.arch", arch), ("fovi.arch.knn", ref_knn),
                      ("fovi.arch.knnalexnet", ref_alex)):
        monkeypatch.setitem(sys.modules, name, mod)
    return ref_knn, ref_alex


def _golden_coords(tag):
    """Plain namespace with the reference SamplingCoords attributes of a stride-1 golden
    layer geometry (output points = input points)."""
    cart = torch.from_numpy(GOLDEN[f"{tag}__in_cartesian"])
    cort = torch.from_numpy(GOLDEN[f"{tag}__in_cortical"])
    return types.SimpleNamespace(shape=cart.shape, style="logpolar", cartesian=cart, cortical=cort,
                                 dtype=torch.float32, resolution=int(round(cart.shape[0] ** 0.5)))


def _run_snippet(monkeypatch, device, tag="c2_l3", c_in=192, c_out=384, k=9):
    ref_knn, ref_alex = _reference_stand_ins(monkeypatch)
    coords = _golden_coords(tag)
    env = {"in_channels": c_in, "out_channels": c_out, "k": k, "in_coords": coords, "out_coords": coords,
           "device": device}
    exec(compile(_registry_snippet(), GUIDE, "exec"), env)
    return env, ref_knn, ref_alex, coords


def test_registry_snippet_builds_reference_identical_tables(monkeypatch):
    env, ref_knn, ref_alex, coords = _run_snippet(monkeypatch, "cpu")
    conv = env["conv"]
    assert isinstance(conv, KNNConvLayer) and isinstance(conv, ref_knn.KNNBaseLayer)
    assert ref_knn.KNN_CONV_REGISTRY["mi355x"] is env["conv_cls"]
    # FoviNet.list_knn_layers (fovinet.py:504-514) walks modules() with this isinstance test
    net = nn.Sequential(nn.Identity(), conv)
    assert [m for m in net.modules() if isinstance(m, ref_knn.KNNBaseLayer)] == [conv]
    # tables from the reference's coords equal the reference-written ones bit for bit
    assert np.array_equal(conv.knn_indices.numpy(), GOLDEN["c2_l3__idx"].astype(np.int64))
    assert np.array_equal(conv.slots.numpy(), GOLDEN["c2_l3__slots"].astype(np.int64))
    # the blocks' pooling layer is the kernel-backed one, and it takes the same coords
    assert ref_alex.KNNPoolingLayer is env["pool_cls"]
    pool = ref_alex.KNNPoolingLayer(k=9, in_coords=coords, out_coords=coords, mode="max", device="cpu")
    assert isinstance(pool, KNNPoolingLayer) and isinstance(pool, ref_knn.KNNBaseLayer)
    assert torch.equal(pool.knn_indices.cpu(), conv.knn_indices.cpu())
    # state dicts are the reference layer's: weight [C_out, C_in * V] and no bias
    assert list(conv.state_dict()) == ["weight"] and conv.weight.shape == (384, 192 * 9)


def test_coords_without_reference_attributes_are_rejected():
    c = types.SimpleNamespace(shape=(16, 2), cartesian=torch.zeros(16, 2))
    with pytest.raises(TypeError, match="style"):
        KNNConvLayer(4, 8, 9, c, c, device="cpu")


# --- Conv2d weight import (knn.py:649-715) -----------------------------------------------------

def _cpu_layer(side, c_in=2, c_out=3, bias=False):
    coords = SamplingCoords(16, 2.78, 16, style="logpolar")
    return KNNConvLayer(c_in, c_out, side * side, coords, coords, device="cpu", bias=bias,
                        ref_frame_side_length=side)


@pytest.mark.parametrize("side", [3, 5, 16])
def test_conv2d_tap_lands_on_its_ref_point(side):
    """A one-hot Conv2d tap at (row r, column c) of input channel ci lands in the weight
    column ci * V + v of the ref point at x = lin[c], y = -lin[r] (lin = linspace(-1, 1, s))."""
    layer = _cpu_layer(side)
    lin = torch.linspace(-1, 1, side)
    ref = layer.ref_coords.cpu()
    V = side * side
    rng = np.random.default_rng(0)
    cases = [(0, 0, 0), (1, side - 1, 0), (0, 0, side - 1), (1, side - 1, side - 1)]
    cases += [(int(rng.integers(2)), int(rng.integers(side)), int(rng.integers(side))) for _ in range(6)]
    for ci, r, c in cases:
        conv = nn.Conv2d(2, 3, side, bias=False)
        with torch.no_grad():
            conv.weight.zero_()
            conv.weight[1, ci, r, c] = 1.0
        layer.load_conv2d_weights(conv, strict=True)
        w = layer.weight.detach()
        nz = torch.nonzero(w)
        assert nz.shape[0] == 1 and int(nz[0, 0]) == 1, (ci, r, c)
        col = int(nz[0, 1])
        assert col // V == ci
        v = col % V
        assert torch.equal(ref[v], torch.stack([lin[c], -lin[r]])), (ci, r, c, v, ref[v])


def test_conv2d_resample_reproduces_a_linear_kernel():
    """A 7x7 kernel W[r, c] = a r + b c + d, bilinearly resampled (align_corners=True) to the
    3x3 ref grid, equals the same linear function at the ref points' pixel positions:
    column (x + 1) / 2 * 6, row (1 - y) / 2 * 6."""
    layer = _cpu_layer(3, c_in=1, c_out=1)
    n, a, b, d = 7, 0.25, -0.75, 0.125
    rr, cc = torch.meshgrid(torch.arange(n, dtype=torch.float32), torch.arange(n, dtype=torch.float32),
                            indexing="ij")
    conv = nn.Conv2d(1, 1, n, bias=False)
    with torch.no_grad():
        conv.weight.copy_((a * rr + b * cc + d)[None, None])
    layer.load_conv2d_weights(conv)
    ref = layer.ref_coords.cpu().double()
    want = a * (1 - ref[:, 1]) / 2 * (n - 1) + b * (ref[:, 0] + 1) / 2 * (n - 1) + d
    assert torch.allclose(layer.weight.detach()[0].double(), want, atol=1e-6)
    with pytest.raises(ValueError, match="ref_grid_size"):
        layer.load_conv2d_weights(conv, strict=True)


def test_conv2d_bias_and_conv3d_strategies():
    layer = _cpu_layer(3, c_in=2, c_out=3, bias=True)
    conv = nn.Conv2d(2, 3, 3, bias=True)
    layer.load_conv2d_weights(conv)
    assert torch.equal(layer.bias.detach(), conv.bias.detach())
    nobias = _cpu_layer(3, c_in=2, c_out=3, bias=False)
    with pytest.raises(ValueError, match="bias"):
        nobias.load_conv2d_weights(conv)
    c3 = nn.Conv3d(2, 3, (4, 3, 3), bias=False)
    ref_mean = nn.Conv2d(2, 3, 3, bias=False)
    ref_first = nn.Conv2d(2, 3, 3, bias=False)
    with torch.no_grad():
        ref_mean.weight.copy_(c3.weight.mean(2))
        ref_first.weight.copy_(c3.weight[:, :, 0])
    for strategy, ref in (("average", ref_mean), ("select_first", ref_first)):
        a, b = _cpu_layer(3, 2, 3), _cpu_layer(3, 2, 3)
        a.load_conv3d_weights(c3, temporal_strategy=strategy)
        b.load_conv2d_weights(ref)
        assert torch.equal(a.weight, b.weight)


def test_conv2d_import_bumps_the_weight_version():
    """The packed weight caches are keyed on the parameter's version: the import must bump it
    (a .data copy would not) and drop the packed copies."""
    layer = _cpu_layer(3)
    v0 = layer.weight._version
    layer._packed[("probe", 0)] = "stale"
    layer.load_conv2d_weights(nn.Conv2d(2, 3, 3, bias=False))
    assert layer.weight._version > v0 and not layer._packed


# --- GPU: the registry path and the import end to end -------------------------------------------

def _oracle_from_golden(tag, x, w, b=None, V=9):
    from oracle import knnconv_ref
    idx = torch.from_numpy(GOLDEN[f"{tag}__idx"].astype(np.int64))
    rf = T.slots_to_one_hot(torch.from_numpy(GOLDEN[f"{tag}__slots"].astype(np.int64)), V)
    return knnconv_ref.knnconv_forward(x.float().cpu(), idx, idx.shape[1], rf, w, b)


@pytest.mark.gpu
def test_registry_snippet_layer_forward_matches_oracle(monkeypatch):
    from tests.helpers import assert_close_rel
    env, ref_knn, _, _ = _run_snippet(monkeypatch, "cuda")
    conv = env["conv"]
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) / (192 * 9) ** 0.5)
    x = torch.randn(3, 192, 256, generator=g)
    w = conv.weight.detach().cpu()
    with torch.no_grad():
        y32 = conv(x.cuda())
        xb = x.bfloat16()
        y16 = conv(xb.cuda().transpose(1, 2).contiguous().transpose(1, 2))
    from oracle import knnconv_ref
    idx, rf = conv.knn_indices.cpu(), conv.local_rf.cpu()
    assert_close_rel(y32.cpu(), knnconv_ref.knnconv_forward(x, idx, 256, rf, w), 1e-5, "fp32 via the registry")
    assert_close_rel(y16.float().cpu(), knnconv_ref.knnconv_forward(xb.float(), idx, 256, rf, w.bfloat16().float()),
                     1e-2, "bf16 via the registry")
    d_idx = int((idx.numpy() != GOLDEN["c2_l3__idx"].astype(np.int64)).sum())
    d_slot = int((conv.slots.numpy() != GOLDEN["c2_l3__slots"].astype(np.int64)).sum())
    print(f"tables vs the reference-written ones on this host: {d_idx} indices, {d_slot} slots differ", flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("c_in,c_out", [(64, 96), (256, 256)])
def test_forward_after_conv2d_import_uses_the_new_weights(c_in, c_out):
    """forward -> load_conv2d_weights -> forward: the second output follows the imported
    weights (row-packed kernel at 64 -> 96, fragment-order kernel at 256 -> 256)."""
    from oracle import knnconv_ref
    from tests.helpers import assert_close_rel
    coords = SamplingCoords(16, 2.78, 16, style="logpolar")
    layer = KNNConvLayer(c_in, c_out, 9, coords, coords, device="cuda", bias=True)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, c_in, 256, generator=g).bfloat16()
    xd = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        layer(xd)
        conv = nn.Conv2d(c_in, c_out, 3, bias=True)
        layer.load_conv2d_weights(conv)
        y = layer(xd)
    w = layer.weight.detach().cpu().bfloat16().float()
    ref = knnconv_ref.knnconv_forward(x.float(), layer.knn_indices.cpu(), 256, layer.local_rf.cpu(), w,
                                      layer.bias.detach().cpu())
    assert_close_rel(y.float().cpu(), ref, 1e-2, "after load_conv2d_weights")
