"""kNN patch embeddings, drop-ins for the reference ``fovi.arch.knnvit`` ones.

``KNNPatchEmbedding``: a ``KNNConvLayer`` from a fine sensor grid onto a coarse
grid of token centres (reference ``fovi/arch/knnvit.py:17-98``). The DINOv3
adapter swaps it in for the backbone's Conv2d patch embedding
(``fovi/arch/dinov3.py:70-94``) and imports the Conv2d weights with
``load_conv2d_weights``. ``PartitioningPatchEmbedding`` (``knnvit.py:102-220``)
gives every input point to its nearest token centre and pads the groups with
index -1 to the largest; ``KNNPartitioningPatchEmbedding``
(``knnvit.py:224-290``) takes k = the most points any centre has nearer than the
farthest point of its group. Both run the same kernels as any kNN-conv layer
(pad and -1 entries carry no input). Their constructors compute Euclidean
distances; the reference's default ``sample_cortex='geodesic'`` needs pygeodesic
and raises here. ``from_reference`` (or ``from_tables``) instead runs a layer the
reference built, geodesic tables included, on the kernels.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn
from einops import rearrange

from .knn import KNNConvLayer, get_in_out_coords

__all__ = ["KNNPatchEmbedding", "PartitioningPatchEmbedding", "KNNPartitioningPatchEmbedding"]


def _partition(distances, n_in, n_out, allow_empty=False):
    """Nearest token centre of every input point (first index on ties), from the distance
    rows of the sensor points (the pad ring takes no part). A centre nearest to no point has
    an empty group: ``PartitioningPatchEmbedding`` gives it an all -1 column, as the
    reference does (``knnvit.py:176-186``); ``KNNPartitioningPatchEmbedding`` cannot size its
    neighbourhood (the reference fails on the empty group's ``max``, ``knnvit.py:272-276``)."""
    part = torch.argmin(distances[:n_in], 1)
    sizes = torch.bincount(part, minlength=n_out)
    if not allow_empty and int(sizes.min()) == 0:
        raise ValueError("a token centre is nearest to no input point")
    return part, sizes


class KNNPatchEmbedding(KNNConvLayer):
    # [B, C, N] tokens when set, else [B, N, C] (reference ``knnvit.py:86-95``)
    transposed = False

    def __init__(self, in_channels, embed_dim, in_res, fov, cmf_a, style="isotropic",
                 auto_match_cart_resources=True, in_cart_res=224, cart_patch_size=16, patch_overlap_factor=1,
                 device="cuda", force_patches_less_than_matched=True, new_parameterization=False,
                 transposed=False, max_coord_val=1, sample_cortex="geodesic", ref_frame_side_length=None,
                 **kwargs):
        if new_parameterization:
            # k fixed to the patch area; the token grid stride follows the overlap factor
            stride = cart_patch_size / patch_overlap_factor
            if float(stride).is_integer():
                stride = int(stride)
            k = cart_patch_size ** 2
        else:
            stride = cart_patch_size
        in_coords, out_coords, out_cart_res = get_in_out_coords(
            in_res, fov, cmf_a, stride, style=style, auto_match_cart_resources=auto_match_cart_resources,
            in_cart_res=in_cart_res, device=device, force_out_match_less_than=force_patches_less_than_matched,
            max_out_coord_val=max_coord_val)
        if not new_parameterization:
            if out_cart_res is None:
                raise ValueError("k from the patch size needs a matched cartesian resolution "
                                 "(auto_match_cart_resources with in_cart_res) or new_parameterization=True")
            k = int((cart_patch_size * out_cart_res / np.sqrt(out_coords.shape[0]) * patch_overlap_factor) ** 2)
        super().__init__(in_channels, embed_dim, k, in_coords, out_coords, device=device,
                         sample_cortex=sample_cortex, ref_frame_side_length=ref_frame_side_length, **kwargs)
        self.transposed = transposed

    def forward(self, x):
        if x.dim() == 4:
            x = rearrange(x, "b n h w -> b n (h w)")
        tokens = super().forward(x)
        return tokens if self.transposed else tokens.transpose(1, 2)

    def __repr__(self):
        return super().__repr__().replace("KNNConvLayer", "KNNPatchEmbedding")


class PartitioningPatchEmbedding(KNNPatchEmbedding):
    """Patches that partition the sensor: each token centre takes the input points nearest
    to it, in increasing index order, padded with -1 up to the largest group (reference
    ``knnvit.py:102-220``)."""

    def __init__(self, in_channels, embed_dim, in_res, fov, cmf_a, style="isotropic", auto_match_cart_resources=True,
                 force_patches_less_than_matched=True, in_cart_res=224, cart_patch_size=16, device="cuda",
                 transposed=False, max_coord_val=1, ref_frame_side_length=None, sample_cortex="geodesic", bias=False,
                 arch_flag="", in_coords=None, out_coords=None):
        nn.Module.__init__(self)
        if in_coords is not None or out_coords is not None:
            assert in_coords is not None and out_coords is not None, \
                "in_coords and out_coords must be provided if provided"
        else:
            in_coords, out_coords, _ = get_in_out_coords(
                in_res, fov, cmf_a, cart_patch_size, style=style, auto_match_cart_resources=auto_match_cart_resources,
                in_cart_res=in_cart_res, device=device, force_out_match_less_than=force_patches_less_than_matched,
                max_out_coord_val=max_coord_val)
        self.in_channels, self.out_channels = in_channels, embed_dim
        self.in_coords, self.out_coords = in_coords, out_coords
        self.device, self.arch_flag, self.sample_cortex = device, arch_flag, sample_cortex
        self.ref_frame_side_length = ref_frame_side_length
        self.batch_size = None
        n_in, n_out = in_coords.shape[0], out_coords.shape[0]
        self.k = int(n_in / n_out)
        self.distances = self._compute_all_distances()
        self.partitioning, sizes = _partition(self.distances, n_in, n_out, allow_empty=True)
        max_len = int(sizes.max())
        # rows of each group in increasing input index, -1 below
        order = torch.argsort(self.partitioning, stable=True)
        col = self.partitioning[order]
        row = torch.arange(n_in) - (torch.cumsum(sizes, 0) - sizes)[col]
        indices = torch.full((max_len, n_out), -1, dtype=torch.long)
        indices[row, col] = order
        self.knn_pad_index_token_val = -1
        self.knn_pad_token_val = n_in
        self.k = torch.tensor(max_len)
        self._k = max_len
        # parameters are initialised on the host, as the reference creates them
        self._setup(indices, None, bias, param_device="cpu")
        self.transposed = transposed

    def __repr__(self):
        return super().__repr__().replace("KNNPatchEmbedding", "PartitioningPatchEmbedding")


class KNNPartitioningPatchEmbedding(KNNPatchEmbedding):
    """k-nearest-neighbour patches sized by a partition: k is the largest number of points
    (pad ring included) any token centre has strictly nearer than the farthest point of its
    own group (reference ``knnvit.py:224-290``); the layer is then a plain kNN-conv layer."""

    def __init__(self, in_channels, embed_dim, in_res, fov, cmf_a, style="isotropic", auto_match_cart_resources=True,
                 in_cart_res=224, cart_patch_size=16, device="cuda", force_patches_less_than_matched=True,
                 transposed=False, max_coord_val="auto", sample_cortex="geodesic", **kwargs):
        in_coords, out_coords, _ = get_in_out_coords(
            in_res, fov, cmf_a, cart_patch_size, style=style, auto_match_cart_resources=auto_match_cart_resources,
            in_cart_res=in_cart_res, device=device, force_out_match_less_than=force_patches_less_than_matched,
            max_out_coord_val=max_coord_val)
        nn.Module.__init__(self)
        self.in_coords, self.out_coords, self.sample_cortex = in_coords, out_coords, sample_cortex
        n_in, n_out = in_coords.shape[0], out_coords.shape[0]
        distances = self._compute_all_distances()
        part, _ = _partition(distances, n_in, n_out)
        own = distances[torch.arange(n_in), part]
        far = torch.full((n_out,), -float("inf"), dtype=distances.dtype).scatter_reduce(0, part, own, "amax")
        k = int((distances < far.unsqueeze(0)).sum(0).max())
        KNNConvLayer.__init__(self, in_channels, embed_dim, k, in_coords, out_coords, device=device,
                              sample_cortex=sample_cortex, **kwargs)
        self.distances = distances
        self.transposed = transposed

    def __repr__(self):
        return super().__repr__().replace("KNNPatchEmbedding", "KNNPartitioningPatchEmbedding")
