"""kNN patch embedding, drop-in for the reference ``fovi.arch.knnvit.KNNPatchEmbedding``.

A ``KNNConvLayer`` from a fine sensor grid onto a coarse grid of token
centres (reference ``fovi/arch/knnvit.py:17-98``). The DINOv3 adapter swaps
it in for the backbone's Conv2d patch embedding (``fovi/arch/dinov3.py:70-94``)
and imports the Conv2d weights with ``load_conv2d_weights``.
"""
from __future__ import annotations

import numpy as np
from einops import rearrange

from .knn import KNNConvLayer, get_in_out_coords

__all__ = ["KNNPatchEmbedding"]


class KNNPatchEmbedding(KNNConvLayer):
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
            k = int((cart_patch_size * out_cart_res / np.sqrt(len(out_coords)) * patch_overlap_factor) ** 2)
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
