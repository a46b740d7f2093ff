"""AlexNet-style kNN-CNN blocks, drop-in for ``fovi.arch.knnalexnet``.

``KNNAlexNetBlock`` = kNN-conv → norm → activation → optional kNN pooling
(reference ``fovi/arch/knnalexnet.py:13-127``). When no norm sits between
the conv and a ReLU, the ReLU is applied in the kNN-conv kernel's store.
Norms other than 'none'/'batch' are not built. ``KNNAlexNet`` chains the
blocks and the optional output average-pooling layer
(``knnalexnet.py:131-241``).
"""
from __future__ import annotations

import numpy as np
import torch.nn as nn

from ..sensing.coords import auto_match_num_coords
from .knn import KNNPoolingLayer, get_in_out_coords, get_knn_conv_layer

__all__ = ["KNNAlexNetBlock", "KNNAlexNet"]


class _KNNBatchNorm(nn.BatchNorm1d):
    """BatchNorm over the channels of ``[B, C, N]`` features."""

    def __init__(self, num_coords, num_channels, device="cuda"):
        super().__init__(num_channels, device=device)


def _get_norm(norm_type, num_coords, num_channels, device):
    if norm_type in (None, "none"):
        return None
    if "batch" in norm_type:
        return _KNNBatchNorm(num_coords, num_channels, device=device)
    raise NotImplementedError(f"norm_type {norm_type!r}: only 'none' and 'batch' are built")


class KNNAlexNetBlock(nn.Module):
    def __init__(self, in_channels, out_channels, k, fov, cmf_a, in_res, stride, style="isotropic",
                 conv_layer="default", cart_res=None, pool=True, pool_mode="max", pool_k=9, pool_stride=2,
                 norm_type="batch", arch_flag="", activation=nn.ReLU, sample_cortex=True, device="cuda",
                 auto_match_cart_resources=0, ref_frame_mult=None):
        super().__init__()
        if isinstance(conv_layer, str):
            conv_layer = get_knn_conv_layer(conv_layer)
        self.in_coords, self.out_coords, out_cart_res = get_in_out_coords(
            in_res, fov, cmf_a, stride, style=style, auto_match_cart_resources=auto_match_cart_resources,
            in_cart_res=cart_res, device=device)
        ref_side = int(np.ceil(ref_frame_mult * np.sqrt(k))) if ref_frame_mult is not None else None
        self.conv = conv_layer(in_channels=in_channels, out_channels=out_channels, k=k, in_coords=self.in_coords,
                               out_coords=self.out_coords, sample_cortex=sample_cortex, arch_flag=arch_flag,
                               device=device, ref_frame_side_length=ref_side) if conv_layer is not None else None
        self.norm = _get_norm(norm_type, self.out_coords.shape[0], out_channels, device)
        self.activation = activation() if activation is not None else None
        self.pool = None
        if pool:
            # pooled grid from the block's input resolution, as the reference builds it
            # (knnalexnet.py:90-101)
            _, pooled_coords, out_cart_res = get_in_out_coords(
                self.in_coords.resolution, fov, cmf_a, pool_stride, style=style,
                auto_match_cart_resources=auto_match_cart_resources, in_cart_res=out_cart_res, device=device)
            self.pool = KNNPoolingLayer(k=pool_k, in_coords=self.out_coords, out_coords=pooled_coords,
                                        mode=pool_mode, device=device, sample_cortex=sample_cortex)
            self.out_coords = pooled_coords
        self.out_res = self.out_coords.resolution
        self.out_cart_res = out_cart_res

    def forward(self, x):
        fused = (self.conv is not None and self.norm is None and isinstance(self.activation, nn.ReLU)
                 and hasattr(self.conv, "forward_fused"))
        if fused:
            x = self.conv.forward_fused(x, "relu")
        else:
            if self.conv is not None:
                x = self.conv(x)
            if self.norm is not None:
                x = self.norm(x)
            if self.activation is not None:
                x = self.activation(x)
        if self.pool is not None:
            x = self.pool(x)
        return x


class KNNAlexNet(nn.Module):
    def __init__(self, in_res, in_channels, features_per_layer, stride_per_layer, pool_after, k_per_layer,
                 n_classes=None, out_res=None, auto_match_cart_resources=0, style="isotropic", layer_cls="default",
                 norm_type="batch", arch_flag="", fov=16, cmf_a=0.5, device="cuda", sample_cortex=True,
                 ref_frame_mult=None, activation=nn.ReLU, final_activation=True):
        super().__init__()
        in_res, cart_res = auto_match_num_coords(fov, cmf_a, in_res, style, auto_match_cart_resources, device,
                                                 quiet=True)
        blocks = []
        for i, feats in enumerate(features_per_layer):
            act = activation if (final_activation or i + 1 < len(features_per_layer)) else None
            block = KNNAlexNetBlock(in_channels=in_channels, out_channels=feats, k=k_per_layer[i], fov=fov,
                                    cmf_a=cmf_a, in_res=in_res, stride=stride_per_layer[i], style=style,
                                    conv_layer=layer_cls, cart_res=cart_res,
                                    auto_match_cart_resources=auto_match_cart_resources, pool=i in pool_after,
                                    norm_type=norm_type, arch_flag=arch_flag, activation=act,
                                    sample_cortex=sample_cortex, device=device, ref_frame_mult=ref_frame_mult)
            in_channels, in_res, cart_res = feats, block.out_res, block.out_cart_res
            blocks.append(block)
        if out_res is not None and out_res != -1:
            # output average pooling (knnalexnet.py:193-209): a stride-1 grid of the last block's
            # points, k = (2 ceil(in_res / out_radii))^2
            in_coords = blocks[-1].out_coords
            out_coords, out_radii, cart_res = in_coords.get_strided_coords(
                1, auto_match_cart_resources=auto_match_cart_resources, in_cart_res=out_res)
            k = int(2 * np.ceil(in_res / out_radii)) ** 2
            blocks.append(KNNPoolingLayer(k=k, mode="avg", in_coords=in_coords, out_coords=out_coords,
                                          sample_cortex=sample_cortex, device=device))
        self.layers = nn.ModuleList(blocks)
        self.n_classes = n_classes
        self.out_channels = features_per_layer[-1]
        self.out_coords = self.layers[-1].out_coords
        self.total_embed_dim = self.out_channels * self.out_coords.shape[0]
        if n_classes is not None:
            self.classifier = nn.Linear(self.total_embed_dim, n_classes, device=device)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        if self.n_classes is not None:
            x = self.classifier(x.reshape(x.shape[0], -1))
        return x
