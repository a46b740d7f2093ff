"""Writes tests/golden/tables.npz: sensor coordinates, neighbour indices and ref-slot
assignments computed by the reference itself (nblauch/fovi, read from
/root/reference), for the log-polar layer geometries of the benchmark configs.

Run only in the build container, where the reference checkout exists:

    python tests/golden/make_golden.py               # tables.npz (log-polar layers)
    python tests/golden/make_golden.py --isotropic   # isotropic.npz (isotropic sensor)
    python tests/golden/make_golden.py --dinov3      # dinov3.npz (the DINOv3 adapter's patch embeddings)

The reference is loaded by file path under a synthetic package name; the two
modules it imports that are absent here and unused on this path (trimesh in
fovi/sensing/manifold.py:3, skimage in fovi/utils/__init__.py:10) are replaced
by empty stand-in modules, and fovi/__init__.py (training-stack imports) is
bypassed. These vectors pin what no closed form does: the tie order of topk at
the log-polar angle seam (fovi/arch/knn.py:137-146) and the argmin of
near-equidistant ref slots (knn.py:637-642). The GPU box never runs this file.
"""
import hashlib
import importlib.util
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference/fovi"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tables.npz")

# name -> (res_in, res_out, k, ref_frame_side_length); fov 16, cmf_a 2.78 (the benchmark configs)
CONFIGS = {
    "c1": (64, 64, 9, None),
    "c2_l1": (64, 32, 49, None),
    "c2_l2": (32, 16, 25, None),
    "c2_l3": (16, 16, 9, None),
    "ragged": (24, 12, 30, None),
    "c4_patch": (128, 16, 256, 16),
    "c3": (128, 128, 25, None),     # stored as digests plus the seam columns
}
FULL_LIMIT = 60_000                  # k * n_out above this: digest + seam subset only


def _load(name, path, package):
    spec = importlib.util.spec_from_file_location(name, path, submodule_search_locations=package)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_reference():
    for stub in ("trimesh", "skimage", "skimage.measure"):
        sys.modules.setdefault(stub, types.ModuleType(stub))
    sys.modules["skimage.measure"].EllipseModel = object
    root = types.ModuleType("fovi_ref")
    root.__path__ = []
    sys.modules["fovi_ref"] = root
    _load("fovi_ref.utils", os.path.join(REF, "utils", "__init__.py"), [os.path.join(REF, "utils")])
    for pkg in ("sensing", "arch"):
        m = types.ModuleType(f"fovi_ref.{pkg}")
        m.__path__ = []
        sys.modules[f"fovi_ref.{pkg}"] = m
    _load("fovi_ref.sensing.manifold", os.path.join(REF, "sensing", "manifold.py"), None)
    coords = _load("fovi_ref.sensing.coords", os.path.join(REF, "sensing", "coords.py"), None)
    knn = _load("fovi_ref.arch.knn", os.path.join(REF, "arch", "knn.py"), None)
    return coords, knn


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    coords_mod, knn_mod = load_reference()
    torch.manual_seed(0)
    out = {"torch_version": np.array(torch.__version__)}
    for name, (r_in, r_out, k, side) in CONFIGS.items():
        cin = coords_mod.SamplingCoords(16, 2.78, r_in, device="cpu", style="logpolar")
        cout = coords_mod.SamplingCoords(16, 2.78, r_out, device="cpu", style="logpolar")
        layer = knn_mod.KNNConvLayer(1, 1, k, cin, cout, device="cpu", ref_frame_side_length=side)
        idx = layer.knn_indices.numpy().astype(np.int32)                  # [k, n_out]
        rf = layer.local_rf.numpy()                                       # [n_out, k, V] one-hot
        assert np.all(rf.sum(2) == 1), "every neighbour has exactly one slot"
        slots = rf.argmax(2).astype(np.uint8)                             # [n_out, k]
        out[f"{name}__in_cartesian"] = cin.cartesian.numpy()
        out[f"{name}__in_cortical"] = cin.cortical.numpy()
        out[f"{name}__out_cortical"] = cout.cortical.numpy()
        out[f"{name}__ref_coords"] = layer.ref_coords.numpy()
        out[f"{name}__idx_sha256"] = np.array(digest(idx))
        out[f"{name}__slots_sha256"] = np.array(digest(slots))
        if cin.cartesian.shape[0] > 4096:        # large point sets: coordinates as digests
            for key in ("in_cartesian", "in_cortical"):
                out[f"{name}__{key}"] = np.array(digest(out[f"{name}__{key}"]))
        if idx.size <= FULL_LIMIT:
            out[f"{name}__idx"] = idx.astype(np.int16)
            out[f"{name}__slots"] = slots
        else:
            ang = np.arange(r_out * r_out) % r_out
            cols = np.flatnonzero((ang <= 1) | (ang >= r_out - 2))       # both sides of the angle seam
            out[f"{name}__seam_cols"] = cols.astype(np.int32)
            out[f"{name}__idx_seam"] = idx[:, cols].astype(np.int16)
            out[f"{name}__slots_seam"] = slots[cols]
            out[f"{name}__out_cortical"] = np.array(digest(out[f"{name}__out_cortical"]))
        print(f"{name}: k={k} n_out={idx.shape[1]} V={rf.shape[2]}", flush=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT) / 1024:.0f} KiB)")


# isotropic sensor (the reference's default style): point sets, pad rings and layers
ISO_RES = (8, 16, 24)
ISO_LAYERS = {"iso_16_8": (16, 8, 9), "iso_24_12": (24, 12, 25), "iso_16_16": (16, 16, 9)}
# visual-field neighbourhoods (sample_cortex=False): name -> (style, res_in, res_out, k)
VIS_LAYERS = {"vis_iso_16_8": ("isotropic", 16, 8, 9), "vis_lp_16_8": ("logpolar", 16, 8, 9)}
# pad rings of the other styles: name -> (style, res)
PAD_RINGS = {"pad_logpolar16": ("logpolar", 16), "pad_uniform8": ("uniform", 8)}
# partitioning patch embeddings: name -> (class, cmf_a, cart_patch_size); 64-pixel input grid
PATCH_LAYERS = {"part_a05": ("PartitioningPatchEmbedding", 0.5, 16),
                "kpart_a05": ("KNNPartitioningPatchEmbedding", 0.5, 16),
                "kpart_a2786": ("KNNPartitioningPatchEmbedding", 2.785765, 8)}
ISO_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "isotropic.npz")


def main_isotropic():
    """Writes tests/golden/isotropic.npz: the 'isotropic' SamplingCoords attributes (its 3-D
    cortical manifold, fovi/sensing/manifold.py:14-215,347-375, and pad ring, coords.py:68-87),
    the neighbour / slot tables of isotropic layers (the 3-D cdist branch of knn.py:101-152
    with pad tokens, and knn.py:599-647), of visual-field layers (sample_cortex=False,
    knn.py:117-119,620-647), the pad rings of the log-polar and uniform styles and seeded
    'isotropic_fixn' sensors (coords.py:224-258) and the tables of the partitioning patch
    embeddings (knnvit.py:102-290, Euclidean distances)."""
    coords_mod, knn_mod = load_reference()
    out = {"torch_version": np.array(torch.__version__), "numpy_version": np.array(np.__version__)}
    for res in ISO_RES:
        c = coords_mod.SamplingCoords(16, 2.78, res, device="cpu", style="isotropic")
        for key in ("cartesian", "polar", "plotting", "cortical", "cartesian_pad_coords", "cortical_pad_coords"):
            out[f"res{res}__{key}"] = getattr(c, key).numpy()
        print(f"isotropic res {res}: {c.cartesian.shape[0]} points, {c.cartesian_pad_coords.shape[0]} pad points",
              flush=True)
    for name, (r_in, r_out, k) in ISO_LAYERS.items():
        cin = coords_mod.SamplingCoords(16, 2.78, r_in, device="cpu", style="isotropic")
        cout = coords_mod.SamplingCoords(16, 2.78, r_out, device="cpu", style="isotropic")
        layer = knn_mod.KNNConvLayer(1, 1, k, cin, cout, device="cpu")
        rf = layer.local_rf.numpy()
        assert np.all(rf.sum(2) == 1)
        out[f"{name}__idx"] = layer.knn_indices.numpy().astype(np.int32)
        out[f"{name}__dist"] = layer.knn_distances.numpy()
        out[f"{name}__slots"] = rf.argmax(2).astype(np.uint8)
        print(f"{name}: k={k} n_in={cin.cartesian.shape[0]} n_out={cout.cartesian.shape[0]} "
              f"pads used {int((layer.knn_indices >= cin.cartesian.shape[0]).sum())}", flush=True)
    for name, (style, r_in, r_out, k) in VIS_LAYERS.items():
        cin = coords_mod.SamplingCoords(16, 2.78, r_in, device="cpu", style=style)
        cout = coords_mod.SamplingCoords(16, 2.78, r_out, device="cpu", style=style)
        layer = knn_mod.KNNConvLayer(1, 1, k, cin, cout, device="cpu", sample_cortex=False)
        rf = layer.local_rf.numpy()
        assert np.all(rf.sum(2) == 1)
        out[f"{name}__idx"] = layer.knn_indices.numpy().astype(np.int32)
        out[f"{name}__dist"] = layer.knn_distances.numpy()
        out[f"{name}__slots"] = rf.argmax(2).astype(np.uint8)
        print(f"{name}: pads used {int((layer.knn_indices >= cin.cartesian.shape[0]).sum())}", flush=True)
    for name, (style, res) in PAD_RINGS.items():
        out[name] = coords_mod.SamplingCoords(16, 2.78, res, device="cpu", style=style).cartesian_pad_coords.numpy()
    # 'isotropic_fixn': the point count fixed to res**2 by seeded random angle moves
    for seed, res in ((0, 16), (1, 24)):
        np.random.seed(seed)
        c = coords_mod.SamplingCoords(16, 2.78, res, device="cpu", style="isotropic_fixn")
        for key in ("cartesian", "polar", "cortical"):
            out[f"fixn{res}__{key}"] = getattr(c, key).numpy()
        print(f"isotropic_fixn res {res} (seed {seed}): {c.cartesian.shape[0]} points", flush=True)
    # a scaled sensor (max_val below 1) and the auto-matched strided pair of the default style
    c = coords_mod.SamplingCoords(16, 2.78, 16, device="cpu", style="isotropic", max_val=0.9)
    for key in ("cartesian", "plotting", "cortical", "cartesian_pad_coords", "cortical_pad_coords"):
        out[f"scaled16__{key}"] = getattr(c, key).numpy()
    cin, cout, out_cart_res = knn_mod.get_in_out_coords(None, 16, 2.78, 2, style="isotropic", in_cart_res=32,
                                                        device="cpu", max_out_coord_val="auto")
    out["auto__resolutions"] = np.array([cin.resolution, cout.resolution, out_cart_res])
    for key in ("cartesian", "cortical"):
        out[f"auto__in_{key}"] = getattr(cin, key).numpy()
        out[f"auto__out_{key}"] = getattr(cout, key).numpy()
    print(f"auto-matched isotropic pair: res {cin.resolution} -> {cout.resolution}, "
          f"{cin.cartesian.shape[0]} -> {cout.cartesian.shape[0]} points", flush=True)
    # partitioning patch embeddings (Euclidean cortical distances; knnvit.py:102-290)
    _load("fovi_ref.arch.vit", os.path.join(REF, "arch", "vit.py"), None)
    vit_mod = _load("fovi_ref.arch.knnvit", os.path.join(REF, "arch", "knnvit.py"), None)
    for name, (cls, cmf_a, patch) in PATCH_LAYERS.items():
        layer = getattr(vit_mod, cls)(3, 8, 64, 16, cmf_a, in_cart_res=64, cart_patch_size=patch, device="cpu",
                                      sample_cortex=True)
        rf = layer.local_rf.numpy()
        assert np.all(rf.sum(2) == 1)
        out[f"{name}__k"] = np.array(int(layer._k))
        out[f"{name}__idx"] = layer.knn_indices.numpy().astype(np.int16)
        out[f"{name}__slots"] = rf.argmax(2).astype(np.uint16)
        print(f"{name}: k={layer._k} n_in={len(layer.in_coords)} n_out={len(layer.out_coords)}", flush=True)
    np.savez_compressed(ISO_OUT, **out)
    print(f"wrote {ISO_OUT} ({os.path.getsize(ISO_OUT) / 1024:.0f} KiB)")


# the DINOv3 adapter's patch embedding as config/fovi-dinov3.yaml and
# config/pretrained_model/dinov3_lora_layers-1012345.yaml configure it (fovi/arch/dinov3.py:50-91):
# 64-pixel isotropic sensor, fov 16, cmf_a 2.785765, 8-pixel patches, 16x16 ref grid (the
# backbone's patch size), ViT-S width 384, bias, transposed tokens. sample_cortex is True
# (Euclidean cortical distances): the shipped 'geodesic' needs pygeodesic, absent here.
DINOV3_ARGS = dict(in_channels=3, embed_dim=384, in_res=64, fov=16.0, cmf_a=2.785765, style="isotropic",
                   auto_match_cart_resources=True, in_cart_res=64, max_coord_val="auto", device="cpu",
                   arch_flag="", sample_cortex=True, force_patches_less_than_matched=False,
                   ref_frame_side_length=16, transposed=True, bias=True, cart_patch_size=8)
DINOV3_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dinov3.npz")


def main_dinov3():
    """Writes tests/golden/dinov3.npz: the sensors' ``cartesian_rowcol`` (coords.py:41-42, the
    RoPE positions of dinov3.py:97, kept in the dtype the reference leaves them in) and the
    tables of the adapter's patch embeddings in the shipped configuration ('KNN' partitioning
    patches, knnvit.py:224-290, and the plain partitioning, knnvit.py:102-220)."""
    coords_mod, knn_mod = load_reference()
    _load("fovi_ref.arch.vit", os.path.join(REF, "arch", "vit.py"), None)
    vit_mod = _load("fovi_ref.arch.knnvit", os.path.join(REF, "arch", "knnvit.py"), None)
    out = {"torch_version": np.array(torch.__version__)}
    for style, res in (("logpolar", 16), ("isotropic", 16), ("uniform", 8)):
        c = coords_mod.SamplingCoords(16, 2.78, res, device="cpu", style=style)
        out[f"rowcol_{style}{res}"] = c.cartesian_rowcol.numpy()
        print(f"{style} {res}: cartesian_rowcol {tuple(c.cartesian_rowcol.shape)} {c.cartesian_rowcol.dtype}",
              flush=True)
    for name, cls in (("dino_kpart", "KNNPartitioningPatchEmbedding"), ("dino_part", "PartitioningPatchEmbedding")):
        torch.manual_seed(0)
        layer = getattr(vit_mod, cls)(**DINOV3_ARGS)
        rf = layer.local_rf.numpy()
        assert np.all(rf.sum(2) == 1)
        out[f"{name}__k"] = np.array(int(layer._k))
        out[f"{name}__idx"] = layer.knn_indices.numpy().astype(np.int16)
        out[f"{name}__slots"] = rf.argmax(2).astype(np.uint16)
        out[f"{name}__ref_coords"] = layer.ref_coords.numpy()
        out[f"{name}__resolutions"] = np.array([layer.in_coords.resolution, layer.out_coords.resolution])
        out[f"{name}__in_rowcol"] = layer.in_coords.cartesian_rowcol.numpy()
        out[f"{name}__out_rowcol"] = layer.out_coords.cartesian_rowcol.numpy()
        print(f"{name}: k={layer._k} n_in={len(layer.in_coords)} n_out={len(layer.out_coords)} "
              f"V={rf.shape[2]}", flush=True)
    np.savez_compressed(DINOV3_OUT, **out)
    print(f"wrote {DINOV3_OUT} ({os.path.getsize(DINOV3_OUT) / 1024:.0f} KiB)")


if __name__ == "__main__":
    if "--isotropic" in sys.argv:
        main_isotropic()
    elif "--dinov3" in sys.argv:
        main_dinov3()
    else:
        main()
