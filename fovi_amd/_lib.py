"""ctypes binding of libfovi_hip.so (declarations in include/fovi_hip.h).

There is no fallback: if the library is missing or fails to load, every call
raises. Tensors are passed as raw device pointers with element strides, and
calls are enqueued on torch's current HIP stream.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfovi_hip.so")

ABI_VERSION = 33
F32, BF16, F8E4M3 = 0, 1, 2
NEAREST, BILINEAR = 0, 1
PAD_ZEROS, PAD_BORDER = 0, 1
ACT_NONE, ACT_RELU = 0, 1
W_ROWS, W_MFMA = 0, 1
POOL_MAX, POOL_AVG, POOL_SUM, POOL_GAUSSIAN = 0, 1, 2, 3

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float8_e4m3fn: F8E4M3}

# Every symbol include/fovi_hip.h declares.
EXPORTED = ("fovi_abi_version", "fovi_last_error", "fovi_sampler_fwd", "fovi_knnconv_fwd",
            "fovi_knnconv_pack_weight", "fovi_knnconv_weight_mfma_elems", "fovi_knnconv_pack_weight_mfma",
            "fovi_quantize_e4m3", "fovi_knnpool_fwd", "fovi_knnconv_slotsum", "fovi_knnconv_bwd_x",
            "fovi_knn_logpolar_candidates", "fovi_knn_select", "fovi_knn_euclid_candidates", "fovi_local_rf_slots", "fovi_knnconv_dw_workspace_bytes",
            "fovi_knnconv_dw", "fovi_knnpool_bwd", "fovi_knnconv_last_path",
            "fovi_knnconv_fwd_noalloc", "fovi_knnconv_wide_tiles")


class SamplerArgs(C.Structure):
    _fields_ = [
        ("img", C.c_void_p), ("img_dtype", C.c_int32), ("reserved0", C.c_int32),
        ("n_img", C.c_int64), ("channels", C.c_int64), ("height", C.c_int64), ("width", C.c_int64),
        ("img_stride", C.c_int64 * 4),
        ("grid", C.c_void_p), ("n_points", C.c_int64), ("n_views", C.c_int64),
        ("fix_loc", C.c_void_p), ("fix_half", C.c_void_p),
        ("fix_half_wide", C.c_int32), ("ring_len", C.c_int32),
        ("view_image", C.c_void_p),
        ("mode", C.c_int32), ("padding", C.c_int32),
        ("out", C.c_void_p), ("out_dtype", C.c_int32), ("reserved2", C.c_int32),
        ("out_stride", C.c_int64 * 3),
        ("grid_out", C.c_void_p),
    ]


class KnnConvArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int32), ("reserved0", C.c_int32),
        ("batch", C.c_int64), ("c_in", C.c_int64), ("n_in", C.c_int64),
        ("x_stride", C.c_int64 * 3),
        ("n_out", C.c_int64), ("k", C.c_int64), ("n_ref", C.c_int64),
        ("slot_ptr", C.c_void_p), ("nbr_sorted", C.c_void_p),
        ("w", C.c_void_p), ("w_dtype", C.c_int32), ("w_layout", C.c_int32),
        ("c_out", C.c_int64), ("k_pad", C.c_int64),
        ("bias", C.c_void_p), ("w_scale", C.c_void_p),
        ("x_scale", C.c_float), ("reserved2", C.c_int32),
        ("y", C.c_void_p), ("y_dtype", C.c_int32), ("reserved3", C.c_int32),
        ("y_stride", C.c_int64 * 3),
        ("tile_lo", C.c_void_p), ("tile_span", C.c_void_p),
        ("tile_ent", C.c_void_p), ("tile_nbr", C.c_void_p),
        ("tile_points", C.c_int32), ("max_span", C.c_int32),
        ("tile_coll", C.c_void_p), ("tile_coll_n", C.c_void_p),
        ("zero_row", C.c_int32), ("activation", C.c_int32),
        ("w_c_slot", C.c_int32), ("reserved5", C.c_int32),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_int64),
        ("x_scale_dev", C.c_void_p),
        ("tile_src", C.c_void_p), ("tile_coll_off", C.c_void_p), ("tile_cent", C.c_void_p),
        ("coll_off_stride", C.c_int32), ("cent_stride", C.c_int32),
        ("tile_heavy", C.c_void_p), ("tile_hlist", C.c_void_p), ("heavy_stride", C.c_int32),
        ("hlist_stride", C.c_int32),
        ("fc_lo", C.c_void_p), ("fc_span", C.c_void_p), ("fc_item", C.c_void_p), ("fc_threads", C.c_int32), ("fc_chunk", C.c_int32),
        ("reserved7", C.c_void_p), ("fc_tile_points", C.c_int32), ("fc_zero_row", C.c_int32),
        ("fc_pairs", C.c_int32), ("wide_units", C.c_int32),
        ("fc_comb", C.c_void_p), ("fc_comb_off", C.c_void_p), ("fc_pmax", C.c_int32), ("wide_tiles", C.c_int32),
        ("vm_idx", C.c_void_p), ("vm_ev", C.c_void_p), ("vm_off", C.c_void_p), ("vm_j0", C.c_void_p),
        ("vm_w", C.c_void_p), ("vm_nb", C.c_int32), ("vm_cb", C.c_int32),
    ]


class QuantizeArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int32), ("reserved0", C.c_int32),
        ("batch", C.c_int64), ("channels", C.c_int64), ("points", C.c_int64),
        ("x_stride", C.c_int64 * 3),
        ("q", C.c_void_p), ("q_stride", C.c_int64 * 3),
        ("headroom", C.c_float), ("reserved1", C.c_int32),
        ("scale_in", C.c_void_p), ("scale_out", C.c_void_p), ("amax_work", C.c_void_p),
    ]


class KnnPoolArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int32), ("mode", C.c_int32),
        ("batch", C.c_int64), ("channels", C.c_int64), ("n_in", C.c_int64),
        ("x_stride", C.c_int64 * 3),
        ("nbr", C.c_void_p), ("weights", C.c_void_p),
        ("n_out", C.c_int64), ("k", C.c_int64),
        ("y", C.c_void_p), ("y_dtype", C.c_int32), ("reserved0", C.c_int32),
        ("y_stride", C.c_int64 * 3),
    ]


class KnnPoolBwdArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int32), ("mode", C.c_int32),
        ("batch", C.c_int64), ("channels", C.c_int64), ("n_in", C.c_int64),
        ("x_stride", C.c_int64 * 3),
        ("nbr", C.c_void_p), ("weights", C.c_void_p),
        ("n_out", C.c_int64), ("k", C.c_int64),
        ("dy", C.c_void_p), ("dy_dtype", C.c_int32), ("dx_dtype", C.c_int32),
        ("dy_stride", C.c_int64 * 3),
        ("inv_ptr", C.c_void_p), ("inv", C.c_void_p), ("state", C.c_void_p),
        ("dx", C.c_void_p), ("dx_stride", C.c_int64 * 3),
    ]


class SlotsumArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_dtype", C.c_int32), ("a_dtype", C.c_int32),
        ("batch", C.c_int64), ("c_in", C.c_int64), ("n_in", C.c_int64),
        ("x_stride", C.c_int64 * 3),
        ("n_out", C.c_int64), ("k", C.c_int64), ("n_ref", C.c_int64),
        ("slot_ptr", C.c_void_p), ("nbr_sorted", C.c_void_p), ("a", C.c_void_p),
    ]


class BwdXArgs(C.Structure):
    _fields_ = [
        ("g", C.c_void_p), ("g_dtype", C.c_int32), ("dx_dtype", C.c_int32),
        ("batch", C.c_int64), ("c_in", C.c_int64), ("n_in", C.c_int64), ("n_out", C.c_int64),
        ("n_ref", C.c_int64),
        ("inv_ptr", C.c_void_p), ("inv", C.c_void_p), ("dx", C.c_void_p),
        ("dx_stride", C.c_int64 * 3),
    ]


class KnnLogpolarArgs(C.Structure):
    _fields_ = [
        ("src", C.c_void_p), ("dst", C.c_void_p),
        ("n_in", C.c_int64), ("n_out", C.c_int64), ("k", C.c_int64),
        ("theta_hi", C.c_float), ("theta_half", C.c_float),
        ("cap", C.c_int64),
        ("cand_idx", C.c_void_p), ("cand_sq", C.c_void_p), ("cand_n", C.c_void_p),
    ]


class KnnEuclidArgs(C.Structure):
    _fields_ = [
        ("src", C.c_void_p), ("dst", C.c_void_p),
        ("n_in", C.c_int64), ("n_out", C.c_int64), ("k", C.c_int64),
        ("dim", C.c_int32), ("src_norm_max", C.c_float),
        ("cap", C.c_int64), ("cand_idx", C.c_void_p), ("cand_sq", C.c_void_p), ("cand_n", C.c_void_p),
    ]


class KnnSelectArgs(C.Structure):
    _fields_ = [
        ("n_out", C.c_int64), ("k", C.c_int64), ("cap", C.c_int64),
        ("cand_idx", C.c_void_p), ("cand_d", C.c_void_p), ("cand_n", C.c_void_p),
        ("idx", C.c_void_p), ("dist", C.c_void_p),
    ]


class LocalRfArgs(C.Structure):
    _fields_ = [
        ("src_cortical", C.c_void_p), ("src_cart", C.c_void_p), ("n_src", C.c_int64), ("dim", C.c_int),
        ("out_cortical", C.c_void_p), ("out_cart", C.c_void_p), ("n_out", C.c_int64),
        ("knn_idx", C.c_void_p), ("k", C.c_int64), ("ref", C.c_void_p), ("n_ref", C.c_int64),
        ("tol", C.c_float), ("slots", C.c_void_p), ("flags", C.c_void_p),
    ]


class KnnConvDwArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_stride", C.c_int64 * 3),
        ("dy", C.c_void_p), ("dy_stride", C.c_int64 * 3),
        ("batch", C.c_int64), ("c_in", C.c_int64), ("c_out", C.c_int64), ("n_in", C.c_int64),
        ("n_out", C.c_int64), ("n_ref", C.c_int64),
        ("pair_off", C.c_void_p), ("pairs", C.c_void_p),
        ("n_chunks", C.c_int64), ("images_per_group", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_int64),
        ("dw", C.c_void_p),
    ]


_lib = None


def load(path: str = LIB_PATH):
    """Loads the library once; raises if it is missing or of another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -m fovi_amd.build` (hipcc, gfx950)")
    lib = C.CDLL(path)
    lib.fovi_abi_version.restype = C.c_int
    lib.fovi_last_error.restype = C.c_char_p
    lib.fovi_knnconv_last_path.restype = C.c_char_p
    lib.fovi_sampler_fwd.argtypes = [C.POINTER(SamplerArgs), C.c_void_p]
    lib.fovi_sampler_fwd.restype = C.c_int
    lib.fovi_knnconv_fwd.argtypes = [C.POINTER(KnnConvArgs), C.c_void_p]
    lib.fovi_knnconv_fwd.restype = C.c_int
    lib.fovi_knnconv_fwd_noalloc.argtypes = [C.POINTER(KnnConvArgs), C.c_void_p]
    lib.fovi_knnconv_fwd_noalloc.restype = C.c_int
    lib.fovi_knnconv_pack_weight.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p,
                                             C.c_int32, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]
    lib.fovi_knnconv_pack_weight.restype = C.c_int
    lib.fovi_knnconv_weight_mfma_elems.argtypes = [C.c_int64, C.c_int64, C.c_int64]
    lib.fovi_knnconv_weight_mfma_elems.restype = C.c_int64
    lib.fovi_knnconv_pack_weight_mfma.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p,
                                                  C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.fovi_knnconv_pack_weight_mfma.restype = C.c_int
    lib.fovi_quantize_e4m3.argtypes = [C.POINTER(QuantizeArgs), C.c_void_p]
    lib.fovi_quantize_e4m3.restype = C.c_int
    lib.fovi_knnpool_fwd.argtypes = [C.POINTER(KnnPoolArgs), C.c_void_p]
    lib.fovi_knnpool_fwd.restype = C.c_int
    lib.fovi_knnconv_slotsum.argtypes = [C.POINTER(SlotsumArgs), C.c_void_p]
    lib.fovi_knnconv_slotsum.restype = C.c_int
    lib.fovi_knnconv_bwd_x.argtypes = [C.POINTER(BwdXArgs), C.c_void_p]
    lib.fovi_knnconv_bwd_x.restype = C.c_int
    lib.fovi_knn_logpolar_candidates.argtypes = [C.POINTER(KnnLogpolarArgs), C.c_void_p]
    lib.fovi_knn_logpolar_candidates.restype = C.c_int
    lib.fovi_knn_select.argtypes = [C.POINTER(KnnSelectArgs), C.c_void_p]
    lib.fovi_knn_select.restype = C.c_int
    lib.fovi_knn_euclid_candidates.argtypes = [C.POINTER(KnnEuclidArgs), C.c_void_p]
    lib.fovi_knn_euclid_candidates.restype = C.c_int
    lib.fovi_local_rf_slots.argtypes = [C.POINTER(LocalRfArgs), C.c_void_p]
    lib.fovi_local_rf_slots.restype = C.c_int
    lib.fovi_knnconv_dw_workspace_bytes.argtypes = [C.c_int64] * 6
    lib.fovi_knnconv_dw_workspace_bytes.restype = C.c_int64
    lib.fovi_knnconv_dw.argtypes = [C.POINTER(KnnConvDwArgs), C.c_void_p]
    lib.fovi_knnconv_dw.restype = C.c_int
    lib.fovi_knnpool_bwd.argtypes = [C.POINTER(KnnPoolBwdArgs), C.c_void_p]
    lib.fovi_knnpool_bwd.restype = C.c_int
    lib.fovi_knnconv_wide_tiles.argtypes = [C.c_int64] + [C.c_int32] * 5 + [C.POINTER(C.c_int64)]
    lib.fovi_knnconv_wide_tiles.restype = C.c_int
    got = lib.fovi_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {got}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def knnconv_wide_tiles(n_ref, zero_row, coll_off_stride, cent_stride, heavy_stride, hlist_stride):
    """(collision tiles, LDS bytes) of the wide-layer kernel's tile layout for tables of these
    sizes (``fovi_knnconv_wide_tiles``, the kernel's own rule; host only)."""
    lds = C.c_int64(0)
    nb = load().fovi_knnconv_wide_tiles(int(n_ref), int(zero_row), int(coll_off_stride), int(cent_stride),
                                        int(heavy_stride), int(hlist_stride), C.byref(lds))
    if nb == 0:
        check(1, "fovi_knnconv_wide_tiles")
    return nb, lds.value


def knnconv_last_path() -> str:
    """The kernel path of this thread's last successful ``fovi_knnconv_fwd`` call."""
    return load().fovi_knnconv_last_path().decode()


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def stream_handle(device=None):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(rc: int, what: str):
    if rc != 0:
        msg = load().fovi_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {msg}")


def require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("fovi_amd HIP kernels need GPU tensors (got a CPU tensor); "
                               "there is no CPU fallback")
