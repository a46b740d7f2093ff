"""The C-ABI library loads and exports every symbol include/fovi_hip.h declares (no GPU calls)."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

from fovi_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "fovi_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fovi_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert set(names) == set(_lib.EXPORTED), names


def test_library_exports_all_symbols():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built (run python -m fovi_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.fovi_abi_version() == _lib.ABI_VERSION
    assert lib.fovi_last_error() == b""


def test_argument_validation_without_gpu():
    """Host-side checks reject bad arguments before any HIP call."""
    lib = _lib.load()
    a = _lib.KnnConvArgs()
    assert lib.fovi_knnconv_fwd(a, None) != 0
    assert b"null pointer" in lib.fovi_last_error()
    s = _lib.SamplerArgs()
    assert lib.fovi_sampler_fwd(s, None) != 0
    assert b"null pointer" in lib.fovi_last_error()
    assert lib.fovi_knnconv_pack_weight(None, 1, 1, 1, None, 0, 64, 0, None, None) != 0
    q = _lib.QuantizeArgs()
    assert lib.fovi_quantize_e4m3(q, None) != 0
    assert b"null argument" in lib.fovi_last_error()
    q.x, q.q, q.x_dtype, q.headroom = 16, 16, _lib.BF16, 8.0
    assert lib.fovi_quantize_e4m3(q, None) != 0           # no scale_in and no amax/scale buffers
    assert b"amax_work" in lib.fovi_last_error()
    q.scale_in, q.headroom = 16, 0.5
    assert lib.fovi_quantize_e4m3(q, None) != 0
    assert b"headroom" in lib.fovi_last_error()
    pa = _lib.KnnPoolArgs()
    assert lib.fovi_knnpool_fwd(pa, None) != 0
    assert b"null pointer" in lib.fovi_last_error()
    pa.x, pa.nbr, pa.y, pa.mode, pa.k = 16, 16, 16, _lib.POOL_GAUSSIAN, 9
    assert lib.fovi_knnpool_fwd(pa, None) != 0             # Gaussian mode without weights
    assert b"weights" in lib.fovi_last_error()
    pa.mode, pa.k = _lib.POOL_MAX, 0
    assert lib.fovi_knnpool_fwd(pa, None) != 0
    assert b"k must be" in lib.fovi_last_error()
    assert lib.fovi_knnconv_slotsum(_lib.SlotsumArgs(), None) != 0
    assert b"null pointer" in lib.fovi_last_error()
    assert lib.fovi_knnconv_bwd_x(_lib.BwdXArgs(), None) != 0
    assert lib.fovi_knn_logpolar_candidates(_lib.KnnLogpolarArgs(), None) != 0
    assert lib.fovi_knn_select(_lib.KnnSelectArgs(), None) != 0
    assert lib.fovi_knnconv_dw(_lib.KnnConvDwArgs(), None) != 0
    assert lib.fovi_knnpool_bwd(_lib.KnnPoolBwdArgs(), None) != 0
    assert lib.fovi_knnconv_dw_workspace_bytes(64, 1, 1, 256, 256, 25) == 25 * 64 * 256 * 256 * 4
    assert lib.fovi_knnconv_dw_workspace_bytes(64, 64, 64, 256, 256, 25) == 25 * 64 * 256 * 256 * 4
    assert b"null pointer" in lib.fovi_last_error()


def _c_layout(struct, fields, tmp_path):
    """offsetof/sizeof of a header struct, from a C program built with gcc."""
    src = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "fovi_hip.h"', "int main(void) {",
             f'  printf("%zu\\n", sizeof({struct}));']
    lines += [f'  printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    return vals[0], vals[1:]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
@pytest.mark.parametrize("py,c", [(_lib.SamplerArgs, "fovi_sampler_args"), (_lib.KnnConvArgs, "fovi_knnconv_args"),
                                  (_lib.QuantizeArgs, "fovi_quantize_args"),
                                  (_lib.KnnPoolArgs, "fovi_knnpool_args"),
                                  (_lib.SlotsumArgs, "fovi_knnconv_slotsum_args"),
                                  (_lib.BwdXArgs, "fovi_knnconv_bwd_x_args"),
                                  (_lib.KnnLogpolarArgs, "fovi_knn_logpolar_args"),
                                  (_lib.KnnSelectArgs, "fovi_knn_select_args"),
                                  (_lib.KnnConvDwArgs, "fovi_knnconv_dw_args"),
                                  (_lib.KnnPoolBwdArgs, "fovi_knnpool_bwd_args")])
def test_struct_layout_matches_header(py, c, tmp_path):
    fields = [f for f, _ in py._fields_]
    size, offs = _c_layout(c, fields, tmp_path)
    assert ctypes.sizeof(py) == size
    for f, off in zip(fields, offs):
        assert getattr(py, f).offset == off, f


def test_wide_tile_rule_is_the_header_layout():
    """fovi_knnconv_wide_tiles (the kernel's rule, which the table builder asks) equals the
    layout include/fovi_hip.h documents, on both sides of the 160 KB boundary: four collision
    tiles while the four-tile layout fits, else three, with that layout's bytes."""
    from fovi_amd.arch import knn_tables as T
    from tests.test_tables_and_oracle import header_wide_lds_bytes
    lim = 160 * 1024
    for n_ref, zero_row, coll_off, heavy, hlist in ((25, 767, 28, 46, 416), (9, 255, 12, 2, 8),
                                                    (49, 1023, 52, 10, 96), (255, 100, 256, 2, 8)):
        base = header_wide_lds_bytes(n_ref, zero_row, coll_off, 0, heavy, hlist, 4)
        edge = (lim - base) // 16                  # the last cent_stride whose four-tile layout fits
        for cent in sorted({max(0, edge + d) for d in (-300, -2, -1, 0, 1, 2, 300)}):
            sizes = (n_ref, zero_row, coll_off, cent, heavy, hlist)
            four = header_wide_lds_bytes(*sizes, 4)
            nb = 4 if four <= lim else 3
            assert _lib.knnconv_wide_tiles(*sizes) == (nb, header_wide_lds_bytes(*sizes, nb)), sizes
            assert T.wide_tile_count(*sizes) == nb
    lib = _lib.load()
    assert lib.fovi_knnconv_wide_tiles(25, -1, 28, 10, 2, 8, None) == 0
    assert b"sizes" in lib.fovi_last_error()
    assert lib.fovi_knnconv_wide_tiles(1 << 16, 0, 0, 0, 0, 0, None) == 0
    assert lib.fovi_knnconv_wide_tiles(25, 767, 28, 10, 2, 8, None) in (3, 4)
