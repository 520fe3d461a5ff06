"""The C-ABI boundary (CPU only): the library builds, loads and exports every
entry point that include/gsplat_hip.h declares; the torch op layer carries
the reference schemas; host tensors are rejected loudly (no CPU fallback)."""

import re
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gsplat_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsplat_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib_path():
    from gsplat_amd import _lib
    if not _lib.LIB_PATH.exists():
        from gsplat_amd.build import build
        build(verbose=False)
    return _lib.LIB_PATH


def test_header_declares_the_survey_export_list():
    names = set(_declared())
    for required in ["gsplat_projection_fused_fwd", "gsplat_projection_fused_bwd",
                     "gsplat_projection_packed_fwd", "gsplat_projection_packed_bwd",
                     "gsplat_sh_fwd", "gsplat_sh_bwd", "gsplat_isect_count",
                     "gsplat_isect_emit", "gsplat_sort_pairs_u64_u32",
                     "gsplat_isect_offsets", "gsplat_rasterize_fwd",
                     "gsplat_rasterize_bwd", "gsplat_grad2d_stats", "gsplat_adam_multi",
                     "gsplat_adam", "gsplat_quat_scale_to_covar_preci_fwd",
                     "gsplat_quat_scale_to_covar_preci_bwd",
                     "gsplat_rasterize_to_indices_count",
                     "gsplat_rasterize_to_indices_write", "gsplat_isect_emit_sorted_dev",
                     "gsplat_rasterize_replay_size", "gsplat_rasterize_fwd_replay",
                     "gsplat_rasterize_bwd_replay", "gsplat_sh_rows_fwd_isect_count",
                     "gsplat_isect_row_starts"]:
        assert required in names, required


def test_library_exports_every_declared_symbol(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (gsplat_[a-z0-9_]+)\b", out))
    missing = [n for n in _declared() if n not in exported]
    assert not missing, missing


def test_library_loads_and_reports_version(lib_path):
    from gsplat_amd import _lib
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name)
    assert _lib.version().startswith("gsplat_hip")


def test_binding_was_written_for_this_header():
    """_lib's recorded interface digest and every hand-typed ctypes
    signature equal the header's declarations, so a header change that the
    binding did not follow fails here, on the CPU."""
    import ctypes

    from gsplat_amd import _lib, abi
    assert _lib._ABI_VERSION == abi.header_abi_hash(), "update _lib._ABI_VERSION"
    protos = abi.header_prototypes()
    assert set(protos) == set(_lib._SIGNATURES)
    arg = {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "int": ctypes.c_int32,
           "float": ctypes.c_float, "size_t": ctypes.c_size_t,
           "gsplat_stream_t": ctypes.c_void_p}
    ret = {"int": ctypes.c_int, "size_t": ctypes.c_size_t, "int64_t": ctypes.c_int64,
           "const char*": ctypes.c_char_p}
    for name, (restype, params) in protos.items():
        want = [ctypes.c_void_p if t.endswith("*") else arg[t] for t in params]
        assert _lib._SIGNATURES[name] == want, name
        assert _lib._RESTYPES.get(name, ctypes.c_int) == ret[restype], name


def test_built_library_reports_the_header_abi(lib_path):
    from gsplat_amd import _lib, abi
    assert _lib.load().gsplat_abi_version().decode() == abi.header_abi_hash()


@pytest.mark.parametrize("reported", ["0123456789abcdef", None])
def test_load_refuses_a_library_of_another_interface(reported, tmp_path, monkeypatch):
    """A stub library whose interface digest differs (or is absent) is
    refused by load() with both versions named, before any signature is
    bound: calling it would pass arguments of the wrong types."""
    from gsplat_amd import _lib
    src = tmp_path / "stub.c"
    body = 'const char *gsplat_version(void) { return "stub"; }\n'
    if reported is not None:
        body += f'const char *gsplat_abi_version(void) {{ return "{reported}"; }}\n'
    src.write_text(body)
    so = tmp_path / "libgsplat_hip.so"
    subprocess.run(["gcc", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    monkeypatch.setattr(_lib, "LIB_PATH", so)
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError) as err:
        _lib.load()
    msg = str(err.value)
    assert _lib._ABI_VERSION in msg
    assert (reported in msg) if reported else ("gsplat_abi_version is missing" in msg)
    assert _lib._lib is None


def test_argument_errors_are_reported_without_a_gpu(lib_path):
    from gsplat_amd import _lib
    with pytest.raises(RuntimeError, match="degree"):
        _lib.call("gsplat_sh_fwd", 10, 16, 7, None, None, None, None, None)
    with pytest.raises(RuntimeError, match="channel"):
        _lib.call("gsplat_rasterize_fwd", 1, 0, 0, 7, None, None, None, None, None, None,
                  16, 16, 16, 1, 1, 1, None, None, None, None, None, None)
    with pytest.raises(RuntimeError, match="pinhole"):
        _lib.call("gsplat_projection_simple_fwd", 1, 1, 1, None, None, None, 16, 16, 2,
                  None, None, None)
    # the allocation-free packed projection rejects sizes beyond its static
    # scratch before touching the device (the pointers are never read)
    limit = _lib.query("gsplat_projection_packed_fwd_noalloc_max_rows")
    fake = [8] * 10
    with pytest.raises(RuntimeError, match="exceed the static scratch"):
        _lib.call("gsplat_projection_packed_fwd_noalloc", 1, 1, limit + 1, 8, None, 8, 8,
                  None, 8, 8, 16, 16, 0.3, 0.01, 1e10, 0.0, 0, *fake, None, None, None)


def test_fused_colour_and_count_checks_without_a_gpu(lib_path):
    """gsplat_sh_rows_fwd_isect_count and gsplat_isect_row_starts refuse bad
    sizes, a short workspace and missing buffers before the device is
    touched (the fake pointers are never read)."""
    from gsplat_amd import _lib
    f = 256
    ws = _lib.query("gsplat_isect_prepare_rows_workspace_size", 1000)
    base = [1, 2, 500, 16, 3, f, f, f, f, f, 1000, f, f, f, f, f, f, f, 16, 4, 3,
            f, ws, f, f, f, None]
    args = list(base)
    args[4] = 5
    with pytest.raises(RuntimeError, match="degree"):
        _lib.call("gsplat_sh_rows_fwd_isect_count", *args)
    args = list(base)
    args[10] = 1001
    with pytest.raises(RuntimeError, match="n_cap"):
        _lib.call("gsplat_sh_rows_fwd_isect_count", *args)
    args = list(base)
    args[22] = ws - 1
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("gsplat_sh_rows_fwd_isect_count", *args)
    args = list(base)
    args[11] = None
    with pytest.raises(RuntimeError, match="NULL"):
        _lib.call("gsplat_sh_rows_fwd_isect_count", *args)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("gsplat_isect_row_starts", 1000, f, ws - 1, f, f, None)
    with pytest.raises(RuntimeError, match="n must be"):
        _lib.call("gsplat_isect_row_starts", 0, f, ws, f, f, None)


def test_replay_workspace_size_and_checks_without_a_gpu(lib_path):
    """The replay workspace: 256 B of count, the unit list (records + tiles
    entries of 8 B, padded to 256 B), each tile's last contributor (4 B,
    padded to 256 B), then ceil(n_isects / Q) records of
    tile_size^2 pixels x (1 + CDIM) floats, Q = tile_size^2 / 4; a short or
    missing workspace is refused before the device is touched (the fake
    pointers are never read)."""
    from gsplat_amd import _lib
    q, n_isects, cdim, tiles = 64, 1000, 3, 6
    n_rec = -(-n_isects // q)
    units = -(-(n_rec + tiles) * 8 // 256) * 256
    tile_last = -(-tiles * 4 // 256) * 256
    want = 256 + units + tile_last + n_rec * 256 * (1 + cdim) * 4
    assert _lib.query("gsplat_rasterize_replay_size", 1, 3, 2, 16, n_isects, cdim) == want
    assert _lib.query("gsplat_rasterize_replay_size", 1, 3, 2, 16, -1, cdim) == 0
    f = 256  # a fake, aligned device address
    # I, n_rows, n_isects, cdim, means2d, conics, colors, color_last,
    # opacities, backgrounds, masks, W, H, tile_size, tile grid, offsets, ids
    args = [1, 50, n_isects, cdim, f, f, f, None, f, None, None, 40, 30, 16, 3, 2, f, f]
    # bwd_replay after args: render_T, last_ids, v_render_colors,
    # v_render_alphas, v_means2d_abs, v_means2d, v_conics, v_colors,
    # v_color_last, v_opacities, tile_counter, replay, replay_bytes,
    # expected_depth, expected_depth_channel, stream
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("gsplat_rasterize_bwd_replay", *args, f, f, f, None, None, f, f, f, None,
                  f, f, f, want - 1, None, -1, None)
    with pytest.raises(RuntimeError, match="NULL replay"):
        _lib.call("gsplat_rasterize_fwd_replay", *args, f, f, f, f, None, want, -1, None,
                  None, 0, None)
    with pytest.raises(RuntimeError, match="zero_fill"):
        _lib.call("gsplat_rasterize_fwd_replay", *args, f, f, f, f, f, want, -1, None,
                  None, 5, None)
    with pytest.raises(RuntimeError, match="tile_counter"):
        _lib.call("gsplat_rasterize_bwd_replay", *args, f, f, f, None, None, f, f, f, None,
                  f, None, f, want, None, -1, None)
    # the expected-depth channel: in range, and the backward needs the
    # forward's copy of it
    with pytest.raises(RuntimeError, match="expected_depth_channel"):
        _lib.call("gsplat_rasterize_fwd_replay", *args, f, f, f, f, f, want, cdim, f,
                  None, 0, None)
    with pytest.raises(RuntimeError, match="expected_depth"):
        _lib.call("gsplat_rasterize_bwd_replay", *args, f, f, f, None, None, f, f, f, None,
                  f, f, f, want, None, cdim - 1, None)
    # a separate last channel: its gradient output goes with it
    split = list(args)
    split[7] = f
    with pytest.raises(RuntimeError, match="color_last and v_color_last"):
        _lib.call("gsplat_rasterize_bwd_replay", *split, f, f, f, None, None, f, f, f, None,
                  f, f, f, want, None, -1, None)


def test_reference_op_schemas_registered():
    import gsplat_amd  # noqa: F401
    for op in ["spherical_harmonics_fwd", "spherical_harmonics_bwd", "intersect_tile",
               "intersect_offset", "projection_ewa_3dgs_fused_fwd",
               "projection_ewa_3dgs_fused_bwd", "projection_ewa_3dgs_packed_fwd",
               "projection_ewa_3dgs_packed_bwd", "rasterize_to_pixels_3dgs_fwd",
               "rasterize_to_pixels_3dgs_bwd", "adam", "quat_scale_to_covar_preci_fwd",
               "quat_scale_to_covar_preci_bwd", "rasterize_to_indices_3dgs",
               "projection_ewa_simple_fwd", "projection_ewa_simple_bwd"]:
        assert hasattr(torch.ops.gsplat, op), op
    s = str(torch.ops.gsplat.adam.default._schema)
    assert "Tensor(a!) param" in s and "Tensor? valid" in s
    assert gsplat_amd.has_3dgs() and gsplat_amd.has_adam()
    # the reference's own probes (_wrapper.py:181-196), unchanged
    assert hasattr(torch.ops.gsplat, "projection_ewa_simple_fwd")
    assert hasattr(torch.ops.gsplat, "adam")


def test_host_tensors_fail_loudly():
    import gsplat_amd as gs
    p = torch.zeros(4, 3)
    with pytest.raises((RuntimeError, NotImplementedError)):
        gs.adam(p, p.clone(), p.clone(), p.clone(), None, 1e-3, 0.9, 0.999, 1e-8)
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.gsplat.intersect_offset(torch.zeros(3, dtype=torch.int64), 1, 2, 2)
