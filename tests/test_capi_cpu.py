"""CPU checks of the C ABI library: it loads, exports exactly what
include/gsplat_hip.h declares, and validates arguments before launching
anything (these calls never reach the GPU)."""
import ctypes
import os
import re

import pytest

from torch_gsplat_bridge_fast import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gsplat_hip.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gsplat_hip_\w+)\s*\(", src)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), f"{n} declared in gsplat_hip.h but not exported"
    # the Python binding covers exactly the declared surface
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version():
    assert _lib.lib().gsplat_hip_abi_version() == _lib.ABI_VERSION == 15


def _meta(**kw):
    m = _lib.make_raster_meta(64, 80, 2, 100, 1 / 255, 1e-4, (0, 0, 0))
    for k, v in kw.items():
        setattr(m, k, v)
    return m


def test_workspace_queries():
    L = _lib.lib()
    assert L.gsplat_hip_bin_count_workspace_bytes(_meta()) > 0
    assert L.gsplat_hip_bin_emit_workspace_bytes(_meta(), 12345) >= 2 * 12345 * 4
    assert L.gsplat_hip_scan_workspace_bytes(1000) > 0           # look-back status + ticket
    assert L.gsplat_hip_scan_workspace_bytes(10_000_000) > 0
    assert L.gsplat_hip_radix_sort_workspace_bytes(100_000, 3) > 0
    # invalid meta -> 0 bytes
    assert L.gsplat_hip_bin_count_workspace_bytes(_meta(tile_size=8)) == 0


@pytest.mark.parametrize("field,value,msg", [
    ("tile_size", 8, "tile_size must be 16"),
    ("height", 0, "must be > 0"),
    ("batch", 0, "must be > 0"),
    ("gaussians_per_batch", -3, "must be > 0"),
    ("max_alpha", 1.0, "max_alpha must lie in [0, 1)"),
    ("max_alpha", float("nan"), "max_alpha must lie in [0, 1)"),
    ("eps", 0.5, "1 - max_alpha >= eps"),
    ("transmittance_threshold", 1.0, "transmittance_threshold must lie in [0, 1)"),
    ("transmittance_threshold", -0.5, "transmittance_threshold must lie in [0, 1)"),
])
def test_invalid_meta_rejected_before_launch(field, value, msg):
    L = _lib.lib()
    m = _meta(**{field: value})
    dummy = ctypes.c_void_p(1)
    rc = L.gsplat_hip_render_forward(m, dummy, dummy, dummy, dummy, None, None, None, 0, None, 0, None)
    assert rc == 1
    assert msg in L.gsplat_hip_last_error().decode()


def test_null_pointers_rejected():
    L = _lib.lib()
    rc = L.gsplat_hip_render_backward(_meta(), None, None, None, None, None, None, None, None, None, None, None,
                                      0, None, 0, None)
    assert rc == 1
    assert "NULL" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_render_forward(_meta(), ctypes.c_void_p(1), ctypes.c_void_p(1), None, ctypes.c_void_p(1),
                                     ctypes.c_void_p(1), None, None, 0, None, 0, None)
    assert rc == 1 and "all be given" in L.gsplat_hip_last_error().decode()


def test_workspace_too_small_rejected():
    L = _lib.lib()
    one = ctypes.c_void_p(1)
    rc = L.gsplat_hip_bin_count(_meta(), *([one] * 4), one, 1, None)
    assert rc == 3
    assert "workspace" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin_pack(_meta(), *([one] * 7), one, 1, None)
    assert rc == 3 and "bin_pack" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin_depth_order(_meta(), one, one, one, 1, None)
    assert rc == 3 and "bin_depth_order" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin_emit(_meta(), one, one, 10, one, one, one, None, one, 1, one, 1, None)
    assert rc == 3
    pm = _lib.make_project_meta(2, 1000, 1e-4)
    need = L.gsplat_hip_project_backward_workspace_bytes(pm)
    assert need >= 2 * 4 * 16 * 4          # B * ceil(G/256) * 16 floats
    rc = L.gsplat_hip_project_backward(pm, *([one] * 16), one, need - 1, None)
    assert rc == 3 and "project_backward" in L.gsplat_hip_last_error().decode()
    need = L.gsplat_hip_render_workspace_bytes(_meta(), 100000)
    assert need > L.gsplat_hip_render_workspace_bytes(_meta(), 1000) > 0
    rc = L.gsplat_hip_render_forward(_meta(), *([one] * 7), 100000, one, need - 1, None)
    assert rc == 3 and "render_forward" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_render_backward(_meta(), *([one] * 11), 100000, one, need - 1, None)
    assert rc == 3 and "render_backward" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_render_forward(_meta(), *([one] * 7), -1, None, 0, None)
    assert rc == 1 and "pair count" in L.gsplat_hip_last_error().decode()


def test_projection_meta_rejected():
    L = _lib.lib()
    pm = _lib.make_project_meta(0, 10, 1e-4)
    one = ctypes.c_void_p(1)
    rc = L.gsplat_hip_project_forward(pm, *([one] * 10), None)
    assert rc == 1 and "batch" in L.gsplat_hip_last_error().decode()


def test_pair_capacity_policy():
    """Host bookkeeping of the pair capacity (no GPU): a count above the capacity fails the check and
    raises the remembered capacity; a much smaller one lowers it; an overflowed count raises."""
    from torch_gsplat_bridge_fast import _ops

    key = ("cpu-test", 1, 2, 3, 4)
    _ops._capacity.pop(key, None)
    st = _ops.BinState(None, None, None, None, None, 1000, _n=900, _key=key)
    assert st.confirm() and _ops._capacity[key] == _ops._headroom(900)
    _ops._capacity[key] = 1000
    st = _ops.BinState(None, None, None, None, None, 1000, _n=1001, _key=key)
    assert not st.confirm() and _ops._capacity[key] == _ops._headroom(1001) >= 1001
    _ops._capacity[key] = 10 ** 7
    st = _ops.BinState(None, None, None, None, None, 10 ** 7, _n=5, _key=key)
    assert st.confirm() and _ops._capacity[key] == _ops._headroom(5)
    st = _ops.BinState(None, None, None, None, None, 10, _n=-1, _key=key)
    with pytest.raises(RuntimeError, match="overflowed"):
        st.confirm()
    _ops._capacity.pop(key, None)


def test_one_call_binning_validation():
    """gsplat_hip_bin checks its arguments before launching: NULL inputs, a negative capacity, a count
    stream without events, a short workspace."""
    L = _lib.lib()
    one = ctypes.c_void_p(1)
    m = _meta()
    need = L.gsplat_hip_bin_workspace_bytes(m, 1000)
    assert need > L.gsplat_hip_bin_workspace_bytes(m, 10) > 0
    rc = L.gsplat_hip_bin(m, *([None] * 5), 10, *([one] * 7), need, None, None, None, None, None)
    assert rc == 1 and "NULL" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin(m, *([one] * 5), -1, *([one] * 7), need, None, None, None, None, None)
    assert rc == 1 and "capacity" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin(m, *([one] * 5), 1000, *([one] * 7), need, one, ctypes.c_void_p(2), None, None, None)
    assert rc == 1 and "events" in L.gsplat_hip_last_error().decode()
    rc = L.gsplat_hip_bin(m, *([one] * 5), 1000, *([one] * 7), need - 1, None, None, None, None, None)
    assert rc == 3 and "workspace" in L.gsplat_hip_last_error().decode()


def test_launch_trace_arguments():
    """gsplat_hip_trace_launches: n outside [0, GSPLAT_TRACE_MAX] or null events are refused;
    n = 0 disarms; nothing is traced while disarmed (no GPU needed: no launch happens)."""
    L = _lib.lib()
    assert L.gsplat_hip_trace_launches(None, -1) != 0
    assert L.gsplat_hip_trace_launches(None, _lib.TRACE_MAX + 1) != 0
    assert L.gsplat_hip_trace_launches(None, 4) != 0
    events = (ctypes.c_void_p * 8)(*([None] * 8))
    assert L.gsplat_hip_trace_launches(events, 4) != 0
    assert "null" in L.gsplat_hip_last_error().decode()
    assert L.gsplat_hip_trace_launches(None, 0) == 0
    assert L.gsplat_hip_trace_count() == 0
    assert L.gsplat_hip_trace_name(0) is None
