"""The C-ABI library: loads, exports every declared symbol, host-only helpers.
No device compute is called here (CPU suite)."""
import ctypes
import os

import pytest

from windlass_amd import moe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_function():
    lib = moe.load()
    names = moe.header_functions()
    assert "wl_run_moe" in names and "wl_create" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing


def test_expert_layout_matches_reference_block():
    # repack_experts_glm.py:46-55 / glm_expert_cache.cuh:101-113
    lay = moe.expert_layout(moe.make_config())
    assert (lay.gw_off, lay.gw_len) == (0, 6291456)
    assert (lay.gs_off, lay.gs_len) == (6291456, 393216)
    assert (lay.uw_off, lay.us_off) == (6684672, 12976128)
    assert (lay.dw_off, lay.ds_off) == (13369344, 19660800)
    assert lay.total == 20054016


def test_invalid_shapes_rejected_without_device():
    lib = moe.load()
    lay = moe.ExpertLayout()
    bad = moe.make_config(hidden=100)
    assert lib.wl_expert_layout_of(ctypes.byref(bad), 0, ctypes.byref(lay)) != 0
    h = ctypes.c_void_p()
    for cfg in [moe.make_config(hidden=100), moe.make_config(n_experts_per_tok=33),
                moe.make_config(n_routed_experts=40), moe.make_config(moe_inter=1000)]:
        assert lib.wl_create(ctypes.byref(cfg), ctypes.byref(h)) == 1  # WL_ERR_INVALID
        assert h.value is None
    # null arguments
    assert lib.wl_dequant_matvec_mxfp4(None, None, None, None, 16, 128, None) == 1


def test_reference_caller_compiles_against_the_shim(tmp_path):
    """include/windlass_glm.hpp keeps the reference's run_moe / run_moe_batched
    spellings: a caller written against them (tests/shim/reference_caller.cpp,
    stand-in types with the reference's fields and its call sites) compiles and
    links against libwindlass_moe.so unchanged. It runs on the GPU in
    tests/test_gpu_shim.py."""
    import shutil

    from tests.shim import build as shim_build
    if shutil.which("/opt/rocm/bin/hipcc") is None:
        pytest.skip("no hipcc")
    out = shim_build.build(str(tmp_path / "caller"))
    assert os.path.exists(out)
