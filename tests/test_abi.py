"""The C ABI on the CPU: the library loads, exports every symbol the header
declares, and its host-only entry points behave like the reference.  No
device is needed (and none is touched beyond counting devices)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "godwit_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gw_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from godwit_amd import _lib
    declared = _declared()
    assert declared, "no declarations parsed"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (gw_[a-z0-9_]+)", out))
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    # the Python binding covers exactly the declared surface
    assert sorted(_lib.SIGNATURES) == declared


def test_device_count_without_gpu_is_callable():
    import godwit_amd as gw
    assert gw.device_count() >= 0


def test_layout_matches_install_layout_tests():
    """InstallLayoutTests.swift:10-61 and Qwen3SupportTests.swift:81-109."""
    import godwit_amd as gw
    lay = gw.ExpertLayout(2880, 2880, 128)
    assert lay.size("gate_up_blocks") == 5760 * 90 * 16
    assert lay.size("gate_up_scales") == 5760 * 90
    assert lay.size("down_blocks") == 2880 * 90 * 16
    assert lay.size("down_scales") == 2880 * 90
    assert lay.size("gate_up_bias") == 5760 * 2
    assert lay.size("down_bias") == 2880 * 2
    mib = lay.payload_per_expert / 1048576
    assert 12.6 < mib < 12.7
    for s in gw.SECTIONS:
        assert lay.offset(0, s) % 16384 == 0
    assert lay.stride % 16384 == 0
    assert lay.padding_overhead < 0.01
    assert lay.layer_file_size == lay.stride * 128
    gib = lay.layer_file_size * 36 / 1073741824
    assert 56 < gib < 58
    # offsets stated in the survey of the reference layout
    assert [lay.offsets[s] for s in gw.SECTIONS] == [0, 8306688, 8830976, 12992512, 13254656,
                                                    13271040]
    assert lay.stride == 13287424
    q = gw.ExpertLayout(2048, 768, 128)
    assert q.size("gate_up_blocks") == 2 * 768 * (2048 // 32) * 16
    assert q.size("gate_up_scales") == 2 * 768 * (2048 // 32)
    assert q.size("down_blocks") == 2048 * (768 // 32) * 16
    assert q.size("down_scales") == 2048 * (768 // 32)
    assert q.size("gate_up_bias") > 0 and q.size("down_bias") > 0
    assert q.stride == 2539520


def test_layout_rejects_partial_blocks():
    import godwit_amd as gw
    with pytest.raises(gw.GodwitError) as e:
        gw.ExpertLayout(2880, 2888, 4)
    assert e.value.status == 2


def test_router_select_host_equals_oracle():
    """gw_router_select restates Router.select on the host; identical to the oracle bit for bit."""
    import godwit_amd as gw
    r = np.random.default_rng(0)
    router = gw.Router.__new__(gw.Router)
    router.expert_count, router.top_k = 128, 4
    for _ in range(300):
        lg = r.standard_normal(128).astype(np.float32)
        lg[r.integers(0, 128, 3)] = lg[0]     # plant ties
        d = router.select(lg)
        ids, w = oracle.router_select(lg, 4)
        assert d.experts == list(ids)
        assert np.array_equal(np.array(d.weights, np.float32), w)


def test_errors_without_device():
    from godwit_amd import _lib
    h = ctypes.c_void_p()
    import godwit_amd as gw
    if gw.device_count() == 0:
        assert _lib.lib.gw_context_create(0, ctypes.byref(h)) == _lib.GW_ERR_NO_DEVICE
        assert b"no HIP device" in _lib.lib.gw_last_error()
    assert _lib.lib.gw_mxfp4_dequant(None, None, None, 4, None) == _lib.GW_ERR_ARG
    assert _lib.lib.gw_router_select(None, 4, 2, None, None) == _lib.GW_ERR_ARG
    lg = np.zeros(4, np.float32)
    ids = np.zeros(8, np.int32)
    w = np.zeros(8, np.float32)
    assert _lib.lib.gw_router_select(lg.ctypes.data, 4, 5, ids.ctypes.data,
                                     w.ctypes.data) == _lib.GW_ERR_SHAPE
