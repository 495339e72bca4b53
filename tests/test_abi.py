"""The C ABI library: built for gfx950, loads without a GPU, exports every function include/qwattn.h
declares, and reports a missing GPU as a status code (no compute calls here)."""
import ctypes
import os
import subprocess

import pytest

import common


def test_library_exports_every_header_function():
    qw = common.load_package()
    lib = qw.load_library()
    names = qw.header_functions()
    assert len(names) >= 13
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_match_header_exactly():
    qw = common.load_package()
    out = subprocess.run(["nm", "-D", "--defined-only", qw.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = sorted({l.split()[-1] for l in out.splitlines() if " T qwattn_" in l})
    assert exported == qw.header_functions()


def test_code_object_is_gfx950_only():
    qw = common.load_package()
    data = open(qw.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    for other in (b"--gfx942", b"--gfx90a", b"--gfx1100"):
        assert other not in data


def test_no_gpu_is_a_status_code():
    """qwattn_create on a machine without a usable gfx950 returns an error code and text."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    qw = common.load_package()
    with pytest.raises(qw.QwattnError, match="device 0 not available"):
        qw.Attention(16, 2, 256, 64)


def test_bad_shapes_rejected_before_any_device_call():
    """Shape checks come first: they fail identically with or without a GPU."""
    qw = common.load_package()
    for args, pat in [((16, 3, 256, 64), "head counts"), ((16, 2, 96, 64), "head_dim"),
                      ((16, 2, 256, 63), "rope dimension"), ((16, 2, 256, 12), "rope dimension"), ((64, 1, 256, 64), "GQA group")]:
        with pytest.raises(qw.QwattnError, match=pat):
            qw.Attention(*args)


def test_q8_unpack_host():
    """qwattn_q8_unpack (host code, no GPU) turns GGUF Q8_0 rows into the planar int8 weights and f32 scales
    of src/qwen4_vk.cpp:98-106: the weights byte for byte, each binary16 scale widened exactly (normal,
    subnormal, zero, negative and infinite scales included); a bad shape is refused."""
    import numpy as np
    from common import q8_blocks
    qw = common.load_package()
    rows, cols = 5, 96
    blocks, w8, s = q8_blocks(61, rows, cols)
    special = np.array([0x0001, 0x03FF, 0x0000, 0x8000, 0xBC00, 0x7C00, 0x7BFF, 0x0400], np.uint16)
    b = blocks.reshape(rows, cols // 32, 34).copy()
    b[:, :, 0:2] = np.resize(special, (rows, cols // 32)).view(np.uint8).reshape(rows, cols // 32, 2)
    w, sc = qw.q8_unpack(b.reshape(rows, -1), rows, cols)
    assert np.array_equal(w, w8)
    assert np.array_equal(sc, np.resize(special, (rows, cols // 32)).view(np.float16).astype(np.float32))
    w, sc = qw.q8_unpack(blocks, rows, cols)
    assert np.array_equal(w, w8) and np.array_equal(sc, s)
    lib = qw.load_library()
    assert lib.qwattn_q8_unpack(None, rows, cols, None, None) == qw.EINVAL


def test_projection_entry_points_need_a_context():
    """qwattn_mat and qwattn_mat_multi without a context return QWATTN_EINVAL (no device touched)."""
    qw = common.load_package()
    lib = qw.load_library()
    assert lib.qwattn_mat(None, None, None, None, 1, 64, 64, None, 64, None, 64, 1, 0, 0.0) == qw.EINVAL
    assert lib.qwattn_mat_multi(None, None, None, 1, 1, 64, None, 64, 1) == qw.EINVAL
