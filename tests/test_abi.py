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
    of src/qwen4_vk.cpp:98-106: the weights byte for byte, the scales widened as the reference widens them
    (normal, subnormal, zero, negative and exponent-31 scales included); a bad shape is refused."""
    import numpy as np
    from common import q8_blocks
    qw = common.load_package()
    rows, cols = 5, 96
    blocks, w8, s = q8_blocks(61, rows, cols)
    special = np.array([0x0001, 0x03FF, 0x0000, 0x8000, 0xBC00, 0x7C00, 0x7BFF, 0x0400, 0xFFFF, 0x7E00], np.uint16)
    b = blocks.reshape(rows, cols // 32, 34).copy()
    b[:, :, 0:2] = np.resize(special, (rows, cols // 32)).view(np.uint8).reshape(rows, cols // 32, 2)
    w, sc = qw.q8_unpack(b.reshape(rows, -1), rows, cols)
    assert np.array_equal(w, w8)
    assert np.array_equal(sc.view(np.uint32), _widen_scales(qw, np.resize(special, (rows, cols // 32))).view(np.uint32))
    w, sc = qw.q8_unpack(blocks, rows, cols)
    assert np.array_equal(w, w8) and np.array_equal(sc, s)
    lib = qw.load_library()
    assert lib.qwattn_q8_unpack(None, rows, cols, None, None) == qw.EINVAL


def _widen_scales(qw, bits):
    """Every binary16 pattern in `bits` widened by qwattn_q8_unpack (one Q8_0 block per pattern, zero weights)."""
    import numpy as np
    flat = bits.reshape(-1).astype(np.uint16)
    blk = np.zeros((flat.size, 34), np.uint8)
    blk[:, 0:2] = flat.view(np.uint8).reshape(-1, 2)
    w, sc = qw.q8_unpack(blk.reshape(1, -1), 1, 32 * flat.size)
    assert not np.any(w)
    return sc.reshape(bits.shape)


def test_q8_scales_bit_exact_with_reference_all_patterns():
    """All 65,536 binary16 scale patterns widen bit for bit as the reference's ck::half_to_f32
    (src/cpu_kernels.cpp:20-34, the function unpack_q8_row applies at src/qwen4_vk.cpp:98-106).

    Pinned three ways: the reference's own compiled half_to_f32 (oracle/_ref/libref.so, when built); IEEE
    binary16 widening (numpy) for every pattern below exponent 31, where the two definitions coincide; and,
    for exponent 31, which the reference treats as an ordinary exponent (no inf / NaN), twice the value of
    the same sign and fraction at exponent 30."""
    import numpy as np
    qw = common.load_package()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = _widen_scales(qw, bits)
    e31 = ((bits >> 10) & 31) == 31
    ieee = bits[~e31].view(np.float16).astype(np.float32)
    assert np.array_equal(got[~e31].view(np.uint32), ieee.view(np.uint32))
    assert np.array_equal(got[e31], 2 * got[bits[e31] - 0x0400])
    assert got[0x7C00] == 65536.0 and got[0xFC00] == -65536.0 and np.all(np.isfinite(got))
    try:
        import oracle
        ref = oracle.RefPrimitives()
    except (FileNotFoundError, OSError):
        pytest.skip("oracle/_ref/libref.so not built (needs /root/reference)")
    want = np.array([ref.lib.ref_half_to_f32(int(h)) for h in bits], np.float32)
    diff = int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
    assert diff == 0, f"{diff} of 65536 patterns differ from the reference's half_to_f32"


def test_projection_entry_points_need_a_context():
    """qwattn_mat and qwattn_mat_multi without a context return QWATTN_EINVAL (no device touched)."""
    qw = common.load_package()
    lib = qw.load_library()
    assert lib.qwattn_mat(None, None, None, None, 1, 64, 64, None, 64, None, 64, 1, 0, 0.0) == qw.EINVAL
    assert lib.qwattn_mat_multi(None, None, None, 1, 1, 64, None, 64, 1) == qw.EINVAL


def test_mat_wrappers_check_operands():
    """The Python mirror refuses projection operands the C ABI would misread, before any device call: a
    transposed (non-contiguous) weight matrix, weights of the wrong dtype, scales of the wrong shape, an
    input narrower than the weights' columns or with a non-unit column stride."""
    import torch
    qw = common.load_package()
    w = torch.zeros((8, 64), dtype=torch.int8)
    s = torch.zeros((8, 2))
    assert qw._check_weights(w, s) == (8, 64)
    assert qw._check_weights(torch.zeros((8, 64)), None) == (8, 64)
    for bad_w, bad_s in ((w.t(), s), (w.float(), s), (w, torch.zeros((8, 3))), (w, s.double()), (w, None),
                         (torch.zeros((64, 8)).t(), None)):
        with pytest.raises(ValueError):
            qw._check_weights(bad_w, bad_s)
    x = torch.zeros((2, 96))
    qw._check_rows(x[:, :64], "x", 64)
    for bad in (x[:, :32], x.t(), x.double(), x[:, ::2]):
        with pytest.raises(ValueError):
            qw._check_rows(bad, "x", 64)
