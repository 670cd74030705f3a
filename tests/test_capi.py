"""CPU checks of the C ABI: the library loads and exports every entry point
include/zmoe.h declares, with the ctypes signatures the Python layer binds.
No compute call is made (no GPU here)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "zmoe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zmoe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for must in ("zmoe_route_topk", "zmoe_flatten_sort_count", "zmoe_scatter2scatter", "zmoe_group_bwd_w",
                 "zmoe_group", "zmoe_rowwise_sum_product", "zmoe_bincount", "zmoe_glu_w1_forward",
                 "zmoe_combine", "zmoe_combine_backward"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from zmoe import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libzmoe_hip.so is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers exactly the declared surface
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_pure_host_entry_points():
    from zmoe import _lib

    lib = _lib.load()
    assert lib.zmoe_abi_version() == 3
    assert lib.zmoe_status_string(0) == b"ok"
    assert lib.zmoe_status_string(4) == b"misaligned pointer or stride"
    # workspace sizing is host arithmetic: header + one int32 per (tile, bucket)
    assert lib.zmoe_sort_workspace_bytes(262144, 128) == 256 + (262144 // 1024) * 129 * 4


def test_argument_errors_are_reported_without_a_gpu():
    """Shape/dtype validation happens on the host before any launch."""
    from zmoe import _lib

    lib = _lib.load()
    # k > E
    rc = lib.zmoe_route_topk(None, 0, 4, 8, 9, None, 0, None, None, None, None)
    assert rc == 2 and b"k" in lib.zmoe_last_error()
    # bad dtype
    rc = lib.zmoe_combine(None, None, None, 4, 2, 8, 7, None, None)
    assert rc == 3
    # E above the sort's limit
    rc = lib.zmoe_flatten_sort_count(None, 16, 5000, None, None, None, None, None, 0, None)
    assert rc == 2
    # workspace too small
    rc = lib.zmoe_flatten_sort_count(None, 16, 8, None, None, ctypes.c_void_p(16), None, ctypes.c_void_p(16), 8,
                                     None)
    assert rc == 5
    # misaligned K for the grouped GEMM (K must be a multiple of 8 bf16 elements)
    p = ctypes.c_void_p(256)
    rc = lib.zmoe_scatter2scatter(p, 12, p, 12 * 16, 16, 1, None, 0, p, p, p, 4, 12, 16, 2, 1, 0, 0, 1, p, 16, None)
    assert rc == 4


def _header_define(name):
    m = re.search(r"#define\s+" + name + r"\s+\(\(size_t\)(\d+) << (\d+)\)", open(HEADER).read())
    assert m, name
    return int(m.group(1)) << int(m.group(2))


def test_noalloc_sort_rejects_sizes_above_its_scratch():
    """The no-allocation sort refuses, on the host, a size whose workspace exceeds its
    scratch array (ZMOE_SORT_NOALLOC_MAX_BYTES, read from the header). Every device
    pointer but the offsets is null, so a regression in the size check would stop at the
    null-pointer check (ERR_NULL) instead of launching."""
    from zmoe import _lib

    lib = _lib.load()
    cap = _header_define("ZMOE_SORT_NOALLOC_MAX_BYTES")
    E = 1024
    header = lib.zmoe_sort_workspace_bytes(1024, E) - (E + 1) * 4  # workspace = header + tiles x (E + 1) x 4
    R = ((cap - header) // ((E + 1) * 4) + 1) * 1024  # the smallest tile count the scratch cannot hold
    assert lib.zmoe_sort_workspace_bytes(R, E) > cap
    assert lib.zmoe_sort_workspace_bytes(R - 1024, E) <= cap
    rc = lib.zmoe_flatten_sort_count_noalloc(None, R, E, None, None, ctypes.c_void_p(256), None, None, None)
    assert rc == 5 and b"maximum" in lib.zmoe_last_error()


def test_dense_wgrad_workspace_holds_every_split_offset():
    """The split offsets (one int64 per split, up to 64 splits) sit in a header ahead of the
    fp32 partials; the header must hold all 64 so that the offsets of splits 32..63 do not
    land in split 0's partials. The automatic choice reaches 64 splits."""
    from zmoe import _lib, ops

    lib = _lib.load()
    assert ops.dense_wgrad_splits(65536, 8, 256) == 64
    assert all(1 <= ops.dense_wgrad_splits(M, 2048, 2176) <= 64 for M in (0, 1000, 32768, 1 << 20))
    hdr = lib.zmoe_dense_wgrad_workspace_bytes(8, 256, 0)
    assert hdr >= 64 * 8 and hdr % 256 == 0
    assert lib.zmoe_dense_wgrad_workspace_bytes(8, 256, 64) == hdr + 64 * 8 * 256 * 4
    # more than 64 splits is refused before any launch
    p = ctypes.c_void_p(256)
    rc = lib.zmoe_dense_wgrad(p, 8, p, 256, 65536, 8, 256, 1, 1, 65, p, p, 1 << 30, None)
    assert rc == 2


def test_newton_schulz_workspace_is_sized_for_one_pass():
    """Stacks of any length run in passes of at most 1024 matrices spanning under 2 GiB,
    so the workspace of a long stack equals that of one full pass."""
    from zmoe import _lib

    lib = _lib.load()
    one = lib.zmoe_newton_schulz5_workspace_bytes(1023, 256, 4096)     # 1023 x 2 MiB fills one pass
    assert one > 0
    assert lib.zmoe_newton_schulz5_workspace_bytes(1100, 256, 4096) == one
    assert lib.zmoe_newton_schulz5_workspace_bytes(5000, 256, 4096) == one
    # C4's W1 stack [256, 4096, 7168] (15 GB) runs in passes of 36 matrices
    c4 = lib.zmoe_newton_schulz5_workspace_bytes(256, 4096, 7168)
    assert c4 == lib.zmoe_newton_schulz5_workspace_bytes(36, 4096, 7168)
    assert lib.zmoe_newton_schulz5_workspace_bytes(1, 65536, 65536) == 0  # one matrix above 2 GiB


def test_sigmoid_table_matches_torch_and_oracle(tmp_path):
    """The build's routing-probability table (kSigmoidBf16, one entry per bf16 logit) equals
    torch's own bf16 sigmoid (what the reference's gate computes under bf16 autocast,
    modeling/moe_gate.py:27) for all 65536 bit patterns, NaNs included, and so does the
    oracle's bf16(sigmoid_f32); the saturated logits (-89 ... -92.5, where float32 exp(-z)
    overflows) are 0 on all three."""
    import sys

    import numpy as np
    import torch

    import oracle as O

    sys.path.insert(0, os.path.join(ROOT, "architecture-zarelga-superposition_amd"))
    import build_lib

    path = tmp_path / "table.inc"
    build_lib.write_sigmoid_table(str(path))
    body = path.read_text().split("\n", 1)[1]
    bits = np.array([int(v, 16) for v in body.replace(",", " ").split()], dtype=np.uint32)
    assert bits.size == 65536
    with np.errstate(all="ignore"):
        z = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
        orc = O.bf16_round(O.sigmoid_f32(z))
    ref = torch.sigmoid(torch.from_numpy(z).to(torch.bfloat16)).float().numpy()
    got = (bits << 16).view(np.float32)
    for other in (ref, orc):
        np.testing.assert_array_equal(np.isnan(got), np.isnan(other))
        ok = ~np.isnan(other)
        np.testing.assert_array_equal(got[ok].view(np.uint32), other[ok].view(np.uint32))
    sat = (z <= -89.0) & (z >= -92.5)
    assert sat.sum() == 8 and not got[sat].any()
