"""The C-ABI library: builds for gfx950, loads, and exports exactly what
include/autosage_hip.h declares.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from autosage_amd import _native

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "autosage_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(as_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    path = _native.package_library_path()
    if not path.exists():
        pytest.skip("HIP library not built")
    return _native.open_library(path)


def test_header_declares_the_bound_symbols():
    assert declared_functions() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_abi_version_and_empty_error(lib):
    assert lib.as_abi_version() == _native.ABI_VERSION
    assert lib.as_last_error() == b""


def test_workspace_sizes_are_host_only_and_monotone(lib):
    for fn in (lib.as_bin_workspace_bytes, lib.as_spmm_split_workspace_bytes, lib.as_sddmm_split_workspace_bytes):
        sizes = [fn(n) for n in (0, 1, 1023, 1024, 10**6)]
        assert all(s > 0 for s in sizes)
        assert sizes == sorted(sizes)
    assert lib.as_spmm_split_workspace_bytes(10**6) >= 4 * 10**6
    assert lib.as_csr_attention_workspace_bytes(10, 1000) >= 4000


def test_argument_errors_are_reported_without_a_launch(lib):
    # Invalid arguments are rejected on the host before any HIP call.
    status = lib.as_spmm_csr_split_f32(None, None, None, None, None, 4, 0, 8, 32, 4, 1, 1, 0, None, 0, None)
    assert status == 1
    assert lib.as_last_error() == b"feature_tile must be 64 or 128"
    status = lib.as_spmm_csr_split_f32(None, None, None, None, None, 4, 0, 8, 64, 3, 1, 1, 0, None, 0, None)
    assert lib.as_last_error() == b"warps_per_block must be 2, 4, or 8"
    status = lib.as_bin_rows_by_degree(None, 4, 0, None, None, None, 0, None)
    assert status == 1 and lib.as_last_error() == b"hub_threshold must be positive"
    status = lib.as_sddmm_csr_split_f32(None, None, None, None, None, 4, 0, 8, 4, 0, None, 0, None)
    assert lib.as_last_error() == b"hub_threshold must be a positive 32-bit integer"
    assert lib.as_csr_validate(None, None, -1, 0, 0, None, None) == 1
    assert lib.as_last_error() == b"sizes must be non-negative"
    assert lib.as_csr_validate(None, None, 4, 0, 4, None, None) == 1
    assert lib.as_last_error() == b"null pointer argument"
    assert lib.as_induced_sample_count(None, None, 10, None, 11, None, None, 0, None) == 1
    assert lib.as_last_error() == b"sample size must lie in [0, N]"
    assert lib.as_induced_sample_workspace_bytes(1000) >= 4000
    # 16-bit SpMM: unknown dtype code, misaligned pointers, null inputs
    assert lib.as_spmm_csr_rounded_16(None, None, None, None, None, 4, 0, 8, 3, 1, None, 0, -1, -1, None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_spmm_csr_rounded_16(None, None, None, 1, None, 4, 0, 8, 1, 1, None, 0, -1, -1, None) == 1
    assert lib.as_last_error() == b"x, y and val must be 2-byte aligned"
    assert lib.as_spmm_csr_rounded_16(None, None, None, None, None, 4, 0, 8, 2, 0, None, 0, -1, -1, None) == 1
    assert lib.as_last_error() == b"null pointer argument"
    # column slices from degree 256 for fp32 rows of at most 64 features, else 128; edge slices from 1024
    assert [lib.as_spmm_colslice_min_degree(1, f, 0) for f in (1, 64, 65, 128)] == [256, 256, 128, 128]
    assert [lib.as_spmm_colslice_min_degree(1, f, 1) for f in (8, 64, 128)] == [512, 512, 512]
    assert lib.as_spmm_colslice_min_degree(0, 64, 0) == 1024 and lib.as_spmm_colslice_min_degree(0, 128, 2) == 1024
    # column-sliced plans: settings and sizes are checked before any device work
    tag = ctypes.c_int64(0)
    assert lib.as_spmm_colslice_plan(None, None, 4, 0, 64, 3, 1, None, 0, ctypes.byref(tag), None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_F32, AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_spmm_colslice_plan(None, None, 4, 0, 64, 0, 0, None, 0, ctypes.byref(tag), None) == 1
    assert lib.as_last_error() == b"float32 features take column slices only (column_slices != 0)"
    assert lib.as_spmm_colslice_plan(256, 256, 4, 0, 64, 0, 1, 256, 16, ctypes.byref(tag), None) == 4
    assert lib.as_last_error().startswith(b"a column-sliced plan needs ")
    assert lib.as_spmm_colslice_plan_bytes(1000) >= 28 * 1000
    # an empty graph builds an empty plan and reports the tag of its settings
    tags = {}
    for code, f, slices in [(0, 64, 1), (0, 128, 1), (1, 64, 1), (1, 128, 0), (2, 128, 0)]:
        assert lib.as_spmm_colslice_plan(None, None, 0, 0, f, code, slices, 256, 1 << 20, ctypes.byref(tag), None) == 0
        tags[(code, f, slices)] = tag.value
    # fp32 F=64 slices from 256, F=128 from 128; bf16 and fp16 with edge slices share their tag
    assert tags[(0, 64, 1)] != tags[(0, 128, 1)] and tags[(0, 128, 1)] != tags[(1, 64, 1)]
    assert tags[(1, 128, 0)] == tags[(2, 128, 0)]
    # a plan of other settings is refused before the plan or any pointer is read
    fake = 256
    assert lib.as_spmm_csr_colslice_planned(fake, fake, None, fake, fake, 4, 4, 128, 0, 1, fake, 1 << 20,
                                            tags[(0, 64, 1)], fake, 1 << 20, -1, 0, None) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    assert lib.as_spmm_csr_colslice_planned(fake, fake, None, fake, fake, 4, 4, 128, 0, 0, fake, 1 << 20,
                                            tags[(0, 128, 1)], fake, 1 << 20, -1, 0, None) == 1
    # the row-shard forms take the column count separately and refuse a bad one before any pointer is read
    rect_tag = ctypes.c_int64(0)
    assert lib.as_spmm_colslice_plan_rect(None, None, 0, 5, 0, 128, 0, 1, 256, 1 << 20, ctypes.byref(rect_tag),
                                          None) == 0
    # a row shard's plan (columns cut over n_cols rows) has a tag of its own,
    # which the square call refuses
    assert rect_tag.value != tags[(0, 128, 1)]
    assert lib.as_spmm_csr_colslice_planned(fake, fake, None, fake, fake, 4, 4, 128, 0, 1, fake, 1 << 20,
                                            rect_tag.value, fake, 1 << 20, -1, 0, None) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    # an attention plan (whole-graph row order) is not an SpMM plan (row
    # blocks), even where the slicing degree and light buckets agree
    att_tag = ctypes.c_int64(0)
    assert lib.as_csr_attention_plan(None, None, 0, 0, 1, 256, 1 << 20, ctypes.byref(att_tag), None) == 0
    assert att_tag.value not in tags.values()
    assert lib.as_spmm_csr_colslice_planned(fake, fake, None, fake, fake, 4, 4, 64, 1, 1, fake, 1 << 20,
                                            att_tag.value, fake, 1 << 20, -1, 0, None) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    assert lib.as_spmm_colslice_plan_rect(None, None, 0, -1, 0, 128, 0, 1, 256, 1 << 20, ctypes.byref(rect_tag),
                                          None) == 1
    assert lib.as_last_error() == b"n_cols exceeds kernel index range"
    assert lib.as_spmm_csr_colslice_planned_rect(fake, fake, None, fake, fake, 4, 1 << 31, 4, 128, 0, 1, fake,
                                                 1 << 20, tags[(0, 128, 1)], fake, 1 << 20, -1, 0, None) == 1
    assert lib.as_last_error() == b"n_cols exceeds kernel index range"
    assert lib.as_spmm_csr_colslice_planned_rect(fake, fake, None, fake, fake, 4, 9, 4, 128, 0, 1, fake, 1 << 20,
                                                 tags[(0, 64, 1)], fake, 1 << 20, -1, 0, None) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    # short rows below 4·G edges run grouped (G lanes per edge: fp32 16 at F <= 64, else 32; 16-bit 8 / 16 / 32)
    assert [lib.as_spmm_colslice_group_degree(f, 0) for f in (64, 128, 256, 66)] == [64, 128, 128, 0]
    for f in (64, 128, 256, 520):
        for code in (1, 2):
            assert lib.as_spmm_colslice_group_degree(f, code) == lib.as_spmm_rounded_16_group_degree(f)
    assert lib.as_spmm_colslice_group_degree(64, 3) == 0
    # two partial buffers of a chunk's rows (all 1,000 rows here: chunks hold at least 32,768), 8 slices of F fp64
    assert lib.as_spmm_colslice_planned_workspace_bytes(1000, 50_000, 128, 0, -1) == 2 * 1000 * 8 * 128 * 8
    assert lib.as_spmm_colslice_planned_workspace_bytes(1000, 50_000, 128, 1, 10) == 2 * 10 * 8 * 128 * 8
    # fp32 keeps a chunk's rows where its chunks would be cut to the buffers: graphs of at most 2^24 edges
    # (cooperative hub rows) and F not a multiple of 4 (narrow lanes); a 20,000-row graph with one sliced
    # row would otherwise run as 20,000 one-row launches
    assert lib.as_spmm_colslice_planned_workspace_bytes(1000, 50_000, 128, 0, 10) == 2 * 1000 * 8 * 128 * 8
    assert lib.as_spmm_colslice_planned_workspace_bytes(1000, 1 << 25, 130, 0, 10) == 2 * 1000 * 8 * 130 * 8
    assert lib.as_spmm_colslice_planned_workspace_bytes(1000, 1 << 25, 128, 0, 10) == 2 * 10 * 8 * 128 * 8
    # attention plans: fp32 and 16-bit tags differ (light buckets), and the
    # forward and the backward refuse a tag of other settings before any device work
    att = {}
    for code in (0, 1, 2):
        assert lib.as_csr_attention_plan(None, None, 0, 0, code, fake, 1 << 20, ctypes.byref(tag), None) == 0
        att[code] = tag.value
    assert att[0] != att[1] and att[1] == att[2]
    # the slicing degree in the tag's low 32 bits: 128 for fp32, 512 for 16-bit
    assert (att[0] & 0xFFFFFFFF, att[1] & 0xFFFFFFFF) == (128, 512)
    assert lib.as_csr_attention_plan(None, None, 4, 0, 3, fake, 1 << 20, ctypes.byref(tag), None) == 1
    assert lib.as_csr_attention_plan(fake, fake, 4, 4, 0, fake, 16, ctypes.byref(tag), None) == 4
    assert lib.as_csr_attention_plan_bytes(1000) == lib.as_spmm_colslice_plan_bytes(1000)
    assert lib.as_csr_attention_colslice_f32(fake, fake, fake, fake, fake, fake, 4, 4, 64, 64, 1.0, fake, att[1],
                                             fake, 1 << 20, None) == 1
    assert lib.as_last_error().startswith(b"the plan was built for other settings")
    assert lib.as_csr_attention_colslice_16(fake, fake, fake, fake, fake, fake, 4, 4, 64, 64, 1.0, 1, fake, att[0],
                                            fake, 1 << 20, None) == 1
    assert lib.as_csr_attention_backward_f32(*([fake] * 12), 4, 4, 64, 64, 1.0, fake, att[0], fake, att[1], fake,
                                             1 << 20, None) == 1
    assert lib.as_last_error().startswith(b"a plan was built for other settings")
    # 16-bit SpMM, rows whole
    assert lib.as_spmm_csr_rows_16(None, None, None, None, None, 4, 0, 8, 3, None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_spmm_csr_rows_16(None, None, None, 1, None, 4, 0, 8, 1, None) == 1
    assert lib.as_last_error() == b"x, y and val must be 2-byte aligned"
    assert lib.as_spmm_csr_rows_16(None, None, None, None, None, 0, 0, 8, 2, None) == 0
    # 16-bit row softmax
    assert lib.as_csr_row_softmax_16(None, None, None, 4, 8, 3, None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_csr_row_softmax_16(None, 1, None, 4, 8, 1, None) == 1
    assert lib.as_last_error() == b"scores and probs must be 2-byte aligned"
    assert lib.as_csr_row_softmax_16(None, None, None, 4, 8, 2, None) == 1
    assert lib.as_last_error() == b"null pointer argument"
    assert lib.as_csr_row_softmax_16(None, None, None, 0, 0, 2, None) == 0
    # 16-bit SDDMM: dtype code, split arguments, alignment, null inputs
    assert lib.as_sddmm_csr_rounded_16(None, None, None, None, None, 4, 0, 8, 3, 4, 1024, None, 0, None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_sddmm_csr_rounded_16(None, None, None, None, None, 4, 0, 8, 1, 3, 1024, None, 0, None) == 1
    assert lib.as_last_error() == b"warps_per_block must be 2, 4, or 8"
    assert lib.as_sddmm_csr_rounded_16(None, None, None, None, None, 4, 0, 8, 1, 4, 0, None, 0, None) == 1
    assert lib.as_last_error() == b"hub_threshold must be a positive 32-bit integer"
    assert lib.as_sddmm_csr_rounded_16(None, None, 1, None, None, 4, 0, 8, 2, 4, 1024, None, 0, None) == 1
    assert lib.as_last_error() == b"query, key and out must be 2-byte aligned"
    assert lib.as_sddmm_csr_rounded_16(None, None, None, None, None, 4, 5, 8, 2, 4, 1024, None, 0, None) == 1
    assert lib.as_last_error() == b"null crow pointer"
    # the same checks for the edge-block schedule, then its workspace (one
    # int32 per wavefront of 128 edges, in 256-byte units)
    assert lib.as_sddmm_csr_edges_16(None, None, None, None, None, 4, 0, 8, 3, None, 0, None) == 1
    assert lib.as_last_error() == b"dtype must be AS_DTYPE_BF16 or AS_DTYPE_F16"
    assert lib.as_sddmm_csr_edges_16(None, None, 1, None, None, 4, 0, 8, 2, None, 0, None) == 1
    assert lib.as_last_error() == b"query, key and out must be 2-byte aligned"
    assert lib.as_sddmm_csr_edges_16(None, None, None, None, None, 4, 5, 8, 2, None, 0, None) == 1
    assert lib.as_last_error() == b"null crow pointer"
    assert lib.as_sddmm_csr_edges_16(None, None, None, None, None, 0, 0, 8, 2, None, 0, None) == 0
    fake = 256
    assert lib.as_sddmm_csr_edges_16(fake, fake, fake, fake, fake, 4, 5, 8, 1, fake, 255, None) == 4
    assert lib.as_last_error().startswith(b"16-bit SDDMM by edge blocks needs 256 workspace bytes")
    assert [lib.as_sddmm_edges_16_workspace_bytes(e) for e in (0, 1, 128 * 64, 128 * 64 + 1, -5)] == [
        256, 256, 256, 512, 256]
    assert [lib.as_spmm_rounded_16_group_degree(f) for f in (8, 64, 72, 128, 136, 512, 7, 0)] == [
        32, 32, 64, 64, 128, 128, 0, 0]
    # n == 0 is a no-op success
    assert lib.as_spmm_csr_f32(None, None, None, None, None, 0, 0, 8, 1, None) == 0
    # feature widths from 2^28 on are refused (the kernels' lane offsets in a
    # feature row are 32-bit), before any pointer is looked at
    big = 1 << 28
    assert lib.as_spmm_csr_f32(None, None, None, None, None, 4, 0, big, 1, None) == 3
    assert lib.as_last_error() == b"F must be below 2^28 (32-bit lane offsets)"
    assert lib.as_spmm_csr_rows_16(None, None, None, None, None, 4, 0, big, 1, None) == 3
    assert lib.as_spmm_csr_rounded_16(None, None, None, None, None, 4, 0, big, 1, 1, None, 0, -1, -1, None) == 3
    assert lib.as_spmm_csr_colslice_f32(None, None, None, None, None, 4, 0, big, None, 0, -1, None) == 3
    assert lib.as_sddmm_csr_f32(None, None, None, None, None, 4, 0, big, None) == 3
    assert lib.as_sddmm_csr_rounded_16(None, None, None, None, None, 4, 0, big, 1, 4, 1024, None, 0, None) == 3
    assert lib.as_sddmm_csr_edges_16(None, None, None, None, None, 4, 0, big, 1, None, 0, None) == 3
    assert lib.as_csr_attention_f32(None, None, None, None, None, None, 4, 0, 8, big, 1.0, None, 0, None) == 3
    assert lib.as_last_error() == b"F_qk and F_v must be below 2^28 (32-bit lane offsets)"
    assert lib.as_spmm_csr_f32(None, None, None, None, None, 4, 0, -1, 1, None) == 1


def test_library_targets_gfx950_only():
    data = _native.package_library_path().read_bytes() if _native.package_library_path().exists() else b""
    if not data:
        pytest.skip("HIP library not built")
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in data
