"""The C-ABI library loads on a host without a GPU and exports every symbol the header declares.

Only host-side argument checks are exercised here (they return before any HIP
call); nothing is launched.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from tokquay_amd import _lib
from tokquay_amd.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "tokquay_amd.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.lib()


def test_header_declares_the_three_kernels_and_helpers():
    names = declared_functions()
    for n in ("tq_cache_write", "tq_paged_decode", "tq_paged_decode_write", "tq_paged_prefill", "tq_argmax_rows",
              "tq_paged_decode_workspace_size",
              "tq_status_string", "tq_abi_version", "tq_last_hip_error"):  # fmt: skip
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(declared_functions()) == set(_lib.SIGNATURES), "ctypes bindings and header disagree"


def test_status_strings_and_version(lib):
    assert lib.tq_abi_version() == 3
    assert lib.tq_status_string(0) == b"ok"
    assert lib.tq_status_string(3) == b"workspace missing or too small"
    assert lib.tq_last_hip_error() == b""


def test_invalid_arguments_are_rejected_before_any_launch(lib):
    # num_blocks = 0
    assert lib.tq_cache_write(None, 0, 1, 12, 16, 64, 0, None, 768, None, 768, None, 1, None, None) == 1
    # layer out of range
    assert lib.tq_cache_write(None, 8, 2, 12, 16, 64, 2, None, 768, None, 768, None, 1, None, None) == 1
    # head_dim 128 is not built
    assert lib.tq_cache_write(None, 8, 2, 12, 16, 128, 0, None, 768, None, 768, None, 1, None, None) == 2
    # zero tokens is a no-op
    assert lib.tq_cache_write(None, 8, 2, 12, 16, 64, 0, None, 768, None, 768, None, 0, None, None) == 0
    # decode: null pointers with sequences to do
    assert lib.tq_paged_decode(None, 768, None, 768, None, 8, 1, 12, 16, 64, 0, None, 4, 4, None, None, 2, 64,
                               0.125, 0, None, 0, None, None) == 1  # fmt: skip
    # decode: partition not a multiple of 16
    assert lib.tq_paged_decode(None, 768, None, 768, None, 8, 1, 12, 16, 64, 0, None, 4, 4, None, None, 2, 64,
                               0.125, 24, None, 0, None, None) == 1  # fmt: skip
    # decode with the write folded in: null new rows with sequences to do
    assert lib.tq_paged_decode_write(None, 768, None, 2304, None, 2304, None, 2304, None, 8, 1, 12, 16, 64, 0,
                                     None, 4, 4, None, None, 2, 64, 0.125, 0, None, 0, None, None) == 1  # fmt: skip
    # ... new-row stride shorter than a row of heads
    assert lib.tq_paged_decode_write(None, 768, None, 2304, 16, 700, 16, 2304, None, 8, 1, 12, 16, 64, 0,
                                     None, 4, 4, None, None, 2, 64, 0.125, 0, None, 0, None, None) == 1  # fmt: skip
    # ... zero sequences is a no-op
    assert lib.tq_paged_decode_write(None, 768, None, 2304, None, 2304, None, 2304, None, 8, 1, 12, 16, 64, 0,
                                     None, 4, 4, None, None, 0, 64, 0.125, 0, None, 0, None, None) == 0  # fmt: skip
    # prefill: zero sequences is a no-op
    assert lib.tq_paged_prefill(None, 768, None, 768, None, 8, 1, 12, 16, 64, 0, None, 4, 4, None, None, None,
                                0, 0, 0, 0.125, None, None) == 0  # fmt: skip
    # prefill: null pointers with rows to do
    assert lib.tq_paged_prefill(None, 768, None, 768, None, 8, 1, 12, 16, 64, 0, None, 4, 4, None, None, None,
                                2, 32, 16, 0.125, None, None) == 1  # fmt: skip


def test_decode_workspace_size(lib):
    # Contexts that fit one partition need no workspace.
    assert lib.tq_paged_decode_workspace_size(64, 12, 64, 200, 256) == 0
    # 256 sequences x 12 heads x 4 partitions of 256 x (64 + 4) floats.
    assert lib.tq_paged_decode_workspace_size(256, 12, 64, 1024, 256) == 256 * 12 * 4 * 68 * 4
    # Automatic: 3072 (sequence, head) pairs already fill the GPU, so one 1024-position partition each.
    assert lib.tq_paged_decode_workspace_size(256, 12, 64, 1024, 0) == 0
    # Automatic, small batches: one workgroup of several waves per (sequence, head), merged in LDS.
    assert lib.tq_paged_decode_workspace_size(64, 12, 64, 512, 0) == 0
    assert lib.tq_paged_decode_workspace_size(4, 12, 64, 1024, 0) == 0
    # Explicit partition sizes keep the partition grid and its partials.
    assert lib.tq_paged_decode_workspace_size(64, 12, 64, 512, 128) == 64 * 12 * 4 * 68 * 4
    assert lib.tq_paged_decode_workspace_size(4, 12, 64, 1024, 32) == 4 * 12 * 32 * 68 * 4
    # Beyond 16 waves x 1024 positions the automatic choice falls back to the partition grid.
    assert lib.tq_paged_decode_workspace_size(1, 12, 64, 32768, 0) == 1 * 12 * 256 * 68 * 4  # 128-position
    assert lib.tq_paged_decode_workspace_size(4, 12, 64, 1024, 20) == 0  # invalid partition
    assert lib.tq_paged_decode_workspace_size(4, 12, 64, 4096, 2048) == 0  # partitions are at most 1024


def test_small_batch_entries_reject_bad_shapes_before_any_launch(lib):
    # tq_skinny_linear(y, y_stride, x, x_stride, M, w, bias, N, K, ln_gamma, ln_beta, ln_eps, epilogue, stream)
    f = lambda *a: lib.tq_skinny_linear(*a, None, 0, None)  # noqa: E731
    assert f(None, 8, None, 768, 65, None, None, 8, 768, None, None, 0.0, 0) == 2  # M > 64
    assert f(None, 8, None, 512, 2, None, None, 8, 512, None, None, 0.0, 0) == 2  # K
    assert f(None, 8, None, 768, 2, None, None, 8, 768, None, None, 0.0, 3) == 1  # epilogue
    assert f(None, 8, None, 768, 0, None, None, 8, 768, None, None, 0.0, 0) == 0  # no rows
    assert f(None, 2304, None, 768, 2, None, None, 2304, 768, None, None, 0.0, 0) == 1  # null y
    assert f(None, 768, None, 3072, 2, None, None, 768, 3072, 1, 1, 1e-5, 0) == 2  # LN over K = 3072
    # Split K without a workspace is refused before any launch (the addresses are never dereferenced).
    assert f(4096, 768, 4096, 3072, 2, 4096, None, 768, 3072, None, None, 0.0, 2) == 3
    ws = lib.tq_skinny_linear_workspace_size
    assert ws(16, 2304, 768, 1) == 0 and ws(16, 768, 768, 0) == 0 and ws(16, 768, 3072, 0) > 0
    # partial tiles per row group: one of 16 rows, or groups of 32
    assert ws(64, 768, 3072, 0) == ws(33, 768, 3072, 0) > ws(32, 768, 3072, 0) > ws(16, 768, 3072, 0)
    assert ws(16, 768, 3072, 1) == 0 and ws(65, 768, 3072, 0) == 0  # unsupported shapes
    # tq_embed_rows(x, x_stride, ids, src, tokens, positions, wte, wpe, rows, C, vocab, n_positions, d_error, stream)
    assert lib.tq_embed_rows(None, 768, None, None, None, None, None, None, 0, 768, 10, 10, None, None) == 0
    assert lib.tq_embed_rows(None, 768, None, None, None, None, None, None, 3, 766, 10, 10, None, None) == 2
    assert lib.tq_embed_rows(None, 768, None, None, None, None, None, None, 3, 768, 10, 10, None, None) == 1
