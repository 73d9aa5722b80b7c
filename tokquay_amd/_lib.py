"""ctypes binding of ``libtokquay_amd.so`` (declared in ``include/tokquay_amd.h``).

There is no fallback: if the library has not been built, :func:`lib` raises.
"""

from __future__ import annotations

import ctypes
import os

from tokquay_amd.build import LIB_PATH

c_f32p = ctypes.c_void_p  # device pointers travel as plain addresses
c_i32p = ctypes.c_void_p
c_i64p = ctypes.c_void_p

TQ_OK = 0
STATIC_SCRATCH_BYTES = 8 << 20  # TQ_STATIC_SCRATCH_BYTES: tq_paged_decode_write_static's per-GPU array
STATUS_NAMES = {0: "ok", 1: "invalid argument", 2: "unsupported shape", 3: "workspace missing or too small", 4: "HIP runtime error"}

# Bits kernels OR into the optional device error word.
DEVERR_BLOCK_ID = 1
DEVERR_SLOT = 2
DEVERR_LENGTH = 4
DEVERR_ORDER = 8

# name -> (restype, argtypes); the order of argtypes is the C declaration's.
SIGNATURES: dict[str, tuple] = {
    "tq_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "tq_abi_version": (ctypes.c_int32, []),
    "tq_last_hip_error": (ctypes.c_char_p, []),
    "tq_set_timing_events": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "tq_cache_write": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,  # pool, num_blocks, num_layers, num_heads
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # block_size, head_dim, layer
            c_f32p, ctypes.c_int64,  # k, k_row_stride
            c_f32p, ctypes.c_int64,  # v, v_row_stride
            c_i64p, ctypes.c_int64,  # slot_mapping, num_tokens
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_decode": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64,  # out, out_row_stride
            c_f32p, ctypes.c_int64,  # q, q_row_stride
            c_f32p, ctypes.c_int64, ctypes.c_int32,  # pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # block_tables, block_table_stride, max_blocks_per_seq
            c_i32p, c_i32p, ctypes.c_int32, ctypes.c_int32,  # context_lens, seq_order, num_seqs, max_context_len
            ctypes.c_float, ctypes.c_int32,  # scale, partition_tokens
            ctypes.c_void_p, ctypes.c_size_t,  # workspace, workspace_bytes
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_decode_write": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64,  # out, out_row_stride
            c_f32p, ctypes.c_int64,  # q, q_row_stride
            c_f32p, ctypes.c_int64,  # k_new, k_new_row_stride
            c_f32p, ctypes.c_int64,  # v_new, v_new_row_stride
            c_f32p, ctypes.c_int64, ctypes.c_int32,  # pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # block_tables, block_table_stride, max_blocks_per_seq
            c_i32p, c_i32p, ctypes.c_int32, ctypes.c_int32,  # context_lens, seq_order, num_seqs, max_context_len
            ctypes.c_float, ctypes.c_int32,  # scale, partition_tokens
            ctypes.c_void_p, ctypes.c_size_t,  # workspace, workspace_bytes
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_decode_write_static": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64,  # out, out_row_stride
            c_f32p, ctypes.c_int64,  # q, q_row_stride
            c_f32p, ctypes.c_int64,  # k_new, k_new_row_stride
            c_f32p, ctypes.c_int64,  # v_new, v_new_row_stride
            c_f32p, ctypes.c_int64, ctypes.c_int32,  # pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # block_tables, block_table_stride, max_blocks_per_seq
            c_i32p, c_i32p, ctypes.c_int32, ctypes.c_int32,  # context_lens, seq_order, num_seqs, max_context_len
            ctypes.c_float, ctypes.c_int32,  # scale, partition_tokens
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_gather": (
        ctypes.c_int,
        [
            c_f32p, c_f32p, c_f32p, ctypes.c_int64, ctypes.c_int32,  # k_out, v_out, pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            c_i32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,  # block_tables, stride, gathered blocks, num_seqs
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_decode_workspace_size": (
        ctypes.c_size_t,
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32],
    ),
    "tq_paged_prefill": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64,  # out, out_row_stride
            c_f32p, ctypes.c_int64,  # q, q_row_stride
            c_f32p, ctypes.c_int64, ctypes.c_int32,  # pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # block_tables, block_table_stride, max_blocks_per_seq
            c_i32p, c_i32p, c_i32p,  # cu_seqlens_q, q_start, seq_order
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_seqs, num_q_rows, max_query_len
            ctypes.c_float, c_i32p, ctypes.c_void_p,  # scale, d_error, stream
        ],
    ),
    "tq_paged_mixed": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64,  # dec_out, dec_out_row_stride, dec_q, dec_q_row_stride
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64,  # k_new, k_new_row_stride, v_new, v_new_row_stride
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # dec_block_tables, dec_block_table_stride, dec_max_blocks_per_seq
            c_i32p, c_i32p,  # context_lens, seq_order
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_decode_seqs, max_context_len, partition_tokens
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64,  # pre_out, pre_out_row_stride, pre_q, pre_q_row_stride
            c_i32p, ctypes.c_int64, ctypes.c_int32,  # pre_block_tables, pre_block_table_stride, pre_max_blocks_per_seq
            c_i32p, c_i32p,  # cu_seqlens_q, q_start
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_prefill_seqs, num_q_rows, max_query_len
            c_f32p, ctypes.c_int64, ctypes.c_int32,  # pool, num_blocks, num_layers
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,  # num_heads, block_size, head_dim, layer
            ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t,  # scale, workspace, workspace_bytes
            c_i32p, ctypes.c_void_p,  # d_error, stream
        ],
    ),
    "tq_paged_mixed_workspace_size": (ctypes.c_size_t, [ctypes.c_int32] * 8),
    "tq_add_layernorm": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64,  # x_out, stride, h_out, stride
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64,  # x, stride, y, stride
            c_f32p, c_f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p,  # gamma, beta, rows, cols, eps, stream
        ],
    ),
    "tq_skinny_linear": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64, c_f32p, ctypes.c_int64, ctypes.c_int32,  # y, y_stride, x, x_stride, M
            c_f32p, c_f32p, ctypes.c_int32, ctypes.c_int32,  # w, bias, N, K
            c_f32p, c_f32p, ctypes.c_float, ctypes.c_int32,  # ln_gamma, ln_beta, ln_eps, epilogue
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "tq_skinny_linear_argmax": (
        ctypes.c_int,
        [
            c_i64p, c_f32p, ctypes.c_int64, ctypes.c_int32,  # ids, x, x_stride, M
            c_f32p, c_f32p, ctypes.c_int32, ctypes.c_int32,  # w, bias, N, K
            c_f32p, c_f32p, ctypes.c_float,  # ln_gamma, ln_beta, ln_eps
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,  # workspace, workspace_bytes, stream
        ],
    ),
    "tq_skinny_linear_argmax_workspace_size": (ctypes.c_size_t, [ctypes.c_int32]),
    "tq_skinny_linear_workspace_size": (ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]),
    "tq_embed_rows": (
        ctypes.c_int,
        [
            c_f32p, ctypes.c_int64, c_i64p, c_i64p, c_i64p, c_i64p,  # x, x_stride, ids, src, tokens, positions
            c_f32p, c_f32p, ctypes.c_int64, ctypes.c_int32,  # wte, wpe, rows, C
            ctypes.c_int64, ctypes.c_int64, c_i32p, ctypes.c_void_p,  # vocab, n_positions, d_error, stream
        ],
    ),
    "tq_argmax_rows": (
        ctypes.c_int,
        [c_i64p, c_f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p],  # out, logits, rows, cols, row_stride, stream
    ),
}

_lib: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A C-ABI entry point returned a status other than TQ_OK."""


def lib() -> ctypes.CDLL:
    """The loaded library with every signature bound; raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP kernels first "
                "(python -m tokquay_amd.build, or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != TQ_OK:
        msg = STATUS_NAMES.get(status, f"status {status}")
        if status == 4:
            msg += f": {lib().tq_last_hip_error().decode(errors='replace')}"
        raise KernelError(f"{what} failed: {msg}")


_native = None


def native():
    """The ``_native`` extension (metadata builder and per-layer launcher); raises if it was never built."""
    global _native
    if _native is None:
        from tokquay_amd.build import NATIVE_PATH

        if not os.path.exists(NATIVE_PATH):
            raise RuntimeError(
                f"{NATIVE_PATH} is missing: build it first (python -m tokquay_amd.build, or __graft_entry__.build())"
            )
        lib()  # binds the kernel library the extension links (same file, loaded once)
        from tokquay_amd import _native as mod

        _native = mod
    return _native
