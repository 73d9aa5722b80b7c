"""``torch.ops.tokquay_amd.*``: the paged-attention entry points as torch operators.

``csrc/torch_ops.cpp`` (built into ``_torch_ops.so`` next to ``libtokquay_amd.so``) registers seven
out-variant operators with torch's dispatcher; each is a thin call into the C ABI on the current
HIP stream. This module loads that library and registers the operators' fake (shape-only)
implementations, so programs that record torch calls (``make_fx``, FX graphs on fake tensors)
see the kernels as single operators. Both the operators and their fakes refuse, before any launch,
every tensor a kernel would read or write past: wrong device, dtype or inner layout, too few rows
or entries, overlapping rows:

* ``cache_write(pool!, layer, k, v, slot_mapping, d_error!?)``
* ``paged_decode(out!, q, pool, layer, block_tables, context_lens, max_context_len, scale,
  partition_tokens, workspace!?, d_error!?, seq_order?)``
* ``paged_decode_write(out!, q, k_new, v_new, pool!, layer, ...)`` (the same, with the cache write)
* ``paged_prefill(out!, q, pool, layer, block_tables, cu_seqlens_q, q_start, max_query_len, scale,
  d_error!?, seq_order?)``
* ``paged_mixed(dec_out!, dec_q, k_new, v_new, dec_block_tables, context_lens, max_context_len,
  pre_out!, pre_q, pre_block_tables, cu_seqlens_q, q_start, max_query_len, pool!, layer, scale,
  partition_tokens, workspace!?, d_error!?, seq_order?)``
* ``paged_gather(k_out!, v_out!, pool, layer, block_tables, d_error!?)`` (the reference view's
  gathered copy)
* ``argmax_rows(logits, out!)``

(``!``: written in place.) ``tokquay_amd.ops`` checks the tensors with the reference's messages
and calls these operators; there is no fallback when the library is missing.
"""

from __future__ import annotations

import os

import torch

from tokquay_amd.build import TORCH_OPS_PATH

OPS = ("cache_write", "paged_decode", "paged_decode_write", "paged_prefill", "paged_mixed", "paged_gather",
       "argmax_rows")

_loaded = False

# ---- fake (shape-only) implementations. Each runs the checks its C++ operator runs before a
# launch (csrc/torch_ops.cpp), with the same messages, and writes nothing.


def _fail(op: str, msg: str) -> None:
    raise RuntimeError(f"tokquay_amd::{op}: {msg}")


def _pool_of(op, pool, layer):
    if not (pool.dim() == 6 and pool.size(2) == 2 and pool.dtype == torch.float32 and pool.is_contiguous()
            and pool.is_cuda):  # fmt: skip
        _fail(op, "pool must be a contiguous float32 [num_blocks, n_layer, 2, n_head, block_size, d_head] tensor "
                  "on a HIP device")  # fmt: skip
    if pool.size(5) != 64:
        _fail(op, f"only d_head 64 is supported, got {pool.size(5)}")
    if not 0 <= layer < pool.size(1):
        _fail(op, f"layer {layer} out of range [0, {pool.size(1)})")
    return pool


def _on_device(op, name, t, pool):
    if t.device != pool.device:
        _fail(op, f"{name} is on {t.device}, the pool on {pool.device}")


def _rows_of(op, name, t, rows, pool):
    _on_device(op, name, t, pool)
    heads, d = pool.size(3), pool.size(5)
    ok = t.dtype == torch.float32
    if t.dim() == 3:
        ok = ok and t.size(1) == heads and t.size(2) == d and t.stride(2) == 1 and t.stride(1) == d
    elif t.dim() == 2:
        ok = ok and t.size(1) == heads * d and t.stride(1) == 1
    else:
        ok = False
    if not ok:
        _fail(op, f"{name} must be float32 [N, {heads}, {d}] or [N, {heads * d}] with contiguous rows")
    if t.size(0) < rows:
        _fail(op, f"{name} has {t.size(0)} rows, needs {rows}")
    if rows > 1 and t.stride(0) < heads * d:
        _fail(op, f"{name}'s rows overlap (row stride {t.stride(0)})")


def _vector_of(op, name, t, dtype, n, pool):
    _on_device(op, name, t, pool)
    if t.dtype != dtype or not t.is_contiguous():
        _fail(op, f"{name} must be a contiguous {dtype} tensor")
    if t.numel() < n:
        _fail(op, f"{name} has {t.numel()} entries, needs {n}")


def _tables_of(op, name, t, rows, pool):
    _on_device(op, name, t, pool)
    if not (t.dtype == torch.int32 and t.dim() == 2 and (t.size(1) <= 1 or t.stride(1) == 1)):
        _fail(op, f"{name} must be an int32 [B, max_blocks] tensor with contiguous rows")
    if t.size(0) < rows:
        _fail(op, f"{name} has {t.size(0)} rows, needs {rows}")
    if rows > 1 and t.stride(0) < t.size(1):
        _fail(op, f"{name}'s rows overlap")


def _error_word(op, t, pool):
    if t is not None:
        _vector_of(op, "d_error", t, torch.int32, 1, pool)


def _workspace(op, t, pool):
    if t is not None:
        _on_device(op, "workspace", t, pool)
        if not t.is_contiguous():
            _fail(op, "workspace must be contiguous")


def _fake_cache_write(pool, layer, k, v, slot_mapping, d_error):
    op = "cache_write"
    _pool_of(op, pool, layer)
    _vector_of(op, "slot_mapping", slot_mapping, torch.int64, 0, pool)
    n = slot_mapping.numel()
    _rows_of(op, "k", k, n, pool)
    _rows_of(op, "v", v, n, pool)
    _error_word(op, d_error, pool)


def _decode_args(op, pool, out, q, block_tables, context_lens, d_error, seq_order):
    _vector_of(op, "context_lens", context_lens, torch.int32, 0, pool)
    n = context_lens.numel()
    _rows_of(op, "out", out, n, pool)
    _rows_of(op, "q", q, n, pool)
    _tables_of(op, "block_tables", block_tables, n, pool)
    if seq_order is not None:
        _vector_of(op, "seq_order", seq_order, torch.int32, n, pool)
    _error_word(op, d_error, pool)
    return n


def _fake_paged_decode(out, q, pool, layer, block_tables, context_lens, max_context_len, scale, partition_tokens,
                       workspace, d_error, seq_order):  # fmt: skip
    op = "paged_decode"
    _pool_of(op, pool, layer)
    _decode_args(op, pool, out, q, block_tables, context_lens, d_error, seq_order)
    _workspace(op, workspace, pool)


def _fake_paged_decode_write(out, q, k_new, v_new, pool, layer, block_tables, context_lens, max_context_len, scale,
                             partition_tokens, workspace, d_error, seq_order):  # fmt: skip
    op = "paged_decode_write"
    _pool_of(op, pool, layer)
    n = _decode_args(op, pool, out, q, block_tables, context_lens, d_error, seq_order)
    _rows_of(op, "k_new", k_new, n, pool)
    _rows_of(op, "v_new", v_new, n, pool)
    _workspace(op, workspace, pool)


def _prefill_args(op, pool, out, q, out_name, q_name, tables_name, block_tables, cu_seqlens_q, q_start):
    _vector_of(op, "q_start", q_start, torch.int32, 0, pool)
    n = q_start.numel()
    _vector_of(op, "cu_seqlens_q", cu_seqlens_q, torch.int32, n + 1, pool)
    if cu_seqlens_q.numel() != n + 1:
        _fail(op, "cu_seqlens_q must have num_seqs + 1 entries")
    _rows_of(op, q_name, q, q.size(0), pool)
    _rows_of(op, out_name, out, q.size(0), pool)
    _tables_of(op, tables_name, block_tables, n, pool)


def _fake_paged_prefill(out, q, pool, layer, block_tables, cu_seqlens_q, q_start, max_query_len, scale, d_error,
                        seq_order):  # fmt: skip
    op = "paged_prefill"
    _pool_of(op, pool, layer)
    _prefill_args(op, pool, out, q, "out", "q", "block_tables", block_tables, cu_seqlens_q, q_start)
    if seq_order is not None:
        _vector_of(op, "seq_order", seq_order, torch.int32, q_start.numel(), pool)
    _error_word(op, d_error, pool)


def _fake_paged_mixed(dec_out, dec_q, k_new, v_new, dec_block_tables, context_lens, max_context_len, pre_out, pre_q,
                      pre_block_tables, cu_seqlens_q, q_start, max_query_len, pool, layer, scale, partition_tokens,
                      workspace, d_error, seq_order):  # fmt: skip
    op = "paged_mixed"
    _pool_of(op, pool, layer)
    n = _decode_args(op, pool, dec_out, dec_q, dec_block_tables, context_lens, d_error, seq_order)
    _rows_of(op, "k_new", k_new, n, pool)
    _rows_of(op, "v_new", v_new, n, pool)
    _prefill_args(op, pool, pre_out, pre_q, "pre_out", "pre_q", "pre_block_tables", pre_block_tables, cu_seqlens_q,
                  q_start)  # fmt: skip
    _workspace(op, workspace, pool)


def _fake_paged_gather(k_out, v_out, pool, layer, block_tables, d_error):
    op = "paged_gather"
    _pool_of(op, pool, layer)
    if block_tables.dim() != 2:
        _fail(op, "block_tables must be an int32 [B, max_blocks] tensor")
    n = block_tables.size(0)
    _tables_of(op, "block_tables", block_tables, n, pool)
    shape = (n, pool.size(3), block_tables.size(1) * pool.size(4), pool.size(5))
    for name, t in (("k_out", k_out), ("v_out", v_out)):
        _on_device(op, name, t, pool)
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape:
            _fail(op, f"{name} must be a contiguous float32 tensor of shape {list(shape)}")
    _error_word(op, d_error, pool)


def _fake_argmax_rows(logits, out):
    op = "argmax_rows"
    if not (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2
            and (logits.size(1) <= 1 or logits.stride(1) == 1)):  # fmt: skip
        _fail(op, "logits must be a float32 [rows, vocab] tensor on a HIP device with contiguous rows")
    if logits.size(0) > 1 and logits.stride(0) < logits.size(1):
        _fail(op, "logits' rows overlap")
    if not (out.device == logits.device and out.dtype == torch.int64 and out.is_contiguous()
            and out.numel() >= logits.size(0)):  # fmt: skip
        _fail(op, "out must be a contiguous int64 tensor with one entry per row, on the logits' device")


FAKES = {name: globals()[f"_fake_{name}"] for name in OPS}


def load():
    """``torch.ops.tokquay_amd`` with the operators registered; raises if the library was never built."""
    global _loaded
    if not _loaded:
        if not os.path.exists(TORCH_OPS_PATH):
            raise RuntimeError(f"{TORCH_OPS_PATH} is missing: build it first (python -m tokquay_amd.build)")
        torch.ops.load_library(TORCH_OPS_PATH)
        for name in OPS:
            torch.library.register_fake(f"tokquay_amd::{name}")(FAKES[name])
        _loaded = True
    return torch.ops.tokquay_amd
