"""``torch.ops.tokquay_amd.*``: the paged-attention entry points as torch operators.

``csrc/torch_ops.cpp`` (built into ``_torch_ops.so`` next to ``libtokquay_amd.so``) registers seven
out-variant operators with torch's dispatcher; each is a thin call into the C ABI on the current
HIP stream. This module loads that library and registers the operators' fake (shape-only)
implementations, so programs that record torch calls (``make_fx``, FX graphs on fake tensors)
see the kernels as single operators:

* ``cache_write(pool!, layer, k, v, slot_mapping, d_error!?)``
* ``paged_decode(out!, q, pool, layer, block_tables, context_lens, max_context_len, scale,
  partition_tokens, workspace?, d_error!?, seq_order?)``
* ``paged_decode_write(out!, q, k_new, v_new, pool!, layer, ...)`` (the same, with the cache write)
* ``paged_prefill(out!, q, pool, layer, block_tables, cu_seqlens_q, q_start, max_query_len, scale,
  d_error!?)``
* ``paged_mixed(dec_out!, dec_q, k_new, v_new, dec_block_tables, context_lens, max_context_len,
  pre_out!, pre_q, pre_block_tables, cu_seqlens_q, q_start, max_query_len, pool!, layer, scale,
  partition_tokens, workspace?, d_error!?, seq_order?)``
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


def _fake(*args, **kwargs) -> None:
    """Shape-only implementation: every operator writes into tensors it is given and returns nothing."""
    return None


def load():
    """``torch.ops.tokquay_amd`` with the operators registered; raises if the library was never built."""
    global _loaded
    if not _loaded:
        if not os.path.exists(TORCH_OPS_PATH):
            raise RuntimeError(f"{TORCH_OPS_PATH} is missing: build it first (python -m tokquay_amd.build)")
        torch.ops.load_library(TORCH_OPS_PATH)
        for name in OPS:
            torch.library.register_fake(f"tokquay_amd::{name}")(_fake)
        _loaded = True
    return torch.ops.tokquay_amd
