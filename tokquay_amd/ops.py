"""Tensor-level entry points of the gfx950 paged-attention kernels.

Each function checks its tensors (device, dtype, shapes, inner contiguity),
then calls the C ABI (``include/tokquay_amd.h``) on torch's current HIP
stream. Nothing here computes on the host and nothing synchronises.

Shapes (fp32 unless noted; ``H`` heads of ``D = 64`` dims):

* ``pool``: ``[num_blocks, n_layer, 2, H, block_size, D]`` contiguous, the
  reference's pool layout (tokquay/kv_cache.py:5, :51-53).
* q / k / v / out rows: ``[N, H, D]`` or ``[N, H*D]``; any row stride, rows
  contiguous inside (so views of the fused QKV projection output work).
* ``block_tables``: int32 ``[B, max_blocks]``, rows padded with any valid id.
* ``slot_mapping``: int64 ``[N]``; -1 marks a padded token that writes nothing.
"""

from __future__ import annotations

import math

import torch

from tokquay_amd import _lib, torch_ops

HEAD_DIM = 64


def _op(name: str, *args) -> None:
    """Calls ``torch.ops.tokquay_amd.<name>``; a failed C-ABI status raises ``_lib.KernelError``."""
    try:
        getattr(torch_ops.load(), name)(*args)
    except RuntimeError as e:
        first = str(e).splitlines()[0] if str(e) else ""
        if " failed: " in first and first.startswith("tq_"):
            raise _lib.KernelError(first) from None
        raise


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _pool_dims(pool: torch.Tensor) -> tuple[int, int, int, int, int]:
    if pool.dim() != 6 or pool.size(2) != 2:
        raise ValueError(f"pool must be [num_blocks, n_layer, 2, n_head, block_size, d_head], got {tuple(pool.shape)}")
    if pool.dtype != torch.float32 or not pool.is_cuda or not pool.is_contiguous():
        raise ValueError("pool must be a contiguous float32 tensor on a HIP device")
    nb, n_layer, _, n_head, bs, d = pool.shape
    if d != HEAD_DIM:
        raise ValueError(f"only d_head={HEAD_DIM} is supported, got {d}")
    return nb, n_layer, n_head, bs, d


def _rows(t: torch.Tensor, name: str, n: int, n_head: int, device: torch.device) -> int:
    """Validates a row tensor and returns its row stride in elements."""
    if t.dtype != torch.float32 or t.device != device:
        raise ValueError(f"{name} must be float32 on {device}")
    if t.size(0) != n:
        raise ValueError(f"{name} has {t.size(0)} rows, expected {n}")
    if t.dim() == 3:
        ok = t.size(1) == n_head and t.size(2) == HEAD_DIM and t.stride(2) == 1 and t.stride(1) == HEAD_DIM
    elif t.dim() == 2:
        ok = t.size(1) == n_head * HEAD_DIM and t.stride(1) == 1
    else:
        ok = False
    if not ok:
        raise ValueError(f"{name} must be [N, {n_head}, {HEAD_DIM}] or [N, {n_head * HEAD_DIM}] with contiguous rows")
    return t.stride(0) if n > 1 else n_head * HEAD_DIM


def _int_tensor(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device) -> None:
    if t.dtype != dtype or t.device != device or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor on {device}")


def cache_write(
    pool: torch.Tensor,
    layer: int,
    k: torch.Tensor,
    v: torch.Tensor,
    slot_mapping: torch.Tensor,
    d_error: torch.Tensor | None = None,
) -> None:
    """Scatter ``k``/``v`` rows into ``pool[:, layer]`` at ``slot_mapping`` (bit-exact copy)."""
    nb, n_layer, n_head, bs, d = _pool_dims(pool)
    if not 0 <= layer < n_layer:
        raise ValueError(f"layer {layer} out of range [0, {n_layer})")
    n = slot_mapping.numel()
    _int_tensor(slot_mapping, "slot_mapping", torch.int64, pool.device)
    _rows(k, "k", n, n_head, pool.device)
    _rows(v, "v", n, n_head, pool.device)
    _op("cache_write", pool, layer, k, v, slot_mapping, d_error)


def decode_workspace_bytes(num_seqs: int, n_head: int, max_context_len: int, partition_tokens: int = 0) -> int:
    return int(_lib.lib().tq_paged_decode_workspace_size(num_seqs, n_head, HEAD_DIM, max_context_len, partition_tokens))


def paged_decode(
    out: torch.Tensor,
    q: torch.Tensor,
    pool: torch.Tensor,
    layer: int,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    max_context_len: int,
    scale: float | None = None,
    partition_tokens: int = 0,
    workspace: torch.Tensor | None = None,
    d_error: torch.Tensor | None = None,
    k_new: torch.Tensor | None = None,
    v_new: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
) -> None:
    """``out[b] = attention(q[b], keys/values 0..context_lens[b]-1 of sequence b)`` read in place.

    With ``k_new`` / ``v_new`` (rows like ``q``), row b's new K/V are first written into the
    slot of position ``context_lens[b] - 1`` (``tq_paged_decode_write``): the cache write of the
    one new token per sequence folded into the same launch. ``seq_order`` (int32 ``[B]``, a
    permutation) is the order the sequences are dispatched in; longest contexts first is fastest."""
    nb, n_layer, n_head, bs, d = _pool_dims(pool)
    if not 0 <= layer < n_layer:
        raise ValueError(f"layer {layer} out of range [0, {n_layer})")
    n = context_lens.numel()
    _int_tensor(context_lens, "context_lens", torch.int32, pool.device)
    if block_tables.dtype != torch.int32 or block_tables.device != pool.device or block_tables.dim() != 2:
        raise ValueError("block_tables must be an int32 [B, max_blocks] tensor on the pool's device")
    if block_tables.size(0) != n or (block_tables.size(1) > 1 and block_tables.stride(1) != 1):
        raise ValueError("block_tables must have one row per sequence with contiguous rows")
    _rows(q, "q", n, n_head, pool.device)
    _rows(out, "out", n, n_head, pool.device)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    need = decode_workspace_bytes(n, n_head, max_context_len, partition_tokens) if n else 0
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    if not need:
        workspace = None
    if seq_order is not None:
        _int_tensor(seq_order, "seq_order", torch.int32, pool.device)
        if seq_order.numel() != n:
            raise ValueError(f"seq_order needs {n} entries")
    tail = (layer, block_tables, context_lens, int(max_context_len), scale, partition_tokens, workspace, d_error,
            seq_order)  # fmt: skip
    if k_new is None and v_new is None:
        _op("paged_decode", out, q, pool, *tail)
        return
    if k_new is None or v_new is None:
        raise ValueError("k_new and v_new go together")
    _rows(k_new, "k_new", n, n_head, pool.device)
    _rows(v_new, "v_new", n, n_head, pool.device)
    _op("paged_decode_write", out, q, k_new, v_new, pool, *tail)


def paged_prefill(
    out: torch.Tensor,
    q: torch.Tensor,
    pool: torch.Tensor,
    layer: int,
    block_tables: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    q_start: torch.Tensor,
    max_query_len: int,
    scale: float | None = None,
    d_error: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
) -> None:
    """Causal attention of each sequence's new rows ``cu_seqlens_q[b]:cu_seqlens_q[b+1]`` (positions
    ``q_start[b]...``) over its keys ``0 .. q_start[b] + n_b - 1`` read in place from the pool.
    ``seq_order`` (int32 ``[B]``, a permutation): the order large launches deal the sequences in;
    most causal work first is fastest."""
    nb, n_layer, n_head, bs, d = _pool_dims(pool)
    if not 0 <= layer < n_layer:
        raise ValueError(f"layer {layer} out of range [0, {n_layer})")
    _int_tensor(cu_seqlens_q, "cu_seqlens_q", torch.int32, pool.device)
    _int_tensor(q_start, "q_start", torch.int32, pool.device)
    n_seq = q_start.numel()
    if cu_seqlens_q.numel() != n_seq + 1:
        raise ValueError("cu_seqlens_q must have num_seqs + 1 entries")
    if block_tables.dtype != torch.int32 or block_tables.device != pool.device or block_tables.dim() != 2:
        raise ValueError("block_tables must be an int32 [B, max_blocks] tensor on the pool's device")
    if block_tables.size(0) != n_seq or (block_tables.size(1) > 1 and block_tables.stride(1) != 1):
        raise ValueError("block_tables must have one row per sequence with contiguous rows")
    n_rows = q.size(0)
    _rows(q, "q", n_rows, n_head, pool.device)
    _rows(out, "out", n_rows, n_head, pool.device)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    if seq_order is not None:
        _int_tensor(seq_order, "seq_order", torch.int32, pool.device)
        if seq_order.numel() != n_seq:
            raise ValueError(f"seq_order needs {n_seq} entries")
    _op("paged_prefill", out, q, pool, layer, block_tables, cu_seqlens_q, q_start, int(max_query_len), scale, d_error,
        seq_order)  # fmt: skip


def _tables(t: torch.Tensor, name: str, n: int, device: torch.device) -> int:
    """Validates an int32 [B, max_blocks] block-table tensor and returns its row stride."""
    if t.dtype != torch.int32 or t.device != device or t.dim() != 2:
        raise ValueError(f"{name} must be an int32 [B, max_blocks] tensor on the pool's device")
    if t.size(0) != n or (t.size(1) > 1 and t.stride(1) != 1):
        raise ValueError(f"{name} must have one row per sequence with contiguous rows")
    return t.stride(0) if n > 1 else t.size(1)


def mixed_workspace_bytes(num_decode: int, n_head: int, max_context_len: int, partition_tokens: int,
                          num_prefill: int, num_q_rows: int, max_query_len: int) -> int:  # fmt: skip
    return int(_lib.lib().tq_paged_mixed_workspace_size(num_decode, n_head, HEAD_DIM, max_context_len, partition_tokens,
                                                        num_prefill, num_q_rows, max_query_len))  # fmt: skip


def paged_mixed(
    dec_out: torch.Tensor,
    dec_q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    dec_block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    max_context_len: int,
    pre_out: torch.Tensor,
    pre_q: torch.Tensor,
    pre_block_tables: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    q_start: torch.Tensor,
    max_query_len: int,
    pool: torch.Tensor,
    layer: int,
    scale: float | None = None,
    partition_tokens: int = 0,
    workspace: torch.Tensor | None = None,
    d_error: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
) -> None:
    """One launch for a step's decode rows (``paged_decode`` with ``k_new`` / ``v_new``: their new K/V
    written, then one query each over its context) and its prefill rows (``paged_prefill``; their
    K/V must already be in the pool). Each output row is bit-identical to the single-kind call's
    (decode rows: at the same explicit ``partition_tokens``)."""
    nb, n_layer, n_head, bs, d = _pool_dims(pool)
    if not 0 <= layer < n_layer:
        raise ValueError(f"layer {layer} out of range [0, {n_layer})")
    nd = context_lens.numel()
    _int_tensor(context_lens, "context_lens", torch.int32, pool.device)
    _tables(dec_block_tables, "dec_block_tables", nd, pool.device)
    for t, name in ((dec_q, "dec_q"), (dec_out, "dec_out"), (k_new, "k_new"), (v_new, "v_new")):
        _rows(t, name, nd, n_head, pool.device)
    _int_tensor(cu_seqlens_q, "cu_seqlens_q", torch.int32, pool.device)
    _int_tensor(q_start, "q_start", torch.int32, pool.device)
    npf = q_start.numel()
    if cu_seqlens_q.numel() != npf + 1:
        raise ValueError("cu_seqlens_q must have num_prefill_seqs + 1 entries")
    _tables(pre_block_tables, "pre_block_tables", npf, pool.device)
    n_rows = pre_q.size(0)
    _rows(pre_q, "pre_q", n_rows, n_head, pool.device)
    _rows(pre_out, "pre_out", n_rows, n_head, pool.device)
    if seq_order is not None:
        _int_tensor(seq_order, "seq_order", torch.int32, pool.device)
        if seq_order.numel() != nd:
            raise ValueError(f"seq_order needs {nd} entries")
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    need = mixed_workspace_bytes(nd, n_head, max_context_len, partition_tokens, npf, n_rows, max_query_len) if nd else 0
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=pool.device)
    if not need:
        workspace = None
    _op("paged_mixed", dec_out, dec_q, k_new, v_new, dec_block_tables, context_lens, int(max_context_len), pre_out,
        pre_q, pre_block_tables, cu_seqlens_q, q_start, int(max_query_len), pool, layer, scale, partition_tokens,
        workspace, d_error, seq_order)  # fmt: skip


def paged_gather(pool: torch.Tensor, layer: int, block_tables: torch.Tensor,
                 d_error: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Every sequence's K and V ``[B, H, nb * block_size, d]`` gathered from ``pool[:, layer]`` in
    table order (``block_tables`` int32 ``[B, nb]``, padded with any valid id): the copy the
    reference's ``PagedBatch.gather`` materialises (tokquay/kv_cache.py:234-242), bit for bit."""
    nb, n_layer, n_head, bs, d = _pool_dims(pool)
    if not 0 <= layer < n_layer:
        raise ValueError(f"layer {layer} out of range [0, {n_layer})")
    B = block_tables.size(0)
    _tables(block_tables, "block_tables", B, pool.device)
    k = torch.empty(B, n_head, block_tables.size(1) * bs, d, dtype=torch.float32, device=pool.device)
    v = torch.empty_like(k)
    _op("paged_gather", k, v, pool, layer, block_tables, d_error)
    return k, v


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy ids ``[R]`` (int64) of float32 logits ``[R, V]``: the reference's ``logits.argmax(-1)``
    (tokquay/engine.py:190) - the lowest index of each row's maximum, NaN above every number."""
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.dim() != 2:
        raise ValueError("logits must be a float32 [rows, vocab] tensor on a HIP device")
    rows, cols = logits.shape
    if cols < 1:
        raise ValueError("logits need at least one column")
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    elif out.dtype != torch.int64 or out.device != logits.device or out.dim() != 1 or out.numel() != rows:
        raise ValueError(f"out must be an int64 [{rows}] tensor on {logits.device}")
    elif rows > 1 and out.stride(0) != 1:
        raise ValueError("out must be contiguous")
    if cols > 1 and logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    _op("argmax_rows", logits, out)
    return out


def add_layernorm(x: torch.Tensor, y: torch.Tensor | None, weight: torch.Tensor, bias: torch.Tensor, eps: float,
                  x_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``(x + y, layer_norm(x + y))`` for float32 rows ``[R, C]`` in one pass (``tq_add_layernorm``): a
    residual add of Block.forward (tokquay/model.py:122-123) and the LayerNorm after it. ``x_out``
    (default: a new tensor) may be ``x`` itself for an in-place residual update. ``y=None``: ``(x,
    layer_norm(x))``."""
    if x.dim() != 2 or (y is not None and y.shape != x.shape) or not x.is_cuda:
        raise ValueError("x and y must be [rows, cols] tensors of one shape on a HIP device")
    rows, cols = x.shape
    for name, t in (("x", x),) + ((("y", y),) if y is not None else ()):
        if t.dtype != torch.float32 or t.device != x.device or t.stride(1) != 1:
            raise ValueError(f"{name} must be float32 with contiguous rows on {x.device}")
    for name, t in (("weight", weight), ("bias", bias)):
        if t.dtype != torch.float32 or t.device != x.device or t.shape != (cols,) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 [{cols}] tensor on {x.device}")
    if x_out is None:
        x_out = torch.empty_like(x, memory_format=torch.contiguous_format)
    elif x_out.shape != x.shape or x_out.dtype != torch.float32 or x_out.stride(1) != 1 or x_out.device != x.device:
        raise ValueError("x_out must be a float32 tensor shaped like x with contiguous rows")
    h = torch.empty(rows, cols, dtype=torch.float32, device=x.device)
    stride = lambda t: t.stride(0) if rows > 1 else cols  # noqa: E731  (a one-row view may carry any stride)
    st = _lib.lib().tq_add_layernorm(x_out.data_ptr(), stride(x_out), h.data_ptr(), cols, x.data_ptr(), stride(x),
                                     y.data_ptr() if y is not None else None, stride(y) if y is not None else cols,
                                     weight.data_ptr(), bias.data_ptr(), rows, cols,
                                     float(eps), _stream(x.device))  # fmt: skip
    _lib.check(st, "tq_add_layernorm")
    return x_out, h


# Decode steps run their linears through tq_skinny_linear up to 64 rows. Measured decode steps
# (graphs + pipelining, contexts ~300-500): 24 / 32 / 48 / 64 sequences 0.95 / 0.98 / 1.13 / 1.18 ms
# on hipBLASLt with separate LayerNorm launches, 0.77 / 0.80 / 1.10 / 1.14 ms with it.
SKINNY_MAX_ROWS = 64
# The tied LM head (154 MB of weights) stays fused with ln_f only while the rows fit one row block:
# beyond 16 rows every row group re-reads the weights, and hipBLASLt plus a separate LayerNorm is
# faster. Decode step p50 at 24 / 32 / 64 sequences 0.73 / 0.74 / 1.08 ms fused, 0.70 / 0.72 / 1.03 ms
# on the library; at 1 / 8 sequences 0.42 / 0.46 fused, 0.44 / 0.47 on the library (graph-timed
# back to back, the library looks faster there too, 29.5 vs 39.9 us at 8 rows, but only because
# repeated calls find the weights in the last-level cache, which a decode step's other 340 MB of
# weights evict).
SKINNY_LM_HEAD_MAX_ROWS = 16
SKINNY_WIDTHS = (768, 3072)
_EPILOGUES = {"none": 0, "gelu": 1, "residual": 2}


_SCRATCH_MIN = 1 << 20
# Per (device, use): zeroed device buffers that the kernels leave zeroed after every call (split-K arrival
# counters and partial tiles). Zeroed once; kept for the life of the process, since captured graphs hold
# their addresses. One per use, so two kernels that may be in flight together never share one.
_scratch: dict[tuple[torch.device, str], list[torch.Tensor]] = {}


def zeroed_scratch(device: torch.device, use: str, nbytes: int) -> torch.Tensor | None:
    """A zero-initialised uint8 buffer of at least ``nbytes`` on ``device`` for ``use`` (None for 0 bytes).
    Grown only outside graph capture: run a shape once before capturing it."""
    if nbytes == 0:
        return None
    bufs = _scratch.setdefault((torch.device(device), use), [])
    if not bufs or bufs[-1].numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"the {use} buffer must exist before graph capture (run the shape once)")
        bufs.append(torch.zeros(max(nbytes, _SCRATCH_MIN), dtype=torch.uint8, device=device))
    return bufs[-1]


def skinny_supported(rows: int, in_features: int) -> bool:
    """Whether decode steps run this shape through ``tq_skinny_linear`` (at most ``SKINNY_MAX_ROWS``
    rows, K = 768 or 3072)."""
    return 0 < rows <= SKINNY_MAX_ROWS and in_features in SKINNY_WIDTHS


def skinny_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                  ln: tuple[torch.Tensor, torch.Tensor, float] | None = None, epilogue: str = "none",
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """``epilogue(LN(x) @ weight.T + bias)`` for at most 64 float32 rows in one launch (``tq_skinny_linear``).

    ``ln = (gamma, beta, eps)`` fuses the LayerNorm in front (tokquay/model.py:117-118); ``epilogue`` is
    ``"none"``, ``"gelu"`` (tanh form, :107) or ``"residual"``: ``out += x @ weight.T + bias`` in place (the
    residual add, :122-123; ``out`` required). ``weight`` is nn.Linear's ``[N, K]``."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda or x.stride(1) != 1:
        raise ValueError("x must be a float32 [rows, K] tensor with contiguous rows on a HIP device")
    M, K = x.shape
    if weight.dtype != torch.float32 or weight.device != x.device or weight.dim() != 2 or weight.size(1) != K \
            or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous float32 [N, {K}] tensor on {x.device}")
    N = weight.size(0)
    if bias is not None and (bias.dtype != torch.float32 or bias.device != x.device or bias.shape != (N,)
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous float32 [{N}] tensor on {x.device}")
    if epilogue not in _EPILOGUES:
        raise ValueError(f"epilogue must be one of {sorted(_EPILOGUES)}")
    gamma = beta = None
    eps = 0.0
    if ln is not None:
        gamma, beta, eps = ln
        for name, t in (("ln weight", gamma), ("ln bias", beta)):
            if t.dtype != torch.float32 or t.device != x.device or t.shape != (K,) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 [{K}] tensor on {x.device}")
    if out is None:
        if epilogue == "residual":
            raise ValueError("the residual epilogue adds into out: pass it")
        out = torch.empty(M, N, dtype=torch.float32, device=x.device)
    elif out.shape != (M, N) or out.dtype != torch.float32 or out.device != x.device or (M > 1 and out.stride(1) != 1):
        raise ValueError(f"out must be a float32 [{M}, {N}] tensor with contiguous rows on {x.device}")
    row = lambda t, w: t.stride(0) if M > 1 else w  # noqa: E731  (a one-row view may carry any stride)
    L = _lib.lib()
    # One buffer per (N, K): the split layout (counters, then tiles) depends on the shape.
    ws = zeroed_scratch(x.device, f"skinny linear {N}x{K}",
                        int(L.tq_skinny_linear_workspace_size(M, N, K, int(ln is not None))))  # fmt: skip
    st = L.tq_skinny_linear(
        out.data_ptr(), row(out, N), x.data_ptr(), row(x, K), M, weight.data_ptr(),
        bias.data_ptr() if bias is not None else None, N, K,
        gamma.data_ptr() if gamma is not None else None, beta.data_ptr() if beta is not None else None,
        float(eps), _EPILOGUES[epilogue], ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream(x.device),
    )  # fmt: skip
    _lib.check(st, "tq_skinny_linear")
    return out


def skinny_linear_argmax(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                         ln: tuple[torch.Tensor, torch.Tensor, float] | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy ids ``[M]`` (int64) of ``LN(x) @ weight.T + bias`` for at most 16 float32 rows of width
    768, with no logits written (``tq_skinny_linear_argmax``): the tied LM head with ``ln_f`` in
    front (tokquay/model.py:180-181) and the batched argmax of Engine._sample (tokquay/engine.py:190)
    in one launch. Ties keep the lowest column; NaN ranks above every number."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda or x.stride(1) != 1:
        raise ValueError("x must be a float32 [rows, K] tensor with contiguous rows on a HIP device")
    M, K = x.shape
    if not 0 < M <= SKINNY_LM_HEAD_MAX_ROWS or K != SKINNY_WIDTHS[0]:
        raise ValueError(f"x must have 1..{SKINNY_LM_HEAD_MAX_ROWS} rows of width {SKINNY_WIDTHS[0]}")
    if weight.dtype != torch.float32 or weight.device != x.device or weight.dim() != 2 or weight.size(1) != K \
            or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous float32 [N, {K}] tensor on {x.device}")
    N = weight.size(0)
    if bias is not None and (bias.dtype != torch.float32 or bias.device != x.device or bias.shape != (N,)
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous float32 [{N}] tensor on {x.device}")
    gamma = beta = None
    eps = 0.0
    if ln is not None:
        gamma, beta, eps = ln
        for name, t in (("ln weight", gamma), ("ln bias", beta)):
            if t.dtype != torch.float32 or t.device != x.device or t.shape != (K,) or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 [{K}] tensor on {x.device}")
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or out.device != x.device or out.shape != (M,) or (M > 1 and out.stride(0) != 1):
        raise ValueError(f"out must be an int64 [{M}] tensor on {x.device}")
    L = _lib.lib()
    # Slice candidates [M][N / 32] (written before they are read: any contents will do).
    ws = zeroed_scratch(x.device, "skinny argmax", int(L.tq_skinny_linear_argmax_workspace_size(N)))
    st = L.tq_skinny_linear_argmax(
        out.data_ptr(), x.data_ptr(), x.stride(0) if M > 1 else K, M, weight.data_ptr(),
        bias.data_ptr() if bias is not None else None, N, K,
        gamma.data_ptr() if gamma is not None else None, beta.data_ptr() if beta is not None else None,
        float(eps), ws.data_ptr(), ws.numel(), _stream(x.device),
    )  # fmt: skip
    _lib.check(st, "tq_skinny_linear_argmax")
    return out


def embed_rows(ids: torch.Tensor, positions: torch.Tensor, wte: torch.Tensor, wpe: torch.Tensor,
               src: torch.Tensor | None = None, tokens: torch.Tensor | None = None,
               error_word: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``wte[id] + wpe[pos]`` per row (tokquay/model.py:172), ``id = tokens[src[r]]`` where ``src[r] >= 0``
    (a token a previous replay left on the device), else ``ids[r]`` (``tq_embed_rows``)."""
    rows = ids.numel()
    dev = wte.device
    V, C = wte.shape
    for name, t in (("ids", ids), ("positions", positions)) + ((("src", src), ("tokens", tokens)) if src is not None else ()):
        if t is None or t.dtype != torch.int64 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int64 tensor on {dev}")
    if positions.numel() != rows or (src is not None and src.numel() != rows):
        raise ValueError("ids, positions and src need one entry per row")
    if out is None:
        out = torch.empty(rows, C, dtype=torch.float32, device=dev)
    elif out.shape != (rows, C) or out.dtype != torch.float32 or out.device != dev or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 [{rows}, {C}] tensor on {dev}")
    st = _lib.lib().tq_embed_rows(
        out.data_ptr(), C, ids.data_ptr(), src.data_ptr() if src is not None else None,
        tokens.data_ptr() if tokens is not None else None, positions.data_ptr(), wte.data_ptr(), wpe.data_ptr(),
        rows, C, V, wpe.size(0), error_word.data_ptr() if error_word is not None else None, _stream(dev),
    )  # fmt: skip
    _lib.check(st, "tq_embed_rows")
    return out



# ------------------------------------------------------------------------------ library GEMMs
# hipBLASLt's default fp32 kernel for a given shape depends on the operand layout. Measured on the
# device (a spin kernel holding the stream while ten calls per layout queue behind it, best of three
# alternating trials), the transposed-weight ("NN") call is clearly faster only at 256 rows for the
# two 768-wide-input projections: c_attn ([768] -> [2304]) 15.8 -> 12.8 us and c_fc (+ GELU,
# [768] -> [3072]) 16.7 -> 13.7 us. At 224 or 320 rows, and for the [3072] -> [768] projection at
# any row count, the weight as stored ("TN") is as fast or faster. The choice is this fixed table,
# not a measurement at run time, so that every process computes every shape the same way (the two
# layouts may round differently) and no live step pays for a probe.
GEMM_NN_SHAPES: frozenset[tuple[int, int, int, bool]] = frozenset({
    (256, 2304, 768, False),  # c_attn at the 256-row decode bucket
    (256, 3072, 768, True),  # c_fc + GELU at the 256-row decode bucket
})  # fmt: skip


def _gemm(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, gelu: bool) -> torch.Tensor:
    if gelu:
        return torch._addmm_activation(bias, x, w, use_gelu=True)
    return torch.addmm(bias, x, w) if bias is not None else x @ w


def transposed_weight(linear: torch.nn.Linear) -> torch.Tensor:
    """A contiguous ``[in, out]`` copy of ``linear.weight``, kept on the module and rebuilt when the
    weight's storage or version changes."""
    w = linear.weight
    key = (w.data_ptr(), w._version, w.device)
    cached = getattr(linear, "_tq_weight_t", None)
    if cached is None or cached[0] != key:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the transposed weight must exist before graph capture (run the shape once)")
        cached = (key, w.detach().t().contiguous())
        linear._tq_weight_t = cached
    return cached[1]


def uses_nn_layout(rows: int, out_features: int, in_features: int, gelu: bool) -> bool:
    """Whether ``linear`` runs this shape with the transposed weight copy (``GEMM_NN_SHAPES``)."""
    return (rows, out_features, in_features, gelu) in GEMM_NN_SHAPES


def linear(x: torch.Tensor, layer: torch.nn.Linear, gelu: bool = False) -> torch.Tensor:
    """``x @ layer.weight.T + layer.bias`` (then the tanh GELU when ``gelu``) through hipBLASLt, in
    the weight layout ``GEMM_NN_SHAPES`` names for this shape. On the CPU: torch's ``F.linear`` and
    the tanh GELU."""
    if not x.is_cuda:
        y = torch.nn.functional.linear(x, layer.weight, layer.bias)
        return torch.nn.functional.gelu(y, approximate="tanh") if gelu else y
    out_f, in_f = layer.weight.shape
    nn_layout = uses_nn_layout(x.shape[0], out_f, in_f, gelu)
    w = transposed_weight(layer) if nn_layout else layer.weight.t()
    return _gemm(x, w, layer.bias, gelu)
