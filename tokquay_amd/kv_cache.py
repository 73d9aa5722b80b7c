"""Paged KV cache: the block pool, its allocator and the per-step batch view.

The pool layout, the allocator and the batch-view contract are the
reference's (tokquay/kv_cache.py:1-157)::

    pool: [num_blocks, n_layer, 2, n_head, block_size, d_head]      (dim 2: 0=K, 1=V)

Position ``p`` of a sequence lives in block ``block_table[p // block_size]`` at
offset ``p % block_size``. ``BlockAllocator`` hands blocks out LIFO (block 0
first), ref-counts them, and raises ``OutOfBlocksError`` with its state
unchanged when the free list is too short.

What differs is ``PagedBatch``, the per-step view the model consumes. Instead of
building scatter/gather index tensors and materialising every sequence's
blocks, it builds - once per step, reused by every layer - the device metadata
the gfx950 kernels read (slot mapping, int32 block tables, context lengths,
query offsets) and exposes ``attend(layer, qkv)``: cache write + paged
attention straight off the pool, in place.
"""

from __future__ import annotations

import math
from typing import TYPE_CHECKING

import numpy as np
import torch

from tokquay_amd import _lib
from tokquay_amd.sequence import Sequence

if TYPE_CHECKING:
    from tokquay_amd.model import GPT2Config

HEAD_DIM = 64


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


class OutOfBlocksError(RuntimeError):
    """Raised (without changing any state) when the free list is too short."""


class BlockAllocator:
    """Owns the pool, the LIFO free list and the ref counts (tokquay/kv_cache.py:38-127)."""

    def __init__(
        self,
        cfg: "GPT2Config",
        num_blocks: int,
        block_size: int = 16,
        device=None,
        dtype: torch.dtype = torch.float32,
    ):
        if num_blocks < 1 or block_size < 1:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.pool = torch.zeros(
            num_blocks, cfg.n_layer, 2, cfg.n_head, block_size, cfg.d_head, device=device, dtype=dtype
        )
        self._free: list[int] = list(range(num_blocks - 1, -1, -1))  # reversed: block 0 is handed out first
        self.ref_counts: list[int] = [0] * num_blocks
        # Device word the kernels OR error bits into (out-of-range block ids / slots / lengths).
        self.error_word = torch.zeros(1, dtype=torch.int32, device=self.pool.device) if self.pool.is_cuda else None
        self.decode_partition_tokens = 0  # 0: the kernel chooses

    # ---- bookkeeping ---------------------------------------------------------------
    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - len(self._free)

    @property
    def bytes_per_block(self) -> int:
        return self.pool[0].numel() * self.pool.element_size()

    def blocks_needed(self, num_tokens: int) -> int:
        return cdiv(num_tokens, self.block_size)

    # ---- allocation ----------------------------------------------------------------
    def can_allocate(self, num_tokens: int) -> bool:
        return self.blocks_needed(num_tokens) <= self.num_free_blocks

    def allocate(self, seq: Sequence, num_tokens: int | None = None) -> None:
        """Give a block-less sequence blocks for ``num_tokens`` positions (default: all its tokens)."""
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already owns blocks")
        n = self.blocks_needed(seq.num_tokens if num_tokens is None else num_tokens)
        seq.block_table = self._take(n)

    def can_append_slot(self, seq: Sequence) -> bool:
        return self.blocks_needed(seq.num_tokens) - len(seq.block_table) <= self.num_free_blocks

    def append_slot(self, seq: Sequence, num_tokens: int | None = None) -> bool:
        """Grow the table to cover ``num_tokens`` positions (default ``seq.num_tokens``); True if a
        block was taken."""
        missing = self.blocks_needed(seq.num_tokens if num_tokens is None else num_tokens) - len(seq.block_table)
        if missing <= 0:
            return False
        seq.block_table.extend(self._take(missing))
        return True

    def free(self, seq: Sequence) -> None:
        """Release the sequence's blocks (a block-less sequence is a no-op; a double free raises)."""
        for b in seq.block_table:
            if self.ref_counts[b] <= 0:
                raise RuntimeError(f"double free of block {b}")
            self.ref_counts[b] -= 1
            if self.ref_counts[b] == 0:
                self._free.append(b)
        seq.block_table = []

    def _take(self, n: int) -> list[int]:
        if n > len(self._free):
            raise OutOfBlocksError(f"need {n} blocks, only {len(self._free)} free")
        blocks = [self._free.pop() for _ in range(n)]
        for b in blocks:
            self.ref_counts[b] = 1
        return blocks

    # ---- model-facing --------------------------------------------------------------
    def batch_for(self, seqs: list[Sequence], new_lens: list[int] | None = None) -> "PagedBatch":
        """Step view for ``seqs``: each feeds ``new_lens[i]`` tokens (default: all uncached ones)
        starting at position ``num_cached_tokens``."""
        starts = [s.num_cached_tokens for s in seqs]
        new_lens = new_lens or [s.num_uncached_tokens for s in seqs]
        return PagedBatch(
            self.pool, self.block_size, [s.block_table for s in seqs], starts, new_lens,
            error_word=self.error_word, partition_tokens=self.decode_partition_tokens,
        )  # fmt: skip

    def check_device_errors(self) -> None:
        """Synchronise and raise if a kernel met an out-of-range id or length since the last check."""
        if self.error_word is None:
            return
        bits = int(self.error_word.item())
        if bits:
            self.error_word.zero_()
            raise RuntimeError(f"paged-attention kernels reported invalid metadata (error bits {bits:#x})")


class BatchedKV:
    """What the model needs from a per-step batch view (tokquay/kv_cache.py:130-157).

    * ``B``, ``T``: batch size and padded number of new tokens per row.
    * ``max_ctx``: longest row after this step.
    * ``positions`` ``[B, T]``, ``last_idx`` ``[B]``, ``mask`` ``[B, 1, T, S]``.
    * ``write(layer, k, v)``: store new K/V ``[B, H, T, d]``; padded slots must not write.
    * ``gather(layer)``: every row's K and V as ``[B, H, S, d]``.
    """

    B: int
    T: int
    max_ctx: int
    positions: torch.Tensor
    last_idx: torch.Tensor
    mask: torch.Tensor

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        raise NotImplementedError

    def gather(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        raise NotImplementedError


class PagedBatch(BatchedKV):
    """One step's view of the paged pool, driving the gfx950 kernels.

    Sequence ``b`` feeds ``new_lens[b]`` tokens at positions ``start[b] ..
    start[b] + new_lens[b] - 1``; everything before is already in the pool.
    Validation and error messages follow the reference (tokquay/kv_cache.py:182-191).

    The model runs on *packed* rows: only real tokens, no right padding. Rows of
    one-token sequences (decode) come first, in batch order, so the decode
    kernel reads q row ``i`` for the i-th of them; the tokens of multi-token
    sequences (prefill, recompute, chunked prefill) follow, contiguous per
    sequence, for the prefill kernel. ``token_index`` maps packed rows to the
    flat ``[B * T]`` padded input, ``last_rows`` gives each sequence's last row.
    """

    # Optional callable(batch, kind) run right before every decode ("decode") and prefill
    # ("prefill") attention launch; a benchmark uses it to arm launch-recorded timing events.
    launch_hook = None

    def __init__(
        self,
        pool: torch.Tensor,
        block_size: int,
        block_tables: list[list[int]],
        start: list[int],
        new_lens: list[int],
        *,
        error_word: torch.Tensor | None = None,
        partition_tokens: int = 0,
    ):
        if not block_tables or not (len(block_tables) == len(start) == len(new_lens)):
            raise ValueError("block_tables, start and new_lens must be non-empty and the same length")
        if min(new_lens) < 1:
            raise ValueError("every sequence must feed at least one token")
        if min(start) < 0:
            raise ValueError("start positions must be non-negative")
        bs = block_size
        ctx = [s + n for s, n in zip(start, new_lens)]  # keys visible after this step (tokquay/kv_cache.py:188)
        for b, (tbl, c) in enumerate(zip(block_tables, ctx)):
            if len(tbl) < cdiv(c, bs):
                raise ValueError(f"sequence {b}: {len(tbl)} blocks cannot hold {c} tokens")

        B, T = len(block_tables), max(new_lens)
        self.pool, self.block_size, self.B, self.T = pool, bs, B, T
        self.num_blocks_gathered = max(cdiv(c, bs) for c in ctx)
        self.max_ctx = max(ctx)
        self.start, self.new_lens, self.context_lens = list(start), list(new_lens), ctx
        self.error_word = error_word
        self.partition_tokens = partition_tokens
        device = pool.device
        self.device = device

        dec = [b for b, n in enumerate(new_lens) if n == 1]
        pre = [b for b, n in enumerate(new_lens) if n > 1]
        Bd, Bp = len(dec), len(pre)
        N = sum(new_lens)
        self.num_decode, self.num_prefill, self.num_tokens = Bd, Bp, N
        nbd = max((cdiv(ctx[b], bs) for b in dec), default=0)
        nbp = max((cdiv(ctx[b], bs) for b in pre), default=0)
        self.decode_max_ctx = max((ctx[b] for b in dec), default=0)
        self.prefill_max_q = max((new_lens[b] for b in pre), default=0)
        self._nbd, self._nbp = nbd, nbp

        pin = device.type == "cuda"
        # int64 metadata: token_index[N] | positions[N] | slot_mapping[N] | last_rows[B]
        h64 = torch.empty(3 * N + B, dtype=torch.int64, pin_memory=pin)
        a64 = h64.numpy()
        tok_idx, pos, slots, last = a64[:N], a64[N : 2 * N], a64[2 * N : 3 * N], a64[3 * N :]
        # int32 metadata: dec_tables[Bd, nbd] | dec_ctx[Bd] | pre_tables[Bp, nbp] | pre_cu[Bp + 1] | pre_start[Bp]
        # | dec_order[Bd] (decode rows, longest context first: the decode kernel's dispatch order)
        n32 = Bd * nbd + Bd + Bp * nbp + (Bp + 1) + Bp + Bd
        h32 = torch.zeros(n32, dtype=torch.int32, pin_memory=pin)
        a32 = h32.numpy()
        o_dt, o_dc = 0, Bd * nbd
        o_pt = o_dc + Bd
        o_pc = o_pt + Bp * nbp
        o_ps = o_pc + Bp + 1
        o_do = o_ps + Bp
        dec_tables = a32[o_dt:o_dc].reshape(Bd, nbd)
        pre_tables = a32[o_pt:o_pc].reshape(Bp, nbp)

        for i, b in enumerate(dec):
            tbl, p = block_tables[b], start[b]
            tok_idx[i] = b * T
            pos[i] = p
            slots[i] = tbl[p // bs] * bs + p % bs
            last[b] = i
            k = cdiv(ctx[b], bs)
            dec_tables[i, :k] = tbl[:k]  # the rest stays block 0 (padding, never read)
            a32[o_dc + i] = ctx[b]
        row = Bd
        for i, b in enumerate(pre):
            n, s = new_lens[b], start[b]
            k = cdiv(ctx[b], bs)
            tbl = np.asarray(block_tables[b][:k], dtype=np.int64)
            ps = np.arange(s, s + n, dtype=np.int64)
            tok_idx[row : row + n] = b * T + np.arange(n)
            pos[row : row + n] = ps
            slots[row : row + n] = tbl[ps // bs] * bs + ps % bs
            last[b] = row + n - 1
            pre_tables[i, :k] = tbl
            a32[o_pc + i] = row - Bd
            a32[o_ps + i] = s
            row += n
        a32[o_pc + Bp] = N - Bd
        a32[o_do:] = np.argsort(-a32[o_dc:o_pt], kind="stable")

        d64 = h64.to(device, non_blocking=True)
        d32 = h32.to(device, non_blocking=True)
        self.token_index = d64[:N]
        self.packed_positions = d64[N : 2 * N]
        self.slot_mapping = d64[2 * N : 3 * N]
        self.last_rows = d64[3 * N :]
        self.decode_block_tables = d32[o_dt:o_dc].view(Bd, nbd)
        self.decode_context_lens = d32[o_dc:o_pt]
        self.prefill_block_tables = d32[o_pt:o_pc].view(Bp, nbp)
        self.prefill_cu_seqlens = d32[o_pc:o_ps]
        self.prefill_start = d32[o_ps:o_do]
        self.decode_order = d32[o_do:]
        self._workspace: torch.Tensor | None = None
        self._ws_bytes = 0
        self._lazy: dict[str, torch.Tensor] = {}

    # ---- reference contract members (built on demand; the HIP path does not need them) ----
    @property
    def positions(self) -> torch.Tensor:
        """``[B, T]`` absolute position of every (padded) new token (tokquay/kv_cache.py:205)."""
        if "positions" not in self._lazy:
            st = torch.tensor(self.start, dtype=torch.long, device=self.device)
            self._lazy["positions"] = st[:, None] + torch.arange(self.T, device=self.device)[None, :]
        return self._lazy["positions"]

    @property
    def last_idx(self) -> torch.Tensor:
        if "last_idx" not in self._lazy:
            self._lazy["last_idx"] = torch.tensor([n - 1 for n in self.new_lens], dtype=torch.long, device=self.device)
        return self._lazy["last_idx"]

    @property
    def mask(self) -> torch.Tensor:
        """``[B, 1, T, nb * block_size]``: key j visible to query (b, t) iff j <= start+t and j < ctx
        (tokquay/kv_cache.py:208-214). The kernels apply the same rule by index arithmetic."""
        if "mask" not in self._lazy:
            ctx_t = torch.tensor(self.context_lens, dtype=torch.long, device=self.device)
            k_pos = torch.arange(self.num_blocks_gathered * self.block_size, device=self.device)[None, None, :]
            self._lazy["mask"] = ((k_pos <= self.positions[:, :, None]) & (k_pos < ctx_t[:, None, None]))[:, None]
        return self._lazy["mask"]

    def padded_slot_mapping(self) -> torch.Tensor:
        """``[B * T]`` slots of the right-padded layout, -1 for padded positions."""
        if "padded_slots" not in self._lazy:
            sm = torch.full((self.B * self.T,), -1, dtype=torch.int64, device=self.device)
            sm[self.token_index] = self.slot_mapping
            self._lazy["padded_slots"] = sm
        return self._lazy["padded_slots"]

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter new K/V given in the reference's ``[B, H, T, d]`` layout (tokquay/kv_cache.py:228-232);
        padded positions write nothing. Runs the HIP cache-write kernel."""
        from tokquay_amd import ops

        rows = [t.transpose(1, 2).reshape(self.B * self.T, t.size(1), t.size(3)) for t in (k, v)]
        ops.cache_write(self.pool, layer, rows[0], rows[1], self.padded_slot_mapping(), self.error_word)

    def gather(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        raise NotImplementedError(
            "the gfx950 batch view never materialises gathered K/V: attend(layer, qkv) reads the pool in place"
        )

    # ---- the HIP path ----------------------------------------------------------------
    def attend(self, layer: int, qkv: torch.Tensor) -> torch.Tensor:
        """Write this step's K/V into ``pool[:, layer]`` and return attention output ``[N, H*d]``.

        ``qkv`` is the fused projection output ``[N, 3*C]`` over packed rows, laid
        out ``[q | k | v]`` with heads contiguous inside each (tokquay/model.py:69-71).
        Launches, all on the current stream: decode attention for the one-token rows
        with their cache write folded in (``tq_paged_decode_write``), then - for the
        rows of sequences feeding several tokens - their cache write and prefill
        attention.
        """
        pool = self.pool
        nb, n_layer, _, n_head, bs, d = pool.shape
        C = n_head * d
        N = self.num_tokens
        if qkv.dtype != torch.float32 or qkv.device != pool.device or tuple(qkv.shape) != (N, 3 * C) or not qkv.is_contiguous():
            raise ValueError(f"qkv must be a contiguous float32 [{N}, {3 * C}] tensor on {pool.device}")
        if not pool.is_cuda or pool.dtype != torch.float32 or d != HEAD_DIM:
            raise ValueError("the HIP path needs a float32 pool with d_head=64 on a HIP device")
        if not 0 <= layer < n_layer:
            raise ValueError(f"layer {layer} out of range [0, {n_layer})")
        L = _lib.lib()
        out = torch.empty(N, C, dtype=torch.float32, device=pool.device)
        stream = torch.cuda.current_stream(pool.device).cuda_stream
        err = self.error_word.data_ptr() if self.error_word is not None else None
        row3 = 3 * C
        qp, pp, op = qkv.data_ptr(), pool.data_ptr(), out.data_ptr()
        scale = 1.0 / math.sqrt(d)

        Bd = self.num_decode
        if Bd:
            if self._workspace is None:
                self._ws_bytes = int(L.tq_paged_decode_workspace_size(Bd, n_head, d, self.decode_max_ctx, self.partition_tokens))
                self._workspace = torch.empty(max(self._ws_bytes, 1), dtype=torch.uint8, device=pool.device)
            if PagedBatch.launch_hook is not None:
                PagedBatch.launch_hook(self, "decode")
            _lib.check(
                L.tq_paged_decode_write(op, C, qp, row3, qp + 4 * C, row3, qp + 8 * C, row3, pp, nb, n_layer,
                                        n_head, bs, d, layer, self.decode_block_tables.data_ptr(), self._nbd,
                                        self._nbd, self.decode_context_lens.data_ptr(), self.decode_order.data_ptr(),
                                        Bd, self.decode_max_ctx,
                                        scale, self.partition_tokens, self._workspace.data_ptr(), self._ws_bytes,
                                        err, stream),
                "tq_paged_decode_write",
            )  # fmt: skip
        if self.num_prefill:
            off = Bd * row3 * 4  # bytes to the first prefill row of qkv
            _lib.check(
                L.tq_cache_write(pp, nb, n_layer, n_head, bs, d, layer, qp + off + 4 * C, row3, qp + off + 8 * C,
                                 row3, self.slot_mapping.data_ptr() + 8 * Bd, N - Bd, err, stream),
                "tq_cache_write",
            )  # fmt: skip
            if PagedBatch.launch_hook is not None:
                PagedBatch.launch_hook(self, "prefill")
            _lib.check(
                L.tq_paged_prefill(op + 4 * Bd * C, C, qp + 4 * Bd * row3, row3, pp, nb, n_layer, n_head, bs, d, layer,
                                   self.prefill_block_tables.data_ptr(), self._nbp, self._nbp,
                                   self.prefill_cu_seqlens.data_ptr(), self.prefill_start.data_ptr(),
                                   self.num_prefill, N - Bd, self.prefill_max_q, scale, err, stream),
                "tq_paged_prefill",
            )  # fmt: skip
        return out
