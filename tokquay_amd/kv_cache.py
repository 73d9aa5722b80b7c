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

    # Optional callable(batch, kind) run right before every decode ("decode"), prefill
    # ("prefill") and mixed ("mixed") attention launch; a benchmark uses it to arm
    # launch-recorded timing events.
    launch_hook = None
    # A step holding both decode and prefill rows runs their attention as one launch
    # (tq_paged_mixed); False keeps two launches, decode then prefill (for comparison).
    one_launch_mixed = True

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
        # Validation (the reference's conditions and messages, tokquay/kv_cache.py:182-191) and the packed
        # metadata below are built by the native extension straight from the Python lists.
        nat = _lib.native()
        tables, start, new_lens = block_tables, start, new_lens
        try:
            plan = nat.plan(tables, start, new_lens, block_size)
        except TypeError:  # the builder reads lists of ints; convert other sequences once
            tables, start, new_lens = [list(t) for t in block_tables], list(start), list(new_lens)
            plan = nat.plan(tables, start, new_lens, block_size)
        bs = block_size
        B, T, N = len(tables), plan["T"], plan["N"]
        Bd, Bp, nbd, nbp = plan["Bd"], plan["Bp"], plan["nbd"], plan["nbp"]
        self.pool, self.block_size, self.B, self.T = pool, bs, B, T
        self.num_blocks_gathered = plan["max_blocks"]
        self.max_ctx = plan["max_ctx"]
        self.start, self.new_lens = list(start), list(new_lens)
        # A copy of the tables as they are now (their first max_blocks entries), for the reference
        # view's gather: a caller may grow, free or reuse its lists before gather() is called.
        nb = plan["max_blocks"]
        self._tables = [t[:nb] for t in tables]
        self.error_word = error_word
        self.partition_tokens = partition_tokens
        device = pool.device
        self.device = device
        self.num_decode, self.num_prefill, self.num_tokens = Bd, Bp, N
        self.decode_max_ctx = plan["decode_max_ctx"]
        self.prefill_max_q = plan["prefill_max_q"]
        self._nbd, self._nbp = nbd, nbp

        pin = device.type == "cuda"
        # int64: token_index[N] | positions[N] | slot_mapping[N] | last_rows[B]
        # int32: dec_tables[Bd, nbd] | dec_ctx[Bd] | pre_tables[Bp, nbp] | pre_cu[Bp + 1] | pre_start[Bp]
        #        | dec_order[Bd] (decode rows, longest context first: the decode kernel's dispatch order)
        #        | pre_order[Bp] (multi-token sequences, most causal work first: the prefill kernel's)
        h64 = torch.empty(plan["n64"], dtype=torch.int64, pin_memory=pin)
        h32 = torch.empty(plan["n32"], dtype=torch.int32, pin_memory=pin)
        nat.fill(tables, start, new_lens, bs, h64.data_ptr(), h64.numel(), h32.data_ptr(), h32.numel())
        self._d64 = h64.to(device, non_blocking=True)
        self._d32 = h32.to(device, non_blocking=True)
        # Element offsets of the int32 sections; the views below are made on first use.
        self._o32 = (0, Bd * nbd, Bd * nbd + Bd, Bd * nbd + Bd + Bp * nbp, Bd * nbd + Bd + Bp * nbp + Bp + 1,
                     Bd * nbd + Bd + Bp * nbp + 2 * Bp + 1, Bd * nbd + 2 * Bd + Bp * nbp + 2 * Bp + 1)  # fmt: skip
        self._workspace: torch.Tensor | None = None
        self._ws_bytes = 0
        self._ws_mixed = False  # the workspace was sized for the one-launch mixed grid
        self._lazy: dict[str, torch.Tensor] = {}

    # ---- device metadata views (sections of the two packed buffers) ----
    def _view(self, name: str, buf: torch.Tensor, lo: int, hi: int, rows: int = -1) -> torch.Tensor:
        t = self._lazy.get(name)
        if t is None:
            t = buf[lo:hi] if rows < 0 else buf[lo:hi].view(rows, -1 if rows else 0)
            self._lazy[name] = t
        return t

    def _ptr32(self, i: int) -> int:
        """Device address of int32 section ``i`` (dec_tables, dec_ctx, pre_tables, pre_cu, pre_start, dec_order,
        pre_order)."""
        return self._d32.data_ptr() + 4 * self._o32[i]

    @property
    def token_index(self) -> torch.Tensor:
        """``[N]`` flat index ``b * T + t`` of each packed row's token."""
        return self._view("token_index", self._d64, 0, self.num_tokens)

    @property
    def packed_positions(self) -> torch.Tensor:
        return self._view("packed_positions", self._d64, self.num_tokens, 2 * self.num_tokens)

    @property
    def slot_mapping(self) -> torch.Tensor:
        """``[N]`` pool slot (``block * block_size + offset``) of each packed row."""
        return self._view("slot_mapping", self._d64, 2 * self.num_tokens, 3 * self.num_tokens)

    @property
    def last_rows(self) -> torch.Tensor:
        return self._view("last_rows", self._d64, 3 * self.num_tokens, 3 * self.num_tokens + self.B)

    @property
    def decode_block_tables(self) -> torch.Tensor:
        return self._view("decode_block_tables", self._d32, self._o32[0], self._o32[1], self.num_decode)

    @property
    def decode_context_lens(self) -> torch.Tensor:
        return self._view("decode_context_lens", self._d32, self._o32[1], self._o32[2])

    @property
    def prefill_block_tables(self) -> torch.Tensor:
        return self._view("prefill_block_tables", self._d32, self._o32[2], self._o32[3], self.num_prefill)

    @property
    def prefill_cu_seqlens(self) -> torch.Tensor:
        return self._view("prefill_cu_seqlens", self._d32, self._o32[3], self._o32[4])

    @property
    def prefill_start(self) -> torch.Tensor:
        return self._view("prefill_start", self._d32, self._o32[4], self._o32[5])

    @property
    def decode_order(self) -> torch.Tensor:
        return self._view("decode_order", self._d32, self._o32[5], self._o32[5] + self.num_decode)

    @property
    def prefill_order(self) -> torch.Tensor:
        return self._view("prefill_order", self._d32, self._o32[6], self._o32[6] + self.num_prefill)

    # ---- reference contract members (built on demand; the HIP path does not need them) ----
    @property
    def context_lens(self) -> list[int]:
        """Keys visible to each sequence after this step: ``start + new_len`` (tokquay/kv_cache.py:188)."""
        return [s + n for s, n in zip(self.start, self.new_lens)]

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
        """Each sequence's K and V as contiguous ``[B, H, nb * block_size, d]`` (tokquay/kv_cache.py:
        234-242): tables padded to ``nb`` entries with block 0, copied by the HIP gather kernel bit
        for bit. The attention path never needs this copy (``attend`` reads the pool in place); it
        serves callers of the reference's ``BatchedKV`` contract."""
        from tokquay_amd import ops

        if "gather_tables" not in self._lazy:
            nb = self.num_blocks_gathered
            padded = [list(t) + [0] * (nb - len(t)) for t in self._tables]
            self._lazy["gather_tables"] = torch.tensor(padded, dtype=torch.int32).to(self.device)
        return ops.paged_gather(self.pool, layer, self._lazy["gather_tables"], self.error_word)

    # ---- the HIP path ----------------------------------------------------------------
    def attend(self, layer: int, qkv: torch.Tensor) -> torch.Tensor:
        """Write this step's K/V into ``pool[:, layer]`` and return attention output ``[N, H*d]``.

        ``qkv`` is the fused projection output ``[N, 3*C]`` over packed rows, laid
        out ``[q | k | v]`` with heads contiguous inside each (tokquay/model.py:69-71).
        Launches, all on the current stream: decode attention for the one-token rows
        with their cache write folded in (``tq_paged_decode_write``), then - for the
        rows of sequences feeding several tokens - their cache write and prefill
        attention. When both kinds of row are present the two attention launches are
        one (``tq_paged_mixed``, after the prefill rows' cache write) unless
        ``one_launch_mixed`` is off. One call into the native extension makes all of
        them; with a ``launch_hook`` set they go one by one through ctypes, the hook
        before each attention kernel.
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
        Bd, Bp = self.num_decode, self.num_prefill
        mixed = bool(Bd and Bp and PagedBatch.one_launch_mixed)
        if Bd and (self._workspace is None or self._ws_mixed != mixed):
            if mixed:
                self._ws_bytes = int(L.tq_paged_mixed_workspace_size(Bd, n_head, d, self.decode_max_ctx, self.partition_tokens,
                                                                     Bp, N - Bd, self.prefill_max_q))  # fmt: skip
            else:
                self._ws_bytes = int(L.tq_paged_decode_workspace_size(Bd, n_head, d, self.decode_max_ctx, self.partition_tokens))
            self._workspace = torch.empty(max(self._ws_bytes, 1), dtype=torch.uint8, device=pool.device)
            self._ws_mixed = mixed
        ws = self._workspace.data_ptr() if Bd else 0
        slots = self._d64.data_ptr() + 8 * 2 * N

        if PagedBatch.launch_hook is None:  # one native call launches the whole layer
            failed = _lib.native().attend(
                op, qp, pp, nb, n_layer, n_head, bs, d, layer, scale, stream, err or 0, N,
                Bd, self._ptr32(0), self._nbd, self._ptr32(1), self._ptr32(5), self.decode_max_ctx,
                self.partition_tokens, ws, self._ws_bytes,
                Bp, slots, self._ptr32(2), self._nbp, self._ptr32(3), self._ptr32(4), self._ptr32(6), self.prefill_max_q,
                int(mixed),
            )  # fmt: skip
            if failed is not None:
                _lib.check(*failed)
            return out

        # Per-kernel launches, with the hook armed before each attention kernel.
        off = Bd * row3 * 4  # bytes to the first prefill row of qkv
        if Bp:
            _lib.check(
                L.tq_cache_write(pp, nb, n_layer, n_head, bs, d, layer, qp + off + 4 * C, row3, qp + off + 8 * C,
                                 row3, slots + 8 * Bd, N - Bd, err, stream),
                "tq_cache_write",
            )  # fmt: skip
        if mixed:
            PagedBatch.launch_hook(self, "mixed")
            _lib.check(
                L.tq_paged_mixed(op, C, qp, row3, qp + 4 * C, row3, qp + 8 * C, row3, self._ptr32(0), self._nbd,
                                 self._nbd, self._ptr32(1), self._ptr32(5), Bd, self.decode_max_ctx,
                                 self.partition_tokens, op + 4 * Bd * C, C, qp + off, row3, self._ptr32(2), self._nbp,
                                 self._nbp, self._ptr32(3), self._ptr32(4), Bp, N - Bd, self.prefill_max_q, pp, nb,
                                 n_layer, n_head, bs, d, layer, scale, ws, self._ws_bytes, err, stream),
                "tq_paged_mixed",
            )  # fmt: skip
            return out
        if Bd:
            PagedBatch.launch_hook(self, "decode")
            _lib.check(
                L.tq_paged_decode_write(op, C, qp, row3, qp + 4 * C, row3, qp + 8 * C, row3, pp, nb, n_layer,
                                        n_head, bs, d, layer, self._ptr32(0), self._nbd, self._nbd, self._ptr32(1),
                                        self._ptr32(5), Bd, self.decode_max_ctx, scale, self.partition_tokens, ws,
                                        self._ws_bytes, err, stream),
                "tq_paged_decode_write",
            )  # fmt: skip
        if Bp:
            PagedBatch.launch_hook(self, "prefill")
            _lib.check(
                L.tq_paged_prefill(op + 4 * Bd * C, C, qp + off, row3, pp, nb, n_layer, n_head, bs, d, layer,
                                   self._ptr32(2), self._nbp, self._nbp, self._ptr32(3), self._ptr32(4),
                                   self._ptr32(6), Bp, N - Bd, self.prefill_max_q, scale, err, stream),
                "tq_paged_prefill",
            )  # fmt: skip
        return out
