"""HIP-graph replay of decode steps.

A decode step (every sequence feeds one token) runs ~120-180 small launches
from Python; at 256 sequences that host work is a third of the step. This module
captures the whole decode forward (embeddings, 12 layers with the paged-decode
kernel that also writes the new K/V, LM head, greedy argmax) once per batch
bucket (powers of two) into a HIP graph and replays it. Buckets of at most 64
rows run the fused small-batch path (``GPT2.skinny_logits``: each linear of a
block with its LayerNorm / GELU / residual add in one ``tq_skinny_linear`` launch,
about 65 launches per step; the LM head fused with ``ln_f`` up to 16 rows, else
``ln_f`` alone and the head on hipBLASLt); larger buckets the library GEMMs with
``tq_add_layernorm``. A step whose rows are all greedy at most 16 rows replays an
ids-only graph instead: the LM head with ``ln_f`` and the argmax in one
``tq_skinny_linear_argmax`` launch, no logits written.

What changes between steps lives in static device buffers at fixed addresses,
refreshed by one host-to-device copy per step: token ids, positions,
block tables (``n_positions / block_size`` columns, padded with block 0),
context lengths and source rows. The graph ends with the greedy argmax of every
row (``tq_argmax_rows``) into a static token buffer; a row whose source row is
``r >= 0`` feeds the token the previous replay chose for its row ``r`` instead
of a host-supplied id, so a step can be launched before the host has read the
previous step's tokens. The decode kernel's grid is sized for ``n_positions`` and its
waves skip partitions past each sequence's real context, so one graph serves
every context length. Rows past the live batch are padding: context 0 (the
decode kernel writes nothing to the pool and zeros to the output); their logits
are ignored.

No memset, host synchronisation or allocation happens inside the captured
region except torch's own graph-pool allocations.
"""

from __future__ import annotations

import math

import torch

from tokquay_amd import _lib, ops
from tokquay_amd.kv_cache import HEAD_DIM, BlockAllocator, cdiv
from tokquay_amd.sequence import Sequence


def bucket_for(n: int) -> int:
    return 1 << max(0, (n - 1).bit_length())


class StaticDecodeBatch:
    """Fixed-address decode metadata for up to ``capacity`` sequences."""

    def __init__(self, allocator: BlockAllocator, capacity: int, n_positions: int):
        pool = allocator.pool
        if not pool.is_cuda or pool.dtype != torch.float32 or pool.shape[-1] != HEAD_DIM:
            raise ValueError("graph decode needs a float32 pool with d_head=64 on a HIP device")
        self.allocator, self.pool, self.capacity = allocator, pool, capacity
        self.block_size = allocator.block_size
        self.max_ctx = n_positions
        self.max_blocks = cdiv(n_positions, self.block_size)
        dev = pool.device
        cap, mb = capacity, self.max_blocks
        # One staging buffer and one device buffer (one copy per step): int64 ids | positions |
        # source rows, then int32 tables | context lengths | dispatch order (rows by decreasing context).
        b64, b32 = 8 * 3 * cap, 4 * (cap * mb + 2 * cap)
        self.dbuf = torch.zeros(b64 + b32, dtype=torch.uint8, device=dev)
        self.hbuf = torch.zeros(b64 + b32, dtype=torch.uint8, pin_memory=True)
        self.d64, self.d32 = self.dbuf[:b64].view(torch.int64), self.dbuf[b64:].view(torch.int32)
        self.h64, self.h32 = self.hbuf[:b64].view(torch.int64), self.hbuf[b64:].view(torch.int32)
        self.copied = torch.cuda.Event()
        self.ids, self.positions, self.src = self.d64[:cap], self.d64[cap : 2 * cap], self.d64[2 * cap :]
        self.tokens = torch.zeros(cap, dtype=torch.int64, device=dev)  # greedy ids of the latest replay
        self.tables = self.d32[: cap * mb].view(cap, mb)
        self.context_lens = self.d32[cap * mb : cap * mb + cap]
        self.order = self.d32[cap * mb + cap :]
        n_head = pool.shape[3]
        L = _lib.lib()
        ws = max(int(L.tq_paged_decode_workspace_size(b, n_head, HEAD_DIM, n_positions, 0))
                 for b in self.buckets())  # fmt: skip
        self.workspace = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self.error_word = allocator.error_word

    def buckets(self) -> list[int]:
        out, b = [], 1
        while b <= self.capacity:
            out.append(b)
            b *= 2
        return out

    def fill(self, seqs: list[Sequence], bucket: int, src_rows: list[int] | None = None) -> None:
        """Write this step's metadata for ``seqs`` and pad to ``bucket``.

        Without ``src_rows`` each sequence feeds its one uncached token. With them, each
        sequence feeds the token the previous replay chose for row ``src_rows[i]``, which
        the host has not appended yet (so the sequence has no uncached token)."""
        self.copied.synchronize()  # the previous step's copy has left the staging buffers
        if not isinstance(seqs, list):
            seqs = list(seqs)
        if src_rows is not None and not isinstance(src_rows, list):
            src_rows = list(src_rows)
        # Native: ids, positions, source rows, padded block tables, context lengths and the
        # longest-first dispatch order, with the padding rows (context 0) up to the bucket.
        _lib.native().fill_decode(seqs, bucket, src_rows, self.h64.data_ptr(), self.h64.numel(), self.h32.data_ptr(),
                                  self.h32.numel(), self.capacity, self.max_blocks, self.block_size, self.max_ctx)
        self.dbuf.copy_(self.hbuf, non_blocking=True)
        self.copied.record()

    def view(self, bucket: int) -> "StaticDecodeView":
        return StaticDecodeView(self, bucket)


class StaticDecodeView:
    """``attend(layer, qkv)`` over the first ``rows`` rows of a StaticDecodeBatch (the graph's batch)."""

    def __init__(self, static: StaticDecodeBatch, rows: int):
        self.s, self.rows = static, rows

    def attend(self, layer: int, qkv: torch.Tensor) -> torch.Tensor:
        s, n = self.s, self.rows
        pool = s.pool
        nb, n_layer, _, n_head, bs, d = pool.shape
        C = n_head * d
        L = _lib.lib()
        out = torch.empty(n, C, dtype=torch.float32, device=pool.device)
        stream = torch.cuda.current_stream(pool.device).cuda_stream
        err = s.error_word.data_ptr() if s.error_word is not None else None
        qp, pp = qkv.data_ptr(), pool.data_ptr()
        _lib.check(
            L.tq_paged_decode_write(out.data_ptr(), C, qp, 3 * C, qp + 4 * C, 3 * C, qp + 8 * C, 3 * C, pp, nb,
                                    n_layer, n_head, bs, d, layer, s.tables.data_ptr(), s.max_blocks, s.max_blocks,
                                    s.context_lens.data_ptr(), s.order.data_ptr(), n, s.max_ctx, 1.0 / math.sqrt(d), 0,
                                    s.workspace.data_ptr(), s.workspace.numel(), err, stream),
            "tq_paged_decode_write",
        )  # fmt: skip
        return out


class DecodeGraphs:
    """Captured decode forwards, one per batch bucket, sharing one StaticDecodeBatch."""

    def __init__(self, model, allocator: BlockAllocator, max_batch: int, skinny: bool = True):
        """``skinny``: buckets of at most 64 rows run the fused small-batch linears
        (``GPT2.skinny_logits``) instead of the library GEMMs."""
        self.model = model
        self.skinny = skinny
        self.static = StaticDecodeBatch(allocator, bucket_for(max_batch), model.cfg.n_positions)
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}

    @property
    def capacity(self) -> int:
        return self.static.capacity

    def fused_greedy(self, rows: int) -> bool:
        """Whether a bucket's ids-only graph runs the LM head with the argmax fused in (no logits):
        the small-batch path with the head on ``tq_skinny_linear_argmax``."""
        return self.skinny and self.model.skinny_ok(rows) and rows <= ops.SKINNY_LM_HEAD_MAX_ROWS

    def _forward(self, rows: int, ids_only: bool) -> torch.Tensor | None:
        m, s = self.model, self.static
        view = s.view(rows)
        # Embeddings in one launch, source rows resolved on the device.
        x = ops.embed_rows(s.ids[:rows], s.positions[:rows], m.wte.weight, m.wpe.weight, src=s.src[:rows],
                           tokens=s.tokens, error_word=s.error_word)  # fmt: skip
        if ids_only:
            # Up to 16 rows, greedy only: the head writes ids, never logits.
            m.skinny_greedy(x, view, out=s.tokens[:rows])
            return None
        if self.skinny and m.skinny_ok(rows):
            # Up to 64 rows: five launches per layer, each linear with its LayerNorm / GELU /
            # residual add fused in.
            logits = m.skinny_logits(x, view)
        else:
            logits = m.trunk(None, None, view, embedded=x) @ m.wte.weight.T
        ops.argmax_rows(logits, out=s.tokens[:rows])
        return logits

    def _capture(self, rows: int, ids_only: bool) -> None:
        s = self.static
        tokens = s.tokens.clone()  # the warm-up runs overwrite what this step's source rows read
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up launches (same inputs: the K/V writes are idempotent)
            for _ in range(2):
                self._forward(rows, ids_only)
                s.tokens.copy_(tokens)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = self._forward(rows, ids_only)
        self.graphs[(rows, ids_only)] = (graph, logits)

    @torch.no_grad()
    def launch(self, seqs: list[Sequence], src_rows: list[int] | None = None,
               logits: bool = True) -> tuple[torch.Tensor | None, torch.Tensor]:  # fmt: skip
        """Enqueue one decode step; returns views of its logits ``[n, vocab]`` and greedy ids ``[n]``
        (valid until the next launch) and advances ``num_cached_tokens``. ``src_rows``: see
        ``StaticDecodeBatch.fill``. ``logits=False``: only the ids are needed; buckets of at most 16
        rows then run the LM head with the argmax fused in and return None for the logits."""
        rows = bucket_for(len(seqs))
        if rows > self.static.capacity:
            raise ValueError(f"{len(seqs)} sequences exceed the graph capacity {self.static.capacity}")
        ids_only = not logits and self.fused_greedy(rows)
        self.static.fill(seqs, rows, src_rows)
        if (rows, ids_only) not in self.graphs:
            self._capture(rows, ids_only)
        graph, out = self.graphs[(rows, ids_only)]
        graph.replay()
        for s in seqs:
            s.num_cached_tokens += 1
        n = len(seqs)
        return (out[:n] if out is not None else None), self.static.tokens[:n]

    def forward(self, seqs: list[Sequence]) -> torch.Tensor:
        """Logits ``[len(seqs), vocab]`` of one decode step; advances ``num_cached_tokens``."""
        return self.launch(seqs)[0]


