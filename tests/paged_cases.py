"""Seeded paged-attention scenarios shared by the parity tests.

A scenario is a batch of sequences, each with ``start`` positions already
cached and ``new_len`` tokens fed this step, over a pool full of garbage
(N(0,1) x 50) whose blocks are dealt out from a seeded permutation, so tables
are non-contiguous and out of order and any unmasked or stray access changes
the answer (the hard mode of tests/test_phase3_paged.py:52-59 in the reference).

The oracle side runs the reference's scatter + gather + masked softmax
(``oracle.paged_ref``) on the CPU; the product side runs
``tokquay_amd.PagedBatch.attend`` (cache write + paged decode / prefill
kernels) on the GPU with the same inputs.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle.paged_ref import RefPagedBatch, brute_force_attention, cdiv, ref_paged_attention_step

H, D = 12, 64
C = H * D
RTOL, ATOL = 1e-5, 1e-4  # fp32 attention outputs vs the reference gather path


def garbage_pool(num_blocks: int, n_layer: int, block_size: int, seed: int, scale: float = 50.0,
                 n_head: int = H) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(num_blocks, n_layer, 2, n_head, block_size, D, generator=g) * scale


def deal_tables(num_blocks: int, ctxs: list[int], block_size: int, seed: int) -> list[list[int]]:
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    tables, i = [], 0
    for c in ctxs:
        n = cdiv(c, block_size)
        tables.append(perm[i : i + n])
        i += n
    if i > num_blocks:
        raise ValueError(f"{i} blocks needed, pool has {num_blocks}")
    return tables


class Scenario:
    def __init__(self, starts, new_lens, block_size=16, n_layer=1, layer=0, num_blocks=None, seed=0, n_head=H):
        self.H, self.C = n_head, n_head * D
        self.starts, self.new_lens = list(starts), list(new_lens)
        self.block_size, self.n_layer, self.layer = block_size, n_layer, layer
        self.ctxs = [s + n for s, n in zip(self.starts, self.new_lens)]
        need = sum(cdiv(c, block_size) for c in self.ctxs)
        self.num_blocks = num_blocks or need + 3
        self.pool = garbage_pool(self.num_blocks, n_layer, block_size, seed, n_head=n_head)
        self.tables = deal_tables(self.num_blocks, self.ctxs, block_size, seed + 1)
        g = torch.Generator().manual_seed(seed + 2)
        # History: K/V of the positions already cached, written straight into their slots.
        blk, off = [], []
        for tbl, s in zip(self.tables, self.starts):
            for p in range(s):
                blk.append(tbl[p // block_size])
                off.append(p % block_size)
        if blk:
            blk_t, off_t = torch.tensor(blk), torch.tensor(off)
            self.pool[blk_t, layer, 0, :, off_t] = torch.randn(len(blk), n_head, D, generator=g)
            self.pool[blk_t, layer, 1, :, off_t] = torch.randn(len(blk), n_head, D, generator=g)
        B, T = len(self.starts), max(self.new_lens)
        # New tokens, [B, H, T, d]; padded columns hold huge values so a stray write or read shows.
        self.q, self.k, self.v = (torch.randn(B, n_head, T, D, generator=g) for _ in range(3))
        for b, n in enumerate(self.new_lens):
            for t in (self.q, self.k, self.v):
                t[b, :, n:] = 1e4

    # ---- oracle -----------------------------------------------------------------------
    def reference(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(pool after the scatter, attention output ``[B, H, T, d]``) from the reference path on CPU fp32."""
        pool = self.pool.clone()
        batch = RefPagedBatch(pool, self.block_size, self.tables, self.starts, self.new_lens)
        out = ref_paged_attention_step(batch, self.layer, self.q, self.k, self.v)
        return pool, out

    def brute_force(self, pool_after: torch.Tensor) -> list[np.ndarray]:
        """Per sequence, float64 textbook attention ``[n_b, H, d]`` over the sequence's own positions."""
        res = []
        bs = self.block_size
        for b, (tbl, n) in enumerate(zip(self.tables, self.new_lens)):
            ctx = self.ctxs[b]
            blocks = torch.tensor([tbl[p // bs] for p in range(ctx)])
            offs = torch.tensor([p % bs for p in range(ctx)])
            keys = pool_after[blocks, self.layer, 0, :, offs].double().numpy()  # [ctx, H, d]
            vals = pool_after[blocks, self.layer, 1, :, offs].double().numpy()
            out = np.stack(
                [brute_force_attention(self.q[b, h, :n].double().numpy(), keys[:, h], vals[:, h], 1 / math.sqrt(D))
                 for h in range(self.H)],
                axis=1,
            )  # fmt: skip
            res.append(out)
        return res

    # ---- product ----------------------------------------------------------------------
    def packed_qkv(self, token_index: torch.Tensor) -> torch.Tensor:
        B, _, T, _ = self.q.shape
        qkv = torch.cat([t.transpose(1, 2).reshape(B, T, self.C) for t in (self.q, self.k, self.v)], dim=-1)
        return qkv.reshape(B * T, 3 * self.C).index_select(0, token_index.cpu())

    def run_product(self, partition_tokens: int = 0):
        """(pool after attend, packed output ``[N, C]``, the PagedBatch) from the HIP path."""
        from tokquay_amd.kv_cache import PagedBatch

        pool = self.pool.cuda()
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        batch = PagedBatch(pool, self.block_size, self.tables, self.starts, self.new_lens,
                           error_word=err, partition_tokens=partition_tokens)  # fmt: skip
        qkv = self.packed_qkv(batch.token_index).cuda()
        out = batch.attend(self.layer, qkv)
        torch.cuda.synchronize()
        assert int(err.item()) == 0, f"kernels reported invalid metadata: {int(err.item()):#x}"
        return pool.cpu(), out.cpu(), batch

    def packed_reference(self, out_ref: torch.Tensor, token_index: torch.Tensor) -> torch.Tensor:
        B, _, T, _ = out_ref.shape
        return out_ref.transpose(1, 2).reshape(B * T, self.C).index_select(0, token_index.cpu())
