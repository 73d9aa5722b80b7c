"""Reference restatement of the paged batch view and attention math (test oracle).

``RefPagedBatch`` follows tokquay/kv_cache.py:174-242 step for step:
block tables padded to the longest row with block 0 (:198-201), positions and
last index (:203-206), the mask ``j <= start+t & j < ctx`` (:208-214), scatter
targets for real tokens only (:216-226), ``write`` as an advanced-index
assignment (:228-232) and ``gather`` as an index + permute + reshape copy
(:234-242). ``ref_attention`` is tokquay/model.py:94-96. Everything runs in torch
on any device / dtype (the CPU float64 copy is the oracle proper).

``brute_force_attention`` is the textbook definition in float64 numpy, with no
pool, no gather and no mask: it is what pins the two above.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def slot_of(block_table: list[int], p: int, block_size: int) -> int:
    """Flat pool slot of position ``p`` (tokquay/kv_cache.py:9-10)."""
    return block_table[p // block_size] * block_size + p % block_size


class RefPagedBatch:
    """The reference's ``PagedBatch`` (tokquay/kv_cache.py:160-242)."""

    def __init__(self, pool: torch.Tensor, block_size: int, block_tables, start, new_lens):
        if not block_tables or not (len(block_tables) == len(start) == len(new_lens)):
            raise ValueError("block_tables, start and new_lens must be non-empty and the same length")
        if min(new_lens) < 1:
            raise ValueError("every sequence must feed at least one token")
        device = pool.device
        bs = block_size
        ctx = [s + n for s, n in zip(start, new_lens)]
        for b, (tbl, c) in enumerate(zip(block_tables, ctx)):
            if len(tbl) < cdiv(c, bs):
                raise ValueError(f"sequence {b}: {len(tbl)} blocks cannot hold {c} tokens")
        B, T = len(block_tables), max(new_lens)
        nb = max(cdiv(c, bs) for c in ctx)
        self.pool, self.block_size, self.B, self.T, self.num_blocks_gathered = pool, bs, B, T, nb
        self.max_ctx = max(ctx)
        padded = [list(tbl[:nb]) + [0] * (nb - len(tbl[:nb])) for tbl in block_tables]
        self.block_tables = torch.tensor(padded, dtype=torch.long, device=device)
        start_t = torch.tensor(start, dtype=torch.long, device=device)
        ctx_t = torch.tensor(ctx, dtype=torch.long, device=device)
        self.positions = start_t[:, None] + torch.arange(T, device=device)[None, :]
        self.last_idx = torch.tensor([n - 1 for n in new_lens], dtype=torch.long, device=device)
        k_pos = torch.arange(nb * bs, device=device)[None, None, :]
        self.mask = ((k_pos <= self.positions[:, :, None]) & (k_pos < ctx_t[:, None, None]))[:, None]
        w_b, w_t, w_blk, w_off = [], [], [], []
        for b, (tbl, s, n) in enumerate(zip(block_tables, start, new_lens)):
            for t in range(n):
                p = s + t
                w_b.append(b)
                w_t.append(t)
                w_blk.append(tbl[p // bs])
                w_off.append(p % bs)
        self._w = torch.tensor([w_b, w_t, w_blk, w_off], dtype=torch.long, device=device)

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        w_b, w_t, w_blk, w_off = self._w
        pl = self.pool[:, layer]  # [num_blocks, 2, H, bs, d]
        pl[w_blk, 0, :, w_off] = k[w_b, :, w_t]
        pl[w_blk, 1, :, w_off] = v[w_b, :, w_t]

    def gather(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        out = []
        for kv in (0, 1):
            g = self.pool[self.block_tables, layer, kv]  # [B, nb, H, bs, d]
            g = g.permute(0, 2, 1, 3, 4)
            out.append(g.reshape(self.B, g.shape[1], -1, g.shape[-1]))
        return out[0], out[1]


def ref_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, allowed: torch.Tensor) -> torch.Tensor:
    """``softmax((q @ k^T) / sqrt(d), masked) @ v`` on ``[B, H, T|S, d]`` (tokquay/model.py:94-96)."""
    scores = (q @ k.transpose(-2, -1)) / math.sqrt(q.size(-1))
    scores = scores.masked_fill(~allowed, float("-inf"))
    return torch.softmax(scores, dim=-1) @ v


def ref_paged_attention_step(batch: RefPagedBatch, layer: int, q, k, v) -> torch.Tensor:
    """The paged branch of Attention.forward (tokquay/model.py:73-78, :94-96): write, gather, attend.
    q, k, v: ``[B, H, T, d]``; returns ``[B, H, T, d]``."""
    batch.write(layer, k, v)
    kg, vg = batch.gather(layer)
    return ref_attention(q, kg, vg, batch.mask)


def brute_force_attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float) -> np.ndarray:
    """Textbook softmax attention in float64 for one query set and one head.

    q ``[T, d]``, keys/values ``[S, d]`` with query ``t`` seeing keys ``0 .. S - T + t``
    (the queries are the last T positions). Returns ``[T, d]``.
    """
    q, keys, values = (np.asarray(x, dtype=np.float64) for x in (q, keys, values))
    T, S = q.shape[0], keys.shape[0]
    out = np.empty((T, values.shape[1]), dtype=np.float64)
    for t in range(T):
        visible = S - T + t + 1
        s = (keys[:visible] @ q[t]) * scale
        w = np.exp(s - s.max())
        out[t] = (w[:, None] * values[:visible]).sum(0) / w.sum()
    return out
