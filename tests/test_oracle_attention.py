"""Pins the oracle's paged attention (oracle/paged_ref.py) without trusting its own formulas.

* brute_force_attention is checked against closed forms and scipy's softmax;
* RefPagedBatch + ref_attention (the reference's scatter / gather / mask /
  masked softmax, restated) is checked against brute force over each
  sequence's own positions, in float64, and against invariants: relabelling
  blocks, garbage in unused slots, and block size 4 vs 16;
* mistakes planted in the oracle (a dropped causal term, a missing scale,
  values swapped for keys, a gather without its permute) make those checks fail.
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest
import scipy.special
import torch

from oracle.paged_ref import RefPagedBatch, brute_force_attention, cdiv, ref_attention, ref_paged_attention_step

H, D = 2, 8  # small heads keep the float64 brute force fast


# ------------------------------------------------------------------------------ brute force itself
def test_brute_force_closed_forms():
    rng = np.random.default_rng(0)
    v = rng.standard_normal((5, D))
    same_keys = np.tile(rng.standard_normal(D), (5, 1))
    q = rng.standard_normal((1, D))
    # Identical keys: uniform weights, the output is the mean of the values.
    np.testing.assert_allclose(brute_force_attention(q, same_keys, v, 0.3)[0], v.mean(0), rtol=1e-13)
    # One visible key: the output is that value.
    np.testing.assert_allclose(brute_force_attention(q, same_keys[:1], v[:1], 0.3)[0], v[0], rtol=1e-13)
    # Causal: query t of T sees keys 0 .. S-T+t; the first of 3 queries over 3 keys sees key 0 only.
    out = brute_force_attention(rng.standard_normal((3, D)), rng.standard_normal((3, D)), v[:3], 1.0)
    np.testing.assert_allclose(out[0], v[0], rtol=1e-13)
    # A dominant score selects its value.
    keys = np.zeros((4, D))
    keys[2, 0] = 1000.0
    qq = np.zeros((1, D))
    qq[0, 0] = 1.0
    np.testing.assert_allclose(brute_force_attention(qq, keys, v[:4], 1.0)[0], v[2], atol=1e-12)


def test_brute_force_matches_scipy_softmax():
    rng = np.random.default_rng(1)
    q, k, v = rng.standard_normal((1, D)), rng.standard_normal((37, D)), rng.standard_normal((37, D))
    w = scipy.special.softmax(k @ q[0] / math.sqrt(D))
    np.testing.assert_allclose(brute_force_attention(q, k, v, 1 / math.sqrt(D))[0], w @ v, rtol=1e-12)


# ------------------------------------------------------------------------------ scenario helpers
def scenario(starts, lens, bs, seed, num_blocks=None, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)  # data: independent of the block size
    g_pool = torch.Generator().manual_seed(seed + 1)
    ctxs = [s + n for s, n in zip(starts, lens)]
    nb = num_blocks or sum(cdiv(c, bs) for c in ctxs) + 5
    pool = (torch.randn(nb, 1, 2, H, bs, D, generator=g_pool) * 50).to(dtype)
    free = list(range(nb))
    random.Random(seed).shuffle(free)
    tables = []
    for c in ctxs:
        tables.append([free.pop() for _ in range(cdiv(c, bs))])
    # History for positions already cached (one K/V per position, shared across block sizes).
    hist_k = torch.randn(len(starts), H, max(starts) + 1, D, generator=g).to(dtype)
    hist_v = torch.randn(len(starts), H, max(starts) + 1, D, generator=g).to(dtype)
    for b, (tbl, s) in enumerate(zip(tables, starts)):
        for p in range(s):
            pool[tbl[p // bs], 0, 0, :, p % bs] = hist_k[b, :, p]
            pool[tbl[p // bs], 0, 1, :, p % bs] = hist_v[b, :, p]
    T = max(lens)
    q, k, v = (torch.randn(len(starts), H, T, D, generator=g).to(dtype) for _ in range(3))
    return pool, tables, q, k, v, hist_k, hist_v


def brute(starts, lens, q, k, v, hist_k, hist_v):
    """Expected outputs {(b, t): [H, D]} from each sequence's own history + new tokens."""
    out = {}
    for b, (s, n) in enumerate(zip(starts, lens)):
        for h in range(H):
            keys = torch.cat([hist_k[b, h, :s], k[b, h, :n]]).numpy()
            vals = torch.cat([hist_v[b, h, :s], v[b, h, :n]]).numpy()
            res = brute_force_attention(q[b, h, :n].numpy(), keys, vals, 1 / math.sqrt(D))
            for t in range(n):
                out.setdefault((b, t), np.zeros((H, D)))[h] = res[t]
    return out


CASES = [
    ([0], [1], 4),
    ([0], [9], 4),
    ([7], [1], 4),
    ([0, 3, 20, 0], [5, 1, 9, 13], 4),
    ([0, 0, 15, 16, 31], [16, 17, 1, 1, 2], 16),
    ([5, 0, 40], [1, 33, 1], 1),
]


@pytest.mark.parametrize("starts,lens,bs", CASES)
def test_oracle_paged_attention_equals_brute_force(starts, lens, bs):
    pool, tables, q, k, v, hk, hv = scenario(starts, lens, bs, seed=len(starts) * 10 + bs)
    batch = RefPagedBatch(pool, bs, tables, starts, lens)
    out = ref_paged_attention_step(batch, 0, q, k, v)
    want = brute(starts, lens, q, k, v, hk, hv)
    for (b, t), exp in want.items():
        np.testing.assert_allclose(out[b, :, t].numpy(), exp, rtol=1e-10, atol=1e-12)


def test_relabelling_blocks_and_garbage_leave_the_output_unchanged():
    starts, lens, bs = [0, 3, 20, 0], [5, 1, 9, 13], 4
    pool, tables, q, k, v, _, _ = scenario(starts, lens, bs, seed=3)
    base = ref_paged_attention_step(RefPagedBatch(pool.clone(), bs, tables, starts, lens), 0, q, k, v)
    # Relabel: move every block to a new id through a permutation of the pool.
    perm = torch.randperm(pool.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    pool2 = pool[perm]  # new block i holds old block perm[i]
    tables2 = [[int(inv[b]) for b in t] for t in tables]
    # Fresh garbage in every slot nobody reads (unused blocks and the tails of last blocks).
    owned = {b for t in tables2 for b in t}
    for b in range(pool2.shape[0]):
        if b not in owned:
            pool2[b] = torch.randn_like(pool2[b]) * 1e3
    out = ref_paged_attention_step(RefPagedBatch(pool2, bs, tables2, starts, lens), 0, q, k, v)
    for b, n in enumerate(lens):
        torch.testing.assert_close(out[b, :, :n], base[b, :, :n], rtol=0, atol=1e-12)


def test_block_size_4_and_16_agree():
    starts, lens = [0, 18, 3], [21, 1, 7]
    outs = []
    for bs in (4, 16):
        pool, tables, q, k, v, hk, hv = scenario(starts, lens, bs, seed=42)
        outs.append(ref_paged_attention_step(RefPagedBatch(pool, bs, tables, starts, lens), 0, q, k, v))
    for b, n in enumerate(lens):
        torch.testing.assert_close(outs[0][b, :, :n], outs[1][b, :, :n], rtol=0, atol=1e-12)


def test_padded_query_rows_never_write():
    starts, lens, bs = [0, 6], [9, 1], 4
    pool, tables, q, k, v, _, _ = scenario(starts, lens, bs, seed=5)
    before = pool.clone()
    RefPagedBatch(pool, bs, tables, starts, lens).write(0, k, v)
    # Exactly the slots of real new tokens changed.
    changed = {(b_, o) for b_ in range(pool.shape[0]) for o in range(bs) if not torch.equal(pool[b_, :, :, :, o], before[b_, :, :, :, o])}
    expected = {(tables[b][p // bs], p % bs) for b, (s, n) in enumerate(zip(starts, lens)) for p in range(s, s + n)}
    assert changed == expected


# ------------------------------------------------------------------------------ planted mistakes
def _run_with(monkeypatch, fn_name, replacement):
    import oracle.paged_ref as pr

    monkeypatch.setattr(pr, fn_name, replacement)
    starts, lens, bs = [0, 3, 20, 0], [5, 1, 9, 13], 4
    pool, tables, q, k, v, hk, hv = scenario(starts, lens, bs, seed=77)
    batch = pr.RefPagedBatch(pool, bs, tables, starts, lens)
    out = pr.ref_paged_attention_step(batch, 0, q, k, v)
    want = brute(starts, lens, q, k, v, hk, hv)
    return max(float(np.abs(out[b, :, t].numpy() - e).max()) for (b, t), e in want.items())


def test_planted_mistakes_are_caught(monkeypatch):
    def no_causal(q, k, v, allowed):
        s = (q @ k.transpose(-2, -1)) / math.sqrt(q.size(-1))
        s = s.masked_fill(~allowed[..., -1:, :], float("-inf"))  # every query sees the last row's keys
        return torch.softmax(s, -1) @ v

    def no_scale(q, k, v, allowed):
        return torch.softmax((q @ k.transpose(-2, -1)).masked_fill(~allowed, float("-inf")), -1) @ v

    def keys_as_values(q, k, v, allowed):
        return ref_attention(q, k, k, allowed)

    assert _run_with(monkeypatch, "ref_attention", ref_attention) < 1e-10  # the unmodified oracle passes
    for bad in (no_causal, no_scale, keys_as_values):
        assert _run_with(monkeypatch, "ref_attention", bad) > 1e-3, bad.__name__


def test_planted_gather_mistake_is_caught(monkeypatch):
    import oracle.paged_ref as pr

    def gather_without_permute(self, layer):
        out = []
        for kv in (0, 1):
            g = self.pool[self.block_tables, layer, kv]  # [B, nb, H, bs, d]
            out.append(g.reshape(self.B, g.shape[2], -1, g.shape[-1]))  # heads and blocks mixed up
        return out[0], out[1]

    monkeypatch.setattr(pr.RefPagedBatch, "gather", gather_without_permute)
    assert _run_with(monkeypatch, "ref_attention", ref_attention) > 1e-3
