"""The per-step metadata PagedBatch hands the kernels, checked against the reference batch view
(the oracle's restatement of tokquay/kv_cache.py:174-226) on the CPU."""

from __future__ import annotations

import random

import pytest
import torch

from oracle.paged_ref import RefPagedBatch, cdiv, slot_of
from tokquay_amd.kv_cache import PagedBatch


def make_case(seed: int, bs: int, B: int):
    rng = random.Random(seed)
    starts = [rng.choice([0, 0, rng.randint(0, 60)]) for _ in range(B)]
    lens = [rng.choice([1, 1, rng.randint(1, 40)]) for _ in range(B)]
    free = list(range(200))
    rng.shuffle(free)
    tables = []
    for s, n in zip(starts, lens):
        k = cdiv(s + n, bs) + rng.randint(0, 2)  # tables may be longer than needed
        tables.append([free.pop() for _ in range(k)])
    return starts, lens, tables


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("bs", [1, 4, 16])
def test_packed_metadata_matches_reference_scatter_targets(seed, bs):
    starts, lens, tables = make_case(seed, bs, B=7)
    pool = torch.zeros(200, 1, 2, 1, bs, 4)
    ref = RefPagedBatch(pool, bs, tables, starts, lens)
    got = PagedBatch(pool, bs, tables, starts, lens)
    B, T = got.B, got.T
    assert (B, T, got.max_ctx, got.num_blocks_gathered) == (ref.B, ref.T, ref.max_ctx, ref.num_blocks_gathered)

    # Every real token appears once; its packed row carries the reference's (block, offset) target.
    w_b, w_t, w_blk, w_off = (x.tolist() for x in ref._w)
    want = {(b * T + t): blk * bs + off for b, t, blk, off in zip(w_b, w_t, w_blk, w_off)}
    tok = got.token_index.tolist()
    assert sorted(tok) == sorted(want)
    assert dict(zip(tok, got.slot_mapping.tolist())) == want
    assert got.packed_positions.tolist() == [starts[i // T] + i % T for i in tok]

    # Decode rows first (batch order), then prefill rows contiguous per sequence.
    dec = [b for b in range(B) if lens[b] == 1]
    assert [i // T for i in tok[: len(dec)]] == dec
    assert got.last_rows.tolist() == [tok.index(b * T + lens[b] - 1) for b in range(B)]

    # Contract members equal the reference's.
    assert torch.equal(got.positions, ref.positions)
    assert torch.equal(got.last_idx, ref.last_idx)
    assert torch.equal(got.mask, ref.mask)

    # Kernel tables: the sequence's own blocks, padded with block 0.
    for i, b in enumerate(dec):
        k = cdiv(starts[b] + 1, bs)
        assert got.decode_block_tables[i, :k].tolist() == tables[b][:k]
        assert int(got.decode_context_lens[i]) == starts[b] + 1
    pre = [b for b in range(B) if lens[b] > 1]
    cu = got.prefill_cu_seqlens.tolist()
    assert cu[0] == 0 and cu[-1] == sum(lens[b] for b in pre)
    for i, b in enumerate(pre):
        assert cu[i + 1] - cu[i] == lens[b]
        assert int(got.prefill_start[i]) == starts[b]
        k = cdiv(starts[b] + lens[b], bs)
        assert got.prefill_block_tables[i, :k].tolist() == tables[b][:k]


def test_slot_rule():
    assert slot_of([7, 3, 9], 0, 4) == 28
    assert slot_of([7, 3, 9], 5, 4) == 13
    assert slot_of([7, 3, 9], 11, 4) == 39


def test_validation_matches_reference_errors():
    pool = torch.zeros(8, 1, 2, 1, 4, 4)
    with pytest.raises(ValueError):
        PagedBatch(pool, 4, [], [], [])
    with pytest.raises(ValueError):
        PagedBatch(pool, 4, [[0]], [0, 1], [1])
    with pytest.raises(ValueError, match="at least one token"):
        PagedBatch(pool, 4, [[0]], [0], [0])
    with pytest.raises(ValueError, match="cannot hold"):
        PagedBatch(pool, 4, [[0]], [0], [9])  # one block for 9 tokens (tests/test_phase3_paged.py:185-190)


def test_gather_refuses_a_cpu_pool():
    """gather runs on the HIP gather kernel only (no CPU fallback); its parity is a GPU test."""
    pool = torch.zeros(8, 1, 2, 1, 4, 64)
    with pytest.raises(ValueError):
        PagedBatch(pool, 4, [[0, 1]], [0], [5]).gather(0)


def test_attend_refuses_a_cpu_pool():
    pool = torch.zeros(8, 1, 2, 1, 4, 64)
    batch = PagedBatch(pool, 4, [[0, 1]], [0], [5])
    with pytest.raises(ValueError):
        batch.attend(0, torch.zeros(5, 3 * 64))
