"""The native metadata builder (``tokquay_amd._native``, csrc/native.cpp) on the CPU.

It replaces the batch view's Python constructor (tokquay/kv_cache.py:174-226):
the same validation order and messages, and packed metadata equal to the
reference batch view's scatter targets and padded tables (the oracle's
restatement), here on large random batches and on the edge cases.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle.paged_ref import RefPagedBatch, cdiv
from tokquay_amd import _lib
from tokquay_amd.kv_cache import PagedBatch


@pytest.fixture(scope="module")
def nat():
    return _lib.native()


def random_batch(rng: random.Random, B: int, bs: int, max_ctx: int = 1024, spare: int = 3):
    starts, lens = [], []
    for _ in range(B):
        kind = rng.random()
        n = 1 if kind < 0.6 else rng.randint(2, min(300, max_ctx))
        s = rng.randint(0, max_ctx - n) if rng.random() < 0.8 else 0
        starts.append(s)
        lens.append(n)
    free = list(range(sum(cdiv(s + n, bs) + spare for s, n in zip(starts, lens))))
    rng.shuffle(free)
    tables = [[free.pop() for _ in range(cdiv(s + n, bs) + rng.randint(0, spare))] for s, n in zip(starts, lens)]
    return tables, starts, lens


def expected(tables, starts, lens, bs):
    """Packed metadata from the reference batch view's definitions, element by element."""
    B, T = len(tables), max(lens)
    dec = [b for b in range(B) if lens[b] == 1]
    pre = [b for b in range(B) if lens[b] > 1]
    nbd = max((cdiv(starts[b] + 1, bs) for b in dec), default=0)
    nbp = max((cdiv(starts[b] + lens[b], bs) for b in pre), default=0)
    rows = [(b, 0) for b in dec] + [(b, t) for b in pre for t in range(lens[b])]
    tok = [b * T + t for b, t in rows]
    pos = [starts[b] + t for b, t in rows]
    slot = [tables[b][p // bs] * bs + p % bs for (b, _), p in zip(rows, pos)]
    last = [rows.index((b, lens[b] - 1)) for b in range(B)]
    dt = np.zeros((len(dec), nbd), np.int32)
    for i, b in enumerate(dec):
        k = cdiv(starts[b] + 1, bs)
        dt[i, :k] = tables[b][:k]
    pt = np.zeros((len(pre), nbp), np.int32)
    for i, b in enumerate(pre):
        k = cdiv(starts[b] + lens[b], bs)
        pt[i, :k] = tables[b][:k]
    dctx = [starts[b] + 1 for b in dec]
    cu = np.cumsum([0] + [lens[b] for b in pre]).tolist()
    order = sorted(range(len(dec)), key=lambda i: (-dctx[i], i))  # longest first, stable
    # Multi-token sequences by causal work (sum over the rows of the keys each sees), most first, stable.
    work = [sum(starts[b] + t + 1 for t in range(lens[b])) for b in pre]
    pre_order = sorted(range(len(pre)), key=lambda i: (-work[i], i))
    i64 = tok + pos + slot + last
    i32 = dt.ravel().tolist() + dctx + pt.ravel().tolist() + cu + [starts[b] for b in pre] + order + pre_order
    return i64, i32


@pytest.mark.parametrize("seed,B,bs", [(0, 1, 16), (1, 7, 1), (2, 64, 4), (3, 300, 16), (4, 513, 32), (5, 40, 48)])
def test_fill_matches_definitions(nat, seed, B, bs):
    rng = random.Random(seed)
    tables, starts, lens = random_batch(rng, B, bs)
    plan = nat.plan(tables, starts, lens, bs)
    want64, want32 = expected(tables, starts, lens, bs)
    assert (plan["n64"], plan["n32"]) == (len(want64), len(want32))
    assert plan["N"] == sum(lens) and plan["T"] == max(lens)
    assert plan["max_ctx"] == max(s + n for s, n in zip(starts, lens))
    h64 = torch.full((plan["n64"],), -7, dtype=torch.int64)
    h32 = torch.full((plan["n32"],), -7, dtype=torch.int32)  # garbage: every element must be written
    nat.fill(tables, starts, lens, bs, h64.data_ptr(), h64.numel(), h32.data_ptr(), h32.numel())
    assert h64.tolist() == want64
    assert h32.tolist() == want32


@pytest.mark.parametrize("seed", range(4))
def test_batch_view_matches_reference_view(seed):
    rng = random.Random(100 + seed)
    bs = 16
    tables, starts, lens = random_batch(rng, 50, bs, max_ctx=200)
    pool = torch.zeros(max(max(t) for t in tables) + 1, 1, 2, 1, bs, 4)
    ref = RefPagedBatch(pool, bs, tables, starts, lens)
    got = PagedBatch(pool, bs, tables, starts, lens)
    assert torch.equal(got.positions, ref.positions)
    assert torch.equal(got.last_idx, ref.last_idx)
    assert torch.equal(got.mask, ref.mask)
    w_b, w_t, w_blk, w_off = (x.tolist() for x in ref._w)
    want = {b * got.T + t: blk * bs + off for b, t, blk, off in zip(w_b, w_t, w_blk, w_off)}
    assert dict(zip(got.token_index.tolist(), got.slot_mapping.tolist())) == want


def test_other_sequence_types_are_accepted():
    pool = torch.zeros(8, 1, 2, 1, 4, 4)
    a = PagedBatch(pool, 4, [[3, 1], [2]], [2, 0], [3, 1])
    b = PagedBatch(pool, 4, ((3, 1), np.array([2])), np.array([2, 0]), (3, 1))
    for name in ("token_index", "slot_mapping", "last_rows", "decode_block_tables", "prefill_block_tables"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert a.context_lens == b.context_lens == [5, 1]


def test_validation_order_and_messages(nat):
    pool = torch.zeros(8, 1, 2, 1, 4, 4)
    with pytest.raises(ValueError, match="non-empty and the same length"):
        PagedBatch(pool, 4, [[0]], [0], [1, 1])
    # Several violations at once: the reference checks new_lens, then starts, then tables.
    with pytest.raises(ValueError, match="at least one token"):
        PagedBatch(pool, 4, [[], [0]], [-1, 0], [1, 0])
    with pytest.raises(ValueError, match="non-negative"):
        PagedBatch(pool, 4, [[], [0]], [0, -1], [1, 1])
    with pytest.raises(ValueError, match=r"sequence 1: 1 blocks cannot hold 5 tokens"):
        PagedBatch(pool, 4, [[0], [1]], [0, 4], [1, 1])
    with pytest.raises((ValueError, OverflowError)):
        PagedBatch(pool, 4, [[2**31]], [0], [1])
    # A start near the top of int64: the context sum must not wrap (it would pass the table check).
    with pytest.raises(ValueError, match=rf"sequence 0: 1 blocks cannot hold {2**62 + 1} tokens"):
        PagedBatch(pool, 4, [[0]], [2**62], [1])
    with pytest.raises(ValueError, match=rf"sequence 0: 1 blocks cannot hold {2**63 + 2**62} tokens"):
        PagedBatch(pool, 4, [[0]], [2**63 - 1], [2**62 + 1])
    # Past int32 (the kernels' position type) even when the table is long enough.
    with pytest.raises(ValueError, match="int32 positions"):
        PagedBatch(pool, 1024, [[0] * (2**21 + 1)], [2**31 - 1], [1])
    # The last context the kernels take is accepted.
    assert PagedBatch(pool, 1024, [[0] * 2**21], [2**31 - 2], [1]).max_ctx == 2**31 - 1
    # Every context fits int32 but the batch's new tokens together do not (row offsets are int32).
    with pytest.raises(ValueError, match="int32 rows"):
        nat.plan([[0] * 16] * 3, [0, 0, 0], [2**30] * 3, 2**26)
    with pytest.raises(ValueError, match="do not match"):
        h = torch.empty(100, dtype=torch.int64)
        nat.fill([[0]], [0], [1], 4, h.data_ptr(), 3, h.data_ptr(), 50)


def test_attend_entry_rejects_bad_sizes_without_launching(nat):
    args = [0] * 31
    args[9] = 0.125
    args[12] = 0  # N = 0
    with pytest.raises(ValueError):
        nat.attend(*args)


# ------------------------------------------------------------------ captured decode step metadata
def decode_seqs(rng: random.Random, n: int, bs: int, mb: int):
    from tokquay_amd.sequence import Sequence

    seqs = []
    for i in range(n):
        p = rng.randint(0, mb * bs - 1)
        prompt = [rng.randrange(50256) for _ in range(rng.randint(1, p + 1))]
        s = Sequence(i, prompt, output_token_ids=[rng.randrange(50256) for _ in range(p + 1 - len(prompt))])
        s.num_cached_tokens = p
        s.block_table = [rng.randrange(10_000) for _ in range(cdiv(p + 1, bs) + rng.randint(0, 2))]
        seqs.append(s)
    return seqs


def decode_expected(seqs, bucket, src_rows, cap, mb, bs):
    ids, pos, src = [0] * cap, [0] * cap, [0] * cap
    tables, ctx = [[0] * mb for _ in range(cap)], [0] * cap
    for i, s in enumerate(seqs):
        p = s.num_cached_tokens
        ids[i] = 0 if src_rows is not None else s.token_ids[p]  # the one token the row feeds
        src[i] = -1 if src_rows is None else src_rows[i]
        pos[i] = p
        k = min(len(s.block_table), mb)
        tables[i][:k] = s.block_table[:k]
        ctx[i] = p + 1
    for i in range(len(seqs), bucket):
        src[i] = -1
    order = sorted(range(bucket), key=lambda r: (-ctx[r], r))
    return ids, pos, src, tables, ctx, order


@pytest.mark.parametrize("n,bucket,with_src", [(1, 1, False), (5, 8, False), (5, 8, True), (200, 256, False),
                                               (256, 256, True), (0, 4, False)])  # fmt: skip
def test_fill_decode_matches_definitions(nat, n, bucket, with_src):
    rng = random.Random(n * 3 + bucket)
    cap, bs, mb = 256, 16, 64
    seqs = decode_seqs(rng, n, bs, mb)
    src_rows = None
    if with_src:
        src_rows = [rng.randrange(cap) for _ in range(n)]
        for s in seqs:  # the fed token is not appended yet
            s.output_token_ids.pop() if s.output_token_ids else None
        seqs = [s for s in seqs if s.num_tokens == s.num_cached_tokens]
        src_rows = src_rows[: len(seqs)]
    h64 = torch.full((3 * cap,), -9, dtype=torch.int64)
    h32 = torch.full((cap * mb + 2 * cap,), -9, dtype=torch.int32)
    before64, before32 = h64.clone(), h32.clone()
    nat.fill_decode(seqs, bucket, src_rows, h64.data_ptr(), h64.numel(), h32.data_ptr(), h32.numel(), cap, mb, bs,
                    mb * bs)  # fmt: skip
    ids, pos, src, tables, ctx, order = decode_expected(seqs, bucket, src_rows, cap, mb, bs)
    a64, a32 = h64.view(3, cap), h32
    assert a64[0, :bucket].tolist() == ids[:bucket]
    assert a64[1, :bucket].tolist() == pos[:bucket]
    assert a64[2, :bucket].tolist() == src[:bucket]
    assert a32[: cap * mb].view(cap, mb)[:bucket].tolist() == tables[:bucket]
    assert a32[cap * mb : cap * mb + bucket].tolist() == ctx[:bucket]
    assert a32[cap * mb + cap : cap * mb + cap + bucket].tolist() == order
    # Rows past the bucket are not touched.
    assert torch.equal(a64[:, bucket:], before64.view(3, cap)[:, bucket:])
    assert torch.equal(a32[: cap * mb].view(cap, mb)[bucket:], before32[: cap * mb].view(cap, mb)[bucket:])


def test_fill_decode_errors(nat):
    from tokquay_amd.sequence import Sequence

    cap, bs, mb = 4, 4, 2
    h64 = torch.zeros(3 * cap, dtype=torch.int64)
    h32 = torch.zeros(cap * mb + 2 * cap, dtype=torch.int32)

    def call(seqs, bucket=4, src=None):
        nat.fill_decode(seqs, bucket, src, h64.data_ptr(), h64.numel(), h32.data_ptr(), h32.numel(), cap, mb, bs, 8)

    s = Sequence(0, [1, 2, 3])
    s.num_cached_tokens, s.block_table = 2, [5]
    call([s])  # feeds position 2 of block 5
    with pytest.raises(ValueError, match="exactly one token"):
        call([s], src=[0])  # nothing uncached is expected with source rows
    with pytest.raises(ValueError, match=r"src_rows needs one entry in \[0, 4\)"):
        s.num_cached_tokens = 3
        call([s], src=[4])
    s.num_cached_tokens = 2
    s.block_table = []
    with pytest.raises(ValueError, match="does not cover"):
        call([s])
    s.block_table = [5, 6, 7]
    s.prompt_token_ids = list(range(9))
    s.num_cached_tokens = 8  # position 8 = max_ctx: past n_positions
    with pytest.raises(ValueError, match="does not cover"):
        call([s])
    with pytest.raises(ValueError, match="do not match"):
        call([s, s], bucket=1)
