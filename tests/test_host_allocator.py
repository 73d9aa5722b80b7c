"""BlockAllocator behaviour (tokquay/kv_cache.py:38-127), restating the reference's allocator tests
(tests/test_phase3_paged.py:193-345) against this package."""

from __future__ import annotations

import pytest
from hypothesis import given, settings, strategies as st
from hypothesis.stateful import RuleBasedStateMachine, invariant, precondition, rule

from tokquay_amd.kv_cache import BlockAllocator, OutOfBlocksError, cdiv
from tokquay_amd.model import GPT2Config
from tokquay_amd.sequence import Sequence

TINY = GPT2Config(vocab_size=8, n_positions=64, n_embd=4, n_layer=1, n_head=1)


def tiny_alloc(num_blocks=8, block_size=4):
    return BlockAllocator(TINY, num_blocks, block_size, device="cpu")


def test_pool_layout():
    alloc = tiny_alloc(8, 4)
    assert alloc.pool.shape == (8, 1, 2, 1, 4, 4)
    full = BlockAllocator(GPT2Config(), 2, 16, device="cpu")
    assert full.pool.shape == (2, 12, 2, 12, 16, 64)
    assert full.bytes_per_block == 12 * 2 * 12 * 16 * 64 * 4  # 1.125 MiB


def test_lifo_free_list_hands_out_block_0_first():
    alloc = tiny_alloc()
    s = Sequence(0, [0] * 9)
    alloc.allocate(s)
    assert s.block_table == [0, 1, 2]


def test_allocate_takes_ceil_blocks_and_free_returns_them():
    alloc = tiny_alloc()
    s = Sequence(0, [0] * 9)
    alloc.allocate(s)
    assert len(s.block_table) == 3 and alloc.num_free_blocks == 5
    assert all(alloc.ref_counts[b] == 1 for b in s.block_table)
    alloc.free(s)
    assert s.block_table == [] and alloc.num_free_blocks == 8 and all(c == 0 for c in alloc.ref_counts)


def test_append_slot_grabs_a_block_only_when_the_current_one_fills():
    alloc = tiny_alloc(block_size=4)
    s = Sequence(0, [0] * 3)
    alloc.allocate(s)
    grabbed = []
    for _ in range(9):
        s.append_token(0)
        grabbed.append(alloc.append_slot(s))
    assert grabbed == [False, True, False, False, False, True, False, False, False]
    assert len(s.block_table) == 3


def test_out_of_blocks_leaves_state_unchanged():
    alloc = tiny_alloc(num_blocks=3, block_size=4)
    s = Sequence(0, [0] * 8)
    alloc.allocate(s)
    big = Sequence(1, [0] * 8)
    assert not alloc.can_allocate(big.num_tokens)
    with pytest.raises(OutOfBlocksError):
        alloc.allocate(big)
    assert big.block_table == [] and alloc.num_free_blocks == 1
    s.append_token(0)
    assert alloc.can_append_slot(s)
    alloc.append_slot(s)
    for _ in range(4):
        s.append_token(0)
    assert not alloc.can_append_slot(s)
    with pytest.raises(OutOfBlocksError):
        alloc.append_slot(s)
    assert len(s.block_table) == 3 and alloc.num_free_blocks == 0


def test_double_allocate_and_double_free_are_caught():
    alloc = tiny_alloc()
    s = Sequence(0, [0] * 4)
    alloc.allocate(s)
    with pytest.raises(ValueError):
        alloc.allocate(s)
    stale = list(s.block_table)
    alloc.free(s)
    alloc.free(s)  # block-less: no-op
    s.block_table = stale
    with pytest.raises(RuntimeError):
        alloc.free(s)


def test_live_sequences_never_share_a_block():
    alloc = tiny_alloc(num_blocks=64, block_size=4)
    seqs = [Sequence(i, list(range(1, 1 + n))) for i, n in enumerate([5, 9, 13, 2])]
    for s in seqs:
        alloc.allocate(s)
    owned = [b for s in seqs for b in s.block_table]
    assert len(owned) == len(set(owned))


@settings(deadline=None, max_examples=200)
@given(sizes=st.lists(st.integers(1, 40), min_size=1, max_size=20), order=st.randoms(use_true_random=False))
def test_free_count_returns_to_initial_after_any_alloc_free_order(sizes, order):
    alloc = tiny_alloc(num_blocks=16, block_size=4)
    live = []
    for i, n in enumerate(sizes):
        s = Sequence(i, [0] * n)
        if alloc.can_allocate(n):
            alloc.allocate(s)
            live.append(s)
    order.shuffle(live)
    for s in live:
        alloc.free(s)
    assert alloc.num_free_blocks == alloc.num_blocks
    assert sorted(alloc._free) == list(range(alloc.num_blocks))


class AllocatorMachine(RuleBasedStateMachine):
    def __init__(self):
        super().__init__()
        self.alloc = tiny_alloc(num_blocks=24, block_size=4)
        self.seqs: dict[int, Sequence] = {}
        self.next_id = 0

    @rule(n=st.integers(1, 30))
    def add(self, n):
        s = Sequence(self.next_id, [0] * n)
        self.next_id += 1
        if self.alloc.can_allocate(n):
            self.alloc.allocate(s)
            self.seqs[s.seq_id] = s
        else:
            before = self.alloc.num_free_blocks
            with pytest.raises(OutOfBlocksError):
                self.alloc.allocate(s)
            assert self.alloc.num_free_blocks == before and s.block_table == []

    @precondition(lambda self: self.seqs)
    @rule(data=st.data())
    def grow(self, data):
        s = self.seqs[data.draw(st.sampled_from(sorted(self.seqs)))]
        s.append_token(0)
        if self.alloc.can_append_slot(s):
            self.alloc.append_slot(s)
        else:
            with pytest.raises(OutOfBlocksError):
                self.alloc.append_slot(s)
            s.output_token_ids.pop()

    @precondition(lambda self: self.seqs)
    @rule(data=st.data())
    def free(self, data):
        self.alloc.free(self.seqs.pop(data.draw(st.sampled_from(sorted(self.seqs)))))

    @invariant()
    def blocks_are_conserved_and_unshared(self):
        owned = [b for s in self.seqs.values() for b in s.block_table]
        assert len(owned) == len(set(owned))
        assert self.alloc.num_free_blocks + len(owned) == self.alloc.num_blocks
        assert set(owned).isdisjoint(self.alloc._free)
        for s in self.seqs.values():
            assert len(s.block_table) == cdiv(s.num_tokens, self.alloc.block_size)


TestAllocatorMachine = AllocatorMachine.TestCase
TestAllocatorMachine.settings = settings(deadline=None, max_examples=60, stateful_step_count=50)
