"""GPU parity of the three kernels against the reference's gather-and-attend path.

Bar: bit-exact pool after the cache write (it is a copy); fp32 attention
outputs within 1e-5 relative / 1e-4 absolute of the reference path (CPU fp32)
and of float64 brute-force attention.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from tests.paged_cases import ATOL, RTOL, Scenario, cdiv

pytestmark = pytest.mark.gpu


def check(sc: Scenario, partition_tokens: int = 0, brute: bool = True):
    pool_ref, out_ref = sc.reference()
    pool_gpu, out_gpu, batch = sc.run_product(partition_tokens)
    assert torch.equal(pool_gpu, pool_ref), "pool differs from the reference scatter"
    want = sc.packed_reference(out_ref, batch.token_index)
    torch.testing.assert_close(out_gpu, want, rtol=RTOL, atol=ATOL)
    if brute:
        rows = batch.token_index.cpu().tolist()
        exact = sc.brute_force(pool_ref)
        T = sc.q.shape[2]
        got = out_gpu.view(-1, sc.H, 64).double().numpy()
        for r, flat in enumerate(rows):
            b, t = divmod(flat, T)
            np.testing.assert_allclose(got[r], exact[b][t], rtol=RTOL, atol=ATOL)
    return out_gpu, batch


# ------------------------------------------------------------------------------ decode
def config2_contexts(seed: int = 0, num_blocks: int = 1024, block_size: int = 16) -> tuple[list[int], int]:
    """64 context lengths ~ U[16, 512]; redrawn (seed, seed+1, ...) until they fit the 1024-block pool."""
    s = seed
    while True:
        rng = random.Random(s)
        ctx = [rng.randint(16, 512) for _ in range(64)]
        if sum(cdiv(c, block_size) for c in ctx) <= num_blocks:
            return ctx, s
        s += 1


@pytest.mark.parametrize("n_layer,layer", [(1, 0), (12, 7)])
def test_decode_config2_op(n_layer, layer):
    ctx, _ = config2_contexts()
    sc = Scenario([c - 1 for c in ctx], [1] * len(ctx), block_size=16, n_layer=n_layer, layer=layer,
                  num_blocks=1024, seed=11)  # fmt: skip
    out, batch = check(sc)
    assert batch.num_decode == 64 and batch.num_prefill == 0


@pytest.mark.parametrize("block_size", [1, 4, 8, 16, 32])
@pytest.mark.parametrize("partition_tokens", [0, 16, 64, 256, 1024])
def test_decode_edge_contexts(block_size, partition_tokens):
    ctx = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 255, 256, 257, 511, 512, 1023, 1024]
    sc = Scenario([c - 1 for c in ctx], [1] * len(ctx), block_size=block_size, seed=block_size)
    check(sc, partition_tokens)


@pytest.mark.parametrize("partition_tokens", [16, 32])
def test_decode_more_than_64_partitions(partition_tokens):
    """Contexts past 1024 positions at short partitions: up to 188 partitions per sequence, which
    the merge takes 64 at a time (65 = one full pass and one partition)."""
    ctx = [1040, 1025, 3000, 65 * 16, 64 * 16, 17]
    sc = Scenario([c - 1 for c in ctx], [1] * len(ctx), block_size=16, seed=21)
    check(sc, partition_tokens)


@pytest.mark.parametrize("block_size", [1, 16, 32])
@pytest.mark.parametrize("partition_tokens", [0, 16, 1024])
def test_decode_write_equals_cache_write_then_decode(block_size, partition_tokens):
    """tq_paged_decode_write == tq_cache_write + tq_paged_decode, bit for bit (output and pool), with
    a padding row (context 0, writes nothing) and the new position at every block offset class."""
    from tokquay_amd import ops

    ctx = [1, 2, block_size, block_size + 1, 77, 300, 0, 1024]
    n_layer, layer = 2, 1
    nb = sum(cdiv(c, block_size) for c in ctx) + 2
    pool0 = torch.randn(nb, n_layer, 2, 12, block_size, 64, generator=torch.Generator().manual_seed(5)) * 50
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(6)).tolist()
    width = cdiv(1024, block_size)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    slots, i = [], 0
    for b, c in enumerate(ctx):
        n = cdiv(c, block_size)
        tables[b, :n] = torch.tensor(perm[i : i + n], dtype=torch.int32)
        i += n
        slots.append(int(tables[b, (c - 1) // block_size]) * block_size + (c - 1) % block_size if c else -1)
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(len(ctx), 3 * 768, generator=g).cuda()
    q, k, v = qkv[:, :768], qkv[:, 768:1536], qkv[:, 1536:]
    tables, cl = tables.cuda(), torch.tensor(ctx, dtype=torch.int32, device="cuda")
    sm = torch.tensor(slots, dtype=torch.int64, device="cuda")
    pa, pb = pool0.cuda(), pool0.cuda()
    oa, ob = torch.empty(len(ctx), 768, device="cuda"), torch.empty(len(ctx), 768, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.cache_write(pa, layer, k, v, sm, err)
    ops.paged_decode(oa, q, pa, layer, tables, cl, 1024, partition_tokens=partition_tokens, d_error=err)
    ops.paged_decode(ob, q, pb, layer, tables, cl, 1024, partition_tokens=partition_tokens, d_error=err,
                     k_new=k, v_new=v)  # fmt: skip
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.equal(oa, ob)
    assert torch.equal(pa, pb)
    assert not torch.equal(pb, pool0.cuda())  # the new rows did land


def test_decode_dispatch_order_does_not_change_results():
    """seq_order only reorders the dispatch: identical bits for any permutation; an entry out of range
    is reported (TQ_DEVERR_ORDER) and skipped."""
    from tokquay_amd import _lib, ops

    rng = random.Random(12)
    ctx = [rng.randint(1, 700) for _ in range(40)]
    nb = sum(cdiv(c, 16) for c in ctx) + 4
    pool = torch.randn(nb, 1, 2, 12, 16, 64, generator=torch.Generator().manual_seed(12)).cuda()
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(13)).tolist()
    width = max(cdiv(c, 16) for c in ctx)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    i = 0
    for b, c in enumerate(ctx):
        tables[b, : cdiv(c, 16)] = torch.tensor(perm[i : i + cdiv(c, 16)], dtype=torch.int32)
        i += cdiv(c, 16)
    tables, cl = tables.cuda(), torch.tensor(ctx, dtype=torch.int32, device="cuda")
    q = torch.randn(len(ctx), 768, generator=torch.Generator().manual_seed(14)).cuda()
    # 64-position partitions (partition grid + merge) and the automatic choice, which at 40 sequences
    # is the small-batch kernel (one workgroup of several waves per (sequence, head)).
    for partition_tokens in (64, 0):
        outs = []
        for order in (None, sorted(range(len(ctx)), key=lambda b: -ctx[b]), torch.randperm(len(ctx)).tolist()):
            out = torch.empty_like(q)
            so = None if order is None else torch.tensor(order, dtype=torch.int32, device="cuda")
            ops.paged_decode(out, q, pool, 0, tables, cl, max(ctx), partition_tokens=partition_tokens, seq_order=so)
            outs.append(out)
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        bad = torch.arange(len(ctx), dtype=torch.int32, device="cuda")
        bad[3] = len(ctx) + 7
        out = torch.zeros_like(q)
        ops.paged_decode(out, q, pool, 0, tables, cl, max(ctx), partition_tokens=partition_tokens, seq_order=bad,
                         d_error=err)  # fmt: skip
        torch.cuda.synchronize()
        assert int(err.item()) == _lib.DEVERR_ORDER
        keep = [b for b in range(len(ctx)) if b != 3]
        assert torch.equal(out[keep], outs[0][keep])


def test_decode_config4_scale():
    """256 sequences, contexts ~ U[256, 1024], block size 16 (the decode-throughput workload's shape)."""
    rng = random.Random(4)
    ctx = [rng.randint(256, 1024) for _ in range(256)]
    sc = Scenario([c - 1 for c in ctx], [1] * 256, block_size=16, seed=4)
    check(sc, brute=False)


@pytest.mark.parametrize("block_size", [8, 32])
def test_decode_full_grid_other_block_sizes(block_size):
    """256 sequences at contexts U[1, 1024]: the automatic choice splits each (sequence, head) over
    8 waves, here on the block-size-32 instance and the generic one."""
    rng = random.Random(block_size + 100)
    ctx = [rng.randint(1, 1024) for _ in range(256)]
    sc = Scenario([c - 1 for c in ctx], [1] * 256, block_size=block_size, seed=block_size + 100)
    check(sc, brute=False)


@pytest.mark.parametrize("max_ctx", [128, 129, 256, 257, 512, 513, 1024])
def test_decode_automatic_split_width_boundaries(max_ctx):
    """The automatic grid at 256 sequences: one wave per (sequence, head) up to 128 positions, then
    2, 4 or 8 waves per pair (about 128 positions per wave at the longest context), each width on
    both sides of its boundary, against the reference path."""
    rng = random.Random(max_ctx)
    ctx = [rng.randint(max(1, max_ctx // 2), max_ctx) for _ in range(255)] + [max_ctx]
    sc = Scenario([c - 1 for c in ctx], [1] * 256, block_size=16, seed=max_ctx)
    check(sc, brute=False)


@pytest.mark.parametrize("ctx", [[9000, 5000, 300], [16384, 1, 700], [17000, 40]])
def test_decode_long_contexts_split_or_partition_grid(ctx):
    """Small batches at long contexts: 16 waves per (sequence, head) while the longest context fits
    16 x 1024 positions, the partition grid with its merge launch beyond."""
    sc = Scenario([c - 1 for c in ctx], [1] * len(ctx), block_size=16, seed=len(ctx) + ctx[0])
    check(sc, brute=False)


# ------------------------------------------------------------------------------ prefill
@pytest.mark.parametrize("block_size", [8, 32])
def test_prefill_ragged_batch_other_block_sizes(block_size):
    """20 prompts of 1-300 tokens, some continuing at a cached prefix: a launch with several hundred
    query tiles (key split 2-4) on the block-size-32 instance and the generic one."""
    rng = random.Random(block_size + 200)
    starts = [rng.choice([0, 0, 17, 64, 250]) for _ in range(20)]
    lens = [rng.randint(1, 300) for _ in range(20)]
    sc = Scenario(starts, lens, block_size=block_size, seed=block_size + 200)
    check(sc, brute=False)


@pytest.mark.parametrize("block_size", [4, 16, 32, 48])
@pytest.mark.parametrize("start,n", [(0, 2), (0, 15), (0, 16), (0, 17), (0, 100), (5, 40), (16, 16), (250, 300), (0, 1024)])
def test_prefill_single_sequence(block_size, start, n):
    sc = Scenario([start], [n], block_size=block_size, seed=start * 7 + n)
    check(sc)


def test_prefill_batch_of_ragged_prompts():
    lens = [1, 3, 7, 12, 16, 17, 33, 48]  # the reference's headline batch (tests/test_phase3_paged.py:113)
    sc = Scenario([0] * len(lens), lens, block_size=16, seed=8)
    out, batch = check(sc)
    assert batch.num_decode == 1 and batch.num_prefill == 7


@pytest.mark.parametrize("chunk", [0, 1, 2, 3])
def test_mixed_chunked_prefill_and_decode(chunk):
    """4 prompts of 512-1024 tokens fed in 256-token chunks (chunk k starts at 256k) next to 128
    decoding sequences with contexts ~ U[64, 768]: one mixed step."""
    rng = random.Random(5)
    prompts = [rng.randint(512, 1024) for _ in range(4)]
    dec_ctx = [rng.randint(64, 768) for _ in range(128)]
    starts, lens = [], []
    for p in prompts:
        s = 256 * chunk
        starts.append(s)
        lens.append(max(1, min(256, p - s)))
    starts += [c - 1 for c in dec_ctx]
    lens += [1] * len(dec_ctx)
    sc = Scenario(starts, lens, block_size=16, seed=50 + chunk)
    check(sc, brute=False)


# ------------------------------------------------------------------------------ one launch for mixed steps
def mixed_case(name: str):
    """(starts, new_lens) of a step with prefill rows first, then decode rows."""
    rng = random.Random(hash(name) % 1000)
    if name == "config5-chunk1":  # 768 prefill tiles: 4 waves per tile
        pre = [(256, 256)] * 4
        dec = [rng.randint(64, 768) for _ in range(128)]
    elif name == "tail-chunk":  # 3 short tails at 768: 8 waves per tile
        pre = [(768, 5), (768, 102), (768, 9)]
        dec = [rng.randint(64, 768) for _ in range(128)]
    elif name == "wide-prefill":  # 8 x 600-row prompts: 3,648 tiles, 1 wave per tile
        pre = [(0, 600)] * 8
        dec = [rng.randint(16, 300) for _ in range(16)]
    elif name == "long-decoders":  # contexts past 1024 positions: several partitions and a merge
        pre = [(40, 37), (0, 3)]
        dec = [1500, 2100, 17, 1025, 1, 64]
    else:  # "tiny"
        pre = [(0, 3)]
        dec = [5]
    starts = [s for s, _ in pre] + [c - 1 for c in dec]
    lens = [n for _, n in pre] + [1] * len(dec)
    return starts, lens


def run_mixed_modes(sc: Scenario, partition_tokens: int, hook: bool = False):
    """run_product with the one-launch mixed path off, then on (optionally through the per-kernel
    ctypes path, which a launch hook selects)."""
    from tokquay_amd.kv_cache import PagedBatch

    kinds = []
    res = []
    try:
        for one in (False, True):
            PagedBatch.one_launch_mixed = one
            PagedBatch.launch_hook = (lambda batch, kind: kinds.append(kind)) if hook else None
            res.append(sc.run_product(partition_tokens))
    finally:
        PagedBatch.one_launch_mixed = True
        PagedBatch.launch_hook = None
    return res, kinds


@pytest.mark.parametrize("name", ["config5-chunk1", "tail-chunk", "wide-prefill", "long-decoders", "tiny"])
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("partition_tokens", [64, 1024])
def test_one_launch_mixed_equals_two_launches(name, block_size, partition_tokens):
    """tq_paged_mixed == tq_paged_decode_write + tq_paged_prefill, bit for bit (outputs and pool), at an
    explicit partition length (the decode rows' rounding depends on it)."""
    starts, lens = mixed_case(name)
    sc = Scenario(starts, lens, block_size=block_size, n_layer=2, layer=1, seed=block_size + len(starts))
    (pool_a, out_a, batch), (pool_b, out_b, _) = run_mixed_modes(sc, partition_tokens)[0]
    assert batch.num_decode > 0 and batch.num_prefill > 0
    assert torch.equal(out_a, out_b)
    assert torch.equal(pool_a, pool_b)


@pytest.mark.parametrize("name", ["config5-chunk1", "tail-chunk", "long-decoders", "tiny"])
@pytest.mark.parametrize("block_size", [16, 32])
def test_one_launch_mixed_matches_the_reference(name, block_size):
    """The default path (one launch, partitions chosen for the mixed grid) against the reference's
    gather path and float64 brute force."""
    starts, lens = mixed_case(name)
    sc = Scenario(starts, lens, block_size=block_size, seed=3 + block_size)
    check(sc, brute=name != "config5-chunk1")


def test_one_launch_mixed_through_the_per_kernel_path():
    """The ctypes per-kernel path (taken when a launch hook is set) makes the same single launch."""
    starts, lens = mixed_case("tail-chunk")
    sc = Scenario(starts, lens, block_size=16, seed=9)
    res, kinds = run_mixed_modes(sc, 0, hook=True)
    assert kinds == ["decode", "prefill", "mixed"]
    ref_pool, ref_out, _ = sc.run_product(0)  # the native path, one launch
    assert torch.equal(res[1][1], ref_out) and torch.equal(res[1][0], ref_pool)


def test_mixed_entry_point_with_one_side_empty_and_bad_arguments():
    """No prefill rows: tq_paged_decode_write's launch; no decode rows: tq_paged_prefill's; negative sizes
    and a missing k_new are refused before anything is launched."""
    from tokquay_amd import _lib, ops

    starts, lens = mixed_case("long-decoders")
    sc = Scenario(starts, lens, block_size=16, seed=4)
    pool, out_ref, batch = sc.run_product(0)
    Bp = batch.num_prefill
    qkv = sc.packed_qkv(batch.token_index).cuda()
    C = 768
    Nd = batch.num_decode
    N = batch.num_tokens
    # Packed rows: decode rows first, then the prefill rows.
    dq, dk, dv = qkv[:Nd, :C], qkv[:Nd, C : 2 * C], qkv[:Nd, 2 * C :]
    pq = qkv[Nd:, :C]
    dtab = torch.tensor([sc.tables[b] + [0] * (200 - len(sc.tables[b])) for b in range(Bp, Bp + Nd)], dtype=torch.int32).cuda()
    ptab = torch.tensor([sc.tables[b] + [0] * (200 - len(sc.tables[b])) for b in range(Bp)], dtype=torch.int32).cuda()
    dctx = torch.tensor([sc.ctxs[b] for b in range(Bp, Bp + Nd)], dtype=torch.int32, device="cuda")
    cu = torch.tensor([0] + list(np.cumsum(sc.new_lens[:Bp])), dtype=torch.int32, device="cuda")
    qst = torch.tensor(sc.starts[:Bp], dtype=torch.int32, device="cuda")
    maxc, maxq = int(dctx.max()), max(sc.new_lens[:Bp])

    # Decode rows only (no prefill rows): the same bits as paged_decode with k_new / v_new.
    p1, p2 = sc.pool.cuda(), sc.pool.cuda()
    o1, o2 = torch.empty(Nd, C, device="cuda"), torch.empty(Nd, C, device="cuda")
    ops.paged_decode(o1, dq, p1, sc.layer, dtab, dctx, maxc, k_new=dk, v_new=dv)
    empty_cu = torch.zeros(1, dtype=torch.int32, device="cuda")
    empty_st = torch.zeros(0, dtype=torch.int32, device="cuda")
    ops.paged_mixed(o2, dq, dk, dv, dtab, dctx, maxc, torch.empty(0, C, device="cuda"), torch.empty(0, C, device="cuda"),
                    torch.zeros(0, 200, dtype=torch.int32, device="cuda"), empty_cu, empty_st, 0, p2, sc.layer)  # fmt: skip
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(p1, p2)

    # Both sides through ops.paged_mixed: the same bits as PagedBatch.attend's one launch.
    p3 = sc.pool.cuda()
    slots = []
    for b in range(Bp):
        for t in range(sc.new_lens[b]):
            pos = sc.starts[b] + t
            slots.append(sc.tables[b][pos // 16] * 16 + pos % 16)
    ops.cache_write(p3, sc.layer, qkv[Nd:, C : 2 * C], qkv[Nd:, 2 * C :], torch.tensor(slots, device="cuda"))
    o3d, o3p = torch.empty(Nd, C, device="cuda"), torch.empty(N - Nd, C, device="cuda")
    ops.paged_mixed(o3d, dq, dk, dv, dtab, dctx, maxc, o3p, pq, ptab, cu, qst, maxq, p3, sc.layer)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([o3d, o3p]).cpu(), out_ref) and torch.equal(p3.cpu(), pool)

    # Argument errors come back as status codes and launch nothing.
    L = _lib.lib()
    bad = [0] * 40
    bad[13] = -1  # num_decode_seqs
    assert L.tq_paged_mixed(*bad) == 1
    assert L.tq_paged_mixed_workspace_size(4, 12, 64, 3000, 0, 0, 0, 0) == L.tq_paged_decode_workspace_size(4, 12, 64, 3000, 0)
    with pytest.raises(ValueError):
        ops.paged_mixed(o3d, dq, dk, dv, dtab, dctx, maxc, o3p, pq, ptab, cu[:-1], qst, maxq, p3, sc.layer)


# ------------------------------------------------------------------------------ the reference view's gather
@pytest.mark.parametrize("block_size", [1, 8, 16, 32])
def test_gather_equals_the_reference_gather(block_size):
    """PagedBatch.gather (the HIP gather kernel) == the reference's PagedBatch.gather bit for bit on a
    garbage pool with shuffled tables, after the step's write; padded table entries read block 0 as
    the reference's do (tokquay/kv_cache.py:195-200, :234-242)."""
    from oracle.paged_ref import RefPagedBatch
    from tokquay_amd.kv_cache import PagedBatch

    starts = [0, 37, 100, 5, 250, 0]
    lens = [23, 1, 1, 40, 3, 1]
    sc = Scenario(starts, lens, block_size=block_size, n_layer=2, layer=1, seed=30 + block_size)
    ref_pool = sc.pool.clone()
    ref = RefPagedBatch(ref_pool, block_size, sc.tables, sc.starts, sc.new_lens)
    ref.write(sc.layer, sc.k, sc.v)
    rk, rv = ref.gather(sc.layer)

    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pool = sc.pool.cuda()
    tables = [list(t) for t in sc.tables]
    batch = PagedBatch(pool, block_size, tables, sc.starts, sc.new_lens, error_word=err)
    batch.write(sc.layer, sc.k.cuda(), sc.v.cuda())
    for t in tables:  # the caller reuses its lists after the view is made: the view keeps its copy
        t.reverse()
        t.append(0)
    k, v = batch.gather(sc.layer)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert k.shape == rk.shape and v.shape == rv.shape
    assert torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)
    assert torch.equal(pool.cpu(), ref_pool)


def test_the_reference_attention_branch_runs_on_the_product_batch_view():
    """The reference's paged branch of Attention.forward unchanged - write, gather, masked softmax
    (tokquay/model.py:73-78, :94-96) - on tokquay_amd.PagedBatch (write and gather on the HIP kernels,
    the softmax in torch on the CPU) equals PagedBatch.attend at fp32 tolerance."""
    from oracle.paged_ref import ref_attention
    from tokquay_amd.kv_cache import PagedBatch

    starts, lens = mixed_case("tiny")
    starts, lens = starts + [0, 60], lens + [17, 1]
    sc = Scenario(starts, lens, block_size=16, seed=41)
    pool = sc.pool.cuda()
    batch = PagedBatch(pool, 16, sc.tables, sc.starts, sc.new_lens)
    batch.write(sc.layer, sc.k.cuda(), sc.v.cuda())
    k, v = batch.gather(sc.layer)
    got = ref_attention(sc.q, k.cpu(), v.cpu(), batch.mask.cpu())  # [B, H, T, d]
    _, out_gpu, b2 = sc.run_product()
    want = sc.packed_reference(got, b2.token_index)
    torch.testing.assert_close(out_gpu, want, rtol=RTOL, atol=ATOL)


def test_gather_reports_a_bad_block_id_and_zeroes_its_keys():
    from tokquay_amd import _lib, ops

    pool = torch.randn(4, 1, 2, 12, 16, 64, device="cuda")
    tables = torch.tensor([[0, 3], [2, 9]], dtype=torch.int32, device="cuda")  # 9 is outside the pool
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    k, v = ops.paged_gather(pool, 0, tables, err)
    torch.cuda.synchronize()
    assert int(err.item()) & _lib.DEVERR_BLOCK_ID
    assert torch.equal(k[0, :, 16:], pool[3, 0, 0]) and torch.equal(v[1, :, :16], pool[2, 0, 1])
    assert not k[1, :, 16:].any() and not v[1, :, 16:].any()


# ------------------------------------------------------------------------------ contract edges
def test_write_contract_padded_layout_is_bit_exact_and_padding_never_writes():
    """BatchedKV.write with the reference's [B, H, T, d] layout: padded positions write nothing and
    blocks nobody owns stay bit-identical (tests/test_phase3_paged.py:125-129)."""
    from oracle.paged_ref import RefPagedBatch
    from tokquay_amd.kv_cache import PagedBatch

    sc = Scenario([0, 3, 20, 0], [5, 1, 9, 13], block_size=4, num_blocks=40, seed=21)
    pool_ref = sc.pool.clone()
    RefPagedBatch(pool_ref, 4, sc.tables, sc.starts, sc.new_lens).write(0, sc.k, sc.v)
    pool = sc.pool.cuda()
    PagedBatch(pool, 4, sc.tables, sc.starts, sc.new_lens).write(0, sc.k.cuda(), sc.v.cuda())
    assert torch.equal(pool.cpu(), pool_ref)
    owned = {b for t in sc.tables for b in t}
    untouched = [b for b in range(sc.num_blocks) if b not in owned]
    assert untouched and torch.equal(pool.cpu()[untouched], sc.pool[untouched])


def test_out_of_range_block_id_is_reported_not_followed():
    """A block id past the pool is caught by the kernels' bounds check and reported."""
    from tokquay_amd import ops

    pool = torch.zeros(8, 1, 2, 12, 16, 64, device="cuda")
    q = torch.randn(2, 12, 64, device="cuda")
    out = torch.empty_like(q)
    tables = torch.tensor([[0, 1], [2, 8 + 5]], dtype=torch.int32, device="cuda")
    ctx = torch.tensor([20, 20], dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.paged_decode(out, q, pool, 0, tables, ctx, 20, d_error=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert torch.isfinite(out).all()


def test_write_variant_skips_an_out_of_range_block_id():
    """The new position's block id is past the pool: the row is reported and nothing is written."""
    from tokquay_amd import ops

    pool = torch.zeros(8, 1, 2, 12, 16, 64, device="cuda")
    qkv = torch.randn(2, 3 * 768, device="cuda")
    out = torch.empty(2, 768, device="cuda")
    tables = torch.tensor([[0, 1], [2, 8 + 5]], dtype=torch.int32, device="cuda")
    ctx = torch.tensor([20, 20], dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.paged_decode(out, qkv[:, :768], pool, 0, tables, ctx, 20, d_error=err, k_new=qkv[:, 768:1536],
                     v_new=qkv[:, 1536:])  # fmt: skip
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    want = torch.zeros_like(pool)
    want[1, 0, 0, :, 3] = qkv[0, 768:1536].view(12, 64)  # row 0: position 19 = block 1, offset 3
    want[1, 0, 1, :, 3] = qkv[0, 1536:].view(12, 64)
    assert torch.equal(pool, want)
    assert torch.isfinite(out[0]).all()


def test_host_side_argument_errors_raise():
    from tokquay_amd import _lib, ops

    pool = torch.zeros(4, 1, 2, 12, 16, 64, device="cuda")
    q = torch.randn(1, 12, 64, device="cuda")
    tables = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    ctx = torch.tensor([1000], dtype=torch.int32, device="cuda")
    tiny = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.KernelError, match="workspace"):
        ops.paged_decode(torch.empty_like(q), q, pool, 0, tables, ctx, 1000, partition_tokens=16, workspace=tiny)
    with pytest.raises(ValueError):
        ops.paged_decode(torch.empty_like(q), q, pool, 1, tables, ctx, 1000)  # layer out of range


def test_launch_recorded_timing_events():
    """tq_set_timing_events: the decode launch records both events around its own kernels."""
    from tokquay_amd import _lib, ops

    pool = torch.randn(64, 1, 2, 12, 16, 64, device="cuda")
    q = torch.randn(8, 12, 64, device="cuda")
    tables = torch.arange(64, dtype=torch.int32, device="cuda").view(8, 8)
    ctx = torch.full((8,), 128, dtype=torch.int32, device="cuda")
    want = torch.empty_like(q)
    ops.paged_decode(want, q, pool, 0, tables, ctx, 128)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    stop.record()
    assert _lib.lib().tq_set_timing_events(start.cuda_event, stop.cuda_event) == 0
    got = torch.empty_like(q)
    ops.paged_decode(got, q, pool, 0, tables, ctx, 128)
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) > 0
    assert torch.equal(got, want)


@pytest.mark.parametrize("block_size", [8, 16])
@pytest.mark.parametrize("num_seqs", [24, 8, 4, 1])
def test_prefill_key_split_widths(block_size, num_seqs):
    """The prefill launch splits each query tile's keys over 1, 2, 4 or 8 waves depending on how many
    tiles there are (4608 / 1536 / 768 / 192 query tiles -> 1 / 2 / 4 / 8 waves), for the
    block-size-16 path (one block per key tile; software-pipelined at every width; the one-wave
    launch takes two query tiles per wave) and the generic one; every width must match the
    reference, with ragged lengths and chunk starts."""
    rng = random.Random(num_seqs)
    lens = [256] + [rng.randint(100, 256) for _ in range(num_seqs - 1)]
    starts = [rng.choice([0, 0, 100, 300]) for _ in range(num_seqs)]
    sc = Scenario(starts, lens, block_size=block_size, seed=90 + num_seqs)
    check(sc, brute=num_seqs <= 6)


def test_prefill_two_query_tiles_per_wave_edges():
    """A launch of more than 1536 query tiles and at least 8192 row tiles at block size 16 gives each
    wave two consecutive query tiles: lengths that leave the second tile partly or wholly empty,
    starts inside a block."""
    rng = random.Random(77)
    base = [2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 64, 65]
    lens = [base[i % len(base)] for i in range(320)]  # 11,087 rows: 12 x 693 = 8,316 row tiles
    starts = [rng.choice([0, 5, 16, 100]) for _ in lens]
    sc = Scenario(starts, lens, block_size=16, seed=77)
    check(sc, brute=False)


@pytest.mark.parametrize("shape", ["key_split", "two_tiles"])
@pytest.mark.parametrize("scores", ["wide", "all_negative"])
def test_prefill_running_maximum_over_wide_score_ranges(shape, scores):
    """The lazy running maximum under score ranges that move it often: q scaled so that scores spread
    over tens of log2 units (the maximum grows on many key tiles, the per-lane test firing for some
    lanes of a wave only), and every score of every query far below zero (keys share a direction q
    points against: the first visible key sets the maximum, no probability underflows). Both the
    key-split launch (4 prompts) and the two-query-tiles-per-wave launch (8,316 row tiles), against
    the reference."""
    rng = random.Random(31)
    if shape == "key_split":
        lens = [256, 200, 131, 77]
        starts = [0, 100, 16, 300]
    else:
        base = [2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 64, 65]
        lens = [base[i % len(base)] for i in range(320)]
        starts = [rng.choice([0, 5, 16, 100]) for _ in lens]
    sc = Scenario(starts, lens, block_size=16, seed=41)
    if scores == "wide":
        sc.q *= 8.0
    else:
        u = torch.randn(64, generator=torch.Generator().manual_seed(42))
        u = u / u.norm()
        for tbl, s in zip(sc.tables, sc.starts):  # the cached keys: + 6 u
            for p in range(s):
                sc.pool[tbl[p // 16], 0, 0, :, p % 16] += 6.0 * u
        sc.k += 6.0 * u
        sc.q = sc.q * 0.1 - 50.0 * u  # scores about -300 / 8 = -37.5 natural units, all negative
    check(sc, brute=shape == "key_split")


@pytest.mark.parametrize("num_seqs,max_len", [(80, 400), (40, 300), (4, 256)])
def test_prefill_dispatch_order_does_not_change_results(num_seqs, max_len):
    """seq_order only changes how a launch deals its sequences: identical bits for no order, the
    most-work-first order the batch view passes and a random permutation. One-wave launches (two
    query tiles per wave at 80 sequences, one at 40) report an entry out of range (TQ_DEVERR_ORDER)
    and skip that sequence; a key-split launch (4 sequences) ignores the order."""
    from tokquay_amd import _lib, ops

    rng = random.Random(num_seqs)
    lens = [rng.randint(16, max_len) for _ in range(num_seqs)]
    starts = [rng.choice([0, 0, 7, 100]) for _ in range(num_seqs)]
    ctx = [s + n for s, n in zip(starts, lens)]
    nb = sum(cdiv(c, 16) for c in ctx) + 4
    pool = torch.randn(nb, 1, 2, 12, 16, 64, generator=torch.Generator().manual_seed(num_seqs)).cuda()
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(num_seqs + 1)).tolist()
    width = max(cdiv(c, 16) for c in ctx)
    tables = torch.zeros(num_seqs, width, dtype=torch.int32)
    i = 0
    for b, c in enumerate(ctx):
        tables[b, : cdiv(c, 16)] = torch.tensor(perm[i : i + cdiv(c, 16)], dtype=torch.int32)
        i += cdiv(c, 16)
    tables = tables.cuda()
    cu_l = [0]
    for n in lens:
        cu_l.append(cu_l[-1] + n)
    cu = torch.tensor(cu_l, dtype=torch.int32, device="cuda")
    st = torch.tensor(starts, dtype=torch.int32, device="cuda")
    q = torch.randn(cu_l[-1], 768, generator=torch.Generator().manual_seed(num_seqs + 2)).cuda()
    work = [n * (2 * s + n + 1) for s, n in zip(starts, lens)]
    outs = []
    for order in (None, sorted(range(num_seqs), key=lambda b: -work[b]), torch.randperm(num_seqs).tolist()):
        out = torch.empty_like(q)
        so = None if order is None else torch.tensor(order, dtype=torch.int32, device="cuda")
        ops.paged_prefill(out, q, pool, 0, tables, cu, st, max(lens), seq_order=so)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    bad = torch.arange(num_seqs, dtype=torch.int32, device="cuda")
    bad[2] = num_seqs + 5
    out = torch.zeros_like(q)
    ops.paged_prefill(out, q, pool, 0, tables, cu, st, max(lens), d_error=err, seq_order=bad)
    torch.cuda.synchronize()
    rows_of_2 = list(range(cu_l[2], cu_l[3]))
    keep = [r for r in range(cu_l[-1]) if r not in set(rows_of_2)]
    assert torch.equal(out[keep], outs[0][keep])
    if num_seqs > 4:
        assert int(err.item()) == _lib.DEVERR_ORDER
    else:
        assert int(err.item()) == 0 and torch.equal(out, outs[0])


@pytest.mark.parametrize("block_size", [2, 3, 5, 64, 128, 1024])
@pytest.mark.parametrize("kind", ["decode", "prefill", "mixed"])
def test_unusual_block_sizes(block_size, kind):
    """Block sizes the reference accepts beyond the usual powers of two up to 32: odd sizes (a
    16-position chunk then spans blocks at uneven offsets) and large ones up to the 1024 maximum
    (every sequence in one block); each must match the reference path and float64 brute force."""
    rng = random.Random(2000 + block_size)
    if kind == "decode":
        ctx = [rng.randint(1, 600) for _ in range(12)] + [block_size, block_size + 1]
        starts, lens = [c - 1 for c in ctx], [1] * len(ctx)
    elif kind == "prefill":
        starts, lens = [0, 37, block_size - 1, 5], [50, 17, 100, rng.randint(2, 40)]
    else:
        starts = [0, block_size + 3] + [rng.randint(0, 500) for _ in range(8)]
        lens = [40, 21] + [1] * 8
    sc = Scenario(starts, lens, block_size=block_size, seed=block_size)
    check(sc)
    if kind == "decode":
        check(sc, partition_tokens=64)


@pytest.mark.parametrize("n_head", [1, 3, 16, 20, 25])
@pytest.mark.parametrize("kind", ["decode", "prefill", "mixed"])
def test_other_head_counts(n_head, kind):
    """Head counts other than GPT-2 small's 12: GPT-2 medium / large / xl have 16 / 20 / 25 heads of
    64, and 1 and 3 are small odd counts. The prefill grid deals (sequence, head) groups to the 8
    XCDs, the decode split width depends on sequences x heads, and the mixed launch interleaves
    both kinds of workgroup; each must match the reference path and float64 brute force."""
    rng = random.Random(1000 + n_head)
    if kind == "decode":
        ctx = [rng.randint(1, 700) for _ in range(20)]
        starts, lens = [c - 1 for c in ctx], [1] * len(ctx)
    elif kind == "prefill":
        starts, lens = [0, 37, 300, 16], [50, 17, 200, rng.randint(2, 40)]
    else:
        starts = [0, 130] + [rng.randint(0, 600) for _ in range(12)]
        lens = [70, 33] + [1] * 12
    sc = Scenario(starts, lens, block_size=16, seed=n_head, n_head=n_head)
    _, batch = check(sc)
    if kind == "mixed":
        assert batch.num_decode > 0 and batch.num_prefill > 0
    if kind == "decode":
        check(sc, partition_tokens=64)  # the partition grid and its merge kernel


@pytest.mark.parametrize("block_size", [8, 16])
@pytest.mark.parametrize("num_seqs", [1, 3, 40])
def test_prefill_bad_block_id_is_reported_and_contained(block_size, num_seqs):
    """A block-table entry outside the pool is reported (TQ_DEVERR_BLOCK_ID); the kernel takes zeros for
    that block's keys and values, so the bad sequence's rows stay finite and every other sequence's rows
    are bit-identical to a launch with a valid table (1 / 3 / 40 sequences: 8 / 4 / 1 waves per query
    tile)."""
    from tokquay_amd import _lib, ops

    rng = random.Random(70 + num_seqs)
    lens = [rng.randint(20, 200) for _ in range(num_seqs)]
    starts = [rng.choice([0, 16, 300]) for _ in range(num_seqs)]
    need = [cdiv(s + n, block_size) for s, n in zip(starts, lens)]
    nb = sum(need) + 2
    pool = torch.randn(nb, 2, 2, 12, block_size, 64, generator=torch.Generator().manual_seed(71)).cuda()
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(72)).tolist()
    tables = torch.zeros(num_seqs, max(need), dtype=torch.int32)
    i = 0
    for b, k in enumerate(need):
        tables[b, :k] = torch.tensor(perm[i : i + k], dtype=torch.int32)
        i += k
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32, device="cuda")
    st = torch.tensor(starts, dtype=torch.int32, device="cuda")
    q = torch.randn(sum(lens), 768, generator=torch.Generator().manual_seed(73)).cuda()
    good = torch.empty_like(q)
    ops.paged_prefill(good, q, pool, 1, tables.cuda(), cu, st, max(lens))
    bad_seq = min(1, num_seqs - 1)
    bad_tables = tables.clone()
    bad_tables[bad_seq, need[bad_seq] // 2] = nb + 1000
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = torch.full_like(q, float("nan"))
    ops.paged_prefill(got, q, pool, 1, bad_tables.cuda(), cu, st, max(lens), d_error=err)
    torch.cuda.synchronize()
    assert int(err.item()) == _lib.DEVERR_BLOCK_ID
    rows = torch.arange(sum(lens))
    mine = (rows >= int(cu[bad_seq])) & (rows < int(cu[bad_seq + 1]))
    assert torch.equal(got[~mine.cuda()], good[~mine.cuda()])
    assert bool(torch.isfinite(got[mine.cuda()]).all())
