"""Seeded random batches through the whole attention path against the reference gather path.

Each seed draws one batch view: 1-32 sequences, each a decode row (one new token after a cached
context), a prompt (no cached context) or a chunk (new tokens after a cached context), with a
block size, head count, layer and decode partition length drawn too. The batch runs through
PagedBatch.attend (cache write, decode, prefill and the one-launch mixed kernel, whichever the
batch needs) and must match the reference's scatter + gather + masked softmax: the pool bit for
bit, the outputs within the fp32 tolerance, and float64 brute force on the smaller draws. The
seeds are fixed, so every run checks the same batches.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from tests.paged_cases import ATOL, RTOL, Scenario

pytestmark = pytest.mark.gpu

BLOCK_SIZES = [1, 2, 3, 4, 5, 8, 16, 16, 16, 16, 32, 64]
HEADS = [1, 3, 12, 12, 12, 25]
PARTITIONS = [0, 0, 0, 64, 256]


def draw(seed: int) -> tuple[dict, list[int], list[int]]:
    rng = random.Random(seed)
    n = rng.randint(1, 32)
    starts, lens = [], []
    for _ in range(n):
        kind = rng.choice(["decode", "decode", "prompt", "chunk"])
        if kind == "decode":
            starts.append(rng.randint(1, 1200))
            lens.append(1)
        elif kind == "prompt":
            starts.append(0)
            lens.append(rng.randint(1, 300))
        else:
            starts.append(rng.randint(1, 900))
            lens.append(rng.randint(2, 300))
    n_layer = rng.choice([1, 3])
    shape = dict(block_size=rng.choice(BLOCK_SIZES), n_head=rng.choice(HEADS), n_layer=n_layer,
                 layer=rng.randrange(n_layer), partition_tokens=rng.choice(PARTITIONS))
    return shape, starts, lens


@pytest.mark.parametrize("seed", range(100))
def test_random_batch_matches_the_reference(seed):
    shape, starts, lens = draw(seed)
    print(f"seed {seed}: {shape}, {len(starts)} sequences, starts {starts}, new lengths {lens}", flush=True)
    sc = Scenario(starts, lens, block_size=shape["block_size"], n_layer=shape["n_layer"], layer=shape["layer"],
                  seed=1000 + seed, n_head=shape["n_head"])
    pool_ref, out_ref = sc.reference()
    pool_gpu, out_gpu, batch = sc.run_product(shape["partition_tokens"])
    assert torch.equal(pool_gpu, pool_ref), "pool differs from the reference scatter"
    torch.testing.assert_close(out_gpu, sc.packed_reference(out_ref, batch.token_index), rtol=RTOL, atol=ATOL)
    if sum(lens) * shape["n_head"] <= 6000:
        exact = sc.brute_force(pool_ref)
        T = sc.q.shape[2]
        got = out_gpu.view(-1, sc.H, 64).double().numpy()
        for r, flat in enumerate(batch.token_index.cpu().tolist()):
            b, t = divmod(flat, T)
            np.testing.assert_allclose(got[r], exact[b][t], rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("seed", range(40))
def test_random_mixed_step_one_launch_equals_two_launches(seed):
    """Random batch views that hold both decode rows and multi-token rows, at an explicit decode
    partition length: the one-launch mixed kernel gives the two single-kind launches' bits (outputs
    and pool)."""
    from tokquay_amd.kv_cache import PagedBatch

    rng = random.Random(5000 + seed)
    shape, starts, lens = draw(5000 + seed)
    starts.append(rng.randint(1, 900))  # at least one decode row and one chunk
    lens.append(1)
    starts.append(rng.randint(0, 400))
    lens.append(rng.randint(2, 200))
    part = rng.choice([64, 256, 1024])
    print(f"seed {seed}: {shape}, partition {part}, starts {starts}, new lengths {lens}", flush=True)
    sc = Scenario(starts, lens, block_size=shape["block_size"], n_layer=shape["n_layer"], layer=shape["layer"],
                  seed=7000 + seed, n_head=shape["n_head"])
    res = []
    try:
        for one in (False, True):
            PagedBatch.one_launch_mixed = one
            res.append(sc.run_product(part))
    finally:
        PagedBatch.one_launch_mixed = True
    (pool_a, out_a, batch), (pool_b, out_b, _) = res
    assert batch.num_decode > 0 and batch.num_prefill > 0
    assert torch.equal(out_a, out_b)
    assert torch.equal(pool_a, pool_b)


@pytest.mark.parametrize("seed", range(30))
def test_random_decode_write_equals_cache_write_then_decode(seed):
    """Random decode batches (1-64 rows, contexts 0-1,500 where 0 is a padding row, block sizes 1-64,
    1-25 heads, automatic or explicit partitions): tq_paged_decode_write gives the bits of
    tq_cache_write followed by tq_paged_decode, output and pool."""
    from tokquay_amd import ops

    rng = random.Random(9000 + seed)
    bs = rng.choice(BLOCK_SIZES)
    heads = rng.choice(HEADS)
    part = rng.choice([0, 0, 16, 64, 256, 1024])
    ctx = [rng.choice([0, rng.randint(1, 1500), rng.randint(1, 64)]) for _ in range(rng.randint(1, 64))]
    ctx[0] = max(ctx[0], 1)
    print(f"seed {seed}: block {bs}, heads {heads}, partition {part}, contexts {ctx}", flush=True)
    n_layer, layer = 2, rng.randrange(2)
    cdiv = lambda a, b: -(-a // b)  # noqa: E731
    nb = sum(cdiv(c, bs) for c in ctx) + 2
    C = heads * 64
    pool0 = torch.randn(nb, n_layer, 2, heads, bs, 64, generator=torch.Generator().manual_seed(seed)) * 50
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed + 1)).tolist()
    maxc = max(ctx)
    width = cdiv(maxc, bs)
    tables = torch.zeros(len(ctx), width, dtype=torch.int32)
    slots, i = [], 0
    for b, c in enumerate(ctx):
        n = cdiv(c, bs)
        tables[b, :n] = torch.tensor(perm[i : i + n], dtype=torch.int32)
        i += n
        slots.append(int(tables[b, (c - 1) // bs]) * bs + (c - 1) % bs if c else -1)
    qkv = torch.randn(len(ctx), 3 * C, generator=torch.Generator().manual_seed(seed + 2)).cuda()
    q, k, v = qkv[:, :C], qkv[:, C : 2 * C], qkv[:, 2 * C :]
    tables, cl = tables.cuda(), torch.tensor(ctx, dtype=torch.int32, device="cuda")
    sm = torch.tensor(slots, dtype=torch.int64, device="cuda")
    pa, pb = pool0.cuda(), pool0.cuda()
    oa, ob = torch.empty(len(ctx), C, device="cuda"), torch.empty(len(ctx), C, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.cache_write(pa, layer, k, v, sm, err)
    ops.paged_decode(oa, q, pa, layer, tables, cl, maxc, partition_tokens=part, d_error=err)
    ops.paged_decode(ob, q, pb, layer, tables, cl, maxc, partition_tokens=part, d_error=err, k_new=k, v_new=v)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.equal(oa, ob)
    assert torch.equal(pa, pb)


@pytest.mark.parametrize("seed", range(20))
def test_random_prefill_dispatch_order_keeps_the_bits(seed):
    """Random prompt and chunk batches large enough for one-wave launches (one or two query tiles per
    wave, block size 16): the natural order, most causal work first and a random permutation give
    the same bits."""
    from tokquay_amd import ops

    rng = random.Random(11000 + seed)
    n = rng.randint(40, 160)
    lens = [rng.randint(1, rng.choice([64, 300, 700])) for _ in range(n)]
    starts = [rng.choice([0, 0, rng.randint(1, 300)]) for _ in range(n)]
    print(f"seed {seed}: {n} sequences, {sum(lens)} rows", flush=True)
    cdiv = lambda a, b: -(-a // b)  # noqa: E731
    ctx = [s + m for s, m in zip(starts, lens)]
    nb = sum(cdiv(c, 16) for c in ctx) + 4
    pool = torch.randn(nb, 1, 2, 12, 16, 64, generator=torch.Generator().manual_seed(seed)).cuda()
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed + 1)).tolist()
    tables = torch.zeros(n, max(cdiv(c, 16) for c in ctx), dtype=torch.int32)
    i = 0
    for b, c in enumerate(ctx):
        tables[b, : cdiv(c, 16)] = torch.tensor(perm[i : i + cdiv(c, 16)], dtype=torch.int32)
        i += cdiv(c, 16)
    cu_l = [0]
    for m in lens:
        cu_l.append(cu_l[-1] + m)
    tables = tables.cuda()
    cu = torch.tensor(cu_l, dtype=torch.int32, device="cuda")
    st = torch.tensor(starts, dtype=torch.int32, device="cuda")
    q = torch.randn(cu_l[-1], 768, generator=torch.Generator().manual_seed(seed + 2)).cuda()
    work = [m * (2 * s + m + 1) for s, m in zip(starts, lens)]
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    outs = []
    for order in (None, sorted(range(n), key=lambda b: -work[b]), rng.sample(range(n), n)):
        out = torch.empty_like(q)
        so = None if order is None else torch.tensor(order, dtype=torch.int32, device="cuda")
        ops.paged_prefill(out, q, pool, 0, tables, cu, st, max(lens), d_error=err, seq_order=so)
        outs.append(out)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
