"""tq_paged_decode_write_static (no allocation, static per-GPU scratch) gives the same bits as
tq_paged_decode_write with a caller-allocated workspace, on two calls in a row (the second smaller,
so the scratch holds the first call's partials when it starts), and refuses a call whose partials
would not fit the static array before launching anything.

Both entry points are called through the C ABI (ctypes). Explicit partition sizes make the
sequences span several partitions, so the partials (and the merge kernel) are used.
"""

from __future__ import annotations

import ctypes
import math
import random

import pytest
import torch

from oracle.paged_ref import cdiv
from tests.paged_cases import ATOL, RTOL
from tokquay_amd import _lib

pytestmark = pytest.mark.gpu

H, D, C = 12, 64, 768


def _case(num_seqs: int, ctx_lo: int, ctx_hi: int, block_size: int, seed: int):
    rng = random.Random(seed)
    ctx = [rng.randint(ctx_lo, ctx_hi) for _ in range(num_seqs)]
    ctx[0] = 0  # a padding row: writes nothing, zero output
    nb = sum(cdiv(c, block_size) for c in ctx) + 3
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(nb, 2, 2, H, block_size, D, generator=g) * 50
    perm = torch.randperm(nb, generator=g).tolist()
    width = cdiv(max(ctx), block_size)
    tables = torch.zeros(num_seqs, width, dtype=torch.int32)
    i = 0
    for b, c in enumerate(ctx):
        n = cdiv(c, block_size)
        tables[b, :n] = torch.tensor(perm[i : i + n], dtype=torch.int32)
        i += n
    # Blocks that hold context positions get N(0, 1) keys and values (well-conditioned softmax);
    # blocks nobody owns keep the x50 garbage, so a stray read shows.
    owned = torch.tensor(perm[:i], dtype=torch.long)
    pool[owned] = torch.randn(i, 2, 2, H, block_size, D, generator=g)
    qkv = torch.randn(num_seqs, 3 * C, generator=g)
    return ctx, pool, tables, qkv


def _call(fn_name: str, out, qkv, pool, layer, tables, lens, order, max_ctx, part, err, ws=None):
    L = _lib.lib()
    n = lens.numel()
    nb, n_layer, _, _, bs, _ = pool.shape
    qp = qkv.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    common = (out.data_ptr(), C, qp, 3 * C, qp + 4 * C, 3 * C, qp + 8 * C, 3 * C, pool.data_ptr(), nb, n_layer, H, bs,
              D, layer, tables.data_ptr(), tables.size(1), tables.size(1), lens.data_ptr(), order.data_ptr(), n,
              max_ctx, 1.0 / math.sqrt(D), part)  # fmt: skip
    if fn_name == "tq_paged_decode_write":
        return L.tq_paged_decode_write(*common, ws.data_ptr() if ws is not None else None,
                                       ws.numel() if ws is not None else 0, err.data_ptr(), stream)  # fmt: skip
    return L.tq_paged_decode_write_static(*common, err.data_ptr(), stream)


@pytest.mark.parametrize("block_size", [16, 4])
def test_static_entry_matches_the_workspace_entry(block_size):
    L = _lib.lib()
    cases = [(48, 100, 1024, 64, 11), (20, 16, 600, 128, 12)]  # (seqs, ctx lo, hi, partition, seed): smaller second
    for num_seqs, lo, hi, part, seed in cases:
        ctx, pool0, tables, qkv = _case(num_seqs, lo, hi, block_size, seed)
        max_ctx = max(ctx)
        need = L.tq_paged_decode_workspace_size(num_seqs, H, D, max_ctx, part)
        assert 0 < need <= _lib.STATIC_SCRATCH_BYTES, need  # the partials are really used
        lens = torch.tensor(ctx, dtype=torch.int32, device="cuda")
        order = torch.tensor(sorted(range(num_seqs), key=lambda b: -ctx[b]), dtype=torch.int32, device="cuda")
        tables_d, qkv_d = tables.cuda(), qkv.cuda()
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        pa, pb = pool0.cuda(), pool0.cuda()
        oa = torch.full((num_seqs, C), float("nan"), device="cuda")
        ob = torch.full((num_seqs, C), float("nan"), device="cuda")
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        assert _call("tq_paged_decode_write", oa, qkv_d, pa, 1, tables_d, lens, order, max_ctx, part, err, ws) == 0
        assert _call("tq_paged_decode_write_static", ob, qkv_d, pb, 1, tables_d, lens, order, max_ctx, part, err) == 0
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        assert torch.equal(oa, ob), (num_seqs, float((oa - ob).abs().max()))
        assert torch.equal(pa, pb)
        assert not torch.equal(pb.cpu(), pool0)  # the new rows did land
        # And against float64 attention over each sequence's positions (the pool after the write).
        pool_after = pb.cpu().double()
        for b in (0, 1, num_seqs - 1):
            c = ctx[b]
            if c == 0:
                assert torch.equal(ob[b].cpu(), torch.zeros(C))
                continue
            blk = tables[b, [p // block_size for p in range(c)]].long()
            off = torch.tensor([p % block_size for p in range(c)])
            k = pool_after[blk, 1, 0, :, off]  # [c, H, D]
            v = pool_after[blk, 1, 1, :, off]
            q = qkv[b, :C].double().view(H, D)
            w = torch.softmax(torch.einsum("hd,chd->hc", q, k) / math.sqrt(D), dim=-1)
            want = torch.einsum("hc,chd->hd", w, v).reshape(C).float()
            torch.testing.assert_close(ob[b].cpu(), want, rtol=RTOL, atol=ATOL)


def test_static_entry_refuses_partials_beyond_the_array_before_launching():
    L = _lib.lib()
    n, max_ctx, part = 256, 1024, 16
    need = L.tq_paged_decode_workspace_size(n, H, D, max_ctx, part)
    assert need > _lib.STATIC_SCRATCH_BYTES
    # Every pointer is valid-looking but nothing may be touched: the size check comes first.
    dummy = torch.zeros(16, device="cuda")
    p = dummy.data_ptr()
    st = L.tq_paged_decode_write_static(p, C, p, 3 * C, p, 3 * C, p, 3 * C, p, 1, 1, H, 16, D, 0, p, 64, 64, p,
                                        None, n, max_ctx, 0.125, part, None,
                                        torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert st == 3  # TQ_ERR_WORKSPACE
    assert torch.equal(dummy, torch.zeros(16, device="cuda"))
    # No sequences: nothing to do, no scratch needed.
    assert L.tq_paged_decode_write_static(None, C, None, 3 * C, None, 3 * C, None, 3 * C, None, 1, 1, H, 16, D, 0,
                                          None, 0, 0, None, None, 0, 0, 0.125, 0, None, None) == 0  # fmt: skip


def test_ctypes_signature_matches():
    fn = _lib.lib().tq_paged_decode_write_static
    assert fn.restype is ctypes.c_int and len(fn.argtypes) == 26
