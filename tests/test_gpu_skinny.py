"""Small-batch linear layers (``tq_skinny_linear``) and row embeddings (``tq_embed_rows``) on the GPU.

* Against torch on the CPU in fp32: ``F.linear`` with ``F.layer_norm`` in front and the GELU (tanh
  form) or residual add after (tokquay/model.py:62-63, :103-107, :117-123, :180), at GPT-2's shapes
  including the ragged LM head (50257 columns), 1 to 64 rows, strided rows.
* The graph-replayed decode step through the fused path against the same step through the library
  GEMMs: logits within fp32 tolerance and identical greedy ids, across buckets 1 to 64.
"""

from __future__ import annotations

import random

import pytest
import torch
import torch.nn.functional as F

from tokquay_amd import _lib, ops
from tokquay_amd.generate import paged_forward
from tokquay_amd.graphs import DecodeGraphs
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.sequence import Sequence
from tokquay_amd.weights import random_state_dict

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=2e-5)


def weights(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(N, K, generator=g) * 0.02, torch.randn(N, generator=g) * 0.1


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32, 40, 64])
@pytest.mark.parametrize("N,K", [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768), (40, 768)])
def test_plain_and_layernorm_prologue(M, N, K):
    g = torch.Generator().manual_seed(M * 1000 + N + K)
    x = torch.randn(M, K, generator=g) * 2 + 0.5
    w, b = weights(N, K, N + K)
    gamma, beta = torch.randn(K, generator=g), torch.randn(K, generator=g)
    got = ops.skinny_linear(x.cuda(), w.cuda(), b.cuda())
    torch.testing.assert_close(got.cpu(), F.linear(x, w, b), **TOL)
    if K == 3072:  # the LayerNorm is fused only where K is one workgroup's (GPT-2 never needs it here)
        with pytest.raises(_lib.KernelError):
            ops.skinny_linear(x.cuda(), w.cuda(), None, ln=(gamma.cuda(), beta.cuda(), 1e-5))
        return
    got = ops.skinny_linear(x.cuda(), w.cuda(), None, ln=(gamma.cuda(), beta.cuda(), 1e-5))
    torch.testing.assert_close(got.cpu(), F.linear(F.layer_norm(x, (K,), gamma, beta, 1e-5), w), **TOL)


@pytest.mark.parametrize("M", [1, 7, 16, 30, 47, 64])
def test_gelu_and_residual_epilogues(M):
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, 768, generator=g)
    w, b = weights(3072, 768, 1)
    gamma, beta = torch.randn(768, generator=g), torch.randn(768, generator=g)
    got = ops.skinny_linear(x.cuda(), w.cuda(), b.cuda(), ln=(gamma.cuda(), beta.cuda(), 1e-5), epilogue="gelu")
    want = F.gelu(F.linear(F.layer_norm(x, (768,), gamma, beta, 1e-5), w, b), approximate="tanh")
    torch.testing.assert_close(got.cpu(), want, **TOL)
    # Residual: out += h W^T + b, in place, into a strided view of a wider buffer.
    h = torch.randn(M, 3072, generator=g)
    w2, b2 = weights(768, 3072, 2)
    buf = torch.randn(M, 1000, generator=g)
    res = buf.cuda()
    view = res[:, 100:868]
    ops.skinny_linear(h.cuda(), w2.cuda(), b2.cuda(), epilogue="residual", out=view)
    want = buf.clone()
    want[:, 100:868] = buf[:, 100:868] + F.linear(h, w2, b2)
    got = res.cpu()
    torch.testing.assert_close(got[:, 100:868], want[:, 100:868], **TOL)
    assert torch.equal(got[:, :100], buf[:, :100]) and torch.equal(got[:, 868:], buf[:, 868:])


def test_strided_input_rows_and_refused_shapes():
    g = torch.Generator().manual_seed(9)
    wide = torch.randn(6, 2000, generator=g)
    x = wide[:, 32:800]  # rows 2000 apart, 768 columns
    w, b = weights(768, 768, 3)
    got = ops.skinny_linear(x.cuda(), w.cuda(), b.cuda())
    torch.testing.assert_close(got.cpu(), F.linear(x, w, b), **TOL)
    with pytest.raises(_lib.KernelError):
        ops.skinny_linear(torch.zeros(65, 768, device="cuda"), w.cuda())  # more than 64 rows
    with pytest.raises(_lib.KernelError):
        ops.skinny_linear(torch.zeros(2, 512, device="cuda"), torch.zeros(8, 512, device="cuda"))  # K = 512
    with pytest.raises(ValueError):
        ops.skinny_linear(torch.zeros(2, 768, device="cuda"), w.cuda(), epilogue="residual")  # no out


def test_embed_rows_with_source_rows():
    g = torch.Generator().manual_seed(4)
    wte, wpe = torch.randn(50257, 768, generator=g), torch.randn(1024, 768, generator=g)
    ids = torch.tensor([5, 50256, 0, 17, 99], dtype=torch.int64)
    pos = torch.tensor([0, 1023, 7, 300, 2], dtype=torch.int64)
    src = torch.tensor([-1, 3, -1, 0, -1], dtype=torch.int64)
    tokens = torch.tensor([11, 22, 33, 44, 55, 66], dtype=torch.int64)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = ops.embed_rows(ids.cuda(), pos.cuda(), wte.cuda(), wpe.cuda(), src=src.cuda(), tokens=tokens.cuda(),
                         error_word=err)  # fmt: skip
    use = torch.where(src >= 0, tokens[src.clamp(min=0)], ids)
    assert torch.equal(got.cpu(), wte[use] + wpe[pos])
    assert int(err.item()) == 0
    bad = ops.embed_rows(torch.tensor([50257], device="cuda"), torch.tensor([0], device="cuda"), wte.cuda(),
                         wpe.cuda(), error_word=err)  # fmt: skip
    torch.cuda.synchronize()
    assert int(err.item()) & 4 and torch.isfinite(bad).all()  # reported, clamped, in bounds


@pytest.fixture(scope="module")
def model():
    m = GPT2(GPT2Config())
    m.load_state_dict(random_state_dict(m.cfg, seed=0))
    return m.cuda().eval()


@pytest.mark.parametrize("n", [1, 2, 3, 8, 13, 16, 17, 32, 50, 64])
def test_fused_decode_step_matches_library_gemm_step(model, n):
    rng = random.Random(n)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(3, 90))] for _ in range(n)]
    states = []
    for _ in range(2):
        alloc = BlockAllocator(model.cfg, 8 * n + 64, 16, device="cuda")
        seqs = [Sequence(i, list(p)) for i, p in enumerate(prompts)]
        for s in seqs:
            alloc.allocate(s)
        first = paged_forward(model, alloc, seqs).argmax(-1).tolist()
        for s, t in zip(seqs, first):
            s.append_token(t)
            alloc.append_slot(s)
        states.append((alloc, seqs))
    fused = DecodeGraphs(model, states[0][0], max_batch=64, skinny=True)
    plain = DecodeGraphs(model, states[1][0], max_batch=64, skinny=False)
    for _ in range(4):
        lf = fused.forward(states[0][1]).clone()
        lp = plain.forward(states[1][1]).clone()
        torch.testing.assert_close(lf, lp, rtol=1e-4, atol=1e-4)
        nxt = lp.argmax(-1).tolist()
        assert lf.argmax(-1).tolist() == nxt
        for alloc, seqs in states:
            for s, t in zip(seqs, nxt):
                s.append_token(t)
                alloc.append_slot(s)
    for alloc, _ in states:
        alloc.check_device_errors()


@pytest.mark.parametrize("M", [11, 40])
@pytest.mark.parametrize("N,K", [(768, 768), (768, 3072)])
def test_results_are_deterministic(N, K, M):
    """The waves' partial products are summed in a fixed order: repeated calls give the same bits."""
    g = torch.Generator().manual_seed(N + K)
    x = torch.randn(M, K, generator=g).cuda()
    w, b = (t.cuda() for t in weights(N, K, 7))
    first = ops.skinny_linear(x, w, b)
    for _ in range(20):
        assert torch.equal(ops.skinny_linear(x, w, b), first)
    torch.testing.assert_close(first.cpu(), F.linear(x.cpu(), w.cpu(), b.cpu()), **TOL)


@pytest.mark.parametrize("M", [1, 8, 33, 64])
def test_split_k_partials_are_never_stale(M):
    """K = 3072 runs split over four workgroups per column block that hand their partial tiles to
    the last one to arrive (relaxed agent-scope atomics, a wait and a barrier before the counter).
    Three different inputs launched back to back 30 times, with no synchronisation between the
    launches: a partial read before its writer's store is visible, or left over from the previous
    launch, would change the bits. Each output equals its input's first output bit for bit, and
    that one equals torch's fp32 product within tolerance, also with the residual epilogue."""
    g = torch.Generator().manual_seed(100 + M)
    xs = [torch.randn(M, 3072, generator=g).cuda() for _ in range(3)]
    res = torch.randn(M, 768, generator=g).cuda()
    w, b = (t.cuda() for t in weights(768, 3072, 9))
    outs = [[], [], []]
    for it in range(30):
        for i, x in enumerate(xs):
            if it % 2:
                outs[i].append(ops.skinny_linear(x, w, b))
            else:  # out += x @ w.T + b, into a fresh copy of the residual
                outs[i].append(ops.skinny_linear(x, w, b, epilogue="residual", out=res.clone()))
    torch.cuda.synchronize()
    for i, x in enumerate(xs):
        plain, resid = outs[i][1], outs[i][0]
        for it, o in enumerate(outs[i]):
            assert torch.equal(o, plain if it % 2 else resid), (i, it)
        want = F.linear(x.cpu(), w.cpu(), b.cpu())
        torch.testing.assert_close(plain.cpu(), want, **TOL)
        torch.testing.assert_close(resid.cpu(), want + res.cpu(), **TOL)


# ---- the LM head with the greedy argmax fused in (tq_skinny_linear_argmax) ----------------------
def _lm_head_case(M: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, 768, generator=g) * 2 + 0.3
    w = torch.randn(50257, 768, generator=g) * 0.02
    gamma, beta = torch.randn(768, generator=g) * 0.5 + 1, torch.randn(768, generator=g) * 0.1
    return x, w, gamma, beta


@pytest.mark.parametrize("M", [1, 2, 5, 8, 13, 16])
def test_lm_head_argmax_equals_logits_then_argmax(M):
    """Fused ids == tq_argmax_rows over the unfused kernel's logits (the same products summed in the
    same order, so the same bits), and == a float64 CPU argmax wherever its top-1 / top-2 gap is not a
    near tie."""
    x, w, gamma, beta = _lm_head_case(M, M)
    ln = (gamma.cuda(), beta.cuda(), 1e-5)
    xc, wc = x.cuda(), w.cuda()
    got = ops.skinny_linear_argmax(xc, wc, None, ln=ln)
    logits = ops.skinny_linear(xc, wc, None, ln=ln)
    assert torch.equal(got, ops.argmax_rows(logits))
    ref = F.linear(F.layer_norm(x.double(), (768,), gamma.double(), beta.double(), 1e-5), w.double())
    top2 = ref.topk(2, dim=-1)
    gap = top2.values[:, 0] - top2.values[:, 1]
    for m in range(M):
        assert int(got[m]) == int(top2.indices[m, 0]) or float(gap[m]) < 1e-4, (m, float(gap[m]))
    # Without the LayerNorm and with a bias.
    b = torch.randn(50257, generator=torch.Generator().manual_seed(3)) * 0.1
    got = ops.skinny_linear_argmax(xc, wc, b.cuda())
    assert torch.equal(got, ops.argmax_rows(ops.skinny_linear(xc, wc, b.cuda())))


def test_lm_head_argmax_ties_nans_and_workspace_reuse():
    """Ties keep the lowest column, inside one 32-column slice and across slices; a NaN logit wins
    and the first NaN column is taken; calls of different sizes in a row, sharing the workspace
    (the previous call's candidates still in it), are each correct."""
    x, w, gamma, beta = _lm_head_case(3, 99)
    h = F.layer_norm(x, (768,), gamma, beta, 1e-5)
    # Row 0: columns 40000 and 100 (different slices) tie above everything else.
    # Row 1: columns 7 and 5 (one slice) tie above everything else.
    w[100] = w[40000] = h[0] / h[0].norm() * 5
    w[5] = w[7] = h[1] / h[1].norm() * 5
    x[2] = float("nan")  # row 2: every logit is NaN, the first column wins
    ln = (gamma.cuda(), beta.cuda(), 1e-5)
    got = ops.skinny_linear_argmax(x.cuda(), w.cuda(), None, ln=ln).tolist()
    assert got == [100, 5, 0]
    ref = F.linear(F.layer_norm(x, (768,), gamma, beta, 1e-5), w)
    assert got == ref.argmax(-1).tolist()  # torch's rule agrees
    # One NaN column: it wins in every row (torch's argmax does the same).
    xn, wn, gn, bn = _lm_head_case(2, 7)
    wn[777, 0] = float("nan")
    lnn = (gn.cuda(), bn.cuda(), 1e-5)
    got_nan = ops.skinny_linear_argmax(xn.cuda(), wn.cuda(), None, ln=lnn).tolist()
    assert got_nan == [777, 777] == F.linear(F.layer_norm(xn, (768,), gn, bn, 1e-5), wn).argmax(-1).tolist()
    # Calls of other sizes right after, then the first again: each is correct and repeatable.
    for M, seed in ((16, 5), (1, 6)):
        x2, w2, g2, b2 = _lm_head_case(M, seed)
        ln2 = (g2.cuda(), b2.cuda(), 1e-5)
        ids = ops.skinny_linear_argmax(x2.cuda(), w2.cuda(), None, ln=ln2)
        assert torch.equal(ids, ops.argmax_rows(ops.skinny_linear(x2.cuda(), w2.cuda(), None, ln=ln2)))
    assert ops.skinny_linear_argmax(x.cuda(), w.cuda(), None, ln=ln).tolist() == got
    with pytest.raises(ValueError):
        ops.skinny_linear_argmax(torch.zeros(17, 768, device="cuda"), w.cuda())


@pytest.mark.parametrize("n", [1, 3, 8, 16])
def test_ids_only_graph_matches_logits_graph(model, n):
    """The ids-only decode graph (fused head + argmax, no logits) emits the same ids as the graph
    that writes logits and runs tq_argmax_rows, step after step."""
    rng = random.Random(100 + n)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(3, 90))] for _ in range(n)]
    states = []
    for _ in range(2):
        alloc = BlockAllocator(model.cfg, 8 * n + 64, 16, device="cuda")
        seqs = [Sequence(i, list(p)) for i, p in enumerate(prompts)]
        for s in seqs:
            alloc.allocate(s)
        first = paged_forward(model, alloc, seqs).argmax(-1).tolist()
        for s, t in zip(seqs, first):
            s.append_token(t)
            alloc.append_slot(s)
        states.append((alloc, seqs, DecodeGraphs(model, alloc, max_batch=16)))
    for _ in range(5):
        outs = []
        for i, (alloc, seqs, graphs) in enumerate(states):
            logits, ids = graphs.launch(seqs, logits=(i == 1))
            assert (logits is None) == (i == 0)
            outs.append(ids.tolist())
        assert outs[0] == outs[1]
        for alloc, seqs, _ in states:
            for s, t in zip(seqs, outs[1]):
                s.append_token(t)
                alloc.append_slot(s)
    for alloc, _, _ in states:
        alloc.check_device_errors()
