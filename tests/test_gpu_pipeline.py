"""Greedy argmax kernel and pipelined graph decode on the GPU.

* ``tq_argmax_rows`` against torch's ``argmax(-1)`` (the reference's batched
  greedy pick, tokquay/engine.py:190) on the CPU: exact indices, with planted
  ties, NaNs, infinities and signed zeros, several widths and row strides.
* A graph replay whose rows take their input token from the previous replay's
  argmax (source rows) against the same replay fed those tokens from the host:
  bit-identical logits.
* The pipelined engine against the synchronous engine and the CPU reference:
  identical greedy ids, also when sequences stop on EOS or are aborted while
  their step is in flight.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.gpt2_ref import RefConfig, build_ref_model, ref_greedy_generate
from tokquay_amd import ops
from tokquay_amd.engine import Engine
from tokquay_amd.generate import paged_forward
from tokquay_amd.graphs import DecodeGraphs
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.sequence import SamplingParams, Sequence, SequenceStatus
from tokquay_amd.weights import random_state_dict

pytestmark = pytest.mark.gpu


def cpu_argmax(x: torch.Tensor) -> list[int]:
    return x.cpu().argmax(-1).tolist()


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 2), (7, 63), (5, 1024), (9, 1025), (256, 50257), (2, 300_000)])
def test_argmax_random_rows(rows, cols):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, generator=g)
    got = ops.argmax_rows(x.cuda()).tolist()
    assert got == cpu_argmax(x)


def test_argmax_ties_nans_infinities_and_zeros():
    cols = 5000
    x = torch.randn(12, cols, generator=torch.Generator().manual_seed(1))
    x[0, [17, 3000, 4999]] = 9.0  # tie: the lowest index wins
    x[1, :] = 2.5  # every column ties
    x[2, [10, 2000]] = float("nan")  # the first NaN wins over everything
    x[2, 5] = float("inf")
    x[3, :] = float("-inf")  # all -inf: index 0
    x[4, :] = -1.0
    x[4, [40, 41]] = 0.0
    x[4, 40] = -0.0  # -0 ties +0: the lower index
    x[5, 4999] = float("inf")
    x[6, :] = float("nan")
    x[7, 1023:1025] = 50.0  # tie across a thread's stride
    x[8, [1, 1025, 2049]] = 7.0
    x[9, 0] = 1e30
    x[10, -1] = 1e30
    x[11, :] = torch.arange(cols, dtype=torch.float32).flip(0)  # strictly decreasing: index 0
    got = ops.argmax_rows(x.cuda()).tolist()
    assert got == cpu_argmax(x)
    assert got[:5] == [17, 0, 10, 0, 40]


def test_argmax_row_stride_and_out_view():
    g = torch.Generator().manual_seed(2)
    wide = torch.randn(33, 700, generator=g).cuda()
    view = wide[:, :513]  # rows 700 apart, 513 columns
    out = torch.full((40,), -5, dtype=torch.int64, device="cuda")
    ops.argmax_rows(view, out=out[3:36])
    res = out.cpu()
    assert res[3:36].tolist() == cpu_argmax(view)
    assert res[:3].tolist() == [-5] * 3 and res[36:].tolist() == [-5] * 4  # nothing outside the view
    assert ops.argmax_rows(torch.empty(0, 10, device="cuda")).numel() == 0
    with pytest.raises(ValueError):
        ops.argmax_rows(torch.empty(3, 0, device="cuda"))
    with pytest.raises(ValueError):
        ops.argmax_rows(wide.t())  # columns not contiguous


@pytest.fixture(scope="module")
def weights():
    return random_state_dict(GPT2Config(), seed=0)


@pytest.fixture(scope="module")
def model(weights):
    m = GPT2(GPT2Config())
    m.load_state_dict(weights)
    return m.cuda().eval()


def text(seed, n):
    rng = random.Random(seed)
    return [rng.randrange(50256) for _ in range(n)]


def test_source_rows_feed_the_previous_replays_tokens(model):
    """Step k+1 fed from step k's on-device argmax (rows permuted) == step k+1 fed from the host."""
    prompts = [text(80 + i, 7 + 9 * i) for i in range(6)]
    states = []
    for _ in range(2):
        alloc = BlockAllocator(model.cfg, 64, 16, device="cuda")
        seqs = [Sequence(i, list(p)) for i, p in enumerate(prompts)]
        for s in seqs:
            alloc.allocate(s)
        first = paged_forward(model, alloc, seqs).argmax(-1).tolist()
        for s, t in zip(seqs, first):
            s.append_token(t)
            alloc.append_slot(s)
        states.append((alloc, seqs, DecodeGraphs(model, alloc, max_batch=8)))
    (a1, s1, g1), (a2, s2, g2) = states
    # Step k on both copies, from host ids.
    _, ids1 = g1.launch(s1)
    _, ids2 = g2.launch(s2)
    tok = ids2.tolist()
    assert ids1.tolist() == tok
    # Step k+1: copy 1 drops sequence 2 and reverses the order, taking tokens from the device.
    keep = [5, 4, 3, 1, 0]
    seqs1 = [s1[i] for i in keep]
    for s in seqs1:
        a1.append_slot(s, s.num_cached_tokens + 1)
    logits1, _ = g1.launch(seqs1, src_rows=keep)
    logits1 = logits1.clone()
    # Copy 2 appends the tokens on the host first, as the synchronous engine does.
    seqs2 = [s2[i] for i in keep]
    for i, s in zip(keep, seqs2):
        s.append_token(tok[i])
        a2.append_slot(s)
    logits2, _ = g2.launch(seqs2)
    assert torch.equal(logits1, logits2)
    a1.check_device_errors()
    a2.check_device_errors()


def run_engine(model, specs, pipeline, eos=None, abort_at=None, blocks=256):
    engine = Engine(model, BlockAllocator(model.cfg, blocks, 16, device="cuda"), pipeline=pipeline,
                    **({"eos_token_id": eos} if eos is not None else {}))  # fmt: skip
    pending = sorted(specs, key=lambda a: a[0])
    seqs, step = [], 0
    while pending or engine.has_unfinished():
        while pending and pending[0][0] <= step:
            _, prompt, params = pending.pop(0)
            seqs.append(engine.add_request(prompt, params))
        if abort_at and step == abort_at[0]:
            engine.abort_request(seqs[abort_at[1]])
        engine.step()
        step += 1
        assert step < 5000
    engine.allocator.check_device_errors()
    assert engine.allocator.num_free_blocks == engine.allocator.num_blocks
    return engine, seqs


def test_pipelined_engine_matches_reference(model, weights):
    specs = [(0, text(1, 5), 30), (0, text(2, 30), 12), (3, text(3, 8), 25), (6, text(4, 1), 20),
             (6, text(5, 33), 15), (11, text(6, 17), 18)]  # fmt: skip
    engine, seqs = run_engine(model, [(t, p, SamplingParams(max_tokens=n, ignore_eos=True)) for t, p, n in specs], True)
    assert engine.stats.lookahead_steps > 0
    ref = build_ref_model(RefConfig(), weights)
    for seq, (_, prompt, n) in zip(seqs, specs):
        assert seq.output_token_ids == ref_greedy_generate(ref, list(prompt), n)


def test_pipelined_engine_eos_and_abort_match_synchronous_engine(model):
    specs = [(0, text(20 + i, 6 + 5 * i), 24) for i in range(6)]
    base, seqs = run_engine(model, [(t, p, SamplingParams(max_tokens=n, ignore_eos=True)) for t, p, n in specs],
                            pipeline=False)  # fmt: skip
    # An EOS id that sequence 2 emits part-way through (and that ends it there, and any other that emits it).
    eos = seqs[2].output_token_ids[10]
    params = [SamplingParams(max_tokens=n, ignore_eos=(i % 2 == 1)) for i, (_, _, n) in enumerate(specs)]
    outs = []
    for pipeline in (False, True):
        engine, seqs = run_engine(model, [(t, p, q) for (t, p, _), q in zip(specs, params)], pipeline, eos=eos,
                                  abort_at=(9, 4))  # fmt: skip
        outs.append([(s.output_token_ids, s.finish_reason) for s in seqs])
        assert seqs[2].finish_reason == "stop" and seqs[4].finish_reason == "abort"
        assert all(s.status is SequenceStatus.FINISHED for s in seqs)
        if pipeline:
            assert engine.stats.lookahead_steps > 0
    # The aborted sequence may stop one step apart; every other sequence is identical.
    for i, (a, b) in enumerate(zip(*outs)):
        if i == 4:
            short, long_ = sorted((a[0], b[0]), key=len)
            assert long_[: len(short)] == short and len(long_) - len(short) <= 1
        else:
            assert a == b, i


# ------------------------------------------------------------------------------ add + LayerNorm
@pytest.mark.parametrize("rows,cols", [(1, 768), (256, 768), (37, 64), (5, 2048), (3, 4), (9, 1028)])
def test_add_layernorm_matches_torch(rows, cols):
    """tq_add_layernorm == (x + y, F.layer_norm(x + y)) in fp32 (torch on the CPU as the reference)."""
    g = torch.Generator().manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, generator=g) * 3 + 1
    y = torch.randn(rows, cols, generator=g)
    w = torch.randn(cols, generator=g)
    b = torch.randn(cols, generator=g)
    s_ref = x + y
    h_ref = torch.nn.functional.layer_norm(s_ref, (cols,), w, b, 1e-5)
    s, h = ops.add_layernorm(x.cuda(), y.cuda(), w.cuda(), b.cuda(), 1e-5)
    assert torch.equal(s.cpu(), s_ref)  # one fp32 add per element: exact
    torch.testing.assert_close(h.cpu(), h_ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(256, 768), (3, 4), (9, 1028)])
def test_layernorm_without_add(rows, cols):
    """``y=None``: the plain LayerNorm of x, x_out == x bit for bit (also in place)."""
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g) * 2 - 1
    w, b = torch.randn(cols, generator=g), torch.randn(cols, generator=g)
    xd = x.cuda()
    s, h = ops.add_layernorm(xd, None, w.cuda(), b.cuda(), 1e-5, x_out=xd)
    assert s.data_ptr() == xd.data_ptr() and torch.equal(s.cpu(), x)
    torch.testing.assert_close(h.cpu(), torch.nn.functional.layer_norm(x, (cols,), w, b, 1e-5), rtol=1e-5, atol=1e-5)


def test_add_layernorm_in_place_and_strided_views():
    g = torch.Generator().manual_seed(3)
    big = torch.randn(16, 2 * 768, generator=g).cuda()
    y = big[:, 768:]  # rows 1536 apart
    x = torch.randn(16, 768, generator=g).cuda()
    w, b = torch.randn(768, generator=g).cuda(), torch.randn(768, generator=g).cuda()
    want_s = (x + y).cpu()
    want_h = torch.nn.functional.layer_norm(want_s, (768,), w.cpu(), b.cpu(), 1e-5)
    out, h = ops.add_layernorm(x, y, w, b, 1e-5, x_out=x)
    assert out.data_ptr() == x.data_ptr()
    assert torch.equal(x.cpu(), want_s)
    torch.testing.assert_close(h.cpu(), want_h, rtol=1e-5, atol=1e-5)
    from tokquay_amd import _lib

    with pytest.raises(_lib.KernelError):
        ops.add_layernorm(x[:, :766], y[:, :766], w[:766], b[:766], 1e-5)  # 766 columns: not a multiple of 4
