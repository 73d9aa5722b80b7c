"""HIP-graph decode steps equal eager decode steps.

Each replay is compared with an eager step on an identical copy of the state,
with unrelated eager work and synchronisations between replays, across batch
buckets (the batch shrinks as sequences finish) and growing contexts.
"""

from __future__ import annotations

import random

import pytest
import torch

from tokquay_amd.engine import Engine
from tokquay_amd.generate import paged_forward
from tokquay_amd.graphs import DecodeGraphs, bucket_for
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.sequence import SamplingParams, Sequence
from tokquay_amd.weights import random_state_dict

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    m = GPT2(GPT2Config())
    m.load_state_dict(random_state_dict(m.cfg, seed=0))
    return m.cuda().eval()


def test_bucket_for():
    assert [bucket_for(n) for n in (1, 2, 3, 4, 5, 64, 65, 256)] == [1, 2, 4, 4, 8, 64, 128, 256]


def make_state(model, prompts):
    alloc = BlockAllocator(model.cfg, 256, 16, device="cuda")
    seqs = [Sequence(i, list(p)) for i, p in enumerate(prompts)]
    for s in seqs:
        alloc.allocate(s)
    return alloc, seqs


def test_graph_replays_match_eager_steps(model):
    rng = random.Random(0)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(5, 60))] for _ in range(7)]
    ga, gseqs = make_state(model, prompts)
    ea, eseqs = make_state(model, prompts)
    for alloc, seqs in ((ga, gseqs), (ea, eseqs)):
        first = paged_forward(model, alloc, seqs).argmax(-1).tolist()
        for s, t in zip(seqs, first):
            s.append_token(t)
            alloc.append_slot(s)
    graphs = DecodeGraphs(model, ga, max_batch=8)
    junk = torch.randn(512, 512, device="cuda")
    for step in range(12):
        if step == 6:  # four sequences finish: the batch moves from bucket 8 to bucket 4
            for seqs, alloc in ((gseqs, ga), (eseqs, ea)):
                for s in seqs[:4]:
                    alloc.free(s)
                del seqs[:4]
        lg = graphs.forward(gseqs).clone()
        le = paged_forward(model, ea, eseqs)
        torch.cuda.synchronize()
        junk = torch.tanh(junk @ junk) * 0.5  # unrelated eager work between replays
        torch.cuda.synchronize()
        torch.testing.assert_close(lg, le, rtol=1e-4, atol=1e-4)
        nxt = le.argmax(-1).tolist()
        assert lg.argmax(-1).tolist() == nxt
        for seqs, alloc in ((gseqs, ga), (eseqs, ea)):
            for s, t in zip(seqs, nxt):
                s.append_token(t)
                alloc.append_slot(s)
    ga.check_device_errors()
    # 7 sequences -> bucket 8, then 3 -> bucket 4, each captured once (logits graphs: forward() wants them)
    assert set(graphs.graphs) == {(8, False), (4, False)}
    for s_g, s_e in zip(gseqs, eseqs):
        assert s_g.num_cached_tokens == s_e.num_cached_tokens
    # Identical pools: the replayed cache writes landed in the same slots with the same bits... up to
    # GEMM rounding, so compare the blocks the live sequences own at fp32 tolerance.
    own = sorted({b for s in gseqs for b in s.block_table})
    own_e = sorted({b for s in eseqs for b in s.block_table})
    assert own == own_e
    torch.testing.assert_close(ga.pool[own], ea.pool[own], rtol=1e-4, atol=1e-4)


def test_engine_with_and_without_graphs_emits_the_same_tokens(model):
    rng = random.Random(1)
    reqs = [([rng.randrange(50256) for _ in range(rng.randint(4, 50))], rng.randint(5, 30)) for _ in range(10)]
    outs = []
    for use_graphs, pipeline in ((True, True), (True, False), (False, False)):
        engine = Engine(model, BlockAllocator(model.cfg, 128, 16, device="cuda"), use_graphs=use_graphs,
                        pipeline=pipeline)  # fmt: skip
        seqs = []
        for i, (p, n) in enumerate(reqs):
            seqs.append(engine.add_request(p, SamplingParams(max_tokens=n, ignore_eos=True)))
            if i % 3 == 2:
                engine.step()
        engine.run_until_done()
        outs.append([s.output_token_ids for s in seqs])
        if use_graphs:
            assert engine.graphs.graphs, "no decode step went through a graph"
        assert (engine.stats.lookahead_steps > 0) == pipeline
    assert outs[0] == outs[1] == outs[2]
