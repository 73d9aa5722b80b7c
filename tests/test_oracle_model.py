"""Pins the oracle's GPT-2 (oracle/gpt2_ref.py) against HuggingFace and against itself.

* HuggingFace ``GPT2LMHeadModel``, built offline from a config (no download)
  and loaded with the same all-random weights (biases and LayerNorm included),
  gives the same logits in float64 to 1e-9 - the reference's own HF parity
  check (tests/test_phase1_model.py:35-72), here on random weights;
* paged == contiguous cache == full forward in float64 across block
  boundaries, with a garbage pool and shuffled block tables, and for a mixed
  prefill + decode batch (tests/test_phase3_paged.py:87-106, :143-164);
* a model with a planted mistake (exact instead of tanh GELU) misses HF.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.gpt2_ref import (
    RefAllocator,
    RefConfig,
    RefContiguousKVCache,
    RefSeq,
    build_ref_model,
    ref_greedy_generate,
    ref_paged_forward,
    ref_paged_greedy_generate,
)
from tokquay_amd.weights import hf_state_dict, random_state_dict

TINY = RefConfig(vocab_size=97, n_positions=64, n_embd=128, n_layer=2, n_head=2)


@pytest.fixture(scope="module")
def sd():
    return random_state_dict(TINY, seed=1, all_random=True)


@pytest.fixture(scope="module")
def m64(sd):
    return build_ref_model(TINY, sd, dtype=torch.float64)


@pytest.fixture(scope="module")
def hf64(sd):
    transformers = pytest.importorskip("transformers")
    hc = transformers.GPT2Config(vocab_size=97, n_positions=64, n_embd=128, n_layer=2, n_head=2,
                                 resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0, bos_token_id=0, eos_token_id=0)  # fmt: skip
    hf = transformers.GPT2LMHeadModel(hc)
    hf.load_state_dict(hf_state_dict(sd))
    return hf.double().eval()


def ids(seed, n):
    rng = random.Random(seed)
    return [rng.randrange(97) for _ in range(n)]


def test_full_forward_matches_huggingface_float64(m64, hf64):
    x = torch.tensor([ids(1, 40), ids(2, 40)])
    with torch.no_grad():
        got = m64(x)
        want = hf64(x).logits
    torch.testing.assert_close(got, want, atol=1e-9, rtol=0)


def test_planted_gelu_mistake_misses_huggingface(sd, hf64, monkeypatch):
    import oracle.gpt2_ref as g

    monkeypatch.setattr(g._MLP, "forward", lambda self, x: self.c_proj(torch.nn.functional.gelu(self.c_fc(x))))
    bad = build_ref_model(TINY, sd, dtype=torch.float64)
    x = torch.tensor([ids(3, 30)])
    with torch.no_grad():
        assert (bad(x) - hf64(x).logits).abs().max() > 1e-6


def test_contiguous_cache_matches_full_forward_float64(m64):
    x = torch.tensor([ids(4, 30)])
    with torch.no_grad():
        full = m64(x)
        cache = RefContiguousKVCache(TINY, 1, 30, dtype=torch.float64)
        got = [m64(x[:, :4], cache)] + [m64(x[:, t : t + 1], cache) for t in range(4, 30)]
    torch.testing.assert_close(torch.cat(got, 1), full, atol=1e-9, rtol=0)


def hard_allocator(num_blocks, bs, seed):
    alloc = RefAllocator(TINY, num_blocks, bs, dtype=torch.float64)
    g = torch.Generator().manual_seed(seed)
    alloc.pool.copy_(torch.randn(alloc.pool.shape, generator=g, dtype=torch.float64) * 50)
    random.Random(seed).shuffle(alloc.free_list)
    return alloc


def test_paged_decode_across_block_boundaries_matches_full_forward_float64(m64):
    toks = ids(5, 40)
    with torch.no_grad():
        full = m64(torch.tensor([toks]))[0]
    alloc = hard_allocator(32, 4, 0)
    seq = RefSeq(toks[:6])
    alloc.allocate(seq)
    got = [ref_paged_forward(m64, alloc, [seq])[0]]
    for t in range(6, 40):
        seq.output.append(toks[t])
        alloc.append_slot(seq)
        got.append(ref_paged_forward(m64, alloc, [seq])[0])
    torch.testing.assert_close(torch.stack(got), full[5:], atol=1e-9, rtol=0)


def test_mixed_prefill_and_decode_batch_matches_full_forward_float64(m64):
    a_ids, b_ids = ids(6, 17), ids(7, 23)
    with torch.no_grad():
        fa, fb = m64(torch.tensor([a_ids]))[0, -1], m64(torch.tensor([b_ids]))[0, -1]
    alloc = hard_allocator(64, 4, 1)
    a = RefSeq(a_ids[:-1])
    alloc.allocate(a)
    ref_paged_forward(m64, alloc, [a])
    a.output.append(a_ids[-1])
    alloc.append_slot(a)
    b = RefSeq(b_ids)
    alloc.allocate(b)
    logits = ref_paged_forward(m64, alloc, [a, b])
    torch.testing.assert_close(logits[0], fa, atol=1e-9, rtol=0)
    torch.testing.assert_close(logits[1], fb, atol=1e-9, rtol=0)


def test_chunked_prefill_equals_one_shot_float64(m64):
    toks = ids(8, 50)
    alloc = hard_allocator(64, 4, 2)
    one, chunked = RefSeq(toks), RefSeq(toks)
    alloc.allocate(one)
    alloc.allocate(chunked)
    want = ref_paged_forward(m64, alloc, [one])
    for n in (16, 16, 18):
        got = ref_paged_forward(m64, alloc, [chunked], [n])
    torch.testing.assert_close(got, want, atol=1e-9, rtol=0)


def test_paged_batch_greedy_equals_each_alone():
    """Batched paged greedy decode of 8 ragged prompts equals each prompt decoded alone on the
    contiguous cache (tests/test_phase3_paged.py:109-129), fp32."""
    m = build_ref_model(TINY, random_state_dict(TINY, seed=2))
    lengths = [1, 3, 7, 12, 16, 17, 33, 40]
    prompts = [ids(20 + i, n) for i, n in enumerate(lengths)]
    alloc = RefAllocator(TINY, 128, 16)
    batched = ref_paged_greedy_generate(m, alloc, prompts, 12)
    for p, got in zip(prompts, batched):
        assert got == ref_greedy_generate(m, p, 12)
    assert sorted(alloc.free_list) == list(range(128))


def test_weights_are_deterministic_and_seeded():
    a = random_state_dict(TINY, seed=3)
    b = random_state_dict(TINY, seed=3)
    c = random_state_dict(TINY, seed=4)
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert not torch.equal(a["wte.weight"], c["wte.weight"])
    assert float(a["wte.weight"].std()) == pytest.approx(0.02, rel=0.05)
    assert torch.all(a["h.0.ln_1.weight"] == 1) and torch.all(a["h.0.attn.c_attn.bias"] == 0)
