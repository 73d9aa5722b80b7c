"""Oracle: a CPU restatement of the reference's paged-attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``tokquay_amd``) imports,
calls or links anything here. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or the
timed CPU baseline), never as the thing measured on the GPU.

Modules
  paged_ref   the reference's per-step batch view (scatter / gather / mask,
              tokquay/kv_cache.py:38-242) and attention math
              (tokquay/model.py:94-96), in torch, any dtype / device; plus a
              float64 numpy brute-force softmax attention used to pin it.
  gpt2_ref    the reference's GPT-2 forward (tokquay/model.py:24-181) with its
              three cache modes and the greedy drivers of tokquay/generate.py.

How each part is pinned (the reference ships no golden vectors or fixtures;
its own tests are self-consistency and HuggingFace parity on pretrained
weights, which need the network):
  * scatter / gather / mask + attention: against brute-force float64 softmax
    attention over each sequence's own positions (no pool, no mask), and
    against invariants - block relabelling, garbage in unused slots, block
    size 4 vs 16 (tests/test_oracle_attention.py);
  * GPT-2 forward: against HuggingFace ``GPT2LMHeadModel`` built offline from a
    config with the same all-random weights (biases and LayerNorm included),
    float64 at 1e-9, and paged == contiguous == full forward in float64
    (tests/test_oracle_model.py);
  * allocator / scheduler / metrics: the reference's property tests and
    hand-worked scenarios, restated (tests/test_host_*.py).
"""
