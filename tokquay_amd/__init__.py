"""MI355X (gfx950) paged attention for the Tokquay GPT-2 engine.

The hot path - cache write, paged decode attention and paged causal/chunked
prefill attention - runs in hand-written HIP kernels behind the C ABI of
``include/tokquay_amd.h`` (``libtokquay_amd.so``, built by
``python -m tokquay_amd.build``). The Python modules keep the reference's
pool layout, allocator, batch-view contract, scheduler and engine, and drive
the kernels; there is no CPU or PyTorch fallback for attention.
"""

from tokquay_amd.kv_cache import BatchedKV, BlockAllocator, OutOfBlocksError, PagedBatch, cdiv
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.sequence import SamplingParams, Sequence, SequenceStatus

__all__ = [
    "BatchedKV",
    "BlockAllocator",
    "GPT2",
    "GPT2Config",
    "OutOfBlocksError",
    "PagedBatch",
    "SamplingParams",
    "Sequence",
    "SequenceStatus",
    "cdiv",
]
