"""Reference restatement of the GPT-2 forward and greedy drivers (test oracle).

``RefGPT2`` follows tokquay/model.py:24-181: embeddings, pre-LN blocks, fused
QKV, attention with one of three caches - none (full causal forward),
``RefContiguousKVCache`` (:38-53, :80-92) or the paged ``RefPagedBatch``
(:73-78) - tanh GELU MLP, last-real-token select (:177-179) and the tied LM
head (:180-181). ``RefAllocator`` is the LIFO block allocator of
tokquay/kv_cache.py:38-127; the drivers are tokquay/generate.py:17-120.

It loads the same ``[out, in]`` state dict as ``tokquay_amd.GPT2`` and runs
in any dtype on any device.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle.paged_ref import RefPagedBatch, cdiv, ref_attention


@dataclass
class RefConfig:
    vocab_size: int = 50257
    n_positions: int = 1024
    n_embd: int = 768
    n_layer: int = 12
    n_head: int = 12
    layer_norm_eps: float = 1e-5

    @property
    def d_head(self) -> int:
        return self.n_embd // self.n_head


class RefContiguousKVCache:
    def __init__(self, cfg: RefConfig, batch_size: int, max_len: int, device=None, dtype=torch.float32):
        shape = (cfg.n_layer, batch_size, cfg.n_head, max_len, cfg.d_head)
        self.k = torch.zeros(shape, device=device, dtype=dtype)
        self.v = torch.zeros(shape, device=device, dtype=dtype)
        self.max_len = max_len
        self.length = 0


class _Attention(nn.Module):
    def __init__(self, cfg: RefConfig):
        super().__init__()
        self.n_head, self.d_head = cfg.n_head, cfg.d_head
        self.c_attn = nn.Linear(cfg.n_embd, 3 * cfg.n_embd)
        self.c_proj = nn.Linear(cfg.n_embd, cfg.n_embd)

    def forward(self, x, cache, layer):
        B, T, C = x.shape
        q, k, v = self.c_attn(x).split(C, dim=-1)
        q, k, v = (t.view(B, T, self.n_head, self.d_head).transpose(1, 2) for t in (q, k, v))
        if isinstance(cache, RefPagedBatch):
            cache.write(layer, k, v)
            k, v = cache.gather(layer)
            allowed = cache.mask
        else:
            start = 0
            if cache is not None:
                start = cache.length
                cache.k[layer, :, :, start : start + T] = k
                cache.v[layer, :, :, start : start + T] = v
                k = cache.k[layer, :, :, : start + T]
                v = cache.v[layer, :, :, : start + T]
            q_pos = torch.arange(start, start + T, device=x.device)[:, None]
            k_pos = torch.arange(start + T, device=x.device)[None, :]
            allowed = k_pos <= q_pos
        out = ref_attention(q, k, v, allowed)
        return self.c_proj(out.transpose(1, 2).reshape(B, T, C))


class _MLP(nn.Module):
    def __init__(self, cfg: RefConfig):
        super().__init__()
        self.c_fc = nn.Linear(cfg.n_embd, 4 * cfg.n_embd)
        self.c_proj = nn.Linear(4 * cfg.n_embd, cfg.n_embd)

    def forward(self, x):
        return self.c_proj(F.gelu(self.c_fc(x), approximate="tanh"))


class _Block(nn.Module):
    def __init__(self, cfg: RefConfig):
        super().__init__()
        self.ln_1 = nn.LayerNorm(cfg.n_embd, eps=cfg.layer_norm_eps)
        self.attn = _Attention(cfg)
        self.ln_2 = nn.LayerNorm(cfg.n_embd, eps=cfg.layer_norm_eps)
        self.mlp = _MLP(cfg)

    def forward(self, x, cache, layer):
        x = x + self.attn(self.ln_1(x), cache, layer)
        return x + self.mlp(self.ln_2(x))


class RefGPT2(nn.Module):
    def __init__(self, cfg: RefConfig | None = None):
        super().__init__()
        self.cfg = cfg or RefConfig()
        self.wte = nn.Embedding(self.cfg.vocab_size, self.cfg.n_embd)
        self.wpe = nn.Embedding(self.cfg.n_positions, self.cfg.n_embd)
        self.h = nn.ModuleList(_Block(self.cfg) for _ in range(self.cfg.n_layer))
        self.ln_f = nn.LayerNorm(self.cfg.n_embd, eps=self.cfg.layer_norm_eps)

    def forward(self, input_ids, cache=None, last_only: bool = False):
        B, T = input_ids.shape
        paged = isinstance(cache, RefPagedBatch)
        if paged:
            if (B, T) != (cache.B, cache.T):
                raise ValueError(f"input_ids {tuple(input_ids.shape)} does not match batch {(cache.B, cache.T)}")
            if cache.max_ctx > self.cfg.n_positions:
                raise ValueError(f"sequence length {cache.max_ctx} exceeds n_positions={self.cfg.n_positions}")
            pos = cache.positions.clamp(max=self.cfg.n_positions - 1)
        else:
            start = cache.length if cache is not None else 0
            if start + T > self.cfg.n_positions:
                raise ValueError(f"sequence length {start + T} exceeds n_positions={self.cfg.n_positions}")
            if cache is not None and start + T > cache.max_len:
                raise ValueError(f"sequence length {start + T} exceeds cache max_len={cache.max_len}")
            pos = torch.arange(start, start + T, device=input_ids.device)
        x = self.wte(input_ids) + self.wpe(pos)
        for i, block in enumerate(self.h):
            x = block(x, cache, i)
        if isinstance(cache, RefContiguousKVCache):
            cache.length += T
        if last_only:
            x = x[torch.arange(B, device=x.device), cache.last_idx][:, None] if paged else x[:, -1:]
        x = self.ln_f(x)
        return x @ self.wte.weight.T


class RefSeq:
    """The fields of the reference ``Sequence`` the drivers touch (tokquay/sequence.py:34-81)."""

    def __init__(self, prompt: list[int]):
        self.prompt = list(prompt)
        self.output: list[int] = []
        self.block_table: list[int] = []
        self.num_cached_tokens = 0

    @property
    def token_ids(self) -> list[int]:
        return self.prompt + self.output

    @property
    def num_tokens(self) -> int:
        return len(self.prompt) + len(self.output)


class RefAllocator:
    """LIFO block allocator over a ``[NB, L, 2, H, bs, d]`` pool (tokquay/kv_cache.py:38-119)."""

    def __init__(self, cfg: RefConfig, num_blocks: int, block_size: int, device=None, dtype=torch.float32):
        self.block_size = block_size
        self.pool = torch.zeros(num_blocks, cfg.n_layer, 2, cfg.n_head, block_size, cfg.d_head,
                                device=device, dtype=dtype)  # fmt: skip
        self.free_list = list(range(num_blocks - 1, -1, -1))

    def take(self, n: int) -> list[int]:
        if n > len(self.free_list):
            raise RuntimeError(f"need {n} blocks, only {len(self.free_list)} free")
        return [self.free_list.pop() for _ in range(n)]

    def allocate(self, seq: RefSeq) -> None:
        seq.block_table = self.take(cdiv(seq.num_tokens, self.block_size))

    def append_slot(self, seq: RefSeq) -> None:
        missing = cdiv(seq.num_tokens, self.block_size) - len(seq.block_table)
        if missing > 0:
            seq.block_table.extend(self.take(missing))

    def free(self, seq: RefSeq) -> None:
        self.free_list.extend(seq.block_table)
        seq.block_table = []


@torch.no_grad()
def ref_paged_forward(model: RefGPT2, alloc: RefAllocator, seqs: list[RefSeq], new_lens=None) -> torch.Tensor:
    """tokquay/generate.py:63-87."""
    lens = new_lens or [s.num_tokens - s.num_cached_tokens for s in seqs]
    batch = RefPagedBatch(alloc.pool, alloc.block_size, [s.block_table for s in seqs],
                          [s.num_cached_tokens for s in seqs], lens)  # fmt: skip
    rows = []
    for s, n in zip(seqs, lens):
        row = s.token_ids[s.num_cached_tokens : s.num_cached_tokens + n]
        rows.append(row + [0] * (batch.T - n))
    ids = torch.tensor(rows, dtype=torch.long, device=alloc.pool.device)
    logits = model(ids, batch, last_only=True)[:, 0]
    for s, n in zip(seqs, lens):
        s.num_cached_tokens += n
    return logits


@torch.no_grad()
def ref_paged_greedy_generate(model: RefGPT2, alloc: RefAllocator, prompts, max_new_tokens: int,
                              margins: list[float] | None = None) -> list[list[int]]:  # fmt: skip
    """tokquay/generate.py:90-120. If ``margins`` is given, appends every step's per-row
    top-1 minus top-2 logit gap (how close the greedy pick was to a tie)."""
    seqs = [RefSeq(p) for p in prompts]
    for s in seqs:
        alloc.allocate(s)
    running = seqs
    while running:
        logits = ref_paged_forward(model, alloc, running)
        if margins is not None:
            top2 = logits.topk(2, dim=-1).values
            margins.extend((top2[:, 0] - top2[:, 1]).tolist())
        nxt = logits.argmax(-1).tolist()
        still = []
        for s, t in zip(running, nxt):
            s.output.append(t)
            if len(s.output) >= max_new_tokens:
                alloc.free(s)
            else:
                alloc.append_slot(s)
                still.append(s)
        running = still
    return [s.output for s in seqs]


@torch.no_grad()
def ref_greedy_generate(model: RefGPT2, prompt: list[int], max_new_tokens: int,
                        margins: list[float] | None = None) -> list[int]:  # fmt: skip
    """Batch-of-one greedy decode on the contiguous cache (tokquay/generate.py:17-49). If
    ``margins`` is given, appends each pick's top-1 minus top-2 logit gap."""
    dtype = next(model.parameters()).dtype
    device = next(model.parameters()).device
    ids = torch.tensor([prompt], device=device)
    cache = RefContiguousKVCache(model.cfg, 1, len(prompt) + max_new_tokens, device=device, dtype=dtype)

    def pick(logits: torch.Tensor) -> torch.Tensor:
        row = logits[:, -1]
        if margins is not None:
            top2 = row[0].topk(2).values
            margins.append(float(top2[0] - top2[1]))
        return row.argmax(-1, keepdim=True)

    nxt = pick(model(ids, cache, last_only=True))
    out = [int(nxt)]
    for _ in range(max_new_tokens - 1):
        nxt = pick(model(nxt, cache, last_only=True))
        out.append(int(nxt))
    return out


def build_ref_model(cfg: RefConfig, state_dict: dict, dtype=torch.float32, device="cpu") -> RefGPT2:
    m = RefGPT2(cfg)
    m.load_state_dict(state_dict)
    return m.to(device=device, dtype=dtype).eval()
