"""GPT-2 forward over the paged pool, with attention on the gfx950 kernels.

Architecture and parameter names follow the reference's hand-written GPT-2
(tokquay/model.py:24-181): pre-LN blocks, fused ``c_attn`` QKV projection,
tanh-approximated GELU, tied LM head, ``nn.Linear`` weights ``[out, in]``.

The paged forward differs in how rows are laid out. The reference runs every
layer on right-padded ``[B, T, C]`` activations and attends through a gathered
copy of each sequence's blocks. Here the input ids are packed to the real
tokens once (``PagedBatch.token_index``), every GEMM / LayerNorm / GELU runs on
``[N, C]`` with ``N = sum(new_lens)``, and attention is ``PagedBatch.attend``:
cache write + paged attention read in place from the pool. Padded positions
are never computed, which is why their logits come back as zeros when
``last_only`` is False.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from tokquay_amd import ops
from tokquay_amd.kv_cache import PagedBatch


@dataclass
class GPT2Config:
    vocab_size: int = 50257
    n_positions: int = 1024
    n_embd: int = 768
    n_layer: int = 12
    n_head: int = 12
    layer_norm_eps: float = 1e-5

    @property
    def d_head(self) -> int:
        return self.n_embd // self.n_head


class Attention(nn.Module):
    def __init__(self, cfg: GPT2Config):
        super().__init__()
        self.c_attn = nn.Linear(cfg.n_embd, 3 * cfg.n_embd)
        self.c_proj = nn.Linear(cfg.n_embd, cfg.n_embd)

    def forward(self, x: torch.Tensor, cache: PagedBatch, layer: int) -> torch.Tensor:
        # x: [N, C] packed rows. c_attn gives [N, 3C] = [q | k | v], heads contiguous in each.
        return ops.linear(cache.attend(layer, ops.linear(x, self.c_attn)), self.c_proj)


class MLP(nn.Module):
    def __init__(self, cfg: GPT2Config):
        super().__init__()
        self.c_fc = nn.Linear(cfg.n_embd, 4 * cfg.n_embd)
        self.c_proj = nn.Linear(4 * cfg.n_embd, cfg.n_embd)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # GELU (tanh form, tokquay/model.py:107) as the GEMM's epilogue on the GPU (hipBLASLt): one launch
        # instead of two. On the CPU torch's fused path computes the erf form, so ops.linear applies it apart.
        return ops.linear(ops.linear(x, self.c_fc, gelu=True), self.c_proj)


class Block(nn.Module):
    def __init__(self, cfg: GPT2Config):
        super().__init__()
        self.ln_1 = nn.LayerNorm(cfg.n_embd, eps=cfg.layer_norm_eps)
        self.attn = Attention(cfg)
        self.ln_2 = nn.LayerNorm(cfg.n_embd, eps=cfg.layer_norm_eps)
        self.mlp = MLP(cfg)

    # Block.forward of the reference (tokquay/model.py:121-123) is GPT2.trunk's loop body here: each
    # residual add runs fused with the LayerNorm after it (tq_add_layernorm).


class GPT2(nn.Module):
    def __init__(self, cfg: GPT2Config | None = None):
        super().__init__()
        self.cfg = cfg or GPT2Config()
        self.wte = nn.Embedding(self.cfg.vocab_size, self.cfg.n_embd)
        self.wpe = nn.Embedding(self.cfg.n_positions, self.cfg.n_embd)
        self.h = nn.ModuleList(Block(self.cfg) for _ in range(self.cfg.n_layer))
        self.ln_f = nn.LayerNorm(self.cfg.n_embd, eps=self.cfg.layer_norm_eps)

    def trunk(self, ids: torch.Tensor | None, positions: torch.Tensor | None, cache,
              embedded: torch.Tensor | None = None) -> torch.Tensor:
        """Final hidden states ``ln_f(x)`` ``[N, C]`` of packed rows (token ids and positions ``[N]``).

        The reference's loop (tokquay/model.py:172-180): embeddings, ``x = x + attn(ln_1(x))``,
        ``x = x + mlp(ln_2(x))`` per block, ``ln_f``. Every residual add runs fused with the
        LayerNorm that follows it (``tq_add_layernorm``); the embedding sum is fused with the
        first ``ln_1``. ``cache`` provides ``attend(layer, qkv)``. ``embedded``: the rows' embedding
        sums ``wte[id] + wpe[pos]`` ``[N, C]`` if already computed (``ops.embed_rows``; ``ids`` and
        ``positions`` are then unused), updated in place as the residual stream."""
        blocks = self.h
        first = blocks[0].ln_1 if len(blocks) else self.ln_f  # no blocks: ln_f on the embeddings
        if embedded is None:
            x, h = ops.add_layernorm(self.wte(ids), self.wpe(positions), first.weight, first.bias, first.eps)
        else:
            x, h = ops.add_layernorm(embedded, None, first.weight, first.bias, first.eps, x_out=embedded)
        for i, block in enumerate(blocks):
            a = block.attn(h, cache, i)
            x, h = ops.add_layernorm(x, a, block.ln_2.weight, block.ln_2.bias, block.ln_2.eps, x_out=x)
            nxt = blocks[i + 1].ln_1 if i + 1 < len(blocks) else self.ln_f
            x, h = ops.add_layernorm(x, block.mlp(h), nxt.weight, nxt.bias, nxt.eps, x_out=x)
        return h

    def skinny_ok(self, rows: int) -> bool:
        """Whether a batch of ``rows`` can run through :meth:`skinny_logits` (at most
        ``ops.SKINNY_MAX_ROWS`` rows; the linears' input widths n_embd and 4 * n_embd must be ones
        ``tq_skinny_linear`` takes)."""
        C = self.cfg.n_embd
        return ops.skinny_supported(rows, C) and ops.skinny_supported(rows, 4 * C)

    def skinny_trunk(self, x: torch.Tensor, cache) -> torch.Tensor:
        """The 12 blocks over ``M <= ops.SKINNY_MAX_ROWS`` rows whose embeddings ``x`` ``[M, C]`` become
        the residual stream (updated in place and returned). The reference's loop (tokquay/model.py:
        172-175) as five launches per block: ``c_attn`` with ``ln_1`` in front, attention, ``c_proj``
        adding into x, ``c_fc`` with ``ln_2`` in front and the GELU after, ``mlp.c_proj`` adding into x
        (``tq_skinny_linear``)."""
        for i, block in enumerate(self.h):
            at, mlp = block.attn, block.mlp
            qkv = ops.skinny_linear(x, at.c_attn.weight, at.c_attn.bias,
                                    ln=(block.ln_1.weight, block.ln_1.bias, block.ln_1.eps))  # fmt: skip
            a = cache.attend(i, qkv)
            ops.skinny_linear(a, at.c_proj.weight, at.c_proj.bias, epilogue="residual", out=x)
            h = ops.skinny_linear(x, mlp.c_fc.weight, mlp.c_fc.bias, ln=(block.ln_2.weight, block.ln_2.bias,
                                                                        block.ln_2.eps), epilogue="gelu")  # fmt: skip
            ops.skinny_linear(h, mlp.c_proj.weight, mlp.c_proj.bias, epilogue="residual", out=x)
        return x

    def skinny_logits(self, x: torch.Tensor, cache) -> torch.Tensor:
        """Logits ``[M, vocab]`` of ``M <= ops.SKINNY_MAX_ROWS`` rows from their embeddings ``x``
        (:meth:`skinny_trunk`), then the tied LM head with ``ln_f`` in front (tokquay/model.py:180-181),
        fused up to ``ops.SKINNY_LM_HEAD_MAX_ROWS`` rows, else ``ln_f`` on its own and the head on
        hipBLASLt."""
        x = self.skinny_trunk(x, cache)
        if x.shape[0] <= ops.SKINNY_LM_HEAD_MAX_ROWS:
            return ops.skinny_linear(x, self.wte.weight, None, ln=(self.ln_f.weight, self.ln_f.bias, self.ln_f.eps))
        _, h = ops.add_layernorm(x, None, self.ln_f.weight, self.ln_f.bias, self.ln_f.eps, x_out=x)
        return h @ self.wte.weight.T

    def skinny_greedy(self, x: torch.Tensor, cache, out: torch.Tensor) -> torch.Tensor:
        """Greedy ids ``[M]`` of ``M <= ops.SKINNY_LM_HEAD_MAX_ROWS`` rows into ``out`` without logits:
        :meth:`skinny_trunk`, then ``ln_f``, the tied LM head and the argmax in one launch
        (``tq_skinny_linear_argmax``; tokquay/model.py:180-181, tokquay/engine.py:190)."""
        x = self.skinny_trunk(x, cache)
        return ops.skinny_linear_argmax(x, self.wte.weight, None, ln=(self.ln_f.weight, self.ln_f.bias,
                                                                      self.ln_f.eps), out=out)  # fmt: skip

    def forward(self, input_ids: torch.Tensor, cache: PagedBatch, last_only: bool = False) -> torch.Tensor:
        """input_ids ``[B, T]`` (new tokens, right-padded) -> logits ``[B, T, vocab]``, or ``[B, 1, vocab]``
        of each row's last real token when ``last_only``. Validation follows tokquay/model.py:154-160."""
        if not isinstance(cache, PagedBatch):
            raise TypeError("this GPT-2 runs only on the paged pool: pass a PagedBatch")
        B, T = input_ids.shape
        if (B, T) != (cache.B, cache.T):
            raise ValueError(f"input_ids {tuple(input_ids.shape)} does not match batch {(cache.B, cache.T)}")
        if cache.max_ctx > self.cfg.n_positions:
            raise ValueError(f"sequence length {cache.max_ctx} exceeds n_positions={self.cfg.n_positions}")

        ids = input_ids.reshape(-1).index_select(0, cache.token_index)  # [N] real tokens only
        h = self.trunk(ids, cache.packed_positions, cache)  # positions of real tokens are < n_positions
        if last_only:
            return (h.index_select(0, cache.last_rows) @ self.wte.weight.T)[:, None]  # tied LM head, [B, 1, V]
        logits = h @ self.wte.weight.T  # [N, vocab]
        full = logits.new_zeros(B * T, logits.size(-1))
        full[cache.token_index] = logits
        return full.view(B, T, -1)
