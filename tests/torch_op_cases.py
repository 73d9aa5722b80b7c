"""Well-formed arguments for every ``torch.ops.tokquay_amd`` operator, and ways to spoil them.

Each spoiled case breaks one argument in a way the operator must refuse before any launch:
too few rows or entries, a wrong dtype, rows that are not contiguous inside or that overlap,
the wrong width, a layer out of range, a tensor on another device. A case marked ``gpu_safe``
stays inside memory the tensors own even if the check were missing (a short view of a longer
tensor, a wider dtype), so it may be tried on a GPU; the others (host tensors) are checked
only against the fake implementations.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

SIGS = {
    "cache_write": ["pool", "layer", "k", "v", "slot_mapping", "d_error"],
    "paged_decode": ["out", "q", "pool", "layer", "block_tables", "context_lens", "max_context_len", "scale",
                     "partition_tokens", "workspace", "d_error", "seq_order"],
    "paged_decode_write": ["out", "q", "k_new", "v_new", "pool", "layer", "block_tables", "context_lens",
                           "max_context_len", "scale", "partition_tokens", "workspace", "d_error", "seq_order"],
    "paged_prefill": ["out", "q", "pool", "layer", "block_tables", "cu_seqlens_q", "q_start", "max_query_len", "scale",
                      "d_error", "seq_order"],
    "paged_mixed": ["dec_out", "dec_q", "k_new", "v_new", "dec_block_tables", "context_lens", "max_context_len",
                    "pre_out", "pre_q", "pre_block_tables", "cu_seqlens_q", "q_start", "max_query_len", "pool", "layer",
                    "scale", "partition_tokens", "workspace", "d_error", "seq_order"],
    "paged_gather": ["k_out", "v_out", "pool", "layer", "block_tables", "d_error"],
    "argmax_rows": ["logits", "out"],
}  # fmt: skip

NB, L, H, BS, D = 8, 2, 2, 4, 64
W = H * D
ROW_ARGS = {"k", "v", "out", "q", "k_new", "v_new", "dec_out", "dec_q", "pre_out", "pre_q"}
TABLE_ARGS = {"block_tables", "dec_block_tables", "pre_block_tables"}
INT_ARGS = {"slot_mapping": torch.int64, "context_lens": torch.int32, "seq_order": torch.int32,
            "cu_seqlens_q": torch.int32, "q_start": torch.int32, "d_error": torch.int32}  # fmt: skip
# Integer arguments whose length is checked against another (the others define it).
COUNTED = {"seq_order", "cu_seqlens_q", "d_error"}


def base_args(op: str, device, workspace_bytes: Callable[[str], int] = lambda op: 4096) -> dict:
    """Well-formed arguments with valid contents: 3 decode sequences of context 16, 6 and 1;
    2 prefill sequences of 3 rows at position 0 and 4 rows at position 2; 5 cache-write rows."""
    def f(*shape):
        return torch.randn(*shape, device=device)

    def i32(vals):
        return torch.tensor(vals, dtype=torch.int32, device=device)

    pool = torch.randn(NB, L, 2, H, BS, D, device=device)
    dec = dict(block_tables=i32([[3, 1, 4, 0], [5, 2, 0, 0], [7, 0, 0, 0]]), context_lens=i32([16, 6, 1]),
               max_context_len=16, seq_order=i32([0, 1, 2]))  # fmt: skip
    pre = dict(block_tables=i32([[6, 0], [2, 5]]), cu_seqlens_q=i32([0, 3, 7]), q_start=i32([0, 2]), max_query_len=4)
    common = dict(pool=pool, layer=1, scale=0.125, partition_tokens=0,
                  d_error=torch.zeros(1, dtype=torch.int32, device=device))  # fmt: skip
    ws = dict(workspace=torch.zeros(workspace_bytes(op), dtype=torch.uint8, device=device))
    if op == "cache_write":
        a = dict(common, k=f(5, H, D), v=f(5, W),
                 slot_mapping=torch.tensor([0, 5, 31, -1, 9], dtype=torch.int64, device=device))
    elif op == "paged_decode":
        a = dict(common, **dec, **ws, out=f(3, W), q=f(3, H, D))
    elif op == "paged_decode_write":
        a = dict(common, **dec, **ws, out=f(3, W), q=f(3, H, D), k_new=f(3, W), v_new=f(3, H, D))
    elif op == "paged_prefill":
        a = dict(common, **pre, out=f(7, W), q=f(7, H, D), seq_order=i32([1, 0]))
    elif op == "paged_mixed":
        a = dict(common, **ws, dec_out=f(3, W), dec_q=f(3, H, D), k_new=f(3, W), v_new=f(3, W),
                 dec_block_tables=dec["block_tables"], context_lens=dec["context_lens"],
                 max_context_len=dec["max_context_len"], seq_order=dec["seq_order"], pre_out=f(7, W), pre_q=f(7, W),
                 pre_block_tables=pre["block_tables"], cu_seqlens_q=pre["cu_seqlens_q"], q_start=pre["q_start"],
                 max_query_len=pre["max_query_len"])  # fmt: skip
    elif op == "paged_gather":
        a = dict(common, block_tables=dec["block_tables"], k_out=f(3, H, 4 * BS, D), v_out=f(3, H, 4 * BS, D))
    elif op == "argmax_rows":
        a = dict(logits=f(3, 50), out=torch.zeros(3, dtype=torch.int64, device=device))
    else:
        raise KeyError(op)
    return {k: v for k, v in a.items() if k in SIGS[op]}


def positional(op: str, args: dict) -> list:
    return [args[k] for k in SIGS[op]]


@dataclass
class Spoiled:
    op: str
    arg: str
    how: str
    spoil: Callable[[torch.Tensor], object]
    gpu_safe: bool = True

    @property
    def id(self) -> str:
        return f"{self.op}-{self.arg}-{self.how}"


def _strided_inner(t):  # same shape, every other element of a tensor twice as wide
    return torch.zeros(*t.shape[:-1], 2 * t.shape[-1], dtype=t.dtype, device=t.device)[..., ::2]


def _strided_vector(t):  # every other entry of a buffer twice as long (at least 2 entries, so not contiguous)
    n = max(t.numel(), 2)
    return torch.zeros(2 * n, dtype=t.dtype, device=t.device)[::2]


def _overlapping(t):  # a 2-D t's shape with rows half a row apart, inside a buffer as long as t
    return torch.zeros(t.numel(), dtype=t.dtype, device=t.device).as_strided(t.shape, (t.size(1) // 2, 1))


def cases() -> list[Spoiled]:
    out = [Spoiled("argmax_rows", "logits", "float64", lambda t: t.double()),
           Spoiled("argmax_rows", "logits", "strided_inner", _strided_inner),
           Spoiled("argmax_rows", "logits", "overlap", _overlapping),
           Spoiled("argmax_rows", "out", "fewer", lambda t: t[:-1]),
           Spoiled("argmax_rows", "out", "int32",
                   lambda t: torch.zeros(2 * t.numel(), dtype=torch.int32, device=t.device)[: t.numel()]),
           Spoiled("argmax_rows", "out", "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
    for op, names in SIGS.items():
        if op == "argmax_rows":
            continue
        for a in names:
            if a in ROW_ARGS:
                # A prefill q's row count is the call's row total, so it has no "fewer rows" (a
                # cu_seqlens_q past it is caught by the kernels, through d_error).
                if (op, a) not in (("paged_prefill", "q"), ("paged_mixed", "pre_q")):
                    out.append(Spoiled(op, a, "fewer_rows", lambda t: t[:-1]))
                out += [Spoiled(op, a, "float64", lambda t: t.double()),
                        Spoiled(op, a, "strided_inner", _strided_inner),
                        Spoiled(op, a, "narrow", lambda t: t[:, :1]),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
            elif a in TABLE_ARGS:
                out += [Spoiled(op, a, "fewer_rows", lambda t: t[:-1]),
                        Spoiled(op, a, "int64", lambda t: t.long()),
                        Spoiled(op, a, "strided_inner", _strided_inner),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
            elif a in INT_ARGS:
                if INT_ARGS[a] == torch.int32:
                    out.append(Spoiled(op, a, "int64", lambda t: t.long()))
                else:  # an int32 view as long as the int64 original, in bytes
                    out.append(Spoiled(op, a, "int32", lambda t: torch.zeros(2 * t.numel(), dtype=torch.int32,
                                                                              device=t.device)[: t.numel()]))
                out += [Spoiled(op, a, "strided", _strided_vector),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
                if a in COUNTED:
                    out.append(Spoiled(op, a, "fewer", lambda t: t[:-1]))
            elif a == "pool":
                out += [Spoiled(op, a, "float64", lambda t: t.double()),
                        Spoiled(op, a, "strided", lambda t: torch.zeros(t.size(0), t.size(1) + 1, *t.shape[2:],
                                                                         device=t.device)[:, : t.size(1)]),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
            elif a == "layer":
                out += [Spoiled(op, a, "past_end", lambda v: L), Spoiled(op, a, "negative", lambda v: -1)]
            elif a == "workspace":
                out += [Spoiled(op, a, "strided", _strided_vector),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
            elif a in ("k_out", "v_out"):
                out += [Spoiled(op, a, "fewer_rows", lambda t: t[:-1]),
                        Spoiled(op, a, "float64", lambda t: t.double()),
                        Spoiled(op, a, "host", lambda t: t.cpu(), gpu_safe=False)]  # fmt: skip
    # Overlapping rows of a row tensor (one case per operator: the check is shared).
    for op, a in (("cache_write", "k"), ("paged_decode", "out"), ("paged_prefill", "q"), ("paged_mixed", "pre_out"),
                  ("paged_decode_write", "v_new")):  # fmt: skip
        out.append(Spoiled(op, a, "overlap", lambda t: _overlapping(t.reshape(t.size(0), -1))))
    return out
