"""Deterministic random-init GPT-2 weights (no checkpoint, no network).

``random_state_dict`` draws every tensor from one counter-based Philox stream
in a fixed order, so the same seed gives bit-identical fp32 weights on every
machine with this numpy. Names and shapes are the reference module's
(tokquay/model.py:59-134, ``nn.Linear`` weights ``[out, in]``), so the dict loads
into this package's ``GPT2`` with ``load_state_dict``.

Default (``all_random=False``): Linear and embedding weights ~ N(0, std^2),
biases 0, LayerNorm gamma 1 / beta 0 - the "random-init, normal std 0.02"
model of the benchmarks. ``all_random=True`` also randomises biases and
LayerNorm parameters, so a test comparing two implementations notices a
dropped bias or LayerNorm term.
"""

from __future__ import annotations

import numpy as np
import torch


def parameter_shapes(cfg) -> list[tuple[str, tuple[int, ...]]]:
    C, V, P = cfg.n_embd, cfg.vocab_size, cfg.n_positions
    shapes = [("wte.weight", (V, C)), ("wpe.weight", (P, C))]
    for i in range(cfg.n_layer):
        p = f"h.{i}."
        shapes += [
            (p + "ln_1.weight", (C,)),
            (p + "ln_1.bias", (C,)),
            (p + "attn.c_attn.weight", (3 * C, C)),
            (p + "attn.c_attn.bias", (3 * C,)),
            (p + "attn.c_proj.weight", (C, C)),
            (p + "attn.c_proj.bias", (C,)),
            (p + "ln_2.weight", (C,)),
            (p + "ln_2.bias", (C,)),
            (p + "mlp.c_fc.weight", (4 * C, C)),
            (p + "mlp.c_fc.bias", (4 * C,)),
            (p + "mlp.c_proj.weight", (C, 4 * C)),
            (p + "mlp.c_proj.bias", (C,)),
        ]
    shapes += [("ln_f.weight", (C,)), ("ln_f.bias", (C,))]
    return shapes


def random_state_dict(cfg, seed: int = 0, std: float = 0.02, all_random: bool = False) -> dict[str, torch.Tensor]:
    rng = np.random.Generator(np.random.Philox(key=seed))
    out: dict[str, torch.Tensor] = {}
    for name, shape in parameter_shapes(cfg):
        is_ln = ".ln_" in name or name.startswith("ln_f")
        if name.endswith(".weight") and not is_ln:
            arr = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
        elif all_random:
            noise = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1 if is_ln else std)
            arr = (noise + np.float32(1.0)) if (is_ln and name.endswith(".weight")) else noise
        else:
            arr = np.ones(shape, np.float32) if (is_ln and name.endswith(".weight")) else np.zeros(shape, np.float32)
        out[name] = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32))
    return out


def hf_state_dict(sd: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The same weights under HuggingFace ``GPT2LMHeadModel`` names (Conv1D weights are ``[in, out]``)."""
    out = {}
    for name, t in sd.items():
        conv = any(name.endswith(f"{m}.weight") for m in ("c_attn", "c_proj", "c_fc"))
        out["transformer." + name] = t.t().contiguous() if conv else t
    out["lm_head.weight"] = sd["wte.weight"]
    return out
