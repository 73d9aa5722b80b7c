"""The entry points as torch operators (torch.ops.tokquay_amd.*): registered with their schemas, and
recorded as single operators when a torch program is traced (fake tensors, no GPU needed).

The GPU tests reach the same operators through ``tokquay_amd.ops``, which calls them."""

from __future__ import annotations

import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from tokquay_amd import torch_ops


def test_every_operator_is_registered_with_its_mutations():
    ops = torch_ops.load()
    schemas = {name: str(getattr(ops, name).default._schema) for name in torch_ops.OPS}
    assert "Tensor(a!) pool" in schemas["cache_write"]
    assert "Tensor(a!) out" in schemas["paged_decode"] and "Tensor pool" in schemas["paged_decode"]
    assert "Tensor(b!) pool" in schemas["paged_decode_write"]
    assert "Tensor(a!) out" in schemas["paged_prefill"] and "Tensor pool" in schemas["paged_prefill"]
    assert "Tensor(a!) dec_out" in schemas["paged_mixed"] and "Tensor(b!) pre_out" in schemas["paged_mixed"]
    assert "Tensor(c!) pool" in schemas["paged_mixed"]
    assert "Tensor(a!) k_out" in schemas["paged_gather"] and "Tensor(b!) v_out" in schemas["paged_gather"]
    assert "Tensor(a!) out" in schemas["argmax_rows"]
    for s in schemas.values():
        assert s.endswith("-> ()")


def test_a_traced_decode_layer_records_the_kernels_as_operators():
    torch_ops.load()

    def layer(qkv, pool, tables, ctx, logits, ids):
        out = torch.empty(qkv.shape[0], 768, device=qkv.device)
        q, k, v = qkv[:, :768], qkv[:, 768:1536], qkv[:, 1536:]
        torch.ops.tokquay_amd.paged_decode_write(out, q, k, v, pool, 0, tables, ctx, 256, 0.125, 0, None, None, None)
        torch.ops.tokquay_amd.argmax_rows(logits, ids)
        return out.sum(), ids

    with FakeTensorMode():
        args = (torch.empty(4, 3 * 768, device="cuda"), torch.empty(16, 1, 2, 12, 16, 64, device="cuda"),
                torch.zeros(4, 16, dtype=torch.int32, device="cuda"), torch.zeros(4, dtype=torch.int32, device="cuda"),
                torch.empty(4, 50257, device="cuda"), torch.empty(4, dtype=torch.int64, device="cuda"))  # fmt: skip
        graph = make_fx(layer)(*args)
    targets = [str(n.target) for n in graph.graph.nodes if n.op == "call_function"]
    assert "tokquay_amd.paged_decode_write.default" in targets
    assert "tokquay_amd.argmax_rows.default" in targets


# ---- argument checks: the fakes refuse what the operators refuse (tests/torch_op_cases.py)

import pytest  # noqa: E402

from tests.torch_op_cases import SIGS, base_args, cases, positional  # noqa: E402


@pytest.mark.parametrize("op", list(SIGS))
def test_fake_accepts_well_formed_arguments(op):
    ops = torch_ops.load()
    with FakeTensorMode():
        getattr(ops, op)(*positional(op, base_args(op, "cuda")))


@pytest.mark.parametrize("case", cases(), ids=lambda c: c.id)
def test_fake_refuses_spoiled_arguments(case):
    ops = torch_ops.load()
    with FakeTensorMode():
        args = base_args(case.op, "cuda")
        args[case.arg] = case.spoil(args[case.arg])
        with pytest.raises(RuntimeError, match=f"tokquay_amd::{case.op}: "):
            getattr(ops, case.op)(*positional(case.op, args))


def test_spoiled_cases_cover_every_tensor_argument():
    spoiled = {(c.op, c.arg) for c in cases()}
    for op, names in SIGS.items():
        for a in names:
            if a not in ("max_context_len", "max_query_len", "scale", "partition_tokens"):
                assert (op, a) in spoiled, (op, a)


def test_workspace_is_declared_written():
    ops = torch_ops.load()
    for op in ("paged_decode", "paged_decode_write", "paged_mixed"):
        schema = str(getattr(ops, op).default._schema)
        assert "!)? workspace" in schema, schema
