"""``torch.ops.tokquay_amd.*`` on the GPU refuse malformed tensors before any launch.

Every case of ``tests/torch_op_cases.py`` marked ``gpu_safe`` (each stays inside memory its
tensors own even if a check were missing) must raise the operator's own error; the
well-formed arguments run, leave the error word clear, and the device is still healthy
afterwards.
"""

from __future__ import annotations

import pytest
import torch

from tests.torch_op_cases import SIGS, base_args, cases, positional
from tokquay_amd import ops, torch_ops

pytestmark = pytest.mark.gpu


def workspace_bytes(op: str) -> int:
    if op in ("paged_decode", "paged_decode_write"):
        return max(16, ops.decode_workspace_bytes(3, 2, 16))
    if op == "paged_mixed":
        return max(16, ops.mixed_workspace_bytes(3, 2, 16, 0, 2, 7, 4))
    return 16


@pytest.mark.parametrize("op", list(SIGS))
def test_well_formed_arguments_run(op):
    args = base_args(op, "cuda", workspace_bytes)
    getattr(torch_ops.load(), op)(*positional(op, args))
    torch.cuda.synchronize()
    if "d_error" in args:
        assert int(args["d_error"].item()) == 0


@pytest.mark.parametrize("case", [c for c in cases() if c.gpu_safe], ids=lambda c: c.id)
def test_spoiled_arguments_are_refused_before_a_launch(case):
    print(f"\n{case.id}", flush=True)
    args = base_args(case.op, "cuda", workspace_bytes)
    args[case.arg] = case.spoil(args[case.arg])
    with pytest.raises(RuntimeError, match=f"tokquay_amd::{case.op}: "):
        getattr(torch_ops.load(), case.op)(*positional(case.op, args))
    torch.cuda.synchronize()
    if "d_error" in args and case.arg != "d_error":
        assert int(args["d_error"].item()) == 0  # nothing ran
