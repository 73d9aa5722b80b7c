"""ops.linear: the decode-step linears through hipBLASLt, in the weight layout a fixed table names.

Both layouts compute the same product; the GPU test forces each one, checks it against a float64
CPU reference and reports whether the two round alike."""

from __future__ import annotations

import pytest
import torch

from tokquay_amd import ops


def _layer(out_f: int, in_f: int, seed: int) -> torch.nn.Linear:
    torch.manual_seed(seed)
    lin = torch.nn.Linear(in_f, out_f)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
        lin.bias.normal_(0, 0.02)
    return lin


def test_linear_cpu_is_torch_linear():
    lin = _layer(96, 64, 0)
    x = torch.randn(5, 64)
    assert torch.equal(ops.linear(x, lin), torch.nn.functional.linear(x, lin.weight, lin.bias))
    want = torch.nn.functional.gelu(torch.nn.functional.linear(x, lin.weight, lin.bias), approximate="tanh")
    assert torch.equal(ops.linear(x, lin, gelu=True), want)


def test_layout_table_is_fixed():
    """The layout is a committed table, not a per-process measurement: only the two 768-wide-input
    projections at the 256-row decode bucket use the transposed weight."""
    assert ops.uses_nn_layout(256, 2304, 768, False) and ops.uses_nn_layout(256, 3072, 768, True)
    for shape in ((128, 2304, 768, False), (256, 768, 3072, False), (256, 2304, 768, True), (320, 3072, 768, True)):
        assert not ops.uses_nn_layout(*shape)


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [100, 256])
@pytest.mark.parametrize("gelu", [False, True])
def test_linear_layouts_match_reference(rows, gelu, monkeypatch):
    lin = _layer(2304, 768, rows + gelu).cuda()
    x = torch.randn(rows, 768, generator=torch.Generator().manual_seed(rows)).cuda()
    ref = x.double().cpu() @ lin.weight.double().cpu().t() + lin.bias.double().cpu()
    if gelu:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    key = (rows, 2304, 768, gelu)
    outs = []
    for table in (frozenset(), frozenset({key})):  # stored layout, then the transposed copy
        monkeypatch.setattr(ops, "GEMM_NN_SHAPES", table)
        got = ops.linear(x, lin, gelu=gelu)
        torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4)
        outs.append(got)
    # Repeated calls in one layout give the same bits; whether the two layouts do is reported.
    assert torch.equal(ops.linear(x, lin, gelu=gelu), outs[1])
    print(f"rows {rows} gelu {gelu}: TN and NN bit-identical: {torch.equal(outs[0], outs[1])}, "
          f"max |diff| {float((outs[0] - outs[1]).abs().max()):.3e}")


@pytest.mark.gpu
def test_transposed_weight_follows_updates():
    lin = _layer(64, 32, 3).cuda()
    t0 = ops.transposed_weight(lin)
    assert torch.equal(t0, lin.weight.t())
    with torch.no_grad():
        lin.weight.add_(1.0)
    t1 = ops.transposed_weight(lin)
    assert torch.equal(t1, lin.weight.t())
