"""ops.linear: the decode-step linears through hipBLASLt in whichever weight layout measured faster.

Both layouts compute the same product; the GPU test forces each one and checks it against a
float64 CPU reference, and checks that a row count is measured once and then reused."""

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


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [100, 256])
@pytest.mark.parametrize("gelu", [False, True])
def test_linear_layouts_match_reference(rows, gelu):
    lin = _layer(2304, 768, rows + gelu).cuda()
    x = torch.randn(rows, 768, generator=torch.Generator().manual_seed(rows)).cuda()
    ref = x.double().cpu() @ lin.weight.double().cpu().t() + lin.bias.double().cpu()
    if gelu:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    key = (rows, 2304, 768, gelu)
    saved = ops._gemm_nn.pop(key, None)
    try:
        for nn_layout in (False, True):
            ops._gemm_nn[key] = nn_layout
            got = ops.linear(x, lin, gelu=gelu)
            torch.testing.assert_close(got.double().cpu(), ref, rtol=1e-4, atol=1e-4)
        # A fresh power-of-two row count is measured once and remembered.
        del ops._gemm_nn[key]
        ops.linear(x, lin, gelu=gelu)
        assert (key in ops._gemm_nn) == (rows == 256)
    finally:
        ops._gemm_nn.pop(key, None)
        if saved is not None:
            ops._gemm_nn[key] = saved


@pytest.mark.gpu
def test_transposed_weight_follows_updates():
    lin = _layer(64, 32, 3).cuda()
    t0 = ops.transposed_weight(lin)
    assert torch.equal(t0, lin.weight.t())
    with torch.no_grad():
        lin.weight.add_(1.0)
    t1 = ops.transposed_weight(lin)
    assert torch.equal(t1, lin.weight.t())
