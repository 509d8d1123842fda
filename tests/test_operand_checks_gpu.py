"""The binding refuses device tensors a launch would overrun or misread:
the wrong dtype, too few elements, or a non-contiguous view. Each refusal is
InvalidArgument raised before the launch, so the output stays untouched."""

from __future__ import annotations

import pytest
import torch

import cuvit_amd as cuvit

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _sentinel(n, dtype=torch.float32):
    return torch.full((n,), 7.0, dtype=dtype, device=DEV)


def test_dtype_mismatch_is_refused():
    x = torch.randn(16 * 32, device=DEV)
    out = _sentinel(16 * 32, torch.bfloat16)
    g = torch.ones(32, device=DEV)
    with pytest.raises(cuvit.InvalidArgument, match="out holds torch.bfloat16"):
        cuvit.layer_norm(x, g, g, out, 16, 32)
    with pytest.raises(cuvit.InvalidArgument, match="gamma holds torch.bfloat16"):
        cuvit.layer_norm(x.bfloat16(), g.bfloat16(), g, out, 16, 32)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_short_tensors_are_refused():
    x = torch.randn(10 * 20, device=DEV)
    out = _sentinel(10 * 20 - 1)
    with pytest.raises(cuvit.InvalidArgument, match="out holds 199 elements"):
        cuvit.softmax(x, out, 10, 20)
    a = torch.randn(64 * 32, device=DEV)
    w = torch.randn(48 * 32, device=DEV)
    c = _sentinel(64 * 48 - 48)
    with pytest.raises(cuvit.InvalidArgument, match="C holds"):
        cuvit.gemm(a, w, None, c, cuvit.gemm_problem(64, 48, 32, cuvit.TRANSPOSED))
    p = cuvit.gemm_problem(64, 48, 32, cuvit.TRANSPOSED)
    p.batch.count, p.batch.stride_a, p.batch.stride_b, p.batch.stride_c = 2, 64 * 32, 0, 64 * 48
    with pytest.raises(cuvit.InvalidArgument, match="A holds"):
        cuvit.gemm(a, w, None, _sentinel(2 * 64 * 48), p)
    with pytest.raises(cuvit.InvalidArgument, match="bias holds 47"):
        cuvit.gemm(a, w, torch.zeros(47, device=DEV), _sentinel(64 * 48),
                   cuvit.gemm_problem(64, 48, 32, cuvit.TRANSPOSED))
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())


def test_non_contiguous_views_are_refused():
    x = torch.randn(32, 64, device=DEV).t()
    out = _sentinel(32 * 64)
    with pytest.raises(cuvit.InvalidArgument, match="x is not contiguous"):
        cuvit.softmax(x, out, 64, 32)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_exact_sizes_still_launch():
    """The checks admit a tensor of exactly the touched size, including a
    strided broadcast whose last slot ends the tensor."""
    count, stride, batch = 192, 197 * 192, 3
    dst = torch.zeros((batch - 1) * stride + count, device=DEV)
    src = torch.randn(count, device=DEV)
    cuvit.broadcast(dst, src, count, stride, batch)
    torch.cuda.synchronize()
    assert torch.equal(dst[(batch - 1) * stride:], src)
