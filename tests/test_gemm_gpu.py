"""GPU parity for the batched GEMM and its epilogues.

Mirrors the reference's tests/gemm_test.cu: every ViT-Tiny shape in both
layouts with and without bias (term-scaled comparison, rtol = atol = 1e-6),
alpha, batched strides, a zero stride, the accumulate and GELU epilogues and
their order, degenerate problems and K = 0. Added: the split (image, head)
batch the attention GEMMs use, unaligned leading dimensions, the ViT-Tiny
batch-32 shapes, and tile independence (a row's bits do not depend on M).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import workloads as W
from conftest import to_device, to_host
from numerics import TestFailure, compare_close, require_close, require_close_scaled, \
    require_exact

pytestmark = pytest.mark.gpu

NT, T = 0, 1


def run(cuvit, a, b, bias, m, n, k, layout, alpha, device, **extra):
    da, db = to_device(a, device), to_device(b, device)
    dbias = None if bias is None else to_device(bias, device)
    dc = torch.empty(m * n, device=device)
    problem = cuvit.gemm_problem(m, n, k, layout)
    problem.alpha = alpha
    for key, value in extra.items():
        setattr(problem, key, value)
    cuvit.gemm(da, db, dbias, dc, problem)
    return to_host(dc).reshape(m, n)


def check_case(cuvit, oracle, device, m, n, k, label, layout, with_bias, alpha):
    """gemm_test.cu:53-88."""
    g = oracle.generator(m * 31 + n * 7 + k)
    a = g.normal(m * k)
    b = g.normal(k * n)
    bias = g.normal(n)
    if layout == T:
        expected = oracle.gemm_transposed(a, b, bias if with_bias else None, m, n, k, alpha)
    else:
        expected = oracle.gemm(a, b, bias if with_bias else None, m, n, k, alpha)
    actual = run(cuvit, a, b, bias if with_bias else None, m, n, k, layout, alpha, device)
    scale = oracle.term_magnitudes(a, b, m, n, k, layout == T, alpha)
    require_close_scaled(actual, expected, scale, label, 1.0e-6, 1.0e-6)


CASES = [
    (1, 1, 1, "1x1x1"),
    (1, 1000, 192, "classifier head"),
    (17, 33, 7, "small odd"),
    (63, 63, 63, "just under one tile"),
    (64, 64, 64, "exactly one tile"),
    (65, 65, 65, "just over one tile"),
    (197, 576, 192, "qkv projection"),
    (197, 192, 192, "attention output projection"),
    (197, 768, 192, "mlp fc1"),
    (197, 192, 768, "mlp fc2"),
    (197, 197, 64, "attention logits"),
    (197, 64, 197, "attention times values"),
    # beyond the reference: the 128-wide tile and its edges
    (300, 257, 129, "tall odd"),
    (1024, 256, 64, "tall tile"),
]


@pytest.mark.parametrize("m,n,k,label", CASES)
@pytest.mark.parametrize("layout", [NT, T])
@pytest.mark.parametrize("with_bias", [False, True])
def test_shapes_and_layouts(cuvit, oracle, device, m, n, k, label, layout, with_bias):
    check_case(cuvit, oracle, device, m, n, k, label, layout, with_bias, 1.0)


def test_alpha_scales_the_product(cuvit, oracle, device):
    """gemm_test.cu:116-120."""
    check_case(cuvit, oracle, device, 197, 197, 64, "scaled attention logits", T, False, 0.125)
    check_case(cuvit, oracle, device, 32, 48, 16, "negative scale", NT, True, -2.5)


def test_batched_strides(cuvit, oracle, device):
    """gemm_test.cu:122-171: one GEMM per head by batch stride."""
    heads, tokens, head_dim = 3, 197, 64
    per_in, per_out = tokens * head_dim, tokens * tokens
    g = oracle.generator(2024)
    q = g.normal(per_in * heads)
    k = g.normal(per_in * heads)
    dc = torch.empty(per_out * heads, device=device)
    problem = cuvit.gemm_problem(tokens, tokens, head_dim, T)
    problem.alpha = 0.125
    problem.batch.count = heads
    problem.batch.stride_a = per_in
    problem.batch.stride_b = per_in
    problem.batch.stride_c = per_out
    cuvit.gemm(to_device(q, device), to_device(k, device), None, dc, problem)
    actual = to_host(dc)
    for h in range(heads):
        qh, kh = q[h * per_in:(h + 1) * per_in], k[h * per_in:(h + 1) * per_in]
        expected = oracle.gemm_transposed(qh, kh, None, tokens, tokens, head_dim, 0.125)
        scale = oracle.term_magnitudes(qh, kh, tokens, tokens, head_dim, True, 0.125)
        require_close_scaled(actual[h * per_out:(h + 1) * per_out], expected, scale,
                             "batched attention logits", 1.0e-6, 1.0e-6)


def test_zero_stride_shares_an_operand(cuvit, oracle, device):
    """gemm_test.cu:173-214."""
    batch, m, n, k = 4, 40, 24, 32
    g = oracle.generator(77)
    a = g.normal(batch * m * k)
    b = g.normal(k * n)
    dc = torch.empty(batch * m * n, device=device)
    problem = cuvit.gemm_problem(m, n, k, NT)
    problem.batch.count = batch
    problem.batch.stride_a = m * k
    problem.batch.stride_b = 0
    problem.batch.stride_c = m * n
    cuvit.gemm(to_device(a, device), to_device(b, device), None, dc, problem)
    actual = to_host(dc)
    for i in range(batch):
        sl = a[i * m * k:(i + 1) * m * k]
        expected = oracle.gemm(sl, b, None, m, n, k)
        scale = oracle.term_magnitudes(sl, b, m, n, k, False)
        require_close_scaled(actual[i * m * n:(i + 1) * m * n], expected, scale,
                             "shared weight across a batch", 1.0e-6, 1.0e-6)


def test_accumulate_epilogue_adds_into_the_destination(cuvit, oracle, device):
    """gemm_test.cu:219-274."""
    m, n, k = 70, 40, 24
    g = oracle.generator(404)
    a, b, bias, existing = g.normal(m * k), g.normal(k * n), g.normal(n), g.normal(m * n)
    product = oracle.gemm(a, b, bias, m, n, k)
    expected = existing + product.reshape(-1)
    da, db, dbias = to_device(a, device), to_device(b, device), to_device(bias, device)
    dc = to_device(existing, device)
    problem = cuvit.gemm_problem(m, n, k, NT)
    problem.epilogue.accumulate = 1
    cuvit.gemm(da, db, dbias, dc, problem)
    scale = oracle.term_magnitudes(a, b, m, n, k, False).reshape(-1)
    require_close_scaled(to_host(dc), expected, scale, "accumulate epilogue", 1.0e-6, 1.0e-5)

    dc = to_device(existing, device)
    cuvit.gemm(da, db, dbias, dc, cuvit.gemm_problem(m, n, k, NT))
    require_close_scaled(to_host(dc), product.reshape(-1), scale, "default epilogue overwrites",
                         1.0e-6, 1.0e-5)


def test_gelu_epilogue_matches_the_standalone_kernel(cuvit, oracle, device):
    """gemm_test.cu:276-324, including that the wrong order is distinguishable."""
    m, n, k = 33, 96, 48
    g = oracle.generator(505)
    a, b, bias = g.normal(m * k), g.normal(k * n), g.normal(n)
    expected = oracle.gelu(oracle.gemm(a, b, bias, m, n, k))
    problem_fields = {}
    da, db, dbias = to_device(a, device), to_device(b, device), to_device(bias, device)
    dc = torch.empty(m * n, device=device)
    problem = cuvit.gemm_problem(m, n, k, NT)
    problem.epilogue.gelu = 1
    cuvit.gemm(da, db, dbias, dc, problem, **problem_fields)
    actual = to_host(dc).reshape(m, n)
    require_close(actual, expected, "GELU epilogue", 1.0e-4, 1.0e-5)

    wrong = oracle.gelu(oracle.gemm(a, b, None, m, n, k)) + bias[None, :]
    if compare_close(actual, wrong, 1.0e-3, 1.0e-3):
        raise TestFailure("the GELU epilogue applied the bias in the wrong order")


def test_epilogue_order_with_accumulate_and_gelu(cuvit, oracle, device):
    """alpha -> bias -> GELU -> accumulate, all at once (gemm.cu:153-162)."""
    m, n, k = 45, 70, 33
    g = oracle.generator(606)
    a, b, bias, existing = g.normal(m * k), g.normal(n * k), g.normal(n), g.normal(m * n)
    expected = existing.copy()
    oracle.gemm_problem_run(a, b, bias, expected, m=m, n=n, k=k, layout=T, alpha=0.75,
                            accumulate=1, gelu=1)
    dc = to_device(existing, device)
    problem = cuvit.gemm_problem(m, n, k, T)
    problem.alpha = 0.75
    problem.epilogue.accumulate = 1
    problem.epilogue.gelu = 1
    cuvit.gemm(to_device(a, device), to_device(b, device), to_device(bias, device), dc, problem)
    require_close(to_host(dc), expected, "combined epilogue", 1.0e-4, 1.0e-5)


def test_split_batch_attention_layout(cuvit, oracle, device):
    """The model's Q.K^T and weights.V: split (image, head) batches over the
    packed [tokens, 3 * embed] projection (vit.cu:210-242)."""
    images, heads, tokens, head_dim = 3, 3, 197, 64
    embed = heads * head_dim
    row = 3 * embed
    g = oracle.generator(8080)
    qkv = g.normal(images * tokens * row)
    logits_fields = dict(m=tokens, n=tokens, k=head_dim, layout=T, alpha=0.125, lda=row, ldb=row,
                         ldc=tokens, count=images * heads, inner=heads, stride_a=head_dim,
                         stride_b=head_dim, stride_c=tokens * tokens,
                         outer_stride_a=tokens * row, outer_stride_b=tokens * row,
                         outer_stride_c=heads * tokens * tokens)
    expected = np.zeros(images * heads * tokens * tokens, np.float32)
    oracle.gemm_problem_run(qkv, qkv[embed:], None, expected, **logits_fields)

    dqkv = to_device(qkv, device)
    dl = torch.zeros(expected.size, device=device)
    problem = cuvit.gemm_problem(tokens, tokens, head_dim, T)
    for key in ("alpha", "lda", "ldb", "ldc"):
        setattr(problem, key, logits_fields[key])
    for key in ("count", "inner", "stride_a", "stride_b", "stride_c", "outer_stride_a",
                "outer_stride_b", "outer_stride_c"):
        setattr(problem.batch, key, logits_fields[key])
    cuvit.gemm(dqkv, dqkv[embed:], None, dl, problem)
    actual = to_host(dl)
    # term scale per entry: |q|.|k| summed, from the oracle on absolute values
    scale = np.zeros_like(expected)
    oracle.gemm_problem_run(np.abs(qkv), np.abs(qkv[embed:]), None, scale,
                            **dict(logits_fields, alpha=0.125))
    require_close_scaled(actual, expected, scale, "split-batch logits", 1.0e-6, 1.0e-6)

    # weights.V with an unaligned lda of 197 (the scalar A path)
    weights = oracle.softmax(expected.reshape(-1, tokens)).reshape(-1)
    context_fields = dict(m=tokens, n=head_dim, k=tokens, layout=NT, lda=tokens, ldb=row,
                          ldc=embed, count=images * heads, inner=heads,
                          stride_a=tokens * tokens, stride_b=head_dim, stride_c=head_dim,
                          outer_stride_a=heads * tokens * tokens, outer_stride_b=tokens * row,
                          outer_stride_c=tokens * embed)
    expected_ctx = np.zeros(images * tokens * embed, np.float32)
    oracle.gemm_problem_run(weights, qkv[2 * embed:], None, expected_ctx, **context_fields)
    scale_ctx = np.zeros_like(expected_ctx)
    oracle.gemm_problem_run(np.abs(weights), np.abs(qkv[2 * embed:]), None, scale_ctx,
                            **context_fields)
    dctx = torch.zeros(expected_ctx.size, device=device)
    problem = cuvit.gemm_problem(tokens, head_dim, tokens, NT)
    for key in ("lda", "ldb", "ldc"):
        setattr(problem, key, context_fields[key])
    for key in ("count", "inner", "stride_a", "stride_b", "stride_c", "outer_stride_a",
                "outer_stride_b", "outer_stride_c"):
        setattr(problem.batch, key, context_fields[key])
    cuvit.gemm(to_device(weights, device), dqkv[2 * embed:], None, dctx, problem)
    require_close_scaled(to_host(dctx), expected_ctx, scale_ctx, "split-batch context",
                         1.0e-6, 1.0e-6)


def test_rows_do_not_depend_on_the_problem_height(cuvit, oracle, device):
    """Batch invariance: the same rows computed inside a tall problem (128-wide
    tile) and alone (64-wide tile) are bitwise equal."""
    n, k = 192, 768
    g = oracle.generator(9090)
    a = g.normal(6304 * k)
    w = g.normal(n * k)
    bias = g.normal(n)
    dw, dbias = to_device(w, device), to_device(bias, device)
    tall = torch.empty(6304 * n, device=device)
    p = cuvit.gemm_problem(6304, n, k, T)
    cuvit.gemm(to_device(a, device), dw, dbias, tall, p)
    full = to_host(tall).reshape(6304, n)
    for start, rows in ((0, 197), (197, 197), (4000, 3), (6303, 1)):
        piece = torch.empty(rows * n, device=device)
        cuvit.gemm(to_device(a[start * k:(start + rows) * k], device), dw, dbias, piece,
                   cuvit.gemm_problem(rows, n, k, T))
        require_exact(to_host(piece).reshape(rows, n), full[start:start + rows],
                      f"rows {start}..{start + rows} changed with the problem height")


def test_degenerate_and_invalid_arguments(cuvit, device):
    """gemm_test.cu:326-354."""
    buffer = torch.zeros(16, device=device)
    cuvit.gemm(buffer, buffer, None, buffer, cuvit.gemm_problem(0, 4, 4, NT))
    cuvit.gemm(buffer, buffer, None, buffer, cuvit.gemm_problem(4, 0, 4, NT))
    torch.cuda.synchronize()
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.gemm(None, buffer, None, buffer, cuvit.gemm_problem(4, 4, 4, NT))
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.gemm(buffer, buffer, None, buffer, cuvit.gemm_problem(-1, 4, 4, NT))


def test_zero_k_produces_the_bias(cuvit, oracle, device):
    """gemm_test.cu:356-379."""
    m = n = 8
    bias = oracle.generator(5).normal(n)
    a = torch.zeros(1, device=device)
    b = torch.zeros(1, device=device)
    c = torch.full((m * n,), 7.0, device=device)
    cuvit.gemm(a, b, to_device(bias, device), c, cuvit.gemm_problem(m, n, 0, NT))
    actual = to_host(c).reshape(m, n)
    for row in actual:
        require_exact(row, bias, "a zero-K GEMM did not produce the bias")


@pytest.mark.parametrize("name,m,n,k,gelu,accumulate", [
    ("fc1 gelu b32", 6304, 768, 192, True, False),
    ("proj accumulate b32", 6304, 192, 192, False, True),
    ("fc2 accumulate b32", 6304, 192, 768, False, True),
])
def test_vit_tiny_batch_32_epilogue_gemms(cuvit, oracle, device, name, m, n, k, gelu, accumulate):
    """The C4 epilogue carriers at full size, every row judged against the
    oracle (term-scaled, and GELU's elementwise tolerance after it). Outputs
    that are not accumulated into start as NaN, so an unwritten tile fails."""
    g = oracle.generator(404 + m + n + k)
    a = g.normal(m * k)
    w = g.normal(n * k, 0.0, 0.02)
    bias = g.normal(n, 0.0, 0.02)
    existing = g.normal(m * n) if accumulate else np.full(m * n, np.nan, np.float32)
    dc = to_device(existing, device)
    problem = cuvit.gemm_problem(m, n, k, T)
    problem.epilogue.gelu = int(gelu)
    problem.epilogue.accumulate = int(accumulate)
    cuvit.gemm(to_device(a, device), to_device(w, device), to_device(bias, device), dc, problem)
    actual = to_host(dc).reshape(m, n)
    a = a.reshape(m, k)
    pre = W.in_row_chunks(lambda s, e: oracle.gemm_transposed(a[s:e], w, bias, e - s, n, k), m, 256)
    scale = W.in_row_chunks(lambda s, e: oracle.term_magnitudes(a[s:e], w, e - s, n, k, True), m, 256)
    if gelu:
        require_close(actual, oracle.gelu(pre), name, 1.0e-4, 1.0e-5)
    else:
        expected = existing.reshape(m, n) + pre if accumulate else pre
        require_close_scaled(actual, expected, scale, name, 1.0e-6, 1.0e-5)
