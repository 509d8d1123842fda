"""The twelve-wavefront bf16 GEMM tile (256 x 192, wavefront tiles of 64 x 64,
64-deep stages), which products with B as [N, K] and K of at least 512 take
when one round of such tiles covers the problem and 128 x 128 tiles would need
more than two per compute unit: the ViT-Base FC2 and projection at batch 64
(12608 x 768 x 3072 and 12608 x 768 x 768, accumulating into the residual
stream).

Its results must be bitwise those of the 64 x 64 kernel that small problems
take: both run the same MFMA over the same k-blocks in the same order and
apply alpha, the bias, GELU and the accumulation without fusing them. Each
case launches a problem the tall tile takes (outputs that are not accumulated
into start as NaN), then the same rows in launches of 197 rows, and requires
equality bit for bit over every row; the last 64 rows are also judged
against the oracle, and the columns past N must keep their values.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor, to_device
from numerics import TestFailure, require_exact
from oracle import bf16_to_float

pytestmark = pytest.mark.gpu

RTOL = 1.0e-2


def bf16_inputs(oracle, seed, count, stddev=1.0):
    bits = oracle.round_bf16(oracle.generator(seed).normal(count, 0.0, stddev))
    return bits, bf16_to_float(bits)


def require_gemm_close(actual, expected, scale, context):
    """|a - e| <= 1e-2 |e| + 1e-5 sum|terms| (bf16 output rounding plus the
    accumulation-order difference)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    limit = RTOL * np.abs(e) + 1.0e-5 * np.abs(np.asarray(scale, np.float64)) + 1.0e-6
    bad = ~(np.abs(a - e) <= limit)
    if bad.any():
        i = int(np.argmax(bad.reshape(-1)))
        raise TestFailure(f"{context}: mismatch at {i}: {a.reshape(-1)[i]} vs {e.reshape(-1)[i]}")


CASES = [
    # m, n, k, bias, gelu, accumulate, alpha, lda pad, ldc pad
    (12608, 768, 3072, True, False, True, 1.0, 0, 0),      # ViT-Base FC2 into the residual
    (12000, 760, 2104, True, True, True, 0.75, 8, 8),      # M, N and K tails, GELU + accumulate
    (11008, 768, 2048, False, False, False, -1.25, 0, 0),  # no bias, no accumulation
    (12608, 768, 768, True, False, True, 1.0, 0, 0),       # ViT-Base projection
    (12300, 736, 520, True, True, False, 2.0, 0, 8),       # short K with a tail, N tail, GELU
]


@pytest.mark.parametrize("m,n,k,with_bias,gelu,accumulate,alpha,lda_pad,ldc_pad", CASES)
def test_tall_tile_equals_the_small_tile_kernel(cuvit, oracle, device, m, n, k, with_bias, gelu,
                                                accumulate, alpha, lda_pad, ldc_pad):
    lda, ldc = k + lda_pad, n + ldc_pad
    a_bits, a = bf16_inputs(oracle, m + 5 * k, m * lda)
    w_bits, w = bf16_inputs(oracle, n + 3 * k, n * k, 0.02)
    bias = oracle.generator(n + 1).normal(n, 0.0, 0.5) if with_bias else None
    if accumulate:
        c_bits, c_values = bf16_inputs(oracle, m + n, m * ldc)
    else:
        c_bits = np.full(m * ldc, 0x7FC0, np.uint16)  # bf16 quiet NaN
        c_values = bf16_to_float(c_bits)
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    dbias = to_device(bias, device) if with_bias else None

    def problem(rows):
        p = cuvit.gemm_problem(rows, n, k, cuvit.TRANSPOSED)
        p.alpha = alpha
        p.lda, p.ldc = lda, ldc
        p.epilogue.gelu = int(gelu)
        p.epilogue.accumulate = int(accumulate)
        return p

    c = bf16_tensor(c_bits, device)
    cuvit.gemm(da, dw, dbias, c, problem(m))
    full = bf16_bits(c).reshape(m, ldc)
    rows = 197
    for start in range(0, m, rows):
        count = min(rows, m - start)
        part = bf16_tensor(c_bits[start * ldc:(start + count) * ldc], device)
        cuvit.gemm(da[start * lda:], dw, dbias, part, problem(count))
        require_exact(bf16_bits(part).reshape(count, ldc)[:, :n], full[start:start + count, :n],
                      f"rows {start}..{start + count} differ from launches of {rows} rows")
    require_exact(full[:, n:], c_bits.reshape(m, ldc)[:, n:], "the columns past N changed")
    last = m - 64
    sample = np.ascontiguousarray(a.reshape(m, lda)[last:, :k])
    pre = oracle.gemm_transposed(sample, w, bias, 64, n, k, alpha)
    scale = oracle.term_magnitudes(sample, w, 64, n, k, True, alpha)
    value = oracle.gelu(pre) if gelu else pre
    expected = c_values.reshape(m, ldc)[last:, :n] + value if accumulate else value
    if accumulate:
        scale = scale + np.abs(c_values.reshape(m, ldc)[last:, :n])
    require_gemm_close(bf16_to_float(full[last:, :n]), expected, scale,
                       "last 64 rows against the oracle")


def test_tall_tile_batched_entries(cuvit, oracle, device):
    """Two batch entries of 6304 rows (one round of 200 tall tiles between
    them), B shared: each entry equals its own launch, bit for bit."""
    m, n, k = 6304, 768, 3072
    a_bits, _ = bf16_inputs(oracle, 91, 2 * m * k)
    w_bits, _ = bf16_inputs(oracle, 92, n * k, 0.02)
    c_bits, _ = bf16_inputs(oracle, 93, 2 * m * n)
    bias = to_device(oracle.generator(94).normal(n, 0.0, 0.5), device)
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.epilogue.accumulate = 1
    p.batch.count, p.batch.stride_a, p.batch.stride_b, p.batch.stride_c = 2, m * k, 0, m * n
    c = bf16_tensor(c_bits, device)
    cuvit.gemm(da, dw, bias, c, p)
    both = bf16_bits(c).reshape(2, m, n)
    single = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    single.epilogue.accumulate = 1
    for entry in range(2):
        one = bf16_tensor(c_bits[entry * m * n:(entry + 1) * m * n], device)
        cuvit.gemm(da[entry * m * k:], dw, bias, one, single)
        require_exact(bf16_bits(one).reshape(m, n), both[entry], f"batch entry {entry}")


def test_tall_tile_runs_a_shared_weight_batch_as_one_problem(cuvit, oracle, device):
    """A batch of 64 entries of 196 rows with B shared and A rows following
    one another (the ViT-Base patch embedding's shape) runs as one problem of
    12544 rows on the tall tile; each entry lands at its own C stride (197
    rows apart, so one row per entry is never written) and equals its own
    launch of 196 rows, bit for bit."""
    entries, m, n, k = 64, 196, 768, 768
    a_bits, _ = bf16_inputs(oracle, 95, entries * m * k)
    w_bits, _ = bf16_inputs(oracle, 96, n * k, 0.02)
    c_bits, _ = bf16_inputs(oracle, 97, entries * (m + 1) * n)
    bias = to_device(oracle.generator(98).normal(n, 0.0, 0.5), device)
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.batch.count, p.batch.stride_a, p.batch.stride_b, p.batch.stride_c = entries, m * k, 0, (m + 1) * n
    c = bf16_tensor(c_bits, device)
    cuvit.gemm(da, dw, bias, c, p)
    full = bf16_bits(c).reshape(entries, m + 1, n)
    require_exact(full[:, m], c_bits.reshape(entries, m + 1, n)[:, m], "the rows between entries changed")
    single = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    one = torch.empty(m * n, dtype=torch.bfloat16, device=device)
    for entry in (0, 1, 31, 63):
        cuvit.gemm(da[entry * m * k:], dw, bias, one, single)
        require_exact(bf16_bits(one).reshape(m, n), full[entry, :m], f"batch entry {entry}")
