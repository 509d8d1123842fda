"""The wide-tile bf16 GEMM (128 x 256 workgroup tiles, epilogue through LDS),
which large B-as-[N, K] problems without accumulation take.

Its results must be bitwise those of the 64 x 64 / 128 x 128 kernel that small
problems take: both run the same MFMA over the same k-blocks in the same order
and apply alpha and the bias without fusing them. Each case launches a problem
large enough for the wide kernel (output prefilled with NaN), then the same
rows in launches of 197 rows, small enough for the other kernel, and requires
equality bit for bit; one block of rows is also judged against the oracle.
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
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    limit = RTOL * np.abs(e) + 1.0e-5 * np.abs(np.asarray(scale, np.float64)) + 1.0e-6
    bad = ~(np.abs(a - e) <= limit)
    if bad.any():
        i = int(np.argmax(bad.reshape(-1)))
        raise TestFailure(f"{context}: mismatch at {i}: {a.reshape(-1)[i]} vs {e.reshape(-1)[i]}")


CASES = [
    # m, n, k, bias, gelu, alpha
    (12608, 3072, 768, True, True, 1.0),      # ViT-Base FC1
    (12608, 2304, 768, True, False, 1.0),     # ViT-Base QKV
    (12608, 1544, 776, True, True, 0.75),     # N and K off the tile grid, alpha with the bias
    (12450, 1544, 200, False, False, -1.25),  # M tail, short K, no bias
    (12608, 1320, 768, False, True, 0.5),     # GELU without a bias
]


@pytest.mark.parametrize("m,n,k,with_bias,gelu,alpha", CASES)
def test_wide_equals_the_small_tile_kernel(cuvit, oracle, device, m, n, k, with_bias, gelu, alpha):
    a_bits, a = bf16_inputs(oracle, m + k, m * k)
    w_bits, w = bf16_inputs(oracle, n + k, n * k, 0.05)
    bias = oracle.generator(n).normal(n, 0.0, 0.5) if with_bias else None
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    dbias = to_device(bias, device) if with_bias else None

    def problem(rows):
        p = cuvit.gemm_problem(rows, n, k, cuvit.TRANSPOSED)
        p.alpha = alpha
        p.epilogue.gelu = int(gelu)
        return p

    c = torch.full((m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    cuvit.gemm(da, dw, dbias, c, problem(m))
    full = bf16_bits(c).reshape(m, n)
    rows = 197
    part = torch.full((rows * n,), float("nan"), dtype=torch.bfloat16, device=device)
    for start in range(0, m, rows):
        count = min(rows, m - start)
        cuvit.gemm(da[start * k:], dw, dbias, part, problem(count))
        require_exact(bf16_bits(part)[:count * n].reshape(count, n), full[start:start + count],
                      f"rows {start}..{start + count} differ from launches of {rows} rows")
    last = m - 64
    sample = a.reshape(m, k)[last:]
    pre = oracle.gemm_transposed(sample, w, bias, 64, n, k, alpha)
    scale = oracle.term_magnitudes(sample, w, 64, n, k, True, alpha)
    expected = oracle.gelu(pre) if gelu else pre
    require_gemm_close(bf16_to_float(full[last:]), expected, scale, "last 64 rows against the oracle")


def test_wide_batched_entries(cuvit, oracle, device):
    """Two batch entries with their own A and C, B shared (stride 0): each entry
    equals its own single launch, bit for bit."""
    m, n, k = 6304, 3072, 768
    a_bits, _ = bf16_inputs(oracle, 77, 2 * m * k)
    w_bits, _ = bf16_inputs(oracle, 78, n * k, 0.05)
    bias = to_device(oracle.generator(79).normal(n, 0.0, 0.5), device)
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.epilogue.gelu = 1
    p.batch.count, p.batch.stride_a, p.batch.stride_b, p.batch.stride_c = 2, m * k, 0, m * n
    c = torch.full((2 * m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    cuvit.gemm(da, dw, bias, c, p)
    both = bf16_bits(c).reshape(2, m, n)
    single = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    single.epilogue.gelu = 1
    one = torch.full((m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    for entry in range(2):
        cuvit.gemm(da[entry * m * k:], dw, bias, one, single)
        require_exact(bf16_bits(one).reshape(m, n), both[entry], f"batch entry {entry}")
