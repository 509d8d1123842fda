"""The direct-to-LDS bf16 GEMM (one persistent eight-wavefront workgroup per CU,
BM x 256 tiles with BM 192, 256 or 320), which large single B-as-[N, K]
problems with N a multiple of 256 take: the ViT-Base linear layers.

Its results must be bitwise those of the kernels smaller problems take: all
run the same MFMA over the same k-blocks in the same order and apply alpha,
the bias, GELU and the accumulation in the same unfused order. Each case
launches a problem large enough for it (output prefilled: NaN, or an old C
when accumulating), then the same rows in launches of 197 rows, which the
other kernels take, and requires equality bit for bit; the last 64 rows are
also judged against the oracle.
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
    # m, n, k, bias, gelu, alpha, accumulate
    (12608, 3072, 768, True, True, 1.0, False),     # ViT-Base FC1 (320-row tiles)
    (12608, 2304, 768, True, False, 1.0, False),    # ViT-Base QKV (256-row tiles)
    (12608, 768, 3072, True, False, 1.0, True),     # ViT-Base FC2, accumulating (192-row tiles)
    (12608, 768, 768, True, False, 1.0, True),      # ViT-Base projection, accumulating
    (12450, 2304, 776, True, True, 0.75, False),    # M tail, K off the 128 grid, alpha with the bias
    (12450, 1024, 256, False, False, -1.25, True),  # shortest K, no bias, accumulating with alpha
    (9000, 2048, 520, False, True, 0.5, False),     # GELU without a bias
]


@pytest.mark.parametrize("m,n,k,with_bias,gelu,alpha,accumulate", CASES)
def test_dma_equals_the_small_tile_kernel(cuvit, oracle, device, m, n, k, with_bias, gelu, alpha,
                                          accumulate):
    a_bits, a = bf16_inputs(oracle, m + k, m * k)
    w_bits, w = bf16_inputs(oracle, n + k, n * k, 0.05)
    bias = oracle.generator(n).normal(n, 0.0, 0.5) if with_bias else None
    da, dw = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device)
    dbias = to_device(bias, device) if with_bias else None
    old_bits, old = bf16_inputs(oracle, m + n + k, m * n) if accumulate else (None, None)

    def problem(rows):
        p = cuvit.gemm_problem(rows, n, k, cuvit.TRANSPOSED)
        p.alpha = alpha
        p.epilogue.gelu = int(gelu)
        p.epilogue.accumulate = int(accumulate)
        return p

    def output(count, start=0):
        if accumulate:
            return bf16_tensor(old_bits[start * n:(start + count) * n], device)
        return torch.full((count * n,), float("nan"), dtype=torch.bfloat16, device=device)

    c = output(m)
    cuvit.gemm(da, dw, dbias, c, problem(m))
    full = bf16_bits(c).reshape(m, n)
    rows = 197
    for start in range(0, m, rows):
        count = min(rows, m - start)
        part = output(count, start)
        cuvit.gemm(da[start * k:], dw, dbias, part, problem(count))
        require_exact(bf16_bits(part).reshape(count, n), full[start:start + count],
                      f"rows {start}..{start + count} differ from launches of {rows} rows")
    last = m - 64
    sample = a.reshape(m, k)[last:]
    pre = oracle.gemm_transposed(sample, w, bias, 64, n, k, alpha)
    scale = oracle.term_magnitudes(sample, w, 64, n, k, True, alpha)
    expected = oracle.gelu(pre) if gelu else pre
    if accumulate:
        base = old.reshape(m, n)[last:].astype(np.float64)
        expected = base + expected
        scale = np.abs(base) + scale
    require_gemm_close(bf16_to_float(full[last:]), expected, scale, "last 64 rows against the oracle")


def test_dma_two_calls_in_a_row_and_a_smaller_one(cuvit, oracle, device):
    """The persistent kernel keeps nothing between launches: FC1 twice, then
    a problem with fewer tiles, each equal to its 197-row launches."""
    n, k = 3072, 768
    w_bits, _ = bf16_inputs(oracle, 91, n * k, 0.05)
    dw = bf16_tensor(w_bits, device)
    bias = to_device(oracle.generator(92).normal(n, 0.0, 0.5), device)
    for m in (12608, 12608, 8000):
        a_bits, _ = bf16_inputs(oracle, m + 93, m * k)
        da = bf16_tensor(a_bits, device)
        p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
        p.epilogue.gelu = 1
        c = torch.full((m * n,), float("nan"), dtype=torch.bfloat16, device=device)
        cuvit.gemm(da, dw, bias, c, p)
        full = bf16_bits(c).reshape(m, n)
        if np.isnan(bf16_to_float(full)).any():
            raise TestFailure(f"m = {m}: an output was not written")
        part_rows = 1000
        part = torch.empty(part_rows * n, dtype=torch.bfloat16, device=device)
        q = cuvit.gemm_problem(part_rows, n, k, cuvit.TRANSPOSED)
        q.epilogue.gelu = 1
        cuvit.gemm(da[(m - part_rows) * k:], dw, bias, part, q)
        require_exact(bf16_bits(part).reshape(part_rows, n), full[m - part_rows:],
                      f"m = {m}: the last {part_rows} rows differ")
