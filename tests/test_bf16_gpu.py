"""GPU parity for the bf16-storage twins (ViT-Base/16 batch-64 shapes).

The reference has no reduced-precision path, so these are an extension. The
oracle is the reference's fp32 CPU path run on the bf16-rounded inputs; the
GPU's bf16 output (fp32 arithmetic, one rounding at the store) must agree
within 1e-2 relative. The gather moves bits and must be bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor, to_device
from numerics import TestFailure, require_close, require_exact
from oracle import bf16_to_float

pytestmark = pytest.mark.gpu

RTOL = 1.0e-2


def bf16_inputs(oracle, seed, count, mean=0.0, stddev=1.0):
    bits = oracle.round_bf16(oracle.generator(seed).normal(count, mean, stddev))
    return bits, bf16_to_float(bits)


@pytest.mark.parametrize("rows,columns", [(12608, 768), (197, 768), (1, 192), (6304, 192),
                                          (5, 31), (3, 1), (7, 2056)])
def test_layer_norm_bf16(cuvit, oracle, device, rows, columns):
    bits, values = bf16_inputs(oracle, 505 + rows + columns, rows * columns)
    g = oracle.generator(506)
    gamma, beta = g.normal(columns, 1.0, 0.02), g.normal(columns, 0.0, 0.02)
    expected = oracle.layer_norm(values.reshape(rows, columns), gamma, beta, 1e-6)
    x = bf16_tensor(bits, device)
    y = torch.empty_like(x)
    cuvit.layer_norm(x, to_device(gamma, device), to_device(beta, device), y, rows, columns, 1e-6)
    actual = bf16_to_float(bf16_bits(y)).reshape(rows, columns)
    require_close(actual, expected, "bf16 layer norm", RTOL, 1.0e-3)


@pytest.mark.parametrize("rows,columns", [(151296, 197), (591, 197), (7, 197), (3, 1000),
                                          (2, 1500), (4, 1)])
@pytest.mark.parametrize("in_place", [False, True])
def test_softmax_bf16(cuvit, oracle, device, rows, columns, in_place):
    bits, values = bf16_inputs(oracle, 505 + rows, rows * columns)
    expected = oracle.softmax(values.reshape(rows, columns))
    x = bf16_tensor(bits, device)
    y = x if in_place else torch.empty_like(x)
    cuvit.softmax(x, y, rows, columns)
    actual = bf16_to_float(bf16_bits(y)).reshape(rows, columns)
    require_close(actual, expected, "bf16 softmax", RTOL, 1.0e-6)
    sums = actual.astype(np.float64).sum(axis=1)
    if np.abs(sums - 1.0).max() > 2.0e-2:
        raise TestFailure("a bf16 softmax row does not sum to one")


def test_gelu_bf16(cuvit, oracle, device):
    bits, values = bf16_inputs(oracle, 31, 4099, 0.0, 3.0)
    expected = oracle.gelu(values)
    x = bf16_tensor(bits, device)
    y = torch.empty_like(x)
    cuvit.gelu(x, y, bits.size)
    require_close(bf16_to_float(bf16_bits(y)), expected, "bf16 GELU", RTOL, 1.0e-3)


@pytest.mark.parametrize("batch,size,patch", [(64, 224, 16), (3, 32, 8), (2, 12, 3)])
def test_extract_patches_bf16_bit_exact(cuvit, oracle, device, batch, size, patch):
    bits, _ = bf16_inputs(oracle, 505, batch * 3 * size * size)
    # The gather permutes bits; run the oracle's permutation on the bit patterns.
    as_float = bits.astype(np.float32)  # exact: every uint16 is representable
    expected = oracle.extract_patches(as_float, batch, 3, size, size, patch).astype(np.uint16)
    x = bf16_tensor(bits, device)
    y = torch.empty_like(x)
    cuvit.extract_patches(x, y, batch, 3, size, size, patch)
    require_exact(bf16_bits(y).reshape(expected.shape), expected, "bf16 patch gather")


def require_gemm_close(actual, expected, scale, context):
    """|a - e| <= 1e-2 |e| + 1e-5 * sum|terms| (bf16 output rounding plus the
    accumulation-order difference)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    limit = RTOL * np.abs(e) + 1.0e-5 * np.abs(np.asarray(scale, np.float64)) + 1.0e-6
    bad = ~(np.abs(a - e) <= limit)
    if bad.any():
        i = int(np.argmax(bad.reshape(-1)))
        raise TestFailure(f"{context}: mismatch at {i}: {a.reshape(-1)[i]} vs {e.reshape(-1)[i]}")


@pytest.mark.parametrize("m,n,k,layout", [(17, 33, 7, 0), (65, 65, 65, 1), (197, 576, 192, 1),
                                          (197, 64, 197, 0), (300, 257, 129, 1), (1, 1000, 768, 1)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_bf16_shapes(cuvit, oracle, device, m, n, k, layout, with_bias):
    a_bits, a = bf16_inputs(oracle, m * 31 + n, m * k)
    b_bits, b = bf16_inputs(oracle, m * 7 + k, n * k)
    bias = oracle.generator(3).normal(n) if with_bias else None
    if layout == 1:
        expected = oracle.gemm_transposed(a, b, bias, m, n, k)
    else:
        expected = oracle.gemm(a, b, bias, m, n, k)
    scale = oracle.term_magnitudes(a, b, m, n, k, layout == 1)
    c = torch.empty(m * n, dtype=torch.bfloat16, device=device)
    problem = cuvit.gemm_problem(m, n, k, layout)
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(b_bits, device),
               None if bias is None else to_device(bias, device), c, problem)
    require_gemm_close(bf16_to_float(bf16_bits(c)).reshape(m, n), expected, scale,
                       f"bf16 GEMM {m}x{n}x{k}")


def test_gemm_bf16_accumulate(cuvit, oracle, device):
    """C += value: the stored bf16 C is widened, added in fp32, rounded once."""
    m, n, k = 70, 40, 24
    a_bits, a = bf16_inputs(oracle, 41, m * k)
    b_bits, b = bf16_inputs(oracle, 42, k * n)
    c_bits, c = bf16_inputs(oracle, 43, m * n)
    bias = oracle.generator(44).normal(n)
    expected = c.reshape(m, n) + oracle.gemm(a, b, bias, m, n, k)
    scale = oracle.term_magnitudes(a, b, m, n, k, False) + np.abs(c.reshape(m, n))
    dc = bf16_tensor(c_bits, device)
    problem = cuvit.gemm_problem(m, n, k, 0)
    problem.epilogue.accumulate = 1
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(b_bits, device), to_device(bias, device),
               dc, problem)
    require_gemm_close(bf16_to_float(bf16_bits(dc)).reshape(m, n), expected, scale,
                       "bf16 accumulate epilogue")


def test_gemm_bf16_vit_base_fc1_gelu(cuvit, oracle, device):
    """C5's GELU epilogue carrier: FC1 of ViT-Base at batch 64, M=12608, N=3072,
    K=768, bf16 activations and weights, fp32 bias; judged on a row sample."""
    m, n, k = 12608, 3072, 768
    a_bits, a = bf16_inputs(oracle, 505, m * k)
    w_bits, w = bf16_inputs(oracle, 507, n * k, 0.0, 0.02)
    bias = oracle.generator(508).normal(n, 0.0, 0.02)
    c = torch.empty(m * n, dtype=torch.bfloat16, device=device)
    problem = cuvit.gemm_problem(m, n, k, 1)
    problem.epilogue.gelu = 1
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(w_bits, device), to_device(bias, device),
               c, problem)
    actual = bf16_to_float(bf16_bits(c)).reshape(m, n)
    rows = np.r_[0:32, 6000:6032, m - 32:m]
    sample = a.reshape(m, k)[rows]
    pre = oracle.gemm_transposed(sample, w, bias, rows.size, n, k)
    scale = oracle.term_magnitudes(sample, w, rows.size, n, k, True)
    require_gemm_close(actual[rows], oracle.gelu(pre), scale, "ViT-Base FC1 + GELU (bf16)")


def test_softmax_bf16_paths_agree_bitwise(cuvit, oracle, device):
    """151296 rows take the staged path, a handful of rows the register path;
    a row's bits must not depend on which (batch invariance)."""
    rows, columns = 151296, 197
    bits, _ = bf16_inputs(oracle, 909, rows * columns)
    x = bf16_tensor(bits, device)
    cuvit.softmax(x, x, rows, columns)
    full = bf16_bits(x).reshape(rows, columns)
    for start in (0, 7, 75000, rows - 5):
        part = bf16_tensor(bits.reshape(rows, columns)[start:start + 5], device)
        cuvit.softmax(part, part, 5, columns)
        require_exact(bf16_bits(part).reshape(5, columns), full[start:start + 5],
                      f"bf16 rows {start}.. differ between paths")


@pytest.mark.parametrize("m,n,k,layout", [(2000, 1100, 96, 1), (1500, 2100, 72, 0), (4100, 1030, 40, 1)])
def test_gemm_bf16_tile_blocks_per_xcd(cuvit, oracle, device, m, n, k, layout):
    """Enough tiles for the XCD block order, with block splits that do not
    divide the tile grid evenly; every output must be produced exactly once."""
    a_bits, a = bf16_inputs(oracle, m + 3 * n, m * k)
    b_bits, b = bf16_inputs(oracle, m + 5 * k, n * k)
    bias = oracle.generator(9).normal(n)
    if layout == 1:
        expected = oracle.gemm_transposed(a, b, bias, m, n, k)
    else:
        expected = oracle.gemm(a, b, bias, m, n, k)
    scale = oracle.term_magnitudes(a, b, m, n, k, layout == 1)
    c = torch.full((m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(b_bits, device), to_device(bias, device), c,
               cuvit.gemm_problem(m, n, k, layout))
    require_gemm_close(bf16_to_float(bf16_bits(c)).reshape(m, n), expected, scale,
                       f"bf16 GEMM {m}x{n}x{k} in XCD blocks")


def test_gemm_bf16_batched_tile_blocks(cuvit, oracle, device):
    """Batched entries (grid rows) each split into XCD blocks."""
    count, m, n, k = 3, 700, 600, 48
    a_bits, a = bf16_inputs(oracle, 61, count * m * k)
    b_bits, b = bf16_inputs(oracle, 62, count * n * k)
    c = torch.full((count * m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    problem = cuvit.gemm_problem(m, n, k, 1)
    problem.batch.count = count
    problem.batch.stride_a, problem.batch.stride_b, problem.batch.stride_c = m * k, n * k, m * n
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(b_bits, device), None, c, problem)
    actual = bf16_to_float(bf16_bits(c)).reshape(count, m, n)
    for e in range(count):
        ae = a.reshape(count, m * k)[e]
        be = b.reshape(count, n * k)[e]
        expected = oracle.gemm_transposed(ae, be, None, m, n, k)
        scale = oracle.term_magnitudes(ae, be, m, n, k, True)
        require_gemm_close(actual[e], expected, scale, f"bf16 batched entry {e}")
