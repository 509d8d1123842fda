"""GPU parity for LayerNorm, softmax, GELU and the residual add.

Mirrors the reference's tests/elementwise_test.cu case by case (shapes, seeds,
distributions, tolerances), driving the HIP kernels through the C ABI and
judging them against the oracle on the same seeded inputs. Added beyond the
reference: the bound max-abs <= 1e-5 for fp32 LN / softmax / GELU,
in-place softmax, and the ViT-Tiny batch-32 shapes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import workloads as W
from conftest import to_device, to_host
from numerics import TestFailure, require_close, require_exact, require_max_abs

pytestmark = pytest.mark.gpu

MAX_ABS_FP32 = 1.0e-5  # stated tolerance for LN, softmax and GELU in fp32


def require(condition, message):  # noqa: F811 - the reference's require()
    if not condition:
        raise TestFailure(message)


def test_gelu_matches_the_erf_form(cuvit, oracle, device):
    """elementwise_test.cu:32-61."""
    count = 4099
    x = oracle.generator(31).normal(count, 0.0, 3.0)
    landmarks = [-30.0, -8.0, -2.7, -2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 2.7, 8.0, 30.0]
    x[: len(landmarks)] = landmarks
    expected = oracle.gelu(x)

    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.gelu(dx, dy, count)
    actual = to_host(dy)
    require_close(actual, expected, "GELU differs from the CPU reference", 1.0e-5, 1.0e-6)
    require_max_abs(actual, expected, MAX_ABS_FP32, "GELU max-abs")

    probe = np.float32(-2.7)
    tanh_form = np.float32(0.5) * probe * (np.float32(1.0) + np.tanh(
        np.float32(0.7978845608) * (probe + np.float32(0.044715) * probe * probe * probe)))
    require(abs(float(tanh_form) - oracle.gelu_scalar(-2.7)) > 4.0e-4,
            "the test cannot tell the erf and tanh GELU forms apart")


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_gelu_unaligned_and_ragged(cuvit, oracle, device, offset):
    """Scalar path: pointers off 16-byte alignment, counts not multiples of 4."""
    count = 1031
    x = oracle.generator(37 + offset).normal(count + 8, 0.0, 3.0)
    expected = oracle.gelu(x[offset:offset + count])
    dx = to_device(x, device)
    dy = torch.zeros_like(dx)
    cuvit.gelu(dx[offset:], dy[offset:], count)
    actual = to_host(dy)
    require_close(actual[offset:offset + count], expected, "unaligned GELU", 1.0e-5, 1.0e-6)
    require_exact(actual[:offset], np.zeros(offset, np.float32), "GELU wrote before its range")
    require_exact(actual[offset + count:], np.zeros(8 - offset, np.float32),
                  "GELU wrote past its range")


def test_residual_add(cuvit, oracle, device):
    """elementwise_test.cu:63-90: a single add rounds identically, so bit-exact."""
    count = 1024
    g = oracle.generator(9)
    acc = g.normal(count)
    addend = g.normal(count)
    expected = oracle.add(acc.copy(), addend)
    dacc, dadd = to_device(acc, device), to_device(addend, device)
    cuvit.add(dacc, dadd, count)
    require_exact(to_host(dacc), expected, "residual add differs from the CPU reference")


@pytest.mark.parametrize("count,offset", [(1, 0), (7, 1), (4097, 3), (1 << 20, 0)])
def test_residual_add_sizes(cuvit, oracle, device, count, offset):
    g = oracle.generator(count + offset)
    acc = g.normal(count + offset)
    addend = g.normal(count + offset)
    expected = acc.copy()
    oracle.add(expected[offset:], addend[offset:])
    dacc, dadd = to_device(acc, device), to_device(addend, device)
    cuvit.add(dacc[offset:], dadd[offset:], count)
    require_exact(to_host(dacc), expected, "residual add")


LN_SHAPES = [(1, 192), (197, 192), (197, 768), (3, 1), (5, 31), (2, 1024),
             # beyond the reference: ViT-Tiny batch 32, ViT-Base rows, odd widths
             (6304, 192), (64, 768), (7, 4), (9, 36), (11, 2048), (4, 4100),
             # more row groups than wavefronts (grid-stride loop)
             (70001, 192)]


@pytest.mark.parametrize("rows,columns", LN_SHAPES)
def test_layer_norm(cuvit, oracle, device, rows, columns):
    """elementwise_test.cu:92-131 (same seeds, N(0,1) rows, gamma N(1,0.2), beta N(0,0.2))."""
    g = oracle.generator(rows * 101 + columns)
    x = g.normal(rows * columns, 0.0, 1.0).reshape(rows, columns)
    gamma = g.normal(columns, 1.0, 0.2)
    beta = g.normal(columns, 0.0, 0.2)
    expected = oracle.layer_norm(x, gamma, beta, 1.0e-6)

    dx = to_device(x, device)
    dg, db = to_device(gamma, device), to_device(beta, device)
    dy = torch.empty_like(dx)
    cuvit.layer_norm(dx, dg, db, dy, rows, columns, 1.0e-6)
    actual = to_host(dy)
    require_close(actual, expected, "layer norm differs from the CPU reference", 1.0e-5, 2.0e-6)
    require_max_abs(actual, expected, MAX_ABS_FP32, "layer norm max-abs")


def test_layer_norm_unaligned_rows(cuvit, oracle, device):
    """A base pointer off 16 bytes forces the generic path; same tolerance."""
    rows, columns = 33, 192
    g = oracle.generator(4242)
    x = g.normal(rows * columns + 1).astype(np.float32)
    gamma = g.normal(columns, 1.0, 0.2)
    beta = g.normal(columns, 0.0, 0.2)
    expected = oracle.layer_norm(x[1:].reshape(rows, columns), gamma, beta, 1.0e-6)
    dx = to_device(x, device)
    dy = torch.zeros_like(dx)
    cuvit.layer_norm(dx[1:], to_device(gamma, device), to_device(beta, device), dy[1:], rows,
                     columns, 1.0e-6)
    actual = to_host(dy)[1:].reshape(rows, columns)
    require_close(actual, expected, "unaligned layer norm", 1.0e-5, 2.0e-6)


def test_layer_norm_tolerates_a_large_offset(cuvit, oracle, device):
    """elementwise_test.cu:153-188: rows around 1000, atol 5e-5."""
    rows, columns = 197, 192
    x = oracle.generator(7).normal(rows * columns, 1000.0, 1.0).reshape(rows, columns)
    gamma = np.ones(columns, np.float32)
    beta = np.zeros(columns, np.float32)
    expected = oracle.layer_norm(x, gamma, beta, 1.0e-6)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.layer_norm(dx, to_device(gamma, device), to_device(beta, device), dy, rows, columns,
                     1.0e-6)
    require_close(to_host(dy), expected,
                  "layer norm degraded beyond what float allows at this offset", 1.0e-5, 5.0e-5)


def test_layer_norm_normalizes(cuvit, oracle, device):
    """elementwise_test.cu:190-229: zero mean, unit variance, independent of the oracle."""
    rows, columns = 8, 192
    x = oracle.generator(3).normal(rows * columns, 5.0, 3.0).reshape(rows, columns)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.layer_norm(dx, to_device(np.ones(columns, np.float32), device),
                     to_device(np.zeros(columns, np.float32), device), dy, rows, columns)
    actual = to_host(dy).astype(np.float64)
    for row in actual:
        require(abs(row.sum() / columns) < 1.0e-4, "a normalized row does not have zero mean")
        require(abs((row * row).sum() / columns - 1.0) < 1.0e-3,
                "a normalized row does not have unit variance")


def test_layer_norm_single_column_gives_beta(cuvit, device):
    """var = 0 and x - mean = 0, so every output equals beta exactly."""
    rows = 3
    x = np.array([[5.0], [-2.0], [1.0e6]], np.float32)
    beta = np.array([0.25], np.float32)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.layer_norm(dx, to_device(np.array([3.0], np.float32), device), to_device(beta, device),
                     dy, rows, 1)
    require_exact(to_host(dy), np.full((rows, 1), 0.25, np.float32), "one-column layer norm")


SOFTMAX_SHAPES = [(1, 2), (197, 197), (4, 1), (3, 1000), (8, 33),
                  # beyond the reference: one attention head-batch, tails of 4-row blocks,
                  # widths across the register-resident limit
                  (591, 197), (5, 197), (6, 197), (7, 197), (13, 64), (3, 1024), (2, 1025),
                  (9, 2500), (4, 255),
                  # LDS tile rows padded to keep the row teams on disjoint banks, vectors
                  # straddling two or more rows
                  (6, 128), (11, 7), (9, 3)]


@pytest.mark.parametrize("rows,columns", SOFTMAX_SHAPES)
@pytest.mark.parametrize("in_place", [False, True])
def test_softmax(cuvit, oracle, device, rows, columns, in_place):
    """elementwise_test.cu:231-267 (N(0,4) logits, rtol 1e-4, rows sum to one)."""
    x = oracle.generator(rows * 17 + columns).normal(rows * columns, 0.0, 4.0).reshape(rows, columns)
    expected = oracle.softmax(x)
    dx = to_device(x, device)
    dy = dx if in_place else torch.empty_like(dx)
    cuvit.softmax(dx, dy, rows, columns)
    actual = to_host(dy)
    require_close(actual, expected, "softmax differs from the CPU reference", 1.0e-4, 1.0e-6)
    require_max_abs(actual, expected, MAX_ABS_FP32, "softmax max-abs")
    require(((actual >= 0.0) & (actual <= 1.0)).all(), "a softmax value is outside [0, 1]")
    sums = actual.astype(np.float64).sum(axis=1)
    require(np.abs(sums - 1.0).max() < 1.0e-4, "a softmax row does not sum to one")


def test_softmax_unaligned(cuvit, oracle, device):
    """Base pointers off 16 bytes take the streaming online-max path."""
    rows, columns = 37, 197
    x = oracle.generator(999).normal(rows * columns + 3, 0.0, 4.0)
    expected = oracle.softmax(x[3:].reshape(rows, columns))
    dx = to_device(x, device)
    dy = torch.zeros_like(dx)
    cuvit.softmax(dx[3:], dy[3:], rows, columns)
    actual = to_host(dy)[3:].reshape(rows, columns)
    require_close(actual, expected, "unaligned softmax", 1.0e-4, 1.0e-6)
    require_max_abs(actual, expected, MAX_ABS_FP32, "unaligned softmax max-abs")


def test_softmax_survives_large_logits(cuvit, device):
    """elementwise_test.cu:269-302: +-500 rows give one-hot outputs."""
    rows, columns = 4, 64
    x = np.full((rows, columns), -500.0, np.float32)
    for row in range(rows):
        x[row, row] = 500.0
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.softmax(dx, dy, rows, columns)
    actual = to_host(dy)
    require(np.isfinite(actual).all(), "softmax produced a non-finite value on large logits")
    require(np.abs(actual - np.eye(rows, columns, dtype=np.float32)).max() < 1.0e-5,
            "softmax of a saturated row is not one-hot")


def test_softmax_single_column_is_one(cuvit, device):
    x = np.array([[3.0], [-1.0e30], [0.0], [7.5]], np.float32)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.softmax(dx, dy, 4, 1)
    require_exact(to_host(dy), np.ones((4, 1), np.float32), "one-column softmax")


def test_softmax_rows_are_position_independent(cuvit, oracle, device):
    """A row's bits do not depend on where it sits in the launch (batch invariance)."""
    columns = 197
    rows = 3 * 197 * 3
    x = oracle.generator(55).normal(rows * columns).reshape(rows, columns)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.softmax(dx, dy, rows, columns)
    full = to_host(dy)
    for start in (1, 2, 3, 591, 593):
        part = to_device(x[start:start + 5], device)
        out = torch.empty_like(part)
        cuvit.softmax(part, out, 5, columns)
        require_exact(to_host(out), full[start:start + 5], f"softmax rows moved by {start}")


def test_layer_norm_rows_are_position_independent(cuvit, oracle, device):
    columns = 192
    rows = 197 * 3
    x = oracle.generator(56).normal(rows * columns).reshape(rows, columns)
    gamma = oracle.generator(57).normal(columns, 1.0, 0.2)
    beta = oracle.generator(58).normal(columns, 0.0, 0.2)
    dg, db = to_device(gamma, device), to_device(beta, device)
    dx = to_device(x, device)
    dy = torch.empty_like(dx)
    cuvit.layer_norm(dx, dg, db, dy, rows, columns)
    full = to_host(dy)
    for start in (1, 2, 3, 197, 199):
        part = to_device(x[start:start + 6], device)
        out = torch.empty_like(part)
        cuvit.layer_norm(part, dg, db, out, 6, columns)
        require_exact(to_host(out), full[start:start + 6], f"layer norm rows moved by {start}")


def test_zero_sizes_are_no_ops(cuvit, device):
    """elementwise_test.cu:304-310: empty launches return before any check."""
    buffer = torch.zeros(16, device=device)
    cuvit.gelu(buffer, buffer, 0)
    cuvit.softmax(buffer, buffer, 0, 4)
    cuvit.layer_norm(buffer, buffer, buffer, buffer, 0, 4)
    cuvit.gelu(None, None, 0)
    torch.cuda.synchronize()
    require_exact(to_host(buffer), np.zeros(16, np.float32), "an empty launch wrote memory")


def test_invalid_arguments(cuvit, device):
    """elementwise_test.cu:312-326."""
    buffer = torch.zeros(16, device=device)
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.gelu(None, buffer, 4)
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.layer_norm(buffer, None, buffer, buffer, 2, 4)


@pytest.mark.parametrize("columns", [197, 64, 1000])
def test_softmax_staged_path_matches_oracle_and_register_path(cuvit, oracle, device, columns):
    """Large row counts take the LDS-staged path; it must agree with the oracle
    and give the same bits per row as the register path small launches take."""
    rows = 40_003
    x = oracle.generator(columns + 7).normal(rows * columns, 0.0, 4.0).reshape(rows, columns)
    dx = to_device(x, device)
    cuvit.softmax(dx, dx, rows, columns)
    actual = to_host(dx).reshape(rows, columns)
    expected = W.in_row_chunks(lambda s, e: oracle.softmax(x[s:e]), rows, 2048)
    require_close(actual, expected, "staged softmax", 1.0e-4, 1.0e-6)
    require_max_abs(actual, expected, MAX_ABS_FP32, "staged softmax max-abs")
    for start in (0, 5, rows - 3):
        part = to_device(x[start:start + 3], device)
        cuvit.softmax(part, part, part.shape[0], columns)
        require_exact(to_host(part), actual[start:start + 3], f"rows {start}.. differ between paths")
