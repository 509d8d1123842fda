"""Softmax over rows holding masked (-inf) logits, the form an attention mask
gives them. The reference computes exp(x - max) / sum(exp(x - max)) per row
(tests/reference/linear_algebra.hpp:98-118, src/kernels/normalization.cu:89-134):
a -inf entry contributes exp(-inf) = 0 and comes out exactly 0, and a row
with every entry -inf has max = -inf, so x - max is NaN and the whole row is
NaN. Both hold here, on the staged path (aligned rows) and the register path
(rows 4 bytes past a 16-byte boundary), in fp32 and bf16, at the attention
width and at a width the full-wavefront teams take.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bf16_tensor, to_device, to_host
from numerics import require_close
from oracle import bf16_to_float

pytestmark = pytest.mark.gpu

NEG_INF_BF16 = np.uint16(0xFF80)


def masked_logits(oracle, seed: int, rows: int, columns: int) -> np.ndarray:
    """N(0, 4) logits, about a third of each row -inf, every row keeping at
    least one finite entry except rows 3 and rows - 1, which are all -inf."""
    g = oracle.generator(seed)
    x = g.normal(rows * columns, 0.0, 4.0).reshape(rows, columns).astype(np.float32)
    mask = np.random.default_rng(seed).random((rows, columns)) < 0.33
    mask[:, seed % columns] = False
    x[mask] = -np.inf
    x[3, :] = -np.inf
    x[rows - 1, :] = -np.inf
    return x


def check(actual: np.ndarray, expected: np.ndarray, x: np.ndarray, rtol: float, context: str):
    dead = np.isneginf(x).all(axis=1)
    assert np.isnan(actual[dead]).all(), f"{context}: an all -inf row is not NaN"
    assert np.isnan(expected[dead]).all()
    live = ~dead
    masked = np.isneginf(x) & live[:, None]
    assert np.all(actual[masked] == 0.0), f"{context}: a masked entry is not 0"
    require_close(actual[live], expected[live], context, rtol, 1.0e-6)


@pytest.mark.parametrize("columns", [197, 1000])
@pytest.mark.parametrize("rows", [40, 40_003])
@pytest.mark.parametrize("aligned", [True, False])
def test_masked_softmax_fp32(cuvit, oracle, device, rows, columns, aligned):
    x = masked_logits(oracle, rows + columns, rows, columns)
    expected = oracle.softmax(x)
    offset = 0 if aligned else 1
    storage = torch.full((rows * columns + offset,), float("nan"), device=device)
    storage[offset:] = to_device(x.reshape(-1), device)
    data = storage[offset:]
    cuvit.softmax(data, data, rows, columns)
    actual = to_host(data).reshape(rows, columns)
    check(actual, expected, x, 1.0e-4, f"fp32 masked softmax [{rows},{columns}] aligned={aligned}")


@pytest.mark.parametrize("columns", [197, 1000])
@pytest.mark.parametrize("rows", [40, 40_003])
@pytest.mark.parametrize("aligned", [True, False])
def test_masked_softmax_bf16(cuvit, oracle, device, rows, columns, aligned):
    x32 = masked_logits(oracle, 7 * rows + columns, rows, columns)
    bits = oracle.round_bf16(np.where(np.isneginf(x32), 0.0, x32))
    bits[np.isneginf(x32)] = NEG_INF_BF16
    x = bf16_to_float(bits).reshape(rows, columns)
    expected = oracle.softmax(x)
    offset = 0 if aligned else 1
    storage = bf16_tensor(np.concatenate([np.zeros(offset, np.uint16), bits.reshape(-1)]), device)
    data = storage[offset:]
    cuvit.softmax(data, data, rows, columns)
    actual = bf16_to_float(bf16_bits(data)).reshape(rows, columns)
    check(actual, expected, x, 1.0e-2, f"bf16 masked softmax [{rows},{columns}] aligned={aligned}")
