"""The resident-panel fp32 GEMM (a B panel held in LDS for the whole of K, A
fragments loaded straight into the MFMA layout), which tall single fp32
products with B as [N, K] take: the model's linear layers at batch 32.

Its results must be bitwise those of the LDS-tiled kernel that small problems
take: both run v_mfma_f32_16x16x4_f32 over the same k-blocks in the same order
and apply alpha, the bias and GELU without fusing them. Each case launches a
problem the panel kernel takes (K of 192 or 768, at least eight wavefront
items per compute unit; outputs that are not accumulated into start as NaN), then the
same rows in launches of 197 rows, small enough for the tiled kernel, and
requires equality bit for bit; one block of rows is also judged against the
oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from numerics import require_close, require_close_scaled, require_exact

pytestmark = pytest.mark.gpu

CASES = [
    # m, n, k, bias, gelu, accumulate, alpha, lda pad, ldc pad
    (6304, 768, 192, True, True, False, 1.0, 0, 0),      # ViT-Tiny FC1 + GELU
    (6304, 576, 192, True, False, False, 1.0, 0, 0),     # QKV
    (6304, 192, 192, True, False, True, 1.0, 0, 0),      # projection into the residual
    (6304, 192, 768, True, False, True, 1.0, 0, 0),      # FC2 into the residual
    (4099, 196, 192, False, True, True, 0.75, 8, 4),     # M and N tails, GELU + accumulate, alpha
    (5000, 580, 768, True, True, False, -1.25, 4, 0),    # 48 k-blocks, N tail, alpha
    (4111, 392, 192, True, False, False, 2.0, 0, 12),    # a partial last panel, padded C rows
]


@pytest.mark.parametrize("m,n,k,with_bias,gelu,accumulate,alpha,lda_pad,ldc_pad", CASES)
def test_panel_equals_the_tiled_kernel(cuvit, oracle, device, m, n, k, with_bias, gelu, accumulate,
                                       alpha, lda_pad, ldc_pad):
    lda, ldc = k + lda_pad, n + ldc_pad
    g = oracle.generator(m + 3 * n + 7 * k)
    a = g.normal(m * lda)
    w = g.normal(n * k, 0.0, 0.05)
    bias = g.normal(n, 0.0, 0.5) if with_bias else None
    start_c = g.normal(m * ldc) if accumulate else np.full(m * ldc, np.nan, np.float32)
    da, dw = to_device(a, device), to_device(w, device)
    dbias = to_device(bias, device) if with_bias else None

    def problem(rows):
        p = cuvit.gemm_problem(rows, n, k, cuvit.TRANSPOSED)
        p.alpha = alpha
        p.lda, p.ldc = lda, ldc
        p.epilogue.gelu = int(gelu)
        p.epilogue.accumulate = int(accumulate)
        return p

    c = to_device(start_c, device)
    cuvit.gemm(da, dw, dbias, c, problem(m))
    full = to_host(c).reshape(m, ldc)[:, :n]
    rows = 197
    for start in range(0, m, rows):
        count = min(rows, m - start)
        part = to_device(start_c[start * ldc:(start + count) * ldc], device)
        cuvit.gemm(da[start * lda:], dw, dbias, part, problem(count))
        require_exact(to_host(part).reshape(count, ldc)[:, :n], full[start:start + count],
                      f"rows {start}..{start + count} differ from launches of {rows} rows")
    last = m - 64
    sample = np.ascontiguousarray(a.reshape(m, lda)[last:, :k])
    pre = oracle.gemm_transposed(sample, w, bias, 64, n, k, alpha)
    scale = oracle.term_magnitudes(sample, w, 64, n, k, True, alpha)
    value = oracle.gelu(pre) if gelu else pre
    existing = start_c.reshape(m, ldc)[last:, :n]
    if gelu:
        expected = existing + value if accumulate else value
        require_close(full[last:], expected, "last 64 rows against the oracle", 1.0e-4, 1.0e-5)
    else:
        expected = existing + value if accumulate else value
        require_close_scaled(full[last:], expected, scale, "last 64 rows against the oracle",
                             1.0e-6, 1.0e-5)
    padding = to_host(c).reshape(m, ldc)[:, n:]
    require_exact(padding, start_c.reshape(m, ldc)[:, n:], "the columns past N changed")


def test_panel_runs_a_shared_weight_batch_as_one_problem(cuvit, oracle, device):
    """A batch of 32 entries of 196 rows with B shared and A rows following one
    another (the ViT-Tiny patch embedding's shape, 6272 x 192 x 768) runs as
    one problem on the panel kernel; each entry lands at its own C stride (197
    rows apart, so one row per entry is never written) and equals its own
    launch of 196 rows, bit for bit."""
    entries, m, n, k = 32, 196, 192, 768
    g = oracle.generator(4242)
    a = g.normal(entries * m * k)
    w = g.normal(n * k, 0.0, 0.05)
    bias = to_device(g.normal(n, 0.0, 0.5), device)
    start = g.normal(entries * (m + 1) * n)
    da, dw = to_device(a, device), to_device(w, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.batch.count, p.batch.stride_a, p.batch.stride_b, p.batch.stride_c = entries, m * k, 0, (m + 1) * n
    c = to_device(start, device)
    cuvit.gemm(da, dw, bias, c, p)
    full = to_host(c).reshape(entries, m + 1, n)
    require_exact(full[:, m], start.reshape(entries, m + 1, n)[:, m], "the rows between entries changed")
    single = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    one = torch.full((m * n,), float("nan"), device=device)
    for entry in (0, 1, 17, 31):
        cuvit.gemm(da[entry * m * k:], dw, bias, one, single)
        require_exact(to_host(one).reshape(m, n), full[entry, :m], f"batch entry {entry}")
