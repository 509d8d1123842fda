"""Operands beyond 2^31 elements: the gather, LayerNorm, softmax, class-token
broadcast, positional add and the GEMM address them with 64-bit offsets. The
reference's launchers take 64-bit counts and reject only grids above 2^31 - 1
blocks (src/kernels/normalization.cu:214-220), so each of these sizes is a
valid call there too. Each test sits just past 2^31 elements and checks the
rows that straddle element 2^31, the first and last rows and a random sample,
against the closed form (gather, broadcast, add: bit-exact) or the oracle
(LayerNorm, softmax, GEMM). At most about 20 GB of device memory per test, freed after it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to_host

pytestmark = pytest.mark.gpu

LIMIT = 2 ** 31
EMBED, TOKENS, IMAGE, PATCH = 192, 197, 224, 16


@pytest.fixture(autouse=True)
def release_memory():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def rows_around(boundary_row: int, rows: int, rng, extra: int = 64) -> np.ndarray:
    """The first and last rows, those around @p boundary_row, and a sample."""
    picked = {0, 1, rows - 2, rows - 1}
    picked.update(range(max(0, boundary_row - 3), min(rows, boundary_row + 4)))
    picked.update(int(r) for r in rng.integers(0, rows, extra))
    return np.array(sorted(picked), dtype=np.int64)


def take_rows(tensor, columns: int, rows: np.ndarray) -> np.ndarray:
    index = torch.from_numpy(rows).to(tensor.device)
    return to_host(tensor.view(-1, columns).index_select(0, index))


def test_gather_beyond_2_31_elements(cuvit, device):
    """Each image element holds its own flat index as bits (mod 2^32), so every
    output element must hold the index of the source element the closed form
    names (vit.hpp:65-87; normalization.cu:168-191)."""
    per_image = 3 * IMAGE * IMAGE
    batch = LIMIT // per_image + 6  # 14272 images
    total = batch * per_image
    assert total > LIMIT
    print(f"gather: {batch} images, {total} elements", flush=True)
    images = torch.empty(total, dtype=torch.int32, device=device)
    chunk = 1 << 28
    for start in range(0, total, chunk):
        end = min(total, start + chunk)
        images[start:end] = torch.arange(start, end, dtype=torch.int64, device=device).to(torch.int32)
    patches = torch.full((total,), -1, dtype=torch.int32, device=device)
    cuvit.extract_patches(images.view(torch.float32), patches.view(torch.float32), batch, 3,
                          IMAGE, IMAGE, PATCH)
    torch.cuda.synchronize()

    rng = np.random.default_rng(31)
    positions = np.concatenate([
        np.arange(0, 4096), np.arange(LIMIT - 4096, LIMIT + 4096), np.arange(total - 4096, total),
        rng.integers(0, total, 1 << 20)]).astype(np.int64)
    row, element = positions // 768, positions % 768
    image, patch = row // 196, row % 196
    channel, within = element // 256, element % 256
    source = (((image * 3 + channel) * IMAGE + (patch // 14) * PATCH + within // PATCH) * IMAGE +
              (patch % 14) * PATCH + within % PATCH)
    expected = source.astype(np.uint64).astype(np.uint32).view(np.int32)
    actual = to_host(patches[torch.from_numpy(positions).to(device)])
    assert np.array_equal(actual, expected)


def test_layer_norm_beyond_2_31_elements(cuvit, oracle, device):
    rows = LIMIT // EMBED + 86  # 11184896 rows
    assert rows * EMBED > LIMIT
    print(f"layer norm: [{rows}, {EMBED}]", flush=True)
    torch.manual_seed(5)
    x = torch.randn(rows * EMBED, device=device)
    gamma = torch.randn(EMBED, device=device) * 0.02 + 1.0
    beta = torch.randn(EMBED, device=device) * 0.02
    y = torch.full_like(x, float("nan"))
    cuvit.layer_norm(x, gamma, beta, y, rows, EMBED, 1e-6)
    torch.cuda.synchronize()
    picked = rows_around(LIMIT // EMBED, rows, np.random.default_rng(32))
    expected = oracle.layer_norm(take_rows(x, EMBED, picked), to_host(gamma), to_host(beta), 1e-6)
    assert np.abs(take_rows(y, EMBED, picked) - expected).max() <= 1.0e-5


def test_softmax_beyond_2_31_elements_in_place(cuvit, oracle, device):
    rows = LIMIT // TOKENS + 66  # 10900998 rows, not a whole number of staged blocks
    assert rows * TOKENS > LIMIT
    print(f"softmax: [{rows}, {TOKENS}] in place", flush=True)
    torch.manual_seed(6)
    logits = torch.randn(rows * TOKENS, device=device)
    picked = rows_around(LIMIT // TOKENS, rows, np.random.default_rng(33))
    expected = oracle.softmax(take_rows(logits, TOKENS, picked))
    cuvit.softmax(logits, logits, rows, TOKENS)
    torch.cuda.synchronize()
    assert np.abs(take_rows(logits, TOKENS, picked) - expected).max() <= 1.0e-5


def test_class_token_and_positional_add_beyond_2_31_elements(cuvit, device):
    """The class token into row 0 of every image (vit.hpp:89-92), then the
    positional table added to every token row (vit.hpp:96-98), one fp32 add
    each: bit-exact."""
    per_image = TOKENS * EMBED
    batch = LIMIT // per_image + 26  # 56801 images
    total = batch * per_image
    assert total > LIMIT
    print(f"class token + positional add: {batch} images, {total} elements", flush=True)
    torch.manual_seed(7)
    tokens = torch.randn(total, device=device)
    cls = torch.randn(EMBED, device=device)
    pos = torch.randn(per_image, device=device)
    picked = rows_around(LIMIT // per_image, batch, np.random.default_rng(34))
    before = take_rows(tokens, per_image, picked).reshape(-1, TOKENS, EMBED)
    cuvit.broadcast(tokens, cls, EMBED, per_image, batch)
    cuvit.add_broadcast(tokens, pos, per_image, batch)
    torch.cuda.synchronize()
    expected = before.copy()
    expected[:, 0, :] = to_host(cls)
    expected = expected + to_host(pos).reshape(TOKENS, EMBED)
    actual = take_rows(tokens, per_image, picked).reshape(-1, TOKENS, EMBED)
    assert np.array_equal(actual.view(np.uint32), expected.astype(np.float32).view(np.uint32))


def test_gemm_gelu_with_a_beyond_2_31_elements(cuvit, oracle, device):
    """FC1's epilogue (bias, erf-GELU) on A [m, 768] with m * 768 > 2^31: the
    rows past element 2^31 of A, and their outputs, against the oracle's
    gemm_transposed + gelu at the GELU tolerance of the GEMM tests."""
    from numerics import require_close

    m, n, k = LIMIT // 768 + 32, 64, 768
    assert m * k > LIMIT
    print(f"gemm + GELU: {m} x {n} x {k}", flush=True)
    torch.manual_seed(8)
    a = torch.randn(m * k, device=device)
    w = torch.randn(n * k, device=device) * 0.02
    bias = torch.randn(n, device=device) * 0.02
    c = torch.full((m * n,), float("nan"), device=device)
    problem = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    problem.epilogue.gelu = 1
    cuvit.gemm(a, w, bias, c, problem)
    torch.cuda.synchronize()
    picked = rows_around(LIMIT // k, m, np.random.default_rng(35))
    pre = oracle.gemm_transposed(take_rows(a, k, picked), to_host(w), to_host(bias), picked.size, n, k)
    require_close(take_rows(c, n, picked), oracle.gelu(pre), "GEMM past 2^31 elements of A",
                  1.0e-4, 1.0e-5)


def test_bf16_gather_beyond_2_31_elements(cuvit, device):
    """The bf16 gather (two 16-byte vectors per patch row) at the element
    count of the fp32 test: each element holds the low 16 bits of its flat
    index, so every output element must hold its source's."""
    per_image = 3 * IMAGE * IMAGE
    batch = LIMIT // per_image + 6
    total = batch * per_image
    print(f"bf16 gather: {batch} images, {total} elements", flush=True)
    images = torch.empty(total, dtype=torch.int16, device=device)
    chunk = 1 << 28
    for start in range(0, total, chunk):
        end = min(total, start + chunk)
        images[start:end] = torch.arange(start, end, dtype=torch.int64, device=device).to(torch.int16)
    patches = torch.full((total,), -1, dtype=torch.int16, device=device)
    cuvit.extract_patches(images.view(torch.bfloat16), patches.view(torch.bfloat16), batch, 3,
                          IMAGE, IMAGE, PATCH)
    torch.cuda.synchronize()
    rng = np.random.default_rng(36)
    positions = np.concatenate([
        np.arange(LIMIT - 4096, LIMIT + 4096), np.arange(total - 4096, total),
        rng.integers(0, total, 1 << 20)]).astype(np.int64)
    row, element = positions // 768, positions % 768
    image, patch = row // 196, row % 196
    channel, within = element // 256, element % 256
    source = (((image * 3 + channel) * IMAGE + (patch // 14) * PATCH + within // PATCH) * IMAGE +
              (patch % 14) * PATCH + within % PATCH)
    expected = source.astype(np.uint64).astype(np.uint16).view(np.int16)
    actual = to_host(patches[torch.from_numpy(positions).to(device)])
    assert np.array_equal(actual, expected)


def test_bf16_softmax_beyond_2_31_elements_in_place(cuvit, oracle, device):
    """The bf16 staged softmax (eight-row blocks) past 2^31 elements, against
    the oracle on the bf16 inputs at the bf16 tolerance."""
    from numerics import require_close
    from oracle import bf16_to_float

    rows = LIMIT // TOKENS + 66
    print(f"bf16 softmax: [{rows}, {TOKENS}] in place", flush=True)
    torch.manual_seed(9)
    logits = torch.randn(rows * TOKENS, device=device).to(torch.bfloat16)
    picked = rows_around(LIMIT // TOKENS, rows, np.random.default_rng(37))
    index = torch.from_numpy(picked).to(device)
    before = to_host(logits.view(-1, TOKENS).index_select(0, index).view(torch.int16))
    expected = oracle.softmax(bf16_to_float(before.view(np.uint16)))
    cuvit.softmax(logits, logits, rows, TOKENS)
    torch.cuda.synchronize()
    after = to_host(logits.view(-1, TOKENS).index_select(0, index).view(torch.int16))
    require_close(bf16_to_float(after.view(np.uint16)), expected, "bf16 softmax past 2^31", 1.0e-2,
                  1.0e-6)


def test_bf16_layer_norm_beyond_2_31_elements(cuvit, oracle, device):
    """The bf16 LayerNorm (fp32 statistics, one rounding at the store) past 2^31
    elements, against the oracle on the bf16 inputs at the bf16 tolerance."""
    from numerics import require_close
    from oracle import bf16_to_float

    rows = LIMIT // EMBED + 86
    print(f"bf16 layer norm: [{rows}, {EMBED}]", flush=True)
    torch.manual_seed(10)
    x = torch.randn(rows * EMBED, device=device).to(torch.bfloat16)
    gamma = torch.randn(EMBED, device=device) * 0.02 + 1.0
    beta = torch.randn(EMBED, device=device) * 0.02
    y = torch.empty_like(x)
    cuvit.layer_norm(x, gamma, beta, y, rows, EMBED, 1e-6)
    torch.cuda.synchronize()
    picked = rows_around(LIMIT // EMBED, rows, np.random.default_rng(38))
    index = torch.from_numpy(picked).to(device)
    inputs = to_host(x.view(-1, EMBED).index_select(0, index).view(torch.int16)).view(np.uint16)
    outputs = to_host(y.view(-1, EMBED).index_select(0, index).view(torch.int16)).view(np.uint16)
    expected = oracle.layer_norm(bf16_to_float(inputs), to_host(gamma), to_host(beta), 1e-6)
    require_close(bf16_to_float(outputs), expected, "bf16 layer norm past 2^31", 1.0e-2, 1.0e-3)
