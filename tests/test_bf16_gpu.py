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

from conftest import bf16_bits, bf16_tensor, to_device, to_host
from numerics import TestFailure, require_close, require_exact
from oracle import bf16_to_float

pytestmark = pytest.mark.gpu

RTOL = 1.0e-2


def bf16_inputs(oracle, seed, count, mean=0.0, stddev=1.0):
    bits = oracle.round_bf16(oracle.generator(seed).normal(count, mean, stddev))
    return bits, bf16_to_float(bits)


@pytest.mark.parametrize("rows,columns", [(12608, 768), (197, 768), (1, 192), (6304, 192),
                                          (5, 31), (3, 1), (7, 2056),
                                          # more row groups than wavefronts: each
                                          # wavefront reads its next group ahead
                                          (40003, 768)])
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
                                          (2, 1500), (4, 1), (16, 3), (24, 128), (40, 65)])
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


@pytest.mark.parametrize("batch,channels,height", [
    (1, 3, 224),    # 42 strips: whole groups of three
    (1, 1, 224),    # 14 strips: the last group of three holds two
    (5, 1, 96),     # one channel, 6 strips per image, not square
    (7, 2, 32),     # two strips per plane, the last group holds one
    (200, 3, 224),  # 8400 strips: persistent workgroups take several turns
])
def test_extract_patches_bf16_staged_strips(cuvit, oracle, device, batch, channels, height):
    """bf16 images 224 wide in 16 x 16 patches take the LDS-staged strip
    kernel (three strips a turn, persistent workgroups); every strip count and
    turn count must land bit for bit where the oracle's permutation puts it."""
    width = 224
    bits, _ = bf16_inputs(oracle, 507 + batch, batch * channels * height * width)
    expected = oracle.extract_patches(bits.astype(np.float32), batch, channels, height, width,
                                      16).astype(np.uint16)
    x = bf16_tensor(bits, device)
    y = torch.full_like(x, float("nan"))
    cuvit.extract_patches(x, y, batch, channels, height, width, 16)
    require_exact(bf16_bits(y).reshape(expected.shape), expected, "staged bf16 patch gather")


@pytest.mark.parametrize("batch,channels,height,width,patch,offset", [
    (64, 3, 224, 224, 16, 0),  # ViT-Base/16 batch 64: two 16-byte vectors per patch row
    (3, 3, 64, 64, 32, 0),     # four vectors per patch row
    (2, 1, 128, 128, 64, 0),   # eight vectors per patch row, one channel
    (2, 4, 96, 96, 32, 0),     # four channels, 3 x 3 patches
    (3, 2, 40, 40, 8, 0),      # one vector per patch row
    (3, 3, 64, 160, 32, 0),    # non-square: 2 x 5 patches of four vectors a row
    (2, 2, 192, 64, 64, 0),    # non-square: 3 x 1 patches of eight vectors a row
    (5, 3, 48, 80, 16, 0),     # non-square: 3 x 5 patches, two vectors a row
    (2, 3, 64, 64, 32, 1),     # images one float off 16-byte alignment (element kernel)
    (2, 3, 36, 36, 12, 0),     # a patch width that is not a multiple of 8 (element kernel)
])
def test_extract_patches_f32_to_bf16_one_pass(cuvit, oracle, device, batch, channels, height, width,
                                              patch, offset):
    """fp32 images into bf16 patch rows in one pass: bitwise the conversion
    followed by the bf16 gather, and bitwise the oracle's gather of the
    images rounded to nearest-even (ties, signed zeros and infinities
    planted)."""
    count = batch * channels * height * width
    images = oracle.generator(515 + height + width + patch).normal(count, 0.0, 2.0)
    images[::97] = np.float32(1.0 + 2.0 ** -8)    # halfway between two bf16 values: even
    images[5::97] = np.float32(1.0 + 3 * 2.0 ** -8)  # halfway: rounds up to even
    images[7::211] = -0.0
    images[11::509] = np.inf
    images[13::509] = -np.inf
    flat = to_device(images, device)
    if offset:
        shifted = torch.empty(count + offset, device=device)
        shifted[offset:] = flat
        flat = shifted[offset:]
    one_pass = torch.empty(count, dtype=torch.bfloat16, device=device)
    cuvit.extract_patches_f32_to_bf16(flat, one_pass, batch, channels, height, width, patch)
    converted = torch.empty(count, dtype=torch.bfloat16, device=device)
    cuvit.convert_to_bf16(flat, converted, count)
    two_pass = torch.empty_like(converted)
    cuvit.extract_patches(converted, two_pass, batch, channels, height, width, patch)
    got = bf16_bits(one_pass)
    require_exact(got, bf16_bits(two_pass), "one-pass gather vs conversion then bf16 gather")
    expected = oracle.round_bf16(oracle.extract_patches(images, batch, channels, height, width, patch))
    require_exact(got, expected.reshape(-1), "one-pass gather vs the oracle's rounded gather")


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


def test_gemm_bf16_vit_base_fc1_rows_equal_small_launches(cuvit, oracle, device):
    """FC1 of ViT-Base at batch 64 (M=12608, N=3072, K=768, GELU): the full
    launch, whose output starts as NaN, equals bitwise 64 launches of one
    image's 197 rows each. Every tile of the tall launch is thus written and
    placed, and with the per-image launches judged against the oracle (here
    the first and last, and every row in the C5 configuration test), the
    whole output is pinned. Tiles run K in the same order whatever the
    problem height, which is what makes the equality exact."""
    m, n, k = 12608, 3072, 768
    a_bits, a = bf16_inputs(oracle, 505, m * k)
    w_bits, w = bf16_inputs(oracle, 507, n * k, 0.0, 0.02)
    bias = oracle.generator(508).normal(n, 0.0, 0.02)
    da, dw, db = bf16_tensor(a_bits, device), bf16_tensor(w_bits, device), to_device(bias, device)
    c = torch.full((m * n,), float("nan"), dtype=torch.bfloat16, device=device)
    problem = cuvit.gemm_problem(m, n, k, 1)
    problem.epilogue.gelu = 1
    cuvit.gemm(da, dw, db, c, problem)
    full = bf16_bits(c).reshape(m, n)
    rows = 197
    part = torch.full((rows * n,), float("nan"), dtype=torch.bfloat16, device=device)
    small = cuvit.gemm_problem(rows, n, k, 1)
    small.epilogue.gelu = 1
    for image in range(m // rows):
        cuvit.gemm(da[image * rows * k:], dw, db, part, small)
        require_exact(bf16_bits(part).reshape(rows, n), full[image * rows:(image + 1) * rows],
                      f"FC1 rows of image {image} differ from a launch of that image alone")
        if image in (0, m // rows - 1):
            sample = a.reshape(m, k)[image * rows:(image + 1) * rows]
            pre = oracle.gemm_transposed(sample, w, bias, rows, n, k)
            scale = oracle.term_magnitudes(sample, w, rows, n, k, True)
            require_gemm_close(bf16_to_float(bf16_bits(part)).reshape(rows, n), oracle.gelu(pre),
                               scale, f"ViT-Base FC1 + GELU (bf16), image {image}")


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


# -- storage conversion and the bf16 broadcast (extensions) ----------------------

SPECIALS = np.array([0.0, -0.0, 1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.0e38,
                     np.finfo(np.float32).max, np.inf, -np.inf, np.nan, 1e-40, -1e-45,
                     np.finfo(np.float32).tiny], np.float32)


@pytest.mark.parametrize("count,offset", [(1 << 20, 0), (4099, 0), (4099, 3), (7, 1), (1, 0)])
def test_convert_to_bf16_rounds_like_the_oracle(cuvit, oracle, device, count, offset):
    """Nearest-even rounding, bit-exact against the oracle's round_bf16 (pinned
    to torch's float32 -> bfloat16), ties and specials included; offsets
    exercise the unaligned scalar path and the vector tail."""
    values = oracle.generator(900 + count).normal(count, 0.0, 50.0)
    values[:min(count, SPECIALS.size)] = SPECIALS[:min(count, SPECIALS.size)]
    x = to_device(np.concatenate([np.zeros(offset, np.float32), values]), device)[offset:]
    y = torch.empty(count + 1, dtype=torch.bfloat16, device=device)[1:] if offset else \
        torch.empty(count, dtype=torch.bfloat16, device=device)
    cuvit.convert_to_bf16(x, y, count)
    actual, expected = bf16_bits(y), oracle.round_bf16(values)
    nan = np.isnan(values)
    require_exact(actual[~nan], expected[~nan], f"fp32 -> bf16 conversion, {count} at +{offset}")
    if nan.any():
        assert np.all((actual[nan] & 0x7F80) == 0x7F80) and np.all((actual[nan] & 0x7F) != 0)


@pytest.mark.parametrize("count,offset", [(1 << 20, 0), (4099, 0), (4099, 5), (3, 1)])
def test_convert_to_f32_is_exact(cuvit, oracle, device, count, offset):
    bits = oracle.generator(910 + count).integers(count + offset, 0, 1 << 16).astype(np.uint16)
    bits[offset] = 0x7FC1  # a NaN payload survives widening
    x = bf16_tensor(bits, device)[offset:]
    y = torch.empty(count, device=device)
    cuvit.convert_to_f32(x, y, count)
    actual = to_host(y).view(np.uint32)
    require_exact(actual, bits[offset:].astype(np.uint32) << 16, "bf16 -> fp32 widening")


@pytest.mark.parametrize("count,stride,batch", [(768, 197 * 768, 64), (192, 197 * 192, 32),
                                                (24, 17 * 24, 5), (7, 11, 3), (768, 768, 1)])
def test_broadcast_bf16_bit_exact(cuvit, oracle, device, count, stride, batch):
    """broadcast (normalization.cu:194-201) moving bf16 bits; whatever lies
    between the slots is left alone."""
    source = oracle.generator(920 + count).integers(count, 0, 1 << 16).astype(np.uint16)
    destination = oracle.generator(921).integers(stride * batch, 0, 1 << 16).astype(np.uint16)
    expected = destination.copy().reshape(batch, stride)
    expected[:, :count] = source
    d = bf16_tensor(destination, device)
    cuvit.broadcast(d, bf16_tensor(source, device), count, stride, batch)
    require_exact(bf16_bits(d), expected.reshape(-1), "bf16 broadcast")


# -- rounding-boundary parity ----------------------------------------------------

def ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 ulps between two arrays of bf16 bit patterns."""
    def ordered(bits):
        bits = bits.astype(np.int32)
        return np.where(bits & 0x8000, -(bits & 0x7FFF), bits & 0x7FFF)
    return np.abs(ordered(a_bits) - ordered(b_bits))


def require_rounded(oracle, actual_bits, expected, context, max_fraction=1.0e-3, max_ulp=None):
    """The GPU's bf16 bits equal the oracle's fp32 result rounded to bf16,
    except where the two fp32 values straddle a rounding boundary because the
    sums ran in a different order: at most @p max_fraction of the values (one
    flip each is ~1e-5 to 2e-4 of the values in practice)."""
    distance = ulp_distance(actual_bits.reshape(-1), oracle.round_bf16(expected.reshape(-1)))
    fraction = np.count_nonzero(distance) / distance.size
    if fraction > max_fraction:
        raise TestFailure(f"{context}: {fraction:.2e} of the values differ from the rounded oracle")
    if max_ulp is not None and distance.max() > max_ulp:
        raise TestFailure(f"{context}: a value is {distance.max()} ulps from the rounded oracle")


@pytest.mark.parametrize("rows,columns", [(6304, 192), (394, 768)])
def test_layer_norm_bf16_rounds_like_the_oracle(cuvit, oracle, device, rows, columns):
    bits, values = bf16_inputs(oracle, 940 + columns, rows * columns)
    g = oracle.generator(941)
    gamma, beta = g.normal(columns, 1.0, 0.02), g.normal(columns, 0.0, 0.02)
    y = torch.empty(rows * columns, dtype=torch.bfloat16, device=device)
    cuvit.layer_norm(bf16_tensor(bits, device), to_device(gamma, device), to_device(beta, device),
                     y, rows, columns, 1e-6)
    expected = oracle.layer_norm(values.reshape(rows, columns), gamma, beta, 1e-6)
    # no ulp bound: where beta cancels the normalized term, the result is near
    # zero and one fp32 ulp of the inputs is several bf16 ulps of it
    require_rounded(oracle, bf16_bits(y), expected, "bf16 layer norm")


@pytest.mark.parametrize("stddev", [0.3, 3.0])
def test_softmax_bf16_rounds_like_the_oracle(cuvit, oracle, device, stddev):
    rows = 32 * 3 * 197
    bits, values = bf16_inputs(oracle, 950, rows * 197, 0.0, stddev)
    x = bf16_tensor(bits, device)
    cuvit.softmax(x, x, rows, 197)
    require_rounded(oracle, bf16_bits(x), oracle.softmax(values.reshape(rows, 197)),
                    "bf16 softmax in place", max_ulp=1)


@pytest.mark.parametrize("m,n,k,gelu,accumulate", [(6304, 576, 192, 0, 0), (6304, 768, 192, 1, 0),
                                                   (6304, 192, 768, 0, 1), (394, 192, 192, 0, 1),
                                                   (392, 192, 768, 0, 0)])
def test_gemm_bf16_rounds_like_the_oracle(cuvit, oracle, device, m, n, k, gelu, accumulate):
    """The model's GEMM shapes at ViT-Tiny: QKV, FC1 + GELU, FC2 and the
    projection accumulating into the residual stream, the embedding."""
    a_bits, a = bf16_inputs(oracle, 960 + n, m * k)
    b_bits, b = bf16_inputs(oracle, 961 + k, n * k, 0.0, 0.02)
    c_bits, c = bf16_inputs(oracle, 962, m * n)
    bias = oracle.generator(963).normal(n, 0.0, 0.02)
    out = bf16_tensor(c_bits, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.epilogue.gelu, p.epilogue.accumulate = gelu, accumulate
    cuvit.gemm(bf16_tensor(a_bits, device), bf16_tensor(b_bits, device), to_device(bias, device),
               out, p)
    expected = c.copy()
    oracle.gemm_problem_run(a, b, bias, expected, m=m, n=n, k=k, layout=1, accumulate=accumulate,
                            gelu=gelu)
    require_rounded(oracle, bf16_bits(out), expected, f"bf16 GEMM {m}x{n}x{k}")


@pytest.mark.parametrize("k", [192, 520, 768, 1000, 3072])
@pytest.mark.parametrize("gelu,accumulate", [(0, 0), (1, 0), (0, 1)])
def test_gemm_bf16_rows_do_not_depend_on_the_tile(cuvit, oracle, device, k, gelu, accumulate):
    """The same rows inside a tall problem (128 x 128 tile, 32- or 64-deep
    stages by K) and alone (64 x 64 tile, 32- or 64-deep by K) are bitwise
    equal: every bf16 tile walks K over the same k-blocks."""
    m, n = 11008, 768  # 86 x 6 tiles of 128: past the 128 x 128 threshold (two per CU)
    a_bits, _ = bf16_inputs(oracle, 9300 + k, m * k)
    b_bits, _ = bf16_inputs(oracle, 9301 + k, n * k, 0.0, 0.05)
    c_bits, _ = bf16_inputs(oracle, 9302, m * n)
    bias = to_device(oracle.generator(9303).normal(n, 0.0, 0.02), device)
    w = bf16_tensor(b_bits, device)
    p = cuvit.gemm_problem(m, n, k, cuvit.TRANSPOSED)
    p.epilogue.gelu, p.epilogue.accumulate = gelu, accumulate
    tall = bf16_tensor(c_bits, device)
    cuvit.gemm(bf16_tensor(a_bits, device), w, bias, tall, p)
    full = bf16_bits(tall).reshape(m, n)
    for start, rows in ((0, 197), (1000, 5), (m - 1, 1)):
        q = cuvit.gemm_problem(rows, n, k, cuvit.TRANSPOSED)
        q.epilogue.gelu, q.epilogue.accumulate = gelu, accumulate
        piece = bf16_tensor(c_bits[start * n:(start + rows) * n], device)
        cuvit.gemm(bf16_tensor(a_bits[start * k:(start + rows) * k], device), w, bias, piece, q)
        require_exact(bf16_bits(piece).reshape(rows, n), full[start:start + rows],
                      f"bf16 rows {start}..{start + rows} (K {k}) changed with the problem height")
