"""Fused attention (an extension): softmax(Q.K^T / sqrt(64)).V per (image, head).

It must equal, bit for bit, the reference's three launches (vit.cu:205-245)
run through this library: the split-batch Q.K^T GEMM with alpha 1/8, softmax
in place, and the weights.V GEMM into the context layout. Against the oracle
(the reference CPU path: gemm_transposed, softmax, gemm) it is held to the
same term-scaled tolerance as the GEMMs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from numerics import require_close_scaled, require_exact

pytestmark = pytest.mark.gpu

HEAD_DIM = 64


def unfused(cuvit, qkv, images, heads, tokens, device):
    """The launcher sequence of the model's attention (vit.cu:205-245)."""
    embed = heads * HEAD_DIM
    row = 3 * embed
    logits = torch.zeros(images * heads * tokens * tokens, device=device)
    p = cuvit.gemm_problem(tokens, tokens, HEAD_DIM, cuvit.TRANSPOSED)
    p.alpha = 1.0 / np.sqrt(np.float32(HEAD_DIM))
    p.lda, p.ldb, p.ldc = row, row, tokens
    b = p.batch
    b.count, b.inner = images * heads, heads
    b.stride_a, b.stride_b, b.stride_c = HEAD_DIM, HEAD_DIM, tokens * tokens
    b.outer_stride_a = b.outer_stride_b = tokens * row
    b.outer_stride_c = heads * tokens * tokens
    cuvit.gemm(qkv, qkv[embed:], None, logits, p)
    cuvit.softmax(logits, logits, images * heads * tokens, tokens)
    context = torch.zeros(images * tokens * embed, device=device)
    p = cuvit.gemm_problem(tokens, HEAD_DIM, tokens, cuvit.NO_TRANSPOSE)
    p.lda, p.ldb, p.ldc = tokens, row, embed
    b = p.batch
    b.count, b.inner = images * heads, heads
    b.stride_a, b.stride_b, b.stride_c = tokens * tokens, HEAD_DIM, HEAD_DIM
    b.outer_stride_a = heads * tokens * tokens
    b.outer_stride_b = tokens * row
    b.outer_stride_c = tokens * embed
    cuvit.gemm(logits, qkv[2 * embed:], None, context, p)
    return context


@pytest.mark.parametrize("images,heads,tokens", [(32, 3, 197), (2, 12, 197), (3, 2, 17), (1, 1, 1),
                                                 (2, 3, 16), (2, 3, 65), (1, 2, 256), (4, 1, 200)])
def test_fused_attention_is_bitwise_the_launch_sequence(cuvit, oracle, device, images, heads, tokens):
    embed = heads * HEAD_DIM
    qkv = to_device(oracle.generator(7000 + tokens).normal(images * tokens * 3 * embed), device)
    expected = unfused(cuvit, qkv, images, heads, tokens, device)
    context = torch.full((images * tokens * embed,), float("nan"), device=device)
    cuvit.attention(qkv, context, images, heads, tokens, HEAD_DIM)
    require_exact(to_host(context), to_host(expected),
                  f"fused attention {images}x{heads}x{tokens} differs from the launch sequence")


@pytest.mark.parametrize("key_tiles", range(1, 17))
def test_every_key_tile_count_is_bitwise_the_launch_sequence(cuvit, oracle, device, key_tiles):
    """The fp32 kernel is one instance per count of 16-key tiles: each, with
    a full last tile and with one holding 9 keys."""
    images, heads = 2, 2
    embed = heads * HEAD_DIM
    for tokens in (16 * key_tiles, 16 * key_tiles - 7):
        qkv = to_device(oracle.generator(7200 + tokens).normal(images * tokens * 3 * embed), device)
        expected = unfused(cuvit, qkv, images, heads, tokens, device)
        context = torch.full((images * tokens * embed,), float("nan"), device=device)
        cuvit.attention(qkv, context, images, heads, tokens, HEAD_DIM)
        require_exact(to_host(context), to_host(expected),
                      f"fused attention {images}x{heads}x{tokens} differs from the launch sequence")


def test_fused_attention_matches_the_oracle(cuvit, oracle, device):
    images, heads, tokens = 2, 3, 37
    embed = heads * HEAD_DIM
    row = 3 * embed
    qkv = oracle.generator(7100).normal(images * tokens * row).reshape(images, tokens, 3, heads,
                                                                          HEAD_DIM)
    expected = np.zeros((images, tokens, heads, HEAD_DIM), np.float32)
    scale = np.zeros_like(expected)
    for i in range(images):
        for h in range(heads):
            q = np.ascontiguousarray(qkv[i, :, 0, h])
            k = np.ascontiguousarray(qkv[i, :, 1, h])
            v = np.ascontiguousarray(qkv[i, :, 2, h])
            logits = oracle.gemm_transposed(q, k, None, tokens, tokens, HEAD_DIM) * np.float32(0.125)
            weights = oracle.softmax(logits)
            expected[i, :, h] = oracle.gemm(weights, v, None, tokens, HEAD_DIM, tokens)
            scale[i, :, h] = oracle.gemm(np.abs(weights), np.abs(v), None, tokens, HEAD_DIM, tokens)
    context = torch.zeros(expected.size, device=device)
    cuvit.attention(to_device(qkv.reshape(-1), device), context, images, heads, tokens, HEAD_DIM)
    require_close_scaled(to_host(context), expected.reshape(-1), scale.reshape(-1),
                         "fused attention vs oracle", 1.0e-5, 1.0e-6)


def test_fused_attention_rows_are_batch_invariant(cuvit, oracle, device):
    """Each (image, head) gives the same bits alone as inside a batch."""
    images, heads, tokens = 5, 3, 197
    embed = heads * HEAD_DIM
    per_image = tokens * 3 * embed
    qkv = to_device(oracle.generator(7200).normal(images * per_image), device)
    full = torch.zeros(images * tokens * embed, device=device)
    cuvit.attention(qkv, full, images, heads, tokens, HEAD_DIM)
    for i in (0, 3):
        one = torch.zeros(tokens * embed, device=device)
        cuvit.attention(qkv[i * per_image:(i + 1) * per_image].clone(), one, 1, heads, tokens, HEAD_DIM)
        require_exact(to_host(one), to_host(full[i * tokens * embed:(i + 1) * tokens * embed]),
                      f"image {i} differs alone")


# -- bf16 (an extension of the extension) ---------------------------------------

def unfused_bf16(cuvit, qkv, images, heads, tokens, device):
    """The bf16 model's launch sequence: the bf16 GEMM, softmax and GEMM twins."""
    embed = heads * HEAD_DIM
    row = 3 * embed
    logits = torch.zeros(images * heads * tokens * tokens, device=device, dtype=torch.bfloat16)
    p = cuvit.gemm_problem(tokens, tokens, HEAD_DIM, cuvit.TRANSPOSED)
    p.alpha = 1.0 / np.sqrt(np.float32(HEAD_DIM))
    p.lda, p.ldb, p.ldc = row, row, tokens
    b = p.batch
    b.count, b.inner = images * heads, heads
    b.stride_a, b.stride_b, b.stride_c = HEAD_DIM, HEAD_DIM, tokens * tokens
    b.outer_stride_a = b.outer_stride_b = tokens * row
    b.outer_stride_c = heads * tokens * tokens
    cuvit.gemm(qkv, qkv[embed:], None, logits, p)
    cuvit.softmax(logits, logits, images * heads * tokens, tokens)
    context = torch.zeros(images * tokens * embed, device=device, dtype=torch.bfloat16)
    p = cuvit.gemm_problem(tokens, HEAD_DIM, tokens, cuvit.NO_TRANSPOSE)
    p.lda, p.ldb, p.ldc = tokens, row, embed
    b = p.batch
    b.count, b.inner = images * heads, heads
    b.stride_a, b.stride_b, b.stride_c = tokens * tokens, HEAD_DIM, HEAD_DIM
    b.outer_stride_a = heads * tokens * tokens
    b.outer_stride_b = tokens * row
    b.outer_stride_c = tokens * embed
    cuvit.gemm(logits, qkv[2 * embed:], None, context, p)
    return context


def bf16_qkv(oracle, seed, count, device, stddev=1.0):
    from conftest import bf16_tensor

    return bf16_tensor(oracle.round_bf16(oracle.generator(seed).normal(count, 0.0, stddev)), device)


@pytest.mark.parametrize("images,heads,tokens", [(64, 12, 197), (32, 3, 197), (2, 12, 197), (3, 2, 17),
                                                 (1, 1, 1), (2, 3, 32), (2, 3, 65), (1, 2, 256),
                                                 (4, 1, 200), (2, 2, 150), (5, 3, 97),
                                                 # the persistent kernel with a runtime count
                                                 (48, 12, 200), (48, 12, 193),
                                                 # and with 1, 2 and 5 key tiles, two or three
                                                 # pairs per workgroup
                                                 (520, 1, 20), (130, 4, 64), (44, 12, 150)])
def test_fused_attention_bf16_is_bitwise_the_launch_sequence(cuvit, oracle, device, images, heads,
                                                             tokens):
    from conftest import bf16_bits

    embed = heads * HEAD_DIM
    qkv = bf16_qkv(oracle, 7300 + tokens, images * tokens * 3 * embed, device)
    expected = unfused_bf16(cuvit, qkv, images, heads, tokens, device)
    context = torch.full((images * tokens * embed,), float("nan"), device=device, dtype=torch.bfloat16)
    cuvit.attention(qkv, context, images, heads, tokens, HEAD_DIM)
    require_exact(bf16_bits(context), bf16_bits(expected),
                  f"bf16 fused attention {images}x{heads}x{tokens} differs from the launch sequence")


@pytest.mark.parametrize("images,heads", [(2, 3), (64, 12)])
@pytest.mark.parametrize("stddev", [1.1e-19, 1.0e-10, 30.0])
def test_fused_attention_bf16_extreme_logits_are_bitwise_the_launch_sequence(cuvit, oracle, device,
                                                                            stddev, images, heads):
    """Logits whose scaled values straddle the smallest normal float (inputs
    of about 1e-19: the GEMM rounds sum / 8, the fused kernel folds the 1/8
    into its exponential), tiny normal ones, and large ones whose
    exponentials underflow: the same bits as the three launches, on the
    per-pair kernel (6 pairs) and on the persistent 197-token instance (768)."""
    from conftest import bf16_bits

    tokens = 197
    embed = heads * HEAD_DIM
    qkv = bf16_qkv(oracle, 7500, images * tokens * 3 * embed, device, stddev)
    expected = unfused_bf16(cuvit, qkv, images, heads, tokens, device)
    context = torch.full((images * tokens * embed,), float("nan"), device=device, dtype=torch.bfloat16)
    cuvit.attention(qkv, context, images, heads, tokens, HEAD_DIM)
    require_exact(bf16_bits(context), bf16_bits(expected),
                  f"bf16 fused attention with inputs of scale {stddev} differs from the launch sequence")


def test_fused_attention_bf16_rounds_like_the_oracle(cuvit, oracle, device):
    """Against the oracle's fp32 attention with the bf16 rounding points
    (logits and probabilities rounded as the model stores them): equal bits
    except where GPU and CPU sums straddle a bf16 rounding boundary."""
    from conftest import bf16_bits
    from oracle import bf16_to_float

    images, heads, tokens = 2, 3, 197
    embed = heads * HEAD_DIM
    row = 3 * embed
    bits = oracle.round_bf16(oracle.generator(7400).normal(images * tokens * row, 0.0, 0.5))
    values = bf16_to_float(bits).reshape(images, tokens, 3, heads, HEAD_DIM)
    expected = np.zeros((images, tokens, heads, HEAD_DIM), np.float32)
    for i in range(images):
        for h in range(heads):
            q = np.ascontiguousarray(values[i, :, 0, h])
            k = np.ascontiguousarray(values[i, :, 1, h])
            v = np.ascontiguousarray(values[i, :, 2, h])
            logits = oracle.gemm_transposed(q, k, None, tokens, tokens, HEAD_DIM, np.float32(0.125))
            logits = bf16_to_float(oracle.round_bf16(logits)).reshape(tokens, tokens)
            weights = bf16_to_float(oracle.round_bf16(oracle.softmax(logits))).reshape(tokens, tokens)
            expected[i, :, h] = oracle.gemm(weights, v, None, tokens, HEAD_DIM, tokens).reshape(tokens, HEAD_DIM)
    from conftest import bf16_tensor

    context = torch.zeros(expected.size, device=device, dtype=torch.bfloat16)
    cuvit.attention(bf16_tensor(bits, device), context, images, heads, tokens, HEAD_DIM)
    distance = np.abs(bf16_bits(context).astype(np.int32) -
                      oracle.round_bf16(expected.reshape(-1)).astype(np.int32))
    fraction = np.count_nonzero(distance) / distance.size
    assert fraction <= 1.0e-2, f"{fraction:.2e} of the context differs from the rounded oracle"
