"""GPU parity for the patch gather, the class-token broadcast and the
positional-embedding add.

The reference has no direct test of these three launchers (they are covered
only end to end through vit_test at a 4x4 patch grid), so the cases here pin
them directly: bit-exact against the oracle on the batch-32 ViT-Tiny geometry
with U(-1,1) images (seed 303), an iota known answer where every output must
equal its own source index, the permutation property, and the other
geometries each code path takes (vector strips, element path, unaligned).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from numerics import TestFailure, require_exact

pytestmark = pytest.mark.gpu


def gather_index_map(batch, channels, height, width, patch):
    """Closed form of the source index of every patch-matrix element
    (include/cuvit/kernels.hpp:125-138): row = (b, py, px), column = (c, ly, lx)."""
    across, down = width // patch, height // patch
    b, py, px, c, ly, lx = np.meshgrid(np.arange(batch), np.arange(down), np.arange(across),
                                       np.arange(channels), np.arange(patch), np.arange(patch),
                                       indexing="ij")
    source = ((b * channels + c) * height + py * patch + ly) * width + px * patch + lx
    return source.reshape(batch * down * across, channels * patch * patch)


GEOMETRIES = [
    (32, 3, 224, 224, 16),  # ViT-Tiny batch 32 (the measured workload)
    (1, 3, 224, 224, 16),
    (5, 3, 32, 32, 8),      # vit_test geometry
    (2, 2, 12, 8, 4),       # one vector per patch row
    (3, 1, 64, 96, 32),     # eight vectors per patch row
    (2, 2, 9, 12, 3),       # patch not a multiple of 4: element path
    (1, 3, 10, 10, 2),
    (2, 3, 14, 21, 7),
]


@pytest.mark.parametrize("geometry", GEOMETRIES)
def test_extract_patches_iota_known_answer(cuvit, device, geometry):
    batch, channels, height, width, patch = geometry
    total = batch * channels * height * width
    assert total < (1 << 24)  # every index is exact in fp32
    images = np.arange(total, dtype=np.float32)
    out = torch.full((total,), -1.0, device=device)
    cuvit.extract_patches(to_device(images, device), out, batch, channels, height, width, patch)
    actual = to_host(out).reshape(-1)
    expected = gather_index_map(batch, channels, height, width, patch).reshape(-1).astype(np.float32)
    require_exact(actual, expected, "patch gather does not place each element at its index")


@pytest.mark.parametrize("geometry", GEOMETRIES)
def test_extract_patches_matches_oracle(cuvit, oracle, device, geometry):
    batch, channels, height, width, patch = geometry
    images = oracle.generator(303).uniform(batch * channels * height * width, -1.0, 1.0)
    expected = oracle.extract_patches(images, batch, channels, height, width, patch)
    out = torch.empty(expected.size, device=device)
    cuvit.extract_patches(to_device(images, device), out, batch, channels, height, width, patch)
    actual = to_host(out).reshape(expected.shape)
    require_exact(actual, expected, "patch gather differs from the CPU reference")
    require_exact(np.sort(actual.reshape(-1)), np.sort(images), "patch gather is not a permutation")


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_extract_patches_unaligned(cuvit, oracle, device, offset):
    batch, channels, height, width, patch = 2, 3, 32, 32, 16
    total = batch * channels * height * width
    images = oracle.generator(77).uniform(total + offset)
    expected = oracle.extract_patches(images[offset:], batch, channels, height, width, patch)
    out = torch.zeros(total + offset, device=device)
    cuvit.extract_patches(to_device(images, device)[offset:], out[offset:], batch, channels,
                          height, width, patch)
    actual = to_host(out)
    require_exact(actual[offset:].reshape(expected.shape), expected, "unaligned gather")
    require_exact(actual[:offset], np.zeros(offset, np.float32), "gather wrote before its range")


def test_class_token_and_positional_add_batch_32(cuvit, oracle, device):
    """The C3 sequence on a zeroed token buffer: cls into row 0 of every image,
    then pos broadcast-added over the batch; bit-exact (one fp32 add each)."""
    batch, tokens, embed = 32, 197, 192
    g = oracle.generator(303)
    g.uniform(batch * 3 * 224 * 224)  # the images come first in this stream
    pos = g.normal(tokens * embed, 0.0, 0.02)
    cls = g.normal(embed, 0.0, 0.02)
    body = oracle.generator(304).normal(batch * tokens * embed)  # stand-in for the embedding GEMM
    expected = body.copy()
    oracle.broadcast(expected, cls, embed, tokens * embed, batch)
    oracle.add_broadcast(expected, pos, tokens * embed, batch)

    dtokens = to_device(body, device)
    cuvit.broadcast(dtokens, to_device(cls, device), embed, tokens * embed, batch)
    cuvit.add_broadcast(dtokens, to_device(pos, device), tokens * embed, batch)
    require_exact(to_host(dtokens), expected, "class token / positional add differ")


@pytest.mark.parametrize("count,stride,batch,offset", [
    (192, 37824, 3, 0), (5, 7, 9, 0), (6, 6, 4, 1), (1, 1, 70000, 0), (4, 8, 2, 2)])
def test_broadcast_shapes(cuvit, oracle, device, count, stride, batch, offset):
    size = stride * batch + offset
    destination = oracle.generator(count * 13 + batch).normal(size)
    source = oracle.generator(count).normal(count)
    expected = destination.copy()
    oracle.broadcast(expected[offset:], source, count, stride, batch)
    d = to_device(destination, device)
    cuvit.broadcast(d[offset:], to_device(source, device), count, stride, batch)
    require_exact(to_host(d), expected, "broadcast")


@pytest.mark.parametrize("count,batch,offset", [(37824, 32, 0), (7, 5, 0), (12, 3, 1),
                                               (3, 70000, 0), (1, 1, 0)])
def test_add_broadcast_shapes(cuvit, oracle, device, count, batch, offset):
    accumulator = oracle.generator(count + batch).normal(count * batch + offset)
    addend = oracle.generator(count * 3).normal(count)
    expected = accumulator.copy()
    oracle.add_broadcast(expected[offset:], addend, count, batch)
    d = to_device(accumulator, device)
    cuvit.add_broadcast(d[offset:], to_device(addend, device), count, batch)
    require_exact(to_host(d), expected, "add_broadcast")


def test_invalid_arguments(cuvit, device):
    buffer = torch.zeros(64, device=device)
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.broadcast(buffer, buffer, 8, 4, 2)  # stride < count
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.extract_patches(buffer, buffer, 1, 1, 6, 6, 4)  # not whole patches
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.add_broadcast(None, buffer, 4, 1)
    cuvit.extract_patches(None, None, 0, 3, 224, 224, 16)  # empty batch: no-op
    cuvit.broadcast(None, None, 0, 0, 5)
