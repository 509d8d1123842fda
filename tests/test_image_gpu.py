"""The preprocessing kernel on the GPU, bit-exact against the oracle (itself
bit-exact against the reference's src/runtime/image.cpp): every geometry of
image_support.GEOMETRIES, batches of distinct images in one launch, a batch
wider than one grid dimension, a side stream, and the reference's own
image_test cases (tests/image_test.cu:122-200) run through the kernel.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from image_support import GEOMETRIES, random_pixels

pytestmark = pytest.mark.gpu


def run(cuvit, device, images: np.ndarray, settings, stream=None) -> np.ndarray:
    """images [batch, height, width, 3] uint8 -> [batch, 3, size, size]."""
    batch, height, width, _ = images.shape
    size = settings.size
    pixels = to_device(images, device)
    tensor = torch.full((batch * 3 * size * size,), float("nan"), device=device)
    cuvit.preprocess(pixels, tensor, batch, width, height, settings, stream=stream)
    return to_host(tensor).reshape(batch, 3, size, size)


def bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("index", range(len(GEOMETRIES)))
def test_matches_the_oracle_bitwise(cuvit, oracle, device, index):
    height, width, size, crop, mean, std = GEOMETRIES[index]
    print(f"preprocess {height}x{width} -> {size}, crop {crop}", flush=True)
    pixels = random_pixels(200 + index, height, width)
    settings = cuvit.Preprocessing(size, crop, mean, std)
    actual = run(cuvit, device, pixels[None], settings)[0]
    expected = oracle.preprocess(pixels, size, crop, mean, std)
    assert np.array_equal(bits(actual), bits(expected))


def test_batch_of_distinct_images(cuvit, oracle, device):
    """One launch over five images of one size: each slot is its own image."""
    images = np.stack([random_pixels(300 + i, 250, 330) for i in range(5)])
    settings = cuvit.Preprocessing()
    actual = run(cuvit, device, images, settings)
    for i in range(5):
        assert np.array_equal(bits(actual[i]), bits(oracle.preprocess(images[i])))


def test_batch_beyond_one_grid_dimension(cuvit, oracle, device):
    """70,000 one-pixel images at size 2 (the one-pixel-per-thread kernel):
    more images than the grid's y extent, so the kernel's image loop runs
    more than once per workgroup."""
    batch = 70000
    images = np.random.default_rng(7).integers(0, 256, (batch, 1, 1, 3), dtype=np.uint8)
    settings = cuvit.Preprocessing(size=2, crop_fraction=1.0)
    actual = run(cuvit, device, images, settings)
    # A 1x1 image samples its only pixel everywhere.
    value = (images[:, 0, 0, :].astype(np.float32) / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)
    expected = np.broadcast_to(value[:, :, None, None], actual.shape)
    assert np.array_equal(bits(actual), bits(expected))
    for i in (0, 65534, 65535, 65536, batch - 1):
        assert np.array_equal(bits(actual[i]), bits(oracle.preprocess(images[i], 2, 1.0)))


def test_batch_beyond_one_grid_dimension_vector_kernel(cuvit, oracle, device):
    """The same on the vector kernel (two output pixels a thread): 70,000
    images of 2 x 1 pixels at size 4."""
    batch = 70000
    images = np.random.default_rng(8).integers(0, 256, (batch, 1, 2, 3), dtype=np.uint8)
    settings = cuvit.Preprocessing(size=4, crop_fraction=1.0)
    actual = run(cuvit, device, images, settings)
    assert not np.isnan(actual).any()
    for i in (0, 1, 65534, 65535, 65536, 65537, batch - 1):
        assert np.array_equal(bits(actual[i]), bits(oracle.preprocess(images[i], 4, 1.0))), i


def test_unaligned_tensor_takes_the_scalar_kernel(cuvit, oracle, device):
    """A tensor 4 bytes past a 16-byte boundary does not take the vector
    kernel's stores: the one-pixel-per-thread kernel runs, with the same bits."""
    pixels = random_pixels(13, 150, 170)
    storage = torch.full((3 * 224 * 224 + 1,), float("nan"), device=device)
    cuvit.preprocess(to_device(pixels[None], device), storage[1:], 1, 170, 150,
                     cuvit.Preprocessing())
    actual = to_host(storage)[1:].reshape(3, 224, 224)
    assert np.isnan(to_host(storage)[0])
    assert np.array_equal(bits(actual), bits(oracle.preprocess(pixels)))


def test_side_stream(cuvit, oracle, device):
    pixels = random_pixels(11, 400, 300)
    stream = torch.cuda.Stream()
    settings = cuvit.Preprocessing(size=96)
    with torch.cuda.stream(stream):
        actual = run(cuvit, device, pixels[None], settings, stream=stream)[0]
    assert np.array_equal(bits(actual), bits(oracle.preprocess(pixels, 96)))


def test_host_convenience_form(cuvit, oracle, device):
    """preprocess_image: the reference's preprocess(image) signature."""
    pixels = random_pixels(12, 123, 321)
    image = cuvit.RgbImage(321, 123, pixels)
    assert np.array_equal(bits(cuvit.preprocess_image(image)), bits(oracle.preprocess(pixels)))


def test_reference_image_test_cases(cuvit, device):
    """image_test.cu:122-200 through the kernel."""
    settings = cuvit.Preprocessing()
    expected_grey = (np.float32(128.0) / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)

    grey = np.full((1, 300, 300, 3), 128, np.uint8)
    tensor = run(cuvit, device, grey, settings)[0]
    assert tensor.shape == (3, 224, 224)
    assert np.all(np.abs(tensor - expected_grey) < 1.0e-5)

    planar = np.zeros((1, 256, 256, 3), np.uint8)
    planar[..., 0], planar[..., 2] = 255, 128
    tensor = run(cuvit, device, planar, settings)[0]
    assert np.all(np.abs(tensor[0] - 1.0) < 1.0e-5)
    assert np.all(np.abs(tensor[1] + 1.0) < 1.0e-5)
    assert np.all(np.abs(tensor[2] - expected_grey) < 1.0e-5)

    band = np.zeros((1, 200, 600, 3), np.uint8)
    band[:, :, 250:350, :] = 255
    tensor = run(cuvit, device, band, settings)[0]
    assert tensor[0, 112, 112] > 0.9
    assert tensor[0, 0, 0] < -0.9 and tensor[0, -1, -1] < -0.9


def test_empty_batch_touches_nothing(cuvit, device):
    tensor = torch.full((12,), 7.0, device=device)
    cuvit.preprocess(None, tensor, 0, 2, 2, cuvit.Preprocessing(size=2))
    assert np.all(to_host(tensor) == 7.0)


def test_preprocess_then_forward_matches_the_oracle(cuvit, oracle, device, tmp_path):
    """The pixels-to-logits path of the cu-vit program at the small model
    configuration: kernel preprocessing into the model's input, then the
    forward pass, against the oracle's preprocess and forward."""
    from numerics import require_close
    from vit_support import random_weights, small_config, write_weights

    config = small_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, 4321)
    path = str(tmp_path / "small.cvw")
    write_weights(cuvit, tensors, path)
    weights = cuvit.WeightFile(path)
    model = cuvit.VisionTransformer(config, weights, 2)
    images = np.stack([random_pixels(40 + i, 45, 60) for i in range(2)])
    settings = cuvit.Preprocessing(size=config.image_size)
    pixels = to_device(images, device)
    tensor = torch.empty(2 * 3 * config.image_size ** 2, device=device)
    cuvit.preprocess(pixels, tensor, 2, 60, 45, settings)
    logits = torch.empty(2 * config.classes, device=device)
    model.forward(tensor, logits, 2)
    actual = to_host(logits).reshape(2, config.classes)
    for i in range(2):
        image = oracle.preprocess(images[i], config.image_size)
        expected = oracle.vit_forward(config, [t for _, t in tensors], image.reshape(-1))
        require_close(actual[i], expected, "preprocess + forward differs from the oracle",
                      1.0e-4, 1.0e-4)
    model.close()
    weights.close()
