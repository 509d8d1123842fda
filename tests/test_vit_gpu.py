"""The model driver on the GPU: tests/vit_test.cu's properties, plus the full
ViT-Tiny/16 batch-32 layer-kernel sequence.

Parity is against the oracle's restatement of tests/reference/vit.hpp
(VitReference) at rtol = atol = 1e-4 on the logits (vit_test.cu:128-130).
Determinism, batch invariance and partial-batch invariance are bitwise and
need no oracle (vit_test.cu:134-266).
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from conftest import to_device, to_host
from numerics import TestFailure, require_close, require_exact
from vit_support import random_image, random_weights, small_config, tiny_config, write_weights

pytestmark = pytest.mark.gpu


def build(cuvit, oracle, tmp_path, seed, max_batch=1, config=None, small=True):
    config = config or small_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, seed, small=small)
    path = os.path.join(tmp_path, f"vit_{seed}.cvw")
    write_weights(cuvit, tensors, path)
    weights = cuvit.WeightFile(path)
    model = cuvit.VisionTransformer(config, weights, max_batch)
    return config, tensors, weights, model


def forward(cuvit, model, images: np.ndarray, batch: int, device) -> np.ndarray:
    logits = torch.empty(batch * model.config.classes, device=device)
    model.forward(to_device(images, device), logits, batch)
    return to_host(logits).reshape(batch, model.config.classes)


def test_forward_matches_the_cpu_reference(cuvit, oracle, device, tmp_path):
    """vit_test.cu:108-132."""
    config, tensors, _, model = build(cuvit, oracle, tmp_path, 1234)
    for seed in (1, 2, 3):
        image = random_image(oracle, config, seed)
        actual = forward(cuvit, model, image, 1, device)[0]
        expected = oracle.vit_forward(config, [t for _, t in tensors], image)
        require_close(actual, expected, "forward pass differs from the CPU reference", 1.0e-4, 1.0e-4)


def test_forward_is_deterministic(cuvit, oracle, device, tmp_path):
    """vit_test.cu:134-149."""
    config, _, _, model = build(cuvit, oracle, tmp_path, 77)
    image = random_image(oracle, config, 5)
    first = forward(cuvit, model, image, 1, device)
    second = forward(cuvit, model, image, 1, device)
    require_exact(first, second, "two runs of the same input disagree")


def test_different_inputs_produce_different_logits(cuvit, oracle, device, tmp_path):
    """vit_test.cu:151-172."""
    config, _, _, model = build(cuvit, oracle, tmp_path, 91)
    a = forward(cuvit, model, random_image(oracle, config, 10), 1, device)
    b = forward(cuvit, model, random_image(oracle, config, 11), 1, device)
    if np.array_equal(a, b):
        raise TestFailure("two different images produced identical logits")


def test_allocation_is_bounded_and_reused(cuvit, oracle, device, tmp_path):
    """vit_test.cu:174-197: depth costs weights, not activations."""
    config, _, _, model = build(cuvit, oracle, tmp_path, 5)
    deeper = small_config(cuvit)
    deeper.depth = config.depth * 4
    _, _, _, deep_model = build(cuvit, oracle, tmp_path, 6, config=deeper)
    assert model.weight_bytes() > 0 and model.activation_bytes() > 0
    assert deep_model.activation_bytes() == model.activation_bytes()
    assert deep_model.weight_bytes() > model.weight_bytes()


def test_batch_matches_one_at_a_time(cuvit, oracle, device, tmp_path):
    """vit_test.cu:199-238: bitwise."""
    config = small_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, 606)
    path = os.path.join(tmp_path, "batch.cvw")
    write_weights(cuvit, tensors, path)
    weights = cuvit.WeightFile(path)
    batch = 5
    single = cuvit.VisionTransformer(config, weights, 1)
    batched = cuvit.VisionTransformer(config, weights, batch)
    images = [random_image(oracle, config, 100 + i) for i in range(batch)]
    alone = [forward(cuvit, single, img, 1, device)[0] for img in images]
    together = forward(cuvit, batched, np.concatenate(images), batch, device)
    for i in range(batch):
        require_exact(together[i], alone[i], "an image in a batch differs from the same image run alone")


def test_partial_batch_is_clean(cuvit, oracle, device, tmp_path):
    """vit_test.cu:240-266."""
    config, _, _, model = build(cuvit, oracle, tmp_path, 707, max_batch=4)
    first, second = random_image(oracle, config, 21), random_image(oracle, config, 22)
    four = forward(cuvit, model, np.concatenate([first, second, first, second]), 4, device)
    two = forward(cuvit, model, np.concatenate([first, second]), 2, device)
    require_exact(two, four[:2], "a partial batch disagrees with a full one")


def test_batch_limits_are_enforced(cuvit, oracle, device, tmp_path):
    """vit_test.cu:268-302."""
    config, _, weights, model = build(cuvit, oracle, tmp_path, 808, max_batch=2)
    images = torch.zeros(3 * config.channels * config.image_size ** 2, device=device)
    logits = torch.zeros(3 * config.classes, device=device)
    with pytest.raises(cuvit.InvalidArgument):
        model.forward(images, logits, 3)
    with pytest.raises(cuvit.InvalidArgument):
        cuvit.VisionTransformer(config, weights, 0)
    model.forward(None, None, 0)  # an empty batch is a no-op


def test_activation_memory_scales_with_the_batch(cuvit, oracle, device, tmp_path):
    """vit_test.cu:304-322."""
    config = small_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, 909)
    path = os.path.join(tmp_path, "scale.cvw")
    write_weights(cuvit, tensors, path)
    weights = cuvit.WeightFile(path)
    one = cuvit.VisionTransformer(config, weights, 1)
    eight = cuvit.VisionTransformer(config, weights, 8)
    assert eight.weight_bytes() == one.weight_bytes()
    assert one.activation_bytes() < eight.activation_bytes() <= one.activation_bytes() * 8


def test_missing_and_misshaped_weights_are_rejected(cuvit, oracle, device, tmp_path):
    """vit_test.cu:347-367."""
    config, _, weights, _ = build(cuvit, oracle, tmp_path, 3)
    wrong = small_config(cuvit)
    wrong.embed_dim = 48
    with pytest.raises(cuvit.CuvitError):
        cuvit.VisionTransformer(wrong, weights, 1)


def test_vit_tiny_batch_32_sequence(cuvit, oracle, device, tmp_path):
    """The full ViT-Tiny/16 layer-kernel sequence at batch 32 (random N(0,0.02)
    weights, U(-1,1) images, seed 404): every image against the CPU
    VitReference (the oracle's forward runs on host threads, one image each),
    and images of the batch bitwise equal to the same image run alone."""
    config = tiny_config(cuvit)
    tensors = random_weights(cuvit, oracle, config, 404, small=False)
    path = os.path.join(tmp_path, "tiny.cvw")
    write_weights(cuvit, tensors, path)
    weights = cuvit.WeightFile(path)
    batch = 32
    model = cuvit.VisionTransformer(config, weights, batch)
    per_image = config.channels * config.image_size ** 2
    images = oracle.generator(404).uniform(batch * per_image, -1.0, 1.0)
    together = forward(cuvit, model, images, batch, device)
    assert np.isfinite(together).all()

    weights_list = [t for _, t in tensors]
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
        expected = list(pool.map(
            lambda i: oracle.vit_forward(config, weights_list, images[i * per_image:(i + 1) * per_image]),
            range(batch)))
    for i in range(batch):
        require_close(together[i], expected[i], f"ViT-Tiny logits of image {i} differ from the CPU reference",
                      1.0e-4, 1.0e-4)

    single = cuvit.VisionTransformer(config, weights, 1)
    for i in (0, 13, 31):
        alone = forward(cuvit, single, images[i * per_image:(i + 1) * per_image], 1, device)[0]
        require_exact(together[i], alone, f"image {i} of the batch differs from itself alone")
