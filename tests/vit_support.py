"""Shared helpers for the model tests: configurations and seeded random weights
written through the library's WeightFileWriter, as tests/vit_test.cu:36-106 does."""

from __future__ import annotations

import numpy as np


def small_config(cuvit):
    """vit_test.cu:36-47: 32x32 images, 8x8 patches, E=24, depth 3, 4 heads."""
    config = cuvit.default_config()
    config.image_size = 32
    config.patch_size = 8
    config.channels = 3
    config.embed_dim = 24
    config.depth = 3
    config.heads = 4
    config.mlp_hidden = 48
    config.classes = 7
    return config


def tiny_config(cuvit):
    """ViT-Tiny/16 at 224x224: VitConfig's defaults (vit.hpp:15-24)."""
    return cuvit.default_config()


def _spread(name: str, small: bool):
    """(mean, stddev) per tensor. Small config: vit_test.cu:68-96. Full size:
    N(0, 0.02) everywhere except LN gamma N(1, 0.02) and beta N(0, 0.02)."""
    is_gamma = name.endswith("norm1.weight") or name.endswith("norm2.weight") or name == "norm.weight"
    if not small:
        return (1.0, 0.02) if is_gamma else (0.0, 0.02)
    if is_gamma:
        return 1.0, 0.1
    if name.endswith("norm1.bias") or name.endswith("norm2.bias") or name == "norm.bias":
        return 0.0, 0.1
    if name in ("cls_token", "pos_embed"):
        return 0.0, 0.5
    if name.startswith("patch_embed"):
        return 0.0, 0.1
    if name.endswith(".weight"):
        return 0.0, 0.2
    return 0.0, 0.1


def random_weights(cuvit, oracle, config, seed: int, small: bool = True):
    """[(name, array)] in expected-name order, drawn from one DataGenerator."""
    generator = oracle.generator(seed)
    tensors = []
    for name, shape in cuvit.expected_tensor_names(config):
        mean, stddev = _spread(name, small)
        values = generator.normal(int(np.prod(shape)), mean, stddev).reshape(shape)
        tensors.append((name, values))
    return tensors


def write_weights(cuvit, tensors, path: str) -> None:
    writer = cuvit.WeightWriter()
    for name, values in tensors:
        writer.add(name, values)
    writer.write(path)
    writer.close()


def random_image(oracle, config, seed: int) -> np.ndarray:
    """vit_test.cu:101-106: N(0, 1) planar image."""
    count = config.channels * config.image_size * config.image_size
    return oracle.generator(seed).normal(count)
