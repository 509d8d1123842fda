"""Shared helpers for the image tests: PPM files and seeded pixel data, as
tests/image_test.cu:14-55 builds them."""

from __future__ import annotations

import numpy as np

IMAGENET_MEAN = (0.485, 0.456, 0.406)
IMAGENET_STD = (0.229, 0.224, 0.225)


def ppm_bytes(width: int, height: int, pixels: np.ndarray, comment: str = None,
              maximum: int = 255, separator: bytes = b"\n") -> bytes:
    """A binary PPM: magic, optional comment line, extents, maximum, one
    separator byte, payload (image_test.cu:30-40)."""
    header = b"P6\n"
    if comment is not None:
        header += b"#" + comment.encode() + b"\n"
    header += f"{width} {height}\n{maximum}".encode() + separator
    return header + np.ascontiguousarray(pixels, dtype=np.uint8).tobytes()


def write_ppm(path, width: int, height: int, pixels: np.ndarray, **kwargs) -> None:
    with open(path, "wb") as handle:
        handle.write(ppm_bytes(width, height, pixels, **kwargs))


def gradient(width: int, height: int) -> np.ndarray:
    """image_test.cu:42-55: red ramps across, green down, blue 128."""
    pixels = np.empty((height, width, 3), dtype=np.uint8)
    columns = np.arange(width) * 255 // (width - 1)
    rows = np.arange(height) * 255 // (height - 1)
    pixels[:, :, 0] = columns[None, :]
    pixels[:, :, 1] = rows[:, None]
    pixels[:, :, 2] = 128
    return pixels


def random_pixels(seed: int, height: int, width: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, 256, (height, width, 3), dtype=np.uint8)


# (height, width, size, crop_fraction, mean, stddev): the default geometry, odd
# and tiny images, heavy up- and downscaling, crop fraction 1, other
# normalisations and sizes.
GEOMETRIES = [
    (300, 300, 224, 0.9, (0.5,) * 3, (0.5,) * 3),
    (17, 31, 224, 0.9, (0.5,) * 3, (0.5,) * 3),
    (480, 640, 224, 0.875, IMAGENET_MEAN, IMAGENET_STD),
    (640, 480, 224, 0.875, IMAGENET_MEAN, IMAGENET_STD),
    (224, 224, 224, 1.0, (0.5,) * 3, (0.5,) * 3),
    (5, 3, 7, 0.5, (0.5,) * 3, (0.5,) * 3),
    (1, 1, 4, 1.0, (0.0,) * 3, (1.0,) * 3),
    (1000, 20, 64, 0.9, (0.5,) * 3, (0.5,) * 3),
    (257, 255, 384, 1.0, (0.1, 0.2, 0.3), (0.9, -0.5, 2.0)),
    (2, 2, 224, 0.95, (0.5,) * 3, (0.25,) * 3),
    # the kernel's multiply-and-correct divisions off their guarded range
    # (division operator): a mean of 1e-30, a standard deviation of 1e-7
    (64, 48, 32, 0.9, (1e-30,) * 3, (0.3,) * 3),
    (48, 64, 32, 0.9, (0.4,) * 3, (1e-7, 0.5, 0.5)),
    # and on it with negative and unrounded standard deviations
    (33, 47, 24, 0.8, (-0.485, 0.456, 0.0), (-0.229, 3.7, 0.017)),
    # an even size that is not a multiple of four (the vector kernel)
    (37, 41, 30, 0.85, IMAGENET_MEAN, IMAGENET_STD),
]
