"""Images on the CPU: PPM loading through the C ABI (host code), the oracle's
preprocessing pinned without a GPU, the device entry point's argument checks,
and the cu-vit program's command line.

Follows tests/image_test.cu:57-235. load_ppm is checked against the exact
pixels written and, where oracle/_ref is built, byte- and message-identical
against the reference's own src/runtime/image.cpp. The oracle's preprocess is
pinned bit-exact against the same reference code, and, independently of it, by
closed forms: identity geometry, exact 2x2 box averages at a 2x downscale, and
transposition.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

from image_support import GEOMETRIES, gradient, ppm_bytes, random_pixels, write_ppm


def load(cuvit, path):
    return cuvit.load_ppm(str(path))


# --------------------------------------------------------------------- load_ppm

def test_ppm_round_trip(cuvit, tmp_path):
    """image_test.cu:57-69: a comment between header fields is legal."""
    pixels = gradient(7, 5)
    path = tmp_path / "round_trip.ppm"
    write_ppm(path, 7, 5, pixels, comment=" written by the test suite")
    image = load(cuvit, path)
    assert (image.width, image.height) == (7, 5)
    assert np.array_equal(image.pixels, pixels)


@pytest.mark.parametrize("header", [
    b"P6 7 5 255 ",                      # spaces only
    b"P6\r\n7\t5\r\n255\n",              # CR LF and a tab
    b"P6\n# one\n# two\n7 5\n255\n",     # comments before the width
    b"P6\n7 # width\n5\n# maximum next\n255\n",
    b"P6\n0007 005 00255\n",             # leading zeros
    b"  \nP6\n7 5\n255\t",               # whitespace before the magic, tab separator
])
def test_ppm_header_forms(cuvit, reference_or_none, tmp_path, header):
    pixels = random_pixels(3, 5, 7)
    path = tmp_path / "forms.ppm"
    path.write_bytes(header + pixels.tobytes())
    image = load(cuvit, path)
    assert (image.width, image.height) == (7, 5)
    assert np.array_equal(image.pixels, pixels)
    if reference_or_none is not None:
        width, height, ref_pixels = reference_or_none.load_ppm(str(path))
        assert (width, height) == (7, 5) and np.array_equal(ref_pixels, pixels)


def test_payload_after_the_maximum_takes_one_byte(cuvit, tmp_path):
    """Exactly one byte follows the maximum, whatever it is: a second
    whitespace byte is already payload."""
    pixels = random_pixels(4, 2, 2)
    path = tmp_path / "one_byte.ppm"
    path.write_bytes(b"P6\n2 2\n255\n\n" + pixels.tobytes()[:-1])
    image = load(cuvit, path)
    assert image.pixels.reshape(-1)[0] == ord("\n")
    assert np.array_equal(image.pixels.reshape(-1)[1:], pixels.reshape(-1)[:-1])


def test_trailing_bytes_are_ignored(cuvit, tmp_path):
    pixels = random_pixels(5, 3, 4)
    path = tmp_path / "trailing.ppm"
    path.write_bytes(ppm_bytes(4, 3, pixels) + b"extra bytes after the payload")
    assert np.array_equal(load(cuvit, path).pixels, pixels)


MALFORMED = {
    "ascii": (b"P3\n2 2\n255\n0 0 0 0 0 0 0 0 0 0 0 0\n", "Only binary PPM (P6) images are supported: "),
    "empty": (b"", "Only binary PPM (P6) images are supported: "),
    "magic_glued": (b"P6#c\n2 2\n255\n" + bytes(12), "Only binary PPM (P6) images are supported: "),
    "letters": (b"P6\nab 2\n255\n" + bytes(12), "Malformed PPM header"),
    "negative": (b"P6\n-2 2\n255\n" + bytes(12), "Malformed PPM header"),
    "missing_height": (b"P6\n2", "Malformed PPM header"),
    "comment_to_end": (b"P6\n2 2 # no newline", "Malformed PPM header"),
    "width_overflow": (b"P6\n99999999999 2\n255\n" + bytes(12), "Malformed PPM header"),
    "zero_width": (b"P6\n0 2\n255\n", "PPM image has no extent: "),
    "sixteen_bit": (b"P6\n2 2\n65535\n" + bytes(24), "Only 8-bit PPM images are supported: "),
    "maximum_overflow": (b"P6\n2 2\n99999999999\n" + bytes(12), "Only 8-bit PPM images are supported: "),
    "truncated": (ppm_bytes(8, 8, np.zeros((8, 8, 3), np.uint8))[:-32],
                  "PPM image ends before its payload does: "),
    "no_separator": (b"P6\n1 1\n255", "PPM image ends before its payload does: "),
    "huge_extent": (b"P6\n100000 100000\n255\n" + bytes(30), "PPM image ends before its payload does: "),
}


@pytest.mark.parametrize("case", sorted(MALFORMED))
def test_malformed_images_are_rejected(cuvit, reference_or_none, tmp_path, case):
    """image_test.cu:71-120 (missing, ASCII, truncated) and the other ways a
    header can fail, with the reference's messages."""
    content, message = MALFORMED[case]
    path = tmp_path / f"{case}.ppm"
    path.write_bytes(content)
    with pytest.raises(cuvit.CuvitError) as error:
        load(cuvit, path)
    assert error.value.status == cuvit.ERROR_RUNTIME
    text = str(error.value)
    assert text.startswith(message), text
    if message.endswith(": "):
        assert text == message + str(path)
    # The reference sizes its pixel buffer from the header before reading, so
    # it is not asked to load a header that claims 30 GB.
    if reference_or_none is not None and case != "huge_extent":
        assert reference_or_none.load_ppm(str(path)) == text


def test_missing_image(cuvit, tmp_path):
    path = tmp_path / "absent.ppm"
    with pytest.raises(cuvit.CuvitError, match="^Cannot open image: "):
        load(cuvit, path)


def test_load_ppm_null_arguments(lib):
    handle = ctypes.c_void_p()
    assert lib.cuvit_image_load_ppm(None, ctypes.byref(handle)) == 1
    assert lib.cuvit_image_load_ppm(b"x.ppm", None) == 1
    assert lib.cuvit_image_width(None) == 0 and lib.cuvit_image_height(None) == 0
    assert lib.cuvit_image_pixels(None) is None
    lib.cuvit_image_destroy(None)


def test_random_files_match_the_reference(cuvit, reference, tmp_path):
    """Byte-identical to the reference's load_ppm on assorted sizes."""
    for seed, (height, width) in enumerate([(1, 1), (3, 500), (211, 97), (64, 64)]):
        pixels = random_pixels(seed, height, width)
        path = tmp_path / f"random_{seed}.ppm"
        write_ppm(path, width, height, pixels, comment=f" seed {seed}")
        image = load(cuvit, path)
        ref_width, ref_height, ref_pixels = reference.load_ppm(str(path))
        assert (image.width, image.height) == (ref_width, ref_height) == (width, height)
        assert np.array_equal(image.pixels, ref_pixels)


# ----------------------------------------------------------- oracle preprocess

def test_oracle_matches_the_reference_bitwise(oracle, reference):
    """The restatement against src/runtime/image.cpp compiled in place."""
    for index, (height, width, size, crop, mean, std) in enumerate(GEOMETRIES):
        pixels = random_pixels(100 + index, height, width)
        expected = reference.preprocess(pixels, size, crop, mean, std)
        actual = oracle.preprocess(pixels, size, crop, mean, std)
        assert np.array_equal(actual.view(np.uint32), expected.view(np.uint32)), (height, width)


def test_oracle_rejections_match_the_reference(oracle, reference):
    """The reference's four checks, in its order."""
    pixels = random_pixels(1, 4, 4)
    cases = [
        (np.zeros((0, 0, 3), np.uint8), 224, 0.9, (0.5,) * 3, 1),
        (pixels, 0, 0.9, (0.5,) * 3, 2),
        (pixels, -3, 0.0, (0.0,) * 3, 2),
        (pixels, 224, 0.0, (0.5,) * 3, 3),
        (pixels, 224, 1.5, (0.5,) * 3, 3),
        (pixels, 224, float("nan"), (0.5,) * 3, 3),
        (pixels, 224, 0.9, (1.0, 0.0, 1.0), 4),
    ]
    messages = {1: "Cannot preprocess an empty image", 2: "The preprocessing size must be positive",
                3: "The crop fraction must lie in (0, 1]",
                4: "A preprocessing standard deviation cannot be zero"}
    for image, size, crop, std, code in cases:
        assert oracle.preprocess(image, size, crop, (0.5,) * 3, std) == code
        assert reference.preprocess(image, size, crop, (0.5,) * 3, std) == messages[code]


def normalised(pixels, mean, std):
    """(p / 255 - mean) / std per channel in float32, one rounding per step."""
    out = np.empty((3,) + pixels.shape[:2], dtype=np.float32)
    for c in range(3):
        value = pixels[:, :, c].astype(np.float32) / np.float32(255.0)
        out[c] = (value - np.float32(mean[c])) / np.float32(std[c])
    return out


def test_oracle_identity_geometry(oracle):
    """A size x size image at crop fraction 1: origin 0, step 1, every sample
    lands on a pixel centre, so the tensor is the normalised image."""
    for size in (1, 7, 224):
        pixels = random_pixels(size, size, size)
        mean, std = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)
        actual = oracle.preprocess(pixels, size, 1.0, mean, std)
        assert np.array_equal(actual, normalised(pixels, mean, std))


def test_oracle_two_to_one_is_a_box_average(oracle):
    """A 2S x 2S image at crop fraction 1 to S: samples fall midway between
    four pixels with weights of one half, so each output is the exact mean of
    a 2x2 block (every intermediate is exact in float)."""
    size = 16
    pixels = random_pixels(9, 2 * size, 2 * size)
    blocks = pixels.astype(np.float32).reshape(size, 2, size, 2, 3).mean(axis=(1, 3))
    expected = np.empty((3, size, size), dtype=np.float32)
    for c in range(3):
        expected[c] = (blocks[:, :, c] / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)
    assert np.array_equal(oracle.preprocess(pixels, size, 1.0), expected)


def test_oracle_transposes_with_the_image(oracle):
    """x and y follow one formula: the tensor of the transposed image is the
    transposed tensor, for any aspect ratio. Interpolation runs along x first,
    so the transposed image rounds in the other order: equal to a few ulps."""
    for height, width in ((40, 90), (90, 40), (33, 33)):
        pixels = random_pixels(height + width, height, width)
        straight = oracle.preprocess(pixels, 24, 0.875)
        flipped = oracle.preprocess(np.ascontiguousarray(pixels.transpose(1, 0, 2)), 24, 0.875)
        assert np.max(np.abs(flipped - straight.transpose(0, 2, 1))) < 8.0e-6


def test_oracle_reference_image_test_cases(oracle):
    """image_test.cu:122-200: uniform grey, planar channels, centre crop."""
    grey = np.full((300, 300, 3), 128, np.uint8)
    expected = (np.float32(128.0) / np.float32(255.0) - np.float32(0.5)) / np.float32(0.5)
    assert np.all(np.abs(oracle.preprocess(grey) - expected) < 1.0e-5)

    planar = np.zeros((256, 256, 3), np.uint8)
    planar[:, :, 0], planar[:, :, 2] = 255, 128
    tensor = oracle.preprocess(planar)
    assert np.all(np.abs(tensor[0] - 1.0) < 1.0e-5)
    assert np.all(np.abs(tensor[1] + 1.0) < 1.0e-5)
    assert np.all(np.abs(tensor[2] - expected) < 1.0e-5)

    band = np.zeros((200, 600, 3), np.uint8)
    band[:, 250:350, :] = 255
    tensor = oracle.preprocess(band)
    assert tensor[0, 112, 112] > 0.9
    assert tensor[0, 0, 0] < -0.9 and tensor[0, -1, -1] < -0.9


def test_oracle_crop_geometry_constants():
    """The default geometry in closed form: the shorter side of 300 goes to
    round(224 / 0.9) = 249, so 224 outputs span 224 * 300 / 249 source pixels."""
    resized = np.float32(round(np.float32(224) / np.float32(0.9)))
    assert resized == 249
    scale = np.float32(300) / resized
    crop = np.float32(224) * scale
    assert math.isclose(float(crop), 224 * 300 / 249, rel_tol=1e-6)


# ----------------------------------------------- device entry point, arguments

def test_preprocessing_defaults(cuvit, lib):
    settings = cuvit.Preprocessing()
    lib.cuvit_preprocessing_default(ctypes.byref(settings))
    assert settings.size == 224 and abs(settings.crop_fraction - 0.9) < 1e-7
    assert list(settings.mean) == [0.5] * 3 and list(settings.stddev) == [0.5] * 3
    plain = cuvit.Preprocessing()
    assert plain.size == 224 and list(plain.stddev) == [0.5] * 3


def preprocess_status(cuvit, lib, pixels=1, batch=1, width=4, height=4, settings="default",
                      tensor=1):
    if settings == "default":
        settings = cuvit.Preprocessing()
    pointer = None if settings is None else ctypes.byref(settings)
    status = lib.cuvit_preprocess_u8(pixels, batch, width, height, pointer, tensor, None)
    return status, (lib.cuvit_last_error() or b"").decode()


def test_preprocess_argument_checks(cuvit, lib):
    """Checked before any device work, in the reference's order around the
    extension's batch and pointer checks; nothing here launches."""
    P = cuvit.Preprocessing
    assert preprocess_status(cuvit, lib, pixels=None, batch=0, tensor=None, settings=None)[0] == 0
    cases = [
        (dict(batch=-1), 1, "The preprocessing batch cannot be negative"),
        (dict(settings=None), 1, "Preprocessing settings cannot be null"),
        (dict(width=0), 1, "Cannot preprocess an empty image"),
        (dict(height=-5, settings=P(size=0)), 1, "Cannot preprocess an empty image"),
        (dict(settings=P(size=0)), 1, "The preprocessing size must be positive"),
        (dict(settings=P(size=-1, crop_fraction=0.0)), 1, "The preprocessing size must be positive"),
        (dict(settings=P(crop_fraction=0.0)), 1, "The crop fraction must lie in (0, 1]"),
        (dict(settings=P(crop_fraction=-0.5)), 1, "The crop fraction must lie in (0, 1]"),
        (dict(settings=P(crop_fraction=1.0000001)), 1, "The crop fraction must lie in (0, 1]"),
        (dict(settings=P(crop_fraction=float("nan"))), 1, "The crop fraction must lie in (0, 1]"),
        (dict(settings=P(stddev=(1.0, 1.0, 0.0))), 1,
         "A preprocessing standard deviation cannot be zero"),
        (dict(settings=P(stddev=(-0.0, 1.0, 1.0)), pixels=None), 1,
         "A preprocessing standard deviation cannot be zero"),
        (dict(pixels=None), 1, "Preprocessing operands cannot be null"),
        (dict(tensor=None), 1, "Preprocessing operands cannot be null"),
        (dict(settings=P(size=32769)), 2, "The preprocessing size exceeds the grid limit"),
        (dict(batch=2**30, width=2**31 - 1, height=2**31 - 1), 2,
         "The preprocessing images exceed the addressable size"),
    ]
    for kwargs, status, message in cases:
        assert preprocess_status(cuvit, lib, **kwargs) == (status, message), kwargs


def test_preprocess_raises_the_matching_exceptions(cuvit):
    with pytest.raises(cuvit.InvalidArgument, match="crop fraction"):
        cuvit.preprocess(1, 1, 1, 4, 4, cuvit.Preprocessing(crop_fraction=2.0))
    with pytest.raises(cuvit.LengthError):
        cuvit.preprocess(1, 1, 1, 4, 4, cuvit.Preprocessing(size=40000))
    with pytest.raises(cuvit.InvalidArgument, match="empty image"):
        cuvit.preprocess_image(cuvit.RgbImage(0, 0, np.zeros((0, 0, 3), np.uint8)))


# ------------------------------------------------------------- cu-vit program

def run_cli(cuvit, *arguments):
    path = cuvit.cli_path()
    if not os.path.exists(path):
        pytest.fail(f"cu-vit is not built: {path}")
    return subprocess.run([path, *arguments], capture_output=True, text=True, timeout=60)


def test_cli_help(cuvit):
    result = run_cli(cuvit, "--help")
    assert result.returncode == 0
    assert result.stdout.startswith("Usage: cu-vit --weights FILE.cvw (--image FILE.ppm | --raw FILE.bin)")
    for flag in ("--weights", "--image", "--raw", "--top", "--benchmark", "--batch", "--precision"):
        assert f"  {flag}" in result.stdout
    assert run_cli(cuvit, "-h").stdout == result.stdout


def test_cli_without_inputs_prints_the_usage(cuvit):
    for arguments in ((), ("--weights", "w.cvw"), ("--image", "x.ppm")):
        result = run_cli(cuvit, *arguments)
        assert result.returncode == 1
        assert result.stdout.startswith("Usage: cu-vit")


@pytest.mark.parametrize("arguments, message", [
    (("--bogus",), "Unknown argument: --bogus"),
    (("--weights",), "--weights needs a value"),
    (("--weights", "w", "--top"), "--top needs a value"),
    (("--top", "many"), "stoi"),
    (("--batch", "x"), "stoi"),
    (("--precision", "fp8"), "--precision takes f32 or bf16, not fp8"),
])
def test_cli_argument_errors(cuvit, arguments, message):
    """main.cpp:45-73 and 199-204: a bad command line is one line on stderr
    and exit status 1."""
    result = run_cli(cuvit, *arguments)
    assert result.returncode == 1
    assert result.stderr == f"cu-vit failed: {message}\n"


# ------------------------------------------- the device's division forms (host)
#
# The preprocessing kernel divides by 255 and by the standard deviation as
# multiply-and-correct sequences of fused multiply-adds instead of the
# division operator (preprocess.hip: divide_by_255, divide). Both must round
# exactly as IEEE division does. The float32 fused multiply-add is emulated
# exactly here: a * b is exact in float64, and a TwoSum of the float64 sum
# resolves the one case where rounding it to float32 could differ (a float64
# sum that lands exactly on a float32 midpoint).

F32, F64 = np.float32, np.float64


def _fma32(a, b, c):
    p = a.astype(F64) * b.astype(F64)
    c64 = np.asarray(c).astype(F64)
    s = p + c64
    bp = s - c64
    err = (p - bp) + (c64 - (s - bp))
    r = s.astype(F32)
    lo = np.where(r.astype(F64) <= s, r, np.nextafter(r, F32(-np.inf)))
    hi = np.nextafter(lo, F32(np.inf))
    at_mid = (s == (lo.astype(F64) + hi.astype(F64)) * 0.5) & (err != 0)
    return np.where(at_mid, np.where(err > 0, hi, lo), r)


def _divide_by_255(x):
    inverse = F32(1.0) / F32(255.0)
    q = (x.astype(F64) * F64(inverse)).astype(F32)
    return _fma32(_fma32(np.full_like(x, -255.0), q, x), np.full_like(x, inverse), q)


def _divide(a, b, inverse):
    q0 = (a.astype(F64) * inverse.astype(F64)).astype(F32)
    q1 = _fma32(_fma32(-b, q0, a), inverse, q0)
    return _fma32(_fma32(-b, q1, a), inverse, q1)


def test_fma_emulation_rounds_midpoints_by_the_exact_sum():
    """The emulation against exact rational arithmetic on sums built to land
    on or next to float32 midpoints in float64."""
    from fractions import Fraction

    rng = np.random.default_rng(11)
    a = rng.uniform(1.0, 2.0, 2000).astype(F32)
    b = rng.uniform(1.0, 2.0, 2000).astype(F32)
    c = (-(a.astype(F64) * b.astype(F64))).astype(F32)  # near cancellation
    c[::2] = rng.uniform(-4.0, 4.0, 1000).astype(F32)
    got = _fma32(a, b, c)
    for i in range(0, 2000, 7):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        down = F32(float(exact))
        candidates = [np.nextafter(down, F32(-np.inf)), down, np.nextafter(down, F32(np.inf))]
        best = min(candidates, key=lambda v: (abs(Fraction(float(v)) - exact),
                                              int(np.array([v]).view(np.uint32)[0]) & 1))
        assert got[i].view(np.uint32) == best.view(np.uint32), (a[i], b[i], c[i])


def test_divide_by_255_rounds_as_ieee_division():
    """Every integer and half-integer sample, the floats next to them, and
    one float in 61 over all of [0, 255] (the form was compared with IEEE
    division for all 1.13e9 floats of that range when it was written)."""
    top = int(np.array([255.0], F32).view(np.uint32)[0])
    bits = np.arange(0, top + 1, 61, dtype=np.uint32)
    grid = np.arange(0, 511, dtype=F64) * 0.5
    near = np.concatenate([grid.astype(F32), np.nextafter(grid.astype(F32), F32(0)),
                           np.nextafter(grid.astype(F32), F32(256))])
    x = np.concatenate([bits.view(F32), near[(near >= 0) & (near <= 255)]]).astype(F32)
    got = _divide_by_255(x)
    assert np.array_equal(got.view(np.uint32), (x / F32(255.0)).view(np.uint32))


@pytest.mark.parametrize("stddev", [0.5, 0.229, 0.224, 0.225, 1.0, 3.0e-6, 7.0e5])
def test_corrected_division_rounds_as_ieee_division(stddev):
    """(sample / 255 - mean) / stddev's second division: numerators of every
    binade the kernel can meet (2^-61 to 2^21, both signs), each with
    randomized significands."""
    rng = np.random.default_rng(int(stddev * 1e6) % 1000 + 5)
    exponents = rng.integers(-61, 21, 400_000)
    a = (rng.uniform(1.0, 2.0, exponents.size) * np.exp2(exponents)).astype(F32)
    a[::2] = -a[::2]
    b = np.full_like(a, stddev)
    inverse = np.full_like(a, F32(1.0) / F32(stddev))
    assert np.array_equal(_divide(a, b, inverse).view(np.uint32), (a / b).view(np.uint32))
