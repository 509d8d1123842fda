"""The .cvw weight format, on the CPU.

Mirrors tests/weights_test.cu (round trip, payload alignment, shape mismatch,
duplicate names, missing / wrong-magic / wrong-version / truncated files) and
adds interchange with the reference's own src/runtime/weights.cpp, compiled in
place into oracle/_ref: a file written by either side loads on the other, and
the two writers produce identical bytes. Version 2 (bf16 tensors, an
extension) round-trips, is written only for files holding a bf16 tensor, and
is refused by the reference's reader.
"""

from __future__ import annotations

import os
import struct
from pathlib import Path

import numpy as np
import pytest

from numerics import require_exact


def _tensors(oracle):
    g = oracle.generator(4242)
    return [("patch_embed.weight", g.normal(192 * 3 * 16 * 16).reshape(192, 3, 16, 16)),
            ("blocks.0.attn.proj.weight", g.normal(192 * 192).reshape(192, 192)),
            ("blocks.0.attn.proj.bias", g.normal(192))]


def _write(cuvit, tensors, path):
    writer = cuvit.WeightWriter()
    for name, values in tensors:
        writer.add(name, values)
    writer.write(path)
    writer.close()


def test_round_trip_preserves_shape_and_data(cuvit, oracle, tmp_path):
    """weights_test.cu:39-77."""
    path = str(tmp_path / "round_trip.cvw")
    tensors = _tensors(oracle)
    _write(cuvit, tensors, path)
    loaded = cuvit.WeightFile(path)
    assert len(loaded) == 3
    assert loaded.contains("patch_embed.weight") and not loaded.contains("absent")
    assert loaded.names() == [n for n, _ in tensors]
    assert loaded.payload_bytes() == sum(t.size * 4 for _, t in tensors)
    for name, values in tensors:
        require_exact(loaded.float_data(name, values.shape), values, f"{name} changed on disk")


def test_payloads_are_aligned(cuvit, oracle, tmp_path):
    """weights_test.cu:79-97: every payload offset is a multiple of 64."""
    path = str(tmp_path / "aligned.cvw")
    tensors = [("a", np.ones(3, np.float32)), ("bb", np.ones(17, np.float32)),
               ("ccc", np.ones((5, 7), np.float32))]
    _write(cuvit, tensors, path)
    blob = Path(path).read_bytes()
    magic, version, count, _ = struct.unpack_from("<4I", blob, 0)
    assert (magic, version, count) == (0x54495643, 1, 3)
    cursor = 16
    for name, values in tensors:
        (length,) = struct.unpack_from("<I", blob, cursor)
        cursor += 4
        assert blob[cursor:cursor + length].decode() == name
        cursor += length
        dtype, rank = struct.unpack_from("<2I", blob, cursor)
        cursor += 8
        extents = struct.unpack_from(f"<{rank}q", blob, cursor)
        cursor += 8 * rank
        offset, size = struct.unpack_from("<2Q", blob, cursor)
        cursor += 16
        assert dtype == 1 and tuple(extents) == values.shape
        assert offset % 64 == 0 and size == values.size * 4
        assert np.frombuffer(blob, np.float32, values.size, offset).tolist() == values.reshape(-1).tolist()


def test_shape_mismatch_is_rejected(cuvit, tmp_path):
    """weights_test.cu:99-126."""
    path = str(tmp_path / "mismatch.cvw")
    _write(cuvit, [("weight", np.full((3, 4), 0.5, np.float32))], path)
    loaded = cuvit.WeightFile(path)
    with pytest.raises(cuvit.CuvitError, match=r"\[3, 4\]"):
        loaded.float_data("weight", (4, 3))
    with pytest.raises(cuvit.CuvitError, match="missing"):
        loaded.float_data("missing", (1,))


def test_duplicate_names_are_rejected(cuvit):
    """weights_test.cu:128-140."""
    writer = cuvit.WeightWriter()
    writer.add("weight", np.ones(4, np.float32))
    with pytest.raises(cuvit.InvalidArgument):
        writer.add("weight", np.ones(4, np.float32))


def test_corrupt_files_are_rejected(cuvit, tmp_path):
    """weights_test.cu:142-219."""
    with pytest.raises(cuvit.CuvitError):
        cuvit.WeightFile(str(tmp_path / "does_not_exist.cvw"))

    junk = tmp_path / "junk.cvw"
    junk.write_bytes(b"this is not a weight file at all\0")
    with pytest.raises(cuvit.CuvitError):
        cuvit.WeightFile(str(junk))

    # the reference's test writes kVersion + 1, which here is the bf16
    # version 2; the first version this library does not know is 3
    versioned = str(tmp_path / "version.cvw")
    _write(cuvit, [("weight", np.ones(4, np.float32))], versioned)
    blob = bytearray(Path(versioned).read_bytes())
    struct.pack_into("<I", blob, 4, 3)
    Path(versioned).write_bytes(bytes(blob))
    with pytest.raises(cuvit.CuvitError, match="version"):
        cuvit.WeightFile(versioned)

    truncated = str(tmp_path / "truncated.cvw")
    _write(cuvit, [("weight", np.ones(64, np.float32))], truncated)
    blob = Path(truncated).read_bytes()
    Path(truncated).write_bytes(blob[:-128])
    with pytest.raises(cuvit.CuvitError):
        cuvit.WeightFile(truncated)

    # beyond the reference: a table that ends inside a name, and a byte count
    # that disagrees with the shape
    short = str(tmp_path / "short.cvw")
    Path(short).write_bytes(struct.pack("<4I", 0x54495643, 1, 1, 0) + struct.pack("<I", 50) + b"ab")
    with pytest.raises(cuvit.CuvitError, match="name"):
        cuvit.WeightFile(short)
    lying = str(tmp_path / "lying.cvw")
    _write(cuvit, [("w", np.ones(4, np.float32))], lying)
    blob = bytearray(Path(lying).read_bytes())
    # entry: name_len(4) + 'w'(1) + type(4) + rank(4) + extent(8) + offset(8) + bytes(8)
    struct.pack_into("<Q", blob, 16 + 4 + 1 + 4 + 4 + 8 + 8, 12)
    Path(lying).write_bytes(bytes(blob))
    with pytest.raises(cuvit.CuvitError, match="declares"):
        cuvit.WeightFile(lying)


def test_writer_rejects_bad_tensors(cuvit):
    writer = cuvit.WeightWriter()
    with pytest.raises(cuvit.InvalidArgument):
        writer.add("", np.ones(2, np.float32))
    with pytest.raises(cuvit.InvalidArgument):
        writer.add("rank5", np.ones((1, 1, 1, 1, 1), np.float32))


def test_files_interchange_with_the_reference(cuvit, oracle, reference, tmp_path):
    """Bytes written by the reference's WeightFileWriter equal ours, and each
    side loads the other's file."""
    tensors = _tensors(oracle) + [("scalar_like", np.array([3.5], np.float32))]
    ours = str(tmp_path / "ours.cvw")
    theirs = str(tmp_path / "theirs.cvw")
    _write(cuvit, tensors, ours)
    reference.write_weights(theirs, tensors)
    assert Path(ours).read_bytes() == Path(theirs).read_bytes(), "the two writers disagree"
    loaded = cuvit.WeightFile(theirs)
    for name, values in tensors:
        require_exact(loaded.float_data(name, values.shape), values, f"{name} via our loader")
        require_exact(reference.read_weight(ours, name, values.shape), values,
                      f"{name} via the reference loader")


def test_reference_and_ours_reject_the_same_corruptions(cuvit, reference, tmp_path):
    good = str(tmp_path / "good.cvw")
    _write(cuvit, [("weight", np.ones(64, np.float32))], good)
    blob = Path(good).read_bytes()
    cases = {
        "magic": b"XXXX" + blob[4:],
        "version": blob[:4] + struct.pack("<I", 7) + blob[8:],
        "truncated": blob[:-128],
        "rank": blob[:16 + 4 + 6 + 4] + struct.pack("<I", 9) + blob[16 + 4 + 6 + 8:],
        "type": blob[:16 + 4 + 6] + struct.pack("<I", 2) + blob[16 + 4 + 6 + 4:],
    }
    for label, content in cases.items():
        path = str(tmp_path / f"{label}.cvw")
        Path(path).write_bytes(content)
        assert reference.check_weights(path) is not None, f"the reference accepted {label}"
        with pytest.raises(cuvit.CuvitError):
            cuvit.WeightFile(path)


# -- version 2: bfloat16 tensors (an extension) ---------------------------------

def _bf16_tensors(oracle):
    g = oracle.generator(4343)
    weight = oracle.round_bf16(g.normal(64 * 48, 0.0, 0.2)).reshape(64, 48)
    bias = g.normal(64, 0.0, 0.1)
    return weight, bias


def test_bf16_round_trip_and_version(cuvit, oracle, tmp_path):
    from oracle import bf16_to_float

    weight, bias = _bf16_tensors(oracle)
    specials = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC1, 0x0001, 0x3F80], np.uint16)
    path = str(tmp_path / "mixed.cvw")
    writer = cuvit.WeightWriter()
    writer.add_bf16("fc.weight", weight)
    writer.add("fc.bias", bias)
    writer.add_bf16("specials", specials)
    writer.write(path)
    blob = Path(path).read_bytes()
    assert struct.unpack_from("<2I", blob, 0) == (0x54495643, 2)
    loaded = cuvit.WeightFile(path)
    assert loaded.version == 2
    assert (loaded.dtype("fc.weight"), loaded.dtype("fc.bias"), loaded.dtype("absent")) == (2, 1, 0)
    require_exact(loaded.bf16_data("fc.weight", (64, 48)), weight, "bf16 payload")
    require_exact(loaded.bf16_data("specials", (7,)), specials, "bf16 special values")
    require_exact(loaded.float_data("fc.bias", (64,)), bias, "float32 payload in a version 2 file")
    assert loaded.payload_bytes() == weight.size * 2 + bias.size * 4 + specials.size * 2
    with pytest.raises(cuvit.CuvitError, match="bfloat16, not float32"):
        loaded.float_data("fc.weight", (64, 48))
    with pytest.raises(cuvit.CuvitError, match="float32, not bfloat16"):
        loaded.bf16_data("fc.bias", (64,))
    with pytest.raises(cuvit.CuvitError, match="shape"):
        loaded.bf16_data("fc.weight", (48, 64))
    # payloads stay 64-byte aligned with 2-byte elements
    count = struct.unpack_from("<I", blob, 8)[0]
    cursor = 16
    for _ in range(count):
        (length,) = struct.unpack_from("<I", blob, cursor)
        cursor += 4 + length
        _, rank = struct.unpack_from("<2I", blob, cursor)
        cursor += 8 + 8 * rank
        offset, _ = struct.unpack_from("<2Q", blob, cursor)
        cursor += 16
        assert offset % 64 == 0
    assert np.isnan(bf16_to_float(specials[4:5]))[0]


def test_float32_only_files_stay_version_1(cuvit, oracle, tmp_path):
    path = str(tmp_path / "plain.cvw")
    _write(cuvit, _tensors(oracle), path)
    assert struct.unpack_from("<2I", Path(path).read_bytes(), 0) == (0x54495643, 1)
    assert cuvit.WeightFile(path).version == 1


def test_bf16_type_is_refused_in_a_version_1_file(cuvit, oracle, tmp_path):
    weight, _ = _bf16_tensors(oracle)
    path = str(tmp_path / "v2.cvw")
    writer = cuvit.WeightWriter()
    writer.add_bf16("w", weight)
    writer.write(path)
    blob = bytearray(Path(path).read_bytes())
    struct.pack_into("<I", blob, 4, 1)
    Path(path).write_bytes(bytes(blob))
    with pytest.raises(cuvit.CuvitError, match="unsupported data type 2"):
        cuvit.WeightFile(path)


def test_reference_refuses_version_2_and_reads_version_1(cuvit, oracle, reference, tmp_path):
    """A bf16 file is version 2, which the reference's reader refuses by its
    version check (weights.cpp:105-109) instead of misreading it."""
    weight, bias = _bf16_tensors(oracle)
    path = str(tmp_path / "v2.cvw")
    writer = cuvit.WeightWriter()
    writer.add_bf16("w", weight)
    writer.add("b", bias)
    writer.write(path)
    message = reference.check_weights(path)
    assert message is not None and "version" in message
