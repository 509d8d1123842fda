"""numpy interface to the CPU oracle. TEST INFRASTRUCTURE ONLY.

Imported by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
leg, always as the comparison (or the timed CPU baseline), never as the thing a
product path calls. Two libraries sit behind it:

* liboracle.so - the restatement of the reference's CPU path (oracle.cpp);
* _ref/libref.so - the reference's own tests/reference/*.hpp and
  src/runtime/weights.cpp compiled in place (only where /root/reference exists
  at build time; elsewhere the prebuilt file is used if present).
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libref.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float


class OracleGemmProblem(ctypes.Structure):
    _fields_ = [
        ("m", _I), ("n", _I), ("k", _I), ("layout", ctypes.c_int32), ("alpha", _F),
        ("lda", _I), ("ldb", _I), ("ldc", _I),
        ("count", _I), ("stride_a", _L), ("stride_b", _L), ("stride_c", _L),
        ("inner", _I), ("outer_stride_a", _L), ("outer_stride_b", _L), ("outer_stride_c", _L),
        ("accumulate", ctypes.c_uint8), ("gelu", ctypes.c_uint8),
    ]


class OracleVitConfig(ctypes.Structure):
    _fields_ = [
        ("image_size", _I), ("patch_size", _I), ("channels", _I), ("embed_dim", _I),
        ("depth", _I), ("heads", _I), ("mlp_hidden", _I), ("classes", _I),
        ("layer_norm_epsilon", _F),
    ]


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(x: Optional[np.ndarray]):
    return None if x is None else x.ctypes.data


class _Linear:
    """The functions both libraries export under their own prefix."""

    prefix = ""
    lib: ctypes.CDLL

    def _bind_linear(self):
        s = {
            "layer_norm": (None, [_P, _P, _P, _P, _I, _I, _F]),
            "softmax": (None, [_P, _P, _I, _I]),
            "gelu": (None, [_P, _P, _L]),
            "gemm": (None, [_P, _P, _P, _P, _I, _I, _I, _F]),
            "gemm_transposed": (None, [_P, _P, _P, _P, _I, _I, _I, _F]),
            "gemm_term_magnitudes": (None, [_P, _P, _P, _I, _I, _I, _I, _F]),
        }
        for name, (res, args) in s.items():
            fn = getattr(self.lib, self.prefix + name)
            fn.restype = res
            fn.argtypes = args

    def _fn(self, name):
        return getattr(self.lib, self.prefix + name)

    def layer_norm(self, x, gamma, beta, epsilon: float = 1.0e-6) -> np.ndarray:
        x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
        rows, columns = x.shape
        out = np.empty_like(x)
        self._fn("layer_norm")(_p(x), _p(gamma), _p(beta), _p(out), rows, columns, epsilon)
        return out

    def softmax(self, x) -> np.ndarray:
        x = _f32(x)
        rows, columns = x.shape
        out = np.empty_like(x)
        self._fn("softmax")(_p(x), _p(out), rows, columns)
        return out

    def gelu(self, x) -> np.ndarray:
        x = _f32(x)
        out = np.empty_like(x)
        self._fn("gelu")(_p(x), _p(out), x.size)
        return out

    def gemm(self, a, b, bias, m, n, k, alpha: float = 1.0) -> np.ndarray:
        a, b = _f32(a), _f32(b)
        bias = None if bias is None else _f32(bias)
        out = np.empty((m, n), dtype=np.float32)
        self._fn("gemm")(_p(a), _p(b), _p(bias), _p(out), m, n, k, alpha)
        return out

    def gemm_transposed(self, a, b, bias, m, n, k, alpha: float = 1.0) -> np.ndarray:
        a, b = _f32(a), _f32(b)
        bias = None if bias is None else _f32(bias)
        out = np.empty((m, n), dtype=np.float32)
        self._fn("gemm_transposed")(_p(a), _p(b), _p(bias), _p(out), m, n, k, alpha)
        return out

    def term_magnitudes(self, a, b, m, n, k, transposed: bool, alpha: float = 1.0) -> np.ndarray:
        a, b = _f32(a), _f32(b)
        out = np.empty((m, n), dtype=np.float32)
        self._fn("gemm_term_magnitudes")(_p(a), _p(b), _p(out), m, n, k, int(transposed), alpha)
        return out


class Oracle(_Linear):
    """The restatement (liboracle.so)."""

    prefix = "oracle_"

    def __init__(self, path: str = ORACLE_LIB):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library not built: {path} (make -C oracle)")
        self.lib = ctypes.CDLL(path)
        self._bind_linear()
        s = {
            "oracle_gelu_scalar": (_F, [_F]),
            "oracle_gemm_problem_run": (None, [_P, _P, _P, _P, ctypes.POINTER(OracleGemmProblem)]),
            "oracle_extract_patches": (None, [_P, _P, _I, _I, _I, _I, _I]),
            "oracle_add": (None, [_P, _P, _L]),
            "oracle_add_broadcast": (None, [_P, _P, _L, _I]),
            "oracle_broadcast": (None, [_P, _P, _L, _L, _I]),
            "oracle_vit_forward": (None, [ctypes.POINTER(OracleVitConfig), ctypes.POINTER(_P), _P, _P]),
            "oracle_vit_forward_bf16": (None, [ctypes.POINTER(OracleVitConfig), ctypes.POINTER(_P), _P, _P]),
            "oracle_round_bf16": (None, [_P, _P, _L]),
            "oracle_generator_create": (_P, [ctypes.c_uint64]),
            "oracle_generator_uniform": (None, [_P, _P, _L, _F, _F]),
            "oracle_generator_normal": (None, [_P, _P, _L, _F, _F]),
            "oracle_generator_integers": (None, [_P, _P, _L, _L, _L]),
            "oracle_generator_raw": (ctypes.c_uint64, [_P]),
            "oracle_generator_destroy": (None, [_P]),
            "oracle_preprocess": (_I, [_P, _I, _I, _I, _F, _P, _P, _P]),
        }
        for name, (res, args) in s.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    def gelu_scalar(self, value: float) -> float:
        return self.lib.oracle_gelu_scalar(value)

    def gemm_problem_run(self, a, b, bias, c, **fields) -> np.ndarray:
        """Runs a full GemmProblem; @p c is updated in place and returned."""
        problem = OracleGemmProblem()
        problem.alpha = 1.0
        problem.count = 1
        for key, value in fields.items():
            setattr(problem, key, value)
        a, b = _f32(a), _f32(b)
        bias = None if bias is None else _f32(bias)
        assert c.dtype == np.float32 and c.flags.c_contiguous
        self.lib.oracle_gemm_problem_run(_p(a), _p(b), _p(bias), _p(c), ctypes.byref(problem))
        return c

    def preprocess(self, pixels, size: int = 224, crop_fraction: float = 0.9,
                   mean=(0.5, 0.5, 0.5), stddev=(0.5, 0.5, 0.5)):
        """[3, size, size] float32 of one [height, width, 3] uint8 image, or
        the failed check's code (1 empty image, 2 size, 3 crop, 4 stddev)."""
        return _preprocess(self.lib.oracle_preprocess, pixels, size, crop_fraction, mean, stddev)

    def extract_patches(self, images, batch, channels, height, width, patch) -> np.ndarray:
        images = _f32(images)
        rows = batch * (height // patch) * (width // patch)
        out = np.empty((rows, channels * patch * patch), dtype=np.float32)
        self.lib.oracle_extract_patches(_p(images), _p(out), batch, channels, height, width, patch)
        return out

    def add(self, accumulator: np.ndarray, addend) -> np.ndarray:
        addend = _f32(addend)
        self.lib.oracle_add(_p(accumulator), _p(addend), accumulator.size)
        return accumulator

    def add_broadcast(self, accumulator: np.ndarray, addend, count: int, batch: int) -> np.ndarray:
        addend = _f32(addend)
        self.lib.oracle_add_broadcast(_p(accumulator), _p(addend), count, batch)
        return accumulator

    def broadcast(self, destination: np.ndarray, source, count: int, stride: int,
                  batch: int) -> np.ndarray:
        source = _f32(source)
        self.lib.oracle_broadcast(_p(destination), _p(source), count, stride, batch)
        return destination

    def vit_forward(self, config, tensors: Sequence[np.ndarray], image,
                    bf16: bool = False) -> np.ndarray:
        """One image's logits; bf16 selects the bf16 model's rounding points."""
        cfg = OracleVitConfig(config.image_size, config.patch_size, config.channels,
                              config.embed_dim, config.depth, config.heads, config.mlp_hidden,
                              config.classes, config.layer_norm_epsilon)
        arrays = [_f32(t) for t in tensors]
        pointers = (_P * len(arrays))(*[a.ctypes.data for a in arrays])
        image = _f32(image)
        logits = np.empty(config.classes, dtype=np.float32)
        fn = self.lib.oracle_vit_forward_bf16 if bf16 else self.lib.oracle_vit_forward
        fn(ctypes.byref(cfg), pointers, _p(image), _p(logits))
        return logits

    def round_bf16(self, x) -> np.ndarray:
        """float32 -> bfloat16 bits (uint16), round to nearest even."""
        x = _f32(x)
        out = np.empty(x.shape, dtype=np.uint16)
        self.lib.oracle_round_bf16(_p(x), _p(out), x.size)
        return out

    def generator(self, seed: int) -> "Generator":
        return Generator(self, seed)


class Generator:
    """The reference tests' DataGenerator (tests/test_utils.hpp:233-263)."""

    def __init__(self, oracle: Oracle, seed: int):
        self._lib = oracle.lib
        self._g = oracle.lib.oracle_generator_create(seed)

    def uniform(self, count: int, low: float = -1.0, high: float = 1.0) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self._lib.oracle_generator_uniform(self._g, _p(out), count, low, high)
        return out

    def normal(self, count: int, mean: float = 0.0, stddev: float = 1.0) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self._lib.oracle_generator_normal(self._g, _p(out), count, mean, stddev)
        return out

    def integers(self, count: int, low: int, high: int) -> np.ndarray:
        out = np.empty(count, dtype=np.int64)
        self._lib.oracle_generator_integers(self._g, _p(out), count, low, high)
        return out

    def raw(self) -> int:
        return self._lib.oracle_generator_raw(self._g)

    def __del__(self):
        if getattr(self, "_g", None):
            self._lib.oracle_generator_destroy(self._g)
            self._g = None


class Reference(_Linear):
    """The reference's own CPU code, compiled in place (oracle/_ref/libref.so)."""

    prefix = "ref_"

    def __init__(self, path: str = REF_LIB):
        if not os.path.exists(path):
            raise RuntimeError(f"reference CPU library not built: {path}")
        self.lib = ctypes.CDLL(path)
        self._bind_linear()
        s = {
            "ref_vector_add": (None, [_P, _P, _P, _L]),
            "ref_last_error": (ctypes.c_char_p, []),
            "ref_weights_write": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_char_p),
                                       ctypes.POINTER(_I), ctypes.POINTER(_L), ctypes.POINTER(_P)]),
            "ref_weights_read": (_I, [ctypes.c_char_p, ctypes.c_char_p, _I, ctypes.POINTER(_L), _P, _L]),
            "ref_weights_check": (_I, [ctypes.c_char_p]),
            "ref_preprocess": (_I, [_P, _I, _I, _I, _F, _P, _P, _P]),
            "ref_load_ppm": (_I, [ctypes.c_char_p, ctypes.POINTER(_I), ctypes.POINTER(_I), _P, _L]),
        }
        for name, (res, args) in s.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    def vector_add(self, left, right) -> np.ndarray:
        left, right = _f32(left), _f32(right)
        out = np.empty_like(left)
        self.lib.ref_vector_add(_p(left), _p(right), _p(out), left.size)
        return out

    def last_error(self) -> str:
        return (self.lib.ref_last_error() or b"").decode()

    def write_weights(self, path: str, tensors) -> None:
        """tensors: list of (name, array) written with the reference's writer."""
        names = (ctypes.c_char_p * len(tensors))(*[n.encode() for n, _ in tensors])
        arrays = [_f32(a) for _, a in tensors]
        ranks = (_I * len(tensors))(*[a.ndim for a in arrays])
        flat = [d for a in arrays for d in a.shape]
        extents = (_L * max(len(flat), 1))(*flat)
        data = (_P * len(tensors))(*[a.ctypes.data for a in arrays])
        if self.lib.ref_weights_write(os.fsencode(path), len(tensors), names, ranks, extents, data):
            raise RuntimeError(self.last_error())

    def read_weight(self, path: str, name: str, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        extents = (_L * max(len(shape), 1))(*shape)
        if self.lib.ref_weights_read(os.fsencode(path), name.encode(), len(shape), extents,
                                     _p(out), out.size):
            raise RuntimeError(self.last_error())
        return out

    def preprocess(self, pixels, size: int = 224, crop_fraction: float = 0.9,
                   mean=(0.5, 0.5, 0.5), stddev=(0.5, 0.5, 0.5)):
        """The reference's preprocess: [3, size, size] float32, or its error
        message (a str) when it throws."""
        out = _preprocess(self.lib.ref_preprocess, pixels, size, crop_fraction, mean, stddev)
        return self.last_error() if isinstance(out, int) else out

    def load_ppm(self, path: str):
        """(width, height, [height, width, 3] uint8) from the reference's
        load_ppm, or its error message (a str)."""
        width, height = _I(), _I()
        if self.lib.ref_load_ppm(os.fsencode(path), ctypes.byref(width), ctypes.byref(height),
                                 None, 0):
            return self.last_error()
        pixels = np.empty((height.value, width.value, 3), dtype=np.uint8)
        self.lib.ref_load_ppm(os.fsencode(path), ctypes.byref(width), ctypes.byref(height),
                              _p(pixels), pixels.size)
        return width.value, height.value, pixels

    def check_weights(self, path: str) -> Optional[str]:
        """None when the reference loads @p path, else its error message."""
        if self.lib.ref_weights_check(os.fsencode(path)):
            return self.last_error()
        return None


def _preprocess(fn, pixels, size, crop_fraction, mean, stddev):
    pixels = np.ascontiguousarray(pixels, dtype=np.uint8)
    height, width = (pixels.shape[0], pixels.shape[1]) if pixels.ndim == 3 else (0, 0)
    out = np.zeros((3, max(size, 0), max(size, 0)), dtype=np.float32)
    m = (_F * 3)(*mean)
    s = (_F * 3)(*stddev)
    status = fn(_p(pixels) if pixels.size else None, width, height, size, crop_fraction,
                ctypes.cast(m, _P), ctypes.cast(s, _P), _p(out))
    return status if status else out


def reference_available() -> bool:
    return os.path.exists(REF_LIB)


def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bits (uint16) -> float32, exact."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
