"""ctypes wrapper for the float64 CPU oracle (oracle/dinov3_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product path in
dinov3-loom_amd/ never imports it.

The C file restates the reference's float64 oracle
(tests/support/reference.rs:1-192) plus patchify (lib.rs:265-280), float16
packing (weights.rs:6-17) and the RoPE tables (weights.rs:127-144).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "liboracle.so")
SOURCE = os.path.join(HERE, "dinov3_oracle.c")

HIDDEN = 384
PREFIX = 5
LAYERS = 12

LAYER_SUFFIXES = [
    "norm1.weight", "norm1.bias",
    "attention.q_proj.weight", "attention.q_proj.bias",
    "attention.k_proj.weight",
    "attention.v_proj.weight", "attention.v_proj.bias",
    "attention.o_proj.weight", "attention.o_proj.bias",
    "layer_scale1.lambda1",
    "norm2.weight", "norm2.bias",
    "mlp.gate_proj.weight", "mlp.gate_proj.bias",
    "mlp.up_proj.weight", "mlp.up_proj.bias",
    "mlp.down_proj.weight", "mlp.down_proj.bias",
    "layer_scale2.lambda1",
]


def tensor_names() -> list[str]:
    """Canonical tensor order of oracle_forward (the enum in the C file)."""
    names = [
        "embeddings.patch_embeddings.weight",
        "embeddings.patch_embeddings.bias",
        "embeddings.cls_token",
        "embeddings.register_tokens",
    ]
    for i in range(LAYERS):
        names += [f"layer.{i}.{s}" for s in LAYER_SUFFIXES]
    names += ["norm.weight", "norm.bias"]
    return names


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (OpenMP; AVX2/FMA for the f64 loops)."""
    if force or not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(SOURCE):
        os.makedirs(LIB_DIR, exist_ok=True)
        tmp = LIB_PATH + ".tmp"
        subprocess.check_call([
            "gcc", "-O3", "-mavx2", "-mfma", "-fopenmp", "-fPIC", "-shared",
            "-std=c11", "-D_GNU_SOURCE", SOURCE, "-o", tmp, "-lm",
        ])
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        fp = ctypes.POINTER(ctypes.c_float)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        L.oracle_patchify.argtypes = [fp, ctypes.c_int, ctypes.c_int, fp]
        L.oracle_f32_to_f16.argtypes = [fp, u16p, ctypes.c_size_t]
        L.oracle_f16_to_f32.argtypes = [u16p, fp, ctypes.c_size_t]
        L.oracle_rope_tables.argtypes = [ctypes.c_int, fp, fp]
        L.oracle_linear.argtypes = [dp, dp, dp, ctypes.c_int, ctypes.c_int, ctypes.c_int, dp]
        L.oracle_layernorm.argtypes = [dp, dp, dp, ctypes.c_int, dp]
        L.oracle_rope.argtypes = [dp, ctypes.c_int, ctypes.c_int]
        L.oracle_attention.argtypes = [dp, dp, dp, ctypes.c_int, dp]
        L.oracle_swiglu.argtypes = [dp, dp, ctypes.c_size_t, dp]
        L.oracle_forward.argtypes = [ctypes.POINTER(dp), fp, ctypes.c_int, dp]
        L.oracle_block.argtypes = [dp, ctypes.POINTER(dp), ctypes.c_int, ctypes.c_int]
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_max_threads.restype = ctypes.c_int
        L.oracle_tensor_count.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return lib().oracle_max_threads()


def patchify(images: np.ndarray, grid: int) -> np.ndarray:
    images = np.ascontiguousarray(images, dtype=np.float32)
    side = 16 * grid
    n = images.size // (3 * side * side)
    out = np.empty((n * grid * grid, 768), np.float32)
    lib().oracle_patchify(_p(images, ctypes.c_float), n, grid, _p(out, ctypes.c_float))
    return out


def f32_to_f16_bits(values: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.shape, np.uint16)
    lib().oracle_f32_to_f16(_p(v, ctypes.c_float), _p(out, ctypes.c_uint16), v.size)
    return out


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_to_f32(_p(b, ctypes.c_uint16), _p(out, ctypes.c_float), b.size)
    return out


def round_f16(values: np.ndarray) -> np.ndarray:
    """Values rounded through float16 (RNE), returned as float64."""
    return f16_bits_to_f32(f32_to_f16_bits(np.asarray(values, np.float32))).astype(np.float64)


def rope_tables(grid: int) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty((grid * grid, 64), np.float32)
    s = np.empty((grid * grid, 64), np.float32)
    lib().oracle_rope_tables(grid, _p(c, ctypes.c_float), _p(s, ctypes.c_float))
    return c, s


def linear(x, w, bias=None) -> np.ndarray:
    x, w = _f64(x), _f64(w)
    n, k = w.shape
    m = x.size // k
    out = np.empty((m, n), np.float64)
    b = _f64(bias) if bias is not None else None
    lib().oracle_linear(_p(x, ctypes.c_double), _p(w, ctypes.c_double),
                        _p(b, ctypes.c_double) if b is not None else None, m, k, n,
                        _p(out, ctypes.c_double))
    return out


def layernorm(x, g, b) -> np.ndarray:
    x = _f64(x)
    rows = x.size // HIDDEN
    out = np.empty((rows, HIDDEN), np.float64)
    g, b = _f64(g), _f64(b)
    lib().oracle_layernorm(_p(x, ctypes.c_double), _p(g, ctypes.c_double), _p(b, ctypes.c_double),
                           rows, _p(out, ctypes.c_double))
    return out


def rope(values, grid: int) -> np.ndarray:
    """RoPE on the patch tokens of one image's [T, 384] q or k (a copy)."""
    v = _f64(values).copy()
    T = v.size // HIDDEN
    lib().oracle_rope(_p(v, ctypes.c_double), T, grid)
    return v.reshape(T, HIDDEN)


def attention(q, k, v) -> np.ndarray:
    q, k, v = _f64(q), _f64(k), _f64(v)
    T = q.size // HIDDEN
    out = np.empty((T, HIDDEN), np.float64)
    lib().oracle_attention(_p(q, ctypes.c_double), _p(k, ctypes.c_double), _p(v, ctypes.c_double),
                           T, _p(out, ctypes.c_double))
    return out


def swiglu(gate, up) -> np.ndarray:
    g, u = _f64(gate), _f64(up)
    out = np.empty(g.shape, np.float64)
    lib().oracle_swiglu(_p(g, ctypes.c_double), _p(u, ctypes.c_double), g.size, _p(out, ctypes.c_double))
    return out


class Weights:
    """The model tensors as float64 arrays in the oracle's canonical order."""

    def __init__(self, tensors: dict[str, np.ndarray]):
        self.names = tensor_names()
        missing = [n for n in self.names if n not in tensors]
        if missing:
            raise KeyError(f"missing tensors: {missing[:3]}")
        self.arrays = [_f64(tensors[n]) for n in self.names]
        self.by_name = dict(zip(self.names, self.arrays))
        dp = ctypes.POINTER(ctypes.c_double)
        self.pointers = (dp * len(self.arrays))(*[_p(a, ctypes.c_double) for a in self.arrays])

    @classmethod
    def from_file(cls, path: str) -> "Weights":
        from safetensors.numpy import load_file
        return cls(load_file(path))

    def layer(self, i: int) -> dict[str, np.ndarray]:
        return {s: self.by_name[f"layer.{i}.{s}"] for s in LAYER_SUFFIXES}

    def layer_pointers(self, i: int):
        base = 4 + i * len(LAYER_SUFFIXES)
        dp = ctypes.POINTER(ctypes.c_double)
        return ctypes.cast(ctypes.byref(self.pointers, base * ctypes.sizeof(dp)), ctypes.POINTER(dp))


def forward(weights: Weights, image: np.ndarray, grid: int = 14) -> np.ndarray:
    """Float64 forward of one float32 NCHW image; returns [T, 384] float64."""
    img = np.ascontiguousarray(image, dtype=np.float32)
    assert img.size == 3 * (16 * grid) ** 2
    T = grid * grid + PREFIX
    out = np.empty((T, HIDDEN), np.float64)
    lib().oracle_forward(weights.pointers, _p(img, ctypes.c_float), grid, _p(out, ctypes.c_double))
    return out


def block(weights: Weights, layer: int, x: np.ndarray, grid: int) -> np.ndarray:
    """One transformer block (reference.rs:89-190) applied to a copy of x."""
    y = _f64(x).copy()
    T = y.size // HIDDEN
    lib().oracle_block(_p(y, ctypes.c_double), weights.layer_pointers(layer), T, grid)
    return y.reshape(T, HIDDEN)
