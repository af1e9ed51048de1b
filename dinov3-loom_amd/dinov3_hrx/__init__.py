"""Python binding of libdinov3_hrx.so (the MI355X / gfx950 DINOv3 ViT-S+/16
forward pass), mirroring the public API of the crate `dinov3-hrx`
(src/lib.rs:11-148, 302; src/hub.rs:7-28; src/engine.rs:272-284).

    from dinov3_hrx import DINOv3, Options
    model = DINOv3.load("model.safetensors", Options(max_batch=64))
    tokens = model.forward(pixels)          # float32 [batch, 201, 384]

Every call goes through the C ABI of include/dinov3.h; there is no Python or
CPU compute path. Importing fails loudly when the library is not built.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libdinov3_hrx.so")

# lib.rs:11-13
IMAGE_ELEMENTS = 3 * 224 * 224
TOKENS = 201
HIDDEN = 384

# hub.rs:7-11
REPO = ("facebook", "dinov3-vits16plus-pretrain-lvd1689m")
REVISION = "c93d816fc9e567563bc068f01475bec89cc634a6"
FILE = "model.safetensors"

# Kernel ids of include/dinov3_engine.h.
KERNELS = ["patch_embed", "layernorm", "layernorm_f32", "qkv_rope", "attention", "resid", "swiglu", "splitk",
           "splitk_reduce", "patch_embed_stats", "qkv_rope_ln", "resid_stats", "swiglu_ln", "splitk_reduce_stats"]


class DINOv3Error(RuntimeError):
    """An error reported by the library (the reference's anyhow errors)."""


class _Options(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int32), ("max_batch", ctypes.c_uint64), ("image_size", ctypes.c_uint32)]


class _Distribution(ctypes.Structure):
    _fields_ = [("median_ms", ctypes.c_double), ("p95_ms", ctypes.c_double)]


class _Timings(ctypes.Structure):
    _fields_ = [("samples", ctypes.c_uint64), ("graph", _Distribution), ("direct", _Distribution)]


class Region(ctypes.Structure):
    """include/dinov3_engine.h dhx_region (engine.rs:6-20 Region)."""
    _fields_ = [("buffer", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


MAX_SCALARS = 4  # DHX_MAX_SCALARS
MAX_BINDINGS = 12  # DHX_MAX_BINDINGS
MAX_BRANCHES = 4  # DHX_MAX_BRANCHES


class Launch(ctypes.Structure):
    """include/dinov3_engine.h dhx_launch (engine.rs:21-27 Launch)."""
    _fields_ = [("kernel", ctypes.c_uint32), ("scalars", ctypes.c_uint32 * MAX_SCALARS),
                ("n_bindings", ctypes.c_uint32), ("bindings", Region * MAX_BINDINGS)]


def _load_library() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python __graft_entry__.py` or "
                          "`python dinov3-loom_amd/build.py` first")
    L = ctypes.CDLL(LIB_PATH)
    vp, c = ctypes.c_void_p, ctypes
    fp = c.POINTER(c.c_float)
    L.dinov3_last_error.argtypes = [vp]
    L.dinov3_last_error.restype = c.c_char_p
    L.dinov3_options_default.argtypes = [c.POINTER(_Options)]
    L.dinov3_load.argtypes = [c.c_char_p, c.POINTER(_Options), c.POINTER(vp)]
    L.dinov3_from_pretrained.argtypes = [c.POINTER(_Options), c.POINTER(vp)]
    L.dinov3_hub_weights.argtypes = [c.c_char_p, c.c_uint64]
    for name in ("dinov3_forward", "dinov3_cls", "dinov3_patch_mean"):
        getattr(L, name).argtypes = [vp, fp, c.c_uint64, fp, c.c_uint64]
    L.dinov3_benchmark.argtypes = [vp, fp, c.c_uint64, c.c_uint64, c.POINTER(_Timings)]
    L.dinov3_forward_noalloc.argtypes = [vp, vp, c.c_uint64, vp, vp]
    L.dinov3_free.argtypes = [vp]
    L.dinov3_image_elements.argtypes = [vp]
    L.dinov3_image_elements.restype = c.c_uint64
    L.dinov3_tokens.argtypes = [vp]
    L.dinov3_tokens.restype = c.c_uint64
    L.dinov3_engine.argtypes = [vp]
    L.dinov3_engine.restype = vp
    L.dinov3_stage.argtypes = [vp, fp, c.c_uint64]
    L.dinov3_replay.argtypes = [vp, c.c_uint64]
    L.dinov3_set_splitk.argtypes = [vp, c.c_int]
    L.dinov3_set_layernorm_fusion.argtypes = [vp, c.c_int]
    L.dinov3_set_branches.argtypes = [vp, c.c_uint32]
    L.dinov3_launch_timings.argtypes = [vp, c.c_uint64, c.c_uint32, c.POINTER(c.c_double), c.POINTER(c.c_uint32),
                                        c.c_uint64, c.POINTER(c.c_uint64)]
    L.dinov3_write_random_weights.argtypes = [c.c_char_p, c.c_uint64, c.c_int]
    L.dinov3_random_pixels.argtypes = [c.c_uint64, c.c_uint64, c.c_uint32, fp]
    L.dinov3_patchify.argtypes = [fp, c.c_uint64, c.c_uint32, fp]
    L.dinov3_pack_f16.argtypes = [c.c_char_p, fp, c.c_uint64, c.POINTER(c.c_uint16)]
    L.dhx_last_error.argtypes = [vp]
    L.dhx_last_error.restype = c.c_char_p
    L.dhx_synchronize.argtypes = [vp]
    L.dhx_launch_timings.argtypes = [vp, c.c_uint64, c.c_uint32, c.POINTER(c.c_double), c.POINTER(c.c_uint32),
                                     c.c_uint64, c.POINTER(c.c_uint64)]
    L.dhx_has_graph.argtypes = [vp, c.c_uint64]
    L.dhx_test_fail_next_call.argtypes = [vp]
    L.dhx_engine_open.argtypes = [c.c_int32, c.POINTER(vp)]
    L.dhx_engine_free.argtypes = [vp]
    L.dhx_allocate.argtypes = [vp, c.c_uint64, c.POINTER(Region)]
    L.dhx_weight.argtypes = [vp, vp, c.c_uint64, c.POINTER(Region)]
    L.dhx_upload.argtypes = [vp, Region, vp, c.c_uint64]
    L.dhx_record.argtypes = [vp, c.c_uint64, c.POINTER(Launch), c.c_uint64]
    L.dhx_record_branches.argtypes = [vp, c.c_uint64, c.POINTER(Launch), c.POINTER(c.c_uint64), c.c_uint32]
    L.dhx_replay.argtypes = [vp, c.c_uint64]
    L.dhx_dispatch.argtypes = [vp, c.c_uint64]
    L.dhx_reserve_readback.argtypes = [vp, c.c_uint64]
    L.dhx_read.argtypes = [vp, Region, vp, c.c_uint64]
    L.dhx_reserve_staging.argtypes = [vp, c.c_uint64, c.c_uint64]
    L.dhx_fragment_order.argtypes = [vp, c.c_uint64, c.c_uint64, vp]
    L.dhx_row_order.argtypes = [vp, c.c_uint64, c.c_uint64, vp]
    L.dhx_copy_in.argtypes = [vp, Region, vp, c.c_uint64, c.c_uint32]
    L.dhx_replay_slot.argtypes = [vp, c.c_uint64, c.c_uint32]
    L.dhx_copy_out.argtypes = [vp, Region, c.c_uint64, c.c_uint32]
    L.dhx_copy_out_finish.argtypes = [vp, vp, c.c_uint64, c.c_uint32]
    L.dhx_benchmark.argtypes = [vp, c.c_uint64, c.c_uint64, c.POINTER(_Timings)]
    return L


_lib = _load_library()


def _check(rc: int, handle=None) -> None:
    if rc != 0:
        raise DINOv3Error(_lib.dinov3_last_error(handle).decode("utf-8", "replace"))


def _check_engine(rc: int, engine) -> None:
    if rc != 0:
        raise DINOv3Error(_lib.dhx_last_error(engine).decode("utf-8", "replace"))


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@dataclass
class Options:
    """lib.rs:15-27. image_size extends the reference (fixed at 224)."""
    device: int = 0
    max_batch: int = 32
    image_size: int = 224

    def _c(self) -> _Options:
        return _Options(int(self.device), int(self.max_batch), int(self.image_size))


@dataclass
class Distribution:
    median_ms: float
    p95_ms: float


@dataclass
class ForwardTimings:
    """engine.rs:272-284: host-clock timings of a resident forward, excluding transfers."""
    samples: int
    graph: Distribution
    direct: Distribution


class DINOv3:
    """Resident model on one GPU (lib.rs:28-35). Not thread-safe."""

    def __init__(self, handle: int):
        self._h = ctypes.c_void_p(handle)

    @classmethod
    def load(cls, path: str, options: Options | None = None) -> "DINOv3":
        """lib.rs:49-88."""
        o = (options or Options())._c()
        h = ctypes.c_void_p()
        _check(_lib.dinov3_load(os.fsencode(str(path)), ctypes.byref(o), ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_pretrained(cls, options: Options | None = None) -> "DINOv3":
        """lib.rs:40-46 on the local Hugging Face cache (no downloads)."""
        o = (options or Options())._c()
        h = ctypes.c_void_p()
        _check(_lib.dinov3_from_pretrained(ctypes.byref(o), ctypes.byref(h)))
        return cls(h.value)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.dinov3_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def image_elements(self) -> int:
        return int(_lib.dinov3_image_elements(self._h))

    @property
    def tokens(self) -> int:
        return int(_lib.dinov3_tokens(self._h))

    def _pixels(self, pixels) -> np.ndarray:
        return np.ascontiguousarray(pixels, dtype=np.float32).reshape(-1)

    def forward_noalloc(self, d_pixels: int, images: int, d_out: int, stream: int = 0) -> None:
        """dinov3_forward_noalloc: device addresses in and out (images x 3 x S
        x S and images x T x 384 float32), launches queued on `stream` (a
        hipStream_t, 0 = the model's own) without waiting; no allocation."""
        _check(_lib.dinov3_forward_noalloc(self._h, ctypes.c_void_p(d_pixels), images, ctypes.c_void_p(d_out),
                                           ctypes.c_void_p(stream)), self._h)

    def forward(self, pixels) -> np.ndarray:
        """lib.rs:90-114. Returns float32 [batch, T, 384] (T = 201 at 224x224)."""
        px = self._pixels(pixels)
        images = px.size // max(self.image_elements, 1)
        out = np.empty((images, self.tokens, HIDDEN), np.float32)
        _check(_lib.dinov3_forward(self._h, _fptr(px), px.size, _fptr(out), out.size), self._h)
        return out

    def cls(self, pixels) -> np.ndarray:
        """lib.rs:126-132. float32 [batch, 384]."""
        px = self._pixels(pixels)
        images = px.size // max(self.image_elements, 1)
        out = np.empty((images, HIDDEN), np.float32)
        _check(_lib.dinov3_cls(self._h, _fptr(px), px.size, _fptr(out), out.size), self._h)
        return out

    def patch_mean(self, pixels) -> np.ndarray:
        """lib.rs:134-148. float32 [batch, 384]."""
        px = self._pixels(pixels)
        images = px.size // max(self.image_elements, 1)
        out = np.empty((images, HIDDEN), np.float32)
        _check(_lib.dinov3_patch_mean(self._h, _fptr(px), px.size, _fptr(out), out.size), self._h)
        return out

    def benchmark(self, pixels, samples: int) -> ForwardTimings:
        """lib.rs:116-124."""
        px = self._pixels(pixels)
        t = _Timings()
        _check(_lib.dinov3_benchmark(self._h, _fptr(px), px.size, int(samples), ctypes.byref(t)), self._h)
        return ForwardTimings(int(t.samples), Distribution(t.graph.median_ms, t.graph.p95_ms),
                              Distribution(t.direct.median_ms, t.direct.p95_ms))

    # -- resident-batch controls (no reference counterpart) -----------------
    def stage(self, pixels) -> None:
        """Upload one batch and replay its graph once (no readback)."""
        px = self._pixels(pixels)
        _check(_lib.dinov3_stage(self._h, _fptr(px), px.size), self._h)

    def replay(self, images: int) -> None:
        """Replay the recorded graph for `images` on the resident input."""
        _check(_lib.dinov3_replay(self._h, int(images)), self._h)

    def synchronize(self) -> None:
        e = _lib.dinov3_engine(self._h)
        _check_engine(_lib.dhx_synchronize(e), e)

    def set_splitk(self, mode: int) -> None:
        """Down projection: 0 (default) the residual GEMM, 1 split-K + reduce, at every batch size."""
        _check(_lib.dinov3_set_splitk(self._h, int(mode)), self._h)

    def set_layernorm_fusion(self, on: bool) -> None:
        """True (default): LayerNorm folded into the QKV / gate-up GEMMs; False: separate LayerNorm kernels."""
        _check(_lib.dinov3_set_layernorm_fusion(self._h, int(bool(on))), self._h)

    def set_branches(self, n: int) -> None:
        """Image groups run as concurrent graph branches for batches >= 4*n (default 3)."""
        _check(_lib.dinov3_set_branches(self._h, int(n)), self._h)

    def launch_timings(self, images: int, iters: int = 20) -> list[tuple[str, float]]:
        """Average device ms of each launch of the plan recorded for `images` (HIP events on the model's stream)."""
        cap = 256
        ms = (ctypes.c_double * cap)()
        kid = (ctypes.c_uint32 * cap)()
        n = ctypes.c_uint64()
        _check(_lib.dinov3_launch_timings(self._h, int(images), int(iters), ms, kid, cap, ctypes.byref(n)), self._h)
        return [(KERNELS[kid[i]], ms[i]) for i in range(n.value)]

    def _fail_next_gpu_call(self) -> None:
        """Test hook: the next HIP-facing engine call fails and poisons the session."""
        e = _lib.dinov3_engine(self._h)
        _check_engine(_lib.dhx_test_fail_next_call(e), e)


def hub_weights() -> str:
    """hub.rs:17-28 with downloads disabled: the cached pinned snapshot path."""
    buf = ctypes.create_string_buffer(4096)
    _check(_lib.dinov3_hub_weights(buf, len(buf)))
    return buf.value.decode()


def write_random_weights(path: str, seed: int = 0, preset: int = 0) -> str:
    """Seeded HF-named float32 safetensors (preset 0 = BASELINE init, 1 = stress)."""
    _check(_lib.dinov3_write_random_weights(os.fsencode(str(path)), int(seed), int(preset)))
    return str(path)


def random_pixels(seed: int, images: int, image_size: int = 224) -> np.ndarray:
    """Seeded i.i.d. N(0,1) float32 NCHW [images, 3, S, S]."""
    out = np.empty((images, 3, image_size, image_size), np.float32)
    _check(_lib.dinov3_random_pixels(int(seed), int(images), int(image_size), _fptr(out)))
    return out


def patchify(pixels, image_size: int = 224) -> np.ndarray:
    """lib.rs:265-280 on the host: [images*P, 768]."""
    px = np.ascontiguousarray(pixels, dtype=np.float32).reshape(-1)
    images = px.size // (3 * image_size * image_size)
    g = image_size // 16
    out = np.empty((images * g * g, 768), np.float32)
    _check(_lib.dinov3_patchify(_fptr(px), images, int(image_size), _fptr(out)))
    return out


def fragment_order(a: np.ndarray) -> np.ndarray:
    """Row-major f16 [rows][k] -> the kernels' fragment order (rows padded to 32)."""
    a = np.ascontiguousarray(a, np.float16)
    rows, k = a.shape
    out = np.empty(((rows + 31) // 32 * 32 * k,), np.float16)
    if _lib.dhx_fragment_order(a.ctypes.data, rows, k, out.ctypes.data) != 0:
        raise DINOv3Error(_lib.dhx_last_error(None).decode())
    return out


def row_order(f: np.ndarray, rows: int, k: int) -> np.ndarray:
    """Inverse of fragment_order."""
    f = np.ascontiguousarray(f, np.float16)
    if f.size < (rows + 31) // 32 * 32 * k:
        raise DINOv3Error("fragment buffer too small")
    out = np.empty((rows, k), np.float16)
    if _lib.dhx_row_order(f.ctypes.data, rows, k, out.ctypes.data) != 0:
        raise DINOv3Error(_lib.dhx_last_error(None).decode())
    return out


def pack_f16(name: str, values) -> np.ndarray:
    """weights.rs:6-17: float16 bits, rejecting values that overflow."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    _check(_lib.dinov3_pack_f16(name.encode(), _fptr(v), v.size, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))))
    return out


class Engine:
    """The engine-level C ABI (include/dinov3_engine.h): one device, one
    stream, resident buffers and one hipGraph per recorded batch key."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        if _lib.dhx_engine_open(int(device), ctypes.byref(h)) != 0:
            raise DINOv3Error(_lib.dhx_last_error(None).decode())
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.dhx_engine_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _c(self, rc: int) -> None:
        _check_engine(rc, self._h)

    def allocate(self, nbytes: int) -> Region:
        r = Region()
        self._c(_lib.dhx_allocate(self._h, int(nbytes), ctypes.byref(r)))
        return r

    def weight(self, array: np.ndarray) -> Region:
        a = np.ascontiguousarray(array)
        r = Region()
        self._c(_lib.dhx_weight(self._h, a.ctypes.data, a.nbytes, ctypes.byref(r)))
        return r

    def upload(self, region: Region, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        self._c(_lib.dhx_upload(self._h, region, a.ctypes.data, a.nbytes))

    def record(self, key: int, launches: list[tuple[int, list[int], list[Region]]]) -> None:
        self.record_branches(key, [launches])

    def record_branches(self, key: int, branches: list[list[tuple[int, list[int], list[Region]]]]) -> None:
        """Record launch lists that may run concurrently (each list in order) as one graph."""
        flat = [l for b in branches for l in b]
        arr = (Launch * max(1, len(flat)))()
        for i, (kernel, scalars, bindings) in enumerate(flat):
            if len(scalars) > MAX_SCALARS or len(bindings) > MAX_BINDINGS:
                raise ValueError("too many scalars or bindings for one launch")
            arr[i].kernel = kernel
            for j, v in enumerate(scalars):
                arr[i].scalars[j] = v
            arr[i].n_bindings = len(bindings)
            for j, b in enumerate(bindings):
                arr[i].bindings[j] = b
        counts = (ctypes.c_uint64 * max(1, len(branches)))(*[len(b) for b in branches])
        self._c(_lib.dhx_record_branches(self._h, int(key), arr, counts, len(branches)))

    def replay(self, key: int) -> None:
        self._c(_lib.dhx_replay(self._h, int(key)))

    def dispatch(self, key: int) -> None:
        self._c(_lib.dhx_dispatch(self._h, int(key)))

    def synchronize(self) -> None:
        self._c(_lib.dhx_synchronize(self._h))

    def reserve_staging(self, in_bytes: int, out_bytes: int) -> None:
        """Pinned staging for the pipelined transfers (two slots)."""
        self._c(_lib.dhx_reserve_staging(self._h, int(in_bytes), int(out_bytes)))

    def copy_in(self, region: Region, array: np.ndarray, slot: int) -> None:
        a = np.ascontiguousarray(array)
        self._c(_lib.dhx_copy_in(self._h, region, a.ctypes.data, a.nbytes, int(slot)))

    def replay_slot(self, key: int, slot: int) -> None:
        self._c(_lib.dhx_replay_slot(self._h, int(key), int(slot)))

    def copy_out(self, region: Region, nbytes: int, slot: int) -> None:
        self._c(_lib.dhx_copy_out(self._h, region, int(nbytes), int(slot)))

    def copy_out_finish(self, dtype, shape, slot: int) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._c(_lib.dhx_copy_out_finish(self._h, out.ctypes.data, out.nbytes, int(slot)))
        return out

    def reserve_readback(self, nbytes: int) -> None:
        self._c(_lib.dhx_reserve_readback(self._h, int(nbytes)))

    def read(self, region: Region, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._c(_lib.dhx_read(self._h, region, out.ctypes.data, out.nbytes))
        return out

    def benchmark(self, key: int, samples: int) -> ForwardTimings:
        t = _Timings()
        self._c(_lib.dhx_benchmark(self._h, int(key), int(samples), ctypes.byref(t)))
        return ForwardTimings(int(t.samples), Distribution(t.graph.median_ms, t.graph.p95_ms),
                              Distribution(t.direct.median_ms, t.direct.p95_ms))

    def launch_timings(self, key: int, iters: int = 20) -> list[tuple[str, float]]:
        cap = 256
        ms = (ctypes.c_double * cap)()
        kid = (ctypes.c_uint32 * cap)()
        n = ctypes.c_uint64()
        self._c(_lib.dhx_launch_timings(self._h, int(key), int(iters), ms, kid, cap, ctypes.byref(n)))
        return [(KERNELS[kid[i]], ms[i]) for i in range(n.value)]


def region_slice(region: Region, offset: int, nbytes: int) -> Region:
    """A sub-range of a region (Buffer::try_slice)."""
    if offset + nbytes > region.bytes:
        raise ValueError("slice exceeds region")
    return Region(region.buffer, region.offset + offset, nbytes)
