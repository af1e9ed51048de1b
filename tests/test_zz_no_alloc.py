"""dinov3_forward_noalloc (include/dinov3.h) through the C ABI, against
dinov3_forward on the same images: bitwise the same outputs on two calls in a
row, the second smaller than the first, on a stream of the caller's and on
the model's own stream; batch 1 with the split-K plan (its f32 slabs in the
array too) and 512x512; a batch beyond the
scratch array refused before anything is queued. Device memory for the
inputs and outputs comes from the HIP runtime the library itself links
(/opt/rocm), allocated here by the test, never by the entry point."""
import ctypes
import os

import numpy as np
import pytest

import dinov3_hrx as d

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip(gpu):
    lib = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so.7")
    vp, c = ctypes.c_void_p, ctypes
    lib.hipMalloc.argtypes = [c.POINTER(vp), c.c_size_t]
    lib.hipFree.argtypes = [vp]
    lib.hipMemcpy.argtypes = [vp, vp, c.c_size_t, c.c_int]
    lib.hipStreamCreate.argtypes = [c.POINTER(vp)]
    lib.hipStreamSynchronize.argtypes = [vp]
    lib.hipStreamDestroy.argtypes = [vp]
    lib.hipDeviceSynchronize.argtypes = []
    return lib


class Device:
    """Device buffers and copies through the library's own HIP runtime."""

    def __init__(self, hip):
        self.hip, self.ptrs = hip, []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(p), nbytes) == 0
        self.ptrs.append(p.value)
        return p.value

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        p = self.alloc(a.nbytes)
        assert self.hip.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0  # hipMemcpyHostToDevice
        return p

    def download(self, p, shape):
        out = np.empty(shape, np.float32)
        assert self.hip.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # hipMemcpyDeviceToHost
        return out

    def free(self):
        self.hip.hipDeviceSynchronize()
        for p in self.ptrs:
            self.hip.hipFree(p)


def noalloc(hip, dev, model, px, stream):
    images = px.shape[0]
    dpx = dev.upload(px)
    dout = dev.alloc(images * model.tokens * 384 * 4)
    model.forward_noalloc(dpx, images, dout, stream)
    assert hip.hipStreamSynchronize(ctypes.c_void_p(stream)) == 0
    return dev.download(dout, (images, model.tokens, 384))


def test_noalloc_matches_forward(hip, weight_file):
    dev = Device(hip)
    stream = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        with d.DINOv3.load(weight_file(1), d.Options(0, 8)) as m:
            # two calls in a row, the second smaller (the array keeps the
            # first call's data), on the caller's stream
            for images, seed in ((6, 41), (2, 42)):
                px = d.random_pixels(seed, images)
                got = noalloc(hip, dev, m, px, stream.value)
                want = m.forward(px)
                print(f"noalloc {images} images: max |diff| {np.abs(got - want).max()}")
                assert np.array_equal(got, want), images
            # batch 1 with the split-K down projection, on the model's own stream
            px = d.random_pixels(43, 1)
            dpx, dout = dev.upload(px), dev.alloc(201 * 384 * 4)
            m.set_splitk(1)
            try:
                m.forward_noalloc(dpx, 1, dout, 0)
                m.synchronize()
                assert np.array_equal(dev.download(dout, (1, 201, 384)), m.forward(px))
            finally:
                m.set_splitk(0)
            # a batch the array cannot hold is refused before anything is queued
            big = dev.alloc(44 * 3 * 224 * 224 * 4)
            with pytest.raises(d.DINOv3Error, match="bytes of scratch"):
                m.forward_noalloc(big, 44, big, stream.value)
            with pytest.raises(d.DINOv3Error, match="16-byte aligned"):
                m.forward_noalloc(dpx + 4, 1, dout, stream.value)
            got = noalloc(hip, dev, m, d.random_pixels(44, 3), stream.value)  # still usable
            assert np.array_equal(got, m.forward(d.random_pixels(44, 3)))
        with d.DINOv3.load(weight_file(1), d.Options(0, 2, 512)) as m:
            px = d.random_pixels(45, 2, 512)
            got = noalloc(hip, dev, m, px, stream.value)
            assert np.array_equal(got, m.forward(px))
    finally:
        dev.free()
        hip.hipStreamDestroy(stream)
