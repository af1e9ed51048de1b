"""dinov3_forward_noalloc (include/dinov3.h) through the C ABI, against
dinov3_forward on the same images: bitwise the same outputs on two calls in a
row, the second smaller than the first, on a stream of the caller's and on
the model's own stream; batch 1 with the split-K plan (its f32 slabs in the
array too), the unfused LayerNorm plan (its h buffer in the array instead of
the statistics) and 512x512; a batch beyond the scratch array refused before
anything is queued. The contract itself: calls queued back to back on two
streams (and from two models) without a host wait in between run in turn;
the caller's current device is left as it was; a call captured into a HIP
graph replays correctly between eager calls; and a call allocates no device
memory (free memory unchanged). Device memory for the inputs and outputs
comes from the HIP runtime the library itself links (/opt/rocm), allocated
here by the test, never by the entry point."""
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
    lib.hipGetDevice.argtypes = [c.POINTER(c.c_int)]
    lib.hipSetDevice.argtypes = [c.c_int]
    lib.hipMemset.argtypes = [vp, c.c_int, c.c_size_t]
    lib.hipMemGetInfo.argtypes = [c.POINTER(c.c_size_t), c.POINTER(c.c_size_t)]
    lib.hipStreamBeginCapture.argtypes = [vp, c.c_int]
    lib.hipStreamEndCapture.argtypes = [vp, c.POINTER(vp)]
    lib.hipGraphInstantiate.argtypes = [c.POINTER(vp), vp, vp, c.c_char_p, c.c_size_t]
    lib.hipGraphLaunch.argtypes = [vp, vp]
    lib.hipGraphExecDestroy.argtypes = [vp]
    lib.hipGraphDestroy.argtypes = [vp]
    return lib


def new_stream(hip):
    s = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    return s


def current_device(hip):
    dev = ctypes.c_int(-1)
    assert hip.hipGetDevice(ctypes.byref(dev)) == 0
    return dev.value


def free_bytes(hip):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


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


def test_noalloc_unfused_layernorm_plan(hip, weight_file):
    # With the LayerNorm kernels run separately the array holds an h buffer
    # and no row statistics: another layout of the same array.
    dev = Device(hip)
    stream = new_stream(hip)
    try:
        with d.DINOv3.load(weight_file(1), d.Options(0, 8)) as m:
            m.set_layernorm_fusion(0)
            for images, seed in ((5, 61), (2, 62)):
                px = d.random_pixels(seed, images)
                assert np.array_equal(noalloc(hip, dev, m, px, stream.value), m.forward(px)), images
    finally:
        dev.free()
        hip.hipStreamDestroy(stream)


def test_noalloc_overlapping_calls_run_in_turn(hip, weight_file):
    # Calls queued back to back on two streams, with no host wait between
    # them, from one model and then from two models on the same GPU: each
    # call's stream waits for the one before, so both outputs are right. The
    # caller's current device is unchanged by every call.
    dev = Device(hip)
    s1, s2 = new_stream(hip), new_stream(hip)
    try:
        assert hip.hipSetDevice(0) == 0
        with d.DINOv3.load(weight_file(1), d.Options(0, 8)) as m1, d.DINOv3.load(weight_file(0), d.Options(0, 4)) as m2:
            cases = [(m1, d.random_pixels(71, 7), s1), (m1, d.random_pixels(72, 3), s2),
                     (m2, d.random_pixels(73, 4), s1), (m1, d.random_pixels(74, 6), s2)]
            bufs = []
            for m, px, _ in cases:  # every upload first: the calls below are queued with no wait between them
                bufs.append((dev.upload(px), dev.alloc(px.shape[0] * 201 * 384 * 4)))
            for (m, px, s), (dpx, dout) in zip(cases, bufs):
                m.forward_noalloc(dpx, px.shape[0], dout, s.value)
                assert current_device(hip) == 0
            for s in (s1, s2):
                assert hip.hipStreamSynchronize(s) == 0
            for i, ((m, px, _), (_, dout)) in enumerate(zip(cases, bufs)):
                got = dev.download(dout, (px.shape[0], 201, 384))
                assert np.array_equal(got, m.forward(px)), f"call {i}"
    finally:
        dev.free()
        hip.hipStreamDestroy(s1)
        hip.hipStreamDestroy(s2)


def test_noalloc_under_graph_capture(hip, weight_file):
    # One call captured on the caller's stream (global capture mode), the
    # graph instantiated and replayed three times, each replay after eager
    # calls of other images (which leave their own data in the array) and
    # a host synchronisation; every replay bitwise equal to forward().
    dev = Device(hip)
    stream = new_stream(hip)
    graph, exec_ = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        with d.DINOv3.load(weight_file(1), d.Options(0, 8)) as m:
            px = d.random_pixels(81, 5)
            want = m.forward(px)
            dpx, dout = dev.upload(px), dev.alloc(5 * 201 * 384 * 4)
            m.forward_noalloc(dpx, 5, dout, stream.value)  # warm-up, outside the capture
            assert hip.hipStreamSynchronize(stream) == 0
            assert hip.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
            try:
                m.forward_noalloc(dpx, 5, dout, stream.value)
            finally:
                end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
            assert end == 0 and graph.value
            assert hip.hipGraphInstantiate(ctypes.byref(exec_), graph, None, None, 0) == 0
            for rep, seed in enumerate((82, 83, 84)):
                other = d.random_pixels(seed, 3 + rep)
                assert np.array_equal(noalloc(hip, dev, m, other, stream.value), m.forward(other))
                assert hip.hipMemset(dout, 0, 5 * 201 * 384 * 4) == 0
                assert hip.hipGraphLaunch(exec_, stream) == 0
                assert hip.hipStreamSynchronize(stream) == 0
                assert np.array_equal(dev.download(dout, (5, 201, 384)), want), f"replay {rep}"
    finally:
        if exec_.value:
            hip.hipGraphExecDestroy(exec_)
        if graph.value:
            hip.hipGraphDestroy(graph)
        dev.free()
        hip.hipStreamDestroy(stream)


def test_noalloc_allocates_nothing(hip, weight_file):
    # After a first call (which may let the runtime set up what its kernels
    # need), further calls leave the device's free memory unchanged.
    dev = Device(hip)
    stream = new_stream(hip)
    try:
        with d.DINOv3.load(weight_file(1), d.Options(0, 8)) as m:
            px = d.random_pixels(91, 8)
            dpx, dout = dev.upload(px), dev.alloc(8 * 201 * 384 * 4)
            m.forward_noalloc(dpx, 8, dout, stream.value)
            assert hip.hipStreamSynchronize(stream) == 0
            before = free_bytes(hip)
            for _ in range(3):
                m.forward_noalloc(dpx, 8, dout, stream.value)
                m.forward_noalloc(dpx, 2, dout, 0)
            assert hip.hipStreamSynchronize(stream) == 0
            m.synchronize()
            after = free_bytes(hip)
            print(f"free device memory before {before}, after {after}")
            assert after == before
    finally:
        dev.free()
        hip.hipStreamDestroy(stream)
