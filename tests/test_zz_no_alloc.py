"""sxh_sort_isect_noalloc (the allocation-free device-buffer sort) against sxh_sort_isect.

Two calls in a row on the same device share the library's scratch array: the first at the array's
capacity (2^21 keys, 45-bit keys: 6 passes, the result's last pass lands in the output after an even
count), the second smaller (36-bit keys: 5 passes, odd), over what the first left in the array. Each
result is compared bit for bit with the staged entry point's, whose sort is the same. Then the
rejections: one key over the capacity, a host pointer, an output aliasing its input (the same address
or one element past it), outputs overlapping each other, buffers shorter than n elements.
"""
import ctypes as C

import numpy as np
import pytest

import splatx_hip as sh

pytestmark = pytest.mark.gpu

MAX_KEYS = 1 << 21


class Hip:
    """The HIP runtime the library itself links (libamdhip64.so.7), for the test's own device buffers."""

    def __init__(self):
        self.lib = C.CDLL("libamdhip64.so.7")
        for f in ("hipMalloc", "hipFree", "hipMemcpy", "hipDeviceSynchronize", "hipMemGetAddressRange"):
            getattr(self.lib, f).restype = C.c_int

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.lib.hipMalloc(C.byref(p), C.c_size_t(max(nbytes, 16))) == 0
        return p

    def size_from(self, p):
        """Bytes of p's allocation from p on, as the runtime reports them."""
        base, size = C.c_void_p(), C.c_size_t()
        assert self.lib.hipMemGetAddressRange(C.byref(base), C.byref(size), p) == 0
        return size.value - (p.value - base.value)

    def free(self, p):
        assert self.lib.hipFree(p) == 0

    def h2d(self, dst, a):
        assert self.lib.hipMemcpy(dst, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) == 0

    def d2h(self, a, src):
        assert self.lib.hipMemcpy(a.ctypes.data_as(C.c_void_p), src, C.c_size_t(a.nbytes), 2) == 0


def tile_depth_keys(rng, n, bits):
    """(tile | depth-bits) keys of `bits` bits with ties (a few depths repeat), values = emit indices."""
    tile_bits = bits - 32
    tiles = rng.integers(0, 1 << tile_bits, n, dtype=np.uint64)
    depths = rng.uniform(0.5, 50.0, n).astype(np.float32)
    depths[rng.integers(0, n, n // 10)] = np.float32(7.25)  # tied depths
    keys = (tiles << np.uint64(32)) | depths.view(np.uint32).astype(np.uint64)
    return keys, np.arange(n, dtype=np.int32)


def noalloc(gpu, hip, keys, vals, bits, out_n=None):
    n = keys.size
    bufs = [hip.alloc(keys.nbytes), hip.alloc(vals.nbytes), hip.alloc(keys.nbytes), hip.alloc(vals.nbytes)]
    try:
        hip.h2d(bufs[0], keys)
        hip.h2d(bufs[1], vals)
        f = gpu.lib.sxh_sort_isect_noalloc
        f.restype = C.c_int32
        f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_uint32, C.c_void_p, C.c_void_p]
        rc = f(gpu.handle, bufs[0], bufs[1], n, bits, bufs[2], bufs[3])
        assert rc == sh.SXH_OK, gpu.lib.sxh_last_error()
        ks, vs = np.zeros_like(keys), np.zeros_like(vals)
        hip.d2h(ks, bufs[2])
        hip.d2h(vs, bufs[3])
        k_in, v_in = np.zeros_like(keys), np.zeros_like(vals)
        hip.d2h(k_in, bufs[0])
        hip.d2h(v_in, bufs[1])
        assert np.array_equal(k_in, keys) and np.array_equal(v_in, vals)  # inputs left as they were
        return ks, vs
    finally:
        for p in bufs:
            hip.free(p)


def test_noalloc_sort_matches_sort_isect_on_two_calls(gpu):
    hip = Hip()
    rng = np.random.Generator(np.random.PCG64(2024))
    for n, bits in ((MAX_KEYS, 45), (300_001, 36)):
        print(f"noalloc sort: n={n} bits={bits}", flush=True)
        keys, vals = tile_depth_keys(rng, n, bits)
        ref_k, ref_v = gpu.sort_isect(keys, vals, bits)
        ks, vs = noalloc(gpu, hip, keys, vals, bits)
        assert np.array_equal(ks, ref_k)
        assert np.array_equal(vs, ref_v)
        # the order itself: ascending, and stable (equal keys keep ascending values, the emit order)
        assert np.all(ks[1:] >= ks[:-1])
        same = ks[1:] == ks[:-1]
        assert same.sum() > 100 and np.all(vs[1:][same] > vs[:-1][same])


def test_noalloc_sort_rejections(gpu):
    hip = Hip()
    f = gpu.lib.sxh_sort_isect_noalloc
    f.restype = C.c_int32
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_uint32, C.c_void_p, C.c_void_p]
    kd, vd, ko, vo = hip.alloc(8 * 64), hip.alloc(4 * 64), hip.alloc(8 * 64), hip.alloc(4 * 64)
    try:
        rc = f(gpu.handle, kd, vd, MAX_KEYS + 1, 45, ko, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"exceeds the scratch capacity" in gpu.lib.sxh_last_error()
        host_keys = np.zeros(64, np.uint64)
        rc = f(gpu.handle, host_keys.ctypes.data_as(C.c_void_p), vd, 64, 45, ko, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"keys is not device memory" in gpu.lib.sxh_last_error()
        rc = f(gpu.handle, kd, vd, 64, 45, kd, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"must not alias" in gpu.lib.sxh_last_error()
        # an output one element past its input (partly overlapping), and one over the other input
        rc = f(gpu.handle, kd, vd, 32, 45, C.c_void_p(kd.value + 8), vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"must not alias" in gpu.lib.sxh_last_error()
        rc = f(gpu.handle, kd, vd, 16, 45, ko, C.c_void_p(kd.value + 8))
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"must not alias" in gpu.lib.sxh_last_error()
        rc = f(gpu.handle, kd, vd, 16, 45, ko, C.c_void_p(ko.value + 64))
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"overlap" in gpu.lib.sxh_last_error()
        # one element more than the keys' allocation holds (as the runtime reports its size), and an
        # output that starts 8 elements before the end of its allocation
        n_over = hip.size_from(kd) // 8 + 1
        assert n_over <= MAX_KEYS
        rc = f(gpu.handle, kd, vd, n_over, 45, ko, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"fewer than n elements" in gpu.lib.sxh_last_error()
        tail = C.c_void_p(ko.value + hip.size_from(ko) - 64)
        rc = f(gpu.handle, kd, vd, 16, 45, tail, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"keys_sorted holds fewer than n" in gpu.lib.sxh_last_error()
        rc = f(gpu.handle, kd, vd, 64, 0, ko, vo)
        assert rc == sh.SXH_ERR_INVALID_ARGUMENT and b"key_n_bits must be 1..64" in gpu.lib.sxh_last_error()
        assert f(gpu.handle, kd, vd, 0, 45, ko, vo) == sh.SXH_OK  # empty: nothing to do
    finally:
        for p in (kd, vd, ko, vo):
            hip.free(p)
