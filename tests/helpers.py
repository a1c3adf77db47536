"""Shared helpers for the GPU parity tests: device buffers (allocated through
the library's own include/lcr_runtime.h, so only one HIP runtime is ever
loaded), seeded inputs rounded through the element type, and comparison
helpers with the reference's tolerance rule."""

from __future__ import annotations

import ctypes

import numpy as np

import oracle

BF16 = oracle.BF16
FP16 = oracle.FP16


def rng(seed=20260904):
    return np.random.default_rng(seed)


def elems(values: np.ndarray, kind=BF16) -> np.ndarray:
    """float32 values rounded to element bits (uint16)."""
    return oracle.f32_to_elems(np.asarray(values, dtype=np.float32), kind)


def to_f32(bits: np.ndarray, kind=BF16) -> np.ndarray:
    return oracle.elems_to_f32(np.asarray(bits, dtype=np.uint16), kind)


def random_elems(r, shape, scale=1.0, kind=BF16) -> np.ndarray:
    return elems(r.normal(0.0, scale, size=shape).astype(np.float32), kind)


def _lcr():
    from conftest import load_lcr
    return load_lcr()


# Every device buffer a test creates stays referenced here until the test's
# teardown (after a device synchronize), so an inline `p(dev(x))` cannot free
# memory that a queued kernel still reads.
LIVE = []


def release_all():
    if LIVE:
        sync()
        LIVE.clear()


def dev(a: np.ndarray):
    """A device copy of a host array (include/lcr_runtime.h memory)."""
    buf = _lcr().DeviceBuffer.from_array(np.ascontiguousarray(a))
    LIVE.append(buf)
    return buf


def zeros_dev(n, dtype=np.uint16):
    dt = np.dtype(dtype)
    buf = _lcr().DeviceBuffer(int(n) * dt.itemsize, dt, int(n))
    LIVE.append(buf)
    return buf


def host(buf, dtype=np.uint16) -> np.ndarray:
    sync()
    return buf.to_numpy(dtype)


def p(buf) -> int:
    return int(buf.ptr)


def sync():
    _lcr().synchronize()


def expect_close(ours, expected, tol=3e-2, what=""):
    """The reference's rule (tests/test_kernels.cu:92-122): worst |diff| over
    max |expected| must not exceed tol."""
    ours = np.asarray(ours, dtype=np.float64).ravel()
    expected = np.asarray(expected, dtype=np.float64).ravel()
    assert ours.shape == expected.shape, f"{what}: {ours.shape} vs {expected.shape}"
    scale = max(np.abs(expected).max(initial=0.0), 1e-6)
    err = np.abs(ours - expected) / scale
    i = int(err.argmax()) if err.size else 0
    assert err.size == 0 or err[i] <= tol, (
        f"{what}: worst relative error {err[i]:.4g} at {i} (got {ours[i]}, expected {expected[i]}, tol {tol})")


def expect_bits_equal(ours, expected, what=""):
    ours = np.asarray(ours).ravel()
    expected = np.asarray(expected).ravel()
    assert ours.shape == expected.shape, f"{what}: shape {ours.shape} vs {expected.shape}"
    diff = np.nonzero(ours != expected)[0]
    assert diff.size == 0, (f"{what}: {diff.size} of {ours.size} differ; first at {diff[0]}: "
                            f"{ours[diff[0]]} vs {expected[diff[0]]}")


def kv_view_structs(lcr, keys_t, values_t, table_t, page_size, page_stride, head_stride, kv_heads, head_dim):
    g = lcr.KvView(p(keys_t), p(values_t), p(table_t) if table_t is not None else None, page_size, page_stride,
                   head_stride, kv_heads, head_dim)
    return g


def oracle_view(keys: np.ndarray, values: np.ndarray, table: np.ndarray | None, page_size, page_stride,
                head_stride, kv_heads, head_dim):
    v = oracle.KvView()
    v.keys = keys.ctypes.data
    v.values = values.ctypes.data
    v.page_table = table.ctypes.data if table is not None else None
    v.page_size = page_size
    v.page_stride = page_stride
    v.head_stride = head_stride
    v.num_kv_heads = kv_heads
    v.head_dim = head_dim
    return v
