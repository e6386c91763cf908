"""mbh_histogram_noalloc (the entry point that allocates nothing) against
mbh_histogram on the same inputs: bit-identical int32 cells, on two calls in a
row, the second with a smaller input (fewer rows and features, a row subset),
so nothing the first call left in the shared scratch can leak into the second.

The test allocates the device buffers itself (hipMalloc through the HIP
runtime), as a caller of the no-alloc entry point does.
"""
import ctypes as C

import numpy as np
import pytest

from mojoboost_amd import _lib
from mojoboost_amd._lib import lib

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class _Hip:
    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.h.hipFree.argtypes = [C.c_void_p]
        self.h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.live = []

    def upload(self, a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        assert self.h.hipMalloc(C.byref(p), C.c_size_t(max(1, a.nbytes))) == 0
        self.live.append(p)
        assert self.h.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, H2D) == 0
        return p

    def empty(self, nbytes):
        p = C.c_void_p()
        assert self.h.hipMalloc(C.byref(p), C.c_size_t(nbytes)) == 0
        self.live.append(p)
        return p

    def download(self, p, like):
        out = np.empty_like(like)
        assert self.h.hipDeviceSynchronize() == 0
        assert self.h.hipMemcpy(out.ctypes.data_as(C.c_void_p), p, out.nbytes, D2H) == 0
        return out

    def free(self):
        for p in self.live:
            self.h.hipFree(p)
        self.live = []


def _noalloc(hip, bins, n, f, nb, qg, qh, rows, B=4):
    d_bins, d_qg, d_qh = hip.upload(bins), hip.upload(qg), hip.upload(qh)
    d_rows = None if rows is None else hip.upload(rows.astype(np.int32))
    cells = f * nb * 3
    d_out = hip.empty(cells * 4)
    d_status = hip.empty(4)
    err = C.create_string_buffer(512)
    rc = lib().mbh_histogram_noalloc(d_bins, n, f, nb, d_qg, d_qh, d_rows,
                                     0 if rows is None else len(rows), B, d_out, d_status, None,
                                     err, 512)
    assert rc == 0, err.value
    out = hip.download(d_out, np.zeros(cells, np.int32))
    status = hip.download(d_status, np.zeros(1, np.int32))
    return out.reshape(f, nb, 3), int(status[0])


def _case(rng, n, f, nb, B):
    bins = rng.integers(0, nb, size=(f, n), dtype=np.uint8)
    bins[min(3, f - 1)] %= 7  # a low-cardinality feature: hot bins
    qg = rng.integers(-(B // 2 + 1), B // 2 + 2, size=n).astype(np.int8)
    qh = rng.integers(0, B + 2, size=n).astype(np.int8)
    return bins, qg, qh


def test_noalloc_matches_mbh_histogram_twice():
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    rng = np.random.default_rng(0xA110C)
    hip = _Hip()
    try:
        # call 1: 300k rows x 28 features x 255 bins, every row
        n, f, nb = 300_000, 28, 255
        bins, qg, qh = _case(rng, n, f, nb, 4)
        ds = device.Dataset(bins, n, f, nb, np.zeros(n))
        want = ds.histogram(qg, qh, None, quant_bins=4)
        got, status = _noalloc(hip, bins, n, f, nb, qg, qh, None)
        assert status == 0
        assert np.array_equal(got, want)
        ds.free()
        # call 2: a smaller input (40k rows x 9 features x 64 bins, a row
        # subset, another lattice) on the same scratch
        n2, f2, nb2 = 40_000, 9, 64
        bins2, qg2, qh2 = _case(rng, n2, f2, nb2, 16)
        rows2 = np.sort(rng.choice(n2, 12_345, replace=False)).astype(np.int32)
        ds2 = device.Dataset(bins2, n2, f2, nb2, np.zeros(n2))
        want2 = ds2.histogram(qg2, qh2, rows2, quant_bins=16)
        got2, status2 = _noalloc(hip, bins2, n2, f2, nb2, qg2, qh2, rows2, B=16)
        assert status2 == 0
        assert np.array_equal(got2, want2)
        ds2.free()
    finally:
        hip.free()


def test_noalloc_flags_out_of_range_entries():
    """Entries out of range are left out and flag status 1, and every kernel
    still exits normally: a row id past n_rows and a bin id >= n_bins (the
    row's other features still count). The cells equal a brute-force
    histogram over the valid entries only."""
    from mojoboost_amd import device

    if device.device_count() < 1:
        pytest.fail("no gfx950 device visible to the HIP library")
    rng = np.random.default_rng(0xBAD1D)
    n, f, nb = 50_000, 6, 32
    bins, qg, qh = _case(rng, n, f, nb, 4)
    bad_row = 1234
    bins[2, bad_row] = 40  # >= n_bins (a valid uint8)
    rows = np.sort(rng.choice(n, 20_000, replace=False)).astype(np.int32)
    if bad_row not in rows:
        rows = np.sort(np.append(rows[1:], bad_row)).astype(np.int32)
    rows = np.append(rows, np.int32(n + 5))  # a row id past n_rows
    want = np.zeros((f, nb, 3), np.int64)
    valid = rows[rows < n]
    for j in range(f):
        b = bins[j, valid].astype(np.int64)
        ok = b < nb
        r = valid[ok]
        np.add.at(want[j, :, 0], b[ok], qg[r].astype(np.int64))
        np.add.at(want[j, :, 1], b[ok], qh[r].astype(np.int64))
        np.add.at(want[j, :, 2], b[ok], 1)
    hip = _Hip()
    try:
        got, status = _noalloc(hip, bins, n, f, nb, qg, qh, rows)
    finally:
        hip.free()
    assert status == 1
    assert np.array_equal(got.astype(np.int64), want)
