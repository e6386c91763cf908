"""Host-side refusals of mbh_histogram_noalloc (the entry point that
allocates nothing): shapes whose one block partial does not fit the static
scratch are refused before anything is enqueued, so these run without a GPU
(no device pointer is touched)."""
import ctypes as C

from mojoboost_amd import _lib
from mojoboost_amd._lib import lib


def test_noalloc_refuses_sizes_beyond_the_scratch():
    """A partial that cannot fit the static scratch is refused on the host,
    before anything is enqueued (no device pointer is touched)."""
    err = C.create_string_buffer(512)
    fake = C.c_void_p(1)
    # 9000 * 256 * 8 bytes > 16 MiB; 2^24 * 256 cells overflow a 32-bit
    # cell count (to 0), which must still be refused, not divided by
    for f, nb in ((9000, 256), (1 << 24, 256), ((1 << 31) - 1, 256)):
        err.value = b""
        rc = lib().mbh_histogram_noalloc(fake, 1000, f, nb, fake, fake, None, 0, 4, fake, None, None,
                                         err, 512)
        assert rc == _lib.ERROR_INVALID_ARGUMENT, (f, nb)
        assert b"scratch" in err.value, (f, nb)
