"""The allocation-free digest entry point (``lcdhip_digest_noalloc``) against
``lcdhip_digest``, through the C ABI: bit-equal 128-bit results on two calls in
a row, the second on a smaller input (so partial results the first call left
in the library's work area would show), plus the empty input, the size limit
and an input large enough to use every partial-result slot."""

import ctypes

import numpy as np
import pytest

from lcd_amd import hip_runtime

pytestmark = pytest.mark.gpu


def _both(device, host_words, out):
    array = device.to_device(host_words)
    device.digest_noalloc(array, out)
    got = out.copy_to_host()          # synchronises the library stream
    expected = device.digest(array)
    return (int(got[0]), int(got[1])), expected


def test_noalloc_digest_matches_the_allocating_one(device):
    rng = np.random.default_rng(7)
    out = device.empty((2,), np.uint64)
    large = rng.integers(0, 2**31 - 1, size=1_500_000, dtype=np.int32)
    small = large[:777].copy()
    print("digest_noalloc: 1.5 M words, then 777 words", flush=True)
    got, expected = _both(device, large, out)
    assert got == expected
    got_small, expected_small = _both(device, small, out)
    assert got_small == expected_small
    assert got_small != got
    # the same bytes again give the same digest; one changed word does not
    again, _ = _both(device, small, out)
    assert again == got_small
    changed = small.copy()
    changed[5] ^= 1
    other, expected_other = _both(device, changed, out)
    assert other == expected_other and other != got_small


def test_noalloc_digest_edges(device):
    out = device.empty((2,), np.uint64)
    lib = device.lib
    # empty input: both entry points agree on the digest of nothing
    host = (ctypes.c_uint64 * 2)()
    assert lib.lcdhip_digest(None, ctypes.c_size_t(0), host, device.stream) == 0
    assert lib.lcdhip_digest_noalloc(None, ctypes.c_size_t(0),
                                     ctypes.c_void_p(out.pointer),
                                     device.stream) == 0
    got = out.copy_to_host()
    assert (int(got[0]), int(got[1])) == (int(host[0]), int(host[1]))
    # more words than one pass of the largest grid covers
    big = np.arange(1024 * 256 * 3 + 11, dtype=np.int32)
    got_big, expected_big = _both(device, big, out)
    assert got_big == expected_big
    # beyond the stated maximum, and a ragged size: clear errors, no launch
    some = device.to_device(np.zeros(4, np.int32))
    too_many = ctypes.c_size_t((1 << 36) + 4)
    assert lib.lcdhip_digest_noalloc(
        ctypes.c_void_p(some.pointer), too_many, ctypes.c_void_p(out.pointer),
        device.stream) == hip_runtime.ERR_ARGUMENT
    lib.lcdhip_last_error.restype = ctypes.c_char_p
    assert b"limit" in lib.lcdhip_last_error()
    assert lib.lcdhip_digest_noalloc(
        ctypes.c_void_p(some.pointer), ctypes.c_size_t(6),
        ctypes.c_void_p(out.pointer), device.stream) == hip_runtime.ERR_ARGUMENT
