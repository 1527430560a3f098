"""hs_op_attend_decode_dev_noalloc (decode attention with its split partials in the library's
fixed per-GPU scratch array, no allocation) against hs_op_attend_decode_dev on the same inputs:
two calls in a row on every kernel path, the second smaller, so it runs over what the first
left in the array; and a shape whose partials do not fit is refused before any device work."""

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

TABLE = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
SCORE_M, SCORE_S, OUT_M, OUT_S = 1_400_000_000, 33, 1_300_000_000, 53


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


def _dev_buf(dev, arr):
    from taco_amd import hip
    p = C.c_void_p()
    hip._check(hip.lib().hs_device_alloc(dev.h, arr.nbytes, C.byref(p)))
    hip._check(hip.lib().hs_device_upload(dev.h, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
    return p


def _run(dev, fn, q, kc, vc, ctx):
    from taco_amd import hip
    B, H, cap, hd = kc.shape
    bufs = [_dev_buf(dev, a) for a in (q, kc, vc, ctx, TABLE)]
    out = np.zeros((B, H * hd), np.int8)
    dout = _dev_buf(dev, out)
    try:
        hip._check(fn(dev.h, bufs[0], bufs[1], bufs[2], bufs[3], B, H, hd, cap, SCORE_M, SCORE_S,
                      OUT_M, OUT_S, bufs[4], len(TABLE), 30, dout, None))
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
    finally:
        for p in bufs + [dout]:
            hip.lib().hs_device_free(dev.h, p)
    return out


def _case(seed, B, H, cap, hd):
    r = np.random.default_rng(seed)
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    kc = r.integers(-127, 128, (B, H, cap, hd)).astype(np.int8)
    vc = r.integers(-127, 128, (B, H, cap, hd)).astype(np.int8)
    ctx = r.integers(1, cap + 1, B).astype(np.uint32)
    ctx[0] = cap
    return q, kc, vc, ctx


# (streams, heads, positions, head_dim) of the first call, then of the second (smaller) call:
# split-key kernels (head dims 16 to 256, head_dim 64 past 1,024 keys), the one-launch kernel
# (head_dim 64, at most 1,024 keys) and the row kernel (head_dim 48).
SHAPES = [
    ((16, 12, 2048, 64), (3, 12, 1100, 64)),
    ((8, 12, 600, 16), (2, 5, 70, 16)),
    ((8, 12, 512, 128), (4, 3, 129, 128)),
    ((6, 4, 700, 256), (1, 4, 65, 256)),
    ((8, 12, 1024, 64), (2, 12, 300, 64)),
    ((4, 6, 320, 48), (1, 2, 20, 48)),
]


@pytest.mark.parametrize("first,second", SHAPES)
def test_noalloc_equals_the_allocating_entry(dev, first, second):
    from taco_amd import hip
    L = hip.lib()
    for i, shape in enumerate((first, second)):
        print(f"noalloc: call {i + 1}, shape {shape}", flush=True)
        q, kc, vc, ctx = _case(97 + 13 * i + shape[3], *shape)
        got = _run(dev, L.hs_op_attend_decode_dev_noalloc, q, kc, vc, ctx)
        want = _run(dev, L.hs_op_attend_decode_dev, q, kc, vc, ctx)
        assert np.array_equal(got, want), f"call {i + 1} {shape}"
        if shape[0] * shape[1] * shape[2] <= 40_000:
            ref = O.attend_decode_ref(q, kc, vc, ctx, SCORE_M, SCORE_S, OUT_M, OUT_S, TABLE, 30)
            assert np.array_equal(got, ref), f"call {i + 1} {shape} against the oracle"


def test_noalloc_refuses_partials_beyond_the_fixed_scratch(dev):
    """One stream, one head of 16 over 20M positions needs 80 MB of dots: refused with
    HS_UNSUPPORTED before any launch (the caches are allocated and never read)."""
    from taco_amd import hip
    L = hip.lib()
    cap, hd = 20_000_000, 16
    ptrs = []
    for nbytes in (hd, cap * hd, cap * hd, 4 * len(TABLE), hd):
        p = C.c_void_p()
        hip._check(L.hs_device_alloc(dev.h, nbytes, C.byref(p)))
        ptrs.append(p)
    ctx = _dev_buf(dev, np.array([cap], np.uint32))
    try:
        st = L.hs_op_attend_decode_dev_noalloc(dev.h, ptrs[0], ptrs[1], ptrs[2], ctx, 1, 1, hd,
                                               cap, SCORE_M, SCORE_S, OUT_M, OUT_S, ptrs[3],
                                               len(TABLE), 30, ptrs[4], None)
        assert st == hip.HS_UNSUPPORTED
        assert b"fixed scratch" in L.hs_last_error_message()
    finally:
        for p in ptrs + [ctx]:
            L.hs_device_free(dev.h, p)
