"""mimir_layernorm_bwd_noalloc -- the LayerNorm backward that allocates
nothing (its scratch is a fixed per-GPU device array) -- against
mimir_layernorm_bwd through the C ABI: bit-identical dx / dgamma / dbeta on
two calls in a row, the second smaller, on every kernel family (register-
resident rows, 4-byte-column rows, generic rows, rows split over many
workgroups); a call that needs more scratch than the array holds is refused;
the device's free memory does not move across the calls; and one context per
GPU holds the array at a time (another context's call is refused with EBUSY
until the holder is destroyed)."""
import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p

import numpy as np
import pytest

import mimir_hip as M

pytestmark = pytest.mark.gpu


def _hip():
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            lib = ctypes.CDLL(name)
            lib.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
            lib.hipMemGetInfo.restype = c_int
            return lib
        except OSError:
            continue
    pytest.skip("libamdhip64 not loadable")


def _free_bytes(hip):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _call(ctx, fn, x, dy, g, dx, dg, db, groups, n, acc=0):
    st = getattr(ctx.lib, fn)(ctx.handle, c_void_p(x.ptr), c_void_p(dy.ptr), None if g is None else c_void_p(g.ptr),
                              c_void_p(dx.ptr), None if dg is None else c_void_p(dg.ptr),
                              None if db is None else c_void_p(db.ptr), c_int64(groups), c_int64(n), c_float(1e-5),
                              c_int(acc))
    return st


def _case(ctx, groups, n, off, with_params=True, seed=0):
    """Inputs for one call (off: a float offset that breaks 16-byte alignment)
    and two sets of outputs, each starting from the same dgamma / dbeta."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(groups * n) * 1.5 + 0.3).astype(np.float32)
    dy = rng.standard_normal(groups * n).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    g0 = rng.standard_normal(n).astype(np.float32)
    b0 = rng.standard_normal(n).astype(np.float32)

    def dev(a):
        d = ctx.to_device(np.concatenate([np.zeros(off, np.float32), a]))
        return d, d.offset(off)
    keep = []
    xs, ys, gs = dev(x), dev(dy), dev(g)
    keep += [xs[0], ys[0], gs[0]]
    outs = []
    for _ in range(2):
        dx = ctx.empty(groups * n + off)
        dg, db = ctx.to_device(g0), ctx.to_device(b0)
        keep += [dx, dg, db]
        outs.append((dx.offset(off), dg if with_params else None, db if with_params else None))
    return xs[1], ys[1], gs[1], outs, keep


# (groups, n, offset): register-resident rows; 4-byte-column rows (odd
# width); the generic kernel (unaligned, wide); rows split over workgroups.
SHAPES = [((8192, 4096, 0), (2048, 4096, 0)),
          ((3000, 1023, 0), (700, 1023, 0)),
          ((300, 5003, 1), (40, 4099, 3)),
          ((40, 20000, 0), (17, 20000, 0))]


@pytest.mark.parametrize("first,second", SHAPES, ids=["rows_vec", "rows_scalar", "generic", "long_rows"])
@pytest.mark.parametrize("with_params", [True, False])
def test_noalloc_matches_the_allocating_entry_point(first, second, with_params):
    with M.Context(0) as ctx:
        for seed, (groups, n, off) in enumerate((first, second)):
            print(f"noalloc groups={groups} n={n} off={off} params={with_params}", flush=True)
            x, dy, g, outs, keep = _case(ctx, groups, n, off, with_params, seed)
            (dx0, dg0, db0), (dx1, dg1, db1) = outs
            assert _call(ctx, "mimir_layernorm_bwd", x, dy, g, dx0, dg0, db0, groups, n) == 0, ctx.lib.mimir_last_error(ctx.handle)
            st = _call(ctx, "mimir_layernorm_bwd_noalloc", x, dy, g, dx1, dg1, db1, groups, n)
            assert st == 0, ctx.lib.mimir_last_error(ctx.handle)
            ctx.sync()
            assert np.array_equal(dx0.numpy().view(np.uint32), dx1.numpy().view(np.uint32)), "dx"
            if with_params:
                assert np.array_equal(dg0.numpy().view(np.uint32), dg1.numpy().view(np.uint32)), "dgamma"
                assert np.array_equal(db0.numpy().view(np.uint32), db1.numpy().view(np.uint32)), "dbeta"
            for d in keep:
                d.free()


def test_noalloc_refuses_more_scratch_than_it_has():
    with M.Context(0) as ctx:
        groups, n = 1024, 16384  # 512 + 16 slots of 2 x 16384 floats: 69 MB
        x, dy, g, outs, keep = _case(ctx, groups, n, 0)
        dx, dg, db = outs[0]
        assert _call(ctx, "mimir_layernorm_bwd_noalloc", x, dy, g, dx, dg, db, groups, n) == M.EINVAL
        assert b"scratch" in ctx.lib.mimir_last_error(ctx.handle)
        for d in keep:
            d.free()


def test_noalloc_allocates_nothing():
    hip = _hip()
    groups, n = 4096, 4096
    with M.Context(0) as ctx:  # a fresh context: its own scratch has never grown
        x, dy, g, outs, keep = _case(ctx, groups, n, 0)
        dx, dg, db = outs[0]
        # Warm the context's stream and the kernels with a call that needs no
        # scratch (no dgamma), then measure around the no-allocation calls.
        assert _call(ctx, "mimir_layernorm_bwd", x, dy, g, dx, None, None, groups, n) == 0
        ctx.sync()
        before = _free_bytes(hip)
        for _ in range(3):
            assert _call(ctx, "mimir_layernorm_bwd_noalloc", x, dy, g, dx, dg, db, groups, n) == 0
        ctx.sync()
        assert _free_bytes(hip) >= before
        for d in keep:
            d.free()


def test_noalloc_array_has_one_holder_per_gpu():
    """The first context to call the entry point holds the GPU's array; a
    second context's call returns EBUSY and launches nothing (its outputs
    keep their bits); once the holder is destroyed the second context takes
    the array and matches the allocating entry point."""
    groups, n = 512, 4096
    a = M.Context(0)
    b = M.Context(0)
    try:
        x, dy, g, outs, keep = _case(a, groups, n, 0)
        dx, dg, db = outs[0]
        assert _call(a, "mimir_layernorm_bwd_noalloc", x, dy, g, dx, dg, db, groups, n) == 0
        a.sync()
        for d in keep:
            d.free()
        xb, dyb, gb, outsb, keepb = _case(b, groups, n, 0, seed=1)
        (dx0, dg0, db0), (dx1, dg1, db1) = outsb
        before = (dx1.numpy().copy(), dg1.numpy().copy(), db1.numpy().copy())
        assert _call(b, "mimir_layernorm_bwd_noalloc", xb, dyb, gb, dx1, dg1, db1, groups, n) == M.EBUSY
        assert b"another context" in b.lib.mimir_last_error(b.handle)
        b.sync()
        for got, was in zip((dx1.numpy(), dg1.numpy(), db1.numpy()), before):
            assert np.array_equal(got.view(np.uint32), was.view(np.uint32)), "a refused call wrote"
        a.close()
        a = None
        assert _call(b, "mimir_layernorm_bwd", xb, dyb, gb, dx0, dg0, db0, groups, n) == 0
        assert _call(b, "mimir_layernorm_bwd_noalloc", xb, dyb, gb, dx1, dg1, db1, groups, n) == 0
        b.sync()
        for u, v in ((dx0, dx1), (dg0, dg1), (db0, db1)):
            assert np.array_equal(u.numpy().view(np.uint32), v.numpy().view(np.uint32))
        for d in keepb:
            d.free()
    finally:
        if a is not None:
            a.close()
        b.close()
