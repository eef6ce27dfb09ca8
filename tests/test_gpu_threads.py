"""Contexts on concurrent host threads (the threading contract of
include/mimir_hip.h: one context per host thread).  Each thread owns a
context, hence its own stream and scratch buffer, and runs the ops that use
the scratch (long-row softmax partials, the LayerNorm backward's dgamma/dbeta
slots, the Embedding backward's sort buffers) next to a row op, repeatedly
and at the same time as the others.  Every kernel here is deterministic, so
each result must equal, bit for bit, what one thread alone computed first.
ctypes drops the GIL for every library call, so the threads really overlap."""
import threading

import numpy as np
import pytest

import mimir_hip as M

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 6


def _inputs(seed):
    rng = np.random.default_rng(seed)
    rows, cols = 512, 1024
    return dict(
        x=rng.standard_normal((rows, cols), dtype=np.float32),
        r=rng.standard_normal((rows, cols), dtype=np.float32),
        w=(1 + 0.1 * rng.standard_normal(cols)).astype(np.float32),
        dy=rng.standard_normal((rows, cols), dtype=np.float32),
        long=(3 * rng.standard_normal(1 << 20)).astype(np.float32),
        ids=rng.integers(-1, 300, 4096).astype(np.int32),
        edy=rng.standard_normal((4096, 64), dtype=np.float32),
    )


def _run(ctx, d):
    """The op sequence; returns host copies of every output."""
    rows, cols = d["x"].shape
    x, r, w, dy = (ctx.to_device(d[k]) for k in ("x", "r", "w", "dy"))
    y, r_out, dx = ctx.empty((rows, cols)), ctx.empty((rows, cols)), ctx.empty((rows, cols))
    dg, db = ctx.to_device(np.zeros(cols, np.float32)), ctx.to_device(np.zeros(cols, np.float32))
    lx, ly = ctx.to_device(d["long"]), ctx.empty(d["long"].size)
    ids, edy = ctx.to_device(d["ids"]), ctx.to_device(d["edy"])
    table = ctx.to_device(np.zeros((300, 64), np.float32))
    bufs = [x, r, w, dy, y, r_out, dx, dg, db, lx, ly, ids, edy, table]
    try:
        ctx.add_rmsnorm(x, r, r_out, w, y, rows, cols, 1e-6)
        ctx.softmax(lx, ly, 1, d["long"].size, M.SOFTMAX_MUL_INV)
        ctx.layernorm_bwd(x, dy, w, dx, dg, db, rows, cols, 1e-5)
        ctx.embedding_bwd(ids, d["ids"].size, edy, table, 300 * 64, 300, 64, -1)
        return [b.numpy() for b in (y, r_out, ly, dx, dg, db, table)]
    finally:
        for b in bufs:
            b.free()


def test_contexts_on_concurrent_threads_match_one_thread():
    inputs = [_inputs(100 + t) for t in range(THREADS)]
    with M.Context(0) as c:
        want = [_run(c, inputs[t]) for t in range(THREADS)]
    errors = []
    start = threading.Barrier(THREADS)

    def worker(t):
        try:
            with M.Context(0) as c:
                start.wait()
                for k in range(ROUNDS):
                    got = _run(c, inputs[t])
                    for i, (a, b) in enumerate(zip(got, want[t])):
                        if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
                            errors.append(f"thread {t} round {k} output {i}: bits differ")
        except Exception as e:  # reported below, with the thread that raised it
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=90)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors[:5]
