"""Golden fixtures written by tests/golden/make_golden.py from the reference's
own op functions (compiled in place).  The CPU oracle must reproduce them
(CPU tests) and so must the HIP path (gpu tests): this pins both to the
reference where the reference tree is absent."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
from _parity import assert_bitexact, assert_close
from mimir_hip import datagen as G

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = json.load(open(os.path.join(GOLD, "MANIFEST.json")))


def gold(name):
    with np.load(os.path.join(GOLD, name + ".npz")) as z:
        return {k: z[k] for k in z.files}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_manifest_hashes_and_regenerated_inputs():
    for name, entry in MANIFEST.items():
        if "file" in entry:  # a fixture kept as the file the reference wrote
            path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"{name}.safetensors")
            data = open(path, "rb").read()
            assert len(data) == entry["file"]["bytes"]
            assert hashlib.sha256(data).hexdigest() == entry["file"]["sha256"], f"{name} changed"
            continue
        g = gold(name)
        for k, meta in entry["arrays"].items():
            assert sha(g[k]) == meta["sha256"], f"{name}.{k} changed"
    x, gm, b, _ = G.cfg0_layernorm()
    assert sha(x) == MANIFEST["layernorm_cfg0"]["regenerated_inputs"]["datagen.cfg0_layernorm"]["x"]
    x, r, w, _ = G.cfg1_add_rmsnorm(rows=8)
    h = MANIFEST["add_rmsnorm_cfg1_rows8"]["regenerated_inputs"]["datagen.cfg1_add_rmsnorm(rows=8)"]
    assert (sha(x), sha(r), sha(w)) == (h["x"], h["residual"], h["w"])
    s = G.cfg2_softmax(batch=1, heads=1)
    assert sha(s.reshape(1024, 1024)) == \
        MANIFEST["softmax_cfg2_rows"]["regenerated_inputs"]["datagen.cfg2_softmax(batch=1, heads=1)"]["scores"]


# ---------------------------------------------------------------------------
# The checks, written once over an "implementation" object so the CPU oracle
# and the HIP path run the same assertions.
# ---------------------------------------------------------------------------

class OracleImpl:
    layernorm = staticmethod(lambda x, n, g, b, eps: O.layernorm(x, n, g, b, eps))
    rmsnorm_rows = staticmethod(lambda x, w, eps: O.rmsnorm_rows(x, w, eps))
    add_rmsnorm = staticmethod(lambda x, r, w, eps: O.add_rmsnorm(x, r, w, eps))
    rmsnorm_whole = staticmethod(lambda x, w, eps: O.rmsnorm_whole(x, w, eps))
    softmax = staticmethod(lambda x, mode: O.softmax_rows(x, mode))
    gelu = staticmethod(O.gelu)
    silu = staticmethod(O.silu)
    add = staticmethod(O.add)
    mul = staticmethod(O.mul)


class HipImpl:
    def __init__(self, ctx):
        self.ctx = ctx

    def _run(self, fn, ins, out_n):
        c = self.ctx
        d = [None if a is None else c.to_device(a) for a in ins]
        y = c.empty(out_n)
        try:
            fn(*d, y)
            return y.numpy()
        finally:
            for a in d:
                if a is not None:
                    a.free()
            y.free()

    def layernorm(self, x, n, g, b, eps):
        x = x.ravel()
        return self._run(lambda dx, dg, db, y: self.ctx.layernorm(dx, dg, db, y, x.size // n if n else 1,
                                                                  n or x.size, eps), [x, g, b], x.size)

    def rmsnorm_rows(self, x, w, eps):
        rows, cols = x.shape
        return self._run(lambda dx, dw, y: self.ctx.rmsnorm(dx, dw, cols, y, rows, cols, eps), [x, w],
                         x.size).reshape(x.shape)

    def add_rmsnorm(self, x, r, w, eps):
        rows, cols = x.shape
        c = self.ctx
        dx, dr, dw = c.to_device(x), c.to_device(r), c.to_device(w)
        dh, dy = c.empty(x.shape), c.empty(x.shape)
        c.add_rmsnorm(dx, dr, dh, dw, dy, rows, cols, eps)
        out = dy.numpy(), dh.numpy()
        for a in (dx, dr, dw, dh, dy):
            a.free()
        return out

    def rmsnorm_whole(self, x, w, eps):
        return self._run(lambda dx, dw, y: self.ctx.rmsnorm(dx, dw, 0 if w is None else w.size, y, 1, x.size,
                                                            eps), [x, w], x.size)

    def softmax(self, x, mode):
        x2 = x.reshape(1, -1) if x.ndim == 1 else x
        return self._run(lambda dx, y: self.ctx.softmax(dx, y, x2.shape[0], x2.shape[1], mode), [x2],
                         x2.size).reshape(x2.shape)

    def gelu(self, x):
        return self._run(lambda dx, y: self.ctx.gelu(dx, y, x.size), [x], x.size)

    def silu(self, x):
        return self._run(lambda dx, y: self.ctx.silu(dx, y, x.size), [x], x.size)

    def add(self, a, b):
        return self._run(lambda da, db, y: self.ctx.add(da, a.size, db, b.size, y), [a, b], max(a.size, b.size))

    def mul(self, a, b):
        return self._run(lambda da, db, y: self.ctx.mul(da, a.size, db, b.size, y), [a, b], a.size)


def check_all(impl):
    g = gold("layernorm_cfg0")
    x, gm, b, eps = G.cfg0_layernorm()
    assert_close(impl.layernorm(x, 512, gm, b, eps).reshape(x.shape), g["y"], "layernorm cfg0")

    g = gold("layernorm_variants")
    n = 33
    gam, bet = g["params33"][:n], g["params33"][n:]
    assert_close(impl.layernorm(g["x33"], n, gam, bet, 1e-5), g["y33_gb"], "LN gamma+beta")
    assert_close(impl.layernorm(g["x33"], n, gam, None, 1e-5), g["y33_g"], "LN gamma only")
    assert_close(impl.layernorm(g["x33"], n, None, None, 1e-5), g["y33_none"], "LN no affine")
    assert_close(impl.layernorm(g["xw"], 0, g["pw"][:300], g["pw"][300:], 1e-5), g["yw"], "LN whole vector")

    g = gold("add_rmsnorm_cfg1_rows8")
    x, r, w, eps = G.cfg1_add_rmsnorm(rows=8)
    y, h = impl.add_rmsnorm(x, r, w, eps)
    assert_bitexact(h, g["h"], "residual'")
    assert_close(y, g["y"], "add+rmsnorm")
    assert_close(impl.rmsnorm_rows(g["h"], w, eps), g["y"], "rmsnorm rows")

    g = gold("rmsnorm_layer")
    assert_close(impl.rmsnorm_whole(g["x"], g["w"], 1e-5), g["y"], "rmsnorm layer")
    assert_close(impl.rmsnorm_whole(g["x"], None, 1e-5), g["y_noaffine"], "rmsnorm layer, no affine")

    g = gold("softmax_cfg2_rows")
    s = G.cfg2_softmax(batch=1, heads=1).reshape(1024, 1024)[992:]
    assert_close(impl.softmax(s, O.SOFTMAX_DIV_EPS), g["y"], "softmax cfg2 rows")

    g = gold("softmax_layer")
    assert_close(impl.softmax(g["x"], O.SOFTMAX_MUL_INV)[0], g["y"], "Softmax layer")
    assert_close(impl.softmax(g["x"], O.SOFTMAX_LOG)[0], g["y_log"], "LogSoftmax layer")
    assert_close(impl.softmax(g["special"], O.SOFTMAX_DIV_EPS), g["special_y"], "special rows")

    g = gold("activations")
    assert_close(impl.gelu(g["x"]), g["gelu"], "gelu")
    assert_close(impl.silu(g["x"]), g["silu"], "silu")

    g = gold("add_mul")
    assert_bitexact(impl.add(g["a"], g["b"]), g["add"], "add specials")
    assert_bitexact(impl.mul(g["a"], g["b"]), g["mul"], "mul specials")
    assert_bitexact(impl.add(g["small"], g["big"]), g["add_repeat"], "add repeat")
    assert_bitexact(impl.add(g["big"], g["small"][:1]), g["add_scalar"], "add scalar")


def test_oracle_reproduces_reference_fixtures():
    check_all(OracleImpl())


@pytest.mark.gpu
def test_hip_reproduces_reference_fixtures(ctx):
    check_all(HipImpl(ctx))
