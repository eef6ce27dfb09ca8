"""Pin the C restatement (oracle/) against the reference's own op functions,
compiled in place into oracle/_ref/libmimir_ref.so, on seeded inputs and on
the edge cases the reference's semantics define.  Skipped where that library
was not built (no reference tree)."""
import numpy as np
import pytest

import oracle as O
from _parity import assert_bitexact, assert_close

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")

rng = np.random.default_rng(20261201)

SPECIALS = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-40, 3.0, -3.0, 9.0, -9.0, 20.0, -20.0,
                     88.0, -88.0, 100.0, -100.0, np.inf, -np.inf, np.nan], np.float32)


@pytest.mark.parametrize("groups,n", [(256, 512), (7, 4096), (3, 1), (1, 33), (5, 100)])
@pytest.mark.parametrize("affine,use_bias", [(True, True), (True, False), (False, False)])
def test_layernorm(groups, n, affine, use_bias):
    x = rng.standard_normal(groups * n, dtype=np.float32) * 2 + 0.5
    g = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    params = np.concatenate([g, b]) if affine else None
    ref = O.ref_layernorm(x, n, params, affine, use_bias, 1e-5)
    got = O.layernorm(x, n, g if affine else None, b if (affine and use_bias) else None, 1e-5)
    assert_close(got, ref, "layernorm")


def test_layernorm_whole_vector_group():
    # in_features = 0 -> one group over all N (LayerOps.hpp:276)
    x = rng.standard_normal(3000, dtype=np.float32)
    ref = O.ref_layernorm(x, 0, np.ones(6000, np.float32), True, True, 1e-5)
    assert_close(O.layernorm(x, 0, np.ones(3000, np.float32), np.ones(3000, np.float32), 1e-5), ref)


@pytest.mark.parametrize("n,wn", [(2, 2), (4096, 4096), (1000, 17), (513, 0)])
def test_rmsnorm_whole(n, wn):
    x = rng.standard_normal(n, dtype=np.float32)
    w = (1 + 0.02 * rng.standard_normal(wn)).astype(np.float32)
    ref = O.ref_rms_norm_forward(x, w, True, 1e-6)
    assert_close(O.rmsnorm_whole(x, w if wn else None, 1e-6), ref)


@pytest.mark.parametrize("rows,cols", [(16, 4096), (9, 1), (4, 37)])
def test_rmsnorm_rows(rows, cols):
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    ref = O.ref_rms_norm_rows(x, g, 1e-6)
    assert_close(O.rmsnorm_rows(x, g, 1e-6), ref)


def test_add_rmsnorm_is_add_then_rmsnorm():
    x = rng.standard_normal((8, 4096), dtype=np.float32)
    r = rng.standard_normal((8, 4096), dtype=np.float32)
    g = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    h_ref = O.ref_add(x, r).reshape(8, 4096)
    y_ref = O.ref_rms_norm_rows(h_ref, g, 1e-6)
    y, h = O.add_rmsnorm(x, r, g, 1e-6)
    assert_bitexact(h, h_ref, "residual")
    assert_close(y, y_ref, "y")


@pytest.mark.parametrize("na,nb", [(1000, 1000), (12, 1), (1, 12), (4096 * 3, 4096), (10, 30), (7, 7)])
def test_add_broadcast_bitexact(na, nb):
    a = rng.standard_normal(na, dtype=np.float32)
    b = rng.standard_normal(nb, dtype=np.float32)
    assert_bitexact(O.add(a, b), O.ref_add(a, b))


def test_add_mul_specials_bitexact():
    a = np.tile(SPECIALS, len(SPECIALS))
    b = np.repeat(SPECIALS, len(SPECIALS))
    assert_bitexact(O.add(a, b), O.ref_add(a, b))
    assert_bitexact(O.mul(a, b), O.ref_mul(a, b))


def test_softmax_rows_causal():
    s = (3 * rng.standard_normal((64, 1024))).astype(np.float32)
    s[np.triu(np.ones((64, 1024), bool), 1)] = -np.inf
    assert_close(O.softmax_rows(s, O.SOFTMAX_DIV_EPS), O.ref_softmax_inplace(s))


def test_softmax_rows_specials():
    s = np.stack([np.full(8, -np.inf, np.float32),  # all -inf -> NaN in both
                  np.array([np.nan, 1, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([1, np.nan, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([np.inf, 1, 2, 3, 4, 5, 6, 7], np.float32),
                  np.array([1e30, -1e30, 0, 0, 0, 0, 0, 0], np.float32),
                  np.zeros(8, np.float32)])
    assert_close(O.softmax_rows(s, O.SOFTMAX_DIV_EPS), O.ref_softmax_inplace(s))


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("n", [1, 2, 1000, 70000])
def test_softmax_layer_whole_vector(n, log):
    x = (3 * rng.standard_normal(n)).astype(np.float32)
    mode = O.SOFTMAX_LOG if log else O.SOFTMAX_MUL_INV
    assert_close(O.softmax_rows(x, mode)[0], O.ref_softmax_forward(x, log))


def test_gelu_silu_dense_grid():
    x = np.concatenate([np.linspace(-12, 12, 200001, dtype=np.float32), SPECIALS,
                        rng.standard_normal(100000, dtype=np.float32)])
    assert_close(O.gelu(x), O.ref_gelu(x), "gelu")
    assert_close(O.silu(x), O.ref_silu(x), "silu")


def test_gated_products_are_the_reference_compositions():
    """oracle_gelu_mul and oracle_silu_mul restate the two reference calls a
    gated product is made of: multiply_forward(gelu_forward(gate), up) and
    multiply_forward(silu_forward(gate), up) (LayerOps.hpp:556-568, 570-581,
    205-230), on the dense grid, the specials and normals."""
    g = np.concatenate([np.linspace(-12, 12, 200001, dtype=np.float32), SPECIALS,
                        rng.standard_normal(100000, dtype=np.float32)])
    u = np.concatenate([rng.standard_normal(200001).astype(np.float32) * 3, SPECIALS[::-1],
                        rng.standard_normal(100000, dtype=np.float32)])
    assert_close(O.gelu_mul(g, u), O.ref_mul(O.ref_gelu(g), u), "gelu*up")
    assert_close(O.silu_mul(g, u), O.ref_mul(O.ref_silu(g), u), "silu*up")
    # The gate and the up operand are not interchangeable.
    with pytest.raises(AssertionError):
        assert_close(O.gelu_mul(u, g), O.ref_mul(O.ref_gelu(g), u))
