"""The reference's own known-answer tests for this path, re-expressed against
the CPU oracle (brit45/mimir-framework Tests/, file:line per test).  Same
inputs, same expected values, same absolute tolerances as the reference."""
import math

import numpy as np
import pytest

import oracle as O


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def test_activations_kat():
    # Tests/test_layers_all_types.cpp:203-239
    x = np.array([-1.0, 0.0, 1.0], np.float32)
    silu = O.silu(x)
    assert abs(silu[1] - 0.0) <= 1e-6
    assert abs(silu[2] - 1.0 * sigmoid(1.0)) <= 1e-6
    gelu = O.gelu(np.array([0.0, 1.0], np.float32))
    assert abs(gelu[0] - 0.0) <= 1e-6
    assert abs(gelu[1] - 0.8413) <= 2e-3


def test_softmax_kat():
    # Tests/test_layers_all_types.cpp:242-262 (Softmax / LogSoftmax layers, whole vector)
    sm = O.softmax_rows(np.array([0.0, 0.0], np.float32), O.SOFTMAX_MUL_INV)[0]
    assert abs(sm[0] - 0.5) <= 1e-6 and abs(sm[1] - 0.5) <= 1e-6
    lsm = O.softmax_rows(np.array([0.0, 0.0], np.float32), O.SOFTMAX_LOG)[0]
    ln2 = math.log(2.0)
    assert abs(lsm[0] + ln2) <= 1e-5 and abs(lsm[1] + ln2) <= 1e-5


def test_layernorm_kat():
    # Tests/test_layers_all_types.cpp:265-301: in_features=4, gamma=1, beta=0, eps=1e-6
    out = O.layernorm(np.array([1, 2, 3, 4], np.float32), 4, np.ones(4, np.float32),
                      np.zeros(4, np.float32), 1e-6)
    assert np.all(np.isfinite(out))
    mean = np.float32(0.0)
    for v in out:
        mean += v
    mean /= np.float32(4.0)
    var = np.float32(0.0)
    for v in out:
        var += (v - mean) * (v - mean)
    var /= np.float32(4.0)
    assert abs(mean) <= 1e-5
    assert abs(var - 1.0) <= 1e-4


def test_rmsnorm_kat():
    # Tests/test_layers_all_types.cpp:304-323: whole-vector layer, w=1, eps=1e-6
    out = O.rmsnorm_whole(np.array([3.0, 4.0], np.float32), np.ones(2, np.float32), 1e-6)
    rms = math.sqrt((9.0 + 16.0) / 2.0 + 1e-6)
    assert abs(out[0] - 3.0 / rms) <= 1e-5
    assert abs(out[1] - 4.0 / rms) <= 1e-5


def test_elementwise_kat():
    # Tests/test_layers_all_types.cpp:392-422 (Add, Multiply)
    x = np.array([1, 2, 3], np.float32)
    y = np.array([4, 5, 6], np.float32)
    np.testing.assert_allclose(O.add(x, y), [5, 7, 9], atol=1e-6)
    np.testing.assert_allclose(O.mul(x, y), [4, 10, 18], atol=1e-6)


def test_named_routing_kat():
    # Tests/test_layers_named_routing.cpp:14-15,39-51: sum = a + b; x = sum * c -> {8, 12}
    s = O.add(np.array([1, 2], np.float32), np.array([3, 4], np.float32))
    x = O.mul(s, np.array([2, 2], np.float32))
    np.testing.assert_allclose(x, [8, 12], atol=1e-6)


def test_residual_merge_kat():
    # Tests/test_runtime_residual_merge.cpp:26-29,46-47: x*scale + skip = {3, 8}
    x = np.array([1, 2], np.float32)
    main = O.mul(x, np.array([2, 3], np.float32))
    np.testing.assert_allclose(O.add(main, x), [3, 8], atol=1e-6)


def test_embedding_float_ids_kat():
    # Tests/test_layers_all_types.cpp:509-533: vocab=3, dim=2, ids {1.0, 2.0}
    table = np.array([0, 0, 1, 10, 2, 20], np.float32)
    out = O.embedding(np.array([1.0, 2.0], np.float32), table, 3, 2, -1).ravel()
    np.testing.assert_allclose(out, [1, 10, 2, 20], atol=1e-6)


def test_embedding_int_ids_kat():
    # Tests/test_runtime_embedding_int_inputs.cpp:8-18,31,45-66: table[id][d] = id*10 + d,
    # padding_idx = 0, ids {1, 0, 2}
    vocab, dim = 4, 4
    table = np.array([[i * 10 + d for d in range(dim)] for i in range(vocab)], np.float32)
    out = O.embedding(np.array([1, 0, 2], np.int32), table, vocab, dim, 0)
    np.testing.assert_allclose(out[0], [10, 11, 12, 13], atol=1e-6)
    np.testing.assert_allclose(out[1], [0, 0, 0, 0], atol=1e-6)
    np.testing.assert_allclose(out[2], [20, 21, 22, 23], atol=1e-6)
    # :68-74: missing ids -> seq_len pad ids -> all zeros
    out = O.embedding(np.zeros(5, np.int32), table, vocab, dim, 0)
    assert out.shape == (5, dim) and not out.any()


def test_reference_error_cases():
    # LayerOps.hpp:150-152 (empty add), :191 (non-broadcastable), :209-211 (mul sizes),
    # :276-279 (LN group size), Model.cpp:1181-1182 (embedding table too small)
    a = np.ones(3, np.float32)
    with pytest.raises(O.OracleError):
        O.add(a, np.zeros(0, np.float32))
    with pytest.raises(O.OracleError):
        O.add(np.ones(5, np.float32), np.ones(3, np.float32))
    with pytest.raises(O.OracleError):
        O.mul(a, np.ones(4, np.float32))
    with pytest.raises(O.OracleError):
        O.layernorm(np.ones(6, np.float32), 4)
    with pytest.raises(O.OracleError):
        O.embedding(np.array([0], np.int32), np.ones(5, np.float32), 3, 2, -1)
