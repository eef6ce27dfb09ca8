"""SafeTensors reads straight into device memory (mimir_safetensors_read /
_load_layers) against the checkpoint the reference's own writer produced
(tests/golden/ref_checkpoint.safetensors) and files written here; every
read is checked bit for bit."""
import os

import numpy as np
import pytest

import mimir_hip as M
from _graphs import checkpoint_layers
from _parity import assert_bitexact
from _safetensors_files import write

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_checkpoint.safetensors")


def _zeroed(layers):
    return [dict(L, weights=np.zeros_like(L["weights"])) if L.get("weights") is not None else dict(L) for L in layers]


def test_loads_the_reference_checkpoint_into_device_weights(ctx):
    want = checkpoint_layers()
    g = M.DeviceGraph(ctx, _zeroed(want))
    try:
        with M.SafeTensors(ctx, GOLD) as f:
            f.load_graph(g, strict=True)
        for L, d in zip(want, g.weights):
            if L.get("weights") is None:
                assert d is None
                continue
            assert_bitexact(d.numpy(), L["weights"], f"{L['name']} weights")
    finally:
        g.close()


def test_strict_missing_and_size_mismatch(ctx, tmp_path):
    p = tmp_path / "partial.safetensors"
    write(p, {"ln/weights": np.arange(16, dtype=np.float32)})
    layers = [dict(name="ln", type="LayerNorm", in_features=8, weights=np.zeros(16, np.float32)),
              dict(name="other", type="RMSNorm", weights=np.full(4, 7.0, np.float32))]
    g = M.DeviceGraph(ctx, layers)
    try:
        with M.SafeTensors(ctx, p) as f:
            with pytest.raises(M.MimirError, match="Missing tensor in strict mode: other/weights"):
                f.load_graph(g, strict=True)
            f.load_graph(g, strict=False)  # the missing tensor is skipped
        assert_bitexact(g.weights[0].numpy(), np.arange(16, dtype=np.float32), "ln")
        assert_bitexact(g.weights[1].numpy(), np.full(4, 7.0, np.float32), "other untouched")
    finally:
        g.close()
    bad = [dict(name="ln", type="LayerNorm", in_features=4, weights=np.zeros(8, np.float32))]
    g = M.DeviceGraph(ctx, bad)
    try:
        with M.SafeTensors(ctx, p) as f:
            with pytest.raises(M.MimirError, match="Size mismatch for ln/weights: expected 16 got 8"):
                f.load_graph(g)
    finally:
        g.close()


@pytest.mark.parametrize("nbytes", [4, 4 * 1000003, (8 << 20) + 5, (8 << 20) * 3, (8 << 20) * 4,
                                    (8 << 20) * 4 + 12, (8 << 20) * 7 + 1])
def test_read_multi_chunk_bitexact(ctx, tmp_path, nbytes):
    # Reads cross the 8 MiB staging chunks: one or two chunks (one reader),
    # three and more (two readers, pairs of chunks over four buffers), a pair
    # whose second chunk is missing, ragged tails.
    rng = np.random.default_rng(nbytes)
    if nbytes % 4:
        a = rng.integers(0, 256, nbytes, dtype=np.uint8)
    else:
        a = rng.standard_normal(nbytes // 4).astype(np.float32)
        a.view(np.uint32)[:3] = [0x7FC00001, 0x80000000, 0x00000001][:a.size]  # NaN payload, -0, denormal
    p = tmp_path / "big.safetensors"
    write(p, {"pad": np.arange(3, dtype=np.uint8), "t": a})  # "t" starts at an unaligned offset
    dst = ctx.empty(((nbytes + 3) // 4,))
    try:
        with M.SafeTensors(ctx, p) as f:
            f.read("t", dst)
            got = dst.numpy().view(np.uint8)[:nbytes]
            assert np.array_equal(got, a.view(np.uint8)), "bytes differ"
            if nbytes > 8:
                small = ctx.empty((nbytes // 8,))
                try:
                    with pytest.raises(M.MimirError, match="Buffer too small for tensor: t"):
                        f.read("t", small)
                finally:
                    small.free()
            with pytest.raises(M.MimirError, match="No tensor named nope"):
                f.read("nope", dst)
    finally:
        dst.free()
