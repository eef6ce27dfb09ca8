"""SafeTensors header parsing of libmimir_hip (mimir_safetensors_open with no
device context, so these run without a GPU) against the reference's
SafeTensorsReader (compiled in place, oracle/_ref) on the same files, and on
the checkpoint the reference's own writer produced (golden fixture)."""
import json
import os
import struct

import numpy as np
import pytest

import mimir_hip as M
import model_ref as MR
from _safetensors_files import cases

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "ref_checkpoint.safetensors")

needs_ref = pytest.mark.skipif(not MR.available(), reason="oracle/_ref/libmimir_ref_model.so not built")


def _open(path):
    return M.SafeTensors(None, path)


def _header(path):
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<Q", raw[:8])
    return json.loads(raw[8:8 + n])


def test_reads_the_reference_writers_checkpoint():
    h = _header(GOLD)
    with _open(GOLD) as f:
        ents = f.entries()
    want = {k: v for k, v in h.items() if k != "__metadata__"}
    assert set(ents) == set(want)
    for k, (dt, shape, nb) in ents.items():
        assert dt == want[k]["dtype"] and list(shape) == want[k]["shape"]
        b, e = want[k]["data_offsets"]
        assert nb == e - b
    assert ents["ln/weights"] == ("F32", (16,), 64)


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    return cases(tmp_path_factory.mktemp("st"))


def test_header_checks(files):
    for name, path, accepted, msg in files:
        if accepted:
            with _open(path) as f:
                assert f.entries(), name
            continue
        with pytest.raises(M.MimirError) as ei:
            _open(path)
        assert msg in str(ei.value) or not msg, f"{name}: {ei.value}"


@needs_ref
def test_header_checks_agree_with_reference(files):
    # The reference's loader on a model with one 8-float weight block named
    # "ln": it parses the header first, so each case is accepted or rejected
    # there exactly as here.
    layers = [dict(name="ln", type="LayerNorm", in_features=4, weights=np.zeros(8, np.float32))]
    for name, path, accepted, msg in files:
        try:
            MR.load_safetensors(layers, path, strict=False)
            ref_ok, ref_msg = True, ""
        except MR.RefModelError as e:
            ref_ok, ref_msg = False, str(e)
        assert ref_ok == accepted, f"{name}: reference accepted={ref_ok} ({ref_msg})"
        if msg:
            assert msg in ref_msg, f"{name}: reference says {ref_msg!r}"
