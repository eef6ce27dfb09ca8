"""Writers of SafeTensors files for the tests: valid files in the format the
reference writes (SafeTensorsWriter.cpp: 8-byte little-endian header
length, JSON header, data section) and malformed ones."""
import json
import struct

import numpy as np

DTYPES = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int32): "I32",
          np.dtype(np.int16): "I16", np.dtype(np.uint16): "U16", np.dtype(np.uint8): "U8"}


def write(path, tensors, metadata=None, header_override=None, raw_len=None, truncate=None):
    """tensors: {name: ndarray}.  header_override(header dict) may edit the
    header before it is written; raw_len forces the length field; truncate
    cuts the file to that many bytes."""
    header = {}
    off = 0
    blobs = []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        header[name] = {"dtype": DTYPES[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
        blobs.append(a.tobytes())
    if metadata is not None:
        header["__metadata__"] = metadata
    if header_override is not None:
        header_override(header)
    text = json.dumps(header).encode()
    data = struct.pack("<Q", len(text) if raw_len is None else raw_len) + text + b"".join(blobs)
    if truncate is not None:
        data = data[:truncate]
    with open(path, "wb") as f:
        f.write(data)


def cases(tmp):
    """(name, path, accepted, message substring) for the header checks of
    SafeTensorsReader::parse_header (SafeTensorsReader.cpp:52-166)."""
    w = np.arange(8, dtype=np.float32)
    out = []

    def case(name, accepted, msg, **kw):
        p = tmp / f"{name}.safetensors"
        write(p, kw.pop("tensors", {"ln/weights": w}), **kw)
        out.append((name, p, accepted, msg))

    case("valid", True, "", metadata={"format": "safetensors", "total_size": 32, "nested": {"a": [1, 2.5, None]}})
    case("valid_mixed_dtypes", True, "",
         tensors={"ln/weights": w, "ids": np.arange(5, dtype=np.int32), "blob": np.frombuffer(b"{}\n", np.uint8),
                  "half": np.ones(3, np.float16)})
    case("zero_header_length", False, "Invalid header length", raw_len=0)
    case("huge_header_length", False, "Invalid header length", raw_len=(100 << 20) + 1)
    case("truncated_header", False, "", truncate=20)
    case("not_json", False, "Header parse error",
         header_override=lambda h: h.__setitem__("ln/weights", {"dtype": "F32"}) or None, raw_len=None)
    out.pop()  # replaced below by a genuinely malformed header
    p = tmp / "not_json.safetensors"
    text = b'{"ln/weights": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]'  # unterminated
    open(p, "wb").write(struct.pack("<Q", len(text)) + text + w.tobytes())
    out.append(("not_json", p, False, "Header parse error"))
    case("missing_dtype", False, "Missing dtype for tensor: ln/weights",
         header_override=lambda h: h["ln/weights"].pop("dtype"))
    case("unknown_dtype", False, "Unknown dtype string: BF16",
         header_override=lambda h: h["ln/weights"].__setitem__("dtype", "BF16"))
    case("lowercase_dtype", True, "", header_override=lambda h: h["ln/weights"].__setitem__("dtype", "float32"))
    case("missing_shape", False, "Missing shape for tensor: ln/weights",
         header_override=lambda h: h["ln/weights"].pop("shape"))
    case("missing_offsets", False, "Missing data_offsets for tensor: ln/weights",
         header_override=lambda h: h["ln/weights"].pop("data_offsets"))
    case("offsets_three", False, "Invalid data_offsets for tensor: ln/weights",
         header_override=lambda h: h["ln/weights"].__setitem__("data_offsets", [0, 16, 32]))
    case("size_mismatch", False, "Size mismatch for tensor: ln/weights",
         header_override=lambda h: h["ln/weights"].__setitem__("shape", [7]))
    return out
