"""Minimal safetensors reader that returns raw little-endian arrays (bf16 as uint16).

The format is data only (an 8-byte header length, a JSON header, then the tensors), so
reading it executes nothing from the file.
"""
import json
import struct

import numpy as np

_DT = {"BF16": np.uint16, "F16": np.uint16, "F32": np.float32, "F64": np.float64,
       "I32": np.int32, "I8": np.int8, "U8": np.uint8, "I64": np.int64, "U32": np.uint32}


def load(path):
    with open(path, "rb") as f:
        blob = f.read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        b, e = info["data_offsets"]
        arr = np.frombuffer(blob[base + b:base + e], dtype=_DT[info["dtype"]])
        out[name] = (info["dtype"], arr.reshape(info["shape"]))
    return out
