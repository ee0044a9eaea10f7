"""Writer of GPQ8 weight files for the tests, from the layout documented in
include/lal_gpq8.h (tools/server/qwen7b_server.c:497-571 reads the same
record sequence): "GPQ8", int32 count, then per tensor int32 key_len, key,
int32 ndim, int32 shape[ndim], uint8 qtype, uint64 data_len, data, int32
n_scale, float scale[n_scale]."""
import struct

import numpy as np

F32, Q8, Q4_0, Q8_0 = 0, 1, 2, 3


def record(key, arr, qtype, scale=None, shape=None):
    k = key.encode()
    shape = list(arr.shape if shape is None else shape)
    data = np.ascontiguousarray(arr).tobytes()
    out = struct.pack("<i", len(k)) + k + struct.pack("<i", len(shape))
    out += b"".join(struct.pack("<i", d) for d in shape)
    out += struct.pack("<BQ", qtype, len(data)) + data
    sc = b"" if scale is None else np.ascontiguousarray(scale, np.float32).tobytes()
    out += struct.pack("<i", 0 if scale is None else len(scale)) + sc
    return out


def image(records):
    return b"GPQ8" + struct.pack("<i", len(records)) + b"".join(records)


def write(path, records):
    with open(path, "wb") as f:
        f.write(image(records))
    return path
