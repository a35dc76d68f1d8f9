"""Reader for the reference's SURGEOPS fixture container (reference
tests/fixture.h:1-112): "SURGEOPS", u32 version 1, u32 record count, then
36-byte directory entries {name_off, dtype, n_dims, dims[4], data_off,
nbytes} (u32 each); dtype 0 = f32, 1 = u16, 2 = u8. The fixture files under
tests/golden/ are the reference's own data files, copied verbatim."""
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_DT = {0: np.float32, 1: np.uint16, 2: np.uint8}


def load(name: str) -> dict:
    b = open(os.path.join(GOLDEN, name), "rb").read()
    assert b[:8] == b"SURGEOPS" and struct.unpack_from("<I", b, 8)[0] == 1
    n = struct.unpack_from("<I", b, 12)[0]
    out = {}
    for i in range(n):
        v = struct.unpack_from("<9I", b, 16 + 36 * i)
        nm = b[v[0]:b.index(b"\0", v[0])].decode()
        dims = v[3:3 + v[2]]
        dt = _DT[v[1]]
        arr = np.frombuffer(b, dtype=dt, count=v[8] // np.dtype(dt).itemsize, offset=v[7])
        out[nm] = arr.reshape(dims).copy()
    return out
