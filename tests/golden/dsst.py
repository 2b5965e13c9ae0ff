"""Reader / writer of the DSST tensor dump format (the stage-dump layout of
the reference's patches/ds4_cpu_stage_dump.patch:17-26): a 32-byte header
(magic "DSST", u32 version 1, u32 dtype 0 = fp32 / 1 = fp16 / 2 = int32, u64
element count, 12 reserved zero bytes) followed by the little-endian payload.
Shapes are not stored; the fixture index (index.json) records them."""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

DTYPES = {0: np.float32, 1: np.float16, 2: np.int32}
CODES = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int32): 2}


def write(path: Path, a: np.ndarray) -> None:
    a = np.ascontiguousarray(a)
    code = CODES[a.dtype]
    hdr = b"DSST" + struct.pack("<IIQ", 1, code, a.size) + b"\0" * 12
    path.write_bytes(hdr + a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes())


def read(path: Path) -> np.ndarray:
    b = path.read_bytes()
    if len(b) < 32 or b[:4] != b"DSST":
        raise ValueError(f"{path}: not a DSST file")
    version, code, n = struct.unpack_from("<IIQ", b, 4)
    if version != 1 or code not in DTYPES or b[20:32] != b"\0" * 12:
        raise ValueError(f"{path}: unsupported DSST header")
    dt = np.dtype(DTYPES[code]).newbyteorder("<")
    if len(b) != 32 + n * dt.itemsize:
        raise ValueError(f"{path}: payload size does not match the element count")
    return np.frombuffer(b, dtype=dt, offset=32, count=n).astype(DTYPES[code])
