"""SBB1 scenario blobs: the self-describing binary container csim and this env read.

Format (little-endian), as parsed by the reference loader
(complete_port/csim/sb_baked.c:19-73) and written by its baker
(complete_port/pysim/sbb.py:4-20,111-120):

  header, 52 bytes : char magic[4] = "SBB1"; u32 version = 1; u32 n_sections;
                     u64 dir_offset; u64 names_offset; u64 names_len;
                     u64 total_size; u64 reserved
  section, 56 bytes: u32 name_off; u32 dtype; u32 ndim; u32 reserved;
                     u64 shape[4]; u64 data_offset
  names            : NUL-terminated ASCII names
  data             : raw arrays, first one 64-byte aligned

dtype codes: 0 f64, 1 f32, 2 i64, 3 i32, 4 i8, 5 u8, 6 u32, 7 str (bytes).
The layout has to match the reference byte for byte, because the compiled
reference core is the parity oracle and reads these files directly.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

MAGIC = b"SBB1"
VERSION = 1
HEADER = struct.Struct("<4sII5Q")   # 52 bytes
SECTION = struct.Struct("<IIII5Q")  # 56 bytes

CODES = {
    "f64": (0, np.float64), "f32": (1, np.float32), "i64": (2, np.int64),
    "i32": (3, np.int32), "i8": (4, np.int8), "u8": (5, np.uint8),
    "u32": (6, np.uint32), "str": (7, np.uint8),
}
BY_CODE = {code: (name, np.dtype(t)) for name, (code, t) in CODES.items()}


class SbbWriter:
    """Collects typed sections in insertion order and writes one blob."""

    def __init__(self) -> None:
        self._items: list[tuple[str, int, tuple[int, ...], bytes]] = []
        self._seen: set[str] = set()

    def add(self, name: str, arr, dtype: str) -> None:
        if name in self._seen:
            raise ValueError(f"duplicate section {name}")
        code, npt = CODES[dtype]
        a = np.ascontiguousarray(np.asarray(arr, dtype=npt))
        if a.ndim > 4:
            raise ValueError(f"{name}: ndim {a.ndim} > 4")
        self._seen.add(name)
        self._items.append((name, code, tuple(int(s) for s in a.shape), a.tobytes()))

    def scalar_f64(self, name: str, v: float) -> None:
        self.add(name, np.asarray([float(v)]), "f64")

    def scalar_i64(self, name: str, v: int) -> None:
        self.add(name, np.asarray([int(v)]), "i64")

    def text(self, name: str, s: str) -> None:
        self.add(name, np.frombuffer(s.encode("utf-8"), dtype=np.uint8), "str")

    def tobytes(self) -> bytes:
        names = bytearray()
        name_off = []
        for name, *_ in self._items:
            name_off.append(len(names))
            names += name.encode("ascii") + b"\x00"
        dir_off = HEADER.size
        names_off = dir_off + SECTION.size * len(self._items)
        data_off = names_off + len(names)
        data_off += (-data_off) % 64
        dir_blob = bytearray()
        cur = data_off
        for (name, code, shape, raw), no in zip(self._items, name_off):
            shape4 = list(shape) + [1] * (4 - len(shape))
            dir_blob += SECTION.pack(no, code, len(shape), 0, *shape4, cur)
            cur += len(raw)
        out = bytearray(HEADER.pack(MAGIC, VERSION, len(self._items), dir_off,
                                    names_off, len(names), cur, 0))
        out += dir_blob
        out += names
        out += b"\x00" * (data_off - len(out))
        for _, _, _, raw in self._items:
            out += raw
        assert len(out) == cur
        return bytes(out)

    def write(self, path) -> int:
        data = self.tobytes()
        p = Path(path)
        tmp = p.with_suffix(p.suffix + ".tmp")
        tmp.write_bytes(data)
        tmp.replace(p)
        return len(data)


def read_sbb(path) -> dict[str, np.ndarray]:
    """Parses a blob into {name: array}; str sections come back as uint8 arrays.

    Zero-dimensional sections are returned with shape (1,), matching the
    reference loader's element count of 1 for ndim == 0.
    """
    raw = Path(path).read_bytes()
    magic, ver, nsec, dir_off, names_off, names_len, total, _ = HEADER.unpack_from(raw, 0)
    if magic != MAGIC or ver != VERSION:
        raise ValueError(f"{path}: not an SBB1 v1 blob")
    out: dict[str, np.ndarray] = {}
    for i in range(nsec):
        no, code, ndim, _, s0, s1, s2, s3, off = SECTION.unpack_from(raw, dir_off + i * SECTION.size)
        end = raw.index(b"\x00", names_off + no)
        name = raw[names_off + no:end].decode("ascii")
        shape = (s0, s1, s2, s3)[:ndim] if ndim else (1,)
        _, dt = BY_CODE[code]
        count = int(np.prod(shape))
        out[name] = np.frombuffer(raw, dtype=dt, count=count, offset=off).reshape(shape)
    return out
