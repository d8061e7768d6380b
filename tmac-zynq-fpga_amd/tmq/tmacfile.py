""".tmac container: reader and writer.

Layout (scripts/extract_tmac.py:6-24, read by load_tmac in
sim/tmac_gguf.cpp:1894-1947), all integers little endian:

    char     magic[4] = "TMAC"
    uint64   n_tensors
    n_tensors x {
        uint64 name_len; char name[name_len]
        uint64 rows      # ggml ne[1] (1 for a 1-D tensor)
        uint64 cols      # ggml ne[0]
        uint32 type      # ggml type: 0 F32, 1 F16, 6 Q5_0, 8 Q8_0, 12 Q4_K, 14 Q6_K
        uint64 n_bytes;  uint8 data[n_bytes]
    }

Every Q8_0 tensor is followed (after all regular tensors) by
`<name>_row_max_abs`, F32, rows x 1: the per-row max |q*d| that the Q8_0
logits path uses instead of scanning the row (sim/matmul_q8.cpp:24-30).
"""
from __future__ import annotations

import io
import struct
from dataclasses import dataclass

import numpy as np

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
MAGIC = b"TMAC"


@dataclass
class TmacTensor:
    name: str
    rows: int
    cols: int
    type: int
    data: np.ndarray  # uint8, 1-D

    @property
    def n_bytes(self) -> int:
        return int(self.data.size)


def q8_row_max_abs(data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """max_j |q_j * d| per row of a Q8_0 tensor, as scripts/extract_tmac.py:231-259
    computes it (fp32 products of int8 and the exact fp16 scale)."""
    nb = cols // 32
    blk = data.reshape(rows, nb, 34)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float32).reshape(rows, nb, 1)
    q = blk[:, :, 2:34].view(np.int8).astype(np.float32)
    return np.abs(q * d).reshape(rows, -1).max(axis=1).astype(np.float32)


def write(f, tensors: list[TmacTensor], q8_aux: bool = True) -> int:
    """Write tensors (plus the Q8_0 row_max_abs tensors when q8_aux) to a
    binary file object or path.  Returns the byte count."""
    aux = []
    if q8_aux:
        for t in tensors:
            if t.type == Q8_0:
                rm = q8_row_max_abs(t.data, t.rows, t.cols)
                aux.append(TmacTensor(t.name + "_row_max_abs", t.rows, 1, F32, rm.view(np.uint8).reshape(-1)))
    allt = list(tensors) + aux
    if isinstance(f, (str, bytes)) or hasattr(f, "__fspath__"):
        with open(f, "wb") as fh:
            return write_all(fh, allt)
    return write_all(f, allt)


def write_all(fh, tensors: list[TmacTensor]) -> int:
    n = fh.write(MAGIC)
    n += fh.write(struct.pack("<Q", len(tensors)))
    for t in tensors:
        name = t.name.encode()
        n += fh.write(struct.pack("<Q", len(name)))
        n += fh.write(name)
        n += fh.write(struct.pack("<QQIQ", t.rows, t.cols, t.type, t.n_bytes))
        n += fh.write(memoryview(np.ascontiguousarray(t.data)))
    return n


def to_bytes(tensors: list[TmacTensor], q8_aux: bool = True) -> bytes:
    buf = io.BytesIO()
    write(buf, tensors, q8_aux)
    return buf.getvalue()


def read(src) -> list[TmacTensor]:
    """Parse a .tmac file (path) or buffer (bytes / uint8 array).  Tensor
    data are views into the buffer (a read-only memory map for paths)."""
    if isinstance(src, str) or hasattr(src, "__fspath__"):
        buf = np.memmap(src, dtype=np.uint8, mode="r")
    else:
        buf = np.frombuffer(src, dtype=np.uint8) if not isinstance(src, np.ndarray) else src
    size = buf.size
    if size < 12 or bytes(buf[:4]) != MAGIC:
        raise ValueError("not a .tmac file (magic)")
    (count,) = struct.unpack("<Q", bytes(buf[4:12]))
    off = 12
    out = []
    for i in range(count):
        if size - off < 8:
            raise ValueError(f"truncated at tensor {i}")
        (nl,) = struct.unpack("<Q", bytes(buf[off:off + 8]))
        off += 8
        if nl == 0 or nl > 4096 or size - off < nl + 28:
            raise ValueError(f"bad name length {nl} at tensor {i}")
        name = bytes(buf[off:off + nl]).decode()
        off += nl
        rows, cols, typ, nbytes = struct.unpack("<QQIQ", bytes(buf[off:off + 28]))
        off += 28
        if nbytes > size - off:
            raise ValueError(f"tensor {name}: data past end of file")
        out.append(TmacTensor(name, rows, cols, typ, buf[off:off + nbytes]))
        off += nbytes
    return out
