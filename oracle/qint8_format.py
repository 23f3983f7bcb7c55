"""CPU restatement of the .qint8 weight-file format (test infrastructure only).

Only tests/ may import this module: the tests check the C-ABI reader in
qwenasr_amd/csrc/qint8_file.hip against it; it is never part of the product path.

* ``write_v1`` restates ``write_qint8_file`` (crates/qwen-asr/src/quantize.rs:385-478):
  INT8 tensors first (data, zero pad to 4, f32 scales), then F32 tensors
  (pad to 4, data, scale_offset 0); table entry without a dtype byte.
* ``write_v2`` restates ``write_qint8_v2_file`` (quantize.rs:481-590): INT8,
  then F32 (pad 4), then BF16 (pad 2); table entry with a dtype byte.
* ``parse`` restates ``QuantFile::open`` (quantize.rs:122-245): magic, table
  loop that stops at the first field cut by the end of the file, V1 dtype from
  scale_offset, unknown V2 dtype byte as INT8, a name that is not UTF-8 fails
  the whole open (``None``), a repeated name maps to its last entry.
* ``fuse_gate_up`` restates the row interleave of ``DecoderInt8::load``
  (crates/qwen-asr/src/decoder.rs:697-719).

Pinning (the reference ships no .qint8 file and no test of the format): the
writer and parser are checked against each other on round trips, and against
hand-assembled byte strings whose expected parse is fixed by the format
description at quantize.rs:1-34 (tests/test_qint8.py).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC_V1 = b"QINT8\x01\x00\x00"
MAGIC_V2 = b"QINT8\x02\x00\x00"
INT8, F32, BF16 = 0, 1, 2


@dataclass
class Meta:
    name: str
    dtype: int
    shape: list[int] = field(default_factory=list)
    data_offset: int = 0
    scale_offset: int = 0

    @property
    def numel(self) -> int:  # quantize.rs:59-61 (empty shape -> 1)
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def out_dim(self) -> int:  # quantize.rs:64-66
        return self.shape[0] if self.shape else 0

    @property
    def in_dim(self) -> int:  # quantize.rs:69-71
        if len(self.shape) < 2:
            return 0
        n = 1
        for d in self.shape[1:]:
            n *= d
        return n


def _pad(buf: bytearray, align: int) -> None:
    while len(buf) % align:
        buf.append(0)


def _entry(m: Meta, v2: bool) -> bytes:
    nb = m.name.encode()
    out = struct.pack("<H", len(nb)) + nb
    if v2:
        out += bytes([m.dtype])
    out += bytes([len(m.shape)]) + b"".join(struct.pack("<I", d) for d in m.shape)
    return out + struct.pack("<QQ", m.data_offset, m.scale_offset)


def _file(magic: bytes, metas: list[Meta], data: bytearray, v2: bool) -> bytes:
    head = magic + struct.pack("<II", len(metas), 0)
    return head + b"".join(_entry(m, v2) for m in metas) + bytes(data)


def _pack_int8(data: bytearray, name, shape, q: np.ndarray, scales: np.ndarray) -> Meta:
    off = len(data)
    data += np.ascontiguousarray(q, dtype=np.int8).tobytes()
    _pad(data, 4)
    soff = len(data)
    data += np.ascontiguousarray(scales, dtype="<f4").tobytes()
    return Meta(name, INT8, list(shape), off, soff)


def write_v1(quant: list, f32: list) -> bytes:
    """quant: [(name, shape, int8 array, f32 scales)]; f32: [(name, shape, f32 array)]."""
    data = bytearray()
    metas = [_pack_int8(data, *e) for e in quant]
    for name, shape, arr in f32:
        _pad(data, 4)
        off = len(data)
        data += np.ascontiguousarray(arr, dtype="<f4").tobytes()
        metas.append(Meta(name, F32, list(shape), off, 0))
    return _file(MAGIC_V1, metas, data, v2=False)


def write_v2(quant: list, f32: list, bf16: list) -> bytes:
    """As write_v1, plus bf16: [(name, shape, uint16 bit patterns)]."""
    data = bytearray()
    metas = [_pack_int8(data, *e) for e in quant]
    for name, shape, arr in f32:
        _pad(data, 4)
        off = len(data)
        data += np.ascontiguousarray(arr, dtype="<f4").tobytes()
        metas.append(Meta(name, F32, list(shape), off, 0))
    for name, shape, arr in bf16:
        _pad(data, 2)
        off = len(data)
        data += np.ascontiguousarray(arr, dtype="<u2").tobytes()
        metas.append(Meta(name, BF16, list(shape), off, 0))
    return _file(MAGIC_V2, metas, data, v2=True)


def parse(buf: bytes):
    """-> None, or (version, [Meta], {name: index}, data_start)."""
    size = len(buf)
    if size < 16:
        return None
    if buf[:8] == MAGIC_V2:
        v2 = True
    elif buf[:8] == MAGIC_V1:
        v2 = False
    else:
        return None
    (n,) = struct.unpack_from("<I", buf, 8)
    pos = 16
    metas: list[Meta] = []
    index: dict[str, int] = {}
    for _ in range(n):
        if pos + 2 > size:
            break
        (name_len,) = struct.unpack_from("<H", buf, pos)
        pos += 2
        if pos + name_len > size:
            break
        try:
            name = buf[pos:pos + name_len].decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            return None
        pos += name_len
        dtype = INT8
        if v2:
            if pos + 1 > size:
                break
            b = buf[pos]
            pos += 1
            dtype = b if b in (INT8, F32, BF16) else INT8
        if pos + 1 > size:
            break
        n_dims = buf[pos]
        pos += 1
        shape = []
        for _ in range(n_dims):
            if pos + 4 > size:
                break
            shape.append(struct.unpack_from("<I", buf, pos)[0])
            pos += 4
        if pos + 16 > size:
            break
        data_offset, scale_offset = struct.unpack_from("<QQ", buf, pos)
        pos += 16
        if not v2:
            dtype = F32 if scale_offset == 0 else INT8
        index[name] = len(metas)
        metas.append(Meta(name, dtype, shape, data_offset, scale_offset))
    return (2 if v2 else 1), metas, index, pos


def tensor_bytes(buf: bytes, data_start: int, m: Meta):
    """(data bytes, scale bytes or None) of tensor m, as QuantFile hands them out."""
    es = {INT8: 1, F32: 4, BF16: 2}[m.dtype]
    a = data_start + m.data_offset
    data = buf[a:a + m.numel * es]
    scales = None
    if m.dtype == INT8:
        s = data_start + m.scale_offset
        scales = buf[s:s + 4 * m.out_dim]
    return data, scales


def fuse_gate_up(gate: np.ndarray, gs: np.ndarray, up: np.ndarray, us: np.ndarray):
    """Fused [2*inter, hidden] int8 matrix and [2*inter] scales: rows g0, u0, g1, u1, ..."""
    inter, hidden = gate.shape
    w = np.empty((2 * inter, hidden), np.int8)
    s = np.empty(2 * inter, np.float32)
    for r in range(inter):
        w[2 * r] = gate[r]
        w[2 * r + 1] = up[r]
        s[2 * r] = gs[r]
        s[2 * r + 1] = us[r]
    return w, s
