"""Minimal GGUF v3 reader/writer for parakeet decoder checkpoints.

Implements the subset of the GGUF container used by parakeet.cpp decoder
GGUFs: scalar/string/array metadata and f32 / f16 / q8_0 / q5_0 / q4_0
tensors (the five ``--quant`` choices of scripts/convert-nemo-to-gguf.py:90-103).  The
tensor naming, shapes and the q8_0-when-``in % 32 == 0`` rule follow the
reference converter (scripts/convert-nemo-to-gguf.py:405-413, 506-525,
563-582); the metadata keys follow its writer (:293-352) and the reader's
defaults (src/parakeet_ctc.cpp:418-458).

Byte layout (GGUF v3, little endian):
  magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
  n_kv x (string key, u32 type, value),
  n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset),
  zero padding to ``general.alignment`` (default 32), tensor data.
Strings are (u64 length, bytes).  ``ne`` lists the innermost dimension
first, so a PyTorch ``[out, in]`` matrix has ``ne = [in, out]``.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q5_0 = 6
GGML_Q8_0 = 8
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34
# 32-weight blocks of ggml's block-quantized types (ggml, pinned by the reference at commit
# 58c38058, scripts/setup-ggml.sh:32): q8_0 {f16 d; i8 q[32]}, q5_0 {f16 d; u8 qh[4]; u8 qs[16]},
# q4_0 {f16 d; u8 qs[16]}
BLOCK_BYTES = {GGML_Q8_0: 34, GGML_Q5_0: 22, GGML_Q4_0: 18}
QUANT_TYPES = {"q8_0": GGML_Q8_0, "q5_0": GGML_Q5_0, "q4_0": GGML_Q4_0}

# GGUF metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
               T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
_NP_DTYPE = {T_U8: np.uint8, T_I8: np.int8, T_U16: np.uint16, T_I16: np.int16, T_U32: np.uint32,
             T_I32: np.int32, T_F32: np.float32, T_BOOL: np.bool_, T_U64: np.uint64,
             T_I64: np.int64, T_F64: np.float64}


def tensor_nbytes(ggml_type: int, n_elements: int) -> int:
    if ggml_type == GGML_F32:
        return 4 * n_elements
    if ggml_type == GGML_F16:
        return 2 * n_elements
    if ggml_type in BLOCK_BYTES:
        if n_elements % QK8_0:
            raise ValueError("block-quantized tensor size must be a multiple of 32")
        return (n_elements // QK8_0) * BLOCK_BYTES[ggml_type]
    raise ValueError(f"unsupported ggml type {ggml_type}")


def quantize_q8_0(x: np.ndarray) -> bytes:
    """q8_0 blocks along the last axis: d = max|x| / 127 (stored f16), q = round(x / d)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape[-1] % QK8_0:
        raise ValueError("q8_0 needs the innermost dimension to be a multiple of 32")
    blocks = x.reshape(-1, QK8_0)
    amax = np.abs(blocks).max(axis=1)
    d = (amax / 127.0).astype(np.float32)
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.rint(blocks * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((blocks.shape[0], Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def _blocks(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape[-1] % QK8_0:
        raise ValueError("block quantization needs the innermost dimension to be a multiple of 32")
    return x.reshape(-1, QK8_0)


def _signed_absmax(blocks: np.ndarray) -> np.ndarray:
    """Per block, the element of largest magnitude with its sign (the first one on ties)."""
    return blocks[np.arange(blocks.shape[0]), np.abs(blocks).argmax(axis=1)]


def quantize_q4_0(x: np.ndarray) -> bytes:
    """ggml's reference q4_0 rule: d = max / -8 (max: the signed value of largest magnitude),
    q = min(15, trunc(x / d + 8.5)); weight j in the low nibble of qs[j], weight j + 16 in the
    high nibble."""
    b = _blocks(x)
    d = (_signed_absmax(b) / np.float32(-8.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0))
    q = np.minimum(15, np.trunc(b * inv[:, None].astype(np.float32) + np.float32(8.5))).astype(np.uint8)
    out = np.empty((b.shape[0], BLOCK_BYTES[GGML_Q4_0]), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.tobytes()


def quantize_q5_0(x: np.ndarray) -> bytes:
    """ggml's reference q5_0 rule: d = max / -16, q = min(31, trunc(x / d + 16.5)); low 4 bits
    packed as in q4_0, bit 4 of weight j is bit j of the little-endian word qh."""
    b = _blocks(x)
    d = (_signed_absmax(b) / np.float32(-16.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0))
    q = np.minimum(31, np.trunc(b * inv[:, None].astype(np.float32) + np.float32(16.5))).astype(np.uint32)
    qh = ((q >> 4) & 1) << np.arange(32, dtype=np.uint32)
    qh = np.bitwise_or.reduce(qh, axis=1).astype(np.uint32)
    out = np.empty((b.shape[0], BLOCK_BYTES[GGML_Q5_0]), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:6] = qh.astype("<u4").view(np.uint8).reshape(-1, 4)
    out[:, 6:] = ((q[:, :16] & 15) | ((q[:, 16:] & 15) << 4)).astype(np.uint8)
    return out.tobytes()


QUANTIZE = {GGML_Q8_0: quantize_q8_0, GGML_Q5_0: quantize_q5_0, GGML_Q4_0: quantize_q4_0}


def block_ints(raw: bytes | np.ndarray, ggml_type: int, n_blocks: int) -> tuple[np.ndarray, np.ndarray]:
    """Scales (float32) and integer weights [n_blocks, 32] of a block-quantized buffer."""
    buf = np.frombuffer(raw, dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    blocks = buf[: n_blocks * BLOCK_BYTES[ggml_type]].reshape(n_blocks, BLOCK_BYTES[ggml_type])
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    if ggml_type == GGML_Q8_0:
        return d, blocks[:, 2:].view(np.int8).astype(np.int32)
    if ggml_type == GGML_Q5_0:
        qh = blocks[:, 2:6].copy().view("<u4").astype(np.uint32).reshape(-1, 1)
        qs = blocks[:, 6:].astype(np.int32)
        hi = ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int32) << 4
        q = np.concatenate([qs & 15, qs >> 4], axis=1) | hi
        return d, q - 16
    qs = blocks[:, 2:].astype(np.int32)
    return d, np.concatenate([qs & 15, qs >> 4], axis=1) - 8


def dequantize(raw: bytes | np.ndarray, ggml_type: int, n_elements: int) -> np.ndarray:
    """ggml ``to_float`` for the supported types (float32 result)."""
    buf = np.frombuffer(raw, dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    if ggml_type == GGML_F32:
        return buf.view(np.float32)[:n_elements].copy()
    if ggml_type == GGML_F16:
        return buf.view(np.float16)[:n_elements].astype(np.float32)
    if ggml_type in BLOCK_BYTES:
        if n_elements % QK8_0:
            raise ValueError("block-quantized tensor size must be a multiple of 32")
        d, q = block_ints(buf, ggml_type, n_elements // QK8_0)
        return (q.astype(np.float32) * d[:, None]).reshape(-1)
    raise ValueError(f"unsupported ggml type {ggml_type}")


@dataclass
class TensorInfo:
    name: str
    ggml_type: int
    ne: tuple          # innermost first
    offset: int        # absolute file offset of the data
    nbytes: int

    @property
    def n_elements(self) -> int:
        n = 1
        for v in self.ne:
            n *= int(v)
        return n


class GGUFWriter:
    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.kv: list[tuple[str, int, object, int | None]] = []
        self.tensors: list[tuple[str, int, tuple, bytes]] = []

    # metadata
    def add(self, key: str, vtype: int, value, elem_type: int | None = None):
        self.kv.append((key, vtype, value, elem_type))

    def add_u32(self, key, v): self.add(key, T_U32, int(v))
    def add_i32(self, key, v): self.add(key, T_I32, int(v))
    def add_f32(self, key, v): self.add(key, T_F32, float(v))
    def add_bool(self, key, v): self.add(key, T_BOOL, bool(v))
    def add_str(self, key, v): self.add(key, T_STR, str(v))
    def add_arr(self, key, elem_type, values): self.add(key, T_ARR, list(values), elem_type)

    def add_tensor(self, name: str, raw: bytes, ne: tuple, ggml_type: int):
        n = 1
        for v in ne:
            n *= int(v)
        if len(raw) != tensor_nbytes(ggml_type, n):
            raise ValueError(f"{name}: {len(raw)} bytes for ne={ne} type={ggml_type}")
        self.tensors.append((name, ggml_type, tuple(int(v) for v in ne), raw))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _value(self, vtype, value, elem_type) -> bytes:
        if vtype == T_STR:
            return self._str(value)
        if vtype == T_ARR:
            out = struct.pack("<IQ", elem_type, len(value))
            if elem_type == T_STR:
                return out + b"".join(self._str(v) for v in value)
            return out + np.asarray(value, dtype=_NP_DTYPE[elem_type]).tobytes()
        return struct.pack(_SCALAR_FMT[vtype], value)

    def write(self, path: str):
        head = bytearray()
        head += b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))
        for key, vtype, value, elem_type in self.kv:
            head += self._str(key) + struct.pack("<I", vtype) + self._value(vtype, value, elem_type)
        offsets, off = [], 0
        for name, gtype, ne, raw in self.tensors:
            offsets.append(off)
            off += len(raw)
            off = (off + self.alignment - 1) // self.alignment * self.alignment
        for (name, gtype, ne, raw), o in zip(self.tensors, offsets):
            head += self._str(name) + struct.pack("<I", len(ne))
            head += struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", gtype, o)
        pad = (-len(head)) % self.alignment
        head += b"\0" * pad
        with open(path, "wb") as f:
            f.write(head)
            pos = 0
            for (name, gtype, ne, raw), o in zip(self.tensors, offsets):
                f.write(b"\0" * (o - pos))
                f.write(raw)
                pos = o + len(raw)


class GGUFReader:
    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            data = f.read()
        self._data = data
        if data[:4] != b"GGUF":
            raise ValueError(f"{path}: not a GGUF file")
        version, n_t, n_kv = struct.unpack_from("<IQQ", data, 4)
        if version not in (2, 3):
            raise ValueError(f"{path}: unsupported GGUF version {version}")
        p = 24
        self.kv: dict[str, object] = {}
        for _ in range(n_kv):
            key, p = self._read_str(p)
            (vtype,) = struct.unpack_from("<I", data, p)
            p += 4
            self.kv[key], p = self._read_value(vtype, p)
        align = int(self.kv.get("general.alignment", 32))
        infos = []
        for _ in range(n_t):
            name, p = self._read_str(p)
            (nd,) = struct.unpack_from("<I", data, p)
            p += 4
            ne = struct.unpack_from(f"<{nd}Q", data, p)
            p += 8 * nd
            gtype, off = struct.unpack_from("<IQ", data, p)
            p += 12
            infos.append((name, gtype, ne, off))
        base = (p + align - 1) // align * align
        self.tensors: dict[str, TensorInfo] = {}
        for name, gtype, ne, off in infos:
            n = 1
            for v in ne:
                n *= int(v)
            self.tensors[name] = TensorInfo(name, gtype, tuple(int(v) for v in ne), base + off,
                                            tensor_nbytes(gtype, n))

    def _read_str(self, p):
        (n,) = struct.unpack_from("<Q", self._data, p)
        p += 8
        return self._data[p:p + n].decode("utf-8", errors="replace"), p + n

    def _read_value(self, vtype, p):
        if vtype == T_STR:
            return self._read_str(p)
        if vtype == T_ARR:
            et, n = struct.unpack_from("<IQ", self._data, p)
            p += 12
            if et == T_STR:
                out = []
                for _ in range(n):
                    s, p = self._read_str(p)
                    out.append(s)
                return out, p
            dt = np.dtype(_NP_DTYPE[et])
            arr = np.frombuffer(self._data, dtype=dt, count=n, offset=p).copy()
            return arr, p + n * dt.itemsize
        fmt = _SCALAR_FMT[vtype]
        (v,) = struct.unpack_from(fmt, self._data, p)
        return v, p + struct.calcsize(fmt)

    def raw(self, name: str) -> bytes:
        t = self.tensors[name]
        return self._data[t.offset:t.offset + t.nbytes]

    def f32(self, name: str) -> np.ndarray:
        """Dequantised tensor, shaped PyTorch-style (outermost first)."""
        t = self.tensors[name]
        arr = dequantize(self.raw(name), t.ggml_type, t.n_elements)
        return arr.reshape(tuple(reversed(t.ne)))
