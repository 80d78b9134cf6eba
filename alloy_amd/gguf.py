"""GGUF tensor-table reading to the raw blobs this library's ops take.

The reference reads GGUF files through the ``gguf`` package and hands each quantized
tensor's bytes to its quantized modules (``packages/alloy-server/src/alloy_server/gguf/
loader.py:97-283``, ``gguf/quant.py:230-267``).  This module reads the file format
itself (GGUF v2/v3: header, metadata key/values, tensor infos, aligned data section)
with a read-only memory map, and returns per tensor:

* Q4_K -> ``blocks`` u8 ``[N, (K/256)*144]`` and Q6_K -> ``qweight`` u8
  ``[N, (K/256)*210]`` (the wire blocks, no copy beyond the host->device upload),
* Q8_0 / Q5_0 -> the reference's split layouts (``split_q8_0_weight``,
  ``split_q5_0_weight``, ``gguf/quant.py:414-521``) or the wire blocks,
* F32 / F16 / BF16 -> dense tensors.

``write_gguf`` writes the same format (used to build files for tests and tools).
Unknown quantization types raise ``NotImplementedError`` like the reference
(``gguf/quant.py:230-249``).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# ggml tensor types this library reads: code -> (name, weights per block, bytes per block)
GGML_TYPES = {
    0: ("f32", 1, 4),
    1: ("f16", 1, 2),
    6: ("q5_0", 32, 22),
    8: ("q8_0", 32, 34),
    12: ("q4_k", 256, 144),
    14: ("q6_k", 256, 210),
    30: ("bf16", 1, 2),
}
GGML_CODE = {v[0]: k for k, v in GGML_TYPES.items()}

# metadata value types
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


@dataclass
class GGUFTensor:
    name: str
    ggml_type: int
    ne: tuple[int, ...]          # ggml order: ne[0] is the row length (contraction dim K)
    offset: int                  # byte offset from the start of the data section

    @property
    def type_name(self) -> str:
        if self.ggml_type not in GGML_TYPES:
            raise NotImplementedError(f"GGUF tensor {self.name!r}: ggml type {self.ggml_type} is not supported")
        return GGML_TYPES[self.ggml_type][0]

    @property
    def shape(self) -> tuple[int, ...]:
        """Row-major (torch) shape: the reverse of ``ne``."""
        return tuple(reversed(self.ne))

    @property
    def nbytes(self) -> int:
        if self.ggml_type not in GGML_TYPES:
            raise NotImplementedError(f"Unsupported quantized GGUF tensor type={self.ggml_type}")
        _, qk, bb = GGML_TYPES[self.ggml_type]
        n = int(np.prod(self.ne, dtype=np.int64))
        if self.ne[0] % qk:
            raise ValueError(f"GGUF tensor {self.name!r}: row length {self.ne[0]} not divisible by {qk}")
        return n // qk * bb


@dataclass
class GGUFFile:
    path: Path
    version: int
    metadata: dict
    tensors: dict[str, GGUFTensor]
    data_offset: int
    alignment: int
    _mm: np.ndarray = field(repr=False, default=None)

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes (read-only view of the file)."""
        t = self.tensors[name]
        start = self.data_offset + t.offset
        return self._mm[start:start + t.nbytes]

    def rows(self, name: str) -> np.ndarray:
        """Quantized tensors as u8 ``[rows, row_bytes]`` wire blocks."""
        t = self.tensors[name]
        if t.type_name not in ("q8_0", "q5_0", "q4_k", "q6_k"):
            raise TypeError(f"{name!r} is {t.type_name}, not a quantized tensor")
        n_rows = int(np.prod(t.ne[1:], dtype=np.int64)) if len(t.ne) > 1 else 1
        return self.raw(name).reshape(n_rows, -1)

    def quantization(self, name: str) -> str | None:
        """``q4_k``/``q5_0``/``q6_k``/``q8_0``, None for the dense types (F32, F16, BF16);
        ``NotImplementedError`` for any other type (``gguf/quant.py:230-249``)."""
        t = self.tensors[name]
        if t.ggml_type not in GGML_TYPES:
            raise NotImplementedError(f"Unsupported quantized GGUF tensor type={t.ggml_type}")
        n = t.type_name
        return None if n in ("f32", "f16", "bf16") else n

    def dense(self, name: str) -> torch.Tensor:
        """F32 / F16 as stored; BF16 widened exactly to f32 and rounded to f16, as the
        reference keeps 16-bit embeddings 16-bit (``gguf/quant.py:252-267``)."""
        t = self.tensors[name]
        if self.quantization(name) is not None:
            raise NotImplementedError(f"Quantized GGUF tensor must stay packed, got type={t.ggml_type}")
        raw = self.raw(name)
        if t.type_name == "f32":
            a = raw.view("<f4")
        elif t.type_name == "f16":
            a = raw.view("<f2")
        elif t.type_name == "bf16":
            a = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32).astype(np.float16)
        return torch.from_numpy(np.array(a).reshape(t.shape))

    def quant_buffers(self, name: str, *, split: bool = True) -> dict[str, torch.Tensor]:
        """Host tensors named as the quantized modules' buffers (``formats.module_buffers``):
        q4_k ``blocks``; q6_k ``qweight``; q8_0 ``qweight``/``scales`` and q5_0
        ``qweight``/``qhigh``/``scales`` in the reference's split layout, or the wire
        ``blocks`` (for ``gguf_q8_0_blocks_mm`` / ``gguf_q5_0_blocks_mm``) with
        ``split=False``."""
        t = self.tensors[name]
        rows = np.array(self.rows(name))   # writable host copy of the mapped bytes
        K = t.ne[0]
        if t.type_name == "q4_k":
            return {"blocks": torch.from_numpy(rows)}
        if t.type_name == "q6_k":
            return {"qweight": torch.from_numpy(rows)}
        if not split:
            return {"blocks": torch.from_numpy(rows)}
        if t.type_name == "q8_0":
            q, s = split_q8_0_weight(rows, K)
            return {"qweight": torch.from_numpy(q), "scales": torch.from_numpy(s)}
        q, h, s = split_q5_0_weight(rows, K)
        return {"qweight": torch.from_numpy(q), "qhigh": torch.from_numpy(h), "scales": torch.from_numpy(s)}


    def linear(self, name: str, bias: torch.Tensor | None = None):
        """The ``GGUF*Linear`` over a quantized 2-D tensor (out_features = rows)."""
        from .modules import GGUFQ4_KLinear, GGUFQ5_0Linear, GGUFQ6_KLinear, GGUFQ8_0Linear
        t = self.tensors[name]
        cls = {"q8_0": GGUFQ8_0Linear, "q5_0": GGUFQ5_0Linear, "q4_k": GGUFQ4_KLinear,
               "q6_k": GGUFQ6_KLinear}.get(self.quantization(name))
        if cls is None or len(t.ne) != 2:
            raise TypeError(f"{name!r} ({t.type_name}, ne={t.ne}) is not a quantized matrix")
        b = torch.nn.Parameter(bias, requires_grad=False) if bias is not None else None
        return cls(in_features=t.ne[0], out_features=t.ne[1], bias=b, **self.quant_buffers(name))

    def embedding(self, name: str, embed_scale: float = 1.0):
        """The ``GGUF*Embedding`` over a quantized 2-D tensor (num_embeddings = rows)."""
        from .modules import GGUFQ4_KEmbedding, GGUFQ5_0Embedding, GGUFQ6_KEmbedding, GGUFQ8_0Embedding
        t = self.tensors[name]
        cls = {"q8_0": GGUFQ8_0Embedding, "q5_0": GGUFQ5_0Embedding, "q4_k": GGUFQ4_KEmbedding,
               "q6_k": GGUFQ6_KEmbedding}.get(self.quantization(name))
        if cls is None or len(t.ne) != 2:
            raise TypeError(f"{name!r} ({t.type_name}, ne={t.ne}) is not a quantized matrix")
        return cls(num_embeddings=t.ne[1], embedding_dim=t.ne[0], embed_scale=embed_scale,
                   **self.quant_buffers(name))

def split_q8_0_weight(rows: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Wire Q8_0 rows -> (qweight int8 [N, K], scales f16 [N, K/32])."""
    N = rows.shape[0]
    blk = rows.reshape(N, K // 32, 34)
    scales = blk[:, :, :2].copy().view("<f2").reshape(N, K // 32)
    qweight = blk[:, :, 2:].copy().view(np.int8).reshape(N, K)
    return qweight, scales.astype(np.float16)


def split_q5_0_weight(rows: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Wire Q5_0 rows -> (qweight u8 [N, K/2], qhigh u8 [N, K/2], scales f16 [N, K/32]):
    the 5-bit values of the row in K order, low nibbles packed two per byte (element
    2j low, 2j+1 high) and the fifth bits likewise (bit 0 and bit 4 of qhigh byte j)."""
    N = rows.shape[0]
    nb = K // 32
    blk = rows.reshape(N, nb, 22)
    scales = blk[:, :, :2].copy().view("<f2").reshape(N, nb).astype(np.float16)
    qh = blk[:, :, 2:6].copy().view("<u4").reshape(N, nb, 1)
    qs = blk[:, :, 6:22]
    low4 = np.concatenate([qs & 0x0F, qs >> 4], axis=2)                       # element l of the block
    fifth = ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)     # bit l of qh
    q5 = (low4 | (fifth << 4)).reshape(N, K)
    even, odd = q5[:, 0::2], q5[:, 1::2]
    qweight = ((even & 0x0F) | ((odd & 0x0F) << 4)).astype(np.uint8)
    qhigh = ((even >> 4) | ((odd >> 4) << 4)).astype(np.uint8)
    return qweight, qhigh, scales


class _Reader:
    def __init__(self, buf: np.ndarray):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise ValueError("truncated GGUF file")
        b = self.buf[self.pos:self.pos + n].tobytes()
        self.pos += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar("<Q")
        return self.take(n).decode("utf-8")

    def value(self, vtype: int):
        if vtype in _SCALARS:
            return self.scalar(_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, count = self.scalar("<I"), self.scalar("<Q")
            return [self.value(etype) for _ in range(count)]
        raise ValueError(f"unknown GGUF metadata value type {vtype}")


def read_gguf(path: str | Path) -> GGUFFile:
    """Parse a GGUF file's tensor table (the tensor data stays memory-mapped)."""
    path = Path(path)
    mm = np.memmap(str(path), dtype=np.uint8, mode="r")
    r = _Reader(mm)
    if r.take(4) != GGUF_MAGIC:
        raise ValueError(f"{path}: not a GGUF file")
    version = r.scalar("<I")
    if version not in (2, 3):
        raise NotImplementedError(f"{path}: GGUF version {version} is not supported")
    n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
    metadata = {}
    for _ in range(n_kv):
        key = r.string()
        metadata[key] = r.value(r.scalar("<I"))
    tensors = {}
    for _ in range(n_tensors):
        name = r.string()
        n_dims = r.scalar("<I")
        ne = tuple(r.scalar("<Q") for _ in range(n_dims))
        ggml_type = r.scalar("<I")
        offset = r.scalar("<Q")
        tensors[name] = GGUFTensor(name, ggml_type, ne, offset)
    alignment = int(metadata.get("general.alignment", DEFAULT_ALIGNMENT))
    data_offset = (r.pos + alignment - 1) // alignment * alignment
    f = GGUFFile(path, version, metadata, tensors, data_offset, alignment, mm)
    for t in tensors.values():
        if t.ggml_type in GGML_TYPES and data_offset + t.offset + t.nbytes > len(mm):
            raise ValueError(f"{path}: tensor {t.name!r} runs past the end of the file")
    return f


def _meta_bytes(value) -> tuple[int, bytes]:
    if isinstance(value, bool):
        return 7, struct.pack("<?", value)
    if isinstance(value, int):
        return (11, struct.pack("<q", value)) if value < 0 else (10, struct.pack("<Q", value))
    if isinstance(value, float):
        return 12, struct.pack("<d", value)
    if isinstance(value, str):
        b = value.encode("utf-8")
        return _STRING, struct.pack("<Q", len(b)) + b
    if isinstance(value, (list, tuple)):
        items = [_meta_bytes(v) for v in value]
        etype = items[0][0] if items else 4
        if any(t != etype for t, _ in items):
            raise TypeError("GGUF arrays must be homogeneous")
        return _ARRAY, struct.pack("<IQ", etype, len(items)) + b"".join(b for _, b in items)
    raise TypeError(f"unsupported GGUF metadata value {value!r}")


def write_gguf(path: str | Path, metadata: dict, tensors: list[tuple[str, str, tuple[int, ...], np.ndarray]],
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.  ``tensors``: (name, type name, ne, bytes) with ``ne`` in
    ggml order (row length first) and the tensor's raw bytes (wire blocks for the
    quantized types)."""
    out = bytearray(GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(metadata)))

    def s(x: str) -> bytes:
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    for k, v in metadata.items():
        vt, vb = _meta_bytes(v)
        out += s(k) + struct.pack("<I", vt) + vb
    offset, blobs = 0, []
    for name, tname, ne, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        t = GGUFTensor(name, GGML_CODE[tname], tuple(int(v) for v in ne), offset)
        if t.nbytes != data.size:
            raise ValueError(f"{name}: {data.size} bytes given, {t.nbytes} expected for {tname} {ne}")
        out += s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", v) for v in t.ne)
        out += struct.pack("<IQ", t.ggml_type, offset)
        blobs.append((offset, data))
        offset = (offset + data.size + alignment - 1) // alignment * alignment
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    out += b"\0" * offset
    for off, data in blobs:
        out[base + off:base + off + data.size] = data.tobytes()
    Path(path).write_bytes(bytes(out))
