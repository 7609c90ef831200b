"""Minimal GGUF v2/v3 container support for the MoE block: reader, writer, in-memory store.

The MoE block constructor only needs three things from a model file: the tensor table
(name -> shape / qtype / byte count), zero-copy access to a tensor's raw bytes, and the
MoE fields of the model config.  This module provides exactly that surface, with the same
attribute names as the reference reader so either object can be handed to
``HipSparseMoEMLP``:

* ``GGUFFile.tensors[name]`` -> ``GGUFTensorInfo`` (``shape`` is the PyTorch row-major
  shape, i.e. the reversed ggml dims)            -- pygguf_engine/gguf_parser.py:125-140, :245
* ``GGUFFile.get_tensor_bytes(name)`` -> uint8 ndarray view of the mmap
                                                   -- pygguf_engine/gguf_parser.py:323-327
* ``GGUFFile.build_model_config()`` -> MoE fields  -- pygguf_engine/gguf_parser.py:399-406

Byte layout of the container follows the public GGUF v3 specification (magic, version,
tensor/kv counts, typed key/value pairs, tensor infos, data aligned to
``general.alignment``).
"""

from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple, Union

import numpy as np

__all__ = [
    "GGMLType",
    "BLOCK_GEOMETRY",
    "GGUFTensorInfo",
    "GGUFFile",
    "GGUFWriter",
    "InMemoryGGUF",
    "MoEConfig",
    "tensor_nbytes",
]


class GGMLType:
    """ggml tensor type ids used on this path (ids are fixed by the GGUF format)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ4_NL = 20
    IQ4_XS = 23
    BF16 = 30
    MXFP4 = 39

    NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
             9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K",
             15: "Q8_K", 20: "IQ4_NL", 23: "IQ4_XS", 30: "BF16", 39: "MXFP4"}


# (weights per block, bytes per block) for the types this reader can size.  Values are
# fixed by the ggml block structs (pygguf_engine/gguf_parser.py:57-91 holds the same table).
BLOCK_GEOMETRY: Dict[int, Tuple[int, int]] = {
    GGMLType.F32: (1, 4),
    GGMLType.F16: (1, 2),
    GGMLType.BF16: (1, 2),
    GGMLType.Q4_0: (32, 18),
    GGMLType.Q4_1: (32, 20),
    GGMLType.Q5_0: (32, 22),
    GGMLType.Q5_1: (32, 24),
    GGMLType.Q8_0: (32, 34),
    GGMLType.Q8_1: (32, 40),
    GGMLType.Q2_K: (256, 84),
    GGMLType.Q3_K: (256, 110),
    GGMLType.Q4_K: (256, 144),
    GGMLType.Q5_K: (256, 176),
    GGMLType.Q6_K: (256, 210),
    GGMLType.Q8_K: (256, 292),
    GGMLType.IQ4_NL: (32, 18),
    GGMLType.IQ4_XS: (256, 136),
    GGMLType.MXFP4: (32, 17),
}


def tensor_nbytes(qtype: int, n_elements: int) -> int:
    per_block, block_bytes = BLOCK_GEOMETRY[qtype]
    if n_elements % per_block:
        raise ValueError(f"{n_elements} elements is not a whole number of type-{qtype} blocks")
    return (n_elements // per_block) * block_bytes


@dataclass
class GGUFTensorInfo:
    name: str
    ggml_dims: Tuple[int, ...]  # innermost first, as stored in the file
    shape: Tuple[int, ...]      # PyTorch order (reversed ggml dims)
    qtype: int
    offset: int                 # relative to the start of the tensor data section
    n_elements: int
    n_bytes: int

    @property
    def qtype_name(self) -> str:
        return GGMLType.NAMES.get(self.qtype, f"TYPE_{self.qtype}")


@dataclass
class MoEConfig:
    """The config fields the MoE block reads (pygguf_engine/gguf_parser.py:168-173)."""

    arch: str = "qwen3moe"
    hidden_size: int = 0
    n_experts: int = 0
    n_experts_used: int = 0
    moe_intermediate_size: int = 0
    shared_expert_intermediate_size: int = 0
    norm_topk_prob: bool = True

    @property
    def is_moe(self) -> bool:
        return self.n_experts > 1


# GGUF metadata value types (format constants).
_VT_U8, _VT_I8, _VT_U16, _VT_I16, _VT_U32, _VT_I32, _VT_F32, _VT_BOOL = range(8)
_VT_STR, _VT_ARR, _VT_U64, _VT_I64, _VT_F64 = 8, 9, 10, 11, 12
_SCALAR_FMT = {
    _VT_U8: "<B", _VT_I8: "<b", _VT_U16: "<H", _VT_I16: "<h", _VT_U32: "<I",
    _VT_I32: "<i", _VT_F32: "<f", _VT_BOOL: "<?", _VT_U64: "<Q", _VT_I64: "<q",
    _VT_F64: "<d",
}


def _norm_topk_default(arch: str) -> bool:
    # qwen2moe keeps raw softmax weights; the others renormalise the top-k
    # (pygguf_engine/gguf_parser.py:404-406).
    return arch in ("qwen3moe", "qwen35moe", "qwen3next", "mixtral", "llama")


def _config_from_metadata(meta: Mapping[str, Any]) -> MoEConfig:
    arch = str(meta.get("general.architecture", "llama"))

    def get(key: str, default: Any) -> Any:
        return meta.get(f"{arch}.{key}", default)

    hidden = int(get("embedding_length", 0) or 0)
    ffn = get("feed_forward_length", 0)
    if isinstance(ffn, list):  # per-layer lists exist in some files
        ffn = max(ffn) if ffn else 0
    ffn = int(ffn or 0)
    return MoEConfig(
        arch=arch,
        hidden_size=hidden,
        n_experts=int(get("expert_count", 0) or 0),
        n_experts_used=int(get("expert_used_count", 0) or 0),
        moe_intermediate_size=int(get("expert_feed_forward_length", ffn) or ffn),
        shared_expert_intermediate_size=int(get("expert_shared_feed_forward_length", 0) or 0),
        norm_topk_prob=bool(get("expert_weights_norm", _norm_topk_default(arch))),
    )


class GGUFFile:
    """Read-only, zero-copy mmap view of a GGUF v2/v3 file."""

    def __init__(self, path: Union[str, Path]) -> None:
        self.path = Path(path)
        self._fh = open(self.path, "rb")
        try:
            self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as exc:  # empty file
            self._fh.close()
            raise ValueError(f"{self.path}: not a GGUF file ({exc})") from None
        self._pos = 0
        if self._take(4) != b"GGUF":
            self.close()
            raise ValueError(f"{self.path}: bad GGUF magic")
        self.version = self._scalar("<I")
        if self.version not in (2, 3):
            self.close()
            raise ValueError(f"{self.path}: unsupported GGUF version {self.version}")
        n_tensors = self._scalar("<Q")
        n_kv = self._scalar("<Q")
        self.metadata: Dict[str, Any] = {}
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._scalar("<I"))
        self.alignment = int(self.metadata.get("general.alignment", 32))
        self.tensors: Dict[str, GGUFTensorInfo] = {}
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._scalar("<I")
            dims = tuple(int(self._scalar("<Q")) for _ in range(n_dims))
            qtype = self._scalar("<I")
            offset = self._scalar("<Q")
            if qtype not in BLOCK_GEOMETRY:
                raise ValueError(f"{name}: tensor type {qtype} is not supported by this reader")
            n_el = int(np.prod(dims, dtype=np.int64)) if dims else 1
            self.tensors[name] = GGUFTensorInfo(
                name=name,
                ggml_dims=dims,
                shape=tuple(reversed(dims)) if dims else (1,),
                qtype=qtype,
                offset=offset,
                n_elements=n_el,
                n_bytes=tensor_nbytes(qtype, n_el),
            )
        pad = (-self._pos) % self.alignment
        self.tensor_data_offset = self._pos + pad

    # -- primitive readers -------------------------------------------------
    def _take(self, n: int) -> bytes:
        out = self._mm[self._pos:self._pos + n]
        self._pos += n
        return out

    def _scalar(self, fmt: str) -> Any:
        (val,) = struct.unpack_from(fmt, self._mm, self._pos)
        self._pos += struct.calcsize(fmt)
        return val

    def _string(self) -> str:
        n = self._scalar("<Q")
        return self._take(n).decode("utf-8", errors="replace")

    def _value(self, vt: int) -> Any:
        if vt == _VT_STR:
            return self._string()
        if vt == _VT_ARR:
            et = self._scalar("<I")
            n = self._scalar("<Q")
            return [self._value(et) for _ in range(n)]
        if vt in _SCALAR_FMT:
            return self._scalar(_SCALAR_FMT[vt])
        raise ValueError(f"unknown GGUF value type {vt}")

    # -- public surface ----------------------------------------------------
    def get_tensor_bytes(self, name: str) -> np.ndarray:
        info = self.tensors[name]
        return np.frombuffer(self._mm, dtype=np.uint8, count=info.n_bytes,
                             offset=self.tensor_data_offset + info.offset)

    def build_model_config(self) -> MoEConfig:
        return _config_from_metadata(self.metadata)

    def close(self) -> None:
        mm, self._mm = getattr(self, "_mm", None), None
        if mm is not None:
            try:
                mm.close()
            except BufferError:
                pass  # live numpy views still reference the map; the OS frees it later
        if not self._fh.closed:
            self._fh.close()

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()


class InMemoryGGUF:
    """Same surface as ``GGUFFile`` over tensors held in memory (synthetic layers)."""

    def __init__(self, metadata: Optional[Mapping[str, Any]] = None) -> None:
        self.metadata: Dict[str, Any] = dict(metadata or {})
        self.tensors: Dict[str, GGUFTensorInfo] = {}
        self._data: Dict[str, np.ndarray] = {}

    def add_tensor(self, name: str, shape: Sequence[int], qtype: int, raw: np.ndarray) -> None:
        shape = tuple(int(s) for s in shape)
        n_el = int(np.prod(shape, dtype=np.int64))
        n_bytes = tensor_nbytes(qtype, n_el)
        raw = np.ascontiguousarray(raw).reshape(-1).view(np.uint8)
        if raw.nbytes != n_bytes:
            raise ValueError(f"{name}: {raw.nbytes} bytes given, {n_bytes} expected")
        self.tensors[name] = GGUFTensorInfo(name, tuple(reversed(shape)), shape, qtype, 0, n_el, n_bytes)
        self._data[name] = raw

    def get_tensor_bytes(self, name: str) -> np.ndarray:
        self.tensors[name]  # KeyError for unknown names, like the file reader
        return self._data[name]

    def build_model_config(self) -> MoEConfig:
        return _config_from_metadata(self.metadata)


class GGUFWriter:
    """Write a GGUF v3 file from metadata and raw tensor bytes (test fixtures, examples)."""

    def __init__(self, alignment: int = 32) -> None:
        self.alignment = alignment
        self.metadata: List[Tuple[str, int, Any]] = []
        self.tensors: List[Tuple[str, Tuple[int, ...], int, np.ndarray]] = []

    def add_meta(self, key: str, value: Any, vtype: Optional[int] = None) -> None:
        if vtype is None:
            if isinstance(value, bool):
                vtype = _VT_BOOL
            elif isinstance(value, int):
                vtype = _VT_U32 if 0 <= value < 2**32 else _VT_I64
            elif isinstance(value, float):
                vtype = _VT_F32
            elif isinstance(value, str):
                vtype = _VT_STR
            else:
                raise TypeError(f"cannot infer GGUF type of {key}={value!r}")
        self.metadata.append((key, vtype, value))

    def add_tensor(self, name: str, shape: Sequence[int], qtype: int, raw: np.ndarray) -> None:
        shape = tuple(int(s) for s in shape)
        raw = np.ascontiguousarray(raw).reshape(-1).view(np.uint8)
        need = tensor_nbytes(qtype, int(np.prod(shape, dtype=np.int64)))
        if raw.nbytes != need:
            raise ValueError(f"{name}: {raw.nbytes} bytes given, {need} expected")
        self.tensors.append((name, shape, qtype, raw))

    @staticmethod
    def _pack_str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _pack_value(self, vt: int, v: Any) -> bytes:
        if vt == _VT_STR:
            return self._pack_str(v)
        if vt == _VT_ARR:
            raise NotImplementedError("array metadata is not needed by this writer")
        return struct.pack(_SCALAR_FMT[vt], v)

    def write(self, path: Union[str, Path]) -> None:
        kv = [("general.alignment", _VT_U32, self.alignment)] + [
            m for m in self.metadata if m[0] != "general.alignment"]
        head = bytearray(b"GGUF")
        head += struct.pack("<IQQ", 3, len(self.tensors), len(kv))
        for key, vt, val in kv:
            head += self._pack_str(key) + struct.pack("<I", vt) + self._pack_value(vt, val)
        offsets, cursor = [], 0
        for _, _, _, raw in self.tensors:
            cursor += (-cursor) % self.alignment
            offsets.append(cursor)
            cursor += raw.nbytes
        for (name, shape, qtype, _), off in zip(self.tensors, offsets):
            dims = tuple(reversed(shape))
            head += self._pack_str(name) + struct.pack("<I", len(dims))
            head += b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", qtype, off)
        head += b"\0" * ((-len(head)) % self.alignment)
        with open(path, "wb") as fh:
            fh.write(head)
            pos = 0
            for (_, _, _, raw), off in zip(self.tensors, offsets):
                fh.write(b"\0" * (off - pos))
                fh.write(raw.tobytes())
                pos = off + raw.nbytes
