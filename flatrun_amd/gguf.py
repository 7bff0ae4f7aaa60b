"""GGUF v2/v3 files: reader, and device residency of their raw blocks.

The reader follows the reference's storage backend
(``src/flatrun/backend/gguf.py``): header ``GGUF`` + version (2 or 3) +
tensor count + KV count (``:435-452``), the metadata KV table (``:478-525``),
the tensor-info table with ``ne[]`` reversed into row-major ``(out, in)``
(``:527-558``), the data section at ``align_up(end of infos,
general.alignment)`` with alignment 32 by default (``:460-468``), tensor
offsets relative to it (``:307``), byte sizes from the block table
(``_GGML_TYPES`` / ``_ggml_block_bytes``, ``:59-103``) and zero-copy
read-only views of the memory-mapped file (``MmapTensorHandle.view``,
``core/tensor.py:227-270``). Names are translated from GGUF to the
HuggingFace Qwen2 spelling exactly when the reference does (see
``GGUFFile``).

Where this reader differs, it is stricter, never more lenient: metadata
value types follow the published GGUF table (10 = uint64, 11 = int64,
12 = float64 -- the reference reads 10 as int64, 11 as float64 and rejects
12), and a tensor whose bytes run past the end of the file is an error at
open time rather than a short buffer later.

Device residency (:class:`ResidentModel`) has no counterpart in the
reference, whose layer scheduler reads the mmap synchronously on the host
(``runtime/scheduler.py:222-325``): every selected tensor goes to one
device arena at 256-byte aligned offsets, copied from the mmap through two
pinned staging slots on a copy stream, so the page-cache -> pinned copy of
one chunk overlaps the PCIe transfer of the previous one. The tensors then
serve every ``NativeBackend.matmul_*`` / ``device.gemv`` call as
:class:`flatrun_amd.DeviceWeight` views, without any further host traffic.
"""

from __future__ import annotations

import mmap
import os
import struct
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"
SUPPORTED_VERSIONS = (2, 3)
DEFAULT_ALIGNMENT = 32
MAX_STRING = 1 << 20          # the reference's sanity bound on a string length (gguf.py:516-518)
ARENA_ALIGN = 256


class GGUFError(RuntimeError):
    """Malformed or unsupported file (the reference raises BackendError)."""


class TensorNotFound(KeyError):
    """No tensor of that name (the reference raises TensorNotFoundError)."""


@dataclass(frozen=True)
class GGMLType:
    name: str
    type_size: int     # bytes per block
    block_size: int    # elements per block


# GGML type id -> block layout; the same table as the reference's
# _GGML_TYPES (backend/gguf.py:59-86): a file-format constant.
GGML_TYPES: dict[int, GGMLType] = {
    0: GGMLType("F32", 4, 1),
    1: GGMLType("F16", 2, 1),
    2: GGMLType("Q4_0", 18, 32),
    3: GGMLType("Q4_1", 20, 32),
    6: GGMLType("Q5_0", 22, 32),
    7: GGMLType("Q5_1", 24, 32),
    8: GGMLType("Q8_0", 34, 32),
    9: GGMLType("Q8_1", 36, 32),
    10: GGMLType("Q2_K", 84, 256),
    11: GGMLType("Q3_K", 110, 256),
    12: GGMLType("Q4_K", 144, 256),
    13: GGMLType("Q5_K", 176, 256),
    14: GGMLType("Q6_K", 210, 256),
    15: GGMLType("Q8_K", 292, 256),
    16: GGMLType("IQ2_XXS", 66, 256),
    17: GGMLType("IQ2_XS", 82, 256),
    18: GGMLType("IQ3_XXS", 98, 256),
    19: GGMLType("IQ1_S", 50, 256),
    20: GGMLType("IQ4_NL", 136, 256),
    21: GGMLType("IQ3_S", 114, 256),
    22: GGMLType("IQ2_S", 82, 256),
    23: GGMLType("IQ4_XS", 136, 256),
    41: GGMLType("Q1_0", 18, 128),
}
TYPE_IDS = {t.name: i for i, t in GGML_TYPES.items()}


def type_name(type_id: int) -> str:
    t = GGML_TYPES.get(type_id)
    return t.name if t is not None else f"Unknown({type_id})"


def tensor_nbytes(type_id: int, numel: int) -> int:
    """Stored bytes of a tensor: whole blocks, the last one padded
    (``_ggml_block_bytes``, gguf.py:89-103; an unknown type is sized as F16
    there too)."""
    t = GGML_TYPES.get(type_id)
    if t is None:
        return numel * 2
    if t.block_size == 1:
        return numel * t.type_size
    return (numel + t.block_size - 1) // t.block_size * t.type_size


def numpy_dtype(type_id: int) -> str:
    """float32 / float16 for the plain types, uint8 (raw blocks) otherwise
    (``_ggml_to_numpy_dtype``, gguf.py:113-127)."""
    return {0: "float32", 1: "float16"}.get(type_id, "uint8")


# GGUF metadata value types (published GGUF table).
_SCALARS = {
    0: ("<B", 1), 1: ("<b", 1), 2: ("<H", 2), 3: ("<h", 2), 4: ("<I", 4), 5: ("<i", 4),
    6: ("<f", 4), 7: ("<?", 1), 10: ("<Q", 8), 11: ("<q", 8), 12: ("<d", 8),
}
_STRING, _ARRAY, _BOOL = 8, 9, 7

# GGUF -> HuggingFace Qwen2 tensor names; the reference's naming table
# (_GGUF_TO_HF_QWEN2, gguf.py:176-189): an interface constant.
_GGUF_TO_HF_QWEN2 = {
    "token_embd": "model.embed_tokens",
    "output_norm": "model.norm",
    "output": "lm_head",
    "attn_norm": "input_layernorm",
    "attn_q": "self_attn.q_proj",
    "attn_k": "self_attn.k_proj",
    "attn_v": "self_attn.v_proj",
    "attn_output": "self_attn.o_proj",
    "ffn_norm": "post_attention_layernorm",
    "ffn_gate": "mlp.gate_proj",
    "ffn_up": "mlp.up_proj",
    "ffn_down": "mlp.down_proj",
}
_SUFFIXES = (".weight", ".bias", ".biases", ".scales")


def translate_gguf_name(name: str, architecture: str | None = None) -> str:
    """``blk.<i>.<base><suffix>`` -> ``model.layers.<i>.<hf base><suffix>``
    and ``<base><suffix>`` -> ``<hf base><suffix>`` for architecture None or
    "qwen2"; any other architecture passes through (gguf.py:192-219)."""
    if architecture not in (None, "qwen2"):
        return name
    if name.startswith("blk."):
        parts = name.split(".", 2)
        if len(parts) == 3:
            idx, rest = parts[1], parts[2]
            for sfx in _SUFFIXES:
                if rest.endswith(sfx):
                    base = rest[: -len(sfx)]
                    return f"model.layers.{idx}.{_GGUF_TO_HF_QWEN2.get(base, base)}{sfx}"
    for sfx in _SUFFIXES:
        if name.endswith(sfx):
            base = name[: -len(sfx)]
            return f"{_GGUF_TO_HF_QWEN2.get(base, base)}{sfx}"
    return name


@dataclass(frozen=True)
class TensorInfo:
    name: str                    # after translation
    gguf_name: str               # as stored in the file
    shape: tuple[int, ...]       # row-major: (out, in) for a matrix
    ggml_type: int
    offset: int                  # absolute byte offset in the file
    nbytes: int

    @property
    def type_name(self) -> str:
        return type_name(self.ggml_type)

    @property
    def dtype(self) -> str:
        return numpy_dtype(self.ggml_type)

    @property
    def quantization(self) -> str | None:
        """The GGML type name for block-quantized tensors, None for F32/F16
        (TensorMetadata.quantization as the reference fills it, gguf.py:324-334)."""
        return self.type_name if self.dtype == "uint8" else None

    @property
    def matrix(self) -> tuple[int, int]:
        """(n, k) of a weight matrix: rows = product of the outer dims."""
        if not self.shape:
            return 1, 1
        k = self.shape[-1]
        n = 1
        for d in self.shape[:-1]:
            n *= d
        return n, k


class _Cursor:
    """Little-endian reads from the mapped file with bounds checks."""

    def __init__(self, buf, size: int):
        self.buf, self.size, self.pos = buf, size, 0

    def take(self, fmt: str, n: int):
        if self.pos + n > self.size:
            raise GGUFError(f"GGUF header truncated at byte {self.pos} (need {n} more, file has {self.size})")
        (v,) = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += n
        return v

    def string(self) -> str:
        n = self.take("<Q", 8)
        if n > MAX_STRING:
            raise GGUFError(f"Suspicious GGUF string length {n}")
        if self.pos + n > self.size:
            raise GGUFError(f"GGUF string runs past the end of the file at byte {self.pos}")
        text = bytes(self.buf[self.pos: self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return text[:-1] if text.endswith("\x00") else text

    def value(self, vtype: int):
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype = self.take("<I", 4)
            count = self.take("<Q", 8)
            if etype in _SCALARS and etype != _BOOL:
                fmt, sz = _SCALARS[etype]
                if self.pos + count * sz > self.size:
                    raise GGUFError(f"GGUF array runs past the end of the file at byte {self.pos}")
                arr = np.frombuffer(self.buf, dtype=np.dtype(fmt), count=count, offset=self.pos)
                self.pos += count * sz
                return arr.tolist()
            return [self.value(etype) for _ in range(count)]
        if vtype in _SCALARS:
            fmt, sz = _SCALARS[vtype]
            v = self.take(fmt, sz)
            return bool(v) if vtype == _BOOL else v
        raise GGUFError(f"Unknown GGUF metadata type id {vtype}")


class GGUFFile:
    """A memory-mapped GGUF file.

    ``translate_names`` (default True) renames tensors with the Qwen2 table
    whatever ``general.architecture`` says: the reference's first pass
    translates with architecture None, i.e. with that table, and its second,
    architecture-aware pass leaves already translated names alone
    (gguf.py:298-365).
    """

    def __init__(self, path, *, translate_names: bool = True):
        self.path = Path(path)
        self.translate = bool(translate_names)
        if not self.path.is_file():
            raise GGUFError(f"GGUF file not found: {self.path}")
        self._fd = os.open(self.path, os.O_RDONLY)
        self._mm = None
        try:
            size = os.fstat(self._fd).st_size
            if size < 24:
                raise GGUFError(f"GGUF file is too small: {self.path}")
            self._mm = mmap.mmap(self._fd, 0, access=mmap.ACCESS_READ)
            self._parse(size)
        except BaseException:
            self.close()
            raise

    # --------------------------------------------------------------- parsing
    def _parse(self, size: int) -> None:
        c = _Cursor(self._mm, size)
        magic = bytes(self._mm[0:4])
        if magic != GGUF_MAGIC:
            raise GGUFError(f"Bad GGUF magic in {self.path}: expected b'GGUF', got {magic!r}")
        c.pos = 4
        self.version = c.take("<I", 4)
        if self.version not in SUPPORTED_VERSIONS:
            raise GGUFError(f"Unsupported GGUF version {self.version}; supported: {SUPPORTED_VERSIONS}")
        n_tensors = c.take("<Q", 8)
        n_kv = c.take("<Q", 8)
        self.metadata: dict[str, object] = {}
        for _ in range(n_kv):
            key = c.string()
            vtype = c.take("<I", 4)
            self.metadata[key] = c.value(vtype)
        raw = []
        for _ in range(n_tensors):
            name = c.string()
            ndim = c.take("<I", 4)
            ne = [c.take("<Q", 8) for _ in range(ndim)]
            gtype = c.take("<I", 4)
            rel = c.take("<Q", 8)
            raw.append((name, tuple(reversed(ne)), gtype, rel))
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0:
            raise GGUFError(f"invalid general.alignment {self.alignment}")
        self.data_offset = (c.pos + self.alignment - 1) // self.alignment * self.alignment
        if self.data_offset > size:
            raise GGUFError(f"Computed GGUF data offset {self.data_offset} exceeds file size {size}")
        self.architecture = self.metadata.get("general.architecture")
        self.tensors: dict[str, TensorInfo] = {}
        for name, shape, gtype, rel in raw:
            numel = 1
            for d in shape:
                numel *= int(d)
            nbytes = tensor_nbytes(gtype, numel)
            off = self.data_offset + int(rel)
            if off + nbytes > size:
                raise GGUFError(f"tensor {name!r} ({nbytes} B at {off}) runs past the end of the file ({size} B)")
            shown = translate_gguf_name(name, None) if self.translate else name
            self.tensors[shown] = TensorInfo(shown, name, tuple(int(d) for d in shape), int(gtype), off, nbytes)

    # ------------------------------------------------------------- interface
    def names(self) -> list[str]:
        return list(self.tensors)

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def info(self, name: str) -> TensorInfo:
        try:
            return self.tensors[name]
        except KeyError as exc:
            raise TensorNotFound(name) from exc

    def raw(self, name: str) -> np.ndarray:
        """Zero-copy read-only view: the raw block bytes (1-D uint8) of a
        quantized tensor, a typed array of its shape for F32 / F16
        (MmapTensorHandle.view, core/tensor.py:227-270)."""
        t = self.info(name)
        if self._mm is None:
            raise GGUFError(f"{self.path} is closed")
        if t.quantization is not None:
            a = np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)
        else:
            dt = np.dtype(t.dtype)
            a = np.frombuffer(self._mm, dtype=dt, count=t.nbytes // dt.itemsize, offset=t.offset).reshape(t.shape)
        return a  # frombuffer over an ACCESS_READ map is read-only

    @property
    def nbytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())

    def close(self) -> None:
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass        # a view is still alive; the map goes with it
            self._mm = None
        if self._fd is not None:
            os.close(self._fd)
            self._fd = None

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ResidentModel:
    """Tensors of a GGUF file resident in one device arena.

    ``names`` selects tensors (default: all). ``staging_bytes`` is the size
    of each of the two pinned staging slots; ``copy_threads`` host threads
    copy a chunk from the page cache into its slot (numpy releases the GIL
    for the copy; default min(8, CPUs): the host copy, not PCIe, bounds the
    load, measured 14-18 GB/s at 4 threads, 21-24 at 8, 23-24 at 12-16,
    warm page cache, MI355X host). Tensor bytes are laid out in file order at 256-byte
    aligned arena offsets. ``model[name]`` is a :class:`DeviceWeight` view
    carrying the tensor's ``qtype`` and ``shape``; ``load_seconds`` and
    ``nbytes`` give the file -> HBM rate.
    """

    def __init__(self, gguf: "GGUFFile | str | os.PathLike", names=None, *, staging_bytes: int = 64 << 20,
                 copy_threads: int | None = None, stream=None):
        from . import device
        from . import DeviceWeight

        own = not isinstance(gguf, GGUFFile)
        self.file = GGUFFile(gguf) if own else gguf
        self._own_file = own
        self.arena = None
        self.weights: dict[str, DeviceWeight] = {}
        try:
            sel = list(self.file.tensors) if names is None else list(names)
            infos = sorted((self.file.info(n) for n in sel), key=lambda t: t.offset)
            offs, total = {}, 0
            for t in infos:
                offs[t.name] = total
                total += (t.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
            self.nbytes = sum(t.nbytes for t in infos)
            self.arena = device.DeviceBuffer(max(total, ARENA_ALIGN))
            t0 = time.perf_counter()
            threads = min(8, os.cpu_count() or 1) if copy_threads is None else int(copy_threads)
            self._upload(infos, offs, int(staging_bytes), threads, stream)
            self.load_seconds = time.perf_counter() - t0
        except BaseException:
            self.close()
            raise
        for t in infos:
            self.weights[t.name] = DeviceWeight.view(self.arena, offs[t.name], t.nbytes, qtype=t.type_name,
                                                     shape=t.shape, name=t.name)

    def _upload(self, infos, offs, staging: int, threads: int, stream) -> None:
        from . import device
        from .streaming import StagedCopier

        cs = device.Stream() if stream is None else stream
        copier = StagedCopier(staging, threads)
        try:
            for t in infos:
                copier.copy(self.arena.ptr + offs[t.name],
                            np.frombuffer(self.file._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset), cs)
            cs.synchronize()
        finally:
            copier.close()
            if stream is None:
                cs.destroy()

    # ------------------------------------------------------------- interface
    def __getitem__(self, name: str):
        try:
            return self.weights[name]
        except KeyError as exc:
            raise TensorNotFound(name) from exc

    def __contains__(self, name: str) -> bool:
        return name in self.weights

    def names(self) -> list[str]:
        return list(self.weights)

    @property
    def load_gbs(self) -> float:
        return self.nbytes / self.load_seconds / 1e9 if self.load_seconds > 0 else float("inf")

    def close(self) -> None:
        self.weights.clear()
        if getattr(self, "arena", None) is not None:
            self.arena.free()
            self.arena = None
        if self._own_file and self.file is not None:
            self.file.close()
        self.file = None

    def __enter__(self) -> "ResidentModel":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def write_gguf(path, tensors, metadata=None, *, alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Writes a GGUF file: ``tensors`` is a list of ``(gguf_name, shape,
    type name or id, payload bytes)`` with ``shape`` row-major (it is stored
    reversed as ``ne[]``); metadata values are str, bool, int (uint64, or
    int64 when negative), float (float32) or lists of one of those. ``alignment`` is recorded as
    ``general.alignment`` (uint32) when it is not 32. Used to make synthetic
    model files; real files come from the GGUF tool chain."""
    meta = dict(metadata or {})
    if alignment != DEFAULT_ALIGNMENT:
        meta["general.alignment"] = ("u32", alignment)

    def s(text: str) -> bytes:
        b = text.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def val(v) -> tuple[int, bytes]:
        if isinstance(v, tuple) and v[0] == "u32":
            return 4, struct.pack("<I", v[1])
        if isinstance(v, bool):
            return _BOOL, struct.pack("<?", v)
        if isinstance(v, int):       # uint64 when non-negative: what both readers decode alike
            return (10, struct.pack("<Q", v)) if v >= 0 else (11, struct.pack("<q", v))
        if isinstance(v, float):
            return 6, struct.pack("<f", v)
        if isinstance(v, str):
            return _STRING, s(v)
        if isinstance(v, (list, tuple)):
            items = [val(e) for e in v]
            et = items[0][0] if items else 4
            return _ARRAY, struct.pack("<IQ", et, len(items)) + b"".join(b for _, b in items)
        raise TypeError(f"unsupported metadata value {v!r}")

    head = bytearray(GGUF_MAGIC + struct.pack("<IQQ", version, len(tensors), len(meta)))
    for k, v in meta.items():
        t, b = val(v)
        head += s(k) + struct.pack("<I", t) + b
    rel, cur = [], 0
    for name, shape, gtype, payload in tensors:
        rel.append(cur)
        cur += (len(payload) + alignment - 1) // alignment * alignment
    for (name, shape, gtype, payload), off in zip(tensors, rel):
        tid = TYPE_IDS[gtype] if isinstance(gtype, str) else int(gtype)
        ne = list(reversed([int(d) for d in shape]))
        head += s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", tid, off)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        for name, shape, gtype, payload in tensors:
            f.write(payload)
            f.write(b"\0" * ((-len(payload)) % alignment))


__all__ = [
    "GGUFFile", "ResidentModel", "TensorInfo", "GGMLType", "GGML_TYPES", "GGUFError", "TensorNotFound",
    "translate_gguf_name", "tensor_nbytes", "type_name", "write_gguf",
]
