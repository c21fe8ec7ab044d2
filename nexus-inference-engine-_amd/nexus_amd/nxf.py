"""NXF files through libnexus_hip.so: NXFReader / NXFWriter with the
reference's interface (nexus/src/format/nxf.h:100-190) over the C-ABI in
include/nexus_nxf.h.

Differences from the reference, as in the C-ABI: errors raise NxError (the
reference returns nullptr / prints), chunk checksums are computed on the GPU
by the writer (so NXFWriter.create takes a Context) and verified on the GPU
by verify() and Model.load_nxf; map_chunk returns a read-only memoryview of
the private mapping.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass, field

import numpy as np

from . import NX_OK, Context, NxError, NxfChunk, NxfManifest, NxfTensor, lib


class Codec(enum.IntEnum):
    """core/config.h:21-36."""
    FP32 = 0
    FP16 = 1
    BF16 = 2
    INT8 = 3
    INT4 = 4
    GPTQ = 5
    AWQ = 6
    QUIP3 = 7
    AQLM2 = 8
    ANS = 9
    TURBO_Q = 10
    Q3K = 11
    Q4K = 12
    Q2K = 13


class DType(enum.IntEnum):
    """core/config.h:39-46."""
    F32 = 0
    F16 = 1
    BF16 = 2
    I8 = 3
    I4 = 4
    I2 = 5


CHUNK_ALIGNMENT = 16384  # core/config.h:10-11
NXF_MAGIC = 0x3146584E   # "NXF1", core/config.h:17
NXF_VERSION = 1


@dataclass
class ChunkDesc:
    file_offset: int
    compressed_size: int
    decompressed_size: int
    checksum: int
    codec: int
    group_size: int


@dataclass
class TensorInfo:
    name: str
    shape: list
    dtype: int
    chunks: list = field(default_factory=list)

    def compressed_bytes(self) -> int:
        return sum(c.compressed_size for c in self.chunks)

    def decompressed_bytes(self) -> int:
        return sum(c.decompressed_size for c in self.chunks)


@dataclass
class ModelManifest:
    architecture: str = ""
    name: str = ""
    num_layers: int = 0
    hidden_dim: int = 0
    num_heads: int = 0
    num_kv_heads: int = 0
    head_dim: int = 0
    vocab_size: int = 0
    max_seq_len: int = 0
    rope_theta: float = 0.0
    rms_norm_eps: float = 0.0
    num_experts: int = 0
    num_active_experts: int = 0
    default_codec: int = 0
    default_group_size: int = 0

    def to_c(self) -> NxfManifest:
        m = NxfManifest()
        for k in self.__dataclass_fields__:
            v = getattr(self, k)
            setattr(m, k, v.encode() if isinstance(v, str) else v)
        return m

    @classmethod
    def from_c(cls, m: NxfManifest) -> "ModelManifest":
        out = cls()
        for k in cls.__dataclass_fields__:
            v = getattr(m, k)
            setattr(out, k, v.decode() if isinstance(v, bytes) else v)
        return out


def _check(st: int, what: str):
    if st != NX_OK:
        raise NxError(st, f"{what}: {lib().nx_nxf_error().decode()}")


class NXFReader:
    """NXFReader (nxf_reader.cpp): header, manifest and tensor index on
    open; tensor data on demand."""

    def __init__(self, handle):
        self.h = handle
        self._maps = {}

    @classmethod
    def open(cls, path) -> "NXFReader":
        h = C.c_void_p()
        _check(lib().nx_nxf_open(str(path).encode(), C.byref(h)), f"open {path}")
        return cls(h)

    def close(self):
        if self.h:
            lib().nx_nxf_close(self.h)
            self.h = None
            self._maps.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def manifest(self) -> ModelManifest:
        m = NxfManifest()
        _check(lib().nx_nxf_get_manifest(self.h, C.byref(m)), "manifest")
        return ModelManifest.from_c(m)

    def _count(self) -> int:
        n = C.c_int()
        _check(lib().nx_nxf_num_tensors(self.h, C.byref(n)), "num_tensors")
        return n.value

    def _info(self, i: int) -> TensorInfo:
        t = NxfTensor()
        _check(lib().nx_nxf_tensor_at(self.h, i, C.byref(t)), "tensor_at")
        chunks = []
        for j in range(t.num_chunks):
            c = NxfChunk()
            _check(lib().nx_nxf_chunk_at(self.h, i, j, C.byref(c)), "chunk_at")
            chunks.append(ChunkDesc(c.file_offset, c.compressed_size, c.decompressed_size,
                                    c.checksum, c.codec, c.group_size))
        info = TensorInfo(t.name.decode(), [t.shape[d] for d in range(t.ndim)], t.dtype, chunks)
        info._index = i
        return info

    def get_tensor(self, name: str) -> TensorInfo | None:
        i = C.c_int()
        _check(lib().nx_nxf_find(self.h, name.encode(), C.byref(i)), "find")
        return None if i.value < 0 else self._info(i.value)

    def tensor_names(self) -> list:
        return [self._info(i).name for i in range(self._count())]

    def tensors(self) -> list:
        """Every TensorInfo in index order."""
        return [self._info(i) for i in range(self._count())]

    def read_chunk(self, info: TensorInfo, j: int) -> bytes:
        buf = C.create_string_buffer(max(info.chunks[j].compressed_size, 1))
        _check(lib().nx_nxf_read_chunk(self.h, info._index, j, buf), "read_chunk")
        return buf.raw[:info.chunks[j].compressed_size]

    def map_chunk(self, info: TensorInfo, j: int) -> memoryview:
        p = C.c_void_p()
        _check(lib().nx_nxf_map_chunk(self.h, info._index, j, C.byref(p)), "map_chunk")
        n = info.chunks[j].compressed_size
        view = memoryview((C.c_uint8 * n).from_address(p.value)).cast("B").toreadonly()
        self._maps[id(view)] = p.value
        return view

    def unmap_chunk(self, view: memoryview):
        p = self._maps.pop(id(view), None)
        if p is None:
            raise NxError(1, "unmap_chunk: view was not mapped by this reader")
        view.release()
        _check(lib().nx_nxf_unmap_chunk(self.h, C.c_void_p(p)), "unmap_chunk")

    def verify(self, ctx: Context):
        """Verify every chunk's checksum on the GPU; returns the bytes
        verified, raises NxError (CHECKSUM) naming the first bad chunk."""
        bt, bc, nb = C.c_int(), C.c_int(), C.c_uint64()
        st = lib().nx_nxf_verify(ctx.h, self.h, C.byref(bt), C.byref(bc), C.byref(nb))
        if st != NX_OK:
            err = NxError(st, lib().nx_nxf_error().decode())
            err.bad = (bt.value, bc.value)
            raise err
        return nb.value


class NXFWriter:
    """NXFWriter (nxf_writer.cpp): chunks are written at 16 KiB boundaries,
    the tensor index, manifest and header at finalize()."""

    def __init__(self, handle):
        self.h = handle

    @classmethod
    def create(cls, ctx: Context, path) -> "NXFWriter":
        h = C.c_void_p()
        _check(lib().nx_nxf_writer_create(ctx.h, str(path).encode(), C.byref(h)), f"create {path}")
        return cls(h)

    def set_manifest(self, m: ModelManifest):
        _check(lib().nx_nxf_writer_set_manifest(self.h, C.byref(m.to_c())), "set_manifest")

    def begin_tensor(self, name: str, shape, dtype):
        arr = (C.c_int64 * max(len(shape), 1))(*[int(s) for s in shape])
        _check(lib().nx_nxf_writer_begin_tensor(self.h, name.encode(), arr, len(shape), int(dtype)),
               "begin_tensor")

    def add_chunk(self, data, codec, group_size: int = 128):
        b = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray)
                                 else data).view(np.uint8)
        _check(lib().nx_nxf_writer_add_chunk(self.h, b.ctypes.data if b.size else None, b.size,
                                             int(codec), int(group_size)), "add_chunk")

    def end_tensor(self):
        _check(lib().nx_nxf_writer_end_tensor(self.h), "end_tensor")

    def finalize(self):
        h, self.h = self.h, None
        _check(lib().nx_nxf_writer_finalize(h), "finalize")

    def __del__(self):
        if getattr(self, "h", None):
            lib().nx_nxf_writer_destroy(self.h)
            self.h = None


def xxh32_chunks(ctx: Context, buf: int, offsets, sizes) -> np.ndarray:
    """XXH32 (seed 0) of byte ranges of a device buffer, on the GPU."""
    off = np.ascontiguousarray(offsets, np.uint64)
    sz = np.ascontiguousarray(sizes, np.uint32)
    out = np.zeros(len(off), np.uint32)
    ctx.check(ctx.L.nx_xxh32_chunks(ctx.h, buf, off.ctypes.data_as(C.POINTER(C.c_uint64)),
                                    sz.ctypes.data_as(C.POINTER(C.c_uint32)), len(off),
                                    out.ctypes.data_as(C.POINTER(C.c_uint32))), "nx_xxh32_chunks")
    return out


def time_xxh32(ctx: Context, buf: int, nbytes: int, chunk_bytes: int, iters: int = 20):
    """(average ms per launch, hashes) of hashing nbytes as consecutive chunks."""
    n = (nbytes + chunk_bytes - 1) // chunk_bytes
    out = np.zeros(n, np.uint32)
    ms = C.c_double()
    ctx.check(ctx.L.nx_time_xxh32(ctx.h, buf, nbytes, chunk_bytes, iters, C.byref(ms),
                                  out.ctypes.data_as(C.POINTER(C.c_uint32))), "nx_time_xxh32")
    return ms.value, out
