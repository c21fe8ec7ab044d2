"""NXF file cases shared by the CPU and GPU format tests: tensors as plain
Python data, written either by the reference's NXFWriter (the checker built
in oracle/_ref) or by this library's writer."""
import ctypes as C
from pathlib import Path

import numpy as np

import oracle

DT_F32, DT_F16, DT_I4 = 0, 1, 4
CODEC_FP32, CODEC_FP16, CODEC_INT4 = 0, 1, 4

# The manifest of nexus/tests/test_nxf_format.cpp:21-36.
REF_TEST_MANIFEST = dict(architecture="llama", name="test-model-7b", num_layers=2, hidden_dim=128,
                         num_heads=4, num_kv_heads=4, head_dim=32, vocab_size=256, max_seq_len=512,
                         rope_theta=10000.0, rms_norm_eps=1e-5, num_experts=0,
                         num_active_experts=0, default_codec=CODEC_FP16, default_group_size=128)


def ref_test_tensors():
    """The tensors of nexus/tests/test_nxf_format.cpp:40-50: wq [128,128]
    F32 with data[i] = i / 1000, a norm of 128 ones."""
    wq = (np.arange(128 * 128, dtype=np.float32) / np.float32(1000.0)).astype(np.float32)
    return [("layers.0.attention.wq.weight", [128, 128], DT_F32, [(wq.tobytes(), CODEC_FP32, 128)]),
            ("layers.0.attention_norm.weight", [128], DT_F32,
             [(np.ones(128, np.float32).tobytes(), CODEC_FP32, 128)])]


def ragged_tensors(seed=7):
    """An int4-g32 tensor (codes chunks + fp16 scale sidecar), ragged chunk
    sizes (1, 5, 15, 16, 17, 4095 bytes ...), a chunk above 1 MiB, a tensor
    with no chunks and a 3-D shape."""
    rng = np.random.default_rng(seed)
    rnd = lambda n: rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    t = [("layers.0.feed_forward.w1.weight", [64, 96], DT_I4,
          [(rnd(48 * 32), CODEC_INT4, 32), (rnd(48 * 32), CODEC_INT4, 32),
           (rnd(96 * 2 * 2), CODEC_FP16, 32)]),
         ("ragged", [7], DT_F16, [(rnd(n), CODEC_FP16, 0) for n in (1, 5, 15, 16, 17, 31, 64, 4095, 16384, 16385)]),
         ("big", [1 << 20], DT_I4, [(rnd((1 << 20) + 7), CODEC_INT4, 32)]),
         ("empty", [0], DT_F32, []),
         ("experts", [4, 32, 8], DT_I4, [(rnd(4 * 8 * 16), CODEC_INT4, 32), (rnd(4 * 8 * 2), CODEC_FP16, 32)])]
    return t


NXF_CASES = {"reference_test": ref_test_tensors, "ragged": ragged_tensors,
             "control_name": ref_test_tensors}
# The manifest of each case: the reference test's, except that "control_name"
# names the model with control bytes, which the reference's JSON escaper
# (format/nxf_writer.cpp:76-89) writes raw (only ", \\, \\n and \\t are escaped).
CONTROL_NAME = "ctl\r\x01\x1f\x7f\n\tend"
CASE_MANIFEST = {"reference_test": REF_TEST_MANIFEST, "ragged": REF_TEST_MANIFEST,
                 "control_name": dict(REF_TEST_MANIFEST, name=CONTROL_NAME)}
GOLDEN = Path(__file__).resolve().parent / "golden" / "nxf_ref_files.npz"


def ref_file_bytes(case: str) -> bytes:
    """The bytes the reference's NXFWriter writes for a case of NXF_CASES
    with its CASE_MANIFEST, rebuilt from the fixture golden/nxf_ref_files.npz
    (the reference writer's file with the payload regions zeroed, and each
    chunk's offset): the case's chunk bytes are put back at those offsets."""
    with np.load(GOLDEN) as z:
        data = z[f"{case}_masked"].copy()
        offs = z[f"{case}_offsets"]
    chunks = [b for _, _, _, ch in NXF_CASES[case]() for b, _, _ in ch]
    assert len(chunks) == len(offs)
    for off, b in zip(offs, chunks):
        data[int(off):int(off) + len(b)] = np.frombuffer(b, np.uint8)
    return data.tobytes()


class _Manifest(C.Structure):
    _fields_ = [
        ("architecture", C.c_char * 64), ("name", C.c_char * 128),
        ("num_layers", C.c_uint32), ("hidden_dim", C.c_uint32), ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("vocab_size", C.c_uint32),
        ("max_seq_len", C.c_uint32), ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float),
        ("num_experts", C.c_uint32), ("num_active_experts", C.c_uint32),
        ("default_codec", C.c_uint8), ("default_group_size", C.c_uint8),
    ]


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ndim", C.c_int), ("shape", C.POINTER(C.c_int64)),
                ("dtype", C.c_int), ("nchunks", C.c_int), ("data", C.POINTER(C.c_void_p)),
                ("sizes", C.POINTER(C.c_uint64)), ("codecs", C.POINTER(C.c_int)),
                ("groups", C.POINTER(C.c_int))]


def ref_write(path, manifest: dict, tensors) -> None:
    """Write a file with the reference's NXFWriter (oracle/_ref)."""
    R = oracle.ref()
    m = _Manifest()
    for k, v in manifest.items():
        setattr(m, k, v.encode() if isinstance(v, str) else v)
    keep = []
    arr = (_Tensor * max(len(tensors), 1))()
    for i, (name, shape, dtype, chunks) in enumerate(tensors):
        shp = (C.c_int64 * max(len(shape), 1))(*shape)
        bufs = [C.create_string_buffer(b, len(b)) for b, _, _ in chunks]
        data = (C.c_void_p * max(len(chunks), 1))(*[C.cast(b, C.c_void_p) for b in bufs])
        sizes = (C.c_uint64 * max(len(chunks), 1))(*[len(b) for b, _, _ in chunks])
        codecs = (C.c_int * max(len(chunks), 1))(*[c for _, c, _ in chunks])
        groups = (C.c_int * max(len(chunks), 1))(*[g for _, _, g in chunks])
        keep += [shp, bufs, data, sizes, codecs, groups]
        arr[i] = _Tensor(name.encode(), len(shape), shp, dtype, len(chunks), data, sizes, codecs, groups)
    assert R.ref_nxf_write(str(path).encode(), C.byref(m), arr, len(tensors)) == 0


def ref_summary(path) -> str:
    R = oracle.ref()
    buf = C.create_string_buffer(1 << 20)
    n = R.ref_nxf_summary(str(path).encode(), buf, len(buf))
    assert 0 <= n < len(buf), n
    return buf.value.decode()


def ref_chunk(path, name, j) -> bytes:
    R = oracle.ref()
    buf = C.create_string_buffer(4 << 20)
    n = R.ref_nxf_chunk_bytes(str(path).encode(), name.encode(), j, buf, len(buf))
    assert n >= 0
    return buf.raw[:n]


def our_summary(reader) -> str:
    """The same text as ref_summary, from this library's reader."""
    m = reader.manifest()
    f32 = lambda x: float(np.float32(x))
    s = "manifest %s|%s|%u %u %u %u %u %u %u|%.9g %.9g|%u %u|%u %u\n" % (
        m.architecture, m.name, m.num_layers, m.hidden_dim, m.num_heads, m.num_kv_heads, m.head_dim,
        m.vocab_size, m.max_seq_len, f32(m.rope_theta), f32(m.rms_norm_eps), m.num_experts,
        m.num_active_experts, m.default_codec, m.default_group_size)
    for t in sorted(reader.tensors(), key=lambda t: t.name):
        s += "tensor " + t.name + " shape" + "".join(" %d" % d for d in t.shape) + " dtype %d\n" % t.dtype
        for c in t.chunks:
            s += "  chunk %d %d %d %08x %d %d\n" % (c.file_offset, c.compressed_size, c.decompressed_size,
                                                    c.checksum, c.codec, c.group_size)
    return s


def our_write(ctx, path, manifest: dict, tensors) -> None:
    from nexus_amd.nxf import ModelManifest, NXFWriter
    w = NXFWriter.create(ctx, path)
    w.set_manifest(ModelManifest(**manifest))
    for name, shape, dtype, chunks in tensors:
        w.begin_tensor(name, shape, dtype)
        for b, codec, g in chunks:
            w.add_chunk(b, codec, g)
        w.end_tensor()
    w.finalize()
