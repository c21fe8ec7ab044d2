"""ctypes binding of libnexus_hip.so, the gfx950 decode-loop library.

This mirrors the C-ABI in include/nexus_hip.h one to one.  Device memory is
owned by a Context (nx_buf handles); numpy arrays are copied in and out with
upload()/download().  There is no CPU fallback: if the library is missing or
no gfx950 device is present, the constructors raise.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import subprocess
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
LIB_PATH = PKG_DIR / "libnexus_hip.so"
HEADER = ROOT.parent / "include" / "nexus_hip.h"
HEADERS = sorted((ROOT.parent / "include").glob("*.h"))

NX_OK = 0
STATUS = {0: "OK", 1: "INVALID", 2: "HIP", 3: "OOM", 4: "UNSUPPORTED", 5: "STATE",
          6: "NO_DEVICE", 7: "CAPACITY", 8: "CHECKSUM", 9: "IO"}


class NxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"nx error {STATUS.get(code, code)}: {msg}")
        self.code = code


def build(jobs: int = 8) -> None:
    """Compile libnexus_hip.so for gfx950 in place."""
    subprocess.run(["make", "-s", "-j", str(jobs), "-B", "-C", str(ROOT)], check=True)


class ModelConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("n_experts", C.c_int), ("top_k", C.c_int), ("max_seq", C.c_int), ("batch", C.c_int),
        ("kv_kind", C.c_int), ("rope_theta", C.c_float), ("eps", C.c_float),
        ("seed", C.c_uint64), ("norm_sigma", C.c_float), ("hot_window", C.c_int),
        ("warm_window", C.c_int), ("cool_window", C.c_int), ("kv_blocks", C.c_int),
        ("qk_norm", C.c_int),
    ]


class NxfManifest(C.Structure):
    """nx_nxf_manifest (ModelManifest, nexus/src/format/nxf.h:76-96)."""
    _fields_ = [
        ("architecture", C.c_char * 64), ("name", C.c_char * 128),
        ("num_layers", C.c_uint32), ("hidden_dim", C.c_uint32), ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("vocab_size", C.c_uint32),
        ("max_seq_len", C.c_uint32), ("rope_theta", C.c_float), ("rms_norm_eps", C.c_float),
        ("num_experts", C.c_uint32), ("num_active_experts", C.c_uint32),
        ("default_codec", C.c_uint8), ("default_group_size", C.c_uint8),
    ]


class NxfChunk(C.Structure):
    """nx_nxf_chunk (ChunkDesc, nexus/src/format/nxf.h:42-50)."""
    _fields_ = [("file_offset", C.c_uint64), ("compressed_size", C.c_uint32),
                ("decompressed_size", C.c_uint32), ("checksum", C.c_uint32),
                ("codec", C.c_uint8), ("group_size", C.c_uint8)]


class NxfTensor(C.Structure):
    """nx_nxf_tensor (TensorInfo, nexus/src/format/nxf.h:54-73)."""
    _fields_ = [("name", C.c_char_p), ("ndim", C.c_int), ("shape", C.c_int64 * 8),
                ("dtype", C.c_int), ("num_chunks", C.c_int),
                ("compressed_bytes", C.c_uint64), ("decompressed_bytes", C.c_uint64)]


_B = C.c_uint64  # nx_buf


class GpuPool(C.Structure):
    """nx_gpu_pool (ComputeDispatch::GPUBufferPool, compute_dispatch.h:137-155)."""
    _fields_ = [(n, C.c_uint64) for n in ("hidden", "residual", "norm", "q", "k", "v", "attn_out", "ffn_gate",
                                          "ffn_up", "ffn_act", "ffn_out", "logits", "token")]
_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_SIGS = {
    "nx_init": (_I, [C.POINTER(_P), _I]),
    "nx_destroy": (_I, [_P]),
    "nx_has_gpu": (_I, []),
    "nx_device_name": (_I, [_P, C.c_char_p, C.c_size_t]),
    "nx_last_error": (C.c_char_p, [_P]),
    "nx_init_error": (C.c_char_p, []),
    "nx_source_hash": (C.c_char_p, []),
    "nx_alloc": (_I, [_P, C.c_size_t, C.POINTER(_B)]),
    "nx_free": (_I, [_P, _B]),
    "nx_upload": (_I, [_P, _B, C.c_size_t, _P, C.c_size_t]),
    "nx_download": (_I, [_P, _P, _B, C.c_size_t, C.c_size_t]),
    "nx_weight_cache": (_I, [_P, _P, _P, C.c_size_t, C.POINTER(_B)]),
    "nx_get_cached_buffer": (_I, [_P, _P, C.POINTER(_B)]),
    "nx_clear_buffer_cache": (_I, [_P]),
    "nx_buffer_size": (_I, [_P, _B, C.POINTER(C.c_size_t)]),
    "nx_synchronize": (_I, [_P]),
    "nx_token_begin": (_I, [_P]),
    "nx_token_end": (_I, [_P]),
    "nx_token_flush": (_I, [_P]),
    "nx_token_resume": (_I, [_P]),
    "nx_gemm_f32": (_I, [_P, _B, _B, _B, _I, _I, _I]),
    "nx_ffn_int4_g32": (_I, [_P, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I]),
    "nx_init_gpu_pool": (_I, [_P, _I, _I, _I, _I, _I, _I, C.POINTER(GpuPool)]),
    "nx_init_kv_cache": (_I, [_P, _I, _I, _I, _I, _I, C.POINTER(_B), C.POINTER(_B), C.POINTER(_B),
                              C.POINTER(_I), C.POINTER(_I)]),
    "nx_reserve_workspace": (_I, [_P, _I, _I, _I, _I, _I, _I, _I]),
    "nx_preload_all_buffers": (_I, [_P, C.POINTER(C.c_size_t)]),
    "nx_gemv_int4_g32": (_I, [_P, _B, _B, _B, _B, _I, _I, _I]),
    "nx_gemv_int4_g32_f32": (_I, [_P, _B, _B, _B, _B, _I, _I, _I, _I]),
    "nx_unpack_int4": (_I, [_P, _B, _B, C.c_size_t]),
    "nx_gemm_int4_g32": (_I, [_P, _B, _B, _B, _B, _I, _I, _I, _I]),
    "nx_time_gemm": (_I, [_P, _B, _B, _B, _B, _I, _I, _I, _I, C.POINTER(C.c_double)]),
    "nx_quantize_int4_g32": (_I, [_P, _B, _B, _B, _I, _I]),
    "nx_rmsnorm": (_I, [_P, _B, _B, _B, _I, _F, _I]),
    "nx_rope": (_I, [_P, _B, _B, _B, _B, _I, _I, _I, _I]),
    "nx_swiglu": (_I, [_P, _B, _B, _B, _I, _I]),
    "nx_residual_add": (_I, [_P, _B, _B, _B, _I]),
    "nx_kv_append_f16": (_I, [_P, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I, _I]),
    "nx_attn_decode_paged_f16": (_I, [_P, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I, _I, _I]),
    "nx_attn_decode_paged_f16_noalloc": (_I, [_P, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I, _I, _I]),
    "nx_tq_codebooks": (_I, [_P, _P, _P, _P]),
    "nx_tq_encode": (_I, [_P, _B, _B, _B, _B, _B, _I]),
    "nx_tq_append": (_I, [_P, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I]),
    "nx_attn_decode_paged_tq": (_I, [_P, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _B, _I, _I,
                                     _I, _I, _I]),
    "nx_moe_route_topk": (_I, [_P, _B, _B, _B, _I, _I, _I]),
    "nx_moe_expert_ffn": (_I, [_P, _B, _B, _B, _B, _B, _B, _B, _B, _I, _I, _I, _I, _I, _I]),
    "nx_argmax": (_I, [_P, _B, _B, _I, _I]),
    "nx_sample": (_I, [_P, _B, _B, _I, _I, _F, _I, _F, C.c_uint64]),
    "nx_model_set_sampling": (_I, [_P, _F, _I, _F, C.c_uint64]),
    "nx_model_create": (_I, [_P, C.POINTER(ModelConfig), C.POINTER(_P)]),
    "nx_model_destroy": (_I, [_P]),
    "nx_model_prefill": (_I, [_P, _P, _I, _P]),
    "nx_model_set_prefill": (_I, [_P, _I]),
    "nx_model_get_config": (_I, [_P, C.POINTER(ModelConfig)]),
    "nx_model_context": (_P, [_P]),
    "nx_model_admit": (_I, [_P, _I, _P, _I, C.POINTER(C.c_int32)]),
    "nx_model_retire": (_I, [_P, _I]),
    "nx_model_slot_active": (_I, [_P, _I, C.POINTER(_I)]),
    "nx_sched_create": (_I, [_P, C.POINTER(_P)]),
    "nx_sched_destroy": (_I, [_P]),
    "nx_sched_submit": (_I, [_P, _P, _I, _I, _I, C.POINTER(_I)]),
    "nx_sched_step": (_I, [_P, C.POINTER(_I), C.POINTER(_I)]),
    "nx_sched_run": (_I, [_P]),
    "nx_sched_result": (_I, [_P, _I, _P, _I, C.POINTER(_I), C.POINTER(_I)]),
    "nx_model_fill_context": (_I, [_P, _I, _I]),
    "nx_model_kv_read": (_I, [_P, _I, _I, _I, _I, C.POINTER(C.c_int), _P, C.c_size_t]),
    "nx_model_kv_pages": (_I, [_P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "nx_model_pending": (_I, [_P, _P]),
    "nx_model_decode": (_I, [_P, _I, _P]),
    "nx_model_decode_forced": (_I, [_P, _P, _I, _P]),
    "nx_model_logits": (_I, [_P, _P]),
    "nx_model_position": (_I, [_P, _I, C.POINTER(_I)]),
    "nx_model_step_bytes": (_I, [_P, C.POINTER(C.c_double)]),
    "nx_model_time_ffn_gemv": (_I, [_P, _I, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "nx_time_gemv": (_I, [_P, _B, C.POINTER(_B), C.POINTER(_B), _I, _B, _I, _I, _I, _I,
                          C.POINTER(C.c_double)]),
    "nx_model_time_attention": (_I, [_P, _I, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    # include/nexus_nxf.h
    "nx_nxf_error": (C.c_char_p, []),
    "nx_nxf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "nx_nxf_close": (_I, [_P]),
    "nx_nxf_get_manifest": (_I, [_P, C.POINTER(NxfManifest)]),
    "nx_nxf_num_tensors": (_I, [_P, C.POINTER(_I)]),
    "nx_nxf_tensor_at": (_I, [_P, _I, C.POINTER(NxfTensor)]),
    "nx_nxf_find": (_I, [_P, C.c_char_p, C.POINTER(_I)]),
    "nx_nxf_chunk_at": (_I, [_P, _I, _I, C.POINTER(NxfChunk)]),
    "nx_nxf_map_chunk": (_I, [_P, _I, _I, C.POINTER(_P)]),
    "nx_nxf_unmap_chunk": (_I, [_P, _P]),
    "nx_nxf_read_chunk": (_I, [_P, _I, _I, _P]),
    "nx_nxf_verify": (_I, [_P, _P, C.POINTER(_I), C.POINTER(_I), C.POINTER(C.c_uint64)]),
    "nx_nxf_writer_create": (_I, [_P, C.c_char_p, C.POINTER(_P)]),
    "nx_nxf_writer_set_manifest": (_I, [_P, C.POINTER(NxfManifest)]),
    "nx_nxf_writer_begin_tensor": (_I, [_P, C.c_char_p, C.POINTER(C.c_int64), _I, _I]),
    "nx_nxf_writer_add_chunk": (_I, [_P, _P, C.c_size_t, _I, _I]),
    "nx_nxf_writer_end_tensor": (_I, [_P]),
    "nx_nxf_writer_finalize": (_I, [_P]),
    "nx_nxf_writer_destroy": (_I, [_P]),
    "nx_xxh32_chunks": (_I, [_P, _B, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), _I,
                             C.POINTER(C.c_uint32)]),
    "nx_time_xxh32": (_I, [_P, _B, C.c_size_t, C.c_uint32, _I, C.POINTER(C.c_double),
                           C.POINTER(C.c_uint32)]),
    "nx_model_save_nxf": (_I, [_P, C.c_char_p]),
    "nx_model_load_nxf": (_I, [_P, C.c_char_p, C.POINTER(ModelConfig), C.POINTER(_P)]),
}

_lib = None


_DEFAULT_LIB = LIB_PATH


def source_hash() -> str:
    """SHA-1 of the library's sources as the Makefile computes it: the
    contents of csrc/*.hip, *.cpp, *.h and ../include/*.h concatenated in the
    byte order of their paths relative to the package root."""
    rel = [f"csrc/{p.name}" for p in (ROOT / "csrc").iterdir() if p.suffix in (".hip", ".cpp", ".h")]
    rel += [f"../include/{p.name}" for p in (ROOT.parent / "include").glob("*.h")]
    h = hashlib.sha1()
    for r in sorted(rel):
        h.update((ROOT / r).read_bytes())
    return h.hexdigest()


def lib() -> C.CDLL:
    """Load libnexus_hip.so (raises if it has not been built, or if the
    in-tree library was built from other sources than the tree holds)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `make -C {ROOT}` "
                "(there is no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if LIB_PATH == _DEFAULT_LIB:
            built, tree = L.nx_source_hash().decode(), source_hash()
            if built != tree:
                raise RuntimeError(f"{LIB_PATH} was built from other sources (sha1 {built}) than the tree "
                                   f"holds ({tree}): rebuild it with `make -C {ROOT}`")
        _lib = L
    return _lib


def has_gpu() -> bool:
    return bool(lib().nx_has_gpu())


def tq_codebooks():
    c4 = np.empty(16, np.float32)
    b4 = np.empty(15, np.float32)
    c3 = np.empty(8, np.float32)
    b3 = np.empty(7, np.float32)
    st = lib().nx_tq_codebooks(c4.ctypes.data, b4.ctypes.data, c3.ctypes.data, b3.ctypes.data)
    if st != NX_OK:
        raise NxError(st, "nx_tq_codebooks")
    return c4, b4, c3, b3


class Context:
    """An nx_ctx on one gfx950 device."""

    def __init__(self, device: int = 0):
        L = lib()
        h = C.c_void_p()
        st = L.nx_init(C.byref(h), device)
        if st != NX_OK:
            raise NxError(st, L.nx_init_error().decode())
        self.h = h
        self.L = L
        self._bufs: dict[int, tuple] = {}

    # ------------------------------------------------------------ helpers --
    def check(self, st: int, what: str = ""):
        if st != NX_OK:
            raise NxError(st, f"{what}: {self.L.nx_last_error(self.h).decode()}")

    def close(self):
        if self.h:
            self.L.nx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        self.check(self.L.nx_device_name(self.h, buf, 256), "nx_device_name")
        return buf.value.decode()

    def alloc(self, nbytes: int) -> int:
        b = C.c_uint64()
        self.check(self.L.nx_alloc(self.h, int(nbytes), C.byref(b)), "nx_alloc")
        return b.value

    def free(self, b: int):
        self.check(self.L.nx_free(self.h, b), "nx_free")

    def upload(self, arr: np.ndarray, buf: int | None = None) -> int:
        a = np.ascontiguousarray(arr)
        if buf is None:
            buf = self.alloc(max(a.nbytes, 1))
        self.check(self.L.nx_upload(self.h, buf, 0, a.ctypes.data, a.nbytes), "nx_upload")
        return buf

    def download(self, buf: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.check(self.L.nx_download(self.h, out.ctypes.data, buf, 0, out.nbytes), "nx_download")
        return out

    def sync(self):
        self.check(self.L.nx_synchronize(self.h), "nx_synchronize")

    # ---------------------------------------------------------------- ops --
    def gemv(self, x, wq, sc, y, N, K, batch=1):
        self.check(self.L.nx_gemv_int4_g32(self.h, x, wq, sc, y, N, K, batch), "nx_gemv_int4_g32")

    def sample(self, logits, out, V, batch=1, temperature=0.7, top_k=40, top_p=0.9, seed=0):
        self.check(self.L.nx_sample(self.h, logits, out, V, batch, temperature, top_k, top_p, seed), "nx_sample")

    def gemm(self, x, wq, sc, y, M, N, K, accumulate=False):
        self.check(self.L.nx_gemm_int4_g32(self.h, x, wq, sc, y, M, N, K, int(accumulate)), "nx_gemm_int4_g32")

    def gemv_f32(self, x, wq, sc, y, N, K, batch=1, accumulate=False):
        self.check(self.L.nx_gemv_int4_g32_f32(self.h, x, wq, sc, y, N, K, batch, int(accumulate)),
                   "nx_gemv_int4_g32_f32")


class Model:
    """An nx_model (the resident decode runner)."""

    def __init__(self, ctx: Context, **cfg):
        self.ctx = ctx
        self.cfg = ModelConfig(**cfg)
        h = C.c_void_p()
        ctx.check(ctx.L.nx_model_create(ctx.h, C.byref(self.cfg), C.byref(h)), "nx_model_create")
        self.h = h

    @classmethod
    def load_nxf(cls, ctx: Context, path, batch=1, max_seq=128, kv_kind=0, seed=0x5EED,
                 hot_window=0, warm_window=0, cool_window=0) -> "Model":
        """A model from an NXF file (nx_model_load_nxf): dimensions from the
        file, every chunk verified on the GPU; batch, max_seq, kv_kind,
        hot_window, warm_window, cool_window and seed are the caller's."""
        self = cls.__new__(cls)
        self.ctx = ctx
        run = ModelConfig(batch=batch, max_seq=max_seq, kv_kind=kv_kind, seed=seed, hot_window=hot_window,
                          warm_window=warm_window, cool_window=cool_window)
        h = C.c_void_p()
        ctx.check(ctx.L.nx_model_load_nxf(ctx.h, str(path).encode(), C.byref(run), C.byref(h)),
                  "nx_model_load_nxf")
        self.h = h
        # the dimensions the library read from the file
        from .nxf import NXFReader
        r = NXFReader.open(path)
        m = r.manifest()
        w1 = r.get_tensor("layers.0.feed_forward.experts.w1.weight" if m.num_experts
                          else "layers.0.feed_forward.w1.weight")
        qk = any(t.name == "layers.0.attn_q_norm.weight" for t in r.tensors())
        r.close()
        self.cfg = ModelConfig(
            n_layers=m.num_layers, d_model=m.hidden_dim, n_heads=m.num_heads,
            n_kv_heads=m.num_kv_heads, head_dim=m.head_dim, ffn=w1.shape[-1], vocab=m.vocab_size,
            n_experts=m.num_experts,
            top_k=(min(10, m.num_experts) if m.num_experts and not m.num_active_experts else m.num_active_experts),
            max_seq=max_seq, batch=batch,
            kv_kind=kv_kind, rope_theta=m.rope_theta, eps=m.rms_norm_eps, seed=seed,
            hot_window=hot_window, warm_window=warm_window, cool_window=cool_window, qk_norm=int(qk))
        return self

    def save_nxf(self, path):
        """Write the model as an NXF file (nx_model_save_nxf)."""
        self.ctx.check(self.ctx.L.nx_model_save_nxf(self.h, str(path).encode()), "nx_model_save_nxf")

    def close(self):
        if self.h:
            self.ctx.L.nx_model_destroy(self.h)
            self.h = None

    def prefill(self, prompt: np.ndarray) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32).reshape(self.cfg.batch, -1)
        nxt = np.empty(self.cfg.batch, np.int32)
        self.ctx.check(self.ctx.L.nx_model_prefill(self.h, p.ctypes.data, p.shape[1], nxt.ctypes.data),
                       "nx_model_prefill")
        return nxt

    def set_sampling(self, temperature=0.7, top_k=40, top_p=0.9, seed=0):
        """SamplingParams of the decode loop; temperature <= 0 is greedy."""
        self.ctx.check(self.ctx.L.nx_model_set_sampling(self.h, temperature, top_k, top_p, seed),
                       "nx_model_set_sampling")

    def set_prefill(self, batched: bool):
        """Batched GEMM prefill (default) or one decode step per prompt token."""
        self.ctx.check(self.ctx.L.nx_model_set_prefill(self.h, int(batched)), "nx_model_set_prefill")

    def fill_context(self, ctx_len: int, n_outlier: int = 0):
        self.ctx.check(self.ctx.L.nx_model_fill_context(self.h, ctx_len, n_outlier),
                       "nx_model_fill_context")

    def kv_read(self, layer: int, b: int, pos: int, kv: int):
        """(form, stored bytes) of one position, all kv heads (nx_model_kv_read):
        form 0 fp16, form 1 TurboQuant (58 bytes per head), form 2 Cool (50),
        form 3 evicted (no bytes)."""
        cap = max(58, 2 * self.cfg.head_dim) * self.cfg.n_kv_heads
        out = np.zeros(cap, np.uint8)
        form = C.c_int()
        self.ctx.check(self.ctx.L.nx_model_kv_read(self.h, layer, b, pos, kv, C.byref(form), out.ctypes.data, cap),
                       "nx_model_kv_read")
        n = {0: 2 * self.cfg.head_dim, 1: 58, 2: 50, 3: 0}[form.value] * self.cfg.n_kv_heads
        return form.value, out[:n]

    def kv_pages(self):
        """(pages of the KV pool, free pages) (nx_model_kv_pages)."""
        total, free = C.c_int(), C.c_int()
        self.ctx.check(self.ctx.L.nx_model_kv_pages(self.h, C.byref(total), C.byref(free)), "nx_model_kv_pages")
        return total.value, free.value

    def pending(self) -> np.ndarray:
        t = np.empty(self.cfg.batch, np.int32)
        self.ctx.check(self.ctx.L.nx_model_pending(self.h, t.ctypes.data), "nx_model_pending")
        return t

    def decode(self, steps: int) -> np.ndarray:
        out = np.empty((self.cfg.batch, steps), np.int32)
        self.ctx.check(self.ctx.L.nx_model_decode(self.h, steps, out.ctypes.data), "nx_model_decode")
        return out

    def decode_forced(self, tokens) -> np.ndarray:
        """Teacher-forced steps (nx_model_decode_forced): sequence b consumes
        tokens[b][s] at step s; returns the logits [batch][steps][vocab]."""
        t = np.ascontiguousarray(tokens, np.int32)
        if t.ndim != 2 or t.shape[0] != self.cfg.batch:
            raise ValueError("tokens must be [batch][steps]")
        out = np.empty((self.cfg.batch, t.shape[1], self.cfg.vocab), np.float32)
        self.ctx.check(self.ctx.L.nx_model_decode_forced(self.h, t.ctypes.data, t.shape[1], out.ctypes.data),
                       "nx_model_decode_forced")
        return out

    def decode_untimed(self, steps: int):
        self.ctx.check(self.ctx.L.nx_model_decode(self.h, steps, None), "nx_model_decode")

    def admit(self, slot: int, prompt) -> int:
        """Sequence `slot` starts over with this prompt (nx_model_admit);
        returns its first generated token."""
        p = np.ascontiguousarray(prompt, np.int32).reshape(-1)
        nxt = C.c_int32()
        self.ctx.check(self.ctx.L.nx_model_admit(self.h, slot, p.ctypes.data, p.size, C.byref(nxt)),
                       "nx_model_admit")
        return int(nxt.value)

    def retire(self, slot: int):
        self.ctx.check(self.ctx.L.nx_model_retire(self.h, slot), "nx_model_retire")

    def slot_active(self, slot: int) -> bool:
        a = C.c_int()
        self.ctx.check(self.ctx.L.nx_model_slot_active(self.h, slot, C.byref(a)), "nx_model_slot_active")
        return bool(a.value)

    def logits(self) -> np.ndarray:
        out = np.empty((self.cfg.batch, self.cfg.vocab), np.float32)
        self.ctx.check(self.ctx.L.nx_model_logits(self.h, out.ctypes.data), "nx_model_logits")
        return out

    def position(self, b: int = 0) -> int:
        p = C.c_int()
        self.ctx.check(self.ctx.L.nx_model_position(self.h, b, C.byref(p)), "nx_model_position")
        return p.value

    def step_bytes(self) -> float:
        v = C.c_double()
        self.ctx.check(self.ctx.L.nx_model_step_bytes(self.h, C.byref(v)), "nx_model_step_bytes")
        return v.value

    def time_ffn_gemv(self, iters: int = 50):
        ms, nb = C.c_double(), C.c_double()
        self.ctx.check(self.ctx.L.nx_model_time_ffn_gemv(self.h, iters, C.byref(ms), C.byref(nb)),
                       "nx_model_time_ffn_gemv")
        return ms.value, nb.value

    def time_attention(self, iters: int = 50):
        ms, nb = C.c_double(), C.c_double()
        self.ctx.check(self.ctx.L.nx_model_time_attention(self.h, iters, C.byref(ms), C.byref(nb)),
                       "nx_model_time_attention")
        return ms.value, nb.value


class Scheduler:
    """nx_sched: requests admitted into a model's free slots in arrival
    order, decoded together, retired when complete."""

    def __init__(self, model: Model):
        self.model = model
        self.L = model.ctx.L
        h = C.c_void_p()
        model.ctx.check(self.L.nx_sched_create(model.h, C.byref(h)), "nx_sched_create")
        self.h = h

    def submit(self, prompt, max_new: int, stop: int = -1) -> int:
        p = np.ascontiguousarray(prompt, np.int32).reshape(-1)
        rid = C.c_int()
        self.model.ctx.check(self.L.nx_sched_submit(self.h, p.ctypes.data, p.size, max_new, stop, C.byref(rid)),
                             "nx_sched_submit")
        return int(rid.value)

    def step(self):
        a, w = C.c_int(), C.c_int()
        self.model.ctx.check(self.L.nx_sched_step(self.h, C.byref(a), C.byref(w)), "nx_sched_step")
        return int(a.value), int(w.value)

    def run(self):
        self.model.ctx.check(self.L.nx_sched_run(self.h), "nx_sched_run")

    def result(self, rid: int):
        n, done = C.c_int(), C.c_int()
        self.model.ctx.check(self.L.nx_sched_result(self.h, rid, None, 0, C.byref(n), C.byref(done)), "result")
        out = np.empty(n.value, np.int32)
        self.model.ctx.check(self.L.nx_sched_result(self.h, rid, out.ctypes.data, n.value, C.byref(n),
                                                    C.byref(done)), "nx_sched_result")
        return out, bool(done.value)

    def close(self):
        if self.h:
            self.L.nx_sched_destroy(self.h)
            self.h = None
