"""CPU oracle for the NEXUS decode loop -- test infrastructure only.

Only the test suite, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package; it is the checker, never the product.

``lib`` is the C restatement (``liboracle.so``, built by ``make -C oracle``).
``ref()`` returns the reference checker compiled in place from the reference
sources (``oracle/_ref/libnexus_ref.so``) or None where it was not built.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libnexus_ref.so"

_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")


class Cfg(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("d_model", C.c_int), ("n_heads", C.c_int),
        ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int),
        ("n_experts", C.c_int), ("top_k", C.c_int), ("max_seq", C.c_int), ("batch", C.c_int),
        ("kv_kind", C.c_int), ("rope_theta", C.c_float), ("eps", C.c_float),
        ("seed", C.c_uint64), ("norm_sigma", C.c_float), ("hot_window", C.c_int),
        ("warm_window", C.c_int), ("cool_window", C.c_int), ("kv_blocks", C.c_int),
        ("qk_norm", C.c_int),
    ]


def build() -> None:
    """Compile liboracle.so (and the reference checker when the sources exist)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "all"], check=True)
    if Path(os.environ.get("NX_REFERENCE_SRC", "/root/reference/nexus/src")).is_dir():
        subprocess.run(["make", "-s", "-C", str(HERE), "-B", "ref"], check=True)


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    L = C.CDLL(str(LIB_PATH))
    sig = {
        "nxo_rand_u64": (C.c_uint64, [C.c_uint64, C.c_uint32, C.c_uint64]),
        "nxo_normal_k": (C.c_float, [C.c_double]),
        "nxo_gen_normal": (None, [_f32p, C.c_size_t, C.c_uint64, C.c_uint32, C.c_float]),
        "nxo_gen_tokens": (None, [_i32p, C.c_int, C.c_uint64, C.c_uint32, C.c_int]),
        "nxo_shuffle_perm": (None, [_i32p, C.c_int, C.c_uint64, C.c_uint32]),
        "nxo_f32_to_f16": (C.c_uint16, [C.c_float]),
        "nxo_f16_to_f32": (C.c_float, [C.c_uint16]),
        "nxo_f32_to_f16_trunc": (C.c_uint16, [C.c_float]),
        "nxo_f16_to_f32_ref": (C.c_float, [C.c_uint16]),
        "nxo_f32_to_f16_array": (None, [_f32p, _u16p, C.c_size_t]),
        "nxo_quantize_int4_g32": (None, [_f32p, C.c_int, C.c_int, _u8p, _u16p]),
        "nxo_unpack_int4": (None, [_u8p, C.c_size_t, _u8p]),
        "nxo_gen_quant_rows": (None, [C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_uint32, C.c_double,
                                      _u8p, _u16p]),
        "nxo_dequant_int4_g32": (None, [_u8p, _u16p, C.c_int, C.c_int, _f32p]),
        "nxo_gemv_int4_g32": (None, [_u8p, _u16p, _f32p, C.c_int, C.c_int, C.c_int, _f32p]),
        "nxo_rmsnorm": (None, [_f32p, C.c_void_p, C.c_int, C.c_float, _f32p]),
        "nxo_xxh32": (C.c_uint32, [C.c_void_p, C.c_size_t, C.c_uint32]),
        "nxo_mt19937": (None, [C.c_uint32, C.c_int, np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")]),
        "nxo_canonical_f32": (C.c_float, [C.c_uint32]),
        "nxo_sample": (C.c_int, [_f32p, C.c_int, C.c_float, C.c_int, C.c_float, C.c_float]),
        "nxo_rope_table": (None, [C.c_int, C.c_int, C.c_double, _f32p, _f32p]),
        "nxo_rope": (None, [_f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]),
        "nxo_head_rmsnorm": (None, [_f32p, C.c_int, C.c_int, C.c_void_p, C.c_float]),
        "nxo_swiglu": (None, [_f32p, _f32p, C.c_int, _f32p]),
        "nxo_argmax": (C.c_int, [_f32p, C.c_int]),
        "nxo_kv_append_f16": (None, [_f32p, _f32p, _u16p, _u16p, _i32p, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_int]),
        "nxo_attn_decode_paged_f16": (None, [_f32p, _u16p, _u16p, _i32p, C.c_int, _i32p, C.c_int,
                                             C.c_int, C.c_int, C.c_int, _f32p]),
        "nxo_attn_decode_contig": (None, [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                          _f32p]),
        "nxo_tq_codebook": (None, [C.c_int, C.c_int, _f32p, _f32p]),
        "nxo_tq_encode_scalar": (C.c_uint8, [C.c_float, _f32p, C.c_int]),
        "nxo_pack_codes": (None, [_u8p, _u8p, C.c_int, C.c_int]),
        "nxo_unpack_codes": (None, [_u8p, _u8p, C.c_int, C.c_int]),
        "nxo_tq_signs": (None, [_f32p, C.c_uint64, C.c_uint32]),
        "nxo_tq_sumsq": (C.c_float, [_f32p]),
        "nxo_fwht128": (None, [_f32p]),
        "nxo_tq_encode": (None, [_f32p, C.c_int, _f32p, _f32p, _f32p, _u8p, _u8p, _u16p, _u8p]),
        "nxo_tq_decode": (None, [_u8p, _u8p, _u16p, C.c_int, _f32p, _f32p, _f32p, _f32p]),
        "nxo_tq_append": (None, [_f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, _f32p, _u8p, _u8p,
                                 _u16p, _u8p, _u8p, _u16p, _i32p, C.c_int, C.c_int, C.c_int]),
        "nxo_attn_decode_paged_tq": (None, [_f32p, _u8p, _u8p, _u16p, _u8p, _u8p, _u16p, _f32p,
                                            _f32p, _f32p, _f32p, _i32p, C.c_int, _i32p, C.c_int,
                                            C.c_int, C.c_int, _f32p]),
        "nxo_tiered_append": (None, [_f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, _f32p, _u16p, _u16p,
                                     _u8p, _u8p, _u16p, _u8p, _u8p, _u16p, _i32p, C.c_int, C.c_int,
                                     C.c_int]),
        "nxo_tiered_cold": (C.c_int, [C.c_int, C.c_int]),
        "nxo_tiered_cool": (C.c_int, [C.c_int, C.c_int, C.c_int]),
        "nxo_tiered_evict": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int]),
        "nxo_attn_decode_tiered_evict": (None, [_f32p, _u16p, _u16p, _u8p, _u8p, _u16p, _u8p, _u8p, _u16p, _u8p,
                                                _u16p, _u8p, _u16p, _f32p, _f32p, _f32p, _f32p, _i32p, C.c_int,
                                                _i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                                _f32p]),
        "nxo_cool_encode": (None, [_f32p, C.c_int, _f32p, _f32p, _u8p, _u16p]),
        "nxo_cool_decode": (None, [_u8p, _u16p, C.c_int, _f32p, _f32p, _f32p]),
        "nxo_tq_to_cool": (None, [_u8p, _u8p, _u16p, C.c_int, _f32p, _f32p, _f32p, _f32p, _u8p, _u16p]),
        "nxo_tiered_append_cool": (None, [C.c_int, _f32p, _f32p, _f32p, _f32p, _f32p, _u8p, _u8p, _u16p, _u8p,
                                          _u8p, _u16p, _u8p, _u16p, _u8p, _u16p, _i32p, C.c_int, C.c_int,
                                          C.c_int]),
        "nxo_attn_decode_tiered_cool": (None, [_f32p, _u16p, _u16p, _u8p, _u8p, _u16p, _u8p, _u8p, _u16p, _u8p,
                                               _u16p, _u8p, _u16p, _f32p, _f32p, _f32p, _f32p, _i32p, C.c_int,
                                               _i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _f32p]),
        "nxo_attn_decode_tiered": (None, [_f32p, _u16p, _u16p, _u8p, _u8p, _u16p, _u8p, _u8p, _u16p,
                                          _f32p, _f32p, _f32p, _f32p, _i32p, C.c_int, _i32p, C.c_int,
                                          C.c_int, C.c_int, C.c_int, _f32p]),
        "nxo_moe_route": (None, [_f32p, C.c_int, C.c_int, _i32p, _f32p]),
        "nxo_model_create": (C.c_void_p, [C.POINTER(Cfg)]),
        "nxo_model_free": (None, [C.c_void_p]),
        "nxo_model_forward": (None, [C.c_void_p, _i32p, _f32p]),
        "nxo_model_forward_timed": (None, [C.c_void_p, _i32p, _f32p, C.POINTER(C.c_double),
                                           C.POINTER(C.c_double)]),
        "nxo_model_generate": (None, [C.c_void_p, _i32p, C.c_int, C.c_int, _i32p, _f32p]),
        "nxo_model_fill_context": (None, [C.c_void_p, C.c_int, C.c_int]),
        "nxo_model_kv_read": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _u8p]),
        "nxo_model_position": (C.c_int, [C.c_void_p, C.c_int]),
        "nxo_num_threads": (C.c_int, []),
        "nxo_set_num_threads": (None, [C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


lib = _load()

_ref_lib = None


def ref():
    """The reference checker library, or None where it is not built."""
    global _ref_lib
    if _ref_lib is None and REF_PATH.exists():
        R = C.CDLL(str(REF_PATH))
        R.ref_tq_codebook.restype = C.c_int
        R.ref_tq_codebook.argtypes = [C.c_int, C.c_int, _f32p, _f32p]
        R.ref_tq_encode_scalar.argtypes = [C.c_int, C.c_int, _f32p, C.c_int, _u8p]
        R.ref_pack_codes.argtypes = [_u8p, _u8p, C.c_int, C.c_int]
        R.ref_unpack_codes.argtypes = [_u8p, _u8p, C.c_int, C.c_int]
        R.ref_tq_quantize_identity.argtypes = [C.c_int, C.c_int, _f32p, C.c_int, _u8p, _f32p]
        R.ref_dequant_int4.argtypes = [_f32p, _u8p, _f32p, _f32p, C.c_int, C.c_int]
        R.ref_paged_gather.argtypes = [C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_int, _f32p,
                                       _f32p]
        R.ref_moe_route.restype = C.c_int
        R.ref_moe_route.argtypes = [C.c_int, C.c_int, C.c_int, _f32p, _f32p, _i32p, _f32p]
        R.ref_f32_to_f16_kv.argtypes = [_f32p, _u16p, C.c_int]
        R.ref_f16_to_f32_kv.argtypes = [_u16p, _f32p, C.c_int]
        R.ref_nxf_write.restype = C.c_int
        R.ref_nxf_write.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_int]
        R.ref_nxf_summary.restype = C.c_long
        R.ref_nxf_summary.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        R.ref_nxf_chunk_bytes.restype = C.c_long
        R.ref_nxf_chunk_bytes.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_void_p, C.c_size_t]
        _ref_lib = R
    return _ref_lib


# ----------------------------------------------------------- numpy helpers --
def gen_normal(n: int, seed: int, tensor: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.nxo_gen_normal(out, n, seed, tensor, lib.nxo_normal_k(sigma))
    return out


def quantize(w: np.ndarray):
    """[N][K] fp32 -> (codes [N][G*16] u8, scales [N][G] u16)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    G = (K + 31) // 32
    codes = np.empty((N, G * 16), np.uint8)
    scales = np.empty((N, G), np.uint16)
    lib.nxo_quantize_int4_g32(w, N, K, codes, scales)
    return codes, scales


def gen_quant_rows(n0: int, count: int, K: int, seed: int, tensor: int, sigma: float):
    G = (K + 31) // 32
    codes = np.empty((count, G * 16), np.uint8)
    scales = np.empty((count, G), np.uint16)
    lib.nxo_gen_quant_rows(n0, count, K, seed, tensor, sigma, codes, scales)
    return codes, scales


def dequantize(codes, scales, N, K) -> np.ndarray:
    w = np.empty((N, K), np.float32)
    lib.nxo_dequant_int4_g32(np.ascontiguousarray(codes), np.ascontiguousarray(scales), N, K, w)
    return w


def gemv(codes, scales, x: np.ndarray, N: int, K: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    B = x.shape[0]
    y = np.empty((B, N), np.float32)
    lib.nxo_gemv_int4_g32(np.ascontiguousarray(codes), np.ascontiguousarray(scales), x, N, K, B, y)
    return y


def f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.nxo_f32_to_f16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def codebook(bits: int, d: int = 128):
    n = 1 << bits
    c = np.empty(n, np.float32)
    b = np.empty(n - 1, np.float32)
    lib.nxo_tq_codebook(d, bits, c, b)
    return c, b


def tq_signs(seed: int, tensor: int) -> np.ndarray:
    s = np.empty(128, np.float32)
    lib.nxo_tq_signs(s, seed, tensor)
    return s


def tq_encode(x: np.ndarray, signs: np.ndarray):
    """[n][128] fp32 -> (codes4 [n][32], codes3 [n][24], norms u16 [n], codes [n][128])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 128)
    n = x.shape[0]
    c4, b4 = codebook(4)
    c3, b3 = codebook(3)
    k4 = np.empty((n, 32), np.uint8)
    k3 = np.empty((n, 24), np.uint8)
    nr = np.empty(n, np.uint16)
    cu = np.empty((n, 128), np.uint8)
    lib.nxo_tq_encode(x, n, np.ascontiguousarray(signs, np.float32), b4, b3, k4, k3, nr, cu)
    return k4, k3, nr, cu


def tq_decode(k4, k3, nr, signs) -> np.ndarray:
    n = k4.shape[0]
    c4, _ = codebook(4)
    c3, _ = codebook(3)
    out = np.empty((n, 128), np.float32)
    lib.nxo_tq_decode(np.ascontiguousarray(k4), np.ascontiguousarray(k3),
                      np.ascontiguousarray(nr), n, np.ascontiguousarray(signs, np.float32),
                      c4, c3, out)
    return out


def cool_encode(x: np.ndarray, signs: np.ndarray):
    """[n][128] fp32 -> Cool form (codes [n][48], norms u16 [n])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 128)
    n = x.shape[0]
    _, b3 = codebook(3)
    cc = np.empty((n, 48), np.uint8)
    nr = np.empty(n, np.uint16)
    lib.nxo_cool_encode(x, n, np.ascontiguousarray(signs, np.float32), b3, cc, nr)
    return cc, nr


def cool_decode(cc, nr, signs) -> np.ndarray:
    n = cc.shape[0]
    c3, _ = codebook(3)
    out = np.empty((n, 128), np.float32)
    lib.nxo_cool_decode(np.ascontiguousarray(cc), np.ascontiguousarray(nr), n,
                        np.ascontiguousarray(signs, np.float32), c3, out)
    return out


def tq_to_cool(k4, k3, nr, signs):
    """TurboQuant (Warm) vectors -> Cool form (codes [n][48], norms u16 [n])."""
    n = k4.shape[0]
    c4, _ = codebook(4)
    c3, b3 = codebook(3)
    cc = np.empty((n, 48), np.uint8)
    cn = np.empty(n, np.uint16)
    lib.nxo_tq_to_cool(np.ascontiguousarray(k4), np.ascontiguousarray(k3), np.ascontiguousarray(nr), n,
                       np.ascontiguousarray(signs, np.float32), c4, c3, b3, cc, cn)
    return cc, cn


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)


class Model:
    """The oracle's synthetic decoder (see nx_oracle.h)."""

    def __init__(self, **kw):
        self.cfg = Cfg(**kw)
        self.h = lib.nxo_model_create(C.byref(self.cfg))

    def close(self):
        if self.h:
            lib.nxo_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty((self.cfg.batch, self.cfg.vocab), np.float32)
        lib.nxo_model_forward(self.h, t, logits)
        return logits

    def forward_timed(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty((self.cfg.batch, self.cfg.vocab), np.float32)
        tl, th = C.c_double(), C.c_double()
        lib.nxo_model_forward_timed(self.h, t, logits, C.byref(tl), C.byref(th))
        return logits, tl.value, th.value

    def generate(self, prompt: np.ndarray, n_new: int):
        p = np.ascontiguousarray(prompt, np.int32).reshape(self.cfg.batch, -1)
        out = np.empty((self.cfg.batch, n_new), np.int32)
        margins = np.empty((self.cfg.batch, n_new), np.float32)
        lib.nxo_model_generate(self.h, p, p.shape[1], n_new, out, margins)
        return out, margins

    def fill_context(self, ctx: int, n_outlier: int = 0):
        lib.nxo_model_fill_context(self.h, ctx, n_outlier)

    def kv_read(self, layer: int, b: int, pos: int, kv: int, form: int) -> np.ndarray:
        """Stored bytes of one position, all kv heads (nxo_model_kv_read)."""
        out = np.zeros(max(58, 2 * self.cfg.head_dim) * self.cfg.n_kv_heads, np.uint8)  # every form fits
        n = lib.nxo_model_kv_read(self.h, layer, b, pos, kv, form, out)
        assert n > 0, "the oracle model does not hold that form"
        return out[:n]

    def position(self, b: int = 0) -> int:
        return lib.nxo_model_position(self.h, b)


def prompt_tokens(seed: int, batch: int, P: int, vocab: int) -> np.ndarray:
    out = np.empty(batch * P, np.int32)
    lib.nxo_gen_tokens(out, batch * P, seed, 4, vocab)
    return out.reshape(batch, P)
