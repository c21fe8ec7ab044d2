"""CPU checks of the C-ABI library: it loads, exports every entry point the
header declares, reports the absence of a GPU as an error code, and its
host-side TurboQuant codebooks equal the oracle's (and so the reference's)."""
import ctypes as C
import re

import numpy as np
import pytest

import nexus_amd
import oracle


def declared_symbols():
    """Every entry point declared in include/*.h."""
    syms = set()
    for h in nexus_amd.HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        syms |= set(re.findall(r"^\s*(?:nx_status|int|const char\s*\*)\s+(nx_\w+)\s*\(", text, flags=re.M))
    return sorted(syms)


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ("nx_init", "nx_gemv_int4_g32", "nx_attn_decode_paged_f16", "nx_attn_decode_paged_tq",
                 "nx_tq_encode", "nx_moe_expert_ffn", "nx_model_decode", "nx_token_begin",
                 "nx_nxf_open", "nx_nxf_verify", "nx_xxh32_chunks", "nx_model_load_nxf"):
        assert must in syms
    assert len(syms) >= 40


def test_library_exports_every_declared_symbol():
    L = nexus_amd.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert missing == []


def test_binding_signatures_cover_header():
    assert set(declared_symbols()) <= set(nexus_amd._SIGS)


def test_codebooks_match_oracle_bitwise():
    c4, b4, c3, b3 = nexus_amd.tq_codebooks()
    oc4, ob4 = oracle.codebook(4)
    oc3, ob3 = oracle.codebook(3)
    for a, b in ((c4, oc4), (b4, ob4), (c3, oc3), (b3, ob3)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_no_device_is_an_error_not_a_fallback():
    if nexus_amd.has_gpu():
        pytest.skip("a GPU is present")
    with pytest.raises(nexus_amd.NxError) as e:
        nexus_amd.Context(0)
    assert e.value.code == 6  # NX_ERR_NO_DEVICE


def test_null_arguments_are_rejected():
    L = nexus_amd.lib()
    assert L.nx_init(None, 0) == 1
    assert L.nx_destroy(None) == 1
    assert L.nx_gemv_int4_g32(None, 0, 0, 0, 0, 1, 32, 1) == 1
    assert L.nx_tq_codebooks(None, None, None, None) == 1


def test_library_built_from_these_sources():
    """The in-tree library reports the SHA-1 of the sources it was built
    from, and the binding refuses one built from other sources."""
    L = nexus_amd.lib()
    assert L.nx_source_hash().decode() == nexus_amd.source_hash()
    assert re.fullmatch(r"[0-9a-f]{40}", nexus_amd.source_hash())
