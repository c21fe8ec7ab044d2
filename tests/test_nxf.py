"""NXF weight files: the format parity of this library's reader and writer
with the reference's NXFReader / NXFWriter (compiled in place into
oracle/_ref), XXH32 chunk checksums on the GPU against the oracle (itself
pinned to the published algorithm through the xxhash package and to the
reference writer's stored checksums), and model save -> load round trips.

CPU tests need no GPU: the reader is host code.  GPU tests are marked."""
import os

import numpy as np
import pytest

import nexus_amd
import oracle
from nexus_amd import NxError
from nexus_amd.nxf import NXFReader
from nxf_cases import (CASE_MANIFEST, CONTROL_NAME, NXF_CASES, REF_TEST_MANIFEST, our_summary, our_write,
                       ragged_tensors, ref_chunk, ref_file_bytes, ref_summary, ref_test_tensors, ref_write)

needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="reference checker oracle/_ref not built")


# ------------------------------------------------------------------ oracle --
def test_oracle_xxh32_published_vectors():
    """XXH32 known answers of the published algorithm (xxHash test vectors)."""
    assert oracle.lib.nxo_xxh32(b"", 0, 0) == 0x02CC5D05
    assert oracle.lib.nxo_xxh32(b"a", 1, 0) == 0x550D7456
    assert oracle.lib.nxo_xxh32(b"abc", 3, 0) == 0x32D153FF


def test_oracle_xxh32_matches_xxhash_package():
    """Every length class (below one stripe, whole stripes, tails of 1-15
    bytes) and two seeds against the xxhash package (xxHash 0.8.2)."""
    xxhash = pytest.importorskip("xxhash")
    rng = np.random.default_rng(3)
    for n in list(range(0, 80)) + [255, 4096, 16383, 65536 + 9]:
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        for seed in (0, 0x9747B28C):
            assert oracle.lib.nxo_xxh32(b, n, seed) == xxhash.xxh32(b, seed=seed).intdigest(), (n, seed)


# ------------------------------------------------------- reader (CPU only) --
@needs_ref
def test_reader_reads_reference_test_file(tmp_path):
    """The reference's own round-trip test (test_nxf_format.cpp:13-89),
    written by the reference writer, read by this library's reader: the
    manifest fields, two tensors, one chunk each, fdata[0] == 0.0 and
    fdata[1000] == 1.0, and each stored checksum equals the oracle's XXH32
    of the chunk bytes."""
    p = tmp_path / "ref.nxf"
    ref_write(p, REF_TEST_MANIFEST, ref_test_tensors())
    with NXFReader.open(p) as r:
        m = r.manifest()
        assert (m.architecture, m.name, m.num_layers, m.hidden_dim, m.vocab_size) == \
            ("llama", "test-model-7b", 2, 128, 256)
        assert sorted(r.tensor_names()) == ["layers.0.attention.wq.weight", "layers.0.attention_norm.weight"]
        wq = r.get_tensor("layers.0.attention.wq.weight")
        assert wq.shape == [128, 128] and len(wq.chunks) == 1
        f = np.frombuffer(r.read_chunk(wq, 0), np.float32)
        assert f[0] == 0.0 and f[1000] == 1.0
        view = r.map_chunk(wq, 0)
        assert bytes(view) == r.read_chunk(wq, 0)
        r.unmap_chunk(view)
        for t in r.tensors():
            for j, c in enumerate(t.chunks):
                b = r.read_chunk(t, j)
                assert oracle.lib.nxo_xxh32(b, len(b), 0) == c.checksum
        assert r.get_tensor("missing") is None
        assert our_summary(r) == ref_summary(p)


@needs_ref
def test_reader_matches_reference_reader_on_ragged_file(tmp_path):
    """Ragged chunk sizes, an int4-g32 tensor with its scale sidecar, a
    chunk above 1 MiB, a tensor with no chunks: both readers see the same
    manifest, tensors and chunk descriptors; the chunk bytes agree."""
    p = tmp_path / "ragged.nxf"
    tensors = ragged_tensors()
    ref_write(p, dict(REF_TEST_MANIFEST, name="ragged \"quoted\"\tname"), tensors)
    with NXFReader.open(p) as r:
        assert our_summary(r) == ref_summary(p)
        for name, _, _, chunks in tensors:
            t = r.get_tensor(name)
            for j, (b, codec, g) in enumerate(chunks):
                assert r.read_chunk(t, j) == b == ref_chunk(p, name, j)
                assert t.chunks[j].file_offset % 16384 == 0
                assert oracle.lib.nxo_xxh32(b, len(b), 0) == t.chunks[j].checksum


@needs_ref
def test_reader_rejects_malformed_files(tmp_path):
    """Bad magic, unsupported version, a size that differs from the
    header's, a truncated tensor index: an IO error, not a crash."""
    p = tmp_path / "ok.nxf"
    ref_write(p, REF_TEST_MANIFEST, ref_test_tensors())
    good = p.read_bytes()

    def expect_io(data, tag):
        q = tmp_path / f"{tag}.nxf"
        q.write_bytes(data)
        with pytest.raises(NxError) as e:
            NXFReader.open(q)
        assert e.value.code == 9, tag

    bad = bytearray(good)
    bad[0] ^= 0xFF
    expect_io(bytes(bad), "magic")
    bad = bytearray(good)
    bad[4] = 2
    expect_io(bytes(bad), "version")
    expect_io(good + b"\0", "size")
    # tensor index: cut the first tensor's name length to claim more bytes than exist
    idx_off = int.from_bytes(good[24:32], "little")
    idx_size = int.from_bytes(good[32:40], "little")
    bad = bytearray(good)
    bad[idx_off:idx_off + 4] = (idx_size + 100).to_bytes(4, "little")
    expect_io(bytes(bad), "index")
    with pytest.raises(NxError):
        NXFReader.open(tmp_path / "does-not-exist.nxf")


# --------------------------------------------------------------------- GPU --
@pytest.mark.gpu
def test_gpu_xxh32_matches_oracle(ctx):
    """The device hash of ragged ranges of one buffer (lengths 0..200, the
    stripe and step boundaries, 64 KiB, 1 MiB + 7, ranges sorted to mixed
    wavefronts) equals the oracle's XXH32, bit for bit."""
    from nexus_amd.nxf import xxh32_chunks
    rng = np.random.default_rng(11)
    sizes = list(range(0, 201)) + [255, 256, 257, 4095, 4096, 4097, 16384, 65536, 65536 + 13, (1 << 20) + 7]
    rng.shuffle(sizes)
    offs, o = [], 0
    for n in sizes:
        offs.append(o)
        o += (n + 15) // 16 * 16 + 16 * int(rng.integers(0, 3))
    data = rng.integers(0, 256, o + 64, dtype=np.uint8)
    buf = ctx.upload(data)
    got = xxh32_chunks(ctx, buf, offs, sizes)
    want = [oracle.lib.nxo_xxh32(data[a:a + n].tobytes(), n, 0) for a, n in zip(offs, sizes)]
    assert [int(x) for x in got] == want
    ctx.free(buf)


@pytest.mark.gpu
def test_gpu_xxh32_rejects_bad_ranges(ctx):
    from nexus_amd.nxf import xxh32_chunks
    buf = ctx.upload(np.zeros(256, np.uint8))
    with pytest.raises(NxError):
        xxh32_chunks(ctx, buf, [8], [16])      # unaligned start
    with pytest.raises(NxError):
        xxh32_chunks(ctx, buf, [240], [32])    # past the end
    ctx.free(buf)


def _with_manifest(tmp_path, text: str):
    """The reference writer's test file with its manifest replaced by
    `text` (appended at the end of the file, header offsets updated)."""
    data = bytearray(ref_file_bytes("reference_test"))
    body = text.encode()
    off = len(data)
    data += body
    data[8:16] = off.to_bytes(8, "little")          # manifest_offset
    data[16:24] = len(body).to_bytes(8, "little")   # manifest_size
    data[48:56] = len(data).to_bytes(8, "little")   # total_file_size
    p = tmp_path / "m.nxf"
    p.write_bytes(bytes(data))
    return p


MANIFEST_OK = ('{"architecture": "llama", "name": "a\\"b\\\\c\\/d\\u0041\\u00e9", "num_layers": 2, '
               '"hidden_dim": 128, "rope_theta": 1e4, "rms_norm_eps": 1E-5, "unknown": "x", "other": -3.5, '
               '"default_codec": 255, "max_seq_len": 4294967295}')


def test_manifest_parser_accepts_standard_json(tmp_path):
    """Escapes (\\", \\\\, \\/, \\u), exponents, unknown keys of either kind and
    the limits of the integer fields are read as JSON defines them."""
    with NXFReader.open(_with_manifest(tmp_path, MANIFEST_OK)) as r:
        m = r.manifest()
    assert m.name == 'a"b\\c/dAé' and m.architecture == "llama"
    assert (m.num_layers, m.hidden_dim, m.default_codec, m.max_seq_len) == (2, 128, 255, 4294967295)
    assert m.rope_theta == 10000.0 and abs(m.rms_norm_eps - 1e-5) < 1e-12


def test_manifest_parser_takes_what_the_reference_reader_takes(tmp_path):
    """Raw control bytes inside a string (the reference writer leaves \\r and
    other control bytes unescaped), default_codec as quoted text (read as
    atoi reads it, format/nxf_reader.cpp:162) and bytes after the closing
    brace are accepted, as the reference reader accepts them."""
    text = '{"name": "a\rb\x01c\x1f", "default_codec": " 3", "num_layers": 2} trailing \x00 bytes'
    with NXFReader.open(_with_manifest(tmp_path, text)) as r:
        m = r.manifest()
    assert m.name == "a\rb\x01c\x1f" and m.default_codec == 3 and m.num_layers == 2
    with NXFReader.open(_with_manifest(tmp_path, '{"default_codec": "x"}')) as r:
        assert r.manifest().default_codec == 0  # no digits: atoi gives 0


def test_reader_reads_the_control_name_fixture(tmp_path):
    """The reference writer's file whose model name holds raw control bytes
    (the fixture of case control_name) opens with that name."""
    p = tmp_path / "c.nxf"
    p.write_bytes(ref_file_bytes("control_name"))
    with NXFReader.open(p) as r:
        m = r.manifest()
    assert m.name == CONTROL_NAME and m.num_layers == 2


@pytest.mark.parametrize("bad", [
    '{"num_layers": -1}', '{"num_layers": 4294967296}', '{"num_layers": 2.5}', '{"default_codec": 256}',
    '{"default_codec": "256"}', '{"default_codec": "-1"}', '{"num_layers": "2"}', '{"name": 3}',
    '{"rope_theta": 1e39}', '{"num_layers": 2,}', '{"num_layers": 2', '{"a": {"b": 1}}', '{"a": [1]}',
    '{"a": true}', '{"num_layers": 01}', '{"num_layers": .5}', '{"name": "x\\q"}'])
def test_manifest_parser_rejects(tmp_path, bad):
    """Values outside a field's range (negative, 2^32 and above, fractions,
    bytes above 255, floats that overflow), a value of the wrong kind, and
    text that is not a flat JSON object of strings and numbers fail the
    open instead of being cast."""
    with pytest.raises(NxError):
        NXFReader.open(_with_manifest(tmp_path, bad))


@needs_ref
@pytest.mark.parametrize("case", list(NXF_CASES))
def test_nxf_fixture_is_the_reference_writers_file(tmp_path, case):
    """The fixture the GPU tests compare against (golden/nxf_ref_files.npz,
    payload put back) is byte for byte the file the reference's NXFWriter
    writes for the case now."""
    p = tmp_path / "ref.nxf"
    ref_write(p, CASE_MANIFEST[case], NXF_CASES[case]())
    assert p.read_bytes() == ref_file_bytes(case)


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(NXF_CASES))
def test_writer_output_is_byte_identical_to_reference_writer(ctx, tmp_path, case):
    """The same manifest and chunks written by the reference's NXFWriter
    (the fixture of its file) and by this library's writer (checksums
    computed on the GPU) give byte-identical files."""
    b = tmp_path / "ours.nxf"
    our_write(ctx, b, CASE_MANIFEST[case], NXF_CASES[case]())
    assert b.read_bytes() == ref_file_bytes(case)


@pytest.mark.gpu
def test_verify_on_gpu_finds_a_corrupt_chunk(ctx, tmp_path):
    """Verification of a reference-written file passes; one flipped byte in
    the second chunk of the ragged tensor is reported as that chunk."""
    p = tmp_path / "v.nxf"
    tensors = ragged_tensors()
    p.write_bytes(ref_file_bytes("ragged"))
    with NXFReader.open(p) as r:
        total = sum(len(b) for _, _, _, ch in tensors for b, _, _ in ch)
        assert r.verify(ctx) == total
        t = r.get_tensor("ragged")
        idx = [x.name for x in r.tensors()].index("ragged")
        off = t.chunks[1].file_offset + 2
    data = bytearray(p.read_bytes())
    data[off] ^= 0x10
    q = tmp_path / "bad.nxf"
    q.write_bytes(bytes(data))
    with NXFReader.open(q) as r:
        with pytest.raises(NxError) as e:
            r.verify(ctx)
        assert e.value.code == 8 and e.value.bad == (idx, 1)
        assert "ragged" in str(e.value)


TINY = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=688, vocab=4096,
            n_experts=0, top_k=0, max_seq=128, batch=1, kv_kind=0, rope_theta=10000.0, eps=1e-5,
            seed=0x5EED, norm_sigma=0.1)


@pytest.mark.gpu
@pytest.mark.parametrize("moe", [False, True])
def test_model_save_load_round_trip(ctx, tmp_path, moe):
    """A seeded tiny model (RMSNorm weights 1 + N(0, 0.1)) saved as NXF and
    loaded back decodes the same greedy tokens and logits, bit for bit, and
    its tensor index names the lm_head with the reference's {in, out} shape."""
    cfg = dict(TINY, n_experts=4, top_k=2, seed=0x0E0E) if moe else TINY
    p = tmp_path / "tiny.nxf"
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 8, cfg["vocab"])
    a = nexus_amd.Model(ctx, **cfg)
    a.save_nxf(p)
    first_a = a.prefill(prompt)
    toks_a = a.decode(12)
    log_a = a.logits()
    a.close()
    b = nexus_amd.Model.load_nxf(ctx, p, batch=1, max_seq=cfg["max_seq"], seed=cfg["seed"])
    assert b.cfg.ffn == cfg["ffn"] and b.cfg.n_experts == cfg["n_experts"]
    first_b = b.prefill(prompt)
    toks_b = b.decode(12)
    log_b = b.logits()
    b.close()
    assert (first_a == first_b).all() and (toks_a == toks_b).all()
    assert np.array_equal(log_a, log_b)
    with NXFReader.open(p) as r:
        s = our_summary(r)
    assert "tensor output.weight shape %d %d dtype 4" % (cfg["d_model"], cfg["vocab"]) in s


@pytest.mark.gpu
@pytest.mark.parametrize("kv_kind,hot", [(1, 0), (2, 32)])
def test_loaded_model_with_turboquant_and_tiered_pages(ctx, tmp_path, kv_kind, hot):
    """The run configuration of a load selects the page kind: a model saved
    as NXF and loaded with TurboQuant or tiered pages (a 32-position window,
    pages compressed during the 60 decode steps) decodes exactly as the
    synthetic model it was saved from."""
    cfg = dict(TINY, n_heads=4, n_kv_heads=2, head_dim=128, d_model=512, kv_kind=kv_kind, hot_window=hot)
    p = tmp_path / "tq.nxf"
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 8, cfg["vocab"])
    a = nexus_amd.Model(ctx, **cfg)
    a.save_nxf(p)
    first_a = a.prefill(prompt)
    toks_a = a.decode(60)
    log_a = a.logits()
    a.close()
    b = nexus_amd.Model.load_nxf(ctx, p, batch=1, max_seq=cfg["max_seq"], kv_kind=kv_kind, seed=cfg["seed"],
                                 hot_window=hot)
    first_b = b.prefill(prompt)
    toks_b = b.decode(60)
    log_b = b.logits()
    b.close()
    assert (first_a == first_b).all() and (toks_a == toks_b).all()
    assert np.array_equal(log_a, log_b)


@pytest.mark.gpu
def test_loaded_model_matches_oracle_with_norm_weights(ctx, tmp_path):
    """The RMSNorm weights travel through the file into the fused kernels:
    greedy tokens of the loaded model equal the oracle's for the same
    seeded weights (norm weights 1 + N(0, 0.1))."""
    from test_gpu_model import assert_greedy_parity
    p = tmp_path / "tiny.nxf"
    a = nexus_amd.Model(ctx, **TINY)
    a.save_nxf(p)
    a.close()
    prompt = oracle.prompt_tokens(TINY["seed"], 1, 8, TINY["vocab"])
    om = oracle.Model(**TINY)
    want, margins = om.generate(prompt, 16)
    om.close()
    b = nexus_amd.Model.load_nxf(ctx, p, batch=1, max_seq=TINY["max_seq"], seed=TINY["seed"])
    got = np.concatenate([b.prefill(prompt)[:, None], b.decode(15)], axis=1)
    b.close()
    assert_greedy_parity(got, want, margins)


@pytest.mark.gpu
def test_qk_norm_weights_round_trip(ctx, tmp_path):
    """A model with per-head Q/K norms writes layers.L.attn_q_norm.weight and
    attn_k_norm.weight (head_dim long, the names hybrid_model.cpp:1952-1953
    loads); loading the file turns the norms on and decodes the original
    model's tokens and logits exactly."""
    cfg = dict(TINY, qk_norm=1, norm_sigma=0.1, seed=0x9C10)
    p = tmp_path / "qk.nxf"
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 9, cfg["vocab"])
    a = nexus_amd.Model(ctx, **cfg)
    a.save_nxf(p)
    ta = a.prefill(prompt)
    toks_a, log_a = a.decode(10), a.logits()
    a.close()
    with NXFReader.open(p) as r:
        t = r.get_tensor("layers.1.attn_k_norm.weight")
        assert t is not None and list(t.shape) == [cfg["head_dim"]]
    b = nexus_amd.Model.load_nxf(ctx, p, batch=1, max_seq=cfg["max_seq"], seed=cfg["seed"])
    assert b.cfg.qk_norm == 1
    tb = b.prefill(prompt)
    toks_b, log_b = b.decode(10), b.logits()
    b.close()
    assert (ta == tb).all() and (toks_a == toks_b).all() and np.array_equal(log_a, log_b)


@pytest.mark.gpu
def test_load_without_expert_count_routes_ten(ctx, tmp_path):
    """A MoE file whose manifest gives no active-expert count
    (num_active_experts 0) runs ten experts per token, as the reference does
    (hybrid_model.cpp:1648): the loaded model decodes as the top-10 model it
    was saved from."""
    import re
    cfg = dict(TINY, n_experts=16, top_k=10, seed=0xA10)
    p = tmp_path / "moe.nxf"
    prompt = oracle.prompt_tokens(cfg["seed"], 1, 6, cfg["vocab"])
    a = nexus_amd.Model(ctx, **cfg)
    a.save_nxf(p)
    ta = a.prefill(prompt)
    toks_a, log_a = a.decode(8), a.logits()
    a.close()
    data = bytearray(p.read_bytes())
    off = int.from_bytes(data[8:16], "little")
    size = int.from_bytes(data[16:24], "little")
    text = data[off:off + size].decode()
    new = re.sub(r'"num_active_experts":\s*10', lambda m: m.group(0)[:-2] + " 0", text)
    assert new != text and len(new) == len(text)
    data[off:off + size] = new.encode()
    p.write_bytes(bytes(data))
    with NXFReader.open(p) as r:
        assert r.manifest().num_active_experts == 0
    b = nexus_amd.Model.load_nxf(ctx, p, batch=1, max_seq=cfg["max_seq"], seed=cfg["seed"])
    tb = b.prefill(prompt)
    toks_b, log_b = b.decode(8), b.logits()
    b.close()
    assert (ta == tb).all() and (toks_a == toks_b).all() and np.array_equal(log_a, log_b)


@pytest.mark.gpu
def test_model_load_rejects_a_corrupt_file(ctx, tmp_path):
    """A flipped byte inside layer 1's wo codes fails the load with a
    checksum error naming that tensor; nothing is returned."""
    p = tmp_path / "tiny.nxf"
    a = nexus_amd.Model(ctx, **TINY)
    a.save_nxf(p)
    a.close()
    with NXFReader.open(p) as r:
        t = r.get_tensor("layers.1.attention.wo.weight")
        off = t.chunks[0].file_offset + 100
    data = bytearray(p.read_bytes())
    data[off] ^= 1
    q = tmp_path / "bad.nxf"
    q.write_bytes(bytes(data))
    with pytest.raises(NxError) as e:
        nexus_amd.Model.load_nxf(ctx, q, batch=1, max_seq=TINY["max_seq"])
    assert e.value.code == 8 and "layers.1.attention.wo.weight" in str(e.value)
