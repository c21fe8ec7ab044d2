/* NXF weight files on the decode library: reader, writer, chunk checksums
 * computed on the GPU, and model load/save.
 *
 * Counterpart of nexus::format::NXFReader / NXFWriter
 * (nexus/src/format/nxf.h:100-190, nxf_reader.cpp, nxf_writer.cpp).  The
 * file format is the reference's, byte for byte: a 64-byte header at offset
 * 0 (nxf.h:27-38), chunk data at 16 KiB-aligned offsets from 16 KiB on, the
 * binary tensor index (nxf_writer.cpp:133-183) and the JSON manifest
 * (nxf_writer.cpp:93-129), each 16 KiB aligned, the file padded to 16 KiB.
 * A chunk's checksum is XXH32 (seed 0) of its stored bytes
 * (nxf_writer.cpp:33-72, :255).
 *
 * Differences from the reference, all deliberate:
 *   - every call returns nx_status (the reference returns bool / nullptr and
 *     prints); the message of the last failing NXF call of this thread is
 *     nx_nxf_error();
 *   - checksums are computed and verified on the GPU (nx_xxh32_chunks,
 *     nx_nxf_verify, the writer and the model loader); the reference stores
 *     checksums but never verifies them on read;
 *   - int4 weights use the build's int4-g32 codec: a tensor of dtype I4 and
 *     shape {..., rows, K} holds chunks of codec INT4 (4) with group_size 32
 *     carrying whole rows of G*16 bytes (G = ceil(K/32); low nibble = even
 *     k, value (q - 8) * scale), followed by sidecar chunks of codec FP16 (1)
 *     with group_size 32 carrying the fp16 scales [rows][G].  (The
 *     reference's importers append fp32 scale and zero tails inside the
 *     INT4 chunk, which its kernels ignore.)
 * The reader and writer are single-threaded objects, like the reference's. */
#ifndef NEXUS_NXF_H
#define NEXUS_NXF_H

#include "nexus_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define NX_ERR_CHECKSUM 8 /* stored checksum differs from the data */
#define NX_ERR_IO 9       /* file system error or malformed file */

/* Codec and DType identifiers of the format (core/config.h:21-46). */
enum { NX_CODEC_FP32 = 0, NX_CODEC_FP16 = 1, NX_CODEC_BF16 = 2, NX_CODEC_INT8 = 3, NX_CODEC_INT4 = 4 };
enum { NX_DTYPE_F32 = 0, NX_DTYPE_F16 = 1, NX_DTYPE_BF16 = 2, NX_DTYPE_I8 = 3, NX_DTYPE_I4 = 4 };

/* ModelManifest (nxf.h:76-96). */
typedef struct {
    char architecture[64];
    char name[128];
    uint32_t num_layers, hidden_dim, num_heads, num_kv_heads, head_dim, vocab_size, max_seq_len;
    float rope_theta, rms_norm_eps;
    uint32_t num_experts, num_active_experts;
    uint8_t default_codec, default_group_size;
} nx_nxf_manifest;

/* ChunkDesc (nxf.h:42-50). */
typedef struct {
    uint64_t file_offset;
    uint32_t compressed_size, decompressed_size, checksum;
    uint8_t codec, group_size;
} nx_nxf_chunk;

/* TensorInfo (nxf.h:54-73); name stays valid while the reader is open. */
typedef struct {
    const char* name;
    int ndim;
    int64_t shape[8];
    int dtype;
    int num_chunks;
    uint64_t compressed_bytes, decompressed_bytes;
} nx_nxf_tensor;

typedef struct nx_nxf nx_nxf;
typedef struct nx_nxf_writer nx_nxf_writer;

/* Message of the last failing NXF call on this thread ("" if none). */
const char* nx_nxf_error(void);

/* ------------------------------------------------------------- reading -- */
/* NXFReader::open (nxf_reader.cpp:192-220): header (magic, version, file
 * size), manifest and tensor index; no tensor data is read.  Host only. */
nx_status nx_nxf_open(const char* path, nx_nxf** out);
/* NXFReader::close (nxf_reader.cpp:277-292), unmapping every chunk. */
nx_status nx_nxf_close(nx_nxf* r);
/* NXFReader::manifest (nxf.h:109). */
nx_status nx_nxf_get_manifest(nx_nxf* r, nx_nxf_manifest* out);
/* Number of tensors; tensors are numbered in index order. */
nx_status nx_nxf_num_tensors(nx_nxf* r, int* n);
nx_status nx_nxf_tensor_at(nx_nxf* r, int i, nx_nxf_tensor* out);
/* NXFReader::get_tensor (nxf_reader.cpp:222-226): *index = -1 if absent. */
nx_status nx_nxf_find(nx_nxf* r, const char* name, int* index);
nx_status nx_nxf_chunk_at(nx_nxf* r, int tensor, int chunk, nx_nxf_chunk* out);
/* NXFReader::map_chunk / unmap_chunk (nxf_reader.cpp:237-275): a read-only
 * private mapping of the chunk's stored bytes. */
nx_status nx_nxf_map_chunk(nx_nxf* r, int tensor, int chunk, const void** data);
nx_status nx_nxf_unmap_chunk(nx_nxf* r, const void* data);
/* Copy a chunk's stored bytes (compressed_size of them) to host memory. */
nx_status nx_nxf_read_chunk(nx_nxf* r, int tensor, int chunk, void* dst);
/* Verify every chunk of the file on the GPU: the chunks are read in
 * batches, uploaded and hashed on the device.  All good: NX_OK with
 * *bad_tensor = *bad_chunk = -1.  Otherwise NX_ERR_CHECKSUM with the first
 * mismatching (tensor, chunk) in index order.  bytes (optional) receives
 * the bytes verified. */
nx_status nx_nxf_verify(nx_ctx* ctx, nx_nxf* r, int* bad_tensor, int* bad_chunk, uint64_t* bytes);

/* ------------------------------------------------------------- writing -- */
/* NXFWriter::create (nxf_writer.cpp:197-223).  ctx hashes the chunks. */
nx_status nx_nxf_writer_create(nx_ctx* ctx, const char* path, nx_nxf_writer** out);
nx_status nx_nxf_writer_set_manifest(nx_nxf_writer* w, const nx_nxf_manifest* m);
/* NXFWriter::begin_tensor / add_chunk / end_tensor (nxf_writer.cpp:229-283):
 * add_chunk writes size bytes at the next 16 KiB boundary; its checksum is
 * computed on the GPU before finalize.  Empty chunks are skipped, as in the
 * reference. */
nx_status nx_nxf_writer_begin_tensor(nx_nxf_writer* w, const char* name, const int64_t* shape, int ndim,
                                     int dtype);
nx_status nx_nxf_writer_add_chunk(nx_nxf_writer* w, const void* data, size_t size, int codec, int group_size);
nx_status nx_nxf_writer_end_tensor(nx_nxf_writer* w);
/* NXFWriter::finalize (nxf_writer.cpp:285-338): tensor index, manifest,
 * header; closes the file and frees the writer (also on error). */
nx_status nx_nxf_writer_finalize(nx_nxf_writer* w);
/* Abandon a writer without finalizing; the partial file is kept (as the
 * reference's destructor does, nxf_writer.cpp:187-195). */
nx_status nx_nxf_writer_destroy(nx_nxf_writer* w);

/* -------------------------------------------------------------- hashing -- */
/* XXH32 (seed 0) of n byte ranges of device buffer data: range i is
 * [offsets[i], offsets[i] + sizes[i]), offsets a multiple of 16; hashes[i]
 * receives its hash.  Host arrays; returns after the hashes are copied. */
nx_status nx_xxh32_chunks(nx_ctx* ctx, nx_buf data, const uint64_t* offsets, const uint32_t* sizes, int n,
                          uint32_t* hashes);
/* Average device time (ms) of hashing `bytes` of data as consecutive
 * chunks of chunk_bytes (a multiple of 16) over `iters` launches, HIP
 * events on the library stream; hashes (optional, ceil(bytes/chunk_bytes)
 * words) receives the result of the last launch. */
nx_status nx_time_xxh32(nx_ctx* ctx, nx_buf data, size_t bytes, uint32_t chunk_bytes, int iters, double* avg_ms,
                        uint32_t* hashes);

/* ------------------------------------------------------ model load/save -- */
/* Save a resident model as an NXF file in the build's layout: manifest
 * from the model's configuration; tensors tok_embeddings.weight (F16
 * [V][d]), norm.weight (F32), output.weight (I4), and per layer L
 * layers.L.attention_norm.weight, layers.L.ffn_norm.weight (F32),
 * layers.L.attention.{wq,wk,wv,wo}.weight (I4) and either
 * layers.L.feed_forward.{w1,w3,w2}.weight (gate, up, down) or
 * layers.L.feed_forward.gate.weight with
 * layers.L.feed_forward.experts.{w1,w3,w2}.weight of shape
 * {E, F, d} / {E, F, d} / {E, d, F} -- the reference's tensor names
 * (hybrid_model.cpp:1806-1868, :2015).  Chunks hold whole rows, at most
 * 64 KiB (one row if a row is larger). */
nx_status nx_model_save_nxf(nx_model* m, const char* path);
/* Create a resident model from an NXF file: dimensions from the manifest
 * and tensor shapes (the FFN width from feed_forward.w1 or the experts'
 * w1), every chunk verified on the GPU before use (NX_ERR_CHECKSUM names
 * the tensor), weights placed in the runner's layout.  batch, max_seq,
 * kv_kind and seed (page shuffle and synthetic context) come from the
 * caller; the other fields of *run are ignored. */
nx_status nx_model_load_nxf(nx_ctx* ctx, const char* path, const nx_model_config* run, nx_model** out);

#ifdef __cplusplus
}
#endif
#endif
