/*
 * g4ckpt.h - the on-disk format of the checkpoint: a safetensors directory reader, the lm_head tie
 * and its guard, the QUANT_RULES family resolution and the text-tensor allow list, with payload
 * reads straight into device memory.
 *
 * Replaces src/safetensors.ts (parseHeader :163-295, coverageGaps :297-307, the tie table and
 * applyTies :616-705, the tie guard :706-800, sha256Hex :819, textTensorNames / selectTextTensors
 * :930-1010) and src/quant.ts (QUANT_RULES / resolveQuantBits :430-513, modulePathForTensor
 * :649-663) of Ar5en1c/gemma4-webgpu-engine. The reference reads the file over HTTP ranges; this
 * build reads a local file (there is no network on the box), with the same validation.
 *
 * Errors: G4_ERR_INVALID with g4_last_error() = "safetensors <code>: <message>", <code> one of the
 * reference's SafetensorsErrorCode strings (safetensors.ts:65-77).
 */
#ifndef G4CKPT_H
#define G4CKPT_H

#include "g4w8a8.h"

#ifdef __cplusplus
extern "C" {
#endif

#define G4_ST_MAX_DIMS 8
#define G4_ST_HEADER_PREFIX_BYTES 8                /* safetensors.ts:56 */
#define G4_ST_MAX_HEADER_BYTES (64 * 1024 * 1024)  /* safetensors.ts:63 */

/* One tensor of the directory (TensorEntry, safetensors.ts:85-105). Strings live as long as the
 * directory. */
typedef struct g4_st_tensor {
    const char *name;
    const char *dtype; /* "BOOL", "U8", "I8", "F8_E4M3", "F8_E5M2", "U16", "I16", "F16", "BF16",
                          "U32", "I32", "F32", "U64", "I64", "F64" */
    int ndim;
    int64_t shape[G4_ST_MAX_DIMS];
    int64_t data_start; /* payload relative, as the header states */
    int64_t data_end;
    int64_t file_start; /* absolute: 8 + header length + data_start */
    int64_t file_end;
    int64_t byte_length;
    int64_t element_count;
} g4_st_tensor;

typedef struct g4_st g4_st;

/* parseHeader: the 8-byte little-endian length, the JSON it sizes, every entry validated (dtype,
 * shape of counts, data_offsets pair, byte length = elements * dtype size), sorted by data_start,
 * overlaps refused when reject_overlaps (the reference's default). `bytes` holds at least the
 * prefix and the header. */
int g4_st_parse(const uint8_t *bytes, size_t n, int reject_overlaps, g4_st **out);
/* Opens a local file: reads its prefix and header, parses them, and keeps the file for payload
 * reads. Refuses a payload that runs past the end of the file. */
int g4_st_open(const char *path, g4_st **out);
int g4_st_close(g4_st *st);

/* Directory geometry: header length, payload start (8 + header length), payload length (the
 * largest data_end), file length implied by the header. */
int g4_st_info(const g4_st *st, int64_t *header_length, int64_t *payload_start,
               int64_t *payload_length, int64_t *file_length);
int64_t g4_st_count(const g4_st *st);
/* Tensor i in payload order. */
int g4_st_tensor_at(const g4_st *st, int64_t i, g4_st_tensor *out);
/* A tensor by name, through the ties once g4_st_apply_ties has run (lookupTensor). */
int g4_st_find(const g4_st *st, const char *name, g4_st_tensor *out);
/* A __metadata__ value (non-string values as their JSON text), or NULL. */
const char *g4_st_metadata(const g4_st *st, const char *key);
/* coverageGaps: payload spans no tensor claims; writes up to cap pairs, returns the count. */
int64_t g4_st_coverage_gaps(const g4_st *st, int64_t *starts, int64_t *ends, int64_t cap);

/* applyTies with the checkpoint's table (lm_head.weight -> embed_tokens.embedding_quantized,
 * lm_head.weight_scale -> embed_tokens.embedding_scale; safetensors.ts:616-637): the alias names
 * then resolve to the source entries. Refuses a table whose source the file lacks. */
int g4_st_apply_ties(g4_st *st);
/* The tie table: the number of ties, and tie i's alias, source and byte length. */
int g4_st_tie_count(void);
int g4_st_tie(int i, const char **alias, const char **source, int64_t *byte_length);

/* Payload reads (opened files only): `bytes` of tensor `name` starting `offset` bytes into it. */
int g4_st_read(const g4_st *st, const char *name, int64_t offset, void *host_dst, size_t bytes);
/* The whole tensor into device memory (a pinned bounce buffer, copies on `stream`, synchronous). */
int g4_st_upload(const g4_st *st, const char *name, void *device_dst, size_t dst_bytes,
                 void *stream);
/*
 * A tensor too large for one buffer, carried as one device buffer per slice (buffers.ts:291-327
 * declareSplit, :369-423 uploadWeight -> uploadSplitWeight). slices[i] gives the byte range
 * {byte_offset, byte_length} of slice i (a g4_table_slice from g4_plan_table_split); the ranges
 * must partition the tensor in offset order with four-byte-aligned starts, and slice_dst[i] holds
 * at least slices[i].byte_length bytes. The payload is read in pieces of up to 64 MiB; each
 * piece's intersection with each slice is written at its offset inside that slice (a piece that
 * straddles a boundary is two writes). Synchronous, like g4_st_upload.
 */
int g4_st_upload_split(const g4_st *st, const char *name, const g4_table_slice *slices,
                       int num_slices, void *const *slice_dst, void *stream);

/*
 * The PLE table's split for a device (engine.ts:308-345 declarePleSplit): rows from the tensor's
 * first dimension, row bytes = bytes / rows (refused when that is not whole), then
 * g4_plan_gather_split with `groups_per_row` f32 scales per row. Refuses an infeasible code plan
 * and a plan whose scale table does not fit one buffer (the sliced gather addresses scales by the
 * absolute row). plans->codes.single means no split is needed (upload the table whole); otherwise
 * up to max_slices code slices are written for g4_st_upload_split.
 */
int g4_st_plan_ple_split(const g4_st *st, const char *codes_name, int64_t groups_per_row,
                         const g4_gather_limits *limits, g4_gather_split_plans *plans,
                         g4_table_slice *slices, int64_t max_slices);

/* A BF16, F16 or F32 tensor widened exactly to f32 in device memory (the norm weights, the layer
 * scalar; quant.ts:400-411 bf16ToF32). */
int g4_st_upload_f32(const g4_st *st, const char *name, float *device_dst, int64_t count,
                     void *stream);

/* The tie guard (checkTieGuard, safetensors.ts:706-800): 1 when `revision` is the pinned one and
 * the 256 KiB sample of the embed tensor hashes to the pinned SHA-256, else 0 (fetch both
 * tensors). digest_hex (65 bytes, may be NULL) receives the sample's digest, reason (may be NULL)
 * the reference's prose. */
int g4_tie_guard(const uint8_t *sample, size_t n, const char *revision, char *digest_hex,
                 char *reason, size_t reason_len);
/* SHA-256 (FIPS 180-4) of n bytes as 64 lowercase hex digits plus NUL. */
void g4_sha256_hex(const uint8_t *data, size_t n, char *out65);

/* resolveQuantBits (quant.ts:430-513): the bit width of a module path by the QUANT_RULES table
 * (leftmost match, the earlier rule on a tie; 4 when none matches), or 0 when the checkpoint
 * stores the module unquantized (modules_to_not_convert, norms, layer_scalar, KV cache scales). */
int g4_quant_bits(const char *module_path);
/* modulePathForTensor (quant.ts:649-663): the tensor name without its stored suffix. */
int g4_module_path_for_tensor(const char *tensor_name, char *buf, size_t len);

/* textTensorNames (safetensors.ts:930-985): the allow list for `layers` layers of which the last
 * `kv_shared` share KV, newline-separated into buf (NUL-terminated); returns the name count, and
 * writes *needed (bytes incl. the NUL) so a first call with buf NULL sizes the buffer. */
int64_t g4_text_tensor_names(int layers, int kv_shared, int fetch_tied_pair, char *buf,
                             size_t len, size_t *needed);

#ifdef __cplusplus
}
#endif

#endif /* G4CKPT_H */
