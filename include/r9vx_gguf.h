/*
 * r9vx_gguf.h -- GGUF ingestion for the quantized matrix path: the container
 * reader, per-entry checksums, split shard sets, and the load step that puts
 * a checkpoint's Q4_K / IQ4_XS tensors into device memory in the layout the
 * matmul and moe_ffn kernels read.
 *
 * Mirrors crates/r9v-format/src/container.rs (GgufFile, ShardSet) for
 * standard GGUF v2/v3 files.  Native R9V containers (r9v.* metadata or tensor
 * type ids 1001-1022, container.rs:2119) are refused: this path consumes
 * GGUF wire blocks as they are, so R9V's repacked L0/L1 entries have no reader
 * here.
 *
 * Conventions: every function returns R9VX_OK (0) or a negative R9VX_ERR_*
 * (include/r9vx.h); r9vx_last_error() holds the text of the last refusal and
 * r9vx_gguf_last_problems() the R9VX_GGUF_P_* kinds of the last failed parse.
 * The parser copies nothing from the tensor data: tensor bytes are ranges of
 * the caller's buffer, which must outlive every use.  A parsed file is
 * immutable and may be read from several threads.
 */
#ifndef R9VX_GGUF_H
#define R9VX_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "r9vx.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Problem kinds of a refused parse; each is one FormatError variant of
 * crates/r9v-format/src/error.rs:160-270.  Several may be set at once
 * (FormatError::Multiple). */
#define R9VX_GGUF_P_TRUNCATED (1u << 0)        /* FormatError::Truncated */
#define R9VX_GGUF_P_BAD_MAGIC (1u << 1)        /* BadMagic */
#define R9VX_GGUF_P_BAD_VERSION (1u << 2)      /* UnsupportedVersion */
#define R9VX_GGUF_P_MALFORMED (1u << 3)        /* Malformed */
#define R9VX_GGUF_P_DUPLICATE_KEY (1u << 4)    /* DuplicateKey */
#define R9VX_GGUF_P_DUPLICATE_TENSOR (1u << 5) /* DuplicateTensor */
#define R9VX_GGUF_P_BAD_ALIGNMENT (1u << 6)    /* InvalidAlignment */
#define R9VX_GGUF_P_KV_TYPE (1u << 7)          /* KvTypeMismatch */
#define R9VX_GGUF_P_MISSING_KEY (1u << 8)      /* MissingKey */
#define R9VX_GGUF_P_UNKNOWN_TYPE (1u << 9)     /* UnknownTensorType */
#define R9VX_GGUF_P_BAD_RANGE (1u << 10)       /* BadTensorRange */
#define R9VX_GGUF_P_OVERFLOW (1u << 11)        /* Overflow */
#define R9VX_GGUF_P_NATIVE (1u << 12)          /* native R9V container: not read here */

/* Metadata value types (KvType, container.rs:60-88; gguf-py GGUFValueType). */
enum r9vx_gguf_kv_type {
    R9VX_KV_U8 = 0,
    R9VX_KV_I8 = 1,
    R9VX_KV_U16 = 2,
    R9VX_KV_I16 = 3,
    R9VX_KV_U32 = 4,
    R9VX_KV_I32 = 5,
    R9VX_KV_F32 = 6,
    R9VX_KV_BOOL = 7,
    R9VX_KV_STR = 8,
    R9VX_KV_ARRAY = 9,
    R9VX_KV_U64 = 10,
    R9VX_KV_I64 = 11,
    R9VX_KV_F64 = 12,
};

typedef struct r9vx_gguf r9vx_gguf;               /* one parsed shard */
typedef struct r9vx_gguf_shards r9vx_gguf_shards; /* an ordered split set */

/* One metadata item.  Integers and bool are in `bits` (signed types sign-
 * extended to 64 bits), f32 / f64 as their IEEE bit patterns; strings are
 * (str, str_len) into the parsed file, not NUL-terminated. */
typedef struct r9vx_gguf_value {
    uint32_t type; /* r9vx_gguf_kv_type of the item (never ARRAY) */
    uint32_t _pad;
    uint64_t bits;
    const char *str;
    uint64_t str_len;
} r9vx_gguf_value;

/* One tensor-info row (TensorInfo, container.rs:701-728).  dims are in file
 * order, innermost first (a matrix [N, K] is dims {K, N}). */
typedef struct r9vx_gguf_tensor {
    const char *name;     /* NUL-terminated, owned by the parsed file */
    uint64_t name_len;    /* bytes of the name (a GGUF name may hold NUL bytes) */
    const uint64_t *dims; /* n_dims entries, owned by the parsed file */
    uint32_t n_dims;
    uint32_t type;        /* GGUF tensor type code (12 = Q4_K, 23 = IQ4_XS, ...) */
    uint64_t offset;      /* relative to the data section start */
    uint64_t nbytes;      /* data bytes (TensorType::data_nbytes, container.rs:673) */
    uint32_t block_len;   /* weights per block (GGML_QUANT_SIZES) */
    uint32_t block_bytes; /* bytes per block */
} r9vx_gguf_tensor;

/* Replaces: GgufFile::parse (container.rs:930), parse_internal + validate
 * (:952-1470).  `bytes` holds the whole file.  Structural errors (magic,
 * version, truncation, malformed fields) stop at the first; table problems
 * (duplicates, alignment, split keys, tensor sizes, ranges, overlaps) are all
 * collected into one refusal. */
int r9vx_gguf_parse(const uint8_t *bytes, uint64_t len, r9vx_gguf **out);
/* Replaces: GgufFile::parse_metadata_only (container.rs:942): `bytes` holds at
 * least the header and both tables; tensor ranges are checked against
 * `file_size`, the size of the whole file. */
int r9vx_gguf_parse_table(const uint8_t *bytes, uint64_t len, uint64_t file_size, r9vx_gguf **out);
void r9vx_gguf_free(r9vx_gguf *f);
/* Problem kinds (R9VX_GGUF_P_*) of the last refused parse or shard-set open
 * on the calling thread; 0 after a success. */
uint32_t r9vx_gguf_last_problems(void);

/* GgufFile::version / alignment / data_start / file_size (container.rs:1472-1490). */
uint32_t r9vx_gguf_version(const r9vx_gguf *f);
uint64_t r9vx_gguf_alignment(const r9vx_gguf *f);
uint64_t r9vx_gguf_data_start(const r9vx_gguf *f);
uint64_t r9vx_gguf_file_size(const r9vx_gguf *f);
/* Byte ranges [begin, end) of the header, metadata table and tensor-info
 * table (header_range / kv_range / ti_range, container.rs:1512-1525). */
void r9vx_gguf_ranges(const r9vx_gguf *f, uint64_t out[6]);

/* Metadata table in file order (GgufFile::kvs / kv, container.rs:1492-1505). */
uint64_t r9vx_gguf_n_kv(const r9vx_gguf *f);
/* Index of `key`, or -1 when absent (a C string cannot name a key that
 * holds a NUL byte; such entries are reachable by index only). */
int64_t r9vx_gguf_find_kv(const r9vx_gguf *f, const char *key);
/* Key of entry i (NUL-terminated; key_len counts its bytes, since a GGUF key
 * may hold NUL bytes), its type, and for arrays the element type and length
 * (a scalar has length 1 and elem == type).  Any out pointer may be NULL. */
int r9vx_gguf_kv_info(const r9vx_gguf *f, uint64_t i, const char **key, uint64_t *key_len,
                      uint32_t *type, uint32_t *elem, uint64_t *count);
/* Item `item` of entry i (item 0 for a scalar). */
int r9vx_gguf_kv_value(const r9vx_gguf *f, uint64_t i, uint64_t item, r9vx_gguf_value *out);

/* Tensor table in file order (GgufFile::tensors / tensor, container.rs:1497-1510). */
uint64_t r9vx_gguf_n_tensors(const r9vx_gguf *f);
/* Index of tensor `name`, or -1 when absent. */
int64_t r9vx_gguf_find_tensor(const r9vx_gguf *f, const char *name);
int r9vx_gguf_tensor_at(const r9vx_gguf *f, uint64_t i, r9vx_gguf_tensor *out);
/* Replaces: GgufFile::tensor_bytes (container.rs:2074): the checked range of
 * tensor `name` inside `bytes` (the buffer that was parsed, or one holding the
 * same file). */
int r9vx_gguf_tensor_bytes(const r9vx_gguf *f, const char *name, const uint8_t *bytes,
                           uint64_t len, const uint8_t **data, uint64_t *nbytes);
/* Replaces: GgufFile::entry_xxh3 (container.rs:2136): XXH3-64 of the entry. */
int r9vx_gguf_entry_xxh3(const r9vx_gguf *f, const char *name, const uint8_t *bytes,
                         uint64_t len, uint64_t *hash);
/* Replaces: GgufFile::is_native (container.rs:2119); always 0 for a file this
 * reader accepted. */
int r9vx_gguf_is_native(const r9vx_gguf *f);

/* Wire geometry and name of a GGUF tensor type code (TensorType::quant_size
 * and name, container.rs:528-612).  Returns R9VX_ERR_UNSUPPORTED for a code
 * with no upstream meaning. */
int r9vx_gguf_type_size(uint32_t type, uint32_t *block_len, uint32_t *block_bytes);
const char *r9vx_gguf_type_name(uint32_t type);

/* XXH3-64 with seed 0 (r9v_common::xxh3_64, crates/r9v-common/src/hash.rs:12). */
uint64_t r9vx_xxh3_64(const void *data, uint64_t len);

/* Replaces: ShardSet::open (container.rs:3476).  The set refers to the
 * parsed shards (it does not own them); every split.* cross-check problem
 * is collected into one refusal. */
int r9vx_gguf_shards_open(const r9vx_gguf *const *shards, uint32_t n, r9vx_gguf_shards **out);
void r9vx_gguf_shards_free(r9vx_gguf_shards *s);
/* Merged tensor count (ShardSet::len, :3584). */
uint64_t r9vx_gguf_shards_len(const r9vx_gguf_shards *s);
/* ShardSet::tensor_at (:3595): merged row i, its shard index and its row. */
int r9vx_gguf_shards_tensor_at(const r9vx_gguf_shards *s, uint64_t i, uint32_t *shard,
                               r9vx_gguf_tensor *out);
/* ShardSet::tensor (:3606): shard index of `name`, or -1 when absent. */
int64_t r9vx_gguf_shards_find(const r9vx_gguf_shards *s, const char *name);

/* ---------------------------------------------------- binding and upload */

/* Variant key of a matmul over the 2-D Q4_K / IQ4_XS / Q6_K / Q8_0 / IQ3_S
 * tensor `name` (file dims {K, N}): sets st->n, st->k, st->w_scheme (the
 * SchemeId code of the tensor's GGUF type, r9vx_scheme_from_ggml_type) and the
 * w_dtype / w_layout of the device layout the weights must be loaded into,
 * leaves the other fields: Q4_K / IQ4_XS GGUF_WIRE (r9vx_gguf_upload copies
 * the blocks), IQ3_S IQ3S_112 (r9vx_gguf_upload repacks the 110-byte blocks
 * into 112-byte ones), Q6_K / Q8_0 SPLIT (r9vx_gguf_upload_split).  This is
 * the shape-and-scheme part of a MatmulStatic the loader derives from a
 * checkpoint (crates/r9v-registry/src/types.rs:727-770). */
int r9vx_gguf_matmul_static(const r9vx_gguf *f, const char *name, r9vx_matmul_static *st);
/* Variant key of a moe_ffn over stacked expert tensors: `gate` and `up`
 * (file dims {Dm, Dff, E} each) or one fused `gate` tensor {Dm, 2*Dff, E}
 * with up == NULL (the ffn_gate_up_exps form of
 * crates/r9v-models/src/generic.rs:1420), and `down` {Dff, Dm, E}.  Sets
 * e_local, dm, dff and the gate_up / down projection keys (dtype, SchemeId code and
 * the device layout the uploads write): Q4_K / IQ4_XS / IQ3_S through
 * r9vx_gguf_upload / r9vx_gguf_upload_gate_up, Q8_0 / Q6_K (split) through
 * r9vx_gguf_upload_split / r9vx_gguf_upload_gate_up_split. */
int r9vx_gguf_moe_ffn_static(const r9vx_gguf *f, const char *gate, const char *up,
                             const char *down, r9vx_moe_ffn_static *st);
/* Loads tensor `name` from the host buffer into device memory `dst` in the
 * device layout its static names, on `stream`; it replaces the load-time
 * repack to R9V's L1 layout (crates/r9v-format/src/repack.rs:282,
 * iq.rs:1155).  GGUF Q4_K / IQ4_XS blocks (and F32 tensors) are copied as
 * they are (dst_bytes >= the entry's size): the call returns after the copy
 * has been enqueued, and `bytes` must stay valid until the stream reaches
 * it.  IQ3_S blocks are repacked on the host into the 112-byte device blocks
 * (dst_bytes >= 112 per 110-byte block; a non-finite d is refused before
 * anything is copied) and the call returns after the copy has completed.
 * Q8_0 / Q6_K are refused: they load with r9vx_gguf_upload_split. */
int r9vx_gguf_upload(const r9vx_gguf *f, const uint8_t *bytes, uint64_t len, const char *name,
                     void *dst, uint64_t dst_bytes, r9vx_stream_t stream);
/* Loads a Q8_0 / Q6_K tensor into the split device layout of include/r9vx.h
 * (body + f16 d array), the load-time repack of these types: the blocks are
 * split on the host, non-finite d values are refused (check_wire_f16,
 * crates/r9v-format/src/ggml.rs:421) before anything is copied, and the call
 * returns after both copies have completed on `stream`. */
int r9vx_gguf_upload_split(const r9vx_gguf *f, const uint8_t *bytes, uint64_t len, const char *name,
                           void *body, uint64_t body_bytes, uint16_t *scales, uint64_t scales_bytes,
                           r9vx_stream_t stream);
/* Builds moe_ffn's w_gate_up [E, 2*Dff, Dm] in device memory from stacked
 * gate and up expert tensors [E, Dff, Dm] (which may sit in different shards):
 * expert e's gate rows, then its up rows (crates/r9v-t0/src/moe_ffn.rs:51-55),
 * with one strided copy per tensor.  IQ3_S experts are repacked on the host
 * into 112-byte device blocks first (dst_bytes >= 2 * 112 per 110-byte
 * block of one tensor), as r9vx_gguf_upload does. */
int r9vx_gguf_upload_gate_up(const r9vx_gguf *gate_file, const uint8_t *gate_bytes,
                             uint64_t gate_len, const char *gate, const r9vx_gguf *up_file,
                             const uint8_t *up_bytes, uint64_t up_len, const char *up, void *dst,
                             uint64_t dst_bytes, r9vx_stream_t stream);
/* The stacked w_gate_up [E, 2*Dff, Dm] of Q8_0 / Q6_K gate and up expert
 * tensors in the split device layout: expert x's gate rows then its up rows
 * in `body` (blocks without d) and their d values in `scales` (f16), the two
 * arrays moe_ffn takes as w_gate_up and w_gate_up_scales (the gate/up
 * stacking of crates/r9v-models/src/generic.rs:1420 with the split of
 * r9vx_gguf_upload_split).  Split on the host; a non-finite d is refused
 * before anything is copied; returns after the copies have completed. */
int r9vx_gguf_upload_gate_up_split(const r9vx_gguf *gate_file, const uint8_t *gate_bytes, uint64_t gate_len,
                                   const char *gate, const r9vx_gguf *up_file, const uint8_t *up_bytes,
                                   uint64_t up_len, const char *up, void *body, uint64_t body_bytes, uint16_t *scales,
                                   uint64_t scales_bytes, r9vx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* R9VX_GGUF_H */
