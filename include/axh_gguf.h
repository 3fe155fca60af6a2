/*
 * axh_gguf: reader for GGUF model files (ggml's on-disk format, versions 2
 * and 3), so tensors of real checkpoints can be uploaded and fed to the
 * matvec kernels.  No counterpart in the reference, which has no loader
 * ("GGUF file parsing - separate", ROADMAP.md:230-234); the layout is the
 * published GGUF specification (ggml docs/gguf.md).
 *
 * The file is mapped read-only for the life of the handle; pointers and
 * names handed out stay valid until axh_gguf_close.  Malformed files
 * (truncation, bad counts, misaligned or out-of-file tensors, unknown value
 * types) fail axh_gguf_open with AXH_ERR_METADATA_PARSE and a message.
 */
#ifndef AXH_GGUF_H
#define AXH_GGUF_H

#include "axh.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct axh_gguf axh_gguf;

/* GGUF metadata value types. */
enum {
    AXH_GGUF_U8 = 0, AXH_GGUF_I8 = 1, AXH_GGUF_U16 = 2, AXH_GGUF_I16 = 3, AXH_GGUF_U32 = 4,
    AXH_GGUF_I32 = 5, AXH_GGUF_F32 = 6, AXH_GGUF_BOOL = 7, AXH_GGUF_STRING = 8,
    AXH_GGUF_ARRAY = 9, AXH_GGUF_U64 = 10, AXH_GGUF_I64 = 11, AXH_GGUF_F64 = 12
};

typedef struct axh_gguf_tensor_info {
    const char *name;   /* NUL-terminated copy of the tensor name */
    uint32_t type;      /* AXH_GGML_* */
    uint32_t n_dims;    /* 1..4 */
    uint64_t ne[4];     /* elements per dimension, ne[0] innermost (a row); unused dims 1 */
    uint64_t offset;    /* absolute file offset of the data */
    uint64_t nbytes;    /* data bytes (0 for a type without a known block size) */
} axh_gguf_tensor_info;

typedef struct axh_gguf_kv_info {
    const char *key;     /* NUL-terminated copy of the key */
    uint32_t type;       /* AXH_GGUF_* */
    uint32_t item_type;  /* arrays: item type */
    uint64_t count;      /* arrays: items; strings: bytes */
    const void *value;   /* scalars: the value; strings: the bytes (no NUL); arrays: the
                            first item (strings in arrays are u64 length + bytes each) */
} axh_gguf_kv_info;

axh_status axh_gguf_open(const char *path, axh_gguf **out);
void axh_gguf_close(axh_gguf *g);
uint32_t axh_gguf_version(const axh_gguf *g);
uint32_t axh_gguf_alignment(const axh_gguf *g);
uint64_t axh_gguf_data_offset(const axh_gguf *g);
uint64_t axh_gguf_tensor_count(const axh_gguf *g);
uint64_t axh_gguf_kv_count(const axh_gguf *g);
axh_status axh_gguf_tensor_at(const axh_gguf *g, uint64_t i, axh_gguf_tensor_info *out);
axh_status axh_gguf_find_tensor(const axh_gguf *g, const char *name, uint64_t *index);
/* Host pointer to tensor i's bytes inside the mapping (NULL if out of range). */
const void *axh_gguf_tensor_data(const axh_gguf *g, uint64_t i);
/* Copies tensor i into device memory dst (capacity bytes available). */
axh_status axh_gguf_upload_tensor(axh_context *ctx, const axh_gguf *g, uint64_t i, void *dst,
                                  uint64_t capacity);
axh_status axh_gguf_kv_at(const axh_gguf *g, uint64_t i, axh_gguf_kv_info *out);
axh_status axh_gguf_find_kv(const axh_gguf *g, const char *key, uint64_t *index);

#ifdef __cplusplus
}
#endif
#endif
