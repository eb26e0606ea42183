/* glmssd_gguf.h — GGUF v3 header reader of libglmssd_hip.so (host code, no GPU).
 *
 * Mirrors GLM-SSD's crates/gguf (src/lib.rs): only the header is parsed (metadata key/values
 * and tensor infos); tensor data is never read. A split model (`*-00001-of-0000N.gguf`, any
 * shard may be named) opens as one logical model whose tensors carry absolute
 * (shard, offset, n_bytes) locations. The file is untrusted: counts, string and array lengths,
 * nesting, alignment and every size are bounded and computed with overflow checks, so a crafted
 * header is an error, never a crash or a huge allocation (lib.rs:1-31, 283-395).
 *
 * Return values: 0 on success, GS_GGUF_ERR (-1) on failure with the reason in gs_gguf_error()
 * (thread-local, valid until the next call on the same thread). Handles are not thread-safe.
 */
#ifndef GLMSSD_GGUF_H
#define GLMSSD_GGUF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_GGUF_ERR (-1)
#define GS_GGUF_NAME_MAX 256 /* longest tensor name returned by gs_gguf_tensor (longer: error) */

/* limits of lib.rs:19-31 */
#define GS_GGUF_MAX_COUNT (1ull << 20) /* tensors / metadata keys per header */
#define GS_GGUF_MAX_LEN (1ull << 26)   /* bytes per metadata string */
#define GS_GGUF_MAX_ARR (1ull << 24)   /* elements per metadata array */
#define GS_GGUF_MAX_ALIGN (1ull << 20) /* largest general.alignment */

/* metadata value types (GGUF spec; lib.rs:263-292) */
enum {
    GS_GGUF_U8 = 0, GS_GGUF_I8 = 1, GS_GGUF_U16 = 2, GS_GGUF_I16 = 3, GS_GGUF_U32 = 4, GS_GGUF_I32 = 5,
    GS_GGUF_F32 = 6, GS_GGUF_BOOL = 7, GS_GGUF_STR = 8, GS_GGUF_ARR = 9, GS_GGUF_U64 = 10, GS_GGUF_I64 = 11,
    GS_GGUF_F64 = 12,
};

/* one tensor (lib.rs:86-95 TensorInfo); dims in GGML order, dims[0] contiguous */
typedef struct GsGgufTensor {
    char name[GS_GGUF_NAME_MAX];
    int n_dims;
    uint64_t dims[4];
    int ty;            /* ggml type id */
    int shard;         /* index into the shard list */
    uint64_t offset;   /* absolute byte offset inside the shard file */
    uint64_t n_bytes;
    uint64_t row_bytes; /* bytes of dims[0] elements */
} GsGgufTensor;

/* Open a model (lib.rs:125-160 Gguf::open / open_headers_only / open_shard). mode 0: every shard
 * of a split model, tensors must lie inside their files; 1: the same without the file-length
 * check (header-only copies); 2: exactly this one file. */
int gs_gguf_open(const char *path, int mode, void **handle);
void gs_gguf_close(void *handle);
const char *gs_gguf_error(void);

int gs_gguf_n_shards(void *handle);
/* path of shard i (NUL-terminated, truncated to n bytes: error if it does not fit) */
int gs_gguf_shard_path(void *handle, int i, char *buf, size_t n);

int gs_gguf_n_tensors(void *handle);
int gs_gguf_tensor(void *handle, int i, GsGgufTensor *out);
/* index of the tensor called name (lib.rs:162-164), or GS_GGUF_ERR */
int gs_gguf_find(void *handle, const char *name);
/* expert e's byte range of a tensor whose last dim counts experts (lib.rs:106-111 slice_range) */
int gs_gguf_slice_range(const GsGgufTensor *t, uint64_t e, uint64_t *offset, uint64_t *n_bytes);

/* metadata (lib.rs:165-183): value type of key (GS_GGUF_ERR if absent); integers and bools as
 * u64 (negative integers: error), any number as f64, strings copied NUL-terminated; for arrays the
 * element type and length */
int gs_gguf_kv_type(void *handle, const char *key);
int gs_gguf_kv_u64(void *handle, const char *key, uint64_t *out);
int gs_gguf_kv_f64(void *handle, const char *key, double *out);
int gs_gguf_kv_str(void *handle, const char *key, char *buf, size_t n);
int gs_gguf_kv_arr(void *handle, const char *key, int *elem_type, uint64_t *len);

#ifdef __cplusplus
}
#endif
#endif
