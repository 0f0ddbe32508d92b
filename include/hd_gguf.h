#ifndef HD_GGUF_HIP_H
#define HD_GGUF_HIP_H

/*
 * GGUF v3 reader for the o1.c weight pack (replaces src/io/gguf.h:1-70, same
 * names, struct layouts and status codes).
 *
 * Layout (little-endian): u32 magic "GGUF", u32 version (3), u64 tensor
 * count, u64 KV count, the KV pairs, the tensor infos (name, n_dims <= 8,
 * dims, ggml type, offset relative to the data section), padding to
 * general.alignment (u32 KV; 32 when absent), then the tensor data.
 * Recognised KVs: general.architecture / general.name / hidream.profile /
 * hidream.variant / hidream.revision / hidream.dtype / hidream.quantization
 * (strings) and hidream.num_layers / hidream.layout_version (strings holding
 * decimal integers, as the pack writes them); every other KV is skipped.
 * Tensor types: F32, F16, BF16 (others fail the parse).
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HD_GGML_TYPE_F32 0
#define HD_GGML_TYPE_F16 1
#define HD_GGML_TYPE_BF16 30

typedef struct {
    char *name;
    uint32_t n_dims;
    uint64_t dims[8];
    uint32_t type;        /* ggml type */
    uint64_t offset;      /* relative to the data section */
    uint64_t nbytes;
} hd_gguf_tensor;

typedef struct {
    char *path;
    int64_t n_tensors;
    hd_gguf_tensor *tensors;  /* file order */
    uint64_t alignment;
    uint64_t tensor_data_off; /* absolute offset of the data section */
    uint64_t payload_bytes;   /* max(offset + nbytes), rounded to alignment */
    char *arch;
    char *name;
    char *profile;
    char *variant;
    char *revision;
    char *dtype;
    char *quantization;
    int64_t num_layers;
    int64_t layout_version;
} hd_gguf_file;

/* gguf.h:60: parses the header and tensor table (no payload I/O).
 * HD_ERR_IO: open/short header; HD_ERR_PARSE: bad magic, version != 3,
 * tensor count 0 or > 2^20, malformed KV/tensor table, unknown type. */
hd_status hd_gguf_open(const char *path, hd_gguf_file *out);
void hd_gguf_close(hd_gguf_file *f);
/* gguf.h:64: reads one tensor's payload (nbytes) into dst. */
hd_status hd_gguf_read_tensor(const hd_gguf_file *f, const hd_gguf_tensor *t, void *dst);
const char *hd_gguf_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HD_GGUF_HIP_H */
