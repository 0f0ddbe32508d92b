#ifndef HD_LORA_HIP_H
#define HD_LORA_HIP_H

/*
 * Merge-on-load LoRA on the GPU:
 *   W' = bf16( float(W) + multiplier * (alpha / rank) * (up @ down) )
 * down [rank, in_dim] fp32, up [out_dim, rank] fp32, W [out_dim, in_dim]
 * bf16 mutated in place.
 *
 * Replaces hd_lora_merge_gpu of the reference (include/hd_lora.h:75,
 * src/model/lora_merge.cu:35-104). The reference forms the fp32 delta with
 * cuBLAS into a 64 MiB row-chunk buffer and adds it in a second kernel;
 * here one kernel computes each delta element in registers (rank-r dot
 * product, fp32) and does the read-modify-write of W, so the delta never
 * touches HBM and no scratch is allocated.
 */

#include <stddef.h>
#include <stdint.h>

#include "hd_weights.h"
#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* include/hd_lora.h:32-45 (the parser-side fields are kept for layout
 * compatibility; only rank/in_dim/out_dim/alpha/multiplier and the three
 * device pointers are read by the merge). */
typedef struct {
    char lora_prefix[256];
    char base_tensor[256];
    uint32_t rank;
    uint32_t in_dim;
    uint32_t out_dim;
    float alpha;
    float multiplier;
    void *down_dev;
    void *up_dev;
    void *base_dev;
} hd_lora_entry;

/* include/hd_lora.h:47-61 */
typedef struct {
    hd_lora_entry *entries;
    size_t count;
    char sha256[65];
    char base_profile[16];
} hd_lora_adapter;

typedef struct {              /* one adapter path and its multiplier */
    const char *path;
    float multiplier;
} hd_lora_spec;

typedef struct {
    const hd_lora_spec *items;
    size_t count;
} hd_lora_config;

/* include/hd_lora.h:71 (src/model/lora.c:126-375): parses every adapter
 * (musubi .safetensors: "<prefix>.lora_down.weight" [rank, in],
 * "<prefix>.lora_up.weight" [out, rank], optional scalar "<prefix>.alpha",
 * default alpha = rank; BF16 / F16 / F32), validates every target against
 * the dev profile's 257 linear layers and the store, then uploads the
 * factors as fp32 and merges them into the store's bf16 weights in place on
 * store->upload_stream (synchronised before returning). A parse or
 * validation error returns before any weight is touched. Each entry takes
 * the factors of its own adapter (the reference fills a target named by two
 * adapters from the first one it reads for both). count == 0 is a no-op. */
hd_status hd_lora_apply(const hd_lora_config *cfg, hd_weight_store *store, int device_id);

/* include/hd_lora.h:79: last error of hd_lora_apply. */
const char *hd_lora_last_error(void);

/* include/hd_lora.h:75. `stream` is a hipStream_t (NULL = library stream).
 * Returns HD_OK, HD_ERR_MISSING on a null pointer, HD_ERR_UNSUPPORTED on a
 * rank above 256, HD_ERR_RUNTIME on a launch failure (every entry is
 * checked before the GPU is touched). Entries of one (out, in, rank) shape
 * that the streaming kernel takes merge in one launch; entries on the same
 * weight merge in entry order. Like the reference's merge (which allocates
 * and frees a delta scratch per call), the call allocates a small device
 * list of the batched targets (32 bytes each), and synchronises `stream`
 * before freeing it. */
hd_status hd_lora_merge_gpu(hd_lora_entry *entries, size_t count, void *stream);


#ifdef __cplusplus
}
#endif

#endif /* HD_LORA_HIP_H */
