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

/* include/hd_lora.h:75. `stream` is a hipStream_t (NULL = library stream).
 * Returns HD_OK, HD_ERR_MISSING on a null pointer, HD_ERR_UNSUPPORTED on a
 * rank above 256, HD_ERR_RUNTIME on a launch failure. */
hd_status hd_lora_merge_gpu(hd_lora_entry *entries, size_t count, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HD_LORA_HIP_H */
