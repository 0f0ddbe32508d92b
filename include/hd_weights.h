#ifndef HD_WEIGHTS_HIP_H
#define HD_WEIGHTS_HIP_H

/*
 * Device weight store: the subset of the reference's hd_weight_store
 * (src/model/weights.h:75-106) that the block/forward bindings read - a
 * table of named device allocations, optionally carved from one arena.
 * Loading real GGUF packs is not part of this library; callers (tests, the
 * bench driver) fill the table with device pointers they own.
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    void *dev_ptr;
    int64_t nbytes;
    char name[256];
} hd_device_alloc;            /* weights.h:75-79 */

typedef struct {
    int device_id;
    hd_device_alloc *allocs;  /* [n_allocs], caller owned */
    int64_t n_allocs;
    void *arena_ptr;          /* optional single arena (weights.h:99-104) */
    int64_t arena_bytes;
    void *upload_stream;      /* hipStream_t used by the LoRA merge */
} hd_weight_store;

/* Looks a tensor up by exact name; NULL when absent. */
const void *hd_weight_store_find(const hd_weight_store *s, const char *name);

#ifdef __cplusplus
}
#endif

#endif /* HD_WEIGHTS_HIP_H */
