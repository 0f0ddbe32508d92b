#ifndef HD_WEIGHTS_HIP_H
#define HD_WEIGHTS_HIP_H

/*
 * Device weight store (replaces src/model/weights.h:75-147 for the device
 * side; same struct layouts): a table of named device allocations, normally
 * carved from one arena, filled by the GGUF pack loader or by the caller.
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"
#include "hd_gemm.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    void *dev_ptr;
    int64_t nbytes;
    char name[256];
} hd_device_alloc;            /* weights.h:75-79 */

typedef struct {              /* weights.h:81-106 */
    int device_id;
    char device_name[256];
    int compute_major;
    int compute_minor;
    int64_t device_mem_bytes;
    int64_t host_bytes_loaded;
    int64_t device_bytes_allocated;
    int64_t n_allocations;
    int64_t largest_numel;
    char largest_name[256];
    hd_device_alloc *allocs;
    int64_t n_allocs;
    hd_gemm_runtime *gemm;    /* created by the loader, freed with the store */
    void *arena_ptr;          /* when set, every allocs[i].dev_ptr is inside it */
    int64_t arena_bytes;
    void *upload_stream;      /* hipStream_t */
} hd_weight_store;

/* weights.h:109: device identity (name = gfx arch name, compute_major/minor =
 * the gfx major/minor) without allocating model memory. HD_ERR_PROFILE for a
 * device id that is not visible. */
hd_status hd_device_info(int device_id, hd_weight_store *out);

/* weights.h:129: loads a GGUF pack into one device arena. The payload
 * streams from the file through pinned staging slots into the arena on the
 * store's upload stream (reads overlap the copies); tensor i is bound at
 * arena + offset_i. Creates the store's GEMM runtime. */
hd_status hd_weights_to_device_gguf(const char *gguf_path, int device_id, hd_weight_store *out);

/* weights.h:132: frees the arena (or each allocation when there is no
 * arena), the upload stream, the GEMM runtime and the table. */
void hd_weight_store_free(hd_weight_store *s);

const char *hd_weights_last_error(void);

/* Looks a tensor up by exact name; NULL when absent. */
const void *hd_weight_store_find(const hd_weight_store *s, const char *name);

#ifdef __cplusplus
}
#endif

#endif /* HD_WEIGHTS_HIP_H */
