#ifndef HIDREAM_HIP_H
#define HIDREAM_HIP_H

/*
 * Status codes and the process-global error string of the o1 MI355X engine.
 *
 * Replaces the status/error part of the reference's public header
 * (include/hidream.h:24-40, model.c:13-20): same enum names and values, so
 * callers written against the reference compile unchanged.
 */

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    HD_OK = 0,
    HD_ERR_IO = 1,
    HD_ERR_PARSE = 2,
    HD_ERR_PROFILE = 3,
    HD_ERR_MANIFEST = 4,
    HD_ERR_MISMATCH = 5,
    HD_ERR_MISSING = 6,      /* null argument / missing tensor            */
    HD_ERR_OOM = 7,          /* scratch or workspace too small, alloc fail */
    HD_ERR_RUNTIME = 8,      /* HIP runtime / kernel launch failure        */
    HD_ERR_UNSUPPORTED = 9,  /* shape or feature not supported (fail closed) */
} hd_status;

/* Last error set by the block / forward / LoRA layers (hidream.h:37). */
const char *hd_last_error(void);
/* printf-style setter shared by every module (hidream.h:40). */
void hd_set_error(const char *fmt, ...);

#ifdef __cplusplus
}
#endif

#endif /* HIDREAM_HIP_H */
