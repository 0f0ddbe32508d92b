#ifndef HD_SEQUENCE_HIP_H
#define HD_SEQUENCE_HIP_H

/*
 * Sequence builders (replaces src/runtime/sequence.h:39-116; same structs,
 * names and status codes): token ids, MRoPE position ids [3, S] with the
 * fix-point semantics, the [S, S] bf16 additive mask (min-bf16 0xFF7F above
 * the diagonal on text rows, token rows zeroed) and the [S] image-row flags.
 * All arrays are host memory owned by the hd_sequence (hd_sequence_free).
 */

#include <stddef.h>
#include <stdint.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HD_SEQ_MAX_REFS 20

typedef struct {              /* sequence.h:40-46 */
    int tokens;               /* reference token count (grid_h * grid_w) */
    int grid_h, grid_w;       /* reference grid in patches */
    int cond_h, cond_w;       /* VLM condition grid (template image pads) */
} hd_ref_geom;

typedef struct {              /* sequence.h:48-63 */
    int64_t *input_ids;       /* [S] for hd_seq_build*, [text_len] for hd_seq_t2i */
    float *pos_f32;           /* [3, S] */
    unsigned char *mask_bf16; /* [S, S] bf16 */
    unsigned char *vinput_mask; /* [S] */
    int64_t sec[3];           /* MRoPE sections (24, 20, 20) */
    int text_len;
    int image_len;
    int img_begin;
    int S;
    int n_refs;
    int ref_len[HD_SEQ_MAX_REFS];
    int ref_begin[HD_SEQ_MAX_REFS];
} hd_sequence;

/* sequence.h:70: closest of the predefined ~2048^2 resolution buckets by
 * aspect ratio; non-positive inputs give 2048 x 2048. */
void hd_resolution_snap(int width, int height, int *out_w, int *out_h);

/* sequence.h:81: text-to-image sequence: text rows at (i, i, i), the
 * (height/patch) x (width/patch) image grid at fix_point + (0, r, c); rows
 * from text_len - 1 on (the timestep token and the image) attend fully. */
hd_status hd_seq_t2i(const int64_t *input_ids, int text_len, int height, int width,
                     int patch_size, int image_token_id, int video_token_id,
                     int vision_start_token_id, int tms_token_id, int timestep_token_num,
                     int spatial_merge_size, int fix_point, hd_sequence *out);

/* Extension: hd_seq_build (sequence.c:166-455) from an already tokenized
 * template (the reference tokenizes req->prompt itself; the tokenizer is not
 * part of this library). template_ids: <|im_start|>user\n + K x
 * (vision_start, image_pad, vision_end) + caption + tail, one placeholder pad
 * per reference. The pads are expanded to cond_h x cond_w, boi and
 * timestep_token_num tms tokens appended, then the target block and the K
 * reference blocks (vision_start + pads); positions follow
 * get_rope_index_fix_point with skip_vision_start = [0]*K + [1] + [1]*K. */
hd_status hd_seq_build_tokens(const int64_t *template_ids, int template_len, int reference_count,
                              int patch_size, int image_token_id, int video_token_id,
                              int vision_start_token_id, int tms_token_id,
                              int timestep_token_num, int spatial_merge_size, int fix_point,
                              int height, int width, const hd_ref_geom *refs, hd_sequence *out);

/* sequence.h:108 */
void hd_sequence_free(hd_sequence *s);

/* sequence.h:116: prints the sequence manifest to stderr; 0 on success. */
int hd_seq_diag(const hd_sequence *s, const char *tag);

#ifdef __cplusplus
}
#endif

#endif /* HD_SEQUENCE_HIP_H */
