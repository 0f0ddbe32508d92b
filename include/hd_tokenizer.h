#ifndef HD_TOKENIZER_HIP_H
#define HD_TOKENIZER_HIP_H

/*
 * Prompt tokenizer (replaces src/model/tokenizer.h:1-95, same names, argument
 * meaning, status codes and error strings through hd_last_error()): the
 * Qwen2 byte-level BPE applied to the im-chat template, with the reference's
 * pre-tokenizer (ASCII letter / digit / whitespace classes, tokenizer.c:333-347)
 * and split-isolated special tokens (tokenizer.c:358-418). The reference
 * embeds its vocabulary and merge table at build time; this library reads
 * them from the files the model ships with (hd_tokenizer_load, an extension
 * with no reference counterpart). Every other entry point returns
 * HD_ERR_MISSING until a vocabulary is loaded. Host code, no GPU use; not
 * thread-safe (one process-wide tokenizer, as in the reference).
 */

#include <stddef.h>

#include "hidream_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HD_TOK_IDENTITY "Qwen2Tokenizer (GPT-2 byte-level BPE)"   /* tokenizer.h:30 */
#define HD_TOK_IM_START     151644                                /* tokenizer.h:33-38 */
#define HD_TOK_IM_END       151645
#define HD_TOK_VISION_START 151652
#define HD_TOK_VISION_END   151653
#define HD_TOK_IMAGE_PAD    151655
#define HD_TOK_VIDEO_PAD    151656

/* Extension: loads the vocabulary (vocab.json: {"piece": id, ...}), the merge
 * table (merges.txt: optional "#version" line, then "left right" per line in
 * rank order) and the special tokens (a tokenizer.json whose "added_tokens"
 * array holds {"id", "content"} objects, or such an array alone). Replaces
 * any loaded tokenizer. HD_ERR_IO: unreadable file; HD_ERR_PARSE: malformed. */
hd_status hd_tokenizer_load(const char *vocab_json, const char *merges_txt,
                            const char *added_tokens_json);
/* Extension: releases the loaded tokenizer. */
void hd_tokenizer_unload(void);

/* tokenizer.h:43-55: im-chat template for one user prompt (generation prompt
 * added), then hd_tokenizer_encode. *out_ids freed with hd_tokenizer_free_ids. */
hd_status hd_tokenizer_encode_prompt(const char *prompt, int **out_ids, size_t *out_count);
/* tokenizer.h:57-62: "<|im_start|>user\n" + prompt + "<|im_end|>\n<|im_start|>assistant\n";
 * *out freed with free(). */
hd_status hd_tokenizer_build_template(const char *prompt, char **out);
/* tokenizer.h:64-72: k x "<|vision_start|><|image_pad|><|vision_end|>" before
 * the caption in the user turn. */
hd_status hd_tokenizer_build_ref_template(const char *caption, int k, char **out);
/* tokenizer.h:74-80: special tokens matched atomically, plain runs
 * pre-tokenized and byte-level BPE'd; HD_ERR_PARSE when a piece is not in the
 * vocabulary (fails closed). */
hd_status hd_tokenizer_encode(const char *text, int **out_ids, size_t *out_count);
/* tokenizer.h:82-83: id of a special-token string, -1 if unknown or nothing loaded. */
int hd_tokenizer_special_id(const char *content);
/* tokenizer.h:85-86 */
void hd_tokenizer_free_ids(int *ids);

#ifdef __cplusplus
}
#endif

#endif
