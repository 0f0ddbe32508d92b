/* Test infrastructure (the checker side, never shipped): writes the
 * reference tokenizer's embedded tables (compiled in place from
 * /root/reference/src/model/tokenizer_tables.h by oracle/ref.mk) as the
 * standard tokenizer files a model ships with, so the library's file-based
 * tokenizer can be loaded with exactly the reference's data:
 *   <dir>/vocab.json         {"piece": id, ...}
 *   <dir>/merges.txt         "#version: 0.2" then "left right" in rank order
 *   <dir>/added_tokens.json  [{"id": n, "content": "..."}, ...]
 * Output goes only to the directory given on the command line (oracle/_ref). */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tokenizer_tables.h"

static void json_str(FILE *f, const char *s) {
    fputc('"', f);
    for (const unsigned char *p = (const unsigned char *)s; *p; p++) {
        if (*p == '"' || *p == '\\') { fputc('\\', f); fputc(*p, f); }
        else if (*p < 0x20) fprintf(f, "\\u%04x", *p);
        else fputc(*p, f);
    }
    fputc('"', f);
}

static int by_rank(const void *a, const void *b) {
    int ra = hd_tok_merge_rank[*(const int *)a], rb = hd_tok_merge_rank[*(const int *)b];
    return ra < rb ? -1 : ra > rb;
}

int main(int argc, char **argv) {
    if (argc != 2) { fprintf(stderr, "usage: tok_dump <dir>\n"); return 2; }
    char path[4096];
    snprintf(path, sizeof path, "%s/vocab.json", argv[1]);
    FILE *f = fopen(path, "wb");
    if (!f) return 1;
    fputc('{', f);
    for (int i = 0; i < hd_tok_vocab_count; i++) {
        if (i) fputc(',', f);
        json_str(f, hd_tok_vocab_str[i]);
        fprintf(f, ":%d", hd_tok_vocab_id[i]);
    }
    fputs("}\n", f);
    fclose(f);
    int *order = malloc(sizeof(int) * hd_tok_merge_count);
    for (int i = 0; i < hd_tok_merge_count; i++) order[i] = i;
    qsort(order, hd_tok_merge_count, sizeof(int), by_rank);
    snprintf(path, sizeof path, "%s/merges.txt", argv[1]);
    f = fopen(path, "wb");
    if (!f) return 1;
    fputs("#version: 0.2\n", f);
    for (int i = 0; i < hd_tok_merge_count; i++)
        fprintf(f, "%s %s\n", hd_tok_merge_left[order[i]], hd_tok_merge_right[order[i]]);
    fclose(f);
    free(order);
    snprintf(path, sizeof path, "%s/added_tokens.json", argv[1]);
    f = fopen(path, "wb");
    if (!f) return 1;
    fputc('[', f);
    for (int i = 0; i < hd_tok_special_count; i++) {
        if (i) fputc(',', f);
        fprintf(f, "{\"id\":%d,\"content\":", hd_tok_special_id[i]);
        json_str(f, hd_tok_special_str[i]);
        fputc('}', f);
    }
    fputs("]\n", f);
    fclose(f);
    return 0;
}
