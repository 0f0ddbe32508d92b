// Sequence builders: token ids, fix-point MRoPE positions, the additive bf16
// mask and image-row flags for text-to-image and reference (edit /
// personalize) requests. Host code.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../include/hd_sequence.h"

namespace {
constexpr uint16_t kMaskMin = 0xFF7Fu;   // lowest finite bf16 (-3.3895e38)
constexpr int64_t kBoiToken = 151669;    // <|boi_token|>

// predefined output resolutions (all near 2048^2), in the order the
// reference searches them (sequence.c:28-33)
constexpr int kRes[][2] = {{2048, 2048}, {2304, 1728}, {1728, 2304}, {2560, 1440},
                           {1440, 2560}, {2496, 1664}, {1664, 2496}, {3104, 1312},
                           {1312, 3104}, {2304, 1792}, {1792, 2304}};

template <class T> T *hmalloc(size_t n) { return (T *)malloc(n * sizeof(T) ? n * sizeof(T) : 1); }

// mask rows: token rows attend everywhere, other rows causally
void fill_mask(unsigned char *mask, int S, const std::vector<unsigned char> &token_row) {
    for (int r = 0; r < S; r++)
        for (int c = 0; c < S; c++) {
            const uint16_t v = (!token_row[r] && c > r) ? kMaskMin : 0;
            mask[((size_t)r * S + c) * 2] = (unsigned char)(v & 0xFF);
            mask[((size_t)r * S + c) * 2 + 1] = (unsigned char)(v >> 8);
        }
}

void set_pos(float *pos, int S, int idx, float a, float b, float c) {
    pos[idx] = a;
    pos[S + idx] = b;
    pos[2 * S + idx] = c;
}
}  // namespace

extern "C" void hd_resolution_snap(int width, int height, int *out_w, int *out_h) {
    int best = 0;
    if (width > 0 && height > 0) {
        const double ratio = (double)width / (double)height;
        double best_d = INFINITY;
        for (int i = 0; i < (int)(sizeof(kRes) / sizeof(kRes[0])); i++) {
            const double d = fabs((double)kRes[i][0] / (double)kRes[i][1] - ratio);
            if (d < best_d) {
                best_d = d;
                best = i;
            }
        }
    }
    if (out_w) *out_w = kRes[best][0];
    if (out_h) *out_h = kRes[best][1];
}

extern "C" void hd_sequence_free(hd_sequence *s) {
    if (!s) return;
    free(s->input_ids);
    free(s->pos_f32);
    free(s->mask_bf16);
    free(s->vinput_mask);
    memset(s, 0, sizeof(*s));
}

extern "C" hd_status hd_seq_t2i(const int64_t *ids, int text_len, int height, int width, int patch,
                                int image_token_id, int video_token_id, int vision_start_token_id,
                                int tms_token_id, int timestep_token_num, int spatial_merge_size,
                                int fix_point, hd_sequence *out) {
    (void)image_token_id; (void)video_token_id; (void)vision_start_token_id;
    (void)tms_token_id; (void)timestep_token_num; (void)spatial_merge_size;
    if (!ids || !out || text_len <= 0 || height <= 0 || width <= 0 || patch <= 0) {
        hd_set_error("sequence: bad t2i args");
        return HD_ERR_MISSING;
    }
    memset(out, 0, sizeof(*out));
    const int gh = height / patch, gw = width / patch, img = gh * gw, S = text_len + img;
    out->input_ids = hmalloc<int64_t>(text_len);
    out->pos_f32 = hmalloc<float>((size_t)3 * S);
    out->mask_bf16 = hmalloc<unsigned char>((size_t)S * S * 2);
    out->vinput_mask = hmalloc<unsigned char>(S);
    if (!out->input_ids || !out->pos_f32 || !out->mask_bf16 || !out->vinput_mask) {
        hd_sequence_free(out);
        hd_set_error("sequence: out of host memory (S=%d)", S);
        return HD_ERR_OOM;
    }
    memcpy(out->input_ids, ids, (size_t)text_len * sizeof(int64_t));
    for (int i = 0; i < text_len; i++) set_pos(out->pos_f32, S, i, (float)i, (float)i, (float)i);
    for (int h = 0; h < gh; h++)
        for (int w = 0; w < gw; w++)
            set_pos(out->pos_f32, S, text_len + h * gw + w, (float)fix_point, (float)(fix_point + h),
                    (float)(fix_point + w));
    std::vector<unsigned char> token_row(S, 0);
    for (int r = text_len - 1; r < S; r++) token_row[r] = 1;   // timestep token + image
    fill_mask(out->mask_bf16, S, token_row);
    for (int i = 0; i < S; i++) out->vinput_mask[i] = i >= text_len;
    out->sec[0] = 24; out->sec[1] = 20; out->sec[2] = 20;
    out->text_len = text_len;
    out->image_len = img;
    out->img_begin = text_len;
    out->S = S;
    return HD_OK;
}

extern "C" hd_status hd_seq_build_tokens(const int64_t *tpl, int tpl_len, int K, int patch,
                                         int image_token_id, int video_token_id, int vs_id,
                                         int tms_token_id, int timestep_token_num,
                                         int spatial_merge_size, int fix_point, int height,
                                         int width, const hd_ref_geom *refs, hd_sequence *out) {
    (void)video_token_id; (void)spatial_merge_size;
    if (!tpl || !out || tpl_len <= 0) {
        hd_set_error("sequence: null template");
        return HD_ERR_MISSING;
    }
    memset(out, 0, sizeof(*out));
    if (K < 0 || K > HD_SEQ_MAX_REFS || (K > 0 && !refs)) {
        hd_set_error("sequence: reference count out of range or geometry missing");
        return HD_ERR_MISSING;
    }
    if (height <= 0 || width <= 0 || patch <= 0 || timestep_token_num < 0) {
        hd_set_error("sequence: bad dims");
        return HD_ERR_MISSING;
    }
    for (int r = 0; r < K; r++)
        if (refs[r].cond_h <= 0 || refs[r].cond_w <= 0 || refs[r].tokens <= 0 ||
            refs[r].grid_h <= 0 || refs[r].grid_w <= 0) {
            hd_set_error("sequence: bad geometry for reference %d", r);
            return HD_ERR_MISSING;
        }
    const int gh = height / patch, gw = width / patch, img = gh * gw;

    // template: each (vision_start, image_pad) placeholder grows to the
    // reference's condition grid of pads
    std::vector<int64_t> ids;
    int placed = 0;
    for (int i = 0; i < tpl_len; i++) {
        if (tpl[i] == vs_id && i + 1 < tpl_len && tpl[i + 1] == image_token_id && placed < K) {
            ids.push_back(vs_id);
            ids.insert(ids.end(), (size_t)refs[placed].cond_h * refs[placed].cond_w, image_token_id);
            placed++;
            i++;
        } else {
            ids.push_back(tpl[i]);
        }
    }
    if (placed != K) {
        hd_set_error("sequence: expanded %d/%d reference placeholders", placed, K);
        return HD_ERR_MISSING;
    }
    const int tpl_n = (int)ids.size();
    ids.push_back(kBoiToken);
    ids.insert(ids.end(), (size_t)timestep_token_num, tms_token_id);
    const int text_len = (int)ids.size();
    // target block, then the reference blocks: vision_start + pads
    ids.push_back(vs_id);
    ids.insert(ids.end(), (size_t)(img > 0 ? img - 1 : 0), image_token_id);
    for (int r = 0; r < K; r++) {
        ids.push_back(vs_id);
        ids.insert(ids.end(), (size_t)refs[r].tokens - 1, image_token_id);
    }
    const int S = (int)ids.size();

    // positions: blocks in id order, each = a text run then a grid. The K
    // template blocks keep their vision_start in the text run and place the
    // grid right after it; the target and the K reference blocks count their
    // vision_start as the grid's first token, the target at fix_point and
    // each later block after the largest position so far.
    std::vector<int> vs;
    for (int i = 0; i < S; i++)
        if (ids[i] == vs_id) vs.push_back(i);
    if ((int)vs.size() != 2 * K + 1) {
        hd_set_error("sequence: %zu vision starts, expected %d", vs.size(), 2 * K + 1);
        return HD_ERR_MISSING;
    }
    std::vector<float> pos((size_t)3 * S, 0.f);
    int max_pos = -1, st = 0, fp = fix_point;
    for (int v = 0; v < 2 * K + 1; v++) {
        const bool skip = v >= K;
        int tlen = vs[v] + 1 - st - (skip ? 1 : 0);
        if (tlen < 0) tlen = 0;
        const int st_idx = max_pos >= 0 ? max_pos + 1 : 0;
        for (int i = 0; i < tlen; i++)
            set_pos(pos.data(), S, st + i, (float)(st_idx + i), (float)(st_idx + i), (float)(st_idx + i));
        max_pos = st_idx + tlen - 1;
        int bh, bw;
        if (v < K) { bh = refs[v].cond_h; bw = refs[v].cond_w; }
        else if (v == K) { bh = gh; bw = gw; }
        else { bh = refs[v - K - 1].grid_h; bw = refs[v - K - 1].grid_w; }
        if (bh <= 0 || bw <= 0) {
            hd_set_error("sequence: empty grid for block %d", v);
            return HD_ERR_MISSING;
        }
        int base;
        if (skip) {
            if (fp > 0) fp -= st_idx;
            base = fp + st_idx;
            fp = 0;
        } else {
            base = tlen + st_idx;
        }
        for (int h = 0; h < bh; h++)
            for (int w = 0; w < bw; w++)
                set_pos(pos.data(), S, st + tlen + h * bw + w, (float)base, (float)(base + h),
                        (float)(base + w));
        const int gmax = base + (bh > bw ? bh : bw) - 1;
        if (gmax > max_pos) max_pos = gmax;
        st += tlen + bh * bw;
    }
    for (int i = st; i < S; i++) {
        const float p = (float)(max_pos + 1 + (i - st));
        set_pos(pos.data(), S, i, p, p, p);
    }

    // row kinds: timestep tokens, target and reference rows attend fully;
    // target and reference rows take pixel input
    std::vector<unsigned char> kind(S, 0);   // 0 text, 1 target, 2 reference, 3 timestep
    for (int i = tpl_n + 1; i < text_len; i++) kind[i] = 3;
    for (int i = text_len; i < text_len + img; i++) kind[i] = 1;
    for (int i = text_len + img; i < S; i++) kind[i] = 2;
    std::vector<unsigned char> token_row(S);
    for (int i = 0; i < S; i++) token_row[i] = kind[i] != 0;

    out->input_ids = hmalloc<int64_t>(S);
    out->pos_f32 = hmalloc<float>((size_t)3 * S);
    out->mask_bf16 = hmalloc<unsigned char>((size_t)S * S * 2);
    out->vinput_mask = hmalloc<unsigned char>(S);
    if (!out->input_ids || !out->pos_f32 || !out->mask_bf16 || !out->vinput_mask) {
        hd_sequence_free(out);
        hd_set_error("sequence: out of host memory (S=%d)", S);
        return HD_ERR_OOM;
    }
    memcpy(out->input_ids, ids.data(), (size_t)S * sizeof(int64_t));
    memcpy(out->pos_f32, pos.data(), pos.size() * sizeof(float));
    fill_mask(out->mask_bf16, S, token_row);
    for (int i = 0; i < S; i++) out->vinput_mask[i] = kind[i] == 1 || kind[i] == 2;
    out->sec[0] = 24; out->sec[1] = 20; out->sec[2] = 20;
    out->text_len = text_len;
    out->image_len = img;
    out->img_begin = text_len;
    out->S = S;
    out->n_refs = K;
    int at = text_len + img;
    for (int r = 0; r < K; r++) {
        out->ref_len[r] = refs[r].tokens;
        out->ref_begin[r] = at;
        at += refs[r].tokens;
    }
    return HD_OK;
}

extern "C" int hd_seq_diag(const hd_sequence *s, const char *tag) {
    if (!s || !s->pos_f32) return 1;
    fprintf(stderr, "[seq %s] S=%d text=%d image=%d (rows %d..%d) refs=%d", tag ? tag : "", s->S,
            s->text_len, s->image_len, s->img_begin, s->img_begin + s->image_len - 1, s->n_refs);
    for (int r = 0; r < s->n_refs; r++) fprintf(stderr, " [%d+%d]", s->ref_begin[r], s->ref_len[r]);
    const int S = s->S;
    fprintf(stderr, " sec=%lld/%lld/%lld pos[last]=(%g,%g,%g)\n", (long long)s->sec[0],
            (long long)s->sec[1], (long long)s->sec[2], s->pos_f32[S - 1], s->pos_f32[2 * S - 1],
            s->pos_f32[3 * S - 1]);
    return 0;
}
