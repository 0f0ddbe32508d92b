// Prompt tokenizer: Qwen2 byte-level BPE over the im-chat template, with the
// reference's pre-tokenizer and special-token rules (src/model/tokenizer.c).
//
// Design (not a translation of the reference's code): the vocabulary, merge
// ranks and special tokens are read from the model's own files into hash
// maps; the pre-tokenizer is one hand-written scanner per alternative of the
// reference's ordered pattern list (tokenizer.c:333-347), tried in that order
// with the first non-empty match winning; BPE merges the adjacent pair of
// lowest rank, leftmost first, until none applies (tokenizer.c:248-318; the
// standard byte-level BPE rule).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/hd_tokenizer.h"

namespace {

struct Tokenizer {
    std::unordered_map<std::string, int> vocab;     // piece -> id
    std::unordered_map<std::string, int> merge;     // left + '\x01' + right -> rank
    std::vector<std::pair<std::string, int>> special;   // (content, id), ascending id
    std::string byte_piece[256];                    // GPT-2 byte -> unicode piece (UTF-8)
};
Tokenizer *g_tok = nullptr;

// ---- GPT-2 byte <-> unicode map: printable Latin-1 bytes map to
// themselves, the other 68 bytes to U+0100 onwards in byte order. ----------
void utf8_append(std::string &s, unsigned cp) {
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xF0 | (cp >> 18));
        s += (char)(0x80 | ((cp >> 12) & 0x3F));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
}
void build_byte_pieces(Tokenizer &t) {
    unsigned next = 256;
    for (int b = 0; b < 256; b++) {
        const bool printable = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        t.byte_piece[b].clear();
        utf8_append(t.byte_piece[b], printable ? (unsigned)b : next++);
    }
}

// ---- a small JSON reader (objects, arrays, strings with escapes, numbers,
// literals), enough for vocab.json and tokenizer.json ----------------------
struct Json {
    const char *p, *end;
    bool ok = true;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) { p++; return true; }
        return false;
    }
    bool hex4(unsigned &v) {
        if (end - p < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool str(std::string &out) {
        out.clear();
        if (!eat('"')) return false;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') { out += c; continue; }
            if (p >= end) return false;
            c = *p++;
            switch (c) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                unsigned v;
                if (!hex4(v)) return false;
                if (v >= 0xD800 && v < 0xDC00) {   // surrogate pair
                    unsigned lo;
                    if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return false;
                    p += 2;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                    v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8_append(out, v);
                break;
            }
            default: return false;
            }
        }
        return eat('"');
    }
    bool num(long long &v) {
        ws();
        char *q;
        v = strtoll(p, &q, 10);
        if (q == p) return false;
        p = q;
        if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {   // skip a fraction / exponent
            strtod(p - 0, &q);
            p = q;
        }
        return true;
    }
    // skips any value
    bool skip() {
        ws();
        if (p >= end) return false;
        std::string s;
        long long n;
        switch (*p) {
        case '"': return str(s);
        case '{':
            p++;
            if (eat('}')) return true;
            do {
                if (!str(s) || !eat(':') || !skip()) return false;
            } while (eat(','));
            return eat('}');
        case '[':
            p++;
            if (eat(']')) return true;
            do {
                if (!skip()) return false;
            } while (eat(','));
            return eat(']');
        case 't': if (end - p >= 4 && !strncmp(p, "true", 4)) { p += 4; return true; } return false;
        case 'f': if (end - p >= 5 && !strncmp(p, "false", 5)) { p += 5; return true; } return false;
        case 'n': if (end - p >= 4 && !strncmp(p, "null", 4)) { p += 4; return true; } return false;
        default: return num(n);
        }
    }
};

bool read_file(const char *path, std::string &out) {
    FILE *f = fopen(path, "rb");
    if (!f) return false;
    out.clear();
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    fclose(f);
    return true;
}

hd_status parse_vocab(const std::string &text, Tokenizer &t) {
    Json j{text.data(), text.data() + text.size()};
    if (!j.eat('{')) return HD_ERR_PARSE;
    if (j.eat('}')) return HD_OK;
    std::string key;
    do {
        long long id;
        if (!j.str(key) || !j.eat(':') || !j.num(id) || id < 0 || id > 0x7FFFFFFF) return HD_ERR_PARSE;
        t.vocab[key] = (int)id;
    } while (j.eat(','));
    return j.eat('}') ? HD_OK : HD_ERR_PARSE;
}

// {"id": n, "content": "..."} objects of an array (the root, or the root
// object's "added_tokens" member)
hd_status parse_added(const std::string &text, Tokenizer &t) {
    Json j{text.data(), text.data() + text.size()};
    j.ws();
    if (j.p < j.end && *j.p == '{') {
        j.p++;
        std::string key;
        bool found = false;
        if (!j.eat('}')) {
            do {
                if (!j.str(key) || !j.eat(':')) return HD_ERR_PARSE;
                if (key == "added_tokens") { found = true; break; }
                if (!j.skip()) return HD_ERR_PARSE;
            } while (j.eat(','));
        }
        if (!found) return HD_ERR_PARSE;
    }
    if (!j.eat('[')) return HD_ERR_PARSE;
    if (j.eat(']')) return HD_OK;
    do {
        if (!j.eat('{')) return HD_ERR_PARSE;
        long long id = -1;
        std::string content, key;
        bool have_content = false;
        if (!j.eat('}')) {
            do {
                if (!j.str(key) || !j.eat(':')) return HD_ERR_PARSE;
                if (key == "id") {
                    if (!j.num(id)) return HD_ERR_PARSE;
                } else if (key == "content") {
                    if (!j.str(content)) return HD_ERR_PARSE;
                    have_content = true;
                } else if (!j.skip()) {
                    return HD_ERR_PARSE;
                }
            } while (j.eat(','));
            if (!j.eat('}')) return HD_ERR_PARSE;
        }
        if (id < 0 || !have_content || content.empty()) return HD_ERR_PARSE;
        t.special.emplace_back(content, (int)id);
    } while (j.eat(','));
    if (!j.eat(']')) return HD_ERR_PARSE;
    // match order: ascending id (the reference's table order)
    std::vector<std::pair<std::string, int>> &sp = t.special;
    for (size_t a = 1; a < sp.size(); a++)
        for (size_t b = a; b > 0 && sp[b - 1].second > sp[b].second; b--) std::swap(sp[b - 1], sp[b]);
    return HD_OK;
}

hd_status parse_merges(const std::string &text, Tokenizer &t) {
    size_t pos = 0;
    int rank = 0;
    bool first = true;
    while (pos < text.size()) {
        size_t nl = text.find('\n', pos);
        if (nl == std::string::npos) nl = text.size();
        std::string line = text.substr(pos, nl - pos);
        pos = nl + 1;
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (first && line.rfind("#version", 0) == 0) { first = false; continue; }
        first = false;
        if (line.empty()) continue;
        const size_t sp = line.find(' ');
        if (sp == std::string::npos || sp == 0 || sp + 1 >= line.size() ||
            line.find(' ', sp + 1) != std::string::npos)
            return HD_ERR_PARSE;
        std::string key = line.substr(0, sp);
        key += '\x01';
        key += line.substr(sp + 1);
        t.merge.emplace(key, rank++);   // a repeated pair keeps its first rank
    }
    return HD_OK;
}

// ---- pre-tokenizer (tokenizer.c:333-347) --------------------------------
// Code points are decoded as the reference decodes them (tokenizer.c:56-71):
// an invalid lead byte is one unit, a sequence broken by a non-continuation
// byte ends before that byte; letters, digits and whitespace are ASCII only.
size_t cp_len(const char *s, unsigned *cp) {
    const unsigned char c = (unsigned char)s[0];
    if (c < 0x80) { *cp = c; return 1; }
    int n;
    unsigned v;
    if ((c & 0xE0) == 0xC0) { n = 2; v = c & 0x1F; }
    else if ((c & 0xF0) == 0xE0) { n = 3; v = c & 0x0F; }
    else if ((c & 0xF8) == 0xF0) { n = 4; v = c & 0x07; }
    else { *cp = 0xFFFFFFFFu; return 1; }
    for (int i = 1; i < n; i++) {
        const unsigned char cc = (unsigned char)s[i];
        if ((cc & 0xC0) != 0x80) { *cp = 0xFFFFFFFFu; return (size_t)i; }
        v = (v << 6) | (cc & 0x3F);
    }
    *cp = v;
    return (size_t)n;
}
bool is_letter(unsigned c) { return (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z'); }
bool is_digit(unsigned c) { return c >= '0' && c <= '9'; }
bool is_space(unsigned c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r' || c == '\f' || c == '\v'; }
bool is_other(unsigned c) { return !is_space(c) && !is_letter(c) && !is_digit(c); }

// [optional literal space] then a maximal run (at least one code point) of
// the class; 0 when it does not match
template <class C>
size_t run_with_space(const char *s, size_t pos, size_t end, C cls) {
    size_t i = pos;
    if (i < end && s[i] == ' ') i++;
    size_t j = i;
    while (j < end) {
        unsigned cp;
        const size_t n = cp_len(s + j, &cp);
        if (!cls(cp)) break;
        j += n;
    }
    return j > i ? j - pos : 0;
}
size_t space_run(const char *s, size_t pos, size_t end) {
    size_t j = pos;
    while (j < end && is_space((unsigned char)s[j])) j++;
    return j - pos;
}
size_t pretoken(const char *s, size_t pos, size_t end) {
    static const char *const contractions[] = {"'s", "'t", "'re", "'ve", "'m", "'ll", "'d"};
    for (const char *c : contractions) {
        const size_t n = strlen(c);
        if (pos + n <= end && !memcmp(s + pos, c, n)) return n;
    }
    size_t n;
    if ((n = run_with_space(s, pos, end, is_letter))) return n;
    if ((n = run_with_space(s, pos, end, is_digit))) return n;
    if ((n = run_with_space(s, pos, end, is_other))) return n;
    const size_t w = space_run(s, pos, end);
    if (w > 0) {
        // whitespace not followed by a non-space: the whole run when it ends
        // the segment, else all but its last character (a lone space before
        // a non-space falls to the plain whitespace rule below)
        if (pos + w == end) return w;
        if (w >= 2) return w - 1;
        return w;
    }
    return 0;
}

// ---- byte-level BPE of one pre-token ---------------------------------------
hd_status bpe(const Tokenizer &t, const char *s, size_t n, std::vector<int> &ids) {
    std::vector<std::string> parts;
    parts.reserve(n);
    for (size_t i = 0; i < n; i++) parts.push_back(t.byte_piece[(unsigned char)s[i]]);
    std::string key;
    for (;;) {
        int best = -1;
        size_t at = 0;
        for (size_t i = 0; i + 1 < parts.size(); i++) {
            key = parts[i];
            key += '\x01';
            key += parts[i + 1];
            auto it = t.merge.find(key);
            if (it != t.merge.end() && (best < 0 || it->second < best)) {
                best = it->second;
                at = i;
            }
        }
        if (best < 0) break;
        parts[at] += parts[at + 1];
        parts.erase(parts.begin() + at + 1);
    }
    for (const std::string &p : parts) {
        auto it = t.vocab.find(p);
        if (it == t.vocab.end()) {
            hd_set_error("tokenizer: piece '%s' not in vocab", p.c_str());
            return HD_ERR_PARSE;
        }
        ids.push_back(it->second);
    }
    return HD_OK;
}

// special token starting at `at` (first in ascending-id order), or nullptr
const std::pair<std::string, int> *special_at(const Tokenizer &t, const char *s, size_t at, size_t len) {
    for (const auto &sp : t.special)
        if (at + sp.first.size() <= len && !memcmp(s + at, sp.first.data(), sp.first.size())) return &sp;
    return nullptr;
}

hd_status copy_out(const std::vector<int> &ids, int **out_ids, size_t *out_count) {
    int *buf = (int *)malloc((ids.empty() ? 1 : ids.size()) * sizeof(int));
    if (!buf) {
        hd_set_error("tokenizer oom (ids)");
        return HD_ERR_OOM;
    }
    if (!ids.empty()) memcpy(buf, ids.data(), ids.size() * sizeof(int));
    *out_ids = buf;
    *out_count = ids.size();
    return HD_OK;
}

const char kUser[] = "<|im_start|>user\n";
const char kAsst[] = "<|im_end|>\n<|im_start|>assistant\n";
const char kImage[] = "<|vision_start|><|image_pad|><|vision_end|>";

}  // namespace

extern "C" hd_status hd_tokenizer_load(const char *vocab_json, const char *merges_txt,
                                       const char *added_tokens_json) {
    if (!vocab_json || !merges_txt || !added_tokens_json) {
        hd_set_error("tokenizer: null path");
        return HD_ERR_MISSING;
    }
    Tokenizer *t = new Tokenizer();
    build_byte_pieces(*t);
    std::string text;
    const char *paths[3] = {vocab_json, merges_txt, added_tokens_json};
    for (int k = 0; k < 3; k++) {
        if (!read_file(paths[k], text)) {
            hd_set_error("tokenizer: cannot read %s", paths[k]);
            delete t;
            return HD_ERR_IO;
        }
        const hd_status st = k == 0 ? parse_vocab(text, *t) : k == 1 ? parse_merges(text, *t) : parse_added(text, *t);
        if (st != HD_OK) {
            hd_set_error("tokenizer: malformed %s", paths[k]);
            delete t;
            return st;
        }
    }
    if (t->vocab.empty()) {
        hd_set_error("tokenizer: empty vocabulary in %s", vocab_json);
        delete t;
        return HD_ERR_PARSE;
    }
    delete g_tok;
    g_tok = t;
    return HD_OK;
}

extern "C" void hd_tokenizer_unload(void) {
    delete g_tok;
    g_tok = nullptr;
}

extern "C" int hd_tokenizer_special_id(const char *content) {
    if (!content || !g_tok) return -1;
    for (const auto &sp : g_tok->special)
        if (sp.first == content) return sp.second;
    return -1;
}

extern "C" hd_status hd_tokenizer_encode(const char *text, int **out_ids, size_t *out_count) {
    if (out_ids) *out_ids = nullptr;
    if (out_count) *out_count = 0;
    if (!out_ids || !out_count) {
        hd_set_error("tokenizer: null output");
        return HD_ERR_MISSING;
    }
    if (!text) {
        hd_set_error("tokenizer: null input");
        return HD_ERR_PARSE;
    }
    if (!g_tok) {
        hd_set_error("tokenizer: no vocabulary loaded (hd_tokenizer_load)");
        return HD_ERR_MISSING;
    }
    const Tokenizer &t = *g_tok;
    const size_t len = strlen(text);
    std::vector<int> ids;
    size_t i = 0;
    while (i < len) {
        if (const auto *sp = special_at(t, text, i, len)) {
            ids.push_back(sp->second);
            i += sp->first.size();
            continue;
        }
        // a plain segment up to the next special token, split into
        // pre-tokens, each BPE'd on its own
        size_t end = i;
        while (end < len && !special_at(t, text, end, len)) end++;
        while (i < end) {
            size_t n = pretoken(text, i, end);
            if (n == 0) n = 1;
            const hd_status st = bpe(t, text + i, n, ids);
            if (st != HD_OK) return st;
            i += n;
        }
    }
    return copy_out(ids, out_ids, out_count);
}

extern "C" hd_status hd_tokenizer_build_template(const char *prompt, char **out) {
    if (!out) {
        hd_set_error("tokenizer: null output");
        return HD_ERR_MISSING;
    }
    *out = nullptr;
    if (!prompt) {
        hd_set_error("tokenizer: null prompt");
        return HD_ERR_PARSE;
    }
    const std::string s = std::string(kUser) + prompt + kAsst;
    *out = (char *)malloc(s.size() + 1);
    if (!*out) {
        hd_set_error("tokenizer oom (template)");
        return HD_ERR_OOM;
    }
    memcpy(*out, s.c_str(), s.size() + 1);
    return HD_OK;
}

extern "C" hd_status hd_tokenizer_build_ref_template(const char *caption, int k, char **out) {
    if (!out) {
        hd_set_error("tokenizer: null output");
        return HD_ERR_MISSING;
    }
    *out = nullptr;
    if (!caption || k < 0) {
        hd_set_error("tokenizer: bad ref template args");
        return HD_ERR_PARSE;
    }
    std::string s = kUser;
    for (int r = 0; r < k; r++) s += kImage;
    s += caption;
    s += kAsst;
    *out = (char *)malloc(s.size() + 1);
    if (!*out) {
        hd_set_error("tokenizer oom (ref template)");
        return HD_ERR_OOM;
    }
    memcpy(*out, s.c_str(), s.size() + 1);
    return HD_OK;
}

extern "C" hd_status hd_tokenizer_encode_prompt(const char *prompt, int **out_ids, size_t *out_count) {
    char *tpl = nullptr;
    const hd_status st = hd_tokenizer_build_template(prompt, &tpl);
    if (st != HD_OK) {
        if (out_ids) *out_ids = nullptr;
        if (out_count) *out_count = 0;
        return st;
    }
    const hd_status se = hd_tokenizer_encode(tpl, out_ids, out_count);
    free(tpl);
    return se;
}

extern "C" void hd_tokenizer_free_ids(int *ids) { free(ids); }
