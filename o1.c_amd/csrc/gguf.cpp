// GGUF v3 header/tensor-table reader (gguf.c semantics: same recognised keys,
// defaults, limits and status codes), reading the header through a bounded
// sequential cursor over the file.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/types.h>

#include <string>

#include "../../include/hd_gguf.h"

static char g_gguf_err[512] = "";

static void gerr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_gguf_err, sizeof(g_gguf_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *hd_gguf_last_error(void) { return g_gguf_err; }

namespace {
// Sequential little-endian reader; any short read marks the header truncated.
struct Cursor {
    FILE *f;
    uint64_t pos = 0;   // bytes consumed after the fixed 24-byte header
    bool eof = false;
    bool bytes(void *dst, size_t n) {
        if (eof) return false;
        if (n && fread(dst, 1, n, f) != n) {
            eof = true;
            return false;
        }
        pos += n;
        return true;
    }
    bool skip(uint64_t n) {
        char tmp[4096];
        while (n) {
            const size_t k = n < sizeof(tmp) ? (size_t)n : sizeof(tmp);
            if (!bytes(tmp, k)) return false;
            n -= k;
        }
        return true;
    }
    bool u32(uint32_t *v) {
        unsigned char b[4];
        if (!bytes(b, 4)) return false;
        *v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
        return true;
    }
    bool u64(uint64_t *v) {
        unsigned char b[8];
        if (!bytes(b, 8)) return false;
        *v = 0;
        for (int i = 7; i >= 0; i--) *v = *v << 8 | b[i];
        return true;
    }
    // GGUF string: u64 length + bytes; longer than 1 MiB is malformed
    bool str(std::string *s) {
        uint64_t n;
        if (!u64(&n) || n > (uint64_t)1 << 20) return false;
        s->resize((size_t)n);
        return bytes(&(*s)[0], (size_t)n);
    }
    // skips one metadata value of GGUF type t (arrays recursively)
    bool skip_value(uint32_t t) {
        switch (t) {
        case 0: case 1: case 7: return skip(1);            // u8, i8, bool
        case 2: case 3: return skip(2);                    // u16, i16
        case 4: case 5: case 6: return skip(4);            // u32, i32, f32
        case 10: case 11: case 12: return skip(8);         // u64, i64, f64
        case 8: { std::string s; return str(&s); }
        case 9: {
            uint32_t at;
            uint64_t n;
            if (!u32(&at) || !u64(&n)) return false;
            for (uint64_t i = 0; i < n; i++)
                if (!skip_value(at)) return false;
            return true;
        }
        default: return false;
        }
    }
};

char *dup(const std::string &s) {
    char *p = (char *)malloc(s.size() + 1);
    if (p) memcpy(p, s.c_str(), s.size() + 1);
    return p;
}
}  // namespace

extern "C" void hd_gguf_close(hd_gguf_file *f) {
    if (!f) return;
    free(f->path);
    free(f->arch);
    free(f->name);
    free(f->profile);
    free(f->variant);
    free(f->revision);
    free(f->dtype);
    free(f->quantization);
    if (f->tensors)
        for (int64_t i = 0; i < f->n_tensors; i++) free(f->tensors[i].name);
    free(f->tensors);
    memset(f, 0, sizeof(*f));
}

extern "C" hd_status hd_gguf_open(const char *path, hd_gguf_file *out) {
    if (!out) return HD_ERR_MISSING;
    memset(out, 0, sizeof(*out));
    if (!path) {
        gerr("null path");
        return HD_ERR_MISSING;
    }
    out->path = strdup(path);
    FILE *fp = fopen(path, "rb");
    if (!fp) {
        gerr("cannot open %s", path);
        return HD_ERR_IO;
    }
    Cursor c{fp};
    uint32_t magic, version;
    uint64_t n_tensors, n_kv;
    if (!c.u32(&magic) || !c.u32(&version) || !c.u64(&n_tensors) || !c.u64(&n_kv)) {
        fclose(fp);
        gerr("short header %s", path);
        return HD_ERR_IO;
    }
    c.pos = 0;
    hd_status st = HD_OK;
    if (magic != 0x46554747u) {
        gerr("%s: bad GGUF magic", path);
        st = HD_ERR_PARSE;
    } else if (version != 3) {
        gerr("%s: unsupported GGUF version %u", path, version);
        st = HD_ERR_PARSE;
    } else if (n_tensors == 0 || n_tensors > (uint64_t)1 << 20) {
        gerr("%s: implausible tensor count %llu", path, (unsigned long long)n_tensors);
        st = HD_ERR_PARSE;
    }
    if (st != HD_OK) {
        fclose(fp);
        return st;
    }
    out->alignment = 32;   // GGUF default
    bool ok = true;
    for (uint64_t i = 0; ok && i < n_kv; i++) {
        std::string key;
        uint32_t vt;
        if (!c.str(&key) || !c.u32(&vt)) {
            ok = false;
            break;
        }
        char **dst = nullptr;
        int64_t *num = nullptr;
        if (key == "general.alignment" && vt == 4) {
            uint32_t a;
            ok = c.u32(&a);
            out->alignment = a;
            continue;
        }
        if (vt == 8) {
            if (key == "general.architecture") dst = &out->arch;
            else if (key == "general.name") dst = &out->name;
            else if (key == "hidream.profile") dst = &out->profile;
            else if (key == "hidream.variant") dst = &out->variant;
            else if (key == "hidream.revision") dst = &out->revision;
            else if (key == "hidream.dtype") dst = &out->dtype;
            else if (key == "hidream.quantization") dst = &out->quantization;
            else if (key == "hidream.num_layers") num = &out->num_layers;
            else if (key == "hidream.layout_version") num = &out->layout_version;
        }
        if (dst || num) {
            std::string v;
            ok = c.str(&v);
            if (ok && dst) {
                free(*dst);
                *dst = dup(v);
            }
            if (ok && num) *num = atoll(v.c_str());
        } else {
            ok = c.skip_value(vt);
        }
    }
    if (ok) {
        out->tensors = (hd_gguf_tensor *)calloc((size_t)n_tensors, sizeof(hd_gguf_tensor));
        ok = out->tensors != nullptr;
        if (ok) out->n_tensors = (int64_t)n_tensors;
    }
    for (uint64_t i = 0; ok && i < n_tensors; i++) {
        hd_gguf_tensor *t = &out->tensors[i];
        std::string nm;
        if (!c.str(&nm) || !c.u32(&t->n_dims) || t->n_dims > 8) {
            ok = false;
            break;
        }
        t->name = dup(nm);
        uint64_t elems = 1;
        for (uint32_t d = 0; ok && d < t->n_dims; d++) {
            ok = c.u64(&t->dims[d]);
            elems *= t->dims[d];
        }
        ok = ok && c.u32(&t->type) && c.u64(&t->offset);
        if (!ok) break;
        if (t->type == HD_GGML_TYPE_F32) t->nbytes = elems * 4;
        else if (t->type == HD_GGML_TYPE_F16 || t->type == HD_GGML_TYPE_BF16) t->nbytes = elems * 2;
        else ok = false;
    }
    const uint64_t header_end = 24 + c.pos;
    fclose(fp);
    if (!ok) {
        hd_gguf_close(out);
        gerr("%s: malformed header", path);
        return HD_ERR_PARSE;
    }
    const uint64_t al = out->alignment ? out->alignment : 32;
    out->tensor_data_off = (header_end + al - 1) & ~(al - 1);
    uint64_t end = 0;
    for (int64_t i = 0; i < out->n_tensors; i++) {
        const uint64_t e = out->tensors[i].offset + out->tensors[i].nbytes;
        if (e > end) end = e;
    }
    out->payload_bytes = (end + al - 1) & ~(al - 1);
    return HD_OK;
}

extern "C" hd_status hd_gguf_read_tensor(const hd_gguf_file *f, const hd_gguf_tensor *t, void *dst) {
    if (!f || !t || !dst || !f->path) {
        gerr("read_tensor: null argument");
        return HD_ERR_MISSING;
    }
    FILE *fp = fopen(f->path, "rb");
    if (!fp) {
        gerr("cannot open %s", f->path);
        return HD_ERR_IO;
    }
    if (fseeko(fp, (off_t)(f->tensor_data_off + t->offset), SEEK_SET) != 0) {
        fclose(fp);
        gerr("seek %s", f->path);
        return HD_ERR_IO;
    }
    const size_t got = fread(dst, 1, (size_t)t->nbytes, fp);
    fclose(fp);
    if (got != (size_t)t->nbytes) {
        gerr("short read %s (%zu/%llu)", t->name ? t->name : "?", got,
             (unsigned long long)t->nbytes);
        return HD_ERR_IO;
    }
    return HD_OK;
}
