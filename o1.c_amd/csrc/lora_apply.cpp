// Merge-on-load of musubi HiDream-O1 LoRA adapters (.safetensors): parse and
// validate every adapter on the host, upload the factors as fp32, merge on
// the GPU (hd_lora_merge_gpu), free the staging. Follows
// src/model/lora.c:126-375 of the reference; the safetensors header reader
// and the target map are this file's own.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/hd_hip.h"
#include "../../include/hd_lora.h"
#include "../../include/hd_weights.h"

namespace {

char g_err[512] = "";

void lerr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    hd_set_error("%s", g_err);
}

// ---- target map --------------------------------------------------------
// The linear layers of the dev profile a LoRA may target (the reference's
// generated lora_map_dev.inc lists the same 257): the 7 projections of each
// of the 36 decoder layers, x_embedder proj1/proj2, final_layer2.linear and
// the two t-embedder linears. A prefix is "lora_unet_" + the checkpoint
// name without ".weight", '.' -> '_'.
struct Target {
    std::string prefix, base;
    int out_dim, in_dim;
};

const std::vector<Target> &target_map() {
    static std::vector<Target> map;
    if (!map.empty()) return map;
    auto add = [](const std::string &base, int out, int in) {
        std::string p = "lora_unet_" + base.substr(0, base.size() - 7);   // drop ".weight"
        for (char &c : p)
            if (c == '.') c = '_';
        map.push_back({p, base, out, in});
    };
    const int H = 4096, KV = 1024, F = 12288;
    for (int l = 0; l < 36; l++) {
        const std::string L = "model.language_model.layers." + std::to_string(l) + ".";
        add(L + "self_attn.q_proj.weight", H, H);
        add(L + "self_attn.k_proj.weight", KV, H);
        add(L + "self_attn.v_proj.weight", KV, H);
        add(L + "self_attn.o_proj.weight", H, H);
        add(L + "mlp.gate_proj.weight", F, H);
        add(L + "mlp.up_proj.weight", F, H);
        add(L + "mlp.down_proj.weight", H, F);
    }
    add("model.x_embedder.proj1.weight", 1024, 3072);
    add("model.x_embedder.proj2.weight", H, 1024);
    add("model.final_layer2.linear.weight", 3072, H);
    add("model.t_embedder1.mlp.0.weight", H, 256);
    add("model.t_embedder1.mlp.2.weight", H, H);
    return map;
}

const Target *find_target(const std::string &prefix) {
    for (const Target &t : target_map())
        if (t.prefix == prefix) return &t;
    return nullptr;
}

// ---- safetensors header --------------------------------------------------
// File: u64 little-endian header length N, N bytes of JSON
//   {"name": {"dtype": "BF16", "shape": [..], "data_offsets": [b, e]}, ...,
//    "__metadata__": {...}}
// then the data section; offsets are relative to its start.
enum Dtype { DT_F32, DT_F16, DT_BF16, DT_OTHER };

struct Tensor {
    std::string name;
    Dtype dtype = DT_OTHER;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

struct StFile {
    std::string path;
    uint64_t data_start = 0, file_size = 0;
    std::vector<Tensor> tensors;
    const Tensor *find(const std::string &n) const {
        for (const Tensor &t : tensors)
            if (t.name == n) return &t;
        return nullptr;
    }
};

struct Json {   // minimal reader for the header's object / array / string / number grammar
    const char *p, *e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    bool lit(char c) {
        ws();
        if (p < e && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool str(std::string &out) {
        ws();
        if (p >= e || *p != '"') return ok = false;
        p++;
        out.clear();
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return ok = false;
                const char c = *p;
                out.push_back(c == 'n' ? '\n' : c == 't' ? '\t' : c == 'u' ? '?' : c);
                if (c == 'u') p = p + 4 < e ? p + 4 : e;
                p++;
                continue;
            }
            out.push_back(*p++);
        }
        if (p >= e) return ok = false;
        p++;
        return true;
    }
    bool num(int64_t &v) {
        ws();
        char *q = nullptr;
        const long long x = strtoll(p, &q, 10);
        if (q == p || q > e) return ok = false;
        p = q;
        v = x;
        return true;
    }
    bool skip() {   // any value
        ws();
        if (p >= e) return ok = false;
        if (*p == '"') {
            std::string s;
            return str(s);
        }
        if (*p == '{' || *p == '[') {
            const char open = *p, close = open == '{' ? '}' : ']';
            p++;
            if (lit(close)) return true;
            do {
                if (open == '{') {
                    std::string k;
                    if (!str(k) || !lit(':')) return ok = false;
                }
                if (!skip()) return false;
            } while (lit(','));
            return lit(close) || (ok = false);
        }
        while (p < e && *p != ',' && *p != '}' && *p != ']') p++;
        return true;
    }
};

hd_status scan_header(const char *path, StFile &st) {
    st.path = path;
    FILE *f = fopen(path, "rb");
    if (!f) {
        lerr("lora %s: cannot open", path);
        return HD_ERR_IO;
    }
    fseek(f, 0, SEEK_END);
    const long fsz = ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t lb[8];
    if (fsz < 8 || fread(lb, 1, 8, f) != 8) {
        fclose(f);
        lerr("lora %s: truncated header", path);
        return HD_ERR_PARSE;
    }
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | lb[i];
    if (n == 0 || n > (uint64_t)fsz - 8 || n > (uint64_t)1 << 30) {
        fclose(f);
        lerr("lora %s: bad header length", path);
        return HD_ERR_PARSE;
    }
    std::string hdr(n, '\0');
    if (fread(&hdr[0], 1, n, f) != n) {
        fclose(f);
        lerr("lora %s: truncated header", path);
        return HD_ERR_PARSE;
    }
    fclose(f);
    st.data_start = 8 + n;
    st.file_size = (uint64_t)fsz;
    Json j{hdr.data(), hdr.data() + hdr.size()};
    if (!j.lit('{')) {
        lerr("lora %s: header is not a JSON object", path);
        return HD_ERR_PARSE;
    }
    if (!j.lit('}')) {
        do {
            std::string name;
            if (!j.str(name) || !j.lit(':')) break;
            if (name == "__metadata__") {
                if (!j.skip()) break;
                continue;
            }
            Tensor t;
            t.name = name;
            bool have_off = false;
            if (!j.lit('{')) {
                j.ok = false;
                break;
            }
            if (!j.lit('}')) {
                do {
                    std::string key;
                    if (!j.str(key) || !j.lit(':')) break;
                    if (key == "dtype") {
                        std::string d;
                        if (!j.str(d)) break;
                        t.dtype = d == "F32" ? DT_F32 : d == "F16" ? DT_F16 : d == "BF16" ? DT_BF16 : DT_OTHER;
                    } else if (key == "shape") {
                        if (!j.lit('[')) {
                            j.ok = false;
                            break;
                        }
                        if (!j.lit(']')) {
                            do {
                                int64_t v;
                                if (!j.num(v) || v < 0) {
                                    j.ok = false;
                                    break;
                                }
                                t.shape.push_back(v);
                            } while (j.lit(','));
                            if (!j.ok || !j.lit(']')) {
                                j.ok = false;
                                break;
                            }
                        }
                    } else if (key == "data_offsets") {
                        int64_t b, e2;
                        if (!j.lit('[') || !j.num(b) || !j.lit(',') || !j.num(e2) || !j.lit(']') || b < 0 ||
                            e2 < b) {
                            j.ok = false;
                            break;
                        }
                        t.begin = (uint64_t)b;
                        t.end = (uint64_t)e2;
                        have_off = true;
                    } else if (!j.skip()) {
                        break;
                    }
                } while (j.lit(','));
                if (!j.ok || !j.lit('}')) {
                    j.ok = false;
                    break;
                }
            }
            if (!have_off || st.data_start + t.end > st.file_size) {
                j.ok = false;
                break;
            }
            st.tensors.push_back(t);
        } while (j.lit(','));
        if (j.ok && !j.lit('}')) j.ok = false;
    }
    if (!j.ok) {
        lerr("lora %s: malformed safetensors header", path);
        return HD_ERR_PARSE;
    }
    return HD_OK;
}

hd_status read_bytes(const StFile &st, const Tensor &t, std::vector<uint8_t> &out) {
    out.resize(t.end - t.begin);
    FILE *f = fopen(st.path.c_str(), "rb");
    if (!f) {
        lerr("lora %s: cannot open", st.path.c_str());
        return HD_ERR_IO;
    }
    const bool ok = fseek(f, (long)(st.data_start + t.begin), SEEK_SET) == 0 &&
                    (out.empty() || fread(out.data(), 1, out.size(), f) == out.size());
    fclose(f);
    if (!ok) {
        lerr("lora %s: short read of %s", st.path.c_str(), t.name.c_str());
        return HD_ERR_IO;
    }
    return HD_OK;
}

// IEEE half -> float by its definition (exact in fp32)
float half_to_float(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    return s ? -v : v;
}

hd_status to_f32(const StFile &st, const Tensor &t, std::vector<float> &out) {
    const size_t esz = t.dtype == DT_F32 ? 4 : 2;
    if (t.dtype == DT_OTHER) {
        lerr("lora %s: tensor %s: unsupported dtype", st.path.c_str(), t.name.c_str());
        return HD_ERR_UNSUPPORTED;
    }
    if ((int64_t)(t.end - t.begin) != t.numel() * (int64_t)esz) {
        lerr("lora %s: tensor %s: size does not match its shape", st.path.c_str(), t.name.c_str());
        return HD_ERR_PARSE;
    }
    std::vector<uint8_t> raw;
    hd_status s = read_bytes(st, t, raw);
    if (s != HD_OK) return s;
    const int64_t n = t.numel();
    out.resize(n);
    for (int64_t i = 0; i < n; i++) {
        if (t.dtype == DT_F32) {
            memcpy(&out[i], &raw[4 * i], 4);
        } else {
            uint16_t b;
            memcpy(&b, &raw[2 * i], 2);
            if (t.dtype == DT_BF16) {
                const uint32_t bits = (uint32_t)b << 16;
                memcpy(&out[i], &bits, 4);
            } else {
                out[i] = half_to_float(b);
            }
        }
    }
    return HD_OK;
}

struct Pending {
    hd_lora_entry e;
    std::vector<float> down, up;
};

}  // namespace

extern "C" const char *hd_lora_last_error(void) { return g_err; }

extern "C" hd_status hd_lora_apply(const hd_lora_config *cfg, hd_weight_store *store, int device_id) {
    g_err[0] = '\0';
    if (!cfg || cfg->count == 0) return HD_OK;
    if (!cfg->items || !store || !store->arena_ptr) {
        lerr("lora: store not loaded");
        return HD_ERR_MISSING;
    }
    // pass 1: parse and validate every adapter, read every factor to fp32 on
    // the host and find every base tensor; nothing on the GPU is touched
    std::vector<Pending> all;
    for (size_t a = 0; a < cfg->count; a++) {
        const char *path = cfg->items[a].path;
        const float mult = cfg->items[a].multiplier;
        if (!path) {
            lerr("lora: null adapter path");
            return HD_ERR_MISSING;
        }
        if (!isfinite(mult)) {
            lerr("lora %s: non-finite multiplier", path);
            return HD_ERR_PARSE;
        }
        StFile st;
        hd_status s = scan_header(path, st);
        if (s != HD_OK) return s;
        const std::string dsuf = ".lora_down.weight";
        for (const Tensor &dt : st.tensors) {
            if (dt.name.size() <= dsuf.size() ||
                dt.name.compare(dt.name.size() - dsuf.size(), dsuf.size(), dsuf) != 0)
                continue;
            const std::string prefix = dt.name.substr(0, dt.name.size() - dsuf.size());
            const Tensor *ut = st.find(prefix + ".lora_up.weight");
            if (!ut) {
                lerr("lora %s: %s missing lora_up pair", path, prefix.c_str());
                return HD_ERR_PARSE;
            }
            const Target *tg = find_target(prefix);
            if (!tg) {
                lerr("lora %s: target unknown for profile 'dev': %s", path, prefix.c_str());
                return HD_ERR_UNSUPPORTED;
            }
            if (dt.shape.size() != 2 || ut->shape.size() != 2) {
                lerr("lora %s: %s non-linear", path, prefix.c_str());
                return HD_ERR_UNSUPPORTED;
            }
            const int64_t rank = dt.shape[0], in_dim = dt.shape[1], out_dim = ut->shape[0];
            if (rank <= 0 || ut->shape[1] != rank) {
                lerr("lora %s: %s rank mismatch", path, prefix.c_str());
                return HD_ERR_PARSE;
            }
            if (in_dim != tg->in_dim || out_dim != tg->out_dim) {
                lerr("lora %s: %s shape mismatch base=[%d,%d] down=[%lld,%lld] up=[%lld,%lld]", path,
                     prefix.c_str(), tg->out_dim, tg->in_dim, (long long)rank, (long long)in_dim,
                     (long long)out_dim, (long long)rank);
                return HD_ERR_PARSE;
            }
            float alpha = (float)rank;
            if (const Tensor *at = st.find(prefix + ".alpha")) {
                std::vector<float> av;
                if (at->numel() != 1) {
                    lerr("lora %s: %s malformed alpha", path, prefix.c_str());
                    return HD_ERR_PARSE;
                }
                if ((s = to_f32(st, *at, av)) != HD_OK) return s;
                alpha = av[0];
                if (!isfinite(alpha) || alpha == 0.0f) {
                    lerr("lora %s: %s invalid alpha %g", path, prefix.c_str(), alpha);
                    return HD_ERR_PARSE;
                }
            }
            Pending p;
            memset(&p.e, 0, sizeof(p.e));
            snprintf(p.e.lora_prefix, sizeof(p.e.lora_prefix), "%s", prefix.c_str());
            snprintf(p.e.base_tensor, sizeof(p.e.base_tensor), "%s", tg->base.c_str());
            p.e.rank = (uint32_t)rank;
            p.e.in_dim = (uint32_t)in_dim;
            p.e.out_dim = (uint32_t)out_dim;
            p.e.alpha = alpha;
            p.e.multiplier = mult;
            p.e.base_dev = const_cast<void *>(hd_weight_store_find(store, tg->base.c_str()));
            if (!p.e.base_dev) {
                lerr("lora %s: base tensor %s not found in store", path, tg->base.c_str());
                return HD_ERR_MISSING;
            }
            if ((s = to_f32(st, dt, p.down)) != HD_OK || (s = to_f32(st, *ut, p.up)) != HD_OK) return s;
            all.push_back(std::move(p));
        }
    }
    if (all.empty()) {
        lerr("lora: no supported linear targets found");
        return HD_ERR_UNSUPPORTED;
    }
    // pass 2: upload the factors (fp32), pass 3: merge on the store's upload
    // stream, then free the staging
    if (hipSetDevice(device_id) != hipSuccess) {
        lerr("lora: hipSetDevice(%d) failed", device_id);
        return HD_ERR_IO;
    }
    hipStream_t stream = (hipStream_t)store->upload_stream;
    std::vector<hd_lora_entry> ents;
    hd_status st = HD_OK;
    for (Pending &p : all) {
        hd_lora_entry e = p.e;
        if (hipMalloc(&e.down_dev, p.down.size() * 4) != hipSuccess ||
            hipMalloc(&e.up_dev, p.up.size() * 4) != hipSuccess) {
            lerr("lora: device allocation failed for %s", e.lora_prefix);
            if (e.down_dev) (void)hipFree(e.down_dev);
            st = HD_ERR_OOM;
            break;
        }
        ents.push_back(e);
        if (hipMemcpy(e.down_dev, p.down.data(), p.down.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(e.up_dev, p.up.data(), p.up.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
            lerr("lora: upload failed for %s", e.lora_prefix);
            st = HD_ERR_IO;
            break;
        }
    }
    if (st == HD_OK) {
        st = hd_lora_merge_gpu(ents.data(), ents.size(), stream);
        if (st == HD_OK && hipStreamSynchronize(stream) != hipSuccess) {
            lerr("lora: merge synchronisation failed");
            st = HD_ERR_IO;
        } else if (st != HD_OK) {
            lerr("lora merge failed: %s", hd_last_error());
        }
    }
    for (hd_lora_entry &e : ents) {
        (void)hipFree(e.down_dev);
        (void)hipFree(e.up_dev);
    }
    return st;
}
