// Device weight store: identity query, the GGUF pack loader and teardown.
// The loader streams the pack's payload file -> pinned staging -> one
// device arena: a reader fills staging slot k while the copies of the other
// slots run on the store's upload stream; slot k is refilled only after its
// previous copy has completed (one event per slot).
#include <hip/hip_runtime.h>
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "../../include/hd_gguf.h"
#include "../../include/hd_weights.h"

static char g_w_err[512] = "";

static void werr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_w_err, sizeof(g_w_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *hd_weights_last_error(void) { return g_w_err; }

extern "C" hd_status hd_device_info(int device_id, hd_weight_store *out) {
    if (!out) return HD_ERR_MISSING;
    memset(out, 0, sizeof(*out));
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) {
        werr("hipGetDeviceCount: %s", hipGetErrorString(e));
        return HD_ERR_IO;
    }
    if (device_id < 0 || device_id >= count) {
        werr("device %d out of range (visible=%d)", device_id, count);
        return HD_ERR_PROFILE;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device_id);
    if (e != hipSuccess) {
        werr("hipGetDeviceProperties: %s", hipGetErrorString(e));
        return HD_ERR_IO;
    }
    out->device_id = device_id;
    snprintf(out->device_name, sizeof(out->device_name), "%s", prop.name);
    out->compute_major = prop.major;
    out->compute_minor = prop.minor;
    out->device_mem_bytes = (int64_t)prop.totalGlobalMem;
    return HD_OK;
}

extern "C" void hd_weight_store_free(hd_weight_store *s) {
    if (!s) return;
    if (s->gemm) hd_gemm_runtime_destroy(s->gemm);
    if (s->upload_stream) (void)hipStreamDestroy((hipStream_t)s->upload_stream);
    if (s->arena_ptr) {
        (void)hipFree(s->arena_ptr);
    } else if (s->allocs) {
        for (int64_t i = 0; i < s->n_allocs; i++)
            if (s->allocs[i].dev_ptr) (void)hipFree(s->allocs[i].dev_ptr);
    }
    free(s->allocs);
    memset(s, 0, sizeof(*s));
}

namespace {
constexpr int kSlots = 4;
constexpr size_t kSlotBytes = (size_t)64 << 20;

struct Staging {
    void *buf[kSlots] = {};
    hipEvent_t ev[kSlots] = {};
    bool used[kSlots] = {};
    ~Staging() {
        for (int k = 0; k < kSlots; k++) {
            if (ev[k]) {
                (void)hipEventSynchronize(ev[k]);
                (void)hipEventDestroy(ev[k]);
            }
            if (buf[k]) (void)hipHostFree(buf[k]);
        }
    }
};
}  // namespace

extern "C" hd_status hd_weights_to_device_gguf(const char *path, int device_id, hd_weight_store *out) {
    if (!path || !out) {
        werr("null argument");
        return HD_ERR_MISSING;
    }
    hd_weight_store info;
    hd_status st = hd_device_info(device_id, &info);
    if (st != HD_OK) return st;
    hipError_t e = hipSetDevice(device_id);
    if (e != hipSuccess) {
        werr("hipSetDevice: %s", hipGetErrorString(e));
        return HD_ERR_IO;
    }
    hd_gguf_file gf;
    st = hd_gguf_open(path, &gf);
    if (st != HD_OK) {
        werr("gguf: %s", hd_gguf_last_error());
        return st;
    }
    auto fail = [&](hd_status s) {
        hd_weight_store_free(&info);
        hd_gguf_close(&gf);
        return s;
    };
    info.allocs = (hd_device_alloc *)calloc((size_t)gf.n_tensors, sizeof(hd_device_alloc));
    if (!info.allocs) {
        werr("oom alloc table");
        return fail(HD_ERR_OOM);
    }
    for (int64_t i = 0; i < gf.n_tensors; i++) {
        const hd_gguf_tensor *t = &gf.tensors[i];
        if (t->offset % gf.alignment || t->offset + t->nbytes > gf.payload_bytes) {
            werr("tensor %s: offset %llu not aligned to %llu or past the payload", t->name,
                 (unsigned long long)t->offset, (unsigned long long)gf.alignment);
            return fail(HD_ERR_PARSE);
        }
    }
    e = hipMalloc(&info.arena_ptr, (size_t)gf.payload_bytes);
    if (e != hipSuccess) {
        info.arena_ptr = nullptr;
        werr("hipMalloc arena %llu bytes: %s", (unsigned long long)gf.payload_bytes,
             hipGetErrorString(e));
        return fail(HD_ERR_OOM);
    }
    info.arena_bytes = (int64_t)gf.payload_bytes;
    info.n_allocations = 1;
    hipStream_t us = nullptr;
    if (hipStreamCreateWithFlags(&us, hipStreamNonBlocking) != hipSuccess) {
        werr("upload stream create failed");
        return fail(HD_ERR_OOM);
    }
    info.upload_stream = us;
    {
        Staging sg;
        for (int k = 0; k < kSlots; k++) {
            // each allocation checked on its own: the Staging destructor
            // frees whatever did succeed
            if (hipHostMalloc(&sg.buf[k], kSlotBytes, hipHostMallocDefault) != hipSuccess) {
                sg.buf[k] = nullptr;
                werr("pinned staging allocation failed");
                return fail(HD_ERR_OOM);
            }
            if (hipEventCreateWithFlags(&sg.ev[k], hipEventDisableTiming) != hipSuccess) {
                sg.ev[k] = nullptr;
                werr("staging event creation failed");
                return fail(HD_ERR_OOM);
            }
        }
        const int fd = open(path, O_RDONLY);
        if (fd < 0) {
            werr("open %s: %s", path, strerror(errno));
            return fail(HD_ERR_IO);
        }
        // the data section may end before payload_bytes (the last tensor's
        // padding need not be on disk): read what is there, zero the rest
        uint64_t off = 0;
        int k = 0;
        hd_status rs = HD_OK;
        while (off < gf.payload_bytes && rs == HD_OK) {
            const size_t n = (size_t)(gf.payload_bytes - off < kSlotBytes ? gf.payload_bytes - off
                                                                           : kSlotBytes);
            if (sg.used[k]) (void)hipEventSynchronize(sg.ev[k]);
            size_t got = 0;
            while (got < n) {
                const ssize_t r = pread(fd, (char *)sg.buf[k] + got, n - got,
                                        (off_t)(gf.tensor_data_off + off + got));
                if (r < 0) {
                    werr("read %s: %s", path, strerror(errno));
                    rs = HD_ERR_IO;
                    break;
                }
                if (r == 0) break;
                got += (size_t)r;
            }
            if (rs != HD_OK) break;
            if (got < n) {
                // end of file: only padding may be missing
                for (int64_t i = 0; i < gf.n_tensors; i++) {
                    const uint64_t te = gf.tensors[i].offset + gf.tensors[i].nbytes;
                    if (te > off + got) {
                        werr("short read: tensor %s ends at %llu, file data ends at %llu",
                             gf.tensors[i].name, (unsigned long long)te,
                             (unsigned long long)(off + got));
                        rs = HD_ERR_IO;
                        break;
                    }
                }
                memset((char *)sg.buf[k] + got, 0, n - got);
            }
            if (rs != HD_OK) break;
            if (hipMemcpyAsync((char *)info.arena_ptr + off, sg.buf[k], n, hipMemcpyHostToDevice, us) !=
                    hipSuccess ||
                hipEventRecord(sg.ev[k], us) != hipSuccess) {
                werr("upload copy failed");
                rs = HD_ERR_IO;
                break;
            }
            sg.used[k] = true;
            off += n;
            k = (k + 1) % kSlots;
        }
        close(fd);
        if (hipStreamSynchronize(us) != hipSuccess && rs == HD_OK) {
            werr("upload stream sync failed");
            rs = HD_ERR_IO;
        }
        if (rs != HD_OK) return fail(rs);
    }
    for (int64_t i = 0; i < gf.n_tensors; i++) {
        const hd_gguf_tensor *t = &gf.tensors[i];
        hd_device_alloc *a = &info.allocs[i];
        a->dev_ptr = (char *)info.arena_ptr + t->offset;
        a->nbytes = (int64_t)t->nbytes;
        snprintf(a->name, sizeof(a->name), "%s", t->name);
        info.n_allocs++;
        info.device_bytes_allocated += (int64_t)t->nbytes;
        info.host_bytes_loaded += (int64_t)t->nbytes;
        if ((int64_t)t->nbytes > info.largest_numel) {
            info.largest_numel = (int64_t)t->nbytes;
            snprintf(info.largest_name, sizeof(info.largest_name), "%s", t->name);
        }
    }
    info.gemm = hd_gemm_runtime_init(device_id, (size_t)64 << 20);
    if (!info.gemm) {
        werr("gemm runtime init failed");
        return fail(HD_ERR_RUNTIME);
    }
    hd_gguf_close(&gf);
    *out = info;
    return HD_OK;
}
