// lal_gpq8.cpp -- GPQ8 weight file reader and the LM head's load-time
// preparation (include/lal_gpq8.h).  Host code of liblal_gpu.so.
//
// Reference: tools/server/qwen7b_server.c:497-571 (load_gpq8 / gp_find /
// get_q8) and :1106-1112 (lm_head.weight quantized to int8 at start-up with
// runtime/lal_q8_kernel.h:357-372).  The directory walk is the same record
// sequence; every length is bounds-checked against the mapping.
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <vector>

#include "lal_gpq8.h"

struct lal_gpq8_file {
    int fd = -1;
    void *base = nullptr;
    size_t size = 0;
    std::vector<std::string> keys;
    std::vector<lal_gpq8_tensor> tensors;
};

namespace {

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const unsigned char *p, *end;
    bool take(void *dst, size_t n)
    {
        if ((size_t)(end - p) < n) return false;
        memcpy(dst, p, n);
        p += n;
        return true;
    }
    bool skip(uint64_t n, const unsigned char **at)
    {
        if ((uint64_t)(end - p) < n) return false;
        *at = p;
        p += n;
        return true;
    }
};

int parse(lal_gpq8_file *f)
{
    Cursor c{(const unsigned char *)f->base, (const unsigned char *)f->base + f->size};
    char magic[4];
    int32_t n = 0;
    if (!c.take(magic, 4) || memcmp(magic, "GPQ8", 4) != 0) return LAL_GPU_E_INVAL;
    if (!c.take(&n, 4) || n < 0) return LAL_GPU_E_INVAL;
    // every record holds at least 21 bytes (key length, ndim, qtype, data
    // length, scale count), so a count the file cannot hold is malformed
    if ((uint64_t)n > (uint64_t)(c.end - c.p) / 21u) return LAL_GPU_E_INVAL;
    f->keys.reserve((size_t)n);
    f->tensors.reserve((size_t)n);
    for (int32_t i = 0; i < n; i++) {
        lal_gpq8_tensor t;
        memset(&t, 0, sizeof t);
        int32_t klen = 0;
        const unsigned char *kp = nullptr;
        if (!c.take(&klen, 4) || klen < 0 || !c.skip((uint64_t)klen, &kp)) return LAL_GPU_E_INVAL;
        f->keys.emplace_back((const char *)kp, (size_t)klen);
        int32_t ndim = 0;
        if (!c.take(&ndim, 4) || ndim < 0 || ndim > LAL_GPQ8_MAX_DIMS) return LAL_GPU_E_INVAL;
        t.ndim = ndim;
        for (int d = 0; d < ndim; d++) {
            int32_t e = 0;
            if (!c.take(&e, 4) || e < 0) return LAL_GPU_E_INVAL;
            t.shape[d] = e;
        }
        uint8_t qt = 0;
        uint64_t len = 0;
        const unsigned char *dp = nullptr;
        if (!c.take(&qt, 1) || !c.take(&len, 8) || !c.skip(len, &dp)) return LAL_GPU_E_INVAL;
        t.qtype = qt;
        t.data_len = len;
        t.data = dp;
        int32_t ns = 0;
        const unsigned char *sp = nullptr;
        if (!c.take(&ns, 4) || ns < 0 || !c.skip((uint64_t)ns * 4u, &sp)) return LAL_GPU_E_INVAL;
        t.n_scale = ns;
        t.scale = ns > 0 ? (const float *)sp : nullptr;
        f->tensors.push_back(t);
    }
    for (size_t i = 0; i < f->tensors.size(); i++) f->tensors[i].key = f->keys[i].c_str();
    return LAL_GPU_OK;
}

bool shape2(const lal_gpq8_tensor &t, int *rows, int *cols)
{
    if (t.ndim != 2 || t.shape[0] <= 0 || t.shape[1] <= 0) return false;
    *rows = t.shape[0];
    *cols = t.shape[1];
    return true;
}

}  // namespace

extern "C" {

int lal_gpq8_open(const char *path, lal_gpq8_file **out)
{
    if (!path || !out) return LAL_GPU_E_INVAL;
    *out = nullptr;
    lal_gpq8_file *f = new (std::nothrow) lal_gpq8_file;
    if (!f) return LAL_GPU_E_NOMEM;
    f->fd = open(path, O_RDONLY);
    struct stat st;
    if (f->fd < 0 || fstat(f->fd, &st) != 0 || st.st_size < 8) {
        lal_gpq8_close(f);
        return LAL_GPU_E_INVAL;
    }
    f->size = (size_t)st.st_size;
    f->base = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (f->base == MAP_FAILED) {
        f->base = nullptr;
        lal_gpq8_close(f);
        return LAL_GPU_E_NOMEM;
    }
    madvise(f->base, f->size, MADV_SEQUENTIAL);
    int rc;
    try {
        rc = parse(f);
    } catch (const std::bad_alloc &) {
        rc = LAL_GPU_E_NOMEM;
    } catch (...) {
        rc = LAL_GPU_E_INVAL;
    }
    if (rc != LAL_GPU_OK) {
        lal_gpq8_close(f);
        return rc;
    }
    *out = f;
    return LAL_GPU_OK;
}

void lal_gpq8_close(lal_gpq8_file *f)
{
    if (!f) return;
    if (f->base) munmap(f->base, f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

int lal_gpq8_count(const lal_gpq8_file *f) { return f ? (int)f->tensors.size() : 0; }

int lal_gpq8_tensor_at(const lal_gpq8_file *f, int i, lal_gpq8_tensor *out)
{
    if (!f || !out || i < 0 || i >= (int)f->tensors.size()) return LAL_GPU_E_INVAL;
    *out = f->tensors[(size_t)i];
    return LAL_GPU_OK;
}

int lal_gpq8_find(const lal_gpq8_file *f, const char *key, lal_gpq8_tensor *out)
{
    if (!f || !key || !out) return LAL_GPU_E_INVAL;
    for (const lal_gpq8_tensor &t : f->tensors)
        if (strcmp(t.key, key) == 0) {
            *out = t;
            return LAL_GPU_OK;
        }
    return LAL_GPU_E_RANGE;
}

int lal_gpu_load_lm_head(lal_gpu_ctx *ctx, const lal_gpq8_file *f, const char *key, int8_t *d_wpk,
                         float *d_sw, int *vocab, int *n, void *stream)
{
    if (!f || !key || !vocab || !n || (d_wpk && !ctx)) return LAL_GPU_E_INVAL;
    lal_gpq8_tensor t;
    int rc = lal_gpq8_find(f, key, &t);
    if (rc != LAL_GPU_OK) return rc;
    int V = 0, N = 0;
    if (!shape2(t, &V, &N)) return LAL_GPU_E_INVAL;
    const uint64_t elems = (uint64_t)V * (uint64_t)N;
    if (t.qtype == LAL_GPQ8_F32) {
        if (t.data_len != elems * 4u) return LAL_GPU_E_INVAL;
    } else if (t.qtype == LAL_GPQ8_Q8) {
        if (t.data_len != elems || t.n_scale != V) return LAL_GPU_E_INVAL;
    } else {
        return LAL_GPU_E_INVAL;  // block formats are not an LM head layout here
    }
    *vocab = V;
    *n = N;
    if (!d_wpk) return LAL_GPU_OK;
    if (!d_sw) return LAL_GPU_E_INVAL;

    // rows in chunks of a multiple of 16 (whole tiles of the packed layout):
    // a chunk packed alone lands at its tiles' offset unchanged
    const size_t tile_bytes = (size_t)((N + 63) / 64) * 1024u;
    int rows = (int)((64u << 20) / ((size_t)N * 4u));  // ~64 MB of F32 per chunk
    rows = rows < 16 ? 16 : rows - rows % 16;
    if (rows > V) rows = V;
    void *d_stage = nullptr, *d_q = nullptr;
    rc = lal_gpu_malloc(&d_stage, (size_t)rows * N * (t.qtype == LAL_GPQ8_F32 ? 4u : 1u));
    if (rc == LAL_GPU_OK && t.qtype == LAL_GPQ8_F32) rc = lal_gpu_malloc(&d_q, (size_t)rows * N);
    const unsigned char *src = (const unsigned char *)t.data;
    for (int r0 = 0; rc == LAL_GPU_OK && r0 < V; r0 += rows) {
        const int nr = (V - r0 < rows) ? V - r0 : rows;
        int8_t *dst = d_wpk + (size_t)(r0 / 16) * tile_bytes;
        if (t.qtype == LAL_GPQ8_F32) {
            rc = lal_gpu_memcpy_h2d(d_stage, src + (size_t)r0 * N * 4u, (size_t)nr * N * 4u, stream);
            if (rc == LAL_GPU_OK)
                rc = lal_gpu_quantize_w_q8(ctx, (const float *)d_stage, nr, N, (int8_t *)d_q, dst, d_sw + r0,
                                           stream);
        } else {
            rc = lal_gpu_memcpy_h2d(d_stage, src + (size_t)r0 * N, (size_t)nr * N, stream);
            if (rc == LAL_GPU_OK) rc = lal_gpu_pack_q8(ctx, (const int8_t *)d_stage, nr, N, dst, stream);
        }
        if (rc == LAL_GPU_OK) rc = lal_gpu_stream_sync(stream);  // the stage is reused
    }
    if (rc == LAL_GPU_OK && t.qtype == LAL_GPQ8_Q8) {
        // scales may sit unaligned in the file: copy through an aligned buffer
        std::vector<float> sw((size_t)V);
        memcpy(sw.data(), t.scale, (size_t)V * 4u);
        rc = lal_gpu_memcpy_h2d(d_sw, sw.data(), (size_t)V * 4u, stream);
        if (rc == LAL_GPU_OK) rc = lal_gpu_stream_sync(stream);
    }
    if (d_stage) lal_gpu_free(d_stage);
    if (d_q) lal_gpu_free(d_q);
    return rc;
}

}  // extern "C"
