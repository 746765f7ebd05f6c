// The C ABI of include/dwim_hip.h: device, memory and operations of the
// reference's `gpu::Device` trait (dwim gpu/mod.rs:176-401), each operation a
// check of the trait's contract followed by a kernel launch on the device's
// one stream.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

static thread_local std::string g_error;

int dwim_fail(const std::string &msg) {
    g_error = msg;
    return 1;
}

extern "C" const char *dwim_last_error(void) { return g_error.c_str(); }

#define LAUNCH(call)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) return dwim_fail(std::string("launch: ") + hipGetErrorString(e_)); \
    } while (0)

// ---------------------------------------------------------------- device

extern "C" int dwim_open(int index, dwim_dev **out) {
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return dwim_fail("no HIP device");
    if (index < 0 || index >= count) return dwim_fail("no HIP device " + std::to_string(index));
    hipDeviceProp_t prop;
    DWIM_HIP(hipGetDeviceProperties(&prop, index));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return dwim_fail(std::string("device is ") + prop.gcnArchName + ", not gfx950 (MI355X)");
    DWIM_HIP(hipSetDevice(index));
    dwim_dev *dev = new dwim_dev();
    dev->index = index;
    dev->name = prop.name[0] ? prop.name : (std::string("AMD ") + prop.gcnArchName);
    dev->cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking) != hipSuccess) {
        delete dev;
        return dwim_fail("creating a stream failed");
    }
    // the activation planes of one-token matrix products (its zero bytes stay zero)
    if (hipMalloc(&dev->planes, planes_scratch_bytes()) != hipSuccess ||
        hipMemset(dev->planes, 0, planes_scratch_bytes()) != hipSuccess) {
        if (dev->planes) (void)hipFree(dev->planes);
        (void)hipStreamDestroy(dev->stream);
        delete dev;
        return dwim_fail("allocating the activation planes failed");
    }
    // the split matrix products' partial sums and counters
    dev->mv_tiles_cap = 4096;
    if (hipMalloc(&dev->mv_partials, (size_t)dev->mv_tiles_cap * 4 * 4 * 32 * sizeof(float)) != hipSuccess ||
        hipMalloc(&dev->mv_counters, (size_t)dev->mv_tiles_cap * sizeof(unsigned)) != hipSuccess ||
        hipMemset(dev->mv_counters, 0, (size_t)dev->mv_tiles_cap * sizeof(unsigned)) != hipSuccess ||
        hipMalloc(&dev->mv_stream, (dev->mv_stream_cap = (size_t)4 << 20) * sizeof(float)) != hipSuccess) {
        dev->refs = 0;
        dwim_dev_release_resources(dev);
        return dwim_fail("allocating the split-product scratch failed");
    }
    // the address of the scratch array dwim_attention_noalloc uses, on this device
    if (attention_scratch_init(dev) != hipSuccess) {
        dev->refs = 0;
        dwim_dev_release_resources(dev);
        return dwim_fail("taking the address of the attention scratch array failed");
    }
    *out = dev;
    return 0;
}

hipError_t dev_grow(dwim_dev *dev, void **ptr, size_t *cap, size_t need, size_t elem) {
    if (*cap >= need) return hipSuccess;
    if (*ptr) {
        // whatever is queued may still read the old buffer
        hipError_t e = hipStreamSynchronize(dev->stream);
        if (e != hipSuccess) return e;
        (void)hipFree(*ptr);
    }
    *ptr = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc(ptr, need * elem);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return e;
    }
    *cap = need;
    return hipSuccess;
}

float *dev_work(dwim_dev *dev, size_t floats) {
    if (dev_grow(dev, (void **)&dev->work, &dev->work_cap, floats, sizeof(float)) != hipSuccess) return nullptr;
    return dev->work;
}

void dwim_dev_release_resources(dwim_dev *dev) {
    (void)hipSetDevice(dev->index);
    (void)hipStreamSynchronize(dev->stream);
    if (dev->mv_partials) (void)hipFree(dev->mv_partials);
    if (dev->mv_counters) (void)hipFree(dev->mv_counters);
    if (dev->mv_stream) (void)hipFree(dev->mv_stream);
    if (dev->partials) (void)hipFree(dev->partials);
    if (dev->argmax_buf) (void)hipFree(dev->argmax_buf);
    if (dev->tokens) (void)hipFree(dev->tokens);
    if (dev->planes) (void)hipFree(dev->planes);
    if (dev->split) (void)hipFree(dev->split);
    if (dev->work) (void)hipFree(dev->work);
    if (dev->gemm_parts) (void)hipFree(dev->gemm_parts);
    if (dev->dn_work) (void)hipFree(dev->dn_work);
    if (dev->kvx) (void)hipFree(dev->kvx);
    (void)hipStreamDestroy(dev->stream);
    delete dev;
}

void dwim_dev_release(dwim_dev *dev) {
    if (--dev->refs > 0) return;
    dwim_dev_release_resources(dev);
}

extern "C" void dwim_close(dwim_dev *dev) {
    if (!dev) return;
    (void)hipStreamSynchronize(dev->stream);
    dwim_dev_release(dev);
}

extern "C" int dwim_name(dwim_dev *dev, char *out, size_t cap) {
    DWIM_CHECK(cap > 0, "no room for the name");
    snprintf(out, cap, "%s", dev->name.c_str());
    return 0;
}

extern "C" int dwim_memory(dwim_dev *dev, uint64_t *free_bytes) {
    size_t f = 0, t = 0;
    DWIM_HIP(hipSetDevice(dev->index));
    DWIM_HIP(hipMemGetInfo(&f, &t));
    *free_bytes = f;
    return 0;
}

// Prefill batches of 4096 tokens: the batch GEMM's 256 × 128 tiles then come
// to over 8 workgroups a CU for the 27B shape's matrices, so that the last,
// partly filled round of workgroups is a small share (at 2048 tokens the
// 17408-row products make 1088 tiles for 256 CUs: 4.25 rounds; measured 4%
// faster prefill at 4096), and a batch's activations (4096 × 17408 f32 at
// most) stay small next to 288 GB.
extern "C" size_t dwim_batch(dwim_dev *) { return 4096; }

extern "C" int dwim_sync(dwim_dev *dev) {
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

extern "C" void *dwim_stream(dwim_dev *dev) { return (void *)dev->stream; }

// ---------------------------------------------------------------- memory

extern "C" int dwim_alloc(dwim_dev *dev, size_t len, dwim_buf **out) {
    *out = nullptr;
    float *p = nullptr;
    DWIM_HIP(hipMalloc(&p, std::max<size_t>(len, 1) * sizeof(float)));
    if (hipMemsetAsync(p, 0, std::max<size_t>(len, 1) * sizeof(float), dev->stream) != hipSuccess) {
        (void)hipFree(p);
        return dwim_fail("zeroing a buffer failed");
    }
    dev->refs++;
    *out = new dwim_buf{dev, p, len, len};
    return 0;
}

extern "C" void dwim_free_buffer(dwim_buf *buf) {
    if (!buf) return;
    dwim_dev *dev = buf->dev;
    (void)hipStreamSynchronize(dev->stream);
    (void)hipFree(buf->data);
    delete buf;
    dwim_dev_release(dev);
}

extern "C" int dwim_alloc_cache(dwim_dev *dev, size_t len, dwim_cache **out) {
    *out = nullptr;
    DWIM_CHECK(len % 32 == 0, "a cache holds whole blocks of 32");
    int8_t *q = nullptr;
    uint16_t *s = nullptr;
    DWIM_HIP(hipMalloc(&q, std::max<size_t>(len, 32)));
    if (hipMalloc(&s, std::max<size_t>(len / 32, 1) * 2) != hipSuccess) {
        (void)hipFree(q);
        return dwim_fail("allocating a cache failed");
    }
    if (hipMemsetAsync(q, 0, std::max<size_t>(len, 32), dev->stream) != hipSuccess ||
        hipMemsetAsync(s, 0, std::max<size_t>(len / 32, 1) * 2, dev->stream) != hipSuccess) {
        (void)hipFree(q);
        (void)hipFree(s);
        return dwim_fail("clearing a new cache failed");
    }
    dev->refs++;
    *out = new dwim_cache{dev, q, s, len};
    return 0;
}

extern "C" int dwim_alloc_cache_f16(dwim_dev *dev, size_t len, dwim_cache **out) {
    *out = nullptr;
    DWIM_CHECK(len % 32 == 0, "a cache holds whole blocks of 32");
    int8_t *q = nullptr;
    DWIM_HIP(hipMalloc(&q, std::max<size_t>(len, 32) * 2));
    if (hipMemsetAsync(q, 0, std::max<size_t>(len, 32) * 2, dev->stream) != hipSuccess) {
        (void)hipFree(q);
        return dwim_fail("clearing a new cache failed");
    }
    dev->refs++;
    *out = new dwim_cache{dev, q, nullptr, len, true};
    return 0;
}

extern "C" void dwim_free_cache(dwim_cache *c) {
    if (!c) return;
    dwim_dev *dev = c->dev;
    (void)hipStreamSynchronize(dev->stream);
    (void)hipFree(c->q);
    (void)hipFree(c->s);
    delete c;
    dwim_dev_release(dev);
}

extern "C" int dwim_resize(dwim_dev *, dwim_buf *buf, size_t len) {
    if (len > buf->cap)
        return dwim_fail("a buffer of " + std::to_string(buf->cap) + " activations can't hold " +
                         std::to_string(len));
    buf->len = len;
    return 0;
}

extern "C" size_t dwim_len(const dwim_buf *buf) { return buf->len; }

extern "C" int dwim_read(dwim_dev *dev, const dwim_buf *buf, float *out, size_t len) {
    DWIM_CHECK(len == buf->len, "reading " + std::to_string(len) + " of a buffer of " +
                                    std::to_string(buf->len));
    if (len) DWIM_HIP(hipMemcpyAsync(out, buf->data, len * 4, hipMemcpyDeviceToHost, dev->stream));
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

extern "C" int dwim_write(dwim_dev *dev, dwim_buf *buf, const float *data, size_t len) {
    DWIM_CHECK(len == buf->len, "writing " + std::to_string(len) + " into a buffer of " +
                                    std::to_string(buf->len));
    if (len) DWIM_HIP(hipMemcpyAsync(buf->data, data, len * 4, hipMemcpyHostToDevice, dev->stream));
    // The host data may be freed as soon as this returns.
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

extern "C" int dwim_copy(dwim_dev *dev, dwim_buf *dst, size_t dst_offset, const dwim_buf *src,
                         size_t src_offset, size_t len) {
    DWIM_CHECK(dst_offset + len <= dst->len && src_offset + len <= src->len,
               "copying past the end of a buffer");
    if (len)
        DWIM_HIP(hipMemcpyAsync(dst->data + dst_offset, src->data + src_offset, len * 4,
                                hipMemcpyDeviceToDevice, dev->stream));
    return 0;
}

extern "C" size_t dwim_cache_bytes(size_t len) { return len + len / 32 * 2; }

extern "C" size_t dwim_cache_bytes_of(const dwim_cache *cache, size_t len) {
    return cache->f16 ? 2 * len : dwim_cache_bytes(len);
}

extern "C" int dwim_store(dwim_dev *dev, dwim_cache *cache, size_t offset, const dwim_buf *src) {
    DWIM_CHECK(offset % 32 == 0 && src->len % 32 == 0, "stores are whole blocks of 32");
    DWIM_CHECK(offset + src->len <= cache->len, "storing past the end of a cache");
    if (src->len == 0) return 0;
    if (cache->f16)
        LAUNCH(launch_store_f16(dev->stream, (uint16_t *)cache->q + offset, src->data, src->len));
    else
        LAUNCH(launch_store(dev->stream, cache->q + offset, cache->s + offset / 32, src->data, src->len / 32));
    return 0;
}

extern "C" int dwim_read_cache(dwim_dev *dev, const dwim_cache *cache, size_t len, uint8_t *out,
                               size_t out_bytes) {
    DWIM_CHECK(len % 32 == 0 && len <= cache->len, "reading a cache past its end or mid-block");
    DWIM_CHECK(out_bytes >= dwim_cache_bytes_of(cache, len), "read_cache: the output holds fewer bytes than the cache gives");
    if (len && cache->f16) {
        DWIM_HIP(hipMemcpyAsync(out, cache->q, 2 * len, hipMemcpyDeviceToHost, dev->stream));
    } else if (len) {
        DWIM_HIP(hipMemcpyAsync(out, cache->q, len, hipMemcpyDeviceToHost, dev->stream));
        DWIM_HIP(hipMemcpyAsync(out + len, cache->s, len / 32 * 2, hipMemcpyDeviceToHost, dev->stream));
    }
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

extern "C" int dwim_write_cache(dwim_dev *dev, dwim_cache *cache, const uint8_t *data, size_t bytes) {
    if (cache->f16) {
        DWIM_CHECK(bytes % 64 == 0, "cache bytes are not whole blocks");
        DWIM_CHECK(bytes / 2 <= cache->len, "writing past the end of a cache");
        if (bytes) DWIM_HIP(hipMemcpyAsync(cache->q, data, bytes, hipMemcpyHostToDevice, dev->stream));
        DWIM_HIP(hipStreamSynchronize(dev->stream));
        return 0;
    }
    size_t len = bytes / 34 * 32;
    DWIM_CHECK(bytes == dwim_cache_bytes(len), "cache bytes are not whole blocks");
    DWIM_CHECK(len <= cache->len, "writing past the end of a cache");
    if (len) {
        DWIM_HIP(hipMemcpyAsync(cache->q, data, len, hipMemcpyHostToDevice, dev->stream));
        DWIM_HIP(hipMemcpyAsync(cache->s, data + len, len / 32 * 2, hipMemcpyHostToDevice, dev->stream));
    }
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

// ---------------------------------------------------------------- weights

static int alloc_copy(dwim_dev *dev, void **dst, const void *src, size_t bytes) {
    DWIM_HIP(hipMalloc(dst, std::max<size_t>(bytes, 16)));
    if (src && bytes) DWIM_HIP(hipMemcpyAsync(*dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
    return 0;
}

extern "C" void dwim_free_weight(dwim_weight *w) {
    if (!w) return;
    dwim_dev *dev = w->dev;
    (void)hipStreamSynchronize(dev->stream);
    for (void *p : {w->q, w->s, w->s2, w->s3})
        if (p) (void)hipFree(p);
    delete w;
    dwim_dev_release(dev);
}

static int check_shape(int fmt, size_t rows, size_t cols) {
    DWIM_CHECK(rows > 0 && cols > 0, "an empty weight matrix");
    switch (fmt) {
    case DWIM_BF16: DWIM_CHECK(cols % 8 == 0, "bf16 rows are whole groups of 8"); break;
    case DWIM_Q4_0:
    case DWIM_Q8_0: DWIM_CHECK(cols % 32 == 0, "rows must be a whole number of blocks"); break;
    case DWIM_Q4_K:
        DWIM_CHECK(cols % 256 == 0, "K-quant rows are whole blocks of 256");
        DWIM_CHECK(cols <= 80 * 256, "Q4_K rows of at most 20480 weights");
        break;
    case DWIM_Q6_K: DWIM_CHECK(cols % 256 == 0, "K-quant rows are whole blocks of 256"); break;
    default: return dwim_fail("unknown weight format " + std::to_string(fmt));
    }
    return 0;
}

extern "C" int dwim_upload(dwim_dev *dev, int fmt, size_t rows, size_t cols, const void *quants,
                           const uint16_t *scales, dwim_weight **out) {
    *out = nullptr;
    if (check_shape(fmt, rows, cols)) return 1;
    DWIM_HIP(hipSetDevice(dev->index));
    dwim_weight *w = new dwim_weight{dev, fmt, rows, cols};
    dev->refs++;
    int err = 0;
    size_t nb = cols / 256;
    switch (fmt) {
    case DWIM_BF16: err = alloc_copy(dev, &w->q, quants, rows * cols * 2); break;
    case DWIM_Q4_0:
        err = alloc_copy(dev, &w->q, quants, rows * cols / 2) ||
              alloc_copy(dev, &w->s, scales, rows * cols / 32 * 2);
        break;
    case DWIM_Q8_0:
        err = alloc_copy(dev, &w->q, quants, rows * cols) ||
              alloc_copy(dev, &w->s, scales, rows * cols / 32 * 2);
        break;
    case DWIM_Q4_K: {
        // 144-byte blocks -> 64-row tiles (layout.h), padding rows zero
        std::vector<uint8_t> tiled(q4kt::bytes(rows, cols), 0);
        const uint8_t *src = (const uint8_t *)quants;
        for (size_t r = 0; r < rows; r++)
            for (size_t b = 0; b < nb; b++) q4kt::place(tiled.data(), nb, r, b, src + (r * nb + b) * 144);
        err = alloc_copy(dev, &w->q, tiled.data(), tiled.size());
        if (!err) err = hipStreamSynchronize(dev->stream) != hipSuccess;
        break;
    }
    case DWIM_Q6_K: {
        std::vector<uint8_t> ql(rows * nb * 128), qh(rows * nb * 64), sc(rows * nb * 16);
        std::vector<uint16_t> d(rows * nb);
        const uint8_t *src = (const uint8_t *)quants;
        for (size_t b = 0; b < rows * nb; b++) {
            memcpy(&ql[b * 128], src + b * 210, 128);
            memcpy(&qh[b * 64], src + b * 210 + 128, 64);
            memcpy(&sc[b * 16], src + b * 210 + 192, 16);
            d[b] = (uint16_t)(src[b * 210 + 208] | src[b * 210 + 209] << 8);
        }
        err = alloc_copy(dev, &w->q, ql.data(), ql.size()) || alloc_copy(dev, &w->s, qh.data(), qh.size()) ||
              alloc_copy(dev, &w->s2, sc.data(), sc.size()) || alloc_copy(dev, &w->s3, d.data(), d.size() * 2);
        if (!err) err = hipStreamSynchronize(dev->stream) != hipSuccess;
        break;
    }
    }
    if (!err && hipStreamSynchronize(dev->stream) != hipSuccess) err = dwim_fail("uploading a weight failed");
    if (err) {
        dwim_free_weight(w);
        return 1;
    }
    *out = w;
    return 0;
}

extern "C" int dwim_upload_synthetic(dwim_dev *dev, int fmt, size_t rows, size_t cols, uint64_t seed,
                                     float sigma, dwim_weight **out) {
    *out = nullptr;
    if (check_shape(fmt, rows, cols)) return 1;
    DWIM_CHECK(fmt == DWIM_Q4_K || fmt == DWIM_Q6_K || fmt == DWIM_BF16,
               "synthetic weights are Q4_K, Q6_K or bf16");
    DWIM_HIP(hipSetDevice(dev->index));
    float c = sigma * (1.7320508075688772f / 65536.0f);
    dwim_weight *w = new dwim_weight{dev, fmt, rows, cols};
    dev->refs++;
    size_t nb = cols / 256;
    int err = 0;
    if (fmt == DWIM_Q4_K) {
        err = alloc_copy(dev, &w->q, nullptr, q4kt::bytes(rows, cols));
        if (!err) err = hipMemsetAsync(w->q, 0, q4kt::bytes(rows, cols), dev->stream) != hipSuccess;
        if (!err) err = launch_synthetic_q4_k(dev->stream, (uint8_t *)w->q, rows, cols, seed, c) != hipSuccess;
    } else if (fmt == DWIM_Q6_K) {
        err = alloc_copy(dev, &w->q, nullptr, rows * nb * 128) || alloc_copy(dev, &w->s, nullptr, rows * nb * 64) ||
              alloc_copy(dev, &w->s2, nullptr, rows * nb * 16) || alloc_copy(dev, &w->s3, nullptr, rows * nb * 2);
        if (!err)
            err = launch_synthetic_q6_k(dev->stream, (uint8_t *)w->q, (uint8_t *)w->s, (int8_t *)w->s2,
                                        (uint16_t *)w->s3, rows, cols, seed, c) != hipSuccess;
    } else {
        err = alloc_copy(dev, &w->q, nullptr, rows * cols * 2);
        if (!err) err = launch_synthetic_bf16(dev->stream, (uint16_t *)w->q, rows, cols, seed, c) != hipSuccess;
    }
    if (!err && hipStreamSynchronize(dev->stream) != hipSuccess) err = 1;
    if (err) {
        dwim_free_weight(w);
        return dwim_fail("building a synthetic weight failed");
    }
    *out = w;
    return 0;
}

// ---------------------------------------------------------------- operations

static int matmul_shapes(const dwim_buf *out, const dwim_weight *w, const dwim_buf *x, size_t *n) {
    *n = x->len / w->cols;
    DWIM_CHECK(*n * w->cols == x->len, "the input is not whole rows of the weight's width");
    DWIM_CHECK(out->len == *n * w->rows, "the output is not a row of the weight's height per token");
    return 0;
}

extern "C" int dwim_matmul(dwim_dev *dev, dwim_buf *out, const dwim_weight *w, const dwim_buf *x) {
    size_t n;
    if (matmul_shapes(out, w, x, &n)) return 1;
    if (n == 0) return 0;
    LAUNCH(launch_matvec(dev, w, out->data, x->data, n, 0));
    return 0;
}

extern "C" int dwim_matmul_add(dwim_dev *dev, dwim_buf *x, const dwim_weight *w, const dwim_buf *input,
                               dwim_buf *scratch) {
    size_t n;
    if (matmul_shapes(x, w, input, &n)) return 1;
    DWIM_CHECK(scratch->cap >= x->len, "the scratch buffer is shorter than x");
    if (n == 0) return 0;
    LAUNCH(launch_matvec(dev, w, x->data, input->data, n, 1));
    return 0;
}

extern "C" int dwim_prepare(dwim_dev *dev, const dwim_buf *x) {
    DWIM_CHECK(x->len > 0 && x->len % 256 == 0 && x->len <= 80 * 256,
               "prepare: one token of whole 256-blocks, at most 20480");
    LAUNCH(launch_planes(dev, x->data, x->len, nullptr, 0.0f, nullptr, 0));
    dev->prepared = x->len;
    return 0;
}

extern "C" int dwim_matmul_prepared(dwim_dev *dev, dwim_buf *out, const dwim_weight *w) {
    DWIM_CHECK(w->fmt == DWIM_Q4_K, "matmul_prepared: a Q4_K weight");
    DWIM_CHECK(dev->prepared == w->cols, "matmul_prepared: no activations of the weight's width prepared");
    DWIM_CHECK(out->len == w->rows, "matmul_prepared: out must hold one row of results");
    const int add = 0;
    float *o = out->data;
    LAUNCH(launch_mv_q4k_mfma(dev, &w, &o, &add, 1, 0, 0));
    return 0;
}

extern "C" int dwim_swiglu_prepared(dwim_dev *dev, dwim_buf *out, const dwim_weight *gate, const dwim_weight *up) {
    DWIM_CHECK(gate->fmt == DWIM_Q4_K && up->fmt == DWIM_Q4_K, "swiglu_prepared: Q4_K weights");
    DWIM_CHECK(up->rows == gate->rows && up->cols == gate->cols, "gate and up differ in shape");
    DWIM_CHECK(dev->prepared == gate->cols, "swiglu_prepared: no activations of the weights' width prepared");
    DWIM_CHECK(out->len == gate->rows, "swiglu_prepared: out must hold one row of results");
    DWIM_CHECK(gate->rows % 256 == 0 && gate->rows <= 80 * 256, "swiglu_prepared: rows in whole planes groups");
    const dwim_weight *ws[2] = {gate, up};
    float *outs[2] = {out->data, nullptr};
    MvExtra e;
    e.emit_area = 1;
    LAUNCH(launch_mv_q4k_mfma(dev, ws, outs, nullptr, 2, 1, 0, &e));
    return 0;
}

extern "C" int dwim_swiglu(dwim_dev *dev, dwim_buf *out, const dwim_weight *gate, const dwim_weight *up,
                           const dwim_buf *x, dwim_buf *scratch) {
    size_t n;
    if (matmul_shapes(out, gate, x, &n)) return 1;
    DWIM_CHECK(up->rows == gate->rows && up->cols == gate->cols, "gate and up differ in shape");
    DWIM_CHECK(scratch->cap >= out->len, "the scratch buffer is shorter than out");
    if (n == 0) return 0;
    LAUNCH(launch_swiglu(dev, gate, up, out->data, scratch->data, x->data, n));
    return 0;
}

extern "C" int dwim_add(dwim_dev *dev, dwim_buf *x, const dwim_buf *y) {
    DWIM_CHECK(y->len == x->len, "adding buffers of different lengths");
    if (x->len) LAUNCH(launch_add(dev->stream, x->data, y->data, x->len));
    return 0;
}

extern "C" int dwim_normalize(dwim_dev *dev, dwim_buf *out, const dwim_buf *x, const dwim_buf *weight,
                              size_t len, float eps) {
    DWIM_CHECK(len <= x->len && out->len == len, "normalize: out must be len long, within x");
    DWIM_CHECK(weight->len > 0 && len % weight->len == 0, "normalize: len is not whole rows");
    if (len) LAUNCH(launch_rmsnorm(dev->stream, out->data, x->data, weight->data, len / weight->len, weight->len, eps));
    return 0;
}

extern "C" int dwim_rmsnorm(dwim_dev *dev, dwim_buf *x, const dwim_buf *weight, float eps) {
    DWIM_CHECK(weight->len > 0, "rmsnorm: an empty weight");
    size_t rows = x->len / weight->len;
    if (rows) LAUNCH(launch_rmsnorm(dev->stream, x->data, x->data, weight->data, rows, weight->len, eps));
    return 0;
}

extern "C" int dwim_l2norm(dwim_dev *dev, dwim_buf *x, size_t dim, float eps) {
    DWIM_CHECK(dim > 0, "l2norm: rows of no width");
    size_t rows = x->len / dim;
    if (rows) LAUNCH(launch_l2norm(dev->stream, x->data, rows, dim, eps));
    return 0;
}

extern "C" int dwim_rope(dwim_dev *dev, dwim_buf *x, const dwim_buf *table, size_t pos, size_t n_heads,
                         size_t head_dim, size_t rot_dim) {
    DWIM_CHECK(rot_dim % 2 == 0 && rot_dim <= head_dim, "rope: rot_dim must be even and within a head");
    size_t width = n_heads * head_dim;
    DWIM_CHECK(width > 0 && x->len % width == 0, "rope: x is not whole tokens of heads");
    size_t n = x->len / width;
    DWIM_CHECK((pos + n) * rot_dim <= table->len, "rope: the table does not reach the last position");
    if (n && rot_dim) LAUNCH(launch_rope(dev->stream, x->data, table->data, n, pos, n_heads, head_dim, rot_dim));
    return 0;
}

extern "C" int dwim_attention(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_cache *k_cache,
                              const dwim_cache *v_cache, size_t pos, size_t n_heads, size_t head_dim,
                              size_t n_kv_heads) {
    DWIM_CHECK(head_dim % 32 == 0 && head_dim <= 256 && head_dim > 0,
               "attention: heads are whole blocks of 32, at most 256");
    DWIM_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 8,
               "attention: at most 8 query heads to a key/value head");
    size_t width = n_heads * head_dim;
    DWIM_CHECK(q->len % width == 0 && out->len == q->len, "attention: q and out are whole tokens");
    size_t n = q->len / width;
    size_t kv_dim = n_kv_heads * head_dim;
    DWIM_CHECK((pos + n) * kv_dim <= k_cache->len && (pos + n) * kv_dim <= v_cache->len,
               "attention: the caches do not hold the tokens' positions");
    DWIM_CHECK(k_cache->f16 == v_cache->f16, "attention: the key and value caches are of different formats");
    if (n) LAUNCH(launch_attention(dev, out->data, q->data, k_cache, v_cache, n, pos, n_heads, head_dim, n_kv_heads));
    return 0;
}

extern "C" int dwim_silu_mul(dwim_dev *dev, dwim_buf *gate, const dwim_buf *up) {
    DWIM_CHECK(up->len == gate->len, "silu_mul: buffers of different lengths");
    if (gate->len) LAUNCH(launch_silu_mul(dev->stream, gate->data, up->data, gate->len));
    return 0;
}

extern "C" int dwim_sigmoid_mul(dwim_dev *dev, dwim_buf *x, const dwim_buf *gate) {
    DWIM_CHECK(gate->len == x->len, "sigmoid_mul: buffers of different lengths");
    if (x->len) LAUNCH(launch_sigmoid_mul(dev->stream, x->data, gate->data, x->len));
    return 0;
}

extern "C" int dwim_conv(dwim_dev *dev, dwim_buf *q, dwim_buf *k, dwim_buf *v, dwim_buf *state_out,
                         const dwim_buf *x, const dwim_buf *state, const dwim_buf *weight) {
    DWIM_CHECK(weight->len % 4 == 0 && weight->len > 0, "conv: 4 taps per channel");
    size_t ch = weight->len / 4;
    size_t n = x->len / ch;
    DWIM_CHECK(n * ch == x->len && n > 0, "conv: x is not whole rows of channels");
    DWIM_CHECK(state->len == 3 * ch && state_out->len == state->len, "conv: states are 3 rows of channels");
    size_t qd = q->len / n, kd = k->len / n, vd = v->len / n;
    DWIM_CHECK(qd * n == q->len && kd * n == k->len && vd * n == v->len && qd + kd + vd == ch,
               "conv: q, k and v do not split the channels");
    DWIM_CHECK(state_out->data != state->data, "conv: state_out must be another buffer than state");
    LAUNCH(launch_conv(dev->stream, q->data, k->data, v->data, state_out->data, x->data, state->data,
                       weight->data, n, qd, kd, vd));
    return 0;
}

static int delta_net_checked(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_buf *k, const dwim_buf *v,
                             const dwim_buf *gates, const dwim_buf *decay, dwim_buf *state, size_t n_k_heads,
                             size_t n_v_heads, size_t head_dim, bool unit_keys) {
    DWIM_CHECK(head_dim == 128, "delta_net: heads of 128");
    DWIM_CHECK(n_k_heads > 0 && n_v_heads % n_k_heads == 0, "delta_net: value heads a multiple of key heads");
    size_t n = v->len / (n_v_heads * head_dim);
    DWIM_CHECK(v->len == n * n_v_heads * head_dim, "delta_net: v is not whole tokens");
    DWIM_CHECK(q->len == n * n_k_heads * head_dim && k->len == q->len && out->len == v->len,
               "delta_net: q, k, out do not match v");
    DWIM_CHECK(gates->len == n * 2 * n_v_heads && decay->len == 2 * n_v_heads, "delta_net: gates or decay");
    DWIM_CHECK(state->len == n_v_heads * head_dim * head_dim, "delta_net: the state");
    if (n)
        LAUNCH(launch_delta_net(dev, out->data, q->data, k->data, v->data, gates->data, decay->data,
                                state->data, n, n_k_heads, n_v_heads, head_dim, nullptr, unit_keys));
    return 0;
}

extern "C" int dwim_delta_net(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_buf *k,
                              const dwim_buf *v, const dwim_buf *gates, const dwim_buf *decay, dwim_buf *state,
                              size_t n_k_heads, size_t n_v_heads, size_t head_dim) {
    return delta_net_checked(dev, out, q, k, v, gates, decay, state, n_k_heads, n_v_heads, head_dim, false);
}

extern "C" int dwim_delta_net_unit_keys(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_buf *k,
                                        const dwim_buf *v, const dwim_buf *gates, const dwim_buf *decay,
                                        dwim_buf *state, size_t n_k_heads, size_t n_v_heads, size_t head_dim) {
    return delta_net_checked(dev, out, q, k, v, gates, decay, state, n_k_heads, n_v_heads, head_dim, true);
}

extern "C" int dwim_conv_l2norm(dwim_dev *dev, dwim_buf *q, dwim_buf *k, dwim_buf *v, dwim_buf *state_out,
                                const dwim_buf *x, const dwim_buf *state, const dwim_buf *weight, size_t dim,
                                float eps) {
    DWIM_CHECK(weight->len % 4 == 0 && weight->len > 0, "conv: 4 taps per channel");
    size_t ch = weight->len / 4;
    size_t n = x->len / ch;
    DWIM_CHECK(n * ch == x->len && n > 0, "conv: x is not whole rows of channels");
    DWIM_CHECK(state->len == 3 * ch && state_out->len == state->len, "conv: states are 3 rows of channels");
    size_t qd = q->len / n, kd = k->len / n, vd = v->len / n;
    DWIM_CHECK(qd * n == q->len && kd * n == k->len && vd * n == v->len && qd + kd + vd == ch,
               "conv: q, k and v do not split the channels");
    DWIM_CHECK(state_out->data != state->data, "conv: state_out must be another buffer than state");
    DWIM_CHECK(dim % 64 == 0 && dim > 0 && dim <= 256 && qd % dim == 0 && kd % dim == 0 && vd % dim == 0,
               "conv_l2norm: rows of a multiple of 64 up to 256 that divide q, k and v");
    LAUNCH(launch_conv_l2(dev->stream, q->data, k->data, v->data, state_out->data, x->data, state->data,
                          weight->data, n, qd, kd, vd, dim, eps));
    return 0;
}

extern "C" int dwim_embed(dwim_dev *dev, dwim_buf *out, const dwim_weight *table, const uint32_t *tokens,
                          size_t n) {
    DWIM_CHECK(out->len == n * table->cols, "embed: out must hold a row per token");
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= table->rows)
            return dwim_fail("embed: token " + std::to_string(tokens[i]) + " is past the table's " +
                             std::to_string(table->rows) + " rows");
    if (n == 0) return 0;
    DWIM_HIP(dev_grow(dev, (void **)&dev->tokens, &dev->tokens_cap, n, 4));
    // the ids go through the stream, after whatever still reads the previous ones
    DWIM_HIP(hipMemcpyAsync(dev->tokens, tokens, n * 4, hipMemcpyHostToDevice, dev->stream));
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    LAUNCH(launch_embed(dev->stream, out->data, table, dev->tokens, n));
    return 0;
}

extern "C" int dwim_argmax(dwim_dev *dev, const dwim_buf *logits, size_t rows, uint32_t *out) {
    DWIM_CHECK(rows > 0 && logits->len % rows == 0, "argmax: logits are not whole rows");
    DWIM_HIP(dev_grow(dev, (void **)&dev->argmax_buf, &dev->argmax_cap, argmax_scratch_words(rows), 4));
    LAUNCH(launch_argmax(dev->stream, logits->data, rows, logits->len / rows, dev->argmax_buf));
    DWIM_HIP(hipMemcpyAsync(out, dev->argmax_buf, rows * 4, hipMemcpyDeviceToHost, dev->stream));
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    return 0;
}

// ---------------------------------------------------------------- host helpers

extern "C" uint16_t dwim_to_f16(float x) { return dq::to_f16(x); }
extern "C" float dwim_from_f16(uint16_t b) { return dq::from_f16(b); }

extern "C" void dwim_quantize_block(const float *block, uint16_t *scale, int8_t *q) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(block[i]));
    uint16_t bits = dq::block_scale(amax);
    float d = dq::from_f16(bits);
    for (int i = 0; i < 32; i++) q[i] = d > 0.0f ? dq::quantize_one(block[i], d) : 0;
    *scale = bits;
}

extern "C" void dwim_quantize_q8_0_row(const float *x, size_t cols, uint16_t *scales, int8_t *quants) {
    for (size_t b = 0; b < cols / 32; b++) dwim_quantize_block(x + 32 * b, scales + b, quants + 32 * b);
}

// gpu/quant.rs:89-109: the block's scale is its weight of largest magnitude,
// sign and all, over -8; each weight clamp(x/d + 8.5, 0, 15), truncated.
extern "C" void dwim_quantize_q4_0_row(const float *x, size_t cols, uint16_t *scales, uint8_t *quants) {
#pragma clang fp contract(off)
    for (size_t b = 0; b < cols / 32; b++) {
        const float *blk = x + 32 * b;
        float max = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(blk[i]) > fabsf(max)) max = blk[i];
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        scales[b] = dq::to_f16(d);
        for (int j = 0; j < 16; j++) {
            float lo = fminf(fmaxf(blk[j] * id + 8.5f, 0.0f), 15.0f);
            float hi = fminf(fmaxf(blk[j + 16] * id + 8.5f, 0.0f), 15.0f);
            quants[16 * b + j] = (uint8_t)((uint8_t)lo | ((uint8_t)hi << 4));
        }
    }
}

extern "C" void dwim_quantize_q4_k_row(const float *x, size_t cols, uint8_t *blocks) {
    for (size_t b = 0; b < cols / 256; b++) dq::quantize_q4_k_block(x + 256 * b, blocks + 144 * b);
}

extern "C" void dwim_quantize_q6_k_row(const float *x, size_t cols, uint8_t *blocks) {
    for (size_t b = 0; b < cols / 256; b++) dq::quantize_q6_k_block(x + 256 * b, blocks + 210 * b);
}

extern "C" void dwim_synthetic_values(uint64_t seed, uint64_t first, size_t n, float sigma, float *out) {
    float c = sigma * (1.7320508075688772f / 65536.0f);
    for (size_t i = 0; i < n; i++) out[i] = dq::synthetic(seed, first + i, c);
}
