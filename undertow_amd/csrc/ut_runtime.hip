// ut_runtime.hip -- context, errors, scratch arena, kernel timing and the
// device QTensor container (undertow-quant/src/qtensor.rs:17-138).
#include <cstdarg>
#include <cstring>

#include "ut_internal.h"

namespace ut {

void set_error(ut_ctx *ctx, const char *fmt, ...) {
    if (!ctx) return;
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->err = buf;
}

int64_t payload_bytes(int32_t fmt, int64_t out_dim, int64_t in_dim) {
    // QuantFormat::payload_bytes (qtensor.rs:43-49)
    switch (fmt) {
    case UT_FMT_F32: return out_dim * in_dim * 4;
    case UT_FMT_INT8: return out_dim * in_dim;
    case UT_FMT_INT4: return out_dim * ((in_dim + 1) / 2);
    default: return -1;
    }
}

int32_t scratch_acquire(ut_ctx *ctx, const ScratchPlan &plan, std::vector<void *> &ptrs) {
    size_t total = 0;
    for (size_t s : plan.sizes) total += s;
    if (total > ctx->scratch.bytes) {
        UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->scratch.ptr) UT_CHECK_HIP(ctx, hipFree(ctx->scratch.ptr));
        ctx->scratch.ptr = nullptr;
        ctx->scratch.bytes = 0;
        size_t want = total + total / 4 + (1 << 20);
        if (hipMalloc(&ctx->scratch.ptr, want) != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx, "scratch allocation of %zu bytes failed", want);
            return UT_ERR_OOM;
        }
        ctx->scratch.bytes = want;
    }
    ptrs.clear();
    char *p = (char *)ctx->scratch.ptr;
    for (size_t s : plan.sizes) {
        ptrs.push_back(p);
        p += s;
    }
    return UT_OK;
}

int32_t pinned_acquire(ut_ctx *ctx, size_t bytes, void **ptr) {
    if (bytes > ctx->pinned_bytes) {
        UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->pinned) UT_CHECK_HIP(ctx, hipHostFree(ctx->pinned));
        ctx->pinned = nullptr;
        ctx->pinned_bytes = 0;
        size_t want = bytes < 65536 ? 65536 : bytes;
        if (hipHostMalloc(&ctx->pinned, want, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx, "pinned allocation of %zu bytes failed", want);
            return UT_ERR_OOM;
        }
        ctx->pinned_bytes = want;
    }
    *ptr = ctx->pinned;
    return UT_OK;
}

static void timing_collect(ut_ctx *ctx, bool wait) {
    size_t keep = 0;
    for (size_t i = 0; i < ctx->pending.size(); i++) {
        PendingTiming &p = ctx->pending[i];
        hipError_t q = wait ? hipEventSynchronize(p.stop) : hipEventQuery(p.stop);
        if (q == hipSuccess) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
                ctx->stats[p.stat].launches += 1;
                ctx->stats[p.stat].total_ms += ms;
            }
            (void)hipEventDestroy(p.start);
            (void)hipEventDestroy(p.stop);
        } else {
            (void)hipGetLastError();
            ctx->pending[keep++] = p;
        }
    }
    ctx->pending.resize(keep);
}

int timing_begin(ut_ctx *ctx, const char *name) {
    // every launch goes through here: drop error state left by unrelated
    // earlier calls so launch_check() reports this launch only
    (void)hipGetLastError();
    if (!ctx->timing) return -1;
    int idx = -1;
    for (size_t i = 0; i < ctx->stats.size(); i++)
        if (ctx->stats[i].name == name) { idx = (int)i; break; }
    if (idx < 0) {
        KernelStat ks;
        ks.name = name;
        ctx->stats.push_back(ks);
        idx = (int)ctx->stats.size() - 1;
    }
    PendingTiming p;
    p.stat = idx;
    if (hipEventCreate(&p.start) != hipSuccess) return -1;
    if (hipEventCreate(&p.stop) != hipSuccess) { (void)hipEventDestroy(p.start); return -1; }
    (void)hipEventRecord(p.start, ctx->stream);
    ctx->pending.push_back(p);
    if (ctx->pending.size() > 4096) timing_collect(ctx, true);
    return (int)ctx->pending.size() - 1;
}

void timing_end(ut_ctx *ctx, int token) {
    if (token < 0 || !ctx->timing || (size_t)token >= ctx->pending.size()) return;
    (void)hipEventRecord(ctx->pending[token].stop, ctx->stream);
}

int32_t device_error_flag(ut_ctx *ctx, int32_t **flag) {
    if (!ctx->dev_err) {
        if (hipMalloc((void **)&ctx->dev_err, 4) != hipSuccess) {
            (void)hipGetLastError();
            set_error(ctx, "error flag allocation failed");
            return UT_ERR_OOM;
        }
        UT_CHECK_HIP(ctx, hipMemset(ctx->dev_err, 0, 4));
    }
    *flag = ctx->dev_err;
    return UT_OK;
}

int32_t splitk_buffer(ut_ctx *ctx, int64_t **part) {
    if (!ctx->splitk) {
        if (hipMalloc(&ctx->splitk, kSplitKPartBytes) != hipSuccess) {
            (void)hipGetLastError();
            ctx->splitk = nullptr;
            set_error(ctx, "split-K buffer allocation failed");
            return UT_ERR_OOM;
        }
    }
    *part = (int64_t *)ctx->splitk;
    return UT_OK;
}

int32_t check_device_error(ut_ctx *ctx) {
    if (!ctx->dev_err) return UT_OK;
    int32_t f = 0;
    UT_CHECK_HIP(ctx, hipMemcpy(&f, ctx->dev_err, 4, hipMemcpyDeviceToHost));
    if (!f) return UT_OK;
    UT_CHECK_HIP(ctx, hipMemset(ctx->dev_err, 0, 4));
    set_error(ctx, "an expert id was out of range or not loaded (reported by a kernel)");
    return UT_ERR_BAD_EXPERT;
}

int32_t launch_check(ut_ctx *ctx, const char *name) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(ctx, "launch of %s failed: %s", name, hipGetErrorString(e));
        return UT_ERR_HIP;
    }
    return UT_OK;
}

// ------------------------------------------------------------ kernels ---
// QTensor::dequantize (qtensor.rs:265-272) = add_scaled_row(r, 1.0) into
// zeros (:516-543): w = 0 + (1*scale)*q = fl(scale*q).
__global__ void k_dequantize(int32_t fmt, const uint8_t *__restrict__ payload,
                             const float *__restrict__ scales, int64_t out_dim, int64_t in_dim,
                             int64_t row_bytes, float *__restrict__ out) {
    int64_t o = blockIdx.y;
    const uint8_t *row = payload + o * row_bytes;
    float s = fmt == UT_FMT_F32 ? 1.0f : scales[o];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < in_dim;
         i += (int64_t)gridDim.x * blockDim.x) {
        float v;
        if (fmt == UT_FMT_F32) {
            v = ((const float *)row)[i];
        } else if (fmt == UT_FMT_INT8) {
            v = __fmul_rn(s, (float)(int8_t)row[i]);
        } else {
            uint8_t b = row[i >> 1];
            int nib = (i & 1) ? (b >> 4) : (b & 0xF);
            int q = (nib ^ 8) - 8;  // sign-extend the two's-complement nibble
            v = __fmul_rn(s, (float)q);
        }
        out[o * in_dim + i] = v;
    }
}

// QTensor::quantize (qtensor.rs:142-213), one workgroup per output row:
// m = max|w| (a max: exact in any order), s = m/qmax, q = round(w/s) (half
// away from zero) clamped to +-qmax; a row of zeros keeps s = 0 and zero
// codes.  A non-finite weight lowers *bad to its flat index (the host
// reports the smallest, as the reference's position() does).
__global__ __launch_bounds__(256) void k_quantize(int32_t fmt, const float *__restrict__ w,
                                                  int64_t in_dim, int64_t row_bytes,
                                                  uint8_t *__restrict__ payload,
                                                  float *__restrict__ scales,
                                                  unsigned long long *__restrict__ bad) {
    __shared__ float red[256];
    const int tid = threadIdx.x;
    const int64_t o = blockIdx.x;
    const float *row = w + o * in_dim;
    float m = 0.0f;
    unsigned long long first = ~0ull;
    for (int64_t i = tid; i < in_dim; i += 256) {
        const float v = row[i];
        if (!isfinite(v) && first == ~0ull) first = (unsigned long long)(o * in_dim + i);
        m = fmaxf(m, fabsf(v));
    }
    if (first != ~0ull) atomicMin(bad, first);
    if (fmt == UT_FMT_F32) return;  // the finiteness check only
    red[tid] = m;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
        __syncthreads();
    }
    m = red[0];
    const float qmax = fmt == UT_FMT_INT4 ? 7.0f : 127.0f;
    const float sc = m > 0.0f ? __fdiv_rn(m, qmax) : 0.0f;
    if (tid == 0) scales[o] = sc;
    auto code = [&](int64_t i) -> int {
        if (!(m > 0.0f)) return 0;
        float v = roundf(__fdiv_rn(row[i], sc));
        v = fminf(fmaxf(v, -qmax), qmax);
        return (int)v;
    };
    uint8_t *prow = payload + o * row_bytes;
    if (fmt == UT_FMT_INT8) {
        for (int64_t i = tid; i < in_dim; i += 256) prow[i] = (uint8_t)(int8_t)code(i);
    } else {
        for (int64_t b = tid; b < row_bytes; b += 256) {
            const int lo = code(2 * b);
            const int hi = 2 * b + 1 < in_dim ? code(2 * b + 1) : 0;
            prow[b] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
        }
    }
}

// QTensor::add_scaled_row (qtensor.rs:516-543): f = factor*scale[row];
// acc[i] += f*q[row,i] (two roundings, no FMA, as the reference).
__global__ void k_add_scaled_row(int32_t fmt, const uint8_t *__restrict__ payload,
                                 const float *__restrict__ scales, int64_t in_dim,
                                 int64_t row_bytes, int64_t row, float factor,
                                 float *__restrict__ acc) {
    const uint8_t *r = payload + row * row_bytes;
    float f = fmt == UT_FMT_F32 ? factor : __fmul_rn(factor, scales[row]);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < in_dim;
         i += (int64_t)gridDim.x * blockDim.x) {
        float q;
        if (fmt == UT_FMT_F32) {
            q = ((const float *)r)[i];
        } else if (fmt == UT_FMT_INT8) {
            q = (float)(int8_t)r[i];
        } else {
            uint8_t b = r[i >> 1];
            int nib = (i & 1) ? (b >> 4) : (b & 0xF);
            q = (float)((nib ^ 8) - 8);
        }
        acc[i] = __fadd_rn(acc[i], __fmul_rn(f, q));
    }
}

}  // namespace ut

using namespace ut;

extern "C" {

int32_t ut_ctx_create(int32_t device, ut_ctx **out) {
    if (!out) return UT_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        (void)hipGetLastError();
        return UT_ERR_HIP;
    }
    if (hipSetDevice(device) != hipSuccess) return UT_ERR_HIP;
    ut_ctx *c = new (std::nothrow) ut_ctx();
    if (!c) return UT_ERR_OOM;
    c->device = device;
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return UT_ERR_HIP;
    }
    c->stream = c->own_stream;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->multiprocessors = prop.multiProcessorCount;
    // set-up that later calls must not repeat (ut_moe_experts_noalloc
    // allocates nothing): the error flag and the fixed working array's address
    int32_t *flag = nullptr;
    int32_t rc = device_error_flag(c, &flag);
    if (rc == UT_OK) rc = moe_noalloc_scratch_init(c);
    if (rc != UT_OK) {
        ctx_release(c);
        return rc;
    }
    *out = c;
    return UT_OK;
}

void ut_ctx_destroy(ut_ctx *ctx) { ctx_release(ctx); }

}  // extern "C"

void ut::ctx_retain(ut_ctx *ctx) { ctx->refs++; }

void ut::ctx_release(ut_ctx *ctx) {
    if (!ctx || --ctx->refs > 0) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    moe_noalloc_release(ctx);
    for (auto &p : ctx->pending) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    if (ctx->scratch.ptr) (void)hipFree(ctx->scratch.ptr);
    if (ctx->dev_err) (void)hipFree(ctx->dev_err);
    if (ctx->splitk) (void)hipFree(ctx->splitk);
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

extern "C" {

const char *ut_last_error(const ut_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int32_t ut_ctx_set_stream(ut_ctx *ctx, void *stream) {
    if (!ctx) return UT_ERR_ARG;
    hipStream_t s = (hipStream_t)stream;  // NULL: the device's null stream
    if (s != ctx->stream) {
        // order the switch: work on the old stream completes first
        UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    ctx->stream = s;
    return UT_OK;
}

void *ut_ctx_stream(ut_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int32_t ut_ctx_synchronize(ut_ctx *ctx) {
    if (!ctx) return UT_ERR_ARG;
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return check_device_error(ctx);
}

int32_t ut_ctx_enable_timing(ut_ctx *ctx, int32_t on) {
    if (!ctx) return UT_ERR_ARG;
    if (!on) timing_collect(ctx, true);
    ctx->timing = on != 0;
    if (on) ctx->stats.clear();
    return UT_OK;
}

int32_t ut_ctx_kernel_time(ut_ctx *ctx, const char *prefix, int64_t *launches, double *total_ms) {
    if (!ctx || !prefix) return UT_ERR_ARG;
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    timing_collect(ctx, true);
    int64_t n = 0;
    double ms = 0.0;
    size_t pl = strlen(prefix);
    for (auto &s : ctx->stats)
        if (s.name.compare(0, pl, prefix) == 0) { n += s.launches; ms += s.total_ms; }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    return UT_OK;
}

int32_t ut_qtensor_upload(ut_ctx *ctx, int32_t fmt, const void *payload, int64_t payload_len,
                          const float *scales, int64_t scales_len, int64_t out_dim,
                          int64_t in_dim, ut_qtensor **out) {
    if (!ctx || !out || !payload || out_dim <= 0 || in_dim <= 0) {
        set_error(ctx, "ut_qtensor_upload: bad argument");
        return UT_ERR_ARG;
    }
    *out = nullptr;
    if (fmt == UT_FMT_INFER) {
        // read_qtensor (reader.rs:421-430): int8 wins when both match.
        if (payload_len == payload_bytes(UT_FMT_INT8, out_dim, in_dim)) fmt = UT_FMT_INT8;
        else if (payload_len == payload_bytes(UT_FMT_INT4, out_dim, in_dim)) fmt = UT_FMT_INT4;
        else {
            set_error(ctx, "payload of %lld bytes matches neither int8 nor int4 for [%lld, %lld]",
                      (long long)payload_len, (long long)out_dim, (long long)in_dim);
            return UT_ERR_FORMAT;
        }
    }
    if (fmt != UT_FMT_F32 && fmt != UT_FMT_INT8 && fmt != UT_FMT_INT4) {
        set_error(ctx, "unknown format %d", fmt);
        return UT_ERR_ARG;
    }
    // QTensor::from_quantized size checks (qtensor.rs:92-117)
    if (payload_len != payload_bytes(fmt, out_dim, in_dim)) {
        set_error(ctx, "payload size %lld does not match %lldx%lld", (long long)payload_len,
                  (long long)out_dim, (long long)in_dim);
        return UT_ERR_FORMAT;
    }
    if (fmt != UT_FMT_F32 && (!scales || scales_len != out_dim)) {
        set_error(ctx, "scales len %lld != out_dim %lld", (long long)scales_len, (long long)out_dim);
        return UT_ERR_FORMAT;
    }
    UT_CHECK_HIP(ctx, hipSetDevice(ctx->device));
    ut_qtensor *q = new (std::nothrow) ut_qtensor();
    if (!q) return UT_ERR_OOM;
    q->fmt = fmt;
    q->out_dim = out_dim;
    q->in_dim = in_dim;
    q->row_bytes = payload_bytes(fmt, 1, in_dim);
    q->device = ctx->device;
    if (hipMalloc(&q->payload, (size_t)payload_len) != hipSuccess ||
        (fmt != UT_FMT_F32 && hipMalloc((void **)&q->scales, (size_t)out_dim * 4) != hipSuccess)) {
        (void)hipGetLastError();
        ut_qtensor_free(q);
        set_error(ctx, "device allocation for a %lldx%lld tensor failed", (long long)out_dim,
                  (long long)in_dim);
        return UT_ERR_OOM;
    }
    // hipMemcpyDefault: the source may be host or device memory
    hipError_t e = hipMemcpy(q->payload, payload, (size_t)payload_len, hipMemcpyDefault);
    if (e == hipSuccess && q->scales)
        e = hipMemcpy(q->scales, scales, (size_t)out_dim * 4, hipMemcpyDefault);
    if (e != hipSuccess) {
        ut_qtensor_free(q);
        set_error(ctx, "upload failed: %s", hipGetErrorString(e));
        return UT_ERR_HIP;
    }
    *out = q;
    return UT_OK;
}

void ut_qtensor_free(ut_qtensor *qt) {
    if (!qt) return;
    if (qt->owns) {
        (void)hipSetDevice(qt->device);
        if (qt->payload) (void)hipFree(qt->payload);
        if (qt->scales) (void)hipFree(qt->scales);
    }
    delete qt;
}

int32_t ut_qtensor_format(const ut_qtensor *qt) { return qt ? qt->fmt : UT_ERR_ARG; }
int64_t ut_qtensor_out_dim(const ut_qtensor *qt) { return qt ? qt->out_dim : UT_ERR_ARG; }
int64_t ut_qtensor_in_dim(const ut_qtensor *qt) { return qt ? qt->in_dim : UT_ERR_ARG; }
int64_t ut_qtensor_nbytes(const ut_qtensor *qt) {
    // QTensor::nbytes (qtensor.rs:240-248): payload plus scales
    if (!qt) return UT_ERR_ARG;
    return payload_bytes(qt->fmt, qt->out_dim, qt->in_dim) +
           (qt->fmt == UT_FMT_F32 ? 0 : qt->out_dim * 4);
}

int32_t ut_qtensor_dequantize(ut_ctx *ctx, const ut_qtensor *qt, float *out_dev) {
    if (!ctx || !qt || !out_dev) return UT_ERR_ARG;
    // grid.y is bounded by 65535: launch in row blocks
    for (int64_t r0 = 0; r0 < qt->out_dim; r0 += 65535) {
        int64_t rows = qt->out_dim - r0 < 65535 ? qt->out_dim - r0 : 65535;
        dim3 grid((unsigned)((qt->in_dim + 255) / 256 < 64 ? (qt->in_dim + 255) / 256 : 64),
                  (unsigned)rows);
        int tok = timing_begin(ctx, "dequantize");
        hipLaunchKernelGGL(k_dequantize, grid, dim3(256), 0, ctx->stream, qt->fmt,
                           (const uint8_t *)qt->payload + r0 * qt->row_bytes,
                           qt->scales ? qt->scales + r0 : nullptr, rows, qt->in_dim,
                           qt->row_bytes, out_dev + r0 * qt->in_dim);
        timing_end(ctx, tok);
        UT_TRY(launch_check(ctx, "k_dequantize"));
    }
    return UT_OK;
}

int32_t ut_qtensor_quantize(ut_ctx *ctx, int32_t fmt, const float *w_dev, int64_t out_dim,
                            int64_t in_dim, ut_qtensor **out) {
    if (!ctx || !w_dev || !out || out_dim <= 0 || in_dim <= 0) return UT_ERR_ARG;
    *out = nullptr;
    if (fmt != UT_FMT_F32 && fmt != UT_FMT_INT8 && fmt != UT_FMT_INT4) {
        set_error(ctx, "quantize: unknown format %d", fmt);
        return UT_ERR_ARG;
    }
    ScratchPlan plan;
    plan.add(8);
    std::vector<void *> ptrs;
    UT_TRY(scratch_acquire(ctx, plan, ptrs));
    unsigned long long *bad = (unsigned long long *)ptrs[0];
    UT_CHECK_HIP(ctx, hipMemsetAsync(bad, 0xFF, 8, ctx->stream));
    ut_qtensor *q = new (std::nothrow) ut_qtensor();
    if (!q) return UT_ERR_OOM;
    q->fmt = fmt;
    q->out_dim = out_dim;
    q->in_dim = in_dim;
    q->row_bytes = payload_bytes(fmt, 1, in_dim);
    q->device = ctx->device;
    const int64_t nb = payload_bytes(fmt, out_dim, in_dim);
    if (hipMalloc(&q->payload, (size_t)nb) != hipSuccess ||
        (fmt != UT_FMT_F32 && hipMalloc((void **)&q->scales, (size_t)out_dim * 4) != hipSuccess)) {
        (void)hipGetLastError();
        ut_qtensor_free(q);
        set_error(ctx, "device allocation for a %lldx%lld tensor failed", (long long)out_dim,
                  (long long)in_dim);
        return UT_ERR_OOM;
    }
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)out_dim), dim3(256), 0, ctx->stream, fmt, w_dev,
                       in_dim, q->row_bytes, (uint8_t *)q->payload, q->scales, bad);
    int32_t rc = launch_check(ctx, "k_quantize");
    // f32: the data as given (QuantFormat::F32 keeps w)
    if (rc == UT_OK && fmt == UT_FMT_F32 &&
        hipMemcpyAsync(q->payload, w_dev, (size_t)nb, hipMemcpyDeviceToDevice, ctx->stream) !=
            hipSuccess)
        rc = UT_ERR_HIP;
    unsigned long long first = ~0ull;
    if (rc == UT_OK &&
        hipMemcpyAsync(&first, bad, 8, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
        rc = UT_ERR_HIP;
    if (rc == UT_OK && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = UT_ERR_HIP;
    if (rc == UT_OK && first != ~0ull) {
        // the reference's Err (qtensor.rs:149-155)
        set_error(ctx, "non-finite weight at flat index %llu (row %lld, col %lld)", first,
                  (long long)(first / (unsigned long long)in_dim),
                  (long long)(first % (unsigned long long)in_dim));
        rc = UT_ERR_FORMAT;
    }
    if (rc != UT_OK) {
        ut_qtensor_free(q);
        return rc;
    }
    *out = q;
    return UT_OK;
}

int32_t ut_qtensor_download(ut_ctx *ctx, const ut_qtensor *qt, void *payload_host,
                            int64_t payload_len, float *scales_host) {
    if (!ctx || !qt || !payload_host) return UT_ERR_ARG;
    if (payload_len != payload_bytes(qt->fmt, qt->out_dim, qt->in_dim) ||
        (qt->fmt != UT_FMT_F32 && !scales_host)) {
        set_error(ctx, "download: payload of %lld bytes for a %lldx%lld tensor of format %d",
                  (long long)payload_len, (long long)qt->out_dim, (long long)qt->in_dim, qt->fmt);
        return UT_ERR_SHAPE;
    }
    UT_CHECK_HIP(ctx, hipMemcpyAsync(payload_host, qt->payload, (size_t)payload_len,
                                     hipMemcpyDeviceToHost, ctx->stream));
    if (qt->fmt != UT_FMT_F32)
        UT_CHECK_HIP(ctx, hipMemcpyAsync(scales_host, qt->scales, (size_t)qt->out_dim * 4,
                                         hipMemcpyDeviceToHost, ctx->stream));
    UT_CHECK_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return UT_OK;
}

int32_t ut_qtensor_add_scaled_row(ut_ctx *ctx, const ut_qtensor *qt, int64_t row, float factor,
                                  float *acc_dev) {
    if (!ctx || !qt || !acc_dev) return UT_ERR_ARG;
    if (row < 0 || row >= qt->out_dim) {
        set_error(ctx, "row %lld out of range %lld", (long long)row, (long long)qt->out_dim);
        return UT_ERR_SHAPE;
    }
    unsigned blocks = (unsigned)((qt->in_dim + 255) / 256);
    if (blocks > 1024) blocks = 1024;
    (void)hipGetLastError();
    hipLaunchKernelGGL(k_add_scaled_row, dim3(blocks), dim3(256), 0, ctx->stream, qt->fmt,
                       (const uint8_t *)qt->payload, qt->scales, qt->in_dim, qt->row_bytes, row,
                       factor, acc_dev);
    return launch_check(ctx, "k_add_scaled_row");
}

}  // extern "C"
