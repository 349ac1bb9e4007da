// Elementwise, reduction, cast and optimizer kernels for gfx950.
//
// Streaming kernels move 16 bytes per lane per access (float4 / 8 x u16) with
// grid-stride loops sized to fill 256 CUs; broadcast and reduction kernels
// take a small by-value descriptor so no index tables live in memory.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"
#include "pgmath.h"

namespace {

constexpr int kBlock = 256;

inline int grid_for(size_t work_items, int per_thread = 1)
{
    size_t threads = (work_items + per_thread - 1) / per_thread;
    size_t blocks = (threads + kBlock - 1) / kBlock;
    if (blocks < 1)
        blocks = 1;
    if (blocks > 256 * 32)
        blocks = 256 * 32;
    return (int)blocks;
}

inline int status() { return (int)hipGetLastError(); }

// ---------------------------------------------------------------- math

__device__ __forceinline__ float unary_f(int op, float x, float p0, float p1)
{
    switch (op) {
    case PGK_NEG: return -x;
    case PGK_EXP: return pgm_exp(x);
    case PGK_LOG: return logf(x);
    case PGK_SQRT: return sqrtf(x);
    case PGK_SIN: return sinf(x);
    case PGK_COS: return cosf(x);
    case PGK_RELU: return x > 0.0f ? x : 0.0f;
    case PGK_SIGMOID: return pgm_sigmoid(x);
    case PGK_TANH: return tanhf(x);
    case PGK_GELU: return pgm_gelu(x);
    case PGK_ERF: return erff(x);
    case PGK_ABS: return fabsf(x);
    case PGK_LEAKY: return x > 0.0f ? x : p0 * x;
    case PGK_CLAMP: return x < p0 ? p0 : (x > p1 ? p1 : x);
    default: return 0.0f;
    }
}

// local derivative d op(x) / dx, in the forms of the reference's grad_*
__device__ __forceinline__ float unary_grad_f(int op, float x, float p0, float p1)
{
    switch (op) {
    case PGK_NEG: return -1.0f;
    case PGK_EXP: return pgm_exp(x);
    case PGK_LOG: return 1.0f / x;
    case PGK_SQRT: return 0.5f / sqrtf(x);
    case PGK_SIN: return cosf(x);
    case PGK_COS: return -sinf(x);
    case PGK_RELU: return x > 0.0f ? 1.0f : 0.0f;
    case PGK_SIGMOID: {
        float s = pgm_sigmoid(x);
        return s * (1.0f - s);
    }
    case PGK_TANH: {
        float t = tanhf(x);
        return 1.0f - t * t;
    }
    case PGK_GELU: return pgm_gelu_grad(x);
    case PGK_ERF: return 1.12837916709551f * pgm_exp(-x * x);
    case PGK_ABS: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    case PGK_LEAKY: return x > 0.0f ? 1.0f : p0;
    case PGK_CLAMP: return (x >= p0 && x <= p1) ? 1.0f : 0.0f;
    default: return 0.0f;
    }
}

__device__ __forceinline__ float binary_f(int op, float a, float b)
{
    switch (op) {
    case PGK_ADD: return a + b;
    case PGK_SUB: return a - b;
    case PGK_MUL: return a * b;
    default: return a / b;
    }
}

// ---------------------------------------------------------------- casts
// f32 -> bf16: round to nearest even on the raw bits; a NaN becomes the
// positive quiet NaN 0x7FC0 | bit 16 (the reference's convert.h rule).
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu) != 0)
        return (uint16_t)(0x7FC0u | ((x >> 16) & 1u));
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// f32 -> f16, IEEE round to nearest even including subnormals; NaN keeps
// its top payload bits and is quieted.
__device__ __forceinline__ uint16_t f32_to_f16(float f)
{
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 255) {
        if (man == 0)
            return (uint16_t)(sign | 0x7C00u);
        uint32_t q = sign | 0x7C00u | (man >> 13);
        if ((q & 0x3FFu) == 0)
            q |= 1u;
        return (uint16_t)(q | 0x200u);
    }
    int e = (int)ex - 112;
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t sh = (uint32_t)(1 - e) + 13u;
        uint32_t keep = man >> sh;
        uint32_t rem = man & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (keep & 1u)))
            keep++;
        return (uint16_t)(sign | keep);
    }
    uint32_t r = man + 0xFFFu + ((man >> 13) & 1u);
    if (r & 0x800000u) {
        r = 0;
        e++;
    }
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (r >> 13));
}

// f16 -> f32 on the raw bits (exact; NaN payloads kept as they are)
__device__ __forceinline__ float f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (ex == 0) {
        if (man == 0)
            return __uint_as_float(sign);
        int e = 1;
        while ((man & 0x400u) == 0) {
            man <<= 1;
            e--;
        }
        man &= 0x3FFu;
        return __uint_as_float(sign | ((uint32_t)(e + 112) << 23) | (man << 13));
    }
    if (ex == 31)
        return __uint_as_float(sign | 0x7F800000u | (man << 13));
    return __uint_as_float(sign | ((ex + 112u) << 23) | (man << 13));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t to16(int dtype, float f)
{
    return dtype == 1 ? f32_to_f16(f) : f32_to_bf16(f);
}

__device__ __forceinline__ float from16(int dtype, uint16_t h)
{
    return dtype == 1 ? f16_to_f32(h) : bf16_to_f32(h);
}

// ---------------------------------------------------------------- kernels

__global__ void __launch_bounds__(kBlock) k_fill_f32(float *__restrict__ dst, size_t n, float v)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t n4 = n / 4;
    float4 v4 = make_float4(v, v, v, v);
    for (size_t j = i; j < n4; j += stride)
        reinterpret_cast<float4 *>(dst)[j] = v4;
    for (size_t j = n4 * 4 + i; j < n; j += stride)
        dst[j] = v;
}

__global__ void __launch_bounds__(kBlock) k_fill_u16(uint16_t *__restrict__ dst, size_t n, uint16_t v)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride)
        dst[j] = v;
}

__global__ void __launch_bounds__(kBlock) k_unary(int op, const float *__restrict__ x,
                                                  float *__restrict__ y, size_t n, float p0, float p1)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride)
        y[j] = unary_f(op, x[j], p0, p1);
}

__global__ void __launch_bounds__(kBlock) k_unary_bwd(int op, const float *__restrict__ g,
                                                      const float *__restrict__ x, float *dx, size_t n,
                                                      float p0, float p1, float scale, int beta)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride) {
        float xv = x ? x[j] : 0.0f;
        float v = scale * g[j] * unary_grad_f(op, xv, p0, p1);
        dx[j] = beta ? dx[j] + v : v;
    }
}

__device__ __forceinline__ void unravel2(const pgk_bcast &bc, size_t idx, int64_t &oa, int64_t &ob)
{
    oa = 0;
    ob = 0;
    for (int d = bc.ndim - 1; d >= 0; --d) {
        int64_t s = bc.shape[d];
        int64_t c = (int64_t)(idx % (size_t)s);
        idx /= (size_t)s;
        oa += c * bc.sa[d];
        ob += c * bc.sb[d];
    }
}

__global__ void __launch_bounds__(kBlock) k_binary(int op, const float *__restrict__ a,
                                                   const float *__restrict__ b, float *__restrict__ y,
                                                   size_t n, pgk_bcast bc)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride) {
        int64_t oa, ob;
        unravel2(bc, j, oa, ob);
        y[j] = binary_f(op, a[oa], b[ob]);
    }
}

// kept dims index the destination; reduced dims are summed in row-major
// order for every destination element (fixed order: deterministic).
struct reduce_desc {
    int nk, nr;
    int64_t kshape[PGK_MAX_NDIM], kstride_src[PGK_MAX_NDIM];
    int64_t rshape[PGK_MAX_NDIM], rstride_src[PGK_MAX_NDIM];
    int64_t rcount;
};

__global__ void __launch_bounds__(kBlock) k_reduce_into(float *dst, size_t dst_n,
                                                        const float *__restrict__ src, reduce_desc d,
                                                        float scale, int beta)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < dst_n; j += stride) {
        int64_t base = 0;
        size_t t = j;
        for (int q = d.nk - 1; q >= 0; --q) {
            int64_t c = (int64_t)(t % (size_t)d.kshape[q]);
            t /= (size_t)d.kshape[q];
            base += c * d.kstride_src[q];
        }
        float acc = 0.0f;
        for (int64_t r = 0; r < d.rcount; ++r) {
            int64_t off = 0, rr = r;
            for (int q = d.nr - 1; q >= 0; --q) {
                int64_t c = rr % d.rshape[q];
                rr /= d.rshape[q];
                off += c * d.rstride_src[q];
            }
            acc += src[base + off];
        }
        float v = scale * acc;
        dst[j] = beta ? dst[j] + v : v;
    }
}

__global__ void __launch_bounds__(kBlock) k_expand_into(float *dst, const float *__restrict__ src,
                                                        size_t n, pgk_bcast bc, float scale, int beta)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride) {
        int64_t oa, ob;
        unravel2(bc, j, oa, ob);
        float v = scale * src[oa];
        dst[j] = beta ? dst[j] + v : v;
    }
}

// y[o, i] = scale * sum_l x[o, l, i]; one thread per output, l ascending.
__global__ void __launch_bounds__(kBlock) k_sum_axis(const float *__restrict__ x, float *__restrict__ y,
                                                     size_t outer, size_t len, size_t inner, float scale)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t total = outer * inner;
    for (size_t j = i; j < total; j += stride) {
        size_t o = j / inner, in = j % inner;
        const float *p = x + o * len * inner + in;
        float acc = 0.0f;
        for (size_t l = 0; l < len; ++l)
            acc += p[l * inner];
        y[j] = acc * scale;
    }
}

__global__ void __launch_bounds__(kBlock) k_cast_to16(int dtype, const float *__restrict__ src,
                                                      uint16_t *__restrict__ dst, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t n4 = n / 4;
    for (size_t j = i; j < n4; j += stride) {
        float4 v = reinterpret_cast<const float4 *>(src)[j];
        ushort4 o;
        o.x = to16(dtype, v.x);
        o.y = to16(dtype, v.y);
        o.z = to16(dtype, v.z);
        o.w = to16(dtype, v.w);
        reinterpret_cast<ushort4 *>(dst)[j] = o;
    }
    for (size_t j = n4 * 4 + i; j < n; j += stride)
        dst[j] = to16(dtype, src[j]);
}

__global__ void __launch_bounds__(kBlock) k_cast_from16(int dtype, const uint16_t *__restrict__ src,
                                                        float *__restrict__ dst, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride)
        dst[j] = from16(dtype, src[j]);
}

// dst[r * ldd + c] = cvt(src[r * lds + c]) for r < rows, c < cols; zeros
// for the padding rows [rows, rows_pad) and columns [cols, ldd)
template <typename TS>
__global__ void __launch_bounds__(kBlock) k_copy16(int dtype, const TS *__restrict__ src, size_t rows, size_t cols,
                                                   size_t lds, uint16_t *__restrict__ dst, size_t ldd,
                                                   size_t rows_pad, size_t sstride, size_t dstride)
{
    const TS *s = src + (size_t)blockIdx.z * sstride;
    uint16_t *d = dst + (size_t)blockIdx.z * dstride;
    size_t total = rows_pad * ldd;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < total; j += stride) {
        size_t r = j / ldd, c = j % ldd;
        uint16_t v = 0;
        if (r < rows && c < cols) {
            if constexpr (sizeof(TS) == 4)
                v = to16(dtype, (float)s[r * lds + c]);
            else
                v = (uint16_t)s[r * lds + c];
        }
        d[j] = v;
    }
}

// ---------------------------------------------------------------- SGD
// One launch updates every parameter: blockIdx.y selects the segment.
// g' = g + wd*p; buf = mu*buf + (1-damp)*g'; u = nesterov ? g' + mu*buf : buf;
// p -= lr*u  (the reference's sgd.c:147-160 update, per element).
#define PGK_SGD_MAX_SEG 32
struct sgd_table {
    pgk_sgd_seg seg[PGK_SGD_MAX_SEG];
};

__device__ __forceinline__ void sgd_elem(float &p, float g, float &b, bool has_buf, float lr, float mu,
                                         float damp, float wd, int nesterov)
{
    // The reference's x86 build (-mavx2, no -mfma) rounds every product and
    // sum separately; keeping them unfused here gives the same bits.
#pragma clang fp contract(off)
    float gj = g;
    if (wd != 0.0f)
        gj = gj + wd * p;
    float u = gj;
    if (has_buf) {
        b = b * mu + gj * (1.0f - damp);
        u = nesterov ? gj + mu * b : b;
    }
    p = p - lr * u;
}

__global__ void __launch_bounds__(kBlock) k_sgd(sgd_table tab, float lr, float mu, float damp, float wd,
                                                int nesterov)
{
    const pgk_sgd_seg sg = tab.seg[blockIdx.y];
    size_t n = sg.n;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    bool has_buf = sg.buf != nullptr;
    bool aligned = ((((uintptr_t)sg.p) | ((uintptr_t)sg.g) | ((uintptr_t)sg.buf)) & 15) == 0 &&
                   (((uintptr_t)sg.shadow) & 7) == 0;
    size_t n4 = aligned ? n / 4 : 0;
    for (size_t j = i; j < n4; j += stride) {
        float4 p = reinterpret_cast<float4 *>(sg.p)[j];
        float4 g = reinterpret_cast<const float4 *>(sg.g)[j];
        float4 b = has_buf ? reinterpret_cast<float4 *>(sg.buf)[j] : make_float4(0, 0, 0, 0);
        sgd_elem(p.x, g.x, b.x, has_buf, lr, mu, damp, wd, nesterov);
        sgd_elem(p.y, g.y, b.y, has_buf, lr, mu, damp, wd, nesterov);
        sgd_elem(p.z, g.z, b.z, has_buf, lr, mu, damp, wd, nesterov);
        sgd_elem(p.w, g.w, b.w, has_buf, lr, mu, damp, wd, nesterov);
        reinterpret_cast<float4 *>(sg.p)[j] = p;
        if (has_buf)
            reinterpret_cast<float4 *>(sg.buf)[j] = b;
        if (sg.shadow) {
            ushort4 o;
            o.x = to16(sg.shadow_dtype, p.x);
            o.y = to16(sg.shadow_dtype, p.y);
            o.z = to16(sg.shadow_dtype, p.z);
            o.w = to16(sg.shadow_dtype, p.w);
            reinterpret_cast<ushort4 *>(sg.shadow)[j] = o;
        }
    }
    for (size_t j = n4 * 4 + i; j < n; j += stride) {
        float p = sg.p[j], b = has_buf ? sg.buf[j] : 0.0f;
        sgd_elem(p, sg.g[j], b, has_buf, lr, mu, damp, wd, nesterov);
        sg.p[j] = p;
        if (has_buf)
            sg.buf[j] = b;
        if (sg.shadow)
            sg.shadow[j] = to16(sg.shadow_dtype, p);
    }
}

} // namespace

// ---------------------------------------------------------------- launchers

extern "C" int pgk_fill_f32(float *dst, size_t n, float v, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_fill_f32, dim3(grid_for(n, 16)), dim3(kBlock), 0, (hipStream_t)s, dst, n, v);
    return status();
}

extern "C" int pgk_fill_u16(uint16_t *dst, size_t n, uint16_t v, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_fill_u16, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, dst, n, v);
    return status();
}

extern "C" int pgk_unary_f32(int op, const float *x, float *y, size_t n, float p0, float p1, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_unary, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, op, x, y, n, p0, p1);
    return status();
}

extern "C" int pgk_unary_bwd_f32(int op, const float *g, const float *x, float *dx, size_t n, float p0,
                                 float p1, float scale, int beta, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_unary_bwd, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, op, g, x, dx, n,
                       p0, p1, scale, beta);
    return status();
}

extern "C" int pgk_binary_f32(int op, const float *a, const float *b, float *y, const pgk_bcast *bc,
                              pgk_stream s)
{
    size_t n = 1;
    for (int d = 0; d < bc->ndim; ++d)
        n *= (size_t)bc->shape[d];
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_binary, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, op, a, b, y, n, *bc);
    return status();
}

extern "C" int pgk_reduce_into_f32(float *dst, size_t dst_numel, const float *src, const pgk_bcast *bc,
                                   float scale, int beta, pgk_stream s)
{
    reduce_desc d = {};
    // source strides of a contiguous bc->shape
    int64_t sstr[PGK_MAX_NDIM];
    int64_t acc = 1;
    for (int q = bc->ndim - 1; q >= 0; --q) {
        sstr[q] = acc;
        acc *= bc->shape[q];
    }
    d.rcount = 1;
    for (int q = 0; q < bc->ndim; ++q) {
        if (bc->sa[q] == 0 && bc->shape[q] > 1) {
            d.rshape[d.nr] = bc->shape[q];
            d.rstride_src[d.nr] = sstr[q];
            d.rcount *= bc->shape[q];
            d.nr++;
        } else {
            d.kshape[d.nk] = bc->shape[q];
            d.kstride_src[d.nk] = sstr[q];
            d.nk++;
        }
    }
    if (!dst_numel)
        return 0;
    hipLaunchKernelGGL(k_reduce_into, dim3(grid_for(dst_numel)), dim3(kBlock), 0, (hipStream_t)s, dst,
                       dst_numel, src, d, scale, beta);
    return status();
}

extern "C" int pgk_expand_into_f32(float *dst, const float *src, const pgk_bcast *bc, float scale, int beta,
                                   pgk_stream s)
{
    size_t n = 1;
    for (int d = 0; d < bc->ndim; ++d)
        n *= (size_t)bc->shape[d];
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_expand_into, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, dst, src, n, *bc,
                       scale, beta);
    return status();
}

extern "C" int pgk_sum_axis_f32(const float *x, float *y, size_t outer, size_t len, size_t inner, float scale,
                                pgk_stream s)
{
    size_t n = outer * inner;
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_sum_axis, dim3(grid_for(n)), dim3(kBlock), 0, (hipStream_t)s, x, y, outer, len, inner,
                       scale);
    return status();
}

extern "C" int pgk_cast_to16(int dtype, const float *src, uint16_t *dst, size_t n, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_cast_to16, dim3(grid_for(n, 16)), dim3(kBlock), 0, (hipStream_t)s, dtype, src, dst, n);
    return status();
}

extern "C" int pgk_cast_from16(int dtype, const uint16_t *src, float *dst, size_t n, pgk_stream s)
{
    if (!n)
        return 0;
    hipLaunchKernelGGL(k_cast_from16, dim3(grid_for(n, 4)), dim3(kBlock), 0, (hipStream_t)s, dtype, src, dst,
                       n);
    return status();
}

extern "C" int pgk_copy_to16(int dtype, int src_dtype, const void *src, size_t rows, size_t cols, size_t lds,
                             uint16_t *dst, size_t ldd, size_t rows_pad, size_t batch, size_t sstride,
                             size_t dstride, pgk_stream s)
{
    if (!rows_pad || !ldd || !batch)
        return 0;
    if (batch > 65535 || rows > rows_pad || cols > ldd)
        return (int)hipErrorInvalidValue;
    dim3 grid((unsigned)grid_for(rows_pad * ldd, 4), 1, (unsigned)batch);
    if (src_dtype == 0)
        hipLaunchKernelGGL(k_copy16<float>, grid, dim3(kBlock), 0, (hipStream_t)s, dtype, (const float *)src,
                           rows, cols, lds, dst, ldd, rows_pad, sstride, dstride);
    else
        hipLaunchKernelGGL(k_copy16<uint16_t>, grid, dim3(kBlock), 0, (hipStream_t)s, dtype,
                           (const uint16_t *)src, rows, cols, lds, dst, ldd, rows_pad, sstride, dstride);
    return status();
}

extern "C" int pgk_sgd_multi(const pgk_sgd_seg *segs, int nseg, float lr, float momentum, float dampening,
                             float weight_decay, int nesterov, pgk_stream s)
{
    for (int base = 0; base < nseg; base += PGK_SGD_MAX_SEG) {
        int cnt = nseg - base < PGK_SGD_MAX_SEG ? nseg - base : PGK_SGD_MAX_SEG;
        sgd_table tab = {};
        size_t maxn = 0;
        for (int q = 0; q < cnt; ++q) {
            tab.seg[q] = segs[base + q];
            if (segs[base + q].n > maxn)
                maxn = segs[base + q].n;
        }
        if (!maxn)
            continue;
        int gx = grid_for(maxn, 16);
        hipLaunchKernelGGL(k_sgd, dim3(gx, cnt), dim3(kBlock), 0, (hipStream_t)s, tab, lr, momentum, dampening,
                           weight_decay, nesterov);
        int st = status();
        if (st)
            return st;
    }
    return 0;
}
