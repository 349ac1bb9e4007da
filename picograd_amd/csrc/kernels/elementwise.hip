// Elementwise, reduction, cast and optimizer kernels for gfx950.
//
// Streaming kernels move 16 bytes per lane per access (float4 / 8 x u16) with
// grid-stride loops sized to fill 256 CUs; broadcast and reduction kernels
// take a small by-value descriptor so no index tables live in memory.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"
#include "convert16.h"
#include "segtab.h"
#include "pgmath.h"

namespace {

constexpr int kBlock = 256;
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// 16-byte streaming (non-temporal) accesses, for data a kernel reads or
// writes once
__device__ __forceinline__ float4 ntl4(const float *q)
{
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(q));
    return make_float4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void nts4(const float4 &v, float *q)
{
    const f32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<f32x4 *>(q));
}

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
    const bool vec = ((((uintptr_t)x) | ((uintptr_t)y)) & 15) == 0;
    size_t n4 = vec ? n / 4 : 0;
    for (size_t j = i; j < n4; j += stride) {
        float4 v = reinterpret_cast<const float4 *>(x)[j];
        v.x = unary_f(op, v.x, p0, p1);
        v.y = unary_f(op, v.y, p0, p1);
        v.z = unary_f(op, v.z, p0, p1);
        v.w = unary_f(op, v.w, p0, p1);
        reinterpret_cast<float4 *>(y)[j] = v;
    }
    for (size_t j = n4 * 4 + i; j < n; j += stride)
        y[j] = unary_f(op, x[j], p0, p1);
}

__device__ __forceinline__ float unary_bwd_elem(int op, float g, float x, float d, float p0, float p1,
                                                float scale, int beta)
{
    float v = scale * g * unary_grad_f(op, x, p0, p1);
    return beta ? d + v : v;
}

__global__ void __launch_bounds__(kBlock) k_unary_bwd(int op, const float *__restrict__ g,
                                                      const float *__restrict__ x, float *dx, size_t n,
                                                      float p0, float p1, float scale, int beta)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool vec = x && ((((uintptr_t)g) | ((uintptr_t)x) | ((uintptr_t)dx)) & 15) == 0;
    size_t n4 = vec ? n / 4 : 0;
    for (size_t j = i; j < n4; j += stride) {
        const float4 gv = reinterpret_cast<const float4 *>(g)[j];
        const float4 xv = reinterpret_cast<const float4 *>(x)[j];
        float4 d = beta ? reinterpret_cast<const float4 *>(dx)[j] : make_float4(0, 0, 0, 0);
        d.x = unary_bwd_elem(op, gv.x, xv.x, d.x, p0, p1, scale, beta);
        d.y = unary_bwd_elem(op, gv.y, xv.y, d.y, p0, p1, scale, beta);
        d.z = unary_bwd_elem(op, gv.z, xv.z, d.z, p0, p1, scale, beta);
        d.w = unary_bwd_elem(op, gv.w, xv.w, d.w, p0, p1, scale, beta);
        reinterpret_cast<float4 *>(dx)[j] = d;
    }
    for (size_t j = n4 * 4 + i; j < n; j += stride)
        dx[j] = unary_bwd_elem(op, g[j], x ? x[j] : 0.0f, beta ? dx[j] : 0.0f, p0, p1, scale, beta);
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

// Broadcast binary op, 4 outputs per lane along the last dim: the output is
// rows x C (C = last dim, a multiple of 4); each operand's last-dim stride
// is 1 (float4 load) or 0 (one value splat); its row offset comes from the
// leading dims.  The host checks that every row offset of a stride-1
// operand is a multiple of 4 and the bases are 16-byte aligned.
__global__ void __launch_bounds__(kBlock) k_binary_rows4(int op, const float *__restrict__ a,
                                                         const float *__restrict__ b, float *__restrict__ y,
                                                         size_t rows, size_t c4, pgk_bcast bc)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    const int nl = bc.ndim - 1;
    const bool avec = bc.sa[nl] != 0, bvec = bc.sb[nl] != 0;
    const size_t n4 = rows * c4;
    for (size_t j = i; j < n4; j += stride) {
        size_t r = j / c4, c = (j - r * c4) * 4;
        int64_t oa = 0, ob = 0;
        for (int d = nl - 1; d >= 0; --d) {
            int64_t sd = bc.shape[d];
            int64_t q = (int64_t)(r % (size_t)sd);
            r /= (size_t)sd;
            oa += q * bc.sa[d];
            ob += q * bc.sb[d];
        }
        float4 va, vb;
        if (avec) {
            va = *reinterpret_cast<const float4 *>(a + oa + c);
        } else {
            const float s0 = a[oa];
            va = make_float4(s0, s0, s0, s0);
        }
        if (bvec) {
            vb = *reinterpret_cast<const float4 *>(b + ob + c);
        } else {
            const float s1 = b[ob];
            vb = make_float4(s1, s1, s1, s1);
        }
        float4 o;
        o.x = binary_f(op, va.x, vb.x);
        o.y = binary_f(op, va.y, vb.y);
        o.z = binary_f(op, va.z, vb.z);
        o.w = binary_f(op, va.w, vb.w);
        reinterpret_cast<float4 *>(y)[j] = o;
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

// y[o, i] = scale * sum_l x[o, l, i] in two deterministic stages: the
// reduced axis is cut into `slices` runs of slice_len; stage 1 writes one
// partial per (slice, o, i) (consecutive lanes take consecutive i, so rows
// are read coalesced), stage 2 adds the partials of each output in slice
// order.  slices == 1 writes y directly.
__global__ void __launch_bounds__(kBlock) k_sum_axis_part(const float *__restrict__ x, float *__restrict__ part,
                                                          size_t outer, size_t len, size_t inner, size_t slices,
                                                          size_t slice_len, float scale)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t n = outer * inner, total = slices * n;
    for (size_t j = i; j < total; j += stride) {
        const size_t sl = j / n, oi = j - sl * n;
        const size_t o = oi / inner, in = oi - o * inner;
        const size_t l0 = sl * slice_len, l1 = l0 + slice_len < len ? l0 + slice_len : len;
        const float *p = x + (o * len) * inner + in;
        float acc = 0.0f;
#pragma unroll 8
        for (size_t l = l0; l < l1; ++l)
            acc += p[l * inner];
        part[j] = slices == 1 ? acc * scale : acc;
    }
}

__global__ void __launch_bounds__(kBlock) k_sum_axis_fin(const float *__restrict__ part, float *__restrict__ y,
                                                         size_t n, size_t slices, float scale)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t j = i; j < n; j += stride) {
        float acc = 0.0f;
#pragma unroll 8
        for (size_t sl = 0; sl < slices; ++sl)
            acc += part[sl * n + j];
        y[j] = acc * scale;
    }
}

// Both reductions of a [rows, cols] reduce_all in one block, when each is a
// single run (sum_axis_plan gives one slice for both): lane j adds column j
// over the rows in row order (y1[j], as k_sum_axis_part with one slice),
// then lane 0 adds y1 in order, times scale (y2).  The same additions in the
// same order as the two k_sum_axis_part launches it replaces.
constexpr int kSumAll2Max = 256;
__global__ void __launch_bounds__(kSumAll2Max) k_sum_all2(const float *__restrict__ x, float *__restrict__ y1,
                                                          float *__restrict__ y2, int rows, int cols, float scale)
{
    // the whole input goes through LDS first (every load of a lane issued
    // at once; rows * cols <= 127 * 127 floats), so the serial column walks
    // wait on LDS, not on memory
    constexpr int kTile = 127 * 127, kPer = (kTile + kSumAll2Max - 1) / kSumAll2Max;
    __shared__ float tile[kTile];
    __shared__ float col[kSumAll2Max];
    const int n = rows * cols, j = threadIdx.x;
    float v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = j + k * kSumAll2Max;
        v[k] = i < n ? x[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = j + k * kSumAll2Max;
        if (i < n)
            tile[i] = v[k];
    }
    __syncthreads();
    if (j < cols) {
        float acc = 0.0f;
#pragma unroll 8
        for (int l = 0; l < rows; ++l)
            acc += tile[l * cols + j];
        col[j] = acc;
        y1[j] = acc;
    }
    __syncthreads();
    if (j == 0) {
        float acc = 0.0f;
        for (int l = 0; l < cols; ++l)
            acc += col[l];
        y2[0] = acc * scale;
    }
}

// Both reductions of a [rows, cols] reduce_all in one block when the
// column sums are sliced: lane (sl, c) adds rows [sl slice_len, ...) of
// column c in row order (k_sum_axis_part's partial), lane c adds the
// slices in order (k_sum_axis_fin, scale 1), then lane 0 adds the column
// sums in order, times scale (k_sum_axis_part with one slice).  The same
// additions in the same order as the three launches it replaces.
constexpr int kSumAll2sThreads = 1024;
__global__ void __launch_bounds__(kSumAll2sThreads) k_sum_all2s(const float *__restrict__ x, float *__restrict__ y1,
                                                               float *__restrict__ y2, int rows, int cols,
                                                               int slices, int slice_len, float scale)
{
    __shared__ float part[kSumAll2sThreads];
    __shared__ float col[kSumAll2sThreads];
    const int t = threadIdx.x;
    if (t < slices * cols) {
        const int sl = t / cols, c = t - sl * cols;
        const int l0 = sl * slice_len, l1 = l0 + slice_len < rows ? l0 + slice_len : rows;
        const float *p = x + c;
        float acc = 0.0f;
        int l = l0;
        // 32 loads in flight before their (ordered) adds: the walk is one
        // lane's, so memory latency, not bandwidth, sets its pace
        for (; l + 32 <= l1; l += 32) {
            float v[32];
#pragma unroll
            for (int q = 0; q < 32; ++q)
                v[q] = p[(size_t)(l + q) * cols];
#pragma unroll
            for (int q = 0; q < 32; ++q)
                acc += v[q];
        }
        for (; l < l1; ++l)
            acc += p[(size_t)l * cols];
        part[t] = acc;
    }
    __syncthreads();
    if (t < cols) {
        float acc = 0.0f;
        for (int sl = 0; sl < slices; ++sl)
            acc += part[sl * cols + t];
        col[t] = acc;
        y1[t] = acc;
    }
    __syncthreads();
    if (t == 0) {
        float acc = 0.0f;
        for (int l = 0; l < cols; ++l)
            acc += col[l];
        y2[0] = acc * scale;
    }
}

// slices for a reduction: about 2^18 partial sums, runs of at least 64
inline void sum_axis_plan(size_t outer, size_t len, size_t inner, size_t *slices, size_t *slice_len)
{
    size_t n = outer * inner;
    size_t want = n ? ((size_t)1 << 18) / n : 1;
    size_t most = len / 64;
    size_t sl = want < most ? want : most;
    if (sl < 1)
        sl = 1;
    *slice_len = (len + sl - 1) / sl;
    *slices = *slice_len ? (len + *slice_len - 1) / *slice_len : 1;
    if (*slices < 1)
        *slices = 1;
}

// f32 -> 16-bit, 8 elements per lane per pass (two 16-byte loads, one
// 16-byte store).  Plain loads and stores: on gfx950 the non-temporal forms
// measured 25-40 % slower for this stream (4.2-5.1 against 7.1 TB/s).
template <int DT>
__global__ void __launch_bounds__(kBlock) k_cast_to16(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                      size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const bool vec = ((((uintptr_t)src) | ((uintptr_t)dst)) & 15) == 0;
    const size_t n8 = vec ? n / 8 : 0;
    for (size_t j = i; j < n8; j += stride) {
        const float4 v0 = reinterpret_cast<const float4 *>(src)[2 * j];
        const float4 v1 = reinterpret_cast<const float4 *>(src)[2 * j + 1];
        uint4 o;
        o.x = to16x2(DT, v0.x, v0.y);
        o.y = to16x2(DT, v0.z, v0.w);
        o.z = to16x2(DT, v1.x, v1.y);
        o.w = to16x2(DT, v1.z, v1.w);
        reinterpret_cast<uint4 *>(dst)[j] = o;
    }
    for (size_t j = n8 * 8 + i; j < n; j += stride)
        dst[j] = to16(DT, src[j]);
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
// One launch updates every parameter: every tensor is cut into chunks of
// kSgdChunk elements, one block each, and first[i] is the first block of
// tensor i (so a 4096-element bias takes 2 blocks and a 16M-element weight
// 8192, with no idle blocks).
// g' = g + wd*p; buf = mu*buf + (1-damp)*g'; u = nesterov ? g' + mu*buf : buf;
// p -= lr*u  (the reference's sgd.c:147-160 update, per element).
#define PGK_SGD_MAX_SEG 32
constexpr int kSgdVec = 2; // float4 per lane per block, all loads issued first
constexpr size_t kSgdChunk = (size_t)kBlock * 4 * kSgdVec;
struct sgd_table {
    pgk_sgd_seg seg[PGK_SGD_MAX_SEG];
    unsigned first[PGK_SGD_MAX_SEG + 1];
    int cnt;
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

// One block's chunk on the vector path.  FULL (the whole chunk in range)
// and HAS_BUF are compile-time, so every load of the chunk is issued before
// the first use: under a per-vector bound or buffer test the compiler
// issues and waits for each group of loads in turn.
// the grad as the update reads it: with a pending clip-by-norm scale,
// (g * gmul) * ginv, the scaling pass's arithmetic (bit for bit the update
// after that pass)
__device__ __forceinline__ float sgd_clipped(const pgk_sgd_seg &sg, float g)
{
#pragma clang fp contract(off)
    return sg.gclip ? (g * sg.gmul) * sg.ginv : g;
}

template <bool FULL, bool HAS_BUF>
__device__ __forceinline__ void sgd_vec(const pgk_sgd_seg &sg, size_t base, size_t n, float lr, float mu, float damp,
                                        float wd, int nesterov)
{
    float4 p[kSgdVec], g[kSgdVec], b[kSgdVec];
    size_t e[kSgdVec];
#pragma unroll
    for (int k = 0; k < kSgdVec; ++k) {
        e[k] = base + 4 * ((size_t)threadIdx.x + (size_t)k * kBlock);
        if (FULL || e[k] + 4 <= n) {
            p[k] = ntl4(sg.p + e[k]);
            g[k] = ntl4(sg.g + e[k]);
            g[k] = make_float4(sgd_clipped(sg, g[k].x), sgd_clipped(sg, g[k].y), sgd_clipped(sg, g[k].z),
                               sgd_clipped(sg, g[k].w));
            b[k] = HAS_BUF ? ntl4(sg.buf + e[k]) : make_float4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int k = 0; k < kSgdVec; ++k) {
        if (FULL || e[k] + 4 <= n) {
            sgd_elem(p[k].x, g[k].x, b[k].x, HAS_BUF, lr, mu, damp, wd, nesterov);
            sgd_elem(p[k].y, g[k].y, b[k].y, HAS_BUF, lr, mu, damp, wd, nesterov);
            sgd_elem(p[k].z, g[k].z, b[k].z, HAS_BUF, lr, mu, damp, wd, nesterov);
            sgd_elem(p[k].w, g[k].w, b[k].w, HAS_BUF, lr, mu, damp, wd, nesterov);
            nts4(p[k], sg.p + e[k]);
            if (HAS_BUF)
                nts4(b[k], sg.buf + e[k]);
            if (sg.shadow) {
                reinterpret_cast<uint2 *>(sg.shadow + e[k])[0] =
                    make_uint2(to16x2(sg.shadow_dtype, p[k].x, p[k].y), to16x2(sg.shadow_dtype, p[k].z, p[k].w));
            }
        } else {
            for (size_t j = e[k]; j < n; ++j) { // the last 1-3 elements
                float pj = sg.p[j], bj = HAS_BUF ? sg.buf[j] : 0.0f;
                sgd_elem(pj, sgd_clipped(sg, sg.g[j]), bj, HAS_BUF, lr, mu, damp, wd, nesterov);
                sg.p[j] = pj;
                if (HAS_BUF)
                    sg.buf[j] = bj;
                if (sg.shadow)
                    sg.shadow[j] = to16(sg.shadow_dtype, pj);
            }
        }
    }
}

__global__ void __launch_bounds__(kBlock) k_sgd(sgd_table tab, float lr, float mu, float damp, float wd,
                                                int nesterov)
{
    const unsigned blk = blockIdx.x;
    const int si = seg_of<PGK_SGD_MAX_SEG>(tab.first, blk);
    const pgk_sgd_seg sg = tab.seg[si];
    const size_t n = sg.n, base = (size_t)(blk - tab.first[si]) * kSgdChunk;
    const bool has_buf = sg.buf != nullptr;
    // a pitched shadow takes the per-element path (its rows break the
    // 4-element groups)
    const bool aligned = ((((uintptr_t)sg.p) | ((uintptr_t)sg.g) | ((uintptr_t)sg.buf)) & 15) == 0 &&
                         (((uintptr_t)sg.shadow) & 7) == 0 && !sg.shadow_cols;
    if (aligned) {
        const bool full = base + kSgdChunk <= n;
        if (full && has_buf)
            sgd_vec<true, true>(sg, base, n, lr, mu, damp, wd, nesterov);
        else if (full)
            sgd_vec<true, false>(sg, base, n, lr, mu, damp, wd, nesterov);
        else if (has_buf)
            sgd_vec<false, true>(sg, base, n, lr, mu, damp, wd, nesterov);
        else
            sgd_vec<false, false>(sg, base, n, lr, mu, damp, wd, nesterov);
    } else {
        const size_t end = base + kSgdChunk < n ? base + kSgdChunk : n;
        for (size_t j = base + threadIdx.x; j < end; j += kBlock) {
            float pj = sg.p[j], bj = has_buf ? sg.buf[j] : 0.0f;
            sgd_elem(pj, sgd_clipped(sg, sg.g[j]), bj, has_buf, lr, mu, damp, wd, nesterov);
            sg.p[j] = pj;
            if (has_buf)
                sg.buf[j] = bj;
            if (sg.shadow)
                sg.shadow[shadow_at(sg, j)] = to16(sg.shadow_dtype, pj);
        }
    }
}

// ---------------------------------------------------------------- bias-grad sums
// job.out[c] (beta ? += : =) sum_b job.part[b n + c], b in order, for
// columns c0, c0 + step, ...: 32 loads in flight before their ordered adds
// (a launch of few waves, paced by memory latency)
__device__ __forceinline__ void colsum_cols(const pgk_colsum_job &job, size_t c0, size_t step)
{
    const size_t n = job.n, nblk = job.nblk;
    for (size_t c = c0; c < n; c += step) {
        float acc = 0.0f;
        size_t b = 0;
        for (; b + 32 <= nblk; b += 32) {
            float v[32];
#pragma unroll
            for (int q = 0; q < 32; ++q)
                v[q] = job.part[(b + q) * n + c];
#pragma unroll
            for (int q = 0; q < 32; ++q)
                acc += v[q];
        }
#pragma unroll 8
        for (; b < nblk; ++b)
            acc += job.part[b * n + c];
        job.out[c] = job.beta ? job.out[c] + acc : acc;
    }
}

// ---------------------------------------------------------------- linear backward
// dz = g * act'(z) (act 0: dz = g) for a [m, n] f32 grad, written as RNE
// 16-bit rows of ldd (ldd % 8 == 0) with zeros in columns [n, ldd); DT 1
// stores f16, 2 bf16.  A block is 16 x 16 lanes over 128 columns: lane
// (cx, ry) takes columns 4 cx .. 4 cx + 3 and 64 + 4 cx .. 64 + 4 cx + 3 of
// rows ry, ry + 16, ... of the block's `rpb` rows, so each load of a wave
// reads 4 rows of two whole 128-byte lines and each 16-bit store writes 4
// rows of one.  The lane's rows go in pairs (r, r + 16), the next pair's
// loads issued before the current pair's products.  With part given, the
// block's column sums (each lane's rows in order, then the 16 row lanes in
// ry order) go to part[row block][n]; k_colsum_fin adds the row blocks in
// order (deterministic).
__device__ __forceinline__ float act_grad(int act, float z)
{
    if (act == 1)
        return z > 0.0f ? 1.0f : 0.0f;
    if (act == 2)
        return pgm_gelu_grad(z);
    return 1.0f;
}

// one row of the lane's eight columns (c0 .. c0 + 3 in gv[0..3], c0 + 64 ..
// in gv[4..7]): the products, their 16-bit stores (each 4-column group
// whose first column is below ldd: ldd % 8 == 0, so a group is inside or
// outside whole) and the column sums (in row order)
template <int ACT, int DT>
__device__ __forceinline__ void act_bwd_row(const float (&gv)[8], const float (&zv)[8], float (&acc)[8],
                                            uint16_t *__restrict__ dst, bool lo, bool hi)
{
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 8; q += 2) {
        // the sums add the rounded f32 products, as a sum over the dz tensor
        // would (no product contracted into the add)
#pragma clang fp contract(off)
        const float d0 = ACT ? gv[q] * act_grad(ACT, zv[q]) : gv[q];
        const float d1 = ACT ? gv[q + 1] * act_grad(ACT, zv[q + 1]) : gv[q + 1];
        acc[q] += d0;
        acc[q + 1] += d1;
        w[q / 2] = to16x2(DT, d0, d1);
    }
    // columns past n hold g = 0, so they store zeros
    if (lo)
        *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
    if (hi)
        *reinterpret_cast<uint2 *>(dst + 64) = make_uint2(w[2], w[3]);
}

// the loads of rows r and r + 16 (off = r * n + c0), non-temporal: the
// grad and the pre-activation are read once
template <int ACT>
__device__ __forceinline__ void act_bwd_load2(const float *__restrict__ g, const float *__restrict__ z, size_t off,
                                              size_t n, float4 (&gq)[2][2], float4 (&zq)[2][2])
{
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const size_t o = off + 16 * u * n;
        gq[u][0] = ntl4(g + o);
        gq[u][1] = ntl4(g + o + 64);
        if (ACT) {
            zq[u][0] = ntl4(z + o);
            zq[u][1] = ntl4(z + o + 64);
        }
    }
}

template <int ACT, int DT>
__device__ __forceinline__ void act_bwd_pair(const float4 (&gq)[2][2], const float4 (&zq)[2][2], float (&acc)[8],
                                             uint16_t *__restrict__ dst, size_t ldd)
{
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float gv[8] = {gq[u][0].x, gq[u][0].y, gq[u][0].z, gq[u][0].w,
                             gq[u][1].x, gq[u][1].y, gq[u][1].z, gq[u][1].w};
        float zv[8] = {};
        if (ACT) {
            const float zt[8] = {zq[u][0].x, zq[u][0].y, zq[u][0].z, zq[u][0].w,
                                 zq[u][1].x, zq[u][1].y, zq[u][1].z, zq[u][1].w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                zv[q] = zt[q];
        }
        act_bwd_row<ACT, DT>(gv, zv, acc, dst + 16 * u * ldd, true, true);
    }
}

template <int ACT, int DT>
__global__ void __launch_bounds__(kBlock) k_act_bwd16(const float *__restrict__ g, const float *__restrict__ z,
                                                      size_t m, size_t n, uint16_t *__restrict__ d16, size_t ldd,
                                                      float *__restrict__ part, size_t rpb, pgk_colsum_job fin)
{
    __shared__ float red[16][129];
    // with an earlier pass's bias-grad sums to finish, the first row of
    // blocks adds them and the pass's row blocks follow
    size_t by = blockIdx.y;
    if (fin.part) {
        if (by == 0) {
            colsum_cols(fin, (size_t)blockIdx.x * kBlock + threadIdx.x, (size_t)gridDim.x * kBlock);
            return;
        }
        --by;
    }
    const int cx = threadIdx.x & 15, ry = threadIdx.x >> 4;
    const size_t cb = (size_t)blockIdx.x * 128, c0 = cb + (size_t)cx * 4;
    const size_t rb = by * rpb, re = rb + rpb < m ? rb + rpb : m;
    const bool lo = c0 < ldd, hi = c0 + 64 < ldd;
    // every column of the block inside n: the 16-byte path for every lane
    const bool vec = cb + 128 <= n && (n & 3) == 0 && ((((uintptr_t)g) | ((uintptr_t)z)) & 15) == 0;
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
        acc[q] = 0.0f;
    size_t r = rb + ry;
    // pairs of rows every row lane of the block has (rows up to re)
    const size_t np = vec ? (re - rb) / 32 : 0;
    if (np) {
        float4 ga[2][2], za[2][2], gb[2][2], zb[2][2];
        act_bwd_load2<ACT>(g, z, r * n + c0, n, ga, za);
        size_t p = 0;
        for (; p + 2 < np; p += 2, r += 64) {
            act_bwd_load2<ACT>(g, z, (r + 32) * n + c0, n, gb, zb);
            act_bwd_pair<ACT, DT>(ga, za, acc, d16 + r * ldd + c0, ldd);
            act_bwd_load2<ACT>(g, z, (r + 64) * n + c0, n, ga, za);
            act_bwd_pair<ACT, DT>(gb, zb, acc, d16 + (r + 32) * ldd + c0, ldd);
        }
        if (p + 1 < np) {
            act_bwd_load2<ACT>(g, z, (r + 32) * n + c0, n, gb, zb);
            act_bwd_pair<ACT, DT>(ga, za, acc, d16 + r * ldd + c0, ldd);
            act_bwd_pair<ACT, DT>(gb, zb, acc, d16 + (r + 32) * ldd + c0, ldd);
            r += 64;
        } else {
            act_bwd_pair<ACT, DT>(ga, za, acc, d16 + r * ldd + c0, ldd);
            r += 32;
        }
    }
    if (lo) {
        for (; r < re; r += 16) {
            float gv[8], zv[8];
            const size_t off = r * n + c0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const size_t o = q < 4 ? q : 60 + q; // columns c0 + q, then c0 + 64 + q - 4
                const bool in = c0 + o < n;
                gv[q] = in ? g[off + o] : 0.0f;
                zv[q] = (in && ACT) ? z[off + o] : 0.0f;
            }
            act_bwd_row<ACT, DT>(gv, zv, acc, d16 + r * ldd + c0, lo, hi);
        }
    }
    if (part) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            red[ry][cx * 4 + q] = acc[q];
            red[ry][64 + cx * 4 + q] = acc[4 + q];
        }
        __syncthreads();
        if (threadIdx.x < 128) {
            const size_t col = cb + threadIdx.x;
            float sum = 0.0f;
#pragma unroll
            for (int y = 0; y < 16; ++y)
                sum += red[y][threadIdx.x];
            if (col < n)
                part[by * n + col] = sum;
        }
    }
}

// The same pass when the grad g is itself the dgrad of a narrow next layer:
// g = dn . wn^T with dn [m, kw] and wn [n, kw] 16-bit, kw = ldn = ldw = 8
// or 16 (a layer of at most 16 outputs, its dz and its weights' copy with
// zero columns past the real width).  g is formed here with the MFMA
// sequence k_gemm16 runs for that dgrad -- one v_mfma_f32_32x32x16 on the
// operands (the upper 8 k zero when kw = 8) from zero accumulators, then
// three on zeros for the rest of its 64-deep k-tile -- so every g element has
// the bits the GEMM writes; g is written out as the grad and used at once,
// so the [m, n] grad is written once and never read back.  A block is four
// waves over 128 columns, wave w taking columns 32 w .. 32 w + 31 of the
// block's rows, 32 rows per step (one 32 x 32 product; the next step's loads
// issued before the current step's product): the product goes through a
// per-wave LDS tile to four columns of four rows per lane (columns
// 4 (lane % 8) .. + 3 of rows lane / 8 + 8 i, so each z load of a wave reads
// 8 whole 128-byte row segments), where z is read, g, dz and the column sums
// formed as in k_act_bwd16 (the lane's rows in order, then the 8 row lanes
// in order).  Without d16 (and part) the pass is the narrow dgrad alone.
typedef __bf16 nbf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 nf16x8 __attribute__((ext_vector_type(8)));
typedef float nf32x16 __attribute__((ext_vector_type(16)));

template <bool F16>
__device__ __forceinline__ nf32x16 narrow_mfma(const uint4 &a, const uint4 &b, const nf32x16 &c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(nf16x8, a), __builtin_bit_cast(nf16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(nbf16x8, a),
                                                       __builtin_bit_cast(nbf16x8, b), c, 0, 0, 0);
}

constexpr int kNarrowLd = 36; // LDS tile pitch (floats): 16-byte rows

// what one lane of a narrow pass works with: the fixed arguments and the
// lane's offsets from a step's first row (row lane / 8 of the step in z, g
// and dz; its fragment row lane % 32 in dn)
struct narrow_lane {
    const uint16_t *dn;
    const float *z;
    float *g;
    uint16_t *d16;
    size_t re, n, ldd, jc;
    size_t zo, dzo, ao;
    int kw, lane;
};

// the loads of the 32-row step at i0: the dz fragment and z of the lane's
// four rows.  In a step with rows past re (the last), those rows read row
// re - 1 instead (zeroed at the product, not used).
template <int ACT, bool VEC>
__device__ __forceinline__ void narrow_load(const narrow_lane &L, size_t i0, uint4 &a, float (&zv)[4][4])
{
    const int h = L.lane >> 5, rl = L.lane >> 3;
    if (i0 + 32 <= L.re) {
        a = *reinterpret_cast<const uint4 *>(L.dn + i0 * (size_t)L.kw + L.ao);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float *zr = L.z + (i0 + 8 * i) * L.n + L.zo;
            if (ACT && VEC) {
                const float4 v = ntl4(zr);
                zv[i][0] = v.x, zv[i][1] = v.y, zv[i][2] = v.z, zv[i][3] = v.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    zv[i][q] = (ACT && L.jc + q < L.n) ? zr[q] : 0.0f;
            }
        }
        return;
    }
    const size_t ia = i0 + (L.lane & 31);
    a = *reinterpret_cast<const uint4 *>(L.dn + (ia < L.re ? ia : L.re - 1) * (size_t)L.kw +
                                         (8 * h < L.kw ? 8 * h : 0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t r = i0 + rl + 8 * i, rr = r < L.re ? r : L.re - 1;
        if (ACT && VEC) {
            const float4 v = *reinterpret_cast<const float4 *>(L.z + rr * L.n + L.jc);
            zv[i][0] = v.x, zv[i][1] = v.y, zv[i][2] = v.z, zv[i][3] = v.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                zv[i][q] = (ACT && L.jc + q < L.n) ? L.z[rr * L.n + L.jc + q] : 0.0f;
        }
    }
}

// the step at i0: the product through the wave's tile, then g, dz and the
// column sums of the lane's four rows
template <int ACT, bool F16, int DT, bool VEC>
__device__ __forceinline__ void narrow_step(const narrow_lane &L, float (*tile)[kNarrowLd], const uint4 &araw,
                                            const uint4 &bfrag, const float (&zv)[4][4], size_t i0, float (&cs)[4])
{
    const int h = L.lane >> 5, rl = L.lane >> 3;
    const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
    const uint4 afrag = (i0 + (L.lane & 31) < L.re && 8 * h < L.kw) ? araw : zero4;
    nf32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e)
        acc[e] = 0.0f;
    acc = narrow_mfma<F16>(afrag, bfrag, acc);
#pragma unroll
    for (int s = 1; s < 4; ++s)
        acc = narrow_mfma<F16>(zero4, zero4, acc);
    // lane holds column lane % 32 of rows 8 (e / 4) + 4 h + e % 4
#pragma unroll
    for (int e = 0; e < 16; ++e)
        tile[8 * (e >> 2) + 4 * h + (e & 3)][L.lane & 31] = acc[e];
    __builtin_amdgcn_wave_barrier();
    float gv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = *reinterpret_cast<const float4 *>(&tile[rl + 8 * i][4 * (L.lane & 7)]);
        gv[i][0] = v.x, gv[i][1] = v.y, gv[i][2] = v.z, gv[i][3] = v.w;
    }
    __builtin_amdgcn_wave_barrier(); // every lane has read the tile before the next step writes it
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool rin = i0 + rl + 8 * i < L.re, row = rin && L.jc < L.n;
        float d[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma clang fp contract(off)
            const bool in = row && L.jc + q < L.n;
            d[q] = in ? (ACT ? gv[i][q] * act_grad(ACT, zv[i][q]) : gv[i][q]) : 0.0f;
            cs[q] += d[q];
        }
        if (!rin)
            continue;
        if (L.g && row) {
            float *gr = L.g + (i0 + 8 * i) * L.n + L.zo;
            if (VEC) {
                *reinterpret_cast<float4 *>(gr) = make_float4(gv[i][0], gv[i][1], gv[i][2], gv[i][3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (L.jc + q < L.n)
                        gr[q] = gv[i][q];
            }
        }
        // columns past n store zeros; ldd % 8 == 0 and jc % 4 == 0, so the
        // lane's 4 columns are inside ldd whole or not at all
        if (L.d16 && L.jc < L.ldd)
            *reinterpret_cast<uint2 *>(L.d16 + (i0 + 8 * i) * L.ldd + L.dzo) =
                make_uint2(to16x2(DT, d[0], d[1]), to16x2(DT, d[2], d[3]));
    }
}

// the steps of rows [rb, re), each step's loads issued before the
// previous step's product
template <int ACT, bool F16, int DT, bool VEC>
__device__ __forceinline__ void narrow_rows(const narrow_lane &L, float (*tile)[kNarrowLd], const uint4 &bfrag,
                                            size_t rb, float (&cs)[4])
{
    if (rb >= L.re)
        return;
    uint4 aa, ab;
    float za[4][4], zb[4][4];
    narrow_load<ACT, VEC>(L, rb, aa, za);
    for (size_t i0 = rb;; i0 += 64) {
        if (i0 + 32 >= L.re) {
            narrow_step<ACT, F16, DT, VEC>(L, tile, aa, bfrag, za, i0, cs);
            break;
        }
        narrow_load<ACT, VEC>(L, i0 + 32, ab, zb);
        narrow_step<ACT, F16, DT, VEC>(L, tile, aa, bfrag, za, i0, cs);
        if (i0 + 64 >= L.re) {
            narrow_step<ACT, F16, DT, VEC>(L, tile, ab, bfrag, zb, i0 + 32, cs);
            break;
        }
        narrow_load<ACT, VEC>(L, i0 + 64, aa, za);
        narrow_step<ACT, F16, DT, VEC>(L, tile, ab, bfrag, zb, i0 + 32, cs);
    }
}

template <int ACT, bool F16, int DT>
__global__ void __launch_bounds__(kBlock, 4) k_act_bwd16n(const uint16_t *__restrict__ dn, const uint16_t *__restrict__ wn,
                                                       int kw, uint16_t *__restrict__ wsnap, float *__restrict__ g,
                                                       const float *__restrict__ z, size_t m, size_t n,
                                                       uint16_t *__restrict__ d16, size_t ldd,
                                                       float *__restrict__ part, size_t rpb, pgk_colsum_job fin)
{
    __shared__ __attribute__((aligned(16))) float tile[4][32][kNarrowLd];
    // an earlier pass's bias-grad sums: the first row of blocks, as in
    // k_act_bwd16
    size_t by = blockIdx.y;
    if (fin.part) {
        if (by == 0) {
            colsum_cols(fin, (size_t)blockIdx.x * kBlock + threadIdx.x, (size_t)gridDim.x * kBlock);
            return;
        }
        --by;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t j0 = (size_t)blockIdx.x * 128 + (size_t)wave * 32;
    const size_t rb = by * rpb, re = rb + rpb < m ? rb + rpb : m;
    const int h = lane >> 5;
    // the weights' fragment: row j0 + lane % 32, k 8 h .. 8 h + 7
    uint4 bfrag = make_uint4(0u, 0u, 0u, 0u);
    {
        const size_t j = j0 + (lane & 31);
        if (j < n && 8 * h < kw) {
            bfrag = *reinterpret_cast<const uint4 *>(wn + j * (size_t)kw + 8 * h);
            // the first row block copies the weights it read (the pending
            // product of a grad not written here keeps this copy)
            if (wsnap && by == 0)
                *reinterpret_cast<uint4 *>(wsnap + j * (size_t)kw + 8 * h) = bfrag;
        }
    }
    const size_t jc = j0 + 4 * (size_t)(lane & 7), rl = (size_t)(lane >> 3);
    const narrow_lane L = {dn,          z,           g,
                           d16,         re,          n,
                           ldd,         jc,          rl * n + jc,
                           rl * ldd + jc, (size_t)(lane & 31) * kw + (8 * h < kw ? 8 * h : 0), kw,
                           lane};
    // the wave's 32 columns inside n: 16-byte accesses for every lane
    const bool vec = j0 + 32 <= n && (n & 3) == 0 && ((((uintptr_t)g) | ((uintptr_t)z)) & 15) == 0;
    float cs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec)
        narrow_rows<ACT, F16, DT, true>(L, tile[wave], bfrag, rb, cs);
    else
        narrow_rows<ACT, F16, DT, false>(L, tile[wave], bfrag, rb, cs);
    if (part) {
        // the 8 row lanes of each column, in row order
        __builtin_amdgcn_wave_barrier();
        *reinterpret_cast<float4 *>(&tile[wave][lane >> 3][4 * (lane & 7)]) = make_float4(cs[0], cs[1], cs[2], cs[3]);
        __builtin_amdgcn_wave_barrier();
        if (lane < 32) {
            float sum = 0.0f;
#pragma unroll
            for (int y = 0; y < 8; ++y)
                sum += tile[wave][y][lane];
            const size_t col = j0 + lane;
            if (col < n)
                part[by * n + col] = sum;
        }
    }
}

__global__ void __launch_bounds__(64) k_colsum_fin(pgk_colsum_job job)
{
    colsum_cols(job, (size_t)blockIdx.x * blockDim.x + threadIdx.x, (size_t)gridDim.x * blockDim.x);
}

// ---------------------------------------------------------------- uploads
// One block per 16 KiB of each entry (first[i] = entry i's first block);
// 16-byte copies when source and destination allow, bytes otherwise.
struct upload_table {
    pgk_upload e[PGK_UPLOAD_MAX];
    unsigned first[PGK_UPLOAD_MAX + 1];
    int cnt;
};
constexpr size_t kUpChunk = (size_t)kBlock * 64;

__global__ void __launch_bounds__(kBlock) k_upload(upload_table tab)
{
    const unsigned b = blockIdx.x;
    const int s = seg_of<PGK_UPLOAD_MAX>(tab.first, b);
    const pgk_upload e = tab.e[s];
    const size_t base = (size_t)(b - tab.first[s]) * kUpChunk;
    const size_t end = base + kUpChunk < e.n ? base + kUpChunk : e.n;
    const unsigned char *__restrict__ src = (const unsigned char *)e.src;
    unsigned char *__restrict__ dst = (unsigned char *)e.dst;
    if ((((uintptr_t)src) | ((uintptr_t)dst)) % 16 == 0) {
        // the source is host memory read over the bus: every 16-byte load
        // of the chunk is issued before the first store, so a chunk costs
        // one bus round trip rather than one per pass of the block
        constexpr int kUpVec = (int)(kUpChunk / (16 * kBlock));
        if (base + kUpChunk <= end) {
            const uint4 *__restrict__ s4 = reinterpret_cast<const uint4 *>(src + base) + threadIdx.x;
            uint4 *__restrict__ d4 = reinterpret_cast<uint4 *>(dst + base) + threadIdx.x;
            uint4 v[kUpVec];
#pragma unroll
            for (int k = 0; k < kUpVec; ++k)
                v[k] = s4[k * kBlock];
#pragma unroll
            for (int k = 0; k < kUpVec; ++k)
                d4[k * kBlock] = v[k];
            return;
        }
        for (size_t j = base + 16 * (size_t)threadIdx.x; j + 16 <= end; j += 16 * (size_t)kBlock)
            *reinterpret_cast<uint4 *>(dst + j) = *reinterpret_cast<const uint4 *>(src + j);
        for (size_t j = (end & ~(size_t)15) + threadIdx.x; j < end; j += kBlock) // the last 0-15 bytes
            dst[j] = src[j];
    } else {
        for (size_t j = base + threadIdx.x; j < end; j += kBlock)
            dst[j] = src[j];
    }
}

// ---------------------------------------------------------------- strided gather
// dst[i] = src[offset of logical index i], row-major over `shape`, source
// strides in elements (a permuted or otherwise strided view made contiguous)
struct gather_desc {
    int ndim;
    int64_t shape[PGK_MAX_NDIM];
    int64_t stride[PGK_MAX_NDIM];
};

template <typename T>
__global__ void __launch_bounds__(kBlock) k_gather(const T *__restrict__ src, T *__restrict__ dst, size_t n,
                                                   gather_desc d)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        size_t t = i;
        int64_t off = 0;
        for (int q = d.ndim - 1; q >= 0; --q) {
            const size_t c = t % (size_t)d.shape[q];
            t /= (size_t)d.shape[q];
            off += (int64_t)c * d.stride[q];
        }
        dst[i] = src[off];
    }
}

} // namespace

extern "C" int pgk_gather_strided(size_t elem_size, const void *src, void *dst, int ndim, const size_t *shape,
                                  const size_t *stride, pgk_stream s)
{
    if (ndim < 0 || ndim > PGK_MAX_NDIM || (elem_size != 2 && elem_size != 4))
        return (int)hipErrorInvalidValue;
    gather_desc d = {};
    d.ndim = ndim;
    size_t n = 1;
    for (int q = 0; q < ndim; ++q) {
        d.shape[q] = (int64_t)shape[q];
        d.stride[q] = (int64_t)stride[q];
        n *= shape[q];
    }
    if (!n)
        return 0;
    if (elem_size == 4)
        hipLaunchKernelGGL(k_gather<uint32_t>, dim3(grid_for(n)), dim3(kBlock), 0, (hipStream_t)s,
                           (const uint32_t *)src, (uint32_t *)dst, n, d);
    else
        hipLaunchKernelGGL(k_gather<uint16_t>, dim3(grid_for(n)), dim3(kBlock), 0, (hipStream_t)s,
                           (const uint16_t *)src, (uint16_t *)dst, n, d);
    return status();
}

extern "C" int pgk_upload_scatter(const pgk_upload *ents, int n, pgk_stream s)
{
    if (n <= 0)
        return 0;
    if (n > PGK_UPLOAD_MAX)
        return (int)hipErrorInvalidValue;
    upload_table tab = {};
    unsigned blocks = 0;
    for (int q = 0; q < n; ++q) {
        tab.e[q] = ents[q];
        tab.first[q] = blocks;
        blocks += (unsigned)((ents[q].n + kUpChunk - 1) / kUpChunk);
    }
    seg_close<PGK_UPLOAD_MAX>(tab.first, n, blocks);
    tab.cnt = n;
    if (!blocks)
        return 0;
    hipLaunchKernelGGL(k_upload, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab);
    return status();
}

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
    const int nl = bc->ndim - 1;
    bool rows4 = bc->ndim >= 1 && bc->shape[nl] % 4 == 0 && (bc->sa[nl] == 0 || bc->sa[nl] == 1) &&
                 (bc->sb[nl] == 0 || bc->sb[nl] == 1) &&
                 (((uintptr_t)a | (uintptr_t)b | (uintptr_t)y) & 15) == 0;
    for (int d = 0; rows4 && d < nl; ++d)
        rows4 = (bc->sa[nl] == 0 || bc->sa[d] % 4 == 0) && (bc->sb[nl] == 0 || bc->sb[d] % 4 == 0);
    if (rows4) {
        size_t c4 = (size_t)bc->shape[nl] / 4;
        hipLaunchKernelGGL(k_binary_rows4, dim3(grid_for(n / 4, 2)), dim3(kBlock), 0, (hipStream_t)s, op, a, b,
                           y, n / 4 / c4, c4, *bc);
        return status();
    }
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

extern "C" size_t pgk_sum_axis_workspace(size_t outer, size_t len, size_t inner)
{
    size_t slices, slice_len;
    sum_axis_plan(outer, len, inner, &slices, &slice_len);
    return slices > 1 ? slices * outer * inner * sizeof(float) : 0;
}

extern "C" int pgk_sum_axis_f32(const float *x, float *y, size_t outer, size_t len, size_t inner, float scale,
                                void *ws, pgk_stream s)
{
    size_t n = outer * inner;
    if (!n)
        return 0;
    size_t slices, slice_len;
    sum_axis_plan(outer, len, inner, &slices, &slice_len);
    if (slices > 1 && !ws)
        return (int)hipErrorInvalidValue;
    float *part = slices > 1 ? (float *)ws : y;
    hipLaunchKernelGGL(k_sum_axis_part, dim3(grid_for(slices * n)), dim3(kBlock), 0, (hipStream_t)s, x, part,
                       outer, len, inner, slices, slice_len, scale);
    if (slices > 1)
        hipLaunchKernelGGL(k_sum_axis_fin, dim3(grid_for(n)), dim3(kBlock), 0, (hipStream_t)s, part, y, n, slices,
                           scale);
    return status();
}

extern "C" int pgk_sum_all2_fits(size_t rows, size_t cols)
{
    size_t s1, l1, s2, l2;
    sum_axis_plan(1, rows, cols, &s1, &l1);
    sum_axis_plan(1, cols, 1, &s2, &l2);
    return rows && cols && rows * cols <= 127 * 127 && cols <= (size_t)kSumAll2Max && s1 == 1 && s2 == 1;
}

extern "C" int pgk_sum_all2_f32(const float *x, float *y1, float *y2, size_t rows, size_t cols, float scale,
                                pgk_stream s)
{
    if (!pgk_sum_all2_fits(rows, cols))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sum_all2, dim3(1), dim3(kSumAll2Max), 0, (hipStream_t)s, x, y1, y2, (int)rows, (int)cols,
                       scale);
    return status();
}

extern "C" int pgk_sum_all2s_fits(size_t rows, size_t cols)
{
    size_t s1, l1, s2, l2;
    sum_axis_plan(1, rows, cols, &s1, &l1);
    sum_axis_plan(1, cols, 1, &s2, &l2);
    return rows && cols && rows < ((size_t)1 << 31) && s1 * cols <= (size_t)kSumAll2sThreads && s2 == 1;
}

extern "C" int pgk_sum_all2s_f32(const float *x, float *y1, float *y2, size_t rows, size_t cols, float scale,
                                 pgk_stream s)
{
    if (!pgk_sum_all2s_fits(rows, cols))
        return (int)hipErrorInvalidValue;
    size_t slices, slice_len;
    sum_axis_plan(1, rows, cols, &slices, &slice_len);
    hipLaunchKernelGGL(k_sum_all2s, dim3(1), dim3(kSumAll2sThreads), 0, (hipStream_t)s, x, y1, y2, (int)rows,
                       (int)cols, (int)slices, (int)slice_len, scale);
    return status();
}

extern "C" int pgk_cast_to16(int dtype, const float *src, uint16_t *dst, size_t n, pgk_stream s)
{
    if (!n)
        return 0;
    // one pass per lane where the grid allows (up to 16384 blocks)
    size_t blocks = (n / 8 + kBlock - 1) / kBlock;
    blocks = blocks < 1 ? 1 : (blocks > 16384 ? 16384 : blocks);
    if (dtype == 1)
        hipLaunchKernelGGL(k_cast_to16<1>, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)s, src, dst, n);
    else
        hipLaunchKernelGGL(k_cast_to16<2>, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)s, src, dst, n);
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
        tab.cnt = cnt;
        size_t blocks = 0;
        for (int q = 0; q < cnt; ++q) {
            tab.seg[q] = segs[base + q];
            tab.first[q] = (unsigned)blocks;
            blocks += (segs[base + q].n + kSgdChunk - 1) / kSgdChunk;
            if (blocks > 0x7fffffffu)
                return (int)hipErrorInvalidValue;
        }
        seg_close<PGK_SGD_MAX_SEG>(tab.first, cnt, (unsigned)blocks);
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_sgd, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)s, tab, lr, momentum,
                           dampening, weight_decay, nesterov);
        int st = status();
        if (st)
            return st;
    }
    return 0;
}

// rows per block of k_act_bwd16: a multiple of 16 giving about 1024 blocks
// (fewer for narrow grads); measured on config 5's [4096, 4096] grads,
// 1024 blocks of 8 rows per lane beat 2048 of 4 (7 %) and 512 of 16
static size_t act_bwd_rpb(size_t m, size_t ldd)
{
    const size_t xb = (ldd + 127) / 128;
    size_t nrb = 1024 / (xb ? xb : 1);
    if (nrb > 64)
        nrb = 64; // the finisher adds at most 64 partials per column
    if (nrb < 1)
        nrb = 1;
    size_t rpb = (m + nrb - 1) / nrb;
    rpb = (rpb + 15) & ~(size_t)15;
    return rpb < 16 ? 16 : rpb;
}

extern "C" size_t pgk_act_bwd16_workspace(size_t m, size_t n)
{
    const size_t ldd = (n + 7) & ~(size_t)7;
    const size_t rpb = act_bwd_rpb(m, ldd);
    return ((m + rpb - 1) / rpb) * n * sizeof(float);
}

extern "C" int pgk_colsum_run(const pgk_colsum_job *job, pgk_stream s)
{
    if (!job || !job->n || !job->nblk)
        return 0;
    if (!job->part || !job->out)
        return (int)hipErrorInvalidValue;
    const size_t blocks = (job->n + 63) / 64;
    hipLaunchKernelGGL(k_colsum_fin, dim3((unsigned)(blocks < 65535 ? blocks : 65535)), dim3(64), 0, (hipStream_t)s,
                       *job);
    return status();
}

// the job an activation pass finishes in its first row of blocks (none: a
// zero job, and no extra row)
static int fold_job(const pgk_colsum_job *fold, pgk_colsum_job *j)
{
    *j = pgk_colsum_job{};
    if (!fold || !fold->n || !fold->nblk)
        return 0;
    if (!fold->part || !fold->out)
        return -1;
    *j = *fold;
    return 1;
}

// the last step of a pass's bias grad: handed to the caller, or launched
static int finish_db(float *part, size_t nrb, size_t n, float *db, int beta, pgk_colsum_job *defer, pgk_stream s)
{
    const pgk_colsum_job j = {part, nrb, n, db, beta};
    if (defer) {
        *defer = j;
        return 0;
    }
    return pgk_colsum_run(&j, s);
}

extern "C" int pgk_act_bwd16(int act, const float *g, const float *z, size_t m, size_t n, uint16_t *d16, size_t ldd,
                             int dtype, float *db, int db_beta, void *ws, const pgk_colsum_job *fold,
                             pgk_colsum_job *defer, pgk_stream s)
{
    if (defer)
        *defer = pgk_colsum_job{};
    pgk_colsum_job fin;
    const int nf = fold_job(fold, &fin);
    if (nf < 0)
        return (int)hipErrorInvalidValue;
    if (!m || !n)
        return nf ? pgk_colsum_run(&fin, s) : 0;
    if ((ldd & 7) || ldd < n || (((uintptr_t)d16) & 15) || (act && !z) || (db && !ws) || act < 0 || act > 2)
        return (int)hipErrorInvalidValue;
    const size_t rpb = act_bwd_rpb(m, ldd), nrb = (m + rpb - 1) / rpb;
    if (nrb + nf > 65535)
        return (int)hipErrorInvalidValue;
    const unsigned gx = (unsigned)((ldd + 127) / 128);
    float *part = db ? (float *)ws : nullptr;
    const dim3 grid(gx, (unsigned)(nrb + nf));
#define PGK_ACT_BWD(A, D)                                                                                              \
    hipLaunchKernelGGL((k_act_bwd16<A, D>), grid, dim3(kBlock), 0, (hipStream_t)s, g, z, m, n, d16, ldd, part, rpb,   \
                       fin)
    const bool f16 = dtype == 1;
    if (act == 0 && f16)
        PGK_ACT_BWD(0, 1);
    else if (act == 0)
        PGK_ACT_BWD(0, 2);
    else if (act == 1 && f16)
        PGK_ACT_BWD(1, 1);
    else if (act == 1)
        PGK_ACT_BWD(1, 2);
    else if (f16)
        PGK_ACT_BWD(2, 1);
    else
        PGK_ACT_BWD(2, 2);
#undef PGK_ACT_BWD
    const int st = status();
    if (st || !db)
        return st;
    return finish_db(part, nrb, n, db, db_beta, defer, s);
}

extern "C" int pgk_act_bwd16n(int act, const uint16_t *dn, const uint16_t *wn, int kw, int ndtype, uint16_t *wsnap,
                              float *g, const float *z, size_t m, size_t n, uint16_t *d16, size_t ldd, int dtype,
                              float *db, int db_beta, void *ws, const pgk_colsum_job *fold, pgk_colsum_job *defer,
                              pgk_stream s)
{
    if (defer)
        *defer = pgk_colsum_job{};
    pgk_colsum_job fin;
    const int nf = fold_job(fold, &fin);
    if (nf < 0)
        return (int)hipErrorInvalidValue;
    if (!m || !n)
        return nf ? pgk_colsum_run(&fin, s) : 0;
    if ((ldd & 7) || ldd < n || (((uintptr_t)d16) & 15) || (act && !z) || (db && !ws) || act < 0 || act > 2 ||
        (kw != 8 && kw != 16) || !dn || !wn || (!g && !d16) ||
        ((((uintptr_t)dn) | ((uintptr_t)wn) | ((uintptr_t)wsnap)) & 15) || (((uintptr_t)g) & 3) ||
        (ndtype != 1 && ndtype != 2))
        return (int)hipErrorInvalidValue;
    const size_t rpb = act_bwd_rpb(m, ldd), nrb = (m + rpb - 1) / rpb;
    if (nrb + nf > 65535)
        return (int)hipErrorInvalidValue;
    const unsigned gx = (unsigned)((ldd + 127) / 128);
    float *part = db ? (float *)ws : nullptr;
    const dim3 grid(gx, (unsigned)(nrb + nf));
#define PGK_NARROW(A, F, D)                                                                                            \
    hipLaunchKernelGGL((k_act_bwd16n<A, F, D>), grid, dim3(kBlock), 0, (hipStream_t)s, dn, wn, kw, wsnap, g, z, m, n,  \
                       d16, ldd, part, rpb, fin)
#define PGK_NARROW_DT(A, F)                                                                                            \
    do {                                                                                                               \
        if (dtype == 1)                                                                                                \
            PGK_NARROW(A, F, 1);                                                                                       \
        else                                                                                                           \
            PGK_NARROW(A, F, 2);                                                                                       \
    } while (0)
    const bool f16 = ndtype == 1;
    if (act == 0 && f16)
        PGK_NARROW_DT(0, true);
    else if (act == 0)
        PGK_NARROW_DT(0, false);
    else if (act == 1 && f16)
        PGK_NARROW_DT(1, true);
    else if (act == 1)
        PGK_NARROW_DT(1, false);
    else if (f16)
        PGK_NARROW_DT(2, true);
    else
        PGK_NARROW_DT(2, false);
#undef PGK_NARROW_DT
#undef PGK_NARROW
    const int st = status();
    if (st || !db)
        return st;
    return finish_db(part, nrb, n, db, db_beta, defer, s);
}
