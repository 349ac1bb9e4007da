// Multi-tensor optimizer and gradient-clipping kernels for gfx950.
//
// One launch covers up to a table's worth of tensors.  Every tensor is cut
// into fixed chunks (one block each) and `first[i]` is the first block of
// tensor i, so the grid is the sum of the chunk counts: a 10-element bias
// costs one block, not a whole row of idle ones, and the large weights keep
// every CU busy.  A block finds its tensor by a scan of `first` (uniform,
// scalar) and moves 16 bytes per lane per access.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"
#include "convert16.h"
#include "segtab.h"

namespace {

constexpr int kBlock = 256;

inline int status() { return (int)hipGetLastError(); }

// 16-byte streaming (non-temporal) accesses: every optimiser array is read
// and written once per step
typedef float f32x4 __attribute__((ext_vector_type(4)));
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

// ---------------------------------------------------------------- Adam
// adam.c:157-177 per element, in the order the reference's -O3 -ffast-math
// build evaluates it: decay (AdamW shrink or L2 grad term), moments
// reassociated to g + b1*(m - g) and g^2 + b2*(v - g^2), amsgrad's running
// max of v, then p -= (m*lr) / ((sqrt(v * (1/bc2)) + eps) * bc1).  Every
// product and sum is rounded on its own (no FMA, as in that x86 build);
// sqrtf and / are IEEE (correctly rounded), as in its remainder loop.
constexpr int kAdamVec = 2; // float4 per lane per block
constexpr size_t kAdamChunk = (size_t)kBlock * 4 * kAdamVec;
#define PGK_ADAM_MAX_SEG 32

struct adam_table {
    pgk_adam_seg seg[PGK_ADAM_MAX_SEG];
    unsigned first[PGK_ADAM_MAX_SEG + 1];
    int cnt;
};

__device__ __forceinline__ void adam_elem(float &p, float g, float &m, float &v, float &vm, bool ams,
                                          const pgk_adam_hyper &h, float lr, float wd)
{
#pragma clang fp contract(off)
    float pj = p, gj = g;
    if (wd != 0.0f) {
        if (h.decoupled)
            pj = pj - lr * wd * pj;
        else
            gj = gj + wd * pj;
    }
    m = gj + h.beta1 * (m - gj);
    const float g2 = gj * gj;
    v = g2 + h.beta2 * (v - g2);
    float vh = v;
    if (ams) {
        if (v > vm)
            vm = v;
        vh = vm;
    }
    const float denom = (sqrtf(vh * h.inv_bc2) + h.eps) * h.bc1;
    p = pj - (m * lr) / denom;
}

// the grad as the update reads it: with a pending clip-by-norm scale,
// (g * mul) * inv -- the scaling pass's arithmetic, so the update equals
// the one after that pass bit for bit
template <class Seg>
__device__ __forceinline__ float clipped(const Seg &sg, float g)
{
#pragma clang fp contract(off)
    return sg.gclip ? (g * sg.gmul) * sg.ginv : g;
}

template <class Seg>
__device__ __forceinline__ float4 clipped4(const Seg &sg, float4 g)
{
    return make_float4(clipped(sg, g.x), clipped(sg, g.y), clipped(sg, g.z), clipped(sg, g.w));
}

__global__ void __launch_bounds__(kBlock) k_adam(adam_table tab, pgk_adam_hyper h)
{
    const unsigned b = blockIdx.x;
    const int si = seg_of<PGK_ADAM_MAX_SEG>(tab.first, b);
    const pgk_adam_seg sg = tab.seg[si];
    const size_t base = (size_t)(b - tab.first[si]) * kAdamChunk;
    const size_t n = sg.n;
    const bool ams = sg.vmax != nullptr;
    float *__restrict__ P = sg.p;
    const float *__restrict__ G = sg.g;
    float *__restrict__ M = sg.m;
    float *__restrict__ V = sg.v;
    float *__restrict__ VM = sg.vmax;
    // a pitched shadow takes the per-element path
    const bool vec = ((((uintptr_t)P) | ((uintptr_t)G) | ((uintptr_t)M) | ((uintptr_t)V) | ((uintptr_t)VM)) & 15) == 0 &&
                     (((uintptr_t)sg.shadow) & 7) == 0 && !sg.shadow_cols;
    if (vec) {
        float4 p[kAdamVec], g[kAdamVec], m[kAdamVec], v[kAdamVec], vm[kAdamVec];
        size_t e[kAdamVec];
#pragma unroll
        for (int k = 0; k < kAdamVec; ++k) {
            e[k] = base + 4 * ((size_t)threadIdx.x + (size_t)k * kBlock);
            if (e[k] + 4 <= n) {
                p[k] = ntl4(P + e[k]);
                g[k] = clipped4(sg, ntl4(G + e[k]));
                m[k] = ntl4(M + e[k]);
                v[k] = ntl4(V + e[k]);
                vm[k] = ams ? ntl4(VM + e[k]) : make_float4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int k = 0; k < kAdamVec; ++k) {
            if (e[k] + 4 <= n) {
                adam_elem(p[k].x, g[k].x, m[k].x, v[k].x, vm[k].x, ams, h, sg.lr, sg.wd);
                adam_elem(p[k].y, g[k].y, m[k].y, v[k].y, vm[k].y, ams, h, sg.lr, sg.wd);
                adam_elem(p[k].z, g[k].z, m[k].z, v[k].z, vm[k].z, ams, h, sg.lr, sg.wd);
                adam_elem(p[k].w, g[k].w, m[k].w, v[k].w, vm[k].w, ams, h, sg.lr, sg.wd);
                nts4(p[k], P + e[k]);
                nts4(m[k], M + e[k]);
                nts4(v[k], V + e[k]);
                if (ams)
                    nts4(vm[k], VM + e[k]);
                if (sg.shadow) {
                    *reinterpret_cast<uint2 *>(sg.shadow + e[k]) =
                        make_uint2(to16x2(sg.shadow_dtype, p[k].x, p[k].y), to16x2(sg.shadow_dtype, p[k].z, p[k].w));
                }
            } else {
                for (size_t j = e[k]; j < n; ++j) { // the last 1-3 elements
                    float pj = P[j], mj = M[j], vj = V[j], vmj = ams ? VM[j] : 0.0f;
                    adam_elem(pj, clipped(sg, G[j]), mj, vj, vmj, ams, h, sg.lr, sg.wd);
                    P[j] = pj, M[j] = mj, V[j] = vj;
                    if (ams)
                        VM[j] = vmj;
                    if (sg.shadow)
                        sg.shadow[j] = to16(sg.shadow_dtype, pj);
                }
            }
        }
    } else {
        const size_t end = base + kAdamChunk < n ? base + kAdamChunk : n;
        for (size_t j = base + threadIdx.x; j < end; j += kBlock) {
            float pj = P[j], mj = M[j], vj = V[j], vmj = ams ? VM[j] : 0.0f;
            adam_elem(pj, clipped(sg, G[j]), mj, vj, vmj, ams, h, sg.lr, sg.wd);
            P[j] = pj, M[j] = mj, V[j] = vj;
            if (ams)
                VM[j] = vmj;
            if (sg.shadow)
                sg.shadow[shadow_at(sg, j)] = to16(sg.shadow_dtype, pj);
        }
    }
}

// ---------------------------------------------------------------- grad norm
// clip.c:5-18 sums the squares in f64.  Each block adds the squares of its
// chunk in f64 (lanes in a fixed order) into part[block]; k_norm_fin adds
// the parts in a fixed order, so the result does not depend on timing.
// The scaling and clamping passes map chunks of kMapChunk elements.
constexpr int kSumVec = 8;
constexpr size_t kSumChunk = (size_t)kBlock * 4 * kSumVec;
constexpr int kMapVec = 4;
constexpr size_t kMapChunk = (size_t)kBlock * 4 * kMapVec;
#define PGK_GRAD_MAX_SEG 64

struct grad_table {
    pgk_grad_seg seg[PGK_GRAD_MAX_SEG];
    unsigned first[PGK_GRAD_MAX_SEG + 1];
    int cnt;
};

__device__ __forceinline__ double block_sum_f64(double x, double *sh)
{
    for (int o = 32; o > 0; o >>= 1)
        x += __shfl_xor(x, o);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0)
        sh[w] = x;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0)
        for (int i = 0; i < kBlock / 64; ++i)
            t += sh[i];
    return t;
}

__global__ void __launch_bounds__(kBlock) k_sumsq(grad_table tab, double *__restrict__ part)
{
    __shared__ double sh[kBlock / 64];
    const unsigned b = blockIdx.x;
    const int si = seg_of<PGK_GRAD_MAX_SEG>(tab.first, b);
    const pgk_grad_seg sg = tab.seg[si];
    const size_t base = (size_t)(b - tab.first[si]) * kSumChunk;
    const size_t n = sg.n;
    const float *__restrict__ G = sg.g;
    double acc = 0.0;
    if ((((uintptr_t)G) & 15) == 0 && base + kSumChunk <= n) {
        // a whole chunk: every load issued before the first square (a load
        // under a per-vector bound check is issued and waited for one at a
        // time); the same per-thread order as the bounded path below
        const float4 *__restrict__ G4 = reinterpret_cast<const float4 *>(G + base) + threadIdx.x;
        float4 g[kSumVec];
#pragma unroll
        for (int k = 0; k < kSumVec; ++k)
            g[k] = G4[k * kBlock];
        __builtin_amdgcn_sched_barrier(0); // no square is moved between the loads
#pragma unroll
        for (int k = 0; k < kSumVec; ++k) {
            const double x0 = g[k].x, x1 = g[k].y, x2 = g[k].z, x3 = g[k].w;
            acc += x0 * x0;
            acc += x1 * x1;
            acc += x2 * x2;
            acc += x3 * x3;
        }
    } else if ((((uintptr_t)G) & 15) == 0) {
        const size_t e0 = base + 4 * (size_t)threadIdx.x;
        float4 g[kSumVec];
#pragma unroll
        for (int k = 0; k < kSumVec; ++k) {
            const size_t e = e0 + (size_t)k * 4 * kBlock;
            g[k] = e + 4 <= n ? *reinterpret_cast<const float4 *>(G + e) : make_float4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < kSumVec; ++k) {
            const size_t e = e0 + (size_t)k * 4 * kBlock;
            if (e + 4 > n)
                for (size_t j = e; j < n; ++j) {
                    const double x = G[j];
                    acc += x * x;
                }
            const double x0 = g[k].x, x1 = g[k].y, x2 = g[k].z, x3 = g[k].w;
            acc += x0 * x0;
            acc += x1 * x1;
            acc += x2 * x2;
            acc += x3 * x3;
        }
    } else {
        const size_t end = base + kSumChunk < n ? base + kSumChunk : n;
        for (size_t j = base + threadIdx.x; j < end; j += kBlock) {
            const double x = G[j];
            acc += x * x;
        }
    }
    const double t = block_sum_f64(acc, sh);
    if (threadIdx.x == 0)
        part[b] = t;
}

constexpr int kFinBlock = 1024;

__global__ void __launch_bounds__(kFinBlock) k_norm_fin(const double *__restrict__ part, unsigned nparts, int clip,
                                                        float max_norm, float eps, float *__restrict__ res)
{
    // thread t adds parts t, t + 1024, ... (eight loads in flight), then a
    // fixed tree over the threads: the same order on every call
    __shared__ double sh[kFinBlock];
    double x = 0.0;
    unsigned i = threadIdx.x;
    for (; i + 7 * kFinBlock < nparts; i += 8 * kFinBlock) {
        double v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            v[q] = part[i + q * kFinBlock];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            x += v[q];
    }
    for (; i < nparts; i += kFinBlock)
        x += part[i];
    sh[threadIdx.x] = x;
    __syncthreads();
    for (int s = kFinBlock / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s)
            sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float total = (float)sqrt(sh[0]);
        res[0] = total;
        if (clip) {
            // clip.c:32-33: nothing happens when total <= max_norm; the
            // scale is applied as (g * max_norm) * (1 / (total + eps)), the
            // order the reference's build uses
            res[1] = 1.0f / (total + eps);
            res[2] = total <= max_norm ? 0.0f : 1.0f;
            res[3] = max_norm;
        }
    }
}

// g = (g * res[3]) * res[1] when res[2] is set (clip.c:34-39); every block
// reads the flag the finisher wrote, so no host round trip sits between the
// two passes.
struct scale_op {
    float mx, inv;
    __device__ float operator()(float g) const { return (g * mx) * inv; }
};

// clip.c:49-61: values above c become c, below -c become -c
struct clamp_op {
    float c;
    __device__ float operator()(float x) const { return x > c ? c : (x < -c ? -c : x); }
};

// g = op(g) over block b's chunk: every load of the chunk issued before the
// first store
template <typename Op>
__device__ __forceinline__ void grad_map(const grad_table &tab, unsigned b, Op op)
{
    const int si = seg_of<PGK_GRAD_MAX_SEG>(tab.first, b);
    const pgk_grad_seg sg = tab.seg[si];
    const size_t base = (size_t)(b - tab.first[si]) * kMapChunk;
    const size_t n = sg.n;
    float *__restrict__ G = sg.g;
    if ((((uintptr_t)G) & 15) == 0) {
        float4 g[kMapVec];
        size_t e[kMapVec];
#pragma unroll
        for (int k = 0; k < kMapVec; ++k) {
            e[k] = base + 4 * ((size_t)threadIdx.x + (size_t)k * kBlock);
            if (e[k] + 4 <= n)
                g[k] = *reinterpret_cast<const float4 *>(G + e[k]);
        }
#pragma unroll
        for (int k = 0; k < kMapVec; ++k) {
            if (e[k] + 4 <= n) {
                float4 r;
                r.x = op(g[k].x), r.y = op(g[k].y), r.z = op(g[k].z), r.w = op(g[k].w);
                *reinterpret_cast<float4 *>(G + e[k]) = r;
            } else {
                for (size_t j = e[k]; j < n; ++j)
                    G[j] = op(G[j]);
            }
        }
    } else {
        const size_t end = base + kMapChunk < n ? base + kMapChunk : n;
        for (size_t j = base + threadIdx.x; j < end; j += kBlock)
            G[j] = op(G[j]);
    }
}

__global__ void __launch_bounds__(kBlock) k_grad_scale(grad_table tab, const float *__restrict__ res)
{
    if (res[2] == 0.0f)
        return;
    grad_map(tab, blockIdx.x, scale_op{res[3], res[1]});
}

__global__ void __launch_bounds__(kBlock) k_grad_scale_const(grad_table tab, float mul, float inv)
{
    grad_map(tab, blockIdx.x, scale_op{mul, inv});
}

__global__ void __launch_bounds__(kBlock) k_grad_clamp(grad_table tab, float c)
{
    grad_map(tab, blockIdx.x, clamp_op{c});
}

// fills a grad table with segs[0..cnt) and their block prefix for chunks
// of `chunk` elements; returns the block count (0 when every tensor is empty)
unsigned grad_table_fill(grad_table &tab, const pgk_grad_seg *segs, int cnt, size_t chunk)
{
    tab = {};
    unsigned blocks = 0;
    for (int q = 0; q < cnt; ++q) {
        tab.seg[q] = segs[q];
        tab.first[q] = blocks;
        blocks += (unsigned)((segs[q].n + chunk - 1) / chunk);
    }
    seg_close<PGK_GRAD_MAX_SEG>(tab.first, cnt, blocks);
    tab.cnt = cnt;
    return blocks;
}

} // namespace

extern "C" int pgk_adam_multi(const pgk_adam_seg *segs, int nseg, const pgk_adam_hyper *h, pgk_stream s)
{
    for (int base = 0; base < nseg; base += PGK_ADAM_MAX_SEG) {
        const int cnt = nseg - base < PGK_ADAM_MAX_SEG ? nseg - base : PGK_ADAM_MAX_SEG;
        adam_table tab = {};
        unsigned blocks = 0;
        for (int q = 0; q < cnt; ++q) {
            tab.seg[q] = segs[base + q];
            tab.first[q] = blocks;
            blocks += (unsigned)((segs[base + q].n + kAdamChunk - 1) / kAdamChunk);
        }
        seg_close<PGK_ADAM_MAX_SEG>(tab.first, cnt, blocks);
        tab.cnt = cnt;
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_adam, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab, *h);
        const int st = status();
        if (st)
            return st;
    }
    return 0;
}

extern "C" size_t pgk_grad_norm_workspace(const pgk_grad_seg *segs, int nseg)
{
    size_t b = 0;
    for (int q = 0; q < nseg; ++q)
        b += (segs[q].n + kSumChunk - 1) / kSumChunk;
    return (b ? b : 1) * sizeof(double);
}

extern "C" int pgk_grad_norm(const pgk_grad_seg *segs, int nseg, int clip, float max_norm, float eps, float *res,
                             void *ws, pgk_stream s)
{
    double *part = (double *)ws;
    unsigned off = 0;
    for (int base = 0; base < nseg; base += PGK_GRAD_MAX_SEG) {
        const int cnt = nseg - base < PGK_GRAD_MAX_SEG ? nseg - base : PGK_GRAD_MAX_SEG;
        grad_table tab;
        const unsigned blocks = grad_table_fill(tab, segs + base, cnt, kSumChunk);
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_sumsq, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab, part + off);
        off += blocks;
        const int st = status();
        if (st)
            return st;
    }
    hipLaunchKernelGGL(k_norm_fin, dim3(1), dim3(kFinBlock), 0, (hipStream_t)s, (const double *)part, off, clip,
                       max_norm, eps, res);
    return status();
}

extern "C" int pgk_grad_scale_const(const pgk_grad_seg *segs, int nseg, float mul, float inv, pgk_stream s)
{
    for (int base = 0; base < nseg; base += PGK_GRAD_MAX_SEG) {
        const int cnt = nseg - base < PGK_GRAD_MAX_SEG ? nseg - base : PGK_GRAD_MAX_SEG;
        grad_table tab;
        const unsigned blocks = grad_table_fill(tab, segs + base, cnt, kMapChunk);
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_grad_scale_const, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab, mul, inv);
        const int st = status();
        if (st)
            return st;
    }
    return 0;
}

extern "C" int pgk_grad_scale(const pgk_grad_seg *segs, int nseg, const float *res, pgk_stream s)
{
    for (int base = 0; base < nseg; base += PGK_GRAD_MAX_SEG) {
        const int cnt = nseg - base < PGK_GRAD_MAX_SEG ? nseg - base : PGK_GRAD_MAX_SEG;
        grad_table tab;
        const unsigned blocks = grad_table_fill(tab, segs + base, cnt, kMapChunk);
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_grad_scale, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab, res);
        const int st = status();
        if (st)
            return st;
    }
    return 0;
}

extern "C" int pgk_clip_value(const pgk_grad_seg *segs, int nseg, float c, pgk_stream s)
{
    for (int base = 0; base < nseg; base += PGK_GRAD_MAX_SEG) {
        const int cnt = nseg - base < PGK_GRAD_MAX_SEG ? nseg - base : PGK_GRAD_MAX_SEG;
        grad_table tab;
        const unsigned blocks = grad_table_fill(tab, segs + base, cnt, kMapChunk);
        if (!blocks)
            continue;
        hipLaunchKernelGGL(k_grad_clamp, dim3(blocks), dim3(kBlock), 0, (hipStream_t)s, tab, c);
        const int st = status();
        if (st)
            return st;
    }
    return 0;
}
