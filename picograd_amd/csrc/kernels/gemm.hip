// GEMM kernels for gfx950.
//
// k_gemm16_nt: C[i,j] (+)= sum_p A[i,p] * B[j,p] with f16/bf16 operands whose
// reduction dim is contiguous ("NT"), f32 accumulation in MFMA
// (v_mfma_f32_32x32x16_{bf16,f16}) and f32 output.  dgrad (dC . W^T) has
// this layout natively; forward and wgrad operands are staged into it by
// the transpose kernels.  Block tile BM x BN x 64, four wave64s as 2 x 2,
// each wave owning a (BM/2) x (BN/2) sub-tile of 32x32 MFMA blocks.
// Operand tiles go global -> registers -> LDS (double buffered, one barrier
// per k-tile); the LDS rows are XOR-swizzled in 16-byte chunks so the
// fragment reads of 8 or 16 consecutive lanes hit distinct banks.
// Block ids are remapped so the tiles that share operand panels run on the
// same XCD (and its L2), grouped GROUP_M tile-rows at a time.
//
// k_gemm_f32: plain LDS-tiled f32 FMA GEMM with either operand transposed,
// for f32 matmuls (not on the bf16/f16 hot path).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;       // k elements per tile (8 chunks of 16 bytes)
constexpr int kThreads = 256;
constexpr int GROUP_M = 8;

__device__ __forceinline__ int swz(int chunk, int row) { return chunk ^ ((row & 7) ^ ((row >> 3) & 1)); }

template <bool F16>
__device__ __forceinline__ f32x16 mfma32(const uint4 &a, const uint4 &b, const f32x16 &c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int BM, int BN, bool F16>
__global__ void __launch_bounds__(kThreads) k_gemm16_nt(const uint16_t *__restrict__ A, size_t lda, size_t sA,
                                                        const uint16_t *__restrict__ B, size_t ldb, size_t sB,
                                                        float *__restrict__ C, size_t ldc, size_t sC, int M, int N,
                                                        int K, int beta, int tiles_m, int tiles_n)
{
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int LA = BM * 8 / kThreads; // 16-byte chunks per thread per k-tile
    constexpr int LB = BN * 8 / kThreads;
    __shared__ uint4 smA[2][BM * 8];
    __shared__ uint4 smB[2][BN * 8];

    // ---- tile assignment: XCD-aware remap, then grouped row-major order
    int nb = gridDim.x;
    int pid = blockIdx.x;
    if ((nb & 7) == 0)
        pid = (pid & 7) * (nb >> 3) + (pid >> 3);
    int per_group = GROUP_M * tiles_n;
    int group = pid / per_group;
    int first_m = group * GROUP_M;
    int gsz = tiles_m - first_m < GROUP_M ? tiles_m - first_m : GROUP_M;
    int in_group = pid - group * per_group;
    int tm = first_m + in_group % gsz;
    int tn = in_group / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const uint16_t *Ab = A + (size_t)blockIdx.z * sA;
    const uint16_t *Bb = B + (size_t)blockIdx.z * sB;
    float *Cb = C + (size_t)blockIdx.z * sC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ch = tid & 7;   // chunk this thread stages
    const int rbase = tid >> 3; // first row this thread stages (+32 per step)

    uint4 ra[LA], rb[LB];
    const uint4 zero = make_uint4(0, 0, 0, 0);

    auto load_tiles = [&](int k0) {
        const int kc = k0 + ch * 8;
        const bool kin = kc < K;
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            int r = m0 + rbase + 32 * i;
            ra[i] = (kin && r < M) ? *reinterpret_cast<const uint4 *>(Ab + (size_t)r * lda + kc) : zero;
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            int r = n0 + rbase + 32 * i;
            rb[i] = (kin && r < N) ? *reinterpret_cast<const uint4 *>(Bb + (size_t)r * ldb + kc) : zero;
        }
    };
    auto store_tiles = [&](int st) {
#pragma unroll
        for (int i = 0; i < LA; ++i) {
            int r = rbase + 32 * i;
            smA[st][r * 8 + swz(ch, r)] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < LB; ++i) {
            int r = rbase + 32 * i;
            smB[st][r * 8 + swz(ch, r)] = rb[i];
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.0f;

    const int KT = (K + BK - 1) / BK;
    load_tiles(0);
    store_tiles(0);
    __syncthreads();

    const int lrow = lane & 31, lk = lane >> 5;
    int cur = 0;
    for (int kt = 0; kt < KT; ++kt) {
        if (kt + 1 < KT)
            load_tiles((kt + 1) * BK);
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            const int chunk = s * 2 + lk;
            uint4 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                int r = wm * WM + i * 32 + lrow;
                fa[i] = smA[cur][r * 8 + swz(chunk, r)];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                int r = wn * WN + j * 32 + lrow;
                fb[j] = smB[cur][r * 8 + swz(chunk, r)];
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = mfma32<F16>(fa[i], fb[j], acc[i][j]);
        }
        if (kt + 1 < KT)
            store_tiles(cur ^ 1);
        __syncthreads();
        cur ^= 1;
    }

    // ---- epilogue: lane holds column lane%32 of rows (e/4)*8 + (lane/32)*4 + e%4
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * WN + j * 32 + lrow;
            if (col >= N)
                continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * WM + i * 32 + (e >> 2) * 8 + lk * 4 + (e & 3);
                if (row < M) {
                    float *p = Cb + (size_t)row * ldc + col;
                    float v = acc[i][j][e];
                    *p = beta ? *p + v : v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- f32 GEMM
constexpr int FT = 64, FK = 16;

__global__ void __launch_bounds__(256) k_gemm_f32(int ta, int tb, int M, int N, int K, const float *__restrict__ A,
                                                  size_t lda, size_t sA, const float *__restrict__ B, size_t ldb,
                                                  size_t sB, float *__restrict__ C, size_t ldc, size_t sC, int beta)
{
    __shared__ float As[FK][FT + 1];
    __shared__ float Bs[FK][FT + 1];
    const float *Ab = A + (size_t)blockIdx.z * sA;
    const float *Bb = B + (size_t)blockIdx.z * sB;
    float *Cb = C + (size_t)blockIdx.z * sC;
    const int m0 = blockIdx.y * FT, n0 = blockIdx.x * FT;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += FK) {
        for (int q = threadIdx.x; q < FK * FT; q += 256) {
            int kk = q / FT, mm = q % FT;
            int gi = m0 + mm, gk = k0 + kk;
            As[kk][mm] = (gi < M && gk < K) ? (ta ? Ab[(size_t)gk * lda + gi] : Ab[(size_t)gi * lda + gk]) : 0.0f;
            int gj = n0 + mm;
            Bs[kk][mm] = (gj < N && gk < K) ? (tb ? Bb[(size_t)gj * ldb + gk] : Bb[(size_t)gk * ldb + gj]) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < FK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u] = As[kk][ty * 4 + u];
                b[u] = Bs[kk][tx * 4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[u][v] += a[u] * b[v];
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        int gi = m0 + ty * 4 + u;
        if (gi >= M)
            continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            int gj = n0 + tx * 4 + v;
            if (gj < N) {
                float *p = Cb + (size_t)gi * ldc + gj;
                *p = beta ? *p + acc[u][v] : acc[u][v];
            }
        }
    }
}

template <int BM, int BN, bool F16>
int launch16(size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, size_t sa, const uint16_t *b, size_t ldb,
             size_t sb, float *c, size_t ldc, size_t sc, size_t batch, int beta, hipStream_t s)
{
    int tm = (int)((m + BM - 1) / BM), tn = (int)((n + BN - 1) / BN);
    dim3 grid((unsigned)(tm * tn), 1, (unsigned)batch);
    hipLaunchKernelGGL((k_gemm16_nt<BM, BN, F16>), grid, dim3(kThreads), 0, s, a, lda, sa, b, ldb, sb, c, ldc, sc,
                       (int)m, (int)n, (int)k, beta, tm, tn);
    return (int)hipGetLastError();
}

} // namespace

extern "C" int pgk_gemm16_nt(int dtype, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda,
                             size_t stride_a, const uint16_t *b, size_t ldb, size_t stride_b, float *c, size_t ldc,
                             size_t stride_c, size_t batch, int beta, pgk_stream s)
{
    if (!m || !n || !batch)
        return 0;
    if ((lda & 7) || (ldb & 7) || (((uintptr_t)a | (uintptr_t)b) & 15) || (k & 7) || batch > 65535 ||
        m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return (int)hipErrorInvalidValue;
    if (!k) { // empty reduction: C = beta ? C : 0
        if (beta)
            return 0;
        for (size_t z = 0; z < batch; ++z)
            for (size_t r = 0; r < m; ++r) {
                hipError_t e = hipMemsetAsync(c + z * stride_c + r * ldc, 0, n * sizeof(float), (hipStream_t)s);
                if (e)
                    return (int)e;
            }
        return 0;
    }
    hipStream_t st = (hipStream_t)s;
    // big tiles when they still give every CU work; else 128 x 128
    size_t big_tiles = ((m + 255) / 256) * ((n + 127) / 128) * batch;
    bool f16 = dtype == 1;
    if (big_tiles >= 192)
        return f16 ? launch16<256, 128, true>(m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch,
                                              beta, st)
                   : launch16<256, 128, false>(m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch,
                                               beta, st);
    return f16 ? launch16<128, 128, true>(m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch, beta,
                                          st)
               : launch16<128, 128, false>(m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch, beta,
                                           st);
}

extern "C" int pgk_gemm_f32(int ta, int tb, size_t m, size_t n, size_t k, const float *a, size_t lda,
                            size_t stride_a, const float *b, size_t ldb, size_t stride_b, float *c, size_t ldc,
                            size_t stride_c, size_t batch, int beta, pgk_stream s)
{
    if (!m || !n || !batch)
        return 0;
    if (batch > 65535 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return (int)hipErrorInvalidValue;
    dim3 grid((unsigned)((n + FT - 1) / FT), (unsigned)((m + FT - 1) / FT), (unsigned)batch);
    hipLaunchKernelGGL(k_gemm_f32, grid, dim3(256), 0, (hipStream_t)s, ta, tb, (int)m, (int)n, (int)k, a, lda,
                       stride_a, b, ldb, stride_b, c, ldc, stride_c, beta);
    return (int)hipGetLastError();
}
