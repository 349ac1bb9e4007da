// GEMM kernels for gfx950.
//
// k_gemm16: C[b][i, j] (beta ? += : =) sum_p A(i, p) B(p, j) with f16/bf16
// operands, f32 accumulation in MFMA (v_mfma_f32_32x32x16_{bf16,f16}) and
// f32 output.  Each operand is either "K-contiguous" (its reduction dim is
// contiguous: A(i, p) = a[i * lda + p], B(p, j) = b[j * ldb + p]) or
// "MN-contiguous" (A(i, p) = a[p * lda + i], B(p, j) = b[p * ldb + j]), so
// dgrad (dC . W^T), wgrad (A^T . dC) and the forward product (A . W) all
// read their operands where they lie, with no transposed copies.
//
// Data path, per block tile BM x BN x KB (KB = 32 or 64):
//  - global -> LDS directly (global_load_lds_dwordx4: 64 lanes x 16 bytes
//    per instruction, no staging registers) into an S-stage LDS ring; the
//    next S - 1 k-tiles' loads are in flight while one is computed;
//  - K-contiguous tiles sit in LDS as [rows][64] with 16-byte chunks
//    XOR-swizzled by (r ^ r >> 3) & 7 and reach the MFMA with ds_read_b128;
//    MN-contiguous tiles sit as [64][rows] with chunks swizzled by
//    4 (k & 3) and reach it with ds_read_b64_tr_b16, the gfx950 transposing
//    LDS read (within each 16-lane group, lane i of the result takes element
//    i % 4 of the 8 bytes lane 4p + i / 4 addressed, for slot p);
//  - fragment reads for the next 16-wide k step are issued one per MFMA of
//    the current one, and the k-loop has no branches between two barriers,
//    so each MFMA waits only for its own fragments;
//  - tiles are remapped so the blocks that share operand panels run on one
//    XCD (and its L2), grouped 8 tile-rows at a time.
// A partial last k-tile loads zeros past K: its out-of-range chunks (K % 8
// == 0 for a K-contiguous operand) or k-rows (MN-contiguous) are DMA'd from
// a 16-byte zero page.  Otherwise the host runs the last K % 64 columns as
// one more launch over zero-padded copies (beta = 1).
//
// k_gemm_f32: plain LDS-tiled f32 FMA GEMM with either operand transposed,
// for f32 matmuls (not on the bf16/f16 hot path).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <math.h>

#include <type_traits>

#include "convert16.h"
#include "launch.h"
#include "pgmath.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
#define LDS __attribute__((address_space(3)))

// alignment of split-K slices and of the zero-padded k-tail slabs: a
// multiple of every kernel k-tile depth (32 and 64)
constexpr int BK = 64;

__device__ __forceinline__ float act_f(int act, float v)
{
    if (act == PGK_ACT_RELU)
        return v > 0.0f ? v : 0.0f;
    if (act == PGK_ACT_GELU)
        return pgm_gelu(v);
    return v;
}

// s_waitcnt immediate waiting for vmcnt <= n and lgkmcnt == 0 (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at its maximum,
// lgkmcnt 11:8)
constexpr int vmcnt_lgkm0_imm(int n) { return (n & 0xF) | 0x70 | (((n >> 4) & 3) << 14); }

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

// One wave's 64 x 16-byte global -> LDS copy: lane i's bytes land at
// M0 + 16 i.  Issued as asm so the compiler's wait insertion does not
// track it (it would otherwise drain every such load before the next LDS
// read); the k-loop waits on these loads explicitly.  M0 is reserved to
// the compiler, which therefore ignores a clobber of it: the GEMM kernels
// below generate no other M0 use (checked on their gfx950 assembly), so
// writing it here disturbs nothing.  An SALU write of M0 needs one wait
// state before an LDS DMA reads it (a gfx9 hazard the compiler's hazard
// recognizer cannot see inside asm): the s_nop.
__device__ __forceinline__ void dma16(const void *src, LDS uint4 *dst)
{
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src) : "memory");
}

// The same copy from a wave-uniform base address in SGPRs plus a 32-bit
// per-lane byte offset: the form for k-tiles that lie wholly below the end
// of the reduction dim, whose per-lane offsets stay fixed from tile to tile
// (only the scalar base moves), so the loop spends no vector ALU work on
// addresses.  `sbase` must be wave-uniform and the compiler must keep it in
// SGPRs: if a change to the kernel leads it to compute the base in VGPRs,
// the assembler rejects the instruction and the build fails.  (Forcing it
// with v_readfirstlane costs two VALU ops per load in the k-loop; when doing
// so, zero-extend each 32-bit half: the builtin returns a signed int.)
__device__ __forceinline__ void dma16s(uint32_t voff, const void *sbase, LDS uint4 *dst)
{
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
                     : "memory");
}

// 16 zero bytes in global memory: the DMA source of every chunk past the
// end of the reduction dim, so a partial last k-tile lands zero-filled
__device__ const uint4 g_zero16 = {0u, 0u, 0u, 0u};

// K-contiguous operand tile: ROWS x KB (KB = 64 or 32), rows of KB / 8
// 16-byte chunks.  Load instruction q of wave w fills chunk slots
// (w NQ + q) 64 .. + 63.  Chunks are XOR-swizzled within a row so the 16
// lanes of each ds_read_b128 pass hit 16 different bank groups: by
// (r ^ r >> 3) & 7 for 8-chunk rows, by (r >> 2) & 3 for 4-chunk rows (four
// 64-byte rows share a 256-byte bank window).
template <int ROWS, int NT, int KB>
struct TileK {
    static constexpr int CH = KB / 8;
    static constexpr int NQ = ROWS * CH / NT;
    static_assert(ROWS * CH % NT == 0, "tile slots must divide by the thread count");
    static_assert(KB == 64 || KB == 32, "k depth");
    __device__ __forceinline__ static int swz(int chunk, int row)
    {
        return CH == 8 ? chunk ^ ((row ^ (row >> 3)) & 7) : chunk ^ ((row >> 2) & 3);
    }

    // rows past `extent` are clamped to its last row (their results are
    // never stored); 1 <= extent
    // chunks at k >= kend read zeros (kend % 8 == 0)
    __device__ __forceinline__ static void load_q(int q, const uint16_t *__restrict__ p, size_t ld, int row0,
                                                  int extent, int k0, int kend, LDS uint4 *dst, int tid)
    {
        const int lane = tid & 63, wave = tid >> 6;
        const int base = (wave * NQ + q) * 64;
        const int slot = base + lane;
        const int row = slot / CH;
        const int logical = swz(slot % CH, row);
        int gr = row0 + row;
        gr = gr < extent ? gr : extent - 1;
        const int kc = k0 + logical * 8;
        const void *src = kc < kend ? (const void *)(p + (size_t)gr * ld + kc) : (const void *)&g_zero16;
        dma16(src, dst + base);
    }
    // Fast form of load q (k-tiles below kend): the scalar base is row
    // `srow` (the first row load q touches, clamped like the rows) and each
    // lane's offset is (its clamped row - srow) ld + its chunk, in bytes;
    // the 64 lanes span 64 / CH rows, so the offset fits 32 bits for
    // ld < 2^26.  `wave` must be wave-uniform.
    struct Fast {
        uint32_t voff;
        int srow;
    };
    __device__ __forceinline__ static Fast fast_q(int q, size_t ld, int row0, int extent, int wave, int lane)
    {
        const int base = (wave * NQ + q) * 64;
        const int qrow = row0 + base / CH;
        const int srow = qrow < extent ? qrow : extent - 1;
        const int slot = base + lane;
        const int row = slot / CH;
        const int logical = swz(slot % CH, row);
        int gr = row0 + row;
        gr = gr < extent ? gr : extent - 1;
        return {(uint32_t)((size_t)(gr - srow) * ld * 2 + (size_t)logical * 16), srow};
    }
    __device__ __forceinline__ static void load_fast(int q, const Fast &f, const uint16_t *__restrict__ p, size_t ld,
                                                     int /*row0*/, int k0, LDS uint4 *dst, int wave)
    {
        dma16s(f.voff, p + (size_t)f.srow * ld + k0, dst + (wave * NQ + q) * 64);
    }

    // MFMA operand fragment: rows r0 + lane % 32, k = 16 s + 8 (lane / 32) .. + 7
    __device__ __forceinline__ static uint4 frag(const LDS uint4 *sm, int r0, int s, int lane)
    {
        const int r = r0 + (lane & 31);
        const u32x4 v = ((const LDS u32x4 *)sm)[r * CH + swz(2 * s + (lane >> 5), r)];
        return __builtin_bit_cast(uint4, v);
    }
};

// MN-contiguous operand tile: held as [KB][ROWS] (k-major rows of ROWS
// values), 16-byte chunks swizzled by 4 (k & 3) so the k-rows one
// transposing read touches fall in distinct banks.
template <int ROWS, int NT, int KB>
struct TileMN {
    static constexpr int CPR = ROWS / 8;
    static constexpr int NQ = KB * CPR / NT;
    static_assert(KB * CPR % NT == 0, "tile slots must divide by the thread count");
    static_assert(CPR >= 16, "the swizzle permutes 16 chunks of a row");
    // chunk swizzle of row k: the 64-byte windows of rows k = 0..3 (mod 4)
    // land on four different quarters of the 64 banks, so the 8 rows x 64
    // bytes one ds_read_b64_tr_b16 touches take the minimum two passes
    __device__ __forceinline__ static int fk(int k) { return (k & 3) << 2; }

    // columns past `extent` are clamped to its last 8 (never stored);
    // extent % 8 == 0, extent >= 8
    // k-rows at k >= kend read zeros
    __device__ __forceinline__ static void load_q(int q, const uint16_t *__restrict__ p, size_t ld, int row0,
                                                  int extent, int k0, int kend, LDS uint4 *dst, int tid)
    {
        const int lane = tid & 63, wave = tid >> 6;
        const int base = (wave * NQ + q) * 64;
        const int slot = base + lane;
        const int k = slot / CPR;
        const int logical = (slot % CPR) ^ fk(k);
        int mn = row0 + logical * 8;
        mn = mn < extent ? mn : extent - 8;
        const void *src =
            k0 + k < kend ? (const void *)(p + (size_t)(k0 + k) * ld + mn) : (const void *)&g_zero16;
        dma16(src, dst + base);
    }
    // Fast form of load q (k-tiles below kend): the scalar base is k-row
    // k0 + kq (the first k-row load q touches), column row0, and each lane's
    // offset is (its k-row - kq) ld + (its clamped column - row0), in bytes;
    // the 64 lanes span 64 / CPR <= 4 k-rows.  `wave` must be wave-uniform.
    struct Fast {
        uint32_t voff;
        int srow;
    };
    __device__ __forceinline__ static Fast fast_q(int q, size_t ld, int row0, int extent, int wave, int lane)
    {
        const int base = (wave * NQ + q) * 64;
        const int kq = base / CPR;
        const int slot = base + lane;
        const int k = slot / CPR;
        const int logical = (slot % CPR) ^ fk(k);
        int mn = row0 + logical * 8;
        mn = mn < extent ? mn : extent - 8;
        return {(uint32_t)(((size_t)(k - kq) * ld + (size_t)(mn - row0)) * 2), kq};
    }
    __device__ __forceinline__ static void load_fast(int q, const Fast &f, const uint16_t *__restrict__ p, size_t ld,
                                                     int row0, int k0, LDS uint4 *dst, int wave)
    {
        dma16s(f.voff, p + (size_t)(k0 + f.srow) * ld + row0, dst + (wave * NQ + q) * 64);
    }

    // MFMA operand fragment from two ds_read_b64_tr_b16: in 16-lane group g
    // source lane q points at [k0 + q / 4][R0 + 4 (q % 4)] and result lane i
    // holds rows R0 + i, k = k0 .. k0 + 3 (R0 = r0 + 16 (g & 1),
    // k0 = 16 s + 8 (g >> 1) + 4 h for half h)
    __device__ __forceinline__ static uint4 frag(const LDS uint4 *sm, int r0, int s, int lane)
    {
        const int g = (lane >> 4) & 3, q = lane & 15;
        const int mn = r0 + 16 * (g & 1) + 4 * (q & 3);
        uint2 h2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 16 * s + 8 * (g >> 1) + 4 * h + (q >> 2);
            const int byte = k * ROWS * 2 + (((mn >> 3) ^ fk(k)) << 4) + (mn & 7) * 2;
            h2[h] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS v4s *)((const LDS char *)sm + byte)));
        }
        return make_uint4(h2[0].x, h2[0].y, h2[1].x, h2[1].y);
    }
};

// A GEMM launch's arguments (one problem; a paired launch takes two).
struct gemm_kargs {
    const uint16_t *A;
    size_t lda, sA;
    int a_extent;
    const uint16_t *B;
    size_t ldb, sB;
    int b_extent;
    float *C;
    size_t ldc, sC;
    int M, N, K, beta, tiles_m, tiles_n;
    pgk_epi epi;
    int k_total, kz_step, fast_ok;
};

// one kernel configuration: block tile BM x BN on WGM x WGN waves, operand
// layouts TA / TB, f16 or bf16, fused epilogue, k-tile depth KB, S stages
template <int BM_, int BN_, int WGM_, int WGN_, bool TA_, bool TB_, bool F16_, bool EPI_, int KB_, int S_>
struct gcfg {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, KB = KB_, S = S_;
    static constexpr bool TA = TA_, TB = TB_, F16 = F16_, EPI = EPI_;
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int LDS_U4 = S * (BM * KB / 8 + BN * KB / 8); // uint4 of LDS
};

// One block tile of problem g: tile pid of the nb tiles of batch entry (or
// split-K slice) z, with the LDS ring at lds.  remap: block ids were dealt
// to the 8 XCDs round-robin with pid % 8 naming the XCD.
template <class CF>
__device__ __forceinline__ void gemm16_block(const gemm_kargs &g, int pid, int nb, bool remap, int z,
                                             LDS uint4 *const lds)
{
    constexpr int BM = CF::BM, BN = CF::BN, WGM = CF::WGM, WGN = CF::WGN, KB = CF::KB, S = CF::S;
    constexpr bool TA = CF::TA, TB = CF::TB, F16 = CF::F16, EPI = CF::EPI;
    const uint16_t *__restrict__ A = g.A;
    const uint16_t *__restrict__ B = g.B;
    float *__restrict__ C = g.C;
    const size_t lda = g.lda, sA = g.sA, ldb = g.ldb, sB = g.sB, ldc = g.ldc, sC = g.sC;
    const int a_extent = g.a_extent, b_extent = g.b_extent, M = g.M, N = g.N, K = g.K, beta = g.beta;
    const int tiles_m = g.tiles_m, tiles_n = g.tiles_n, k_total = g.k_total, kz_step = g.kz_step;
    const int fast_ok = g.fast_ok;
    const pgk_epi &epi = g.epi;
    constexpr int NT = 64 * WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int FM = WM / 32, FN = WN / 32;
    using OA = typename std::conditional<TA, TileMN<BM, NT, KB>, TileK<BM, NT, KB>>::type;
    using OB = typename std::conditional<TB, TileMN<BN, NT, KB>, TileK<BN, NT, KB>>::type;
    // S-stage ring of A and B tiles in one LDS block; the k-loop below is
    // unrolled by S, so every stage index is a compile-time constant
    constexpr int SA = BM * KB / 8, SB = BN * KB / 8; // uint4 per stage
    auto stA = [&](int st) { return lds + st * SA; };
    auto stB = [&](int st) { return lds + S * SA + st * SB; };

    // tile order: XCD-aware (block ids dealt round-robin to the 8 XCDs are
    // regrouped so consecutive ids share an XCD), then 8 tile-rows at a time
    if (remap && (nb & 7) == 0)
        pid = (pid & 7) * (nb >> 3) + (pid >> 3);
    const int GM = 8;
    const int per_group = GM * tiles_n;
    const int group = pid / per_group;
    const int first_m = group * GM;
    const int gsz = tiles_m - first_m < GM ? tiles_m - first_m : GM;
    const int in_group = pid - group * per_group;
    const int m0 = (first_m + in_group % gsz) * BM, n0 = (in_group / gsz) * BN;

    const uint16_t *Ab = A + (size_t)z * sA;
    const uint16_t *Bb = B + (size_t)z * sB;
    float *Cb = C + (size_t)z * sC;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.0f;

    // valid reduction length of this batch entry: K, or for split-K slice z
    // the rest of k_total from z * kz_step; the last partial tile reads
    // zeros past it (kend % 8 == 0)
    const int krem = k_total - z * kz_step;
    const int kend = krem < K ? krem : K;
    const int KT = (kend + KB - 1) / KB;
    // S-stage ring, tile t in stage t % S.  Between two barriers the
    // k-loop is straight-line code, so the compiler's LDS wait counts stay
    // exact: at a control-flow merge it falls back to waiting for every
    // outstanding LDS read, which would stall each wave on the fragment
    // reads it has just issued for the next k-step.
    //  - k-step s of a tile runs its MFMAs on the fragments read one step
    //    earlier and reads those of step s + 1 between them;
    //  - a tile's last k-step ("tail") starts with the one barrier per tile:
    //    every wave has then read the whole stage (its last fragments are in
    //    registers), so the stage is refilled with tile t + S during that
    //    step's MFMAs and the next tile's first fragments are read while
    //    they run -- the matrix units do not drain at the barrier;
    //  - a "link" is the tail of tile t and the other k-steps ("head") of
    //    tile t + 1, so each link starts at the barrier, whose explicit wait
    //    leaves no LDS read outstanding, and the branches between links
    //    (S per loop iteration, for constant stage offsets) cost no waits;
    //  - tiles 0 .. S-1 are in flight before the first tile and tile t + S
    //    is loaded during tile t's tail also when t + S >= KT: such tiles lie
    //    past kend and every chunk comes from the zero page (never read: no
    //    stage is read after the last tile).
    static_assert(S >= 2 && (KB / 16) % 2 == 0, "two or more stages, an even number of k-steps per tile");
    constexpr int LPT = OA::NQ + OB::NQ; // DMA instructions per thread per tile
    static_assert((S - 1) * LPT < 64, "the loads in flight fit the vmcnt counter");
    constexpr int KS = KB / 16, NM = FM * FN;
    const int links = KT > 1 ? KT - 1 : 0;
    auto dma = [&](int q, int t, LDS uint4 *dA, LDS uint4 *dB) {
        if (q < OA::NQ)
            OA::load_q(q, Ab, lda, m0, a_extent, t * KB, kend, dA, tid);
        else
            OB::load_q(q - OA::NQ, Bb, ldb, n0, b_extent, t * KB, kend, dB, tid);
    };
    // per-lane offsets of the fast form (tiles wholly below kend, leading
    // dims under 2^26: fast_ok), fixed for the whole k-loop
    typename OA::Fast fA[OA::NQ];
    typename OB::Fast fB[OB::NQ];
#pragma unroll
    for (int q = 0; q < OA::NQ; ++q)
        fA[q] = OA::fast_q(q, lda, m0, a_extent, wave_u, lane);
#pragma unroll
    for (int q = 0; q < OB::NQ; ++q)
        fB[q] = OB::fast_q(q, ldb, n0, b_extent, wave_u, lane);
    auto dma_fast = [&](int q, int t, LDS uint4 *dA, LDS uint4 *dB) {
        if (q < OA::NQ)
            OA::load_fast(q, fA[q], Ab, lda, m0, t * KB, dA, wave_u);
        else
            OB::load_fast(q - OA::NQ, fB[q - OA::NQ], Bb, ldb, n0, t * KB, dB, wave_u);
    };
    // a bare s_barrier after an explicit wait on this wave's loads (all but
    // the newest NEWER tiles' landed in LDS) and on its LDS reads: the
    // fence of __syncthreads() would drain every outstanding memory
    // operation; the empty asm statements keep LDS accesses from moving
    // across it
    auto sync_tile = [&](auto newer) {
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(decltype(newer)::value * LPT));
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
    };
    uint4 fa[2][FM], fb[2][FN];
    auto rd = [&](const LDS uint4 *cA, const LDS uint4 *cB, int s, uint4(&xa)[FM], uint4(&xb)[FN]) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
            xa[i] = OA::frag(cA, wm * WM + i * 32, s, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            xb[j] = OB::frag(cB, wn * WN + j * 32, s, lane);
    };
    // MFMAs of k-step s; in a tail, tile `reload` goes into stage (dA, dB),
    // a few loads per MFMA rather than one burst at the vector-memory queue,
    // in the fast form when FAST (a compile-time tag).  With `next`, the
    // fragments of k-step ns of the tile in stage (nA, nB) are read into the
    // other fragment buffer one per MFMA, so the LDS reads spread over the
    // step instead of arriving in one burst ahead of it (wgrad's
    // transposing reads, two per fragment, gain the most).  `next` is a
    // flag rather than a null test of nA: LDS address 0 is a valid stage.
    auto mfmas = [&](int s, bool tail, int reload, LDS uint4 *dA, LDS uint4 *dB, auto fast, bool next,
                     const LDS uint4 *nA, const LDS uint4 *nB, int ns) {
        // keep the reads and loads placed here in their slots between the
        // MFMAs: left alone, the scheduler sinks each read to just before
        // its first use and the LDS latency shows at every step
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                acc[i][j] = mfma32<F16>(fa[s & 1][i], fb[s & 1][j], acc[i][j]);
                if (next) {
                    const int g = i * FN + j;
                    static_assert(FM * FN >= FM + FN, "one fragment read per MFMA at most");
                    if (g < FM)
                        fa[(s + 1) & 1][g] = OA::frag(nA, wm * WM + g * 32, ns, lane);
                    else if (g < FM + FN)
                        fb[(s + 1) & 1][g - FM] = OB::frag(nB, wn * WN + (g - FM) * 32, ns, lane);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (tail) {
                    const int g = i * FN + j;
#pragma unroll
                    for (int q = g * LPT / NM; q < (g + 1) * LPT / NM; ++q) {
                        if constexpr (decltype(fast)::value)
                            dma_fast(q, reload, dA, dB);
                        else
                            dma(q, reload, dA, dB);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        __builtin_amdgcn_sched_barrier(0);
    };
    // k-steps 0 .. KS-2 of the tile in stage (cA, cB); step 0's fragments
    // are in fa[0], fb[0]
    auto head = [&](const LDS uint4 *cA, const LDS uint4 *cB) {
#pragma unroll
        for (int s = 0; s < KS - 1; ++s)
            mfmas(s, false, 0, nullptr, nullptr, std::false_type{}, true, cA, cB, s + 1);
    };
    // the tail of tile t (stage cA, cB) and the head of tile t + 1 (oA, oB)
    auto link = [&](int t, LDS uint4 *cA, LDS uint4 *cB, LDS uint4 *oA, LDS uint4 *oB, auto fast) {
        // tile t + 1 landed; tiles t + 2 .. t + S - 1 may be in flight
        sync_tile(std::integral_constant<int, S - 2>{});
        mfmas(KS - 1, true, t + S, cA, cB, fast, true, oA, oB, 0);
        head(oA, oB);
    };
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
        for (int q = 0; q < LPT; ++q)
            dma(q, t, stA(t), stB(t));
    sync_tile(std::integral_constant<int, S - 1>{}); // tile 0 landed
    rd(stA(0), stB(0), 0, fa[0], fb[0]);
    head(stA(0), stB(0));
    // link t reloads tile t + S: in the fast form while that tile lies
    // wholly below kend, for whole groups of S links (so the second loop
    // starts at stage 0), then the general form
    const int full_tiles = kend / KB;
    int fast_links = full_tiles > S ? full_tiles - S : 0;
    fast_links = fast_ok ? (fast_links < links ? fast_links : links) / S * S : 0;
    int t = 0;
    for (; t < fast_links; t += S) {
#pragma unroll
        for (int u = 0; u < S; ++u)
            link(t + u, stA(u), stB(u), stA((u + 1) % S), stB((u + 1) % S), std::true_type{});
    }
    for (; t < links; t += S) {
#pragma unroll
        for (int u = 0; u < S; ++u)
            if (t + u < links)
                link(t + u, stA(u), stB(u), stA((u + 1) % S), stB((u + 1) % S), std::false_type{});
    }
    mfmas(KS - 1, false, 0, nullptr, nullptr, std::false_type{}, false, nullptr, nullptr, 0); // the last tail
    // the loads of the tiles past the end land before the LDS is reused
    // (the epilogue's staging, or the next block on this CU)
    __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));

    // epilogue: lane holds column lane % 32 of rows (e/4)*8 + (lane/32)*4 + e%4
    const int lrow = lane & 31, lk = lane >> 5;
    if constexpr (EPI) {
        // Through LDS, 32 rows of the wave's WM x WN tile at a time: the
        // accumulators land row-major in a per-wave [32][WN + 8] f32 region
        // (in the operand stages, free after the k-loop) and come back as
        // float4 along a row, so bias, activation and the three stores (out,
        // pre-activation, 16-bit out) run 4 columns per lane with 16-byte
        // (8-byte for 16-bit) stores.  Every index into acc stays static.
        static_assert(WN == 64, "one lane group of 16 x 4 columns per row");
        constexpr int RS = WN + 8;
        static_assert(WGM * WGN * 32 * RS * 4 <= S * (SA + SB) * 16, "epilogue regions fit the stages");
        LDS float *reg = (LDS float *)((LDS char *)lds + wave * (32 * RS * 4));
        const int c4 = (lane & 15) * 4;
        const int gcol = n0 + wn * WN + c4;
        float bias4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            bias4[q] = (epi.bias && gcol + q < N) ? epi.bias[gcol + q] : 0.0f;
        const bool v4 = (ldc & 3) == 0 && gcol + 3 < N && (((uintptr_t)Cb) & 15) == 0 &&
                        (((uintptr_t)epi.z) & 15) == 0 && (((uintptr_t)epi.c16) & 7) == 0;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            __syncthreads(); // the k-loop's (or the previous pass') LDS reads are done
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    reg[((e >> 2) * 8 + lk * 4 + (e & 3)) * RS + j * 32 + lrow] = acc[i][j][e];
            __syncthreads();
            for (int t = 0; t < 8; ++t) {
                const int row = (lane >> 4) + 4 * t;
                const int grow = m0 + wm * WM + i * 32 + row;
                if (grow >= M || gcol >= N)
                    continue;
                const f32x4 a4 = *(const LDS f32x4 *)(reg + row * RS + c4);
                const float zv[4] = {a4[0] + bias4[0], a4[1] + bias4[1], a4[2] + bias4[2], a4[3] + bias4[3]};
                float o[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    o[q] = act_f(epi.act, zv[q]);
                const size_t off = (size_t)grow * ldc + gcol;
                if (v4) {
                    if (!epi.skip_out)
                        *reinterpret_cast<float4 *>(Cb + off) = make_float4(o[0], o[1], o[2], o[3]);
                    if (epi.z) { // read again only by the backward, much later
                        const f32x4 zz = {zv[0], zv[1], zv[2], zv[3]};
                        __builtin_nontemporal_store(zz, reinterpret_cast<f32x4 *>(epi.z + off));
                    }
                    if (epi.c16)
                        *reinterpret_cast<uint2 *>(epi.c16 + off) =
                            make_uint2(to16x2(epi.dtype16, o[0], o[1]), to16x2(epi.dtype16, o[2], o[3]));
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (gcol + q >= N)
                            break;
                        if (!epi.skip_out)
                            Cb[off + q] = o[q];
                        if (epi.z)
                            epi.z[off + q] = zv[q];
                        if (epi.c16)
                            epi.c16[off + q] = to16(epi.dtype16, o[q]);
                    }
                }
            }
        }
    } else {
        // dgrad and wgrad outputs take non-temporal stores: the write burst
        // passes the caches by (config 3's GEMM pair 213 -> 210 us and the
        // cast pass after it faster, config 5 +1.6 %); a forward product
        // (A K-contiguous, B MN-contiguous) keeps ordinary stores, as the
        // next kernel reads it (config 5's unfused graph +1.3 %)
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
                        if constexpr (!TA && TB)
                            *p = beta ? *p + acc[i][j][e] : acc[i][j][e];
                        else
                            __builtin_nontemporal_store(beta ? *p + acc[i][j][e] : acc[i][j][e], p);
                    }
                }
            }
        }
    }
}

template <class CF>
__global__ void __launch_bounds__(CF::NT, 1) k_gemm16(gemm_kargs g)
{
    __shared__ uint4 smem[CF::LDS_U4];
    gemm16_block<CF>(g, (int)blockIdx.x, (int)gridDim.x, true, (int)blockIdx.z, (LDS uint4 *)smem);
}

// Two problems in one launch (the dgrad and wgrad of one matmul when each
// alone leaves CUs idle): blocks [0, n1) take problem 1 (tile b % nb1 of
// slice / batch entry b / nb1), the rest problem 2; one LDS ring, sized for
// the larger configuration.  Both configurations have the same thread
// count.  Problem 2's tiles are regrouped by XCD only when n1 % 8 == 0.
template <class C1, class C2>
__global__ void __launch_bounds__(C1::NT, 1) k_gemm16_pair(gemm_kargs g1, gemm_kargs g2, int nb1, int n1, int nb2)
{
    static_assert(C1::NT == C2::NT, "one block size");
    __shared__ uint4 smem[C1::LDS_U4 > C2::LDS_U4 ? C1::LDS_U4 : C2::LDS_U4];
    const int b = (int)blockIdx.x;
    if (b < n1)
        gemm16_block<C1>(g1, b % nb1, nb1, true, b / nb1, (LDS uint4 *)smem);
    else
        gemm16_block<C2>(g2, (b - n1) % nb2, nb2, (n1 & 7) == 0, (b - n1) / nb2, (LDS uint4 *)smem);
}

// the epilogue of one element: C = act(v + bias), the pre-activation and
// the 16-bit copy beside it (gemm16_block's EPI path applies it from LDS)
__device__ __forceinline__ void epi_store(const pgk_epi &epi, float *c, size_t off, int col, float v)
{
    const float zv = v + (epi.bias ? epi.bias[col] : 0.0f);
    const float o = act_f(epi.act, zv);
    if (!epi.skip_out)
        c[off] = o;
    if (epi.z)
        epi.z[off] = zv;
    if (epi.c16)
        epi.c16[off] = to16(epi.dtype16, o);
}

// Skinny product: C[m, n] (+)= A . B for n <= 16 with B MN-contiguous
// (b[p * ldb + j]), A K-contiguous (TA false: the forward x . W of a narrow
// layer) or MN-contiguous (TA true: a narrow layer's weight grad x^T . dz).
// Such a product streams A once, so split-K's partials and summing launch
// dominated it.  A block owns 16 rows of C (256 blocks for 4096 rows: every
// CU streams) and its eight waves split the reduction into runs of 64-deep
// chunks, each wave with a three-stage ring of its own in LDS (no block
// barrier in the k-loop: a wave waits only on its own loads; two chunks
// ahead measured faster than four).  The 32 x 32 x 16 MFMA holds the 16 rows and 16
// columns in a quarter of its outputs: its other rows and columns read
// duplicates or zeros and are never stored.  The waves' partial products
// are added through LDS in wave order, then each element goes through the
// plain store (beta) or the forward epilogue.
constexpr int kSkWaves = 8, kSkStages = 3, kSkRows = 16;
constexpr int kSkA = kSkRows * 64 / 8, kSkB = 64 * 16 / 8; // uint4 of one A and one B stage

template <bool TA, bool F16>
__global__ void __launch_bounds__(kSkWaves * 64, 1)
    k_skinny(const uint16_t *__restrict__ A, size_t lda, int a_extent, const uint16_t *__restrict__ B, size_t ldb,
             int b_extent, float *__restrict__ C, size_t ldc, int m, int n, int k, int beta, pgk_epi epi, int has_epi)
{
    __shared__ uint4 smem[kSkWaves * kSkStages * (kSkA + kSkB)];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // consecutive row tiles on one XCD: with A MN-contiguous four tiles
    // share each 128-byte line of a row
    int pid = (int)blockIdx.x;
    const int nb = (int)gridDim.x;
    if ((nb & 7) == 0)
        pid = (pid & 7) * (nb >> 3) + (pid >> 3);
    const int r0 = pid * kSkRows;
    LDS uint4 *const ring = (LDS uint4 *)smem + wave * kSkStages * (kSkA + kSkB);
    // this wave's run of chunks; loads at k >= kend read the zero page
    const int nct = (k + 63) / 64, cpw = (nct + kSkWaves - 1) / kSkWaves, c0 = wave * cpw;
    const int nc = nct - c0 < cpw ? (nct - c0 > 0 ? nct - c0 : 0) : cpw;
    const int kend = (c0 + nc) * 64 < k ? (c0 + nc) * 64 : k;
    using TK = TileK<kSkRows, 64, 64>;
    static_assert(TK::NQ == 2, "two loads of 8 rows x 128 bytes per A stage");
    constexpr int LPT = 4; // loads per chunk: two of A, two of B
    auto load = [&](int c, int st) {
        LDS uint4 *sa = ring + st * (kSkA + kSkB), *sb = sa + kSkA;
        const int k0 = (c0 + c) * 64;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if constexpr (!TA) {
                TK::load_q(q, A, lda, r0, a_extent, k0, kend, sa, lane);
            } else {
                // [64 p][16 i]: two 16-byte chunks per p-row
                const int slot = q * 64 + lane, p = slot >> 1;
                int i = r0 + (slot & 1) * 8;
                i = i < a_extent ? i : a_extent - 8;
                const void *src = k0 + p < kend ? (const void *)(A + (size_t)(k0 + p) * lda + i) : (const void *)&g_zero16;
                dma16(src, sa + q * 64);
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            // [64 p][16 j]: two 16-byte chunks per p-row
            const int slot = q * 64 + lane, p = slot >> 1, j = (slot & 1) * 8;
            const void *src =
                k0 + p < kend && j < b_extent ? (const void *)(B + (size_t)(k0 + p) * ldb + j) : (const void *)&g_zero16;
            dma16(src, sb + q * 64);
        }
    };
    // ds_read_b64_tr_b16 pair over a [64][16] tile (32-byte rows): in 16-lane
    // group g, source lane q points at [k0 + q / 4][4 (q % 4)] and result lane
    // i holds column i, k = k0 .. k0 + 7 (k0 = 16 s + 8 (g >> 1))
    auto tr_frag = [&](const LDS uint4 *st, int s) {
        const int g = (lane >> 4) & 3, q = lane & 15;
        uint2 h2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = 16 * s + 8 * (g >> 1) + 4 * h + (q >> 2);
            h2[h] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS v4s *)((const LDS char *)st + p * 32 + (q & 3) * 8)));
        }
        return make_uint4(h2[0].x, h2[0].y, h2[1].x, h2[1].y);
    };
    // lanes of B columns 0 .. 15 (the rest hold columns 16 .. 31: zero)
    const bool bcol = ((lane >> 4) & 1) == 0;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e)
        acc[e] = 0.0f;
    if (nc > 0) {
#pragma unroll
        for (int s = 0; s < kSkStages; ++s)
            load(s, s);
        for (int c = 0; c < nc; ++c) {
            const int st = c % kSkStages;
            const LDS uint4 *sa = ring + st * (kSkA + kSkB), *sb = sa + kSkA;
            // chunk c landed (the newest kSkStages - 1 chunks may be in flight)
            __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm((kSkStages - 1) * LPT));
            __asm__ volatile("" ::: "memory");
            uint4 af[4], bf[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if constexpr (!TA) {
                    // rows lane % 16 (lanes 16 .. 31 of each half repeat them)
                    const int r = lane & 15;
                    const u32x4 v = ((const LDS u32x4 *)sa)[r * TK::CH + TK::swz(2 * s + (lane >> 5), r)];
                    af[s] = __builtin_bit_cast(uint4, v);
                } else {
                    af[s] = tr_frag(sa, s);
                }
                const uint4 b = tr_frag(sb, s);
                bf[s] = bcol ? b : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc = mfma32<F16>(af[s], bf[s], acc);
            // the stage's reads are done before its refill
            __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(63));
            __asm__ volatile("" ::: "memory");
            load(c + kSkStages, st);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));
    }
    // the waves' partials through LDS (the rings are done), added in wave
    // order; output rows 8 (e / 4) + 4 (lane / 32) + e % 4 < 16 are e < 8
    __syncthreads();
    constexpr int RP = 17;
    LDS float *red = (LDS float *)smem;
    static_assert(kSkWaves * kSkRows * RP * 4 <= (int)sizeof(smem), "partials fit the rings");
    const int col = lane & 31, lk = lane >> 5;
    if (col < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            red[(wave * kSkRows + (e >> 2) * 8 + lk * 4 + (e & 3)) * RP + col] = acc[e];
    }
    __syncthreads();
    static_assert(kSkWaves * 64 >= kSkRows * 16, "a thread per element of the block's rows");
    const int t = (int)threadIdx.x, row = t >> 4, j = t & 15, gr = r0 + row;
    if (row < kSkRows && gr < m && j < n) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kSkWaves; ++w)
            v += red[(w * kSkRows + row) * RP + j];
        const size_t off = (size_t)gr * ldc + j;
        if (has_epi)
            epi_store(epi, C, off, j, v);
        else
            C[off] = beta ? C[off] + v : v;
    }
}

// the same epilogue as a pass over a finished C (k-tail runs)
__global__ void __launch_bounds__(256) k_bias_act(float *__restrict__ c, size_t ldc, int m, int n, pgk_epi epi)
{
    const size_t mn = (size_t)m * n;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / n, col = i - r * n, off = r * ldc + col;
        epi_store(epi, c, off, (int)col, c[off]);
    }
}

// zero-padded copy of the k-slab [k0, k0 + kn) of an operand, kn <= 64:
// K-contiguous -> dst[r * 64 + c], MN-contiguous -> dst[c * rows_pad + r]
__global__ void __launch_bounds__(256) k_pack_slab(int mn_major, const uint16_t *__restrict__ src, size_t ld,
                                                   size_t sstride, int rows, int rows_pad, int k0, int kn,
                                                   uint16_t *__restrict__ dst, size_t dstride)
{
    const uint16_t *s = src + (size_t)blockIdx.z * sstride;
    uint16_t *d = dst + (size_t)blockIdx.z * dstride;
    const size_t total = (size_t)rows_pad * 64;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        int r, c;
        if (mn_major) {
            c = (int)(i / rows_pad);
            r = (int)(i % rows_pad);
        } else {
            r = (int)(i / 64);
            c = (int)(i % 64);
        }
        uint16_t v = 0;
        if (r < rows && c < kn)
            v = mn_major ? s[(size_t)(k0 + c) * ld + r] : s[(size_t)r * ld + k0 + c];
        d[i] = v;
    }
}

// split-K finish of up to two problems (grid z picks one; a problem with
// splits = 0 is absent): C = (beta ? C : 0) + sum over the `splits` partial
// products (each m x n, dense), added in split order, then with `epi` the
// GEMM's epilogue on that value (k_bias_act's arithmetic, in the same
// pass).  With n and ldc allowing 16-byte accesses, rows run along grid y
// (stride gridDim.y) and columns along x, four per thread; otherwise
// (narrow outputs such as n = 10) one element per thread over the
// flattened m x n, indexed with a 32-bit division when m n fits
struct splitk_desc {
    const float *part;
    int splits, m, n;
    float *c;
    size_t ldc;
    int beta, v4, has_epi;
    pgk_epi epi;
};

splitk_desc splitk_of(const float *part, int splits, size_t m, size_t n, float *c, size_t ldc, int beta,
                      const pgk_epi *epi = nullptr)
{
    int v4 = ((n | (ldc & 3)) & 3) == 0 && (((uintptr_t)c | (uintptr_t)part) & 15) == 0;
    if (epi)
        v4 = v4 && ((((uintptr_t)epi->z) | ((uintptr_t)epi->bias)) & 15) == 0 && (((uintptr_t)epi->c16) & 7) == 0;
    return splitk_desc{part, splits, (int)m, (int)n, c, ldc, beta, v4, epi != nullptr, epi ? *epi : pgk_epi{}};
}

dim3 splitk_grid(const splitk_desc &a, const splitk_desc &b)
{
    unsigned gx = 1, gy = 1;
    for (const splitk_desc *d : {&a, &b}) {
        if (!d->splits)
            continue;
        const size_t mn = (size_t)d->m * d->n;
        const unsigned x = d->v4 ? (unsigned)((d->n / 4 + 255) / 256) : (unsigned)((mn + 255) / 256 < 2048 ? (mn + 255) / 256 : 2048);
        const unsigned y = d->v4 ? (unsigned)(d->m < 65535 ? d->m : 65535) : 1u;
        gx = x > gx ? x : gx;
        gy = y > gy ? y : gy;
    }
    return dim3(gx, gy, &a == &b || !b.splits ? 1u : 2u);
}

__global__ void __launch_bounds__(256) k_splitk_sum(splitk_desc d0, splitk_desc d1)
{
    const splitk_desc &d = blockIdx.z ? d1 : d0;
    if (!d.splits)
        return;
    const float *__restrict__ part = d.part;
    float *__restrict__ c = d.c;
    const int m = d.m, n = d.n, splits = d.splits, beta = d.beta;
    const size_t ldc = d.ldc;
    const size_t mn = (size_t)m * n;
    if (d.v4) {
        const int j = blockIdx.x * blockDim.x + threadIdx.x;
        if (j >= n >> 2)
            return;
        for (int r = blockIdx.y; r < m; r += gridDim.y) {
            const float *p = part + (size_t)r * n + 4 * j;
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int z = 0; z < splits; ++z)
                acc += __builtin_nontemporal_load((const f32x4 *)(p + (size_t)z * mn)); // read once
            f32x4 *q = (f32x4 *)(c + (size_t)r * ldc + 4 * j);
            const f32x4 v = beta ? *q + acc : acc;
            if (!d.has_epi) {
                *q = v;
                continue;
            }
            const pgk_epi &epi = d.epi;
            const size_t off = (size_t)r * ldc + 4 * j;
            f32x4 zv = v, o;
            if (epi.bias)
                zv += *(const f32x4 *)(epi.bias + 4 * j);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = act_f(epi.act, zv[e]);
            if (!epi.skip_out)
                *q = o;
            if (epi.z)
                *(f32x4 *)(epi.z + off) = zv;
            if (epi.c16)
                *(uint2 *)(epi.c16 + off) = make_uint2(to16x2(epi.dtype16, o[0], o[1]), to16x2(epi.dtype16, o[2], o[3]));
        }
        return;
    }
    if (blockIdx.y)
        return;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += (size_t)gridDim.x * blockDim.x) {
        size_t r, col;
        if (mn <= 0xffffffffu) {
            r = (uint32_t)i / (uint32_t)n;
            col = (uint32_t)i - (uint32_t)r * (uint32_t)n;
        } else {
            r = i / n;
            col = i - r * n;
        }
        float acc = 0.0f;
        for (int z = 0; z < splits; ++z)
            acc += part[(size_t)z * mn + i];
        const size_t off = r * ldc + col;
        const float v = beta ? c[off] + acc : acc;
        if (d.has_epi)
            epi_store(d.epi, c, off, (int)col, v);
        else
            c[off] = v;
    }
}

// C rows of an empty reduction: zeros
__global__ void __launch_bounds__(256) k_zero_rows(float *__restrict__ c, size_t ldc, size_t sc, int m, int n)
{
    float *cb = c + (size_t)blockIdx.z * sc;
    const size_t mn = (size_t)m * n;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / n, col = i - r * n;
        cb[r * ldc + col] = 0.0f;
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

struct gemm_args {
    const uint16_t *a;
    size_t lda, sa;
    int a_extent;
    const uint16_t *b;
    size_t ldb, sb;
    int b_extent;
    float *c;
    size_t ldc, sc;
    int m, n, k, beta;
    unsigned batch;
    int tile = 0;     // 2: 256 x 256 tiles, 1: 128 x 128, 0: by tile count
    // split-K: slice z reduces [z kz_step, min(k_total, (z+1) kz_step));
    // k_total = 0: no split
    int k_total = 0, kz_step = 0;
};

template <class CF>
gemm_kargs make_kargs(const gemm_args &g, const pgk_epi &epi)
{
    gemm_kargs k;
    k.A = g.a, k.lda = g.lda, k.sA = g.sa, k.a_extent = g.a_extent;
    k.B = g.b, k.ldb = g.ldb, k.sB = g.sb, k.b_extent = g.b_extent;
    k.C = g.c, k.ldc = g.ldc, k.sC = g.sc;
    k.M = g.m, k.N = g.n, k.K = g.k, k.beta = g.beta;
    k.tiles_m = (g.m + CF::BM - 1) / CF::BM, k.tiles_n = (g.n + CF::BN - 1) / CF::BN;
    k.epi = epi;
    k.k_total = g.k_total ? g.k_total : g.k, k.kz_step = g.kz_step;
    k.fast_ok = (int)(g.lda < ((size_t)1 << 26) && g.ldb < ((size_t)1 << 26));
    return k;
}

template <int BM, int BN, int WGM, int WGN, bool TA, bool TB, bool F16, bool EPI, int KB = 64, int S = 2>
int launch_tile(const gemm_args &g, const pgk_epi &epi, hipStream_t s)
{
    using CF = gcfg<BM, BN, WGM, WGN, TA, TB, F16, EPI, KB, S>;
    const gemm_kargs k = make_kargs<CF>(g, epi);
    hipLaunchKernelGGL(k_gemm16<CF>, dim3((unsigned)(k.tiles_m * k.tiles_n), 1, g.batch), dim3(CF::NT), 0, s, k);
    return (int)hipGetLastError();
}

// The configurations launch_layout picks from (the planner's tile ids):
//  - 2: 256 x 256 tiles, eight waves of 128 x 64; k-tiles of 32 in a
//    four-stage ring (128 KiB of LDS), except with both operands
//    K-contiguous: there a k-tile of 32 covers half of each 128-byte row
//    segment per load, and k-tiles of 64 in two stages measure faster;
//  - 3: 128 x 256 tiles, eight waves of 64 x 64: twice the tiles of 2 for
//    grids 2 leaves short of the chip, without split-K's partials; k-tiles
//    of 64 in three stages (144 KiB) with both operands K-contiguous, else
//    of 32 in four stages (96 KiB);
//  - 1: 128 x 128 tiles, four waves of 64 x 64; k-tiles of 64, two stages.
// An unplanned launch (tile 0) takes 2 when that still gives most CUs a
// tile, else 1.
inline int tile_of(const gemm_args &g)
{
    if (g.tile)
        return g.tile;
    const size_t big = (size_t)((g.m + 255) / 256) * ((g.n + 255) / 256) * g.batch;
    return big >= 128 ? 2 : 1;
}

template <bool TA, bool TB, bool F16, bool EPI, int TILE>
using layout_cfg = typename std::conditional<
    TILE == 2,
    typename std::conditional<!TA && !TB, gcfg<256, 256, 2, 4, TA, TB, F16, EPI, 64, 2>,
                              gcfg<256, 256, 2, 4, TA, TB, F16, EPI, 32, 4>>::type,
    typename std::conditional<
        TILE == 3,
        typename std::conditional<!TA && !TB, gcfg<128, 256, 2, 4, TA, TB, F16, EPI, 64, 3>,
                                  gcfg<128, 256, 2, 4, TA, TB, F16, EPI, 32, 4>>::type,
        gcfg<128, 128, 2, 2, TA, TB, F16, EPI, 64, 2>>::type>::type;

template <class CF>
int launch_cfg(const gemm_args &g, const pgk_epi &epi, hipStream_t s)
{
    return launch_tile<CF::BM, CF::BN, CF::WGM, CF::WGN, CF::TA, CF::TB, CF::F16, CF::EPI, CF::KB, CF::S>(g, epi, s);
}

template <bool TA, bool TB, bool F16, bool EPI = false>
int launch_layout(const gemm_args &g, hipStream_t s, const pgk_epi &epi = pgk_epi{})
{
    switch (tile_of(g)) {
    case 2: return launch_cfg<layout_cfg<TA, TB, F16, EPI, 2>>(g, epi, s);
    case 3: return launch_cfg<layout_cfg<TA, TB, F16, EPI, 3>>(g, epi, s);
    default: return launch_cfg<layout_cfg<TA, TB, F16, EPI, 1>>(g, epi, s);
    }
}

// dgrad (both operands K-contiguous, tile TD) and wgrad (both MN-contiguous,
// tile TW) of one matmul in one launch
template <bool F16, int TD, int TW>
int launch_pair_dw(const gemm_args &gd, const gemm_args &gw, hipStream_t s)
{
    using CD = layout_cfg<false, false, F16, false, TD>;
    using CW = layout_cfg<true, true, F16, false, TW>;
    const gemm_kargs kd = make_kargs<CD>(gd, pgk_epi{}), kw = make_kargs<CW>(gw, pgk_epi{});
    const int nb1 = kd.tiles_m * kd.tiles_n, nb2 = kw.tiles_m * kw.tiles_n;
    const int n1 = nb1 * (int)gd.batch, n2 = nb2 * (int)gw.batch;
    hipLaunchKernelGGL((k_gemm16_pair<CD, CW>), dim3((unsigned)(n1 + n2)), dim3(CD::NT), 0, s, kd, kw, nb1, n1, nb2);
    return (int)hipGetLastError();
}

// both problems on tile `tile`
template <bool F16>
int launch_pair_tiles(int tile, const gemm_args &gd, const gemm_args &gw, hipStream_t s)
{
    switch (tile) {
    case 2: return launch_pair_dw<F16, 2, 2>(gd, gw, s);
    case 3: return launch_pair_dw<F16, 3, 3>(gd, gw, s);
    default: return launch_pair_dw<F16, 1, 1>(gd, gw, s);
    }
}

int launch_any(int f16, int ta, int tb, const gemm_args &g, hipStream_t s)
{
    const int sel = (f16 ? 4 : 0) | (ta ? 2 : 0) | (tb ? 1 : 0);
    switch (sel) {
    case 0: return launch_layout<false, false, false>(g, s);
    case 1: return launch_layout<false, true, false>(g, s);
    case 2: return launch_layout<true, false, false>(g, s);
    case 3: return launch_layout<true, true, false>(g, s);
    case 4: return launch_layout<false, false, true>(g, s);
    case 5: return launch_layout<false, true, true>(g, s);
    case 6: return launch_layout<true, false, true>(g, s);
    default: return launch_layout<true, true, true>(g, s);
    }
}

// ---------------------------------------------------------------- MFMA probe
// The attainable MFMA rate of this chip, for the roofline: eight waves per
// CU run back-to-back v_mfma_f32_32x32x16_bf16 on 4 x 2 fragment tiles,
// either from registers (lds = 0) or read from LDS one k-step ahead as the
// GEMM's inner loop does (lds = 1).  The operands are bf16 values of
// magnitude 0.5 .. 2 with pseudo-random signs and mantissas: the matrix
// units draw more power, and the chip clocks lower, on such data than on
// constant patterns.
__global__ void __launch_bounds__(512, 1) k_mfma_probe(float *sink, int iters, int lds)
{
    __shared__ uint4 sm[8192];
    for (int i = threadIdx.x; i < 8192; i += blockDim.x) {
        uint32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t h = (uint32_t)(i * 4 + q + 1) * 2654435761u;
            h ^= h >> 15;
            h *= 2246822519u;
            h ^= h >> 13;
            const uint32_t lo = (h & 0x7Fu) | ((h >> 9) & 1u ? 0x3F80u : 0x3F00u) | ((h & 0x100u) << 7);
            const uint32_t hi = ((h >> 16) & 0x7Fu) | ((h >> 25) & 1u ? 0x3F80u : 0x3F00u) | ((h >> 9) & 0x8000u);
            v[q] = lo | (hi << 16);
        }
        sm[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.0f;
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint4 fa[2][4], fb[2][2];
    auto rd = [&](int it, uint4(&xa)[4], uint4(&xb)[2]) {
        const int base = lds ? (it & 7) * 512 : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            xa[i] = sm[((w * 8 + i) * 64 + l + base) & 8191];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            xb[j] = sm[((w * 8 + 4 + j) * 64 + l + base) & 8191];
    };
    rd(0, fa[0], fb[0]);
    rd(1, fa[1], fb[1]);
    for (int it = 0; it < iters; it += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (lds)
                rd(it + u + 2, fa[u ^ 1], fb[u ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = mfma32<false>(fa[u][i], fb[u][j], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                sum += acc[i][j][e];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

} // namespace


// Launch plan of one GEMM: the tile (256 x 256 with eight waves, or
// 128 x 128 with four) and a split-K factor, from a small cost model of
// this chip.  A launch takes ceil(blocks / 256 CUs) rounds of one block's
// time, that block running at the per-CU rate measured for its tile
// (~4.4 and ~2.6 TFLOP/s); split-K (slices of the reduction run as a
// batch into dense partials that k_splitk_sum adds in slice order, so the
// result is deterministic) adds a pass over sp + 1 copies of C at ~5 TB/s.
// Ragged shapes such as M = 4097 (33 rows of 128-tiles) and weight grads
// with a short output dim are where it matters.
typedef struct {
    int tile; // 2 = 256 x 256, 3 = 128 x 256, 1 = 128 x 128
    int sp;   // split-K factor, 1 = none
} gemm_plan;

// `cu_budget` is the number of CUs the launch may occupy (another launch
// runs beside it on the rest), 0 for the whole chip.
static constexpr int kCUs = 256;

// Time model: rounds of one block per CU, each block at its tile's rate
// per CU (measured under a loaded chip), plus for a split its partials:
// the slices write sp - 1 more tiles of C than one launch would, the sum
// reads sp and writes one, at ~5 TB/s, and one more launch.  A split must
// still win by 8 % over the best plan without one: its partials also cost
// HBM capacity.
static gemm_plan plan_gemm(size_t m, size_t n, size_t kin, size_t batch, int cu_budget = 0, double *time = nullptr)
{
    const double cus = cu_budget > 0 && cu_budget < kCUs ? (double)cu_budget : (double)kCUs;
    struct shape {
        int tile;
        size_t bm, bn;
        double rate;
    };
    static const shape shapes[3] = {{2, 256, 256, 4.4e12}, {3, 128, 256, 3.75e12}, {1, 128, 128, 2.0e12}};
    const double bw = 5.0e12, launch = 5e-6;
    gemm_plan best = {2, 1};
    double best_t = 1e300;
    for (const shape &sh : shapes) {
        const size_t tiles = ((m + sh.bm - 1) / sh.bm) * ((n + sh.bn - 1) / sh.bn) * batch;
        const int max_sp = batch == 1 && kin >= 1024 ? 8 : 1;
        for (int sp = 1; sp <= max_sp; ++sp) {
            const size_t ks = ((kin + sp - 1) / sp + BK - 1) / BK * BK;
            if (sp > 1 && ks * (size_t)(sp - 1) >= kin)
                break; // the last slice would be empty
            const double rounds = ceil((double)(tiles * sp) / cus);
            double t = rounds * 2.0 * (double)sh.bm * (double)sh.bn * (double)(sp > 1 ? ks : kin) / sh.rate;
            if (sp > 1)
                t += 2.0 * (double)sp * (double)m * (double)n * 4.0 / bw + launch;
            if (t < best_t * (sp > 1 && best.sp == 1 ? 0.92 : 1.0)) {
                best_t = t;
                best.tile = sh.tile;
                best.sp = sp;
            }
        }
    }
    if (time)
        *time = best_t;
    return best;
}

// the k the main kernel covers: all of it when both operands are
// MN-contiguous (a partial last k-tile reads zero rows past k) or k % 8 == 0
// (zero chunks past k), else the 64-aligned part, the rest going through
// zero-padded slabs in one more launch
static size_t k_inkernel(int ta, int tb, size_t k) { return (ta && tb) || k % 8 == 0 ? k : k - k % BK; }

// k_skinny's products: at most 16 columns of C from an MN-contiguous B, one
// problem, a reduction it covers whole (any k with both operands
// MN-contiguous, k % 8 == 0 with A K-contiguous), and rows enough for 64 of
// its 16-row blocks; the rest keep the tiled plans (split-K among them)
static bool skinny_ok(int ta, int tb, size_t m, size_t n, size_t k, size_t batch)
{
    return tb && n <= 16 && batch == 1 && k && (ta || k % 8 == 0) && (m + 15) / 16 >= 64;
}

static size_t tail_ws(int ta, int tb, size_t m, size_t n, size_t k, size_t batch)
{
    if (k_inkernel(ta, tb, k) == k)
        return 0;
    const size_t ma = (m + 7) & ~(size_t)7, nb = (n + 7) & ~(size_t)7;
    const size_t a = (ta ? 64 * (ma < 8 ? 8 : ma) : 64 * m) * batch;
    const size_t b = (tb ? 64 * (nb < 8 ? 8 : nb) : 64 * n) * batch;
    return (a + 64 + b) * sizeof(uint16_t);
}

// the checks of pgk_gemm16_cu's operands
int check_gemm_args(int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, size_t stride_a,
                    size_t a_extent, const uint16_t *b, size_t ldb, size_t stride_b, size_t b_extent, size_t batch)
{
    // k leaves headroom for the k offsets of the tiles the kernel loads
    // past the end (from the zero page) to stay within int
    if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fff0000 || batch > 65535)
        return (int)hipErrorInvalidValue;
    // 16-byte global loads: aligned bases, leading dims and batch strides
    if ((((uintptr_t)a | (uintptr_t)b) & 15) || (lda & 7) || (ldb & 7) || (stride_a & 7) || (stride_b & 7))
        return (int)hipErrorInvalidValue;
    // the clamped loads stay inside [0, extent) of each operand
    if (!a_extent || !b_extent || (ta && ((a_extent & 7) || a_extent < m)) || (tb && ((b_extent & 7) || b_extent < n)) ||
        (!ta && a_extent < m) || (!tb && b_extent < n) || a_extent > 0x7fffffff || b_extent > 0x7fffffff)
        return (int)hipErrorInvalidValue;
    return 0;
}

extern "C" size_t pgk_gemm16_workspace_cu(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget)
{
    if (skinny_ok(ta, tb, m, n, k, batch))
        return 0;
    const gemm_plan pl = plan_gemm(m, n, k_inkernel(ta, tb, k), batch, cu_budget);
    const size_t part = pl.sp > 1 ? (((size_t)pl.sp * m * n * sizeof(float) + 255) & ~(size_t)255) : 0;
    return part + tail_ws(ta, tb, m, n, k, batch);
}

extern "C" size_t pgk_gemm16_workspace(int ta, int tb, size_t m, size_t n, size_t k, size_t batch)
{
    return pgk_gemm16_workspace_cu(ta, tb, m, n, k, batch, 0);
}

extern "C" int pgk_gemm16_plan(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget, int *splits)
{
    if (skinny_ok(ta, tb, m, n, k, batch)) {
        if (splits)
            *splits = 1;
        return 4;
    }
    const gemm_plan pl = plan_gemm(m, n, k_inkernel(ta, tb, k), batch, cu_budget);
    if (splits)
        *splits = pl.sp;
    return pl.tile;
}

extern "C" double pgk_gemm16_time(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget)
{
    if (skinny_ok(ta, tb, m, n, k, batch)) // A streamed once at ~5 TB/s, one launch
        return (double)(m * k * 2 + k * 32 + m * n * 4) / 5.0e12 + 5e-6;
    double t = 0.0;
    plan_gemm(m, n, k_inkernel(ta, tb, k), batch, cu_budget, &t);
    return t;
}

extern "C" int pgk_gemm16(int dtype, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda,
                          size_t stride_a, size_t a_extent, const uint16_t *b, size_t ldb, size_t stride_b,
                          size_t b_extent, float *c, size_t ldc, size_t stride_c, size_t batch, int beta,
                          const pgk_epi *epi, void *ws, pgk_stream s)
{
    return pgk_gemm16_cu(dtype, ta, tb, m, n, k, a, lda, stride_a, a_extent, b, ldb, stride_b, b_extent, c, ldc,
                         stride_c, batch, beta, epi, ws, 0, s);
}

extern "C" int pgk_gemm16_cu(int dtype, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda,
                             size_t stride_a, size_t a_extent, const uint16_t *b, size_t ldb, size_t stride_b,
                             size_t b_extent, float *c, size_t ldc, size_t stride_c, size_t batch, int beta,
                             const pgk_epi *epi, void *ws, int cu_budget, pgk_stream s)
{
    if (!m || !n || !batch)
        return 0;
    const bool has_epi = epi && (epi->bias || epi->act != PGK_ACT_NONE || epi->z || epi->c16);
    if (has_epi && (beta || batch != 1 || (epi->c16 && epi->dtype16 != 1 && epi->dtype16 != 2)))
        return (int)hipErrorInvalidValue;
    // an unwritten C needs the epilogue on the GEMM or the split-K sum: the
    // k-tail and empty-k paths apply it over C's accumulated values
    if (has_epi && epi->skip_out && (!k || k_inkernel(ta, tb, k) != k))
        return (int)hipErrorInvalidValue;
    const int bad = check_gemm_args(ta, tb, m, n, k, a, lda, stride_a, a_extent, b, ldb, stride_b, b_extent, batch);
    if (bad)
        return bad;
    hipStream_t st = (hipStream_t)s;
    const int f16 = dtype == 1;
    const size_t kmain = k_inkernel(ta, tb, k), ktail = k - kmain;
    const size_t mn = m * n;
    const unsigned gmn = (unsigned)((mn + 255) / 256 < 2048 ? (mn + 255) / 256 : 2048);
    if (!k) { // empty reduction: C = beta ? C : 0
        if (!beta)
            hipLaunchKernelGGL(k_zero_rows, dim3(gmn, 1, (unsigned)batch), dim3(256), 0, st, c, ldc, stride_c,
                               (int)m, (int)n);
        if (has_epi)
            hipLaunchKernelGGL(k_bias_act, dim3(gmn), dim3(256), 0, st, c, ldc, (int)m, (int)n, *epi);
        return (int)hipGetLastError();
    }
    if (skinny_ok(ta, tb, m, n, k, batch)) {
        const dim3 grid((unsigned)((m + 15) / 16));
        const pgk_epi e = has_epi ? *epi : pgk_epi{};
        const int he = has_epi ? 1 : 0;
        if (ta) {
            if (f16)
                hipLaunchKernelGGL((k_skinny<true, true>), grid, dim3(kSkWaves * 64), 0, st, a, lda, (int)a_extent, b, ldb,
                                   (int)b_extent, c, ldc, (int)m, (int)n, (int)k, beta, e, he);
            else
                hipLaunchKernelGGL((k_skinny<true, false>), grid, dim3(kSkWaves * 64), 0, st, a, lda, (int)a_extent, b, ldb,
                                   (int)b_extent, c, ldc, (int)m, (int)n, (int)k, beta, e, he);
        } else {
            if (f16)
                hipLaunchKernelGGL((k_skinny<false, true>), grid, dim3(kSkWaves * 64), 0, st, a, lda, (int)a_extent, b, ldb,
                                   (int)b_extent, c, ldc, (int)m, (int)n, (int)k, beta, e, he);
            else
                hipLaunchKernelGGL((k_skinny<false, false>), grid, dim3(kSkWaves * 64), 0, st, a, lda, (int)a_extent, b, ldb,
                                   (int)b_extent, c, ldc, (int)m, (int)n, (int)k, beta, e, he);
        }
        return (int)hipGetLastError();
    }
    const gemm_plan pl = plan_gemm(m, n, kmain, batch, cu_budget);
    const int sp = pl.sp > 1 ? pl.sp : 0;
    // the epilogue rides on the GEMM when one launch of the forward layout
    // finishes C, on the split-K sum when that finishes C, otherwise it is
    // a pass over C afterwards
    if (has_epi && !sp && !ktail && !ta && tb) {
        gemm_args g = {a, lda, stride_a, (int)a_extent, b, ldb, stride_b, (int)b_extent, c, ldc, stride_c,
                       (int)m, (int)n, (int)kmain, 0, 1u, pl.tile};
        return f16 ? launch_layout<false, true, true, true>(g, st, *epi)
                   : launch_layout<false, true, false, true>(g, st, *epi);
    }
    const size_t part_bytes = sp ? (((size_t)sp * m * n * sizeof(float) + 255) & ~(size_t)255) : 0;
    if ((sp || ktail) && !ws)
        return (int)hipErrorInvalidValue;
    int rc = 0;
    if (kmain && sp) {
        // slice z covers k in [z * ks, min(kmain, (z + 1) * ks)): operand
        // offsets along the reduction, dense [m, n] partials
        const size_t ks = ((kmain + sp - 1) / sp + BK - 1) / BK * BK;
        float *part = (float *)ws;
        gemm_args g = {a, lda, ta ? ks * lda : ks, (int)a_extent, b, ldb, tb ? ks * ldb : ks, (int)b_extent, part, n,
                       m * n, (int)m, (int)n, (int)ks, 0, (unsigned)sp, pl.tile, (int)kmain, (int)ks};
        rc = launch_any(f16, ta, tb, g, st);
        if (rc)
            return rc;
        // the epilogue rides on the sum when nothing is added to C after it
        const splitk_desc sd = splitk_of(part, sp, m, n, c, ldc, beta, has_epi && !ktail ? epi : nullptr);
        hipLaunchKernelGGL(k_splitk_sum, splitk_grid(sd, sd), dim3(256), 0, st, sd, sd);
        rc = (int)hipGetLastError();
        if (rc || (has_epi && !ktail))
            return rc;
    } else if (kmain) {
        gemm_args g = {a, lda, stride_a, (int)a_extent, b, ldb, stride_b, (int)b_extent, c, ldc, stride_c,
                       (int)m, (int)n, (int)kmain, beta, (unsigned)batch, pl.tile};
        rc = launch_any(f16, ta, tb, g, st);
        if (rc)
            return rc;
    }
    if (ktail) {
        // (k % 8 != 0) last k-slab of each operand, zero-padded to 64 (and to
        // a multiple of 8 columns for an MN-contiguous copy), then one more
        // launch
        const size_t ma = ta ? (((m + 7) & ~(size_t)7) < 8 ? 8 : ((m + 7) & ~(size_t)7)) : m;
        const size_t nbp = tb ? (((n + 7) & ~(size_t)7) < 8 ? 8 : ((n + 7) & ~(size_t)7)) : n;
        uint16_t *pa = (uint16_t *)((char *)ws + part_bytes);
        const size_t asz = 64 * ma;
        uint16_t *pb = pa + ((asz * batch + 63) & ~(size_t)63);
        const size_t bsz = 64 * nbp;
        const unsigned ga = (unsigned)((asz + 255) / 256 < 4096 ? (asz + 255) / 256 : 4096);
        const unsigned gb = (unsigned)((bsz + 255) / 256 < 4096 ? (bsz + 255) / 256 : 4096);
        hipLaunchKernelGGL(k_pack_slab, dim3(ga, 1, (unsigned)batch), dim3(256), 0, st, ta, a, lda, stride_a, (int)m,
                           (int)ma, (int)kmain, (int)ktail, pa, asz);
        hipLaunchKernelGGL(k_pack_slab, dim3(gb, 1, (unsigned)batch), dim3(256), 0, st, tb, b, ldb, stride_b, (int)n,
                           (int)nbp, (int)kmain, (int)ktail, pb, bsz);
        rc = (int)hipGetLastError();
        if (rc)
            return rc;
        gemm_args g = {pa, ta ? ma : (size_t)64, asz, (int)(ta ? ma : m), pb, tb ? nbp : (size_t)64, bsz,
                       (int)(tb ? nbp : n), c, ldc, stride_c, (int)m, (int)n, BK, kmain ? 1 : beta,
                       (unsigned)batch};
        rc = launch_any(f16, ta, tb, g, st);
        if (rc)
            return rc;
    }
    if (has_epi) {
        hipLaunchKernelGGL(k_bias_act, dim3(gmn), dim3(256), 0, st, c, ldc, (int)m, (int)n, *epi);
        return (int)hipGetLastError();
    }
    return 0;
}

extern "C" size_t pgk_gemm16_pair_dw_workspace(const pgk_gemm_desc *d, const pgk_gemm_desc *w, int cu_d, size_t *off_w)
{
    const size_t wd = pgk_gemm16_workspace_cu(0, 0, d->m, d->n, d->k, d->batch, cu_d);
    *off_w = (wd + 255) & ~(size_t)255;
    return *off_w + pgk_gemm16_workspace_cu(1, 1, w->m, w->n, w->k, w->batch, kCUs - cu_d);
}

extern "C" int pgk_gemm16_pair_dw(int dtype, const pgk_gemm_desc *d, const pgk_gemm_desc *w, int cu_d, void *ws,
                                  pgk_stream s)
{
    if (cu_d < 0 || cu_d >= kCUs || !d->m || !d->n || !d->batch || !w->m || !w->n || !w->batch || !d->k || !w->k)
        return PGK_GEMM_NOT_PAIRED;
    int bad = check_gemm_args(0, 0, d->m, d->n, d->k, d->a, d->lda, d->stride_a, d->a_extent, d->b, d->ldb,
                              d->stride_b, d->b_extent, d->batch);
    if (!bad)
        bad = check_gemm_args(1, 1, w->m, w->n, w->k, w->a, w->lda, w->stride_a, w->a_extent, w->b, w->ldb,
                              w->stride_b, w->b_extent, w->batch);
    if (bad)
        return bad;
    // one launch covers each problem: no k tail, one tile size for both (a
    // skinny wgrad runs alone)
    if (k_inkernel(0, 0, d->k) != d->k || k_inkernel(1, 1, w->k) != w->k ||
        skinny_ok(1, 1, w->m, w->n, w->k, w->batch))
        return PGK_GEMM_NOT_PAIRED;
    const gemm_plan pd = plan_gemm(d->m, d->n, d->k, d->batch, cu_d), pw = plan_gemm(w->m, w->n, w->k, w->batch,
                                                                                      kCUs - cu_d);
    if (pd.tile != pw.tile)
        return PGK_GEMM_NOT_PAIRED;
    size_t off_w = 0;
    pgk_gemm16_pair_dw_workspace(d, w, cu_d, &off_w);
    if ((pd.sp > 1 || pw.sp > 1) && !ws)
        return (int)hipErrorInvalidValue;
    // a split problem writes its slices' partials to its workspace part;
    // one summing launch then adds both problems' slices in order
    auto args = [&](const pgk_gemm_desc *x, int ta, int tb, const gemm_plan &pl, float *part) {
        gemm_args g = {x->a, x->lda, x->stride_a, (int)x->a_extent, x->b, x->ldb, x->stride_b, (int)x->b_extent,
                       x->c, x->ldc, x->stride_c, (int)x->m, (int)x->n, (int)x->k, x->beta, (unsigned)x->batch,
                       pl.tile};
        if (pl.sp > 1) {
            const size_t ks = ((x->k + pl.sp - 1) / pl.sp + BK - 1) / BK * BK;
            g.sa = ta ? ks * x->lda : ks, g.sb = tb ? ks * x->ldb : ks;
            g.c = part, g.ldc = x->n, g.sc = x->m * x->n, g.k = (int)ks, g.beta = 0, g.batch = (unsigned)pl.sp;
            g.k_total = (int)x->k, g.kz_step = (int)ks;
        }
        return g;
    };
    float *part_d = (float *)ws, *part_w = (float *)((char *)ws + off_w);
    const gemm_args gd = args(d, 0, 0, pd, part_d), gw = args(w, 1, 1, pw, part_w);
    hipStream_t st = (hipStream_t)s;
    int rc = dtype == 1 ? launch_pair_tiles<true>(pd.tile, gd, gw, st) : launch_pair_tiles<false>(pd.tile, gd, gw, st);
    if (rc || (pd.sp <= 1 && pw.sp <= 1))
        return rc;
    const splitk_desc s1 = pd.sp > 1 ? splitk_of(part_d, pd.sp, d->m, d->n, d->c, d->ldc, d->beta) : splitk_desc{};
    const splitk_desc s2 = pw.sp > 1 ? splitk_of(part_w, pw.sp, w->m, w->n, w->c, w->ldc, w->beta) : splitk_desc{};
    hipLaunchKernelGGL(k_splitk_sum, splitk_grid(s1, s2), dim3(256), 0, st, s1, s2);
    return (int)hipGetLastError();
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

extern "C" int pgk_mfma_probe(int lds, float *sink, size_t sink_floats, int blocks, int iters, pgk_stream s)
{
    if (blocks < 1 || iters < 2 || (iters & 1) || sink_floats < (size_t)blocks * 512)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mfma_probe, dim3((unsigned)blocks), dim3(512), 0, (hipStream_t)s, sink, iters, lds);
    return (int)hipGetLastError();
}
