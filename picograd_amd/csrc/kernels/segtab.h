// Block -> tensor lookup for the multi-tensor launches (device code only).
//
// A multi-tensor launch cuts every tensor into fixed chunks, one block each;
// first[i] is tensor i's first block and first[cnt .. MAX] all hold the
// block total, which no block index reaches.  A block's tensor is the number
// of entries first[1 .. MAX - 1] at or below its index.  The scan has a
// fixed length and is unrolled, so the compiler issues every scalar load of
// the table at once: a loop bounded by the table's count waits for each
// load in turn, which costs microseconds per block at the start of
// short-lived blocks.
#ifndef PGK_SEGTAB_H
#define PGK_SEGTAB_H

#include <hip/hip_runtime.h>

template <int MAX>
__device__ __forceinline__ int seg_of(const unsigned (&first)[MAX + 1], unsigned b)
{
    // b >= first[i] as the sign bit of first[i] - 1 - b (block counts stay
    // below 2^31): plain scalar arithmetic, where a comparison per entry
    // would become a 64-bit lane mask per entry
    unsigned s = 0;
#pragma unroll
    for (int i = 1; i < MAX; ++i)
        s += (first[i] - 1u - b) >> 31;
    return (int)s;
}

// index of element j's 16-bit copy in a segment's shadow: rows of
// shadow_cols elements at a pitch of shadow_ld when the shadow is pitched
// (shadow_cols != 0), else j
template <class SEG>
__device__ __forceinline__ size_t shadow_at(const SEG &sg, size_t j)
{
    if (!sg.shadow_cols)
        return j;
    const size_t r = j / sg.shadow_cols;
    return r * sg.shadow_ld + (j - r * sg.shadow_cols);
}

// host side: first[cnt .. MAX] = blocks
template <int MAX>
inline void seg_close(unsigned (&first)[MAX + 1], int cnt, unsigned blocks)
{
    for (int i = cnt; i <= MAX; ++i)
        first[i] = blocks;
}

#endif
