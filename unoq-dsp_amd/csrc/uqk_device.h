// Device-side helpers shared by the gfx950 kernel files: requantisation
// (qnn.c:61-83 and its one-multiply forms), byte packing and clamps.
#ifndef UQK_DEVICE_H
#define UQK_DEVICE_H
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Requantisation: qnn.c:61-83 followed by the zero point and clamp.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int uq_scale(int v, int m, int s)
{
    if (s > 0) v = (int)((unsigned)v << s);
    long long p = (long long)v * (long long)m;
    int h = (int)((p + (1LL << 30)) >> 31);
    if (s >= 0) return h;
    const int n = -s;
    const unsigned mask = (1u << n) - 1u;
    const int base = h >> n;
    const unsigned rem = (unsigned)h & mask;
    return base + (rem > ((mask >> 1) + (unsigned)(h < 0)) ? 1 : 0);
}


__device__ __forceinline__ int sbyte(int word, int b) { return (int)(signed char)(word >> (8 * b)); }

// Per-channel constants of the one-multiply requantisation (layout and
// derivation at epilogue_record in graph.c): exact for every shift in
// [-31, 15]; `corr` enables the ties-away correction for layers whose clamp
// can let negative rounded values through (act_min < output zero point).
struct Epi {
    int bias, m, ls, T;
    long long c1, cthr;
};

__device__ __forceinline__ Epi load_epi(const int4 *epi, int c)
{
    const int4 a = epi[2 * c], b = epi[2 * c + 1];
    Epi e;
    e.bias = a.x; e.m = a.y; e.ls = a.z; e.T = a.w;
    e.c1 = (long long)(((unsigned long long)(unsigned)b.y << 32) | (unsigned)b.x);
    e.cthr = (long long)(((unsigned long long)(unsigned)b.w << 32) | (unsigned)b.z);
    return e;
}

__device__ __forceinline__ int uq_requant_affine(int acc, const Epi &e, int corr, int yz, int lo, int hi)
{
    const int v = (int)(((unsigned)acc + (unsigned)e.bias) << e.ls);
    long long q = (long long)v * (long long)e.m + e.c1;
    if (corr && q < e.cthr) q -= (1LL << 31);
    const int r = (int)(q >> e.T);
    return min(max(r + yz, lo), hi);
}

__device__ __forceinline__ int pack4(int v0, int v1, int v2, int v3)
{
    const unsigned lo = __builtin_amdgcn_perm((unsigned)v1, (unsigned)v0, 0x0c0c0400u);
    const unsigned hi = __builtin_amdgcn_perm((unsigned)v3, (unsigned)v2, 0x04000c0cu);
    return (int)(lo | hi);
}

// A value copied into a VGPR once and opaque to the compiler from then on, so
// that it stays there: for the clamp bounds of med3, which otherwise are
// re-copied from their SGPRs before nearly every use.
__device__ __forceinline__ int vgpr(int x)
{
    int r = x;
    asm volatile("" : "+v"(r));
    return r;
}

// Clamp to [lo, hi] in one v_med3_i32 (the compiler keeps min/max apart).
__device__ __forceinline__ int med3(int x, int lo, int hi)
{
    int r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
    return r;
}

// Conv requantisation of an MFMA accumulator.
// HI (layers whose every channel has shift in [-22, -1]): the record's c1
// already holds corrected_bias * m + yz * 2^T (computed mod 2^64 at load
// time), so q = acc * m + c1 is the full affine value; T >= 32 makes q >> T
// the high word of q (or of the corrected q - 2^31) shifted by T - 32.
// Generic: v = (acc + bias) << ls, q = v * m + c1, then the zero point.
// CORR: the clamp lets negative values through (act_min < output zero point).
template <bool HI, bool CORR>
__device__ __forceinline__ int conv_requant(int acc, const Epi &e, int yz, int lo, int hi)
{
    if (HI) {
        const long long q = (long long)acc * (long long)e.m + e.c1;
        int h = (int)(q >> 32);
        if (CORR && q < e.cthr) h = (int)((q - (1LL << 31)) >> 32);
        return med3(h >> (e.T - 32), lo, hi);
    }
    const int v = (int)(((unsigned)acc + (unsigned)e.bias) << e.ls);
    long long q = (long long)v * (long long)e.m + e.c1;
    if (CORR && q < e.cthr) q -= (1LL << 31);
    return med3((int)(q >> e.T) + yz, lo, hi);
}

#endif
