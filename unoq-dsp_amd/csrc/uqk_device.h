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

// x / d without a division: ceil(2^32 / d) as a multiply-high, exact when
// x * d < 2^32 (the rounding error of the magic is below d); d == 1 passes
// x through. The magic comes from udiv_magic on the host.
__device__ __forceinline__ unsigned udiv(unsigned x, unsigned d, unsigned magic)
{
    return d == 1 ? x : __umulhi(x, magic);
}

static inline unsigned udiv_magic(unsigned d)
{
    return d <= 1 ? 0u : (unsigned)((0x100000000ULL + d - 1) / d);
}

// 4x4 byte transpose across a quad of lanes: lane j of the quad ends with
// byte j of each of the four lanes' words.
__device__ __forceinline__ int quad_transpose_bytes(int w, int lane)
{
    const int j = lane & 3;
    const int x = __builtin_amdgcn_mov_dpp(w, 0x4E, 0xF, 0xF, true);        // quad_perm [2,3,0,1]
    const int u = (int)__builtin_amdgcn_perm((unsigned)x, (unsigned)w, j < 2 ? 0x05040100u : 0x03020706u);
    const int y = __builtin_amdgcn_mov_dpp(u, 0xB1, 0xF, 0xF, true);        // quad_perm [1,0,3,2]
    return (int)__builtin_amdgcn_perm((unsigned)y, (unsigned)u, (j & 1) ? 0x03070105u : 0x06020400u);
}

// 4x4 transpose of 16-lane rows across four registers: afterwards row j of
// r[q] holds what row q of r[j] held. One v_permlane32_swap per register pair
// exchanges the upper half of the first with the lower half of the second;
// one v_permlane16_swap exchanges the odd rows of the first with the even
// rows of the second.
__device__ __forceinline__ void rows_transpose4(int (&r)[4])
{
    auto s02 = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
    auto s13 = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
    auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    r[0] = (int)s01[0]; r[1] = (int)s01[1]; r[2] = (int)s23[0]; r[3] = (int)s23[1];
}

// Sixteen bytes of value v at offset 16 * v: the source of staged chunks that
// hold the input zero point (im2col padding), pixel chunks past K (whose
// weights are zero, so any finite bytes do) and weight chunks past kpad (row
// 0: zeros), so that every lane of a staging instruction loads from a valid
// address.
struct PadRows {
    uint8_t b[256 * 16];
};
static constexpr PadRows make_pad_rows()
{
    PadRows p{};
    for (int i = 0; i < 256 * 16; i++) p.b[i] = (uint8_t)(i >> 4);
    return p;
}
static __device__ const PadRows g_pad_rows = make_pad_rows();

// Sixteen bytes from global memory straight into LDS: lane l's bytes land
// at LDS address lds + 16 * l (lds wave-uniform). Issued through asm (with
// no memory clobber) so that the compiler, which would otherwise wait for
// every outstanding LDS load before each LDS read and barrier, leaves the
// ring's waits to wait_vm. Order against the LDS reads of the same buffer
// comes from the barriers: a buffer is refilled only after the barrier that
// follows its last read, and read only after the wait and barrier that
// follow its fill. M0 is the LDS base of the instruction (one wait state
// between writing M0 and the load that reads it).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_load16(const void *src, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

#endif
