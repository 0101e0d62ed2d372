// gfx950 kernels for the INT8 NHWC vision path, behind the C ABI of uqk.h.
//
// Arithmetic contract (bit-exact with the reference's portable C kernels):
//   * conv / pointwise / FC (code 14): acc = sum_k s_k * w_k over the logical
//     K with s = the signed input byte (xz for spatial padding), computed on
//     int8 MFMA; the reference's unsigned column u = s + 128 and its K-tail
//     columns are folded into the per-channel corrected bias at load time, so
//     acc + bias2 equals the reference's acc + bias modulo 2^32, and the
//     loader's int32 bound proof makes that exact.
//   * requantisation (qnn.c:61-83, 734-738): left shift for positive shifts,
//     rounded doubling high multiply, rounding right shift with ties away
//     from zero, output zero point, clamp, optional 256-entry post table.
//   * depthwise (code 15) and pooling (code 16) are bandwidth kernels on the
//     vector ALU; add/mean/LUT/resize/pad/slice are byte-movement kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "uqk.h"

typedef int v4i __attribute__((ext_vector_type(4)));

static hipStream_t g_stream;
static int g_ready;
static int g_err;
static hipEvent_t *g_events;
static uint32_t g_nevents;

#define UQK_TRY(expr)                                  \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) {                        \
            g_err = (int)e_;                           \
            return (int)e_;                            \
        }                                              \
    } while (0)
#define UQK_LAUNCHED() UQK_TRY(hipGetLastError())

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

__device__ __forceinline__ int uq_requant(int acc, int bias, int m, int s, int yz, int lo, int hi)
{
    int v = (int)((unsigned)acc + (unsigned)bias);
    v = uq_scale(v, m, s) + yz;
    return min(max(v, lo), hi);
}

__device__ __forceinline__ int sbyte(int word, int b) { return (int)(signed char)(word >> (8 * b)); }

// ---------------------------------------------------------------------------
// Implicit-GEMM convolution on v_mfma_i32_16x16x64_i8.
//
// A block is 4 waves; each wave owns RB x 16 output rows (pixels) and all
// NT x 16 output channels of the block's channel slice. Each lane gathers one
// 16-byte K slice of one row straight into the MFMA A operand (lane & 15 is
// the row, lane >> 4 the K slice); the B operand is the matching 16-byte K
// slice of the [oc_pad][kpad] weight matrix. A and B use the same lane -> K
// assignment, so the sum is independent of the hardware's K order inside an
// operand. The requantised bytes are staged in LDS and written as coalesced
// 16-byte row segments.
// ---------------------------------------------------------------------------
struct ConvArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;
    const int4 *epi;
    const int4 *kmap;
    const uint8_t *lut;
    int M, ih, iw, ic, oh, ow, oc, sh, sw, pt, pl, xz, yz, lo, hi, K, kpad, ohw;
};

template <int MODE>
__device__ __forceinline__ v4i gather16(const ConvArgs &a, const int8_t *base, int iy0, int ix0, bool valid, int kg, int xzw)
{
    v4i v = {0, 0, 0, 0};
    if (!valid || kg >= a.K) return v;
    if (MODE == UQK_PW) {
        return *(const v4i *)(base + kg);
    } else if (MODE == UQK_G16) {
        const int4 km = a.kmap[kg >> 4];
        const int iy = iy0 + km.x, ix = ix0 + km.y;
        if (iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw)
            return *(const v4i *)(base + ((long)iy * a.iw + ix) * a.ic + km.z);
        return (v4i){xzw, xzw, xzw, xzw};
    } else if (MODE == UQK_G4) {
        int r[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int kk = kg + 4 * j;
            int word = 0;
            if (kk < a.K) {
                const int4 km = a.kmap[kk >> 2];
                const int iy = iy0 + km.x, ix = ix0 + km.y;
                word = (iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw)
                           ? *(const int *)(base + ((long)iy * a.iw + ix) * a.ic + km.z)
                           : xzw;
            }
            r[j] = word;
        }
        return (v4i){r[0], r[1], r[2], r[3]};
    } else {
        int r[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int kk = kg + j;
            int b = 0;
            if (kk < a.K) {
                const int4 km = a.kmap[kk];
                const int iy = iy0 + km.x, ix = ix0 + km.y;
                b = (iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw)
                        ? (int)(uint8_t)base[((long)iy * a.iw + ix) * a.ic + km.z]
                        : (a.xz & 0xff);
            }
            r[j >> 2] |= b << (8 * (j & 3));
        }
        return (v4i){r[0], r[1], r[2], r[3]};
    }
}

template <int RB, int NT, int MODE>
__global__ __launch_bounds__(256) void k_conv(ConvArgs a)
{
    constexpr int R = RB * 16;
    constexpr int BN = NT * 16;
    constexpr int STRIDE = BN + 16;
    __shared__ __attribute__((aligned(16))) int8_t stage[4][R * STRIDE];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int n0 = blockIdx.y * BN;
    const int xzw = (a.xz & 0xff) * 0x01010101;

    const int8_t *base[RB];
    int iy0[RB], ix0[RB];
    bool valid[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int row = row0 + rb * 16 + lr;
        valid[rb] = row < a.M;
        const int r = valid[rb] ? row : 0;
        if (MODE == UQK_PW) {
            base[rb] = a.x + (long)r * a.ic;
            iy0[rb] = ix0[rb] = 0;
        } else {
            const int n = r / a.ohw, rem = r - n * a.ohw;
            const int oy = rem / a.ow, ox = rem - oy * a.ow;
            iy0[rb] = oy * a.sh - a.pt;
            ix0[rb] = ox * a.sw - a.pl;
            base[rb] = a.x + (long)n * a.ih * a.iw * a.ic;
        }
    }

    v4i acc[RB][NT];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rb][nt] = (v4i){0, 0, 0, 0};

    const int8_t *wrow = a.w + (long)(n0 + lr) * a.kpad + lg * 16;
    for (int k0 = 0; k0 < a.kpad; k0 += 64) {
        const int kg = k0 + lg * 16;
        v4i A[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) A[rb] = gather16<MODE>(a, base[rb], iy0[rb], ix0[rb], valid[rb], kg, xzw);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const v4i B = *(const v4i *)(wrow + (long)nt * 16 * a.kpad + k0);
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                acc[rb][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[rb], B, acc[rb][nt], 0, 0, 0);
        }
    }

    // Epilogue: lane holds column (lane & 15) and rows 4*(lane >> 4) + i.
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int col = n0 + nt * 16 + lr;
        const int4 e = col < a.oc ? a.epi[col] : make_int4(0, 0, 0, 0);
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int v = uq_requant(acc[rb][nt][i], e.x, e.y, e.z, a.yz, a.lo, a.hi);
                if (a.lut) v = (int)(signed char)a.lut[v + 128];
                stage[wave][(rb * 16 + lg * 4 + i) * STRIDE + nt * 16 + lr] = (int8_t)v;
            }
    }
    __syncthreads();
    const int ncols = min(BN, a.oc - n0);
    if ((a.oc & 15) == 0) {
        const int cpr = ncols >> 4;
        for (int c = lane; c < R * cpr; c += 64) {
            const int r = c / cpr, cc = c - r * cpr;
            const int row = row0 + r;
            if (row < a.M)
                *(v4i *)(a.y + (long)row * a.oc + n0 + cc * 16) = *(const v4i *)(&stage[wave][r * STRIDE + cc * 16]);
        }
    } else {
        for (int c = lane; c < R * ncols; c += 64) {
            const int r = c / ncols, cc = c - r * ncols;
            const int row = row0 + r;
            if (row < a.M) a.y[(long)row * a.oc + n0 + cc] = stage[wave][r * STRIDE + cc];
        }
    }
}

template <int RB, int NT>
static int launch_conv_mode(const UQKSpatial *d, const ConvArgs &a, dim3 grid)
{
    switch (d->mode) {
    case UQK_PW: hipLaunchKernelGGL((k_conv<RB, NT, UQK_PW>), grid, dim3(256), 0, g_stream, a); break;
    case UQK_G16: hipLaunchKernelGGL((k_conv<RB, NT, UQK_G16>), grid, dim3(256), 0, g_stream, a); break;
    case UQK_G4: hipLaunchKernelGGL((k_conv<RB, NT, UQK_G4>), grid, dim3(256), 0, g_stream, a); break;
    default: hipLaunchKernelGGL((k_conv<RB, NT, UQK_G1>), grid, dim3(256), 0, g_stream, a); break;
    }
    UQK_LAUNCHED();
    return 0;
}

extern "C" int uqk_conv(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    ConvArgs a;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.kmap = (const int4 *)d->kmap;
    a.lut = (const uint8_t *)d->lut;
    a.M = (int)((uint64_t)batches * d->oh * d->ow);
    a.ih = d->ih; a.iw = d->iw; a.ic = d->ic; a.oh = d->oh; a.ow = d->ow; a.oc = d->oc;
    a.sh = d->sh; a.sw = d->sw; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.K = d->K; a.kpad = d->kpad; a.ohw = d->oh * d->ow;
    if (a.M <= 0) return 0;
    const int rows = 4 * 16 * d->rb;
    dim3 grid((unsigned)((a.M + rows - 1) / rows), (unsigned)(d->oc_pad / (16 * d->nt)));
    if (d->rb == 1) {
        switch (d->nt) {
        case 2: return launch_conv_mode<1, 2>(d, a, grid);
        case 4: return launch_conv_mode<1, 4>(d, a, grid);
        case 6: return launch_conv_mode<1, 6>(d, a, grid);
        default: return launch_conv_mode<1, 8>(d, a, grid);
        }
    }
    switch (d->nt) {
    case 2: return launch_conv_mode<2, 2>(d, a, grid);
    case 4: return launch_conv_mode<2, 4>(d, a, grid);
    case 6: return launch_conv_mode<2, 6>(d, a, grid);
    default: return launch_conv_mode<2, 8>(d, a, grid);
    }
}

// ---------------------------------------------------------------------------
// Depthwise (code 15) and pooling (code 16): one thread per output pixel and
// VEC consecutive channels, int32 accumulation, coalesced NHWC loads.
// ---------------------------------------------------------------------------
struct WinArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;
    const int4 *epi;
    const uint8_t *lut;
    long total;
    int groups, ih, iw, c, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, xz, yz, lo, hi, ohw, is_max;
};

template <int VEC>
__device__ __forceinline__ void load_vec(const int8_t *p, int *words)
{
    if (VEC == 16) {
        const v4i v = *(const v4i *)p;
        words[0] = v[0]; words[1] = v[1]; words[2] = v[2]; words[3] = v[3];
    } else if (VEC == 4) {
        words[0] = *(const int *)p;
    } else {
        words[0] = (int)(uint8_t)p[0];
    }
}

template <int VEC>
__device__ __forceinline__ void store_vec(int8_t *p, const int *vals)
{
    int words[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < VEC; j++) words[j >> 2] |= (vals[j] & 0xff) << (8 * (j & 3));
    if (VEC == 16) *(v4i *)p = (v4i){words[0], words[1], words[2], words[3]};
    else if (VEC == 4) *(int *)p = words[0];
    else p[0] = (int8_t)words[0];
}

template <int VEC, bool POOL>
__global__ __launch_bounds__(256) void k_window(WinArgs a)
{
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.total) return;
    const long pix = idx / a.groups;
    const int c0 = (int)(idx - pix * a.groups) * VEC;
    const int n = (int)(pix / a.ohw), rem = (int)(pix - (long)n * a.ohw);
    const int oy = rem / a.ow, ox = rem - oy * a.ow;
    const int8_t *xb = a.x + (long)n * a.ih * a.iw * a.c + c0;
    constexpr int NW = VEC >= 4 ? VEC / 4 : 1;
    const int xzw = VEC >= 4 ? (a.xz & 0xff) * 0x01010101 : (a.xz & 0xff);
    int acc[VEC];
#pragma unroll
    for (int j = 0; j < VEC; j++) acc[j] = POOL && a.is_max ? -128 : 0;
    int count = 0;
    for (int ky = 0; ky < a.kh; ky++) {
        const int iy = oy * a.sh - a.pt + ky * a.dh;
        const bool rowin = iy >= 0 && iy < a.ih;
        for (int kx = 0; kx < a.kw; kx++) {
            const int ix = ox * a.sw - a.pl + kx * a.dw;
            const bool in = rowin && ix >= 0 && ix < a.iw;
            int xw[NW];
            if (in) load_vec<VEC>(xb + ((long)iy * a.iw + ix) * a.c, xw);
            else {
#pragma unroll
                for (int j = 0; j < NW; j++) xw[j] = xzw;
            }
            if (POOL) {
                if (!in) continue;
                count++;
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const int v = VEC >= 4 ? sbyte(xw[j >> 2], j & 3) : (int)(signed char)xw[0];
                    acc[j] = a.is_max ? max(acc[j], v) : acc[j] + v;
                }
            } else {
                int ww[NW];
                load_vec<VEC>(a.w + (long)(ky * a.kw + kx) * a.c + c0, ww);
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    const int xv = VEC >= 4 ? sbyte(xw[j >> 2], j & 3) : (int)(signed char)xw[0];
                    const int wv = VEC >= 4 ? sbyte(ww[j >> 2], j & 3) : (int)(signed char)ww[0];
                    acc[j] += xv * wv;
                }
            }
        }
    }
    int out[VEC];
#pragma unroll
    for (int j = 0; j < VEC; j++) {
        int v;
        if (POOL) {
            v = acc[j];
            if (!a.is_max) {
                const int half = count / 2;
                v = (v + (v > 0 ? half : -half)) / count;
            }
            v = min(max(v, a.lo), a.hi);
        } else {
            const int4 e = a.epi[c0 + j];
            v = uq_requant(acc[j], e.x, e.y, e.z, a.yz, a.lo, a.hi);
            if (a.lut) v = (int)(signed char)a.lut[v + 128];
        }
        out[j] = v;
    }
    store_vec<VEC>(a.y + pix * a.c + c0, out);
}

static int launch_window(const UQKSpatial *d, const void *x, void *y, uint32_t batches, bool pool)
{
    WinArgs a;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.c = d->oc; a.oh = d->oh; a.ow = d->ow;
    a.kh = d->kh; a.kw = d->kw; a.sh = d->sh; a.sw = d->sw; a.dh = d->dh; a.dw = d->dw;
    a.pt = d->pt; a.pl = d->pl; a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.ohw = d->oh * d->ow;
    a.is_max = d->is_max;
    const int vec = d->vec;
    a.groups = d->oc / vec;
    a.total = (long)batches * a.ohw * a.groups;
    if (a.total <= 0) return 0;
    dim3 grid((unsigned)((a.total + 255) / 256));
    if (pool) {
        if (vec == 16) hipLaunchKernelGGL((k_window<16, true>), grid, dim3(256), 0, g_stream, a);
        else if (vec == 4) hipLaunchKernelGGL((k_window<4, true>), grid, dim3(256), 0, g_stream, a);
        else hipLaunchKernelGGL((k_window<1, true>), grid, dim3(256), 0, g_stream, a);
    } else {
        if (vec == 16) hipLaunchKernelGGL((k_window<16, false>), grid, dim3(256), 0, g_stream, a);
        else if (vec == 4) hipLaunchKernelGGL((k_window<4, false>), grid, dim3(256), 0, g_stream, a);
        else hipLaunchKernelGGL((k_window<1, false>), grid, dim3(256), 0, g_stream, a);
    }
    UQK_LAUNCHED();
    return 0;
}

extern "C" int uqk_depthwise(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    return launch_window(d, x, y, batches, false);
}

extern "C" int uqk_pool(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    return launch_window(d, x, y, batches, true);
}

// ---------------------------------------------------------------------------
// Residual add (uq_add, qnn.c:175-183): both 256-entry tables in LDS,
// 16 bytes per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_add(const int8_t *a, const int8_t *b, int8_t *y, uint64_t count,
                                              const int *tables, int m, int s, int yz, int lo, int hi)
{
    __shared__ int tx[256], tb[256];
    tx[threadIdx.x] = tables[threadIdx.x];
    tb[threadIdx.x] = tables[256 + threadIdx.x];
    __syncthreads();
    const uint64_t i0 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i0 >= count) return;
    if (i0 + 16 <= count) {
        const v4i va = *(const v4i *)(a + i0), vb = *(const v4i *)(b + i0);
        int w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int word = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int s1 = tx[sbyte(va[q], j) + 128] + tb[sbyte(vb[q], j) + 128];
                const int v = min(max(uq_scale(s1, m, s) + yz, lo), hi);
                word |= (v & 0xff) << (8 * j);
            }
            w[q] = word;
        }
        *(v4i *)(y + i0) = (v4i){w[0], w[1], w[2], w[3]};
    } else {
        for (uint64_t i = i0; i < count; i++) {
            const int s1 = tx[(int)a[i] + 128] + tb[(int)b[i] + 128];
            y[i] = (int8_t)min(max(uq_scale(s1, m, s) + yz, lo), hi);
        }
    }
}

extern "C" int uqk_add(const void *a, const void *b, void *y, uint64_t count, const void *tables,
                       int32_t m, int32_t shift, int32_t yz, int32_t lo, int32_t hi)
{
    if (!count) return 0;
    const uint64_t threads = (count + 15) / 16;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g_stream,
                       (const int8_t *)a, (const int8_t *)b, (int8_t *)y, count, (const int *)tables, m, shift, yz, lo, hi);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Global spatial mean (uq_mean, qnn.c:184-198): one thread per (batch, channel).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_mean(const int8_t *x, int8_t *y, uint32_t batches, uint32_t pixels,
                                               uint32_t channels, int xz, int yz, int m, int s)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)batches * channels) return;
    const uint32_t n = (uint32_t)(idx / channels), c = (uint32_t)(idx - (uint64_t)n * channels);
    const int8_t *p = x + (uint64_t)n * pixels * channels + c;
    int sum = 0;
    for (uint32_t q = 0; q < pixels; q++) sum += p[(uint64_t)q * channels];
    y[idx] = (int8_t)min(max(uq_scale(sum - (int)pixels * xz, m, s) + yz, -128), 127);
}

extern "C" int uqk_mean(const void *x, void *y, uint32_t batches, uint32_t pixels, uint32_t channels,
                        int32_t xz, int32_t yz, int32_t m, int32_t shift)
{
    const uint64_t total = (uint64_t)batches * channels;
    if (!total) return 0;
    hipLaunchKernelGGL(k_mean, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g_stream,
                       (const int8_t *)x, (int8_t *)y, batches, pixels, channels, xz, yz, m, shift);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// 256-entry byte lookup (code 22): table in LDS, 16 bytes per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_lut(const uint8_t *x, uint8_t *y, uint64_t count, const uint8_t *table, uint32_t flip)
{
    __shared__ uint8_t t[256];
    t[threadIdx.x] = table[threadIdx.x];
    __syncthreads();
    const uint64_t i0 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i0 >= count) return;
    if (i0 + 16 <= count) {
        const v4i v = *(const v4i *)(x + i0);
        int w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int word = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) word |= (int)t[((v[q] >> (8 * j)) & 0xff) ^ flip] << (8 * j);
            w[q] = word;
        }
        *(v4i *)(y + i0) = (v4i){w[0], w[1], w[2], w[3]};
    } else {
        for (uint64_t i = i0; i < count; i++) y[i] = t[x[i] ^ flip];
    }
}

extern "C" int uqk_lut(const void *x, void *y, uint64_t count, const void *table, uint32_t flip)
{
    if (!count) return 0;
    const uint64_t threads = (count + 15) / 16;
    hipLaunchKernelGGL(k_lut, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g_stream,
                       (const uint8_t *)x, (uint8_t *)y, count, (const uint8_t *)table, flip);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Nearest resize (code 21, graph.c:342-346): one thread per output byte group.
// ---------------------------------------------------------------------------
template <int VEC>
__global__ __launch_bounds__(256) void k_resize(const int8_t *x, int8_t *y, uint64_t total, uint32_t groups,
                                                 uint32_t oh, uint32_t ow, uint32_t c, uint64_t in_stride,
                                                 const uint32_t *offs)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const uint64_t pix = idx / groups;
    const uint32_t g = (uint32_t)(idx - pix * groups);
    const uint32_t ox = (uint32_t)(pix % ow);
    const uint64_t t = pix / ow;
    const uint32_t oy = (uint32_t)(t % oh);
    const uint64_t n = t / oh;
    const int8_t *src = x + n * in_stride + offs[oy] + offs[oh + ox] + (uint64_t)g * VEC;
    int8_t *dst = y + pix * c + (uint64_t)g * VEC;
    if (VEC == 16) *(v4i *)dst = *(const v4i *)src;
    else if (VEC == 4) *(int *)dst = *(const int *)src;
    else *dst = *src;
}

extern "C" int uqk_resize(const void *x, void *y, uint32_t batches, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow,
                          uint32_t c, const void *offsets)
{
    const int vec = c % 16 == 0 ? 16 : c % 4 == 0 ? 4 : 1;
    const uint32_t groups = c / vec;
    const uint64_t total = (uint64_t)batches * oh * ow * groups;
    if (!total) return 0;
    const uint64_t in_stride = (uint64_t)ih * iw * c;
    dim3 grid((unsigned)((total + 255) / 256));
    if (vec == 16)
        hipLaunchKernelGGL(k_resize<16>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
    else if (vec == 4)
        hipLaunchKernelGGL(k_resize<4>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
    else
        hipLaunchKernelGGL(k_resize<1>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// 4-D window gather for pad (code 23) and slice (code 26).
// ---------------------------------------------------------------------------
struct Win4 {
    uint32_t in[4], out[4];
    int32_t off[4];
};

__global__ __launch_bounds__(256) void k_window4(const int8_t *x, int8_t *y, uint64_t total, Win4 g, int fill,
                                                  uint64_t in_bytes, uint64_t out_bytes)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const uint64_t img = idx / out_bytes;
    uint64_t r = idx - img * out_bytes;
    int64_t src = 0;
    bool in = true;
    uint64_t stride = 1;
    for (int d = 3; d >= 0; d--) {
        const uint32_t o = (uint32_t)(r % g.out[d]);
        r /= g.out[d];
        const int64_t s = (int64_t)o - g.off[d];
        if (s < 0 || s >= (int64_t)g.in[d]) in = false;
        src += s * (int64_t)stride;
        stride *= g.in[d];
    }
    y[idx] = in ? x[img * in_bytes + (uint64_t)src] : (int8_t)fill;
}

extern "C" int uqk_window4(const void *x, void *y, uint32_t images, const uint32_t in_dims[4], const uint32_t out_dims[4],
                           const int32_t offset[4], int32_t fill)
{
    Win4 g;
    uint64_t in_bytes = 1, out_bytes = 1;
    for (int d = 0; d < 4; d++) {
        g.in[d] = in_dims[d];
        g.out[d] = out_dims[d];
        g.off[d] = offset[d];
        in_bytes *= in_dims[d];
        out_bytes *= out_dims[d];
    }
    const uint64_t total = out_bytes * images;
    if (!total) return 0;
    hipLaunchKernelGGL(k_window4, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g_stream,
                       (const int8_t *)x, (int8_t *)y, total, g, fill, in_bytes, out_bytes);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Runtime plumbing.
// ---------------------------------------------------------------------------
extern "C" int uqk_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int uqk_init(void)
{
    if (g_ready) return 0;
    int n = 0;
    UQK_TRY(hipGetDeviceCount(&n));
    if (n < 1) return (int)hipErrorNoDevice;
    UQK_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_ready = 1;
    return 0;
}

extern "C" void *uqk_malloc(size_t bytes)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
    return p;
}

extern "C" void uqk_free(void *p)
{
    if (p) (void)hipFree(p);
}

extern "C" int uqk_h2d(void *dst, const void *src, size_t bytes)
{
    if (bytes) UQK_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    return 0;
}

extern "C" int uqk_d2h(void *dst, const void *src, size_t bytes)
{
    if (bytes) UQK_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    return 0;
}

extern "C" int uqk_d2d(void *dst, const void *src, size_t bytes)
{
    if (bytes) UQK_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    return 0;
}

extern "C" int uqk_d2d_2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t height)
{
    if (width && height)
        UQK_TRY(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice, g_stream));
    return 0;
}

extern "C" int uqk_sync(void)
{
    UQK_TRY(hipStreamSynchronize(g_stream));
    return 0;
}

extern "C" int uqk_last_error(void) { return g_err; }

extern "C" int uqk_events(uint32_t count)
{
    if (count <= g_nevents) return 0;
    hipEvent_t *ev = (hipEvent_t *)realloc(g_events, sizeof(hipEvent_t) * count);
    if (!ev) return (int)hipErrorOutOfMemory;
    g_events = ev;
    for (uint32_t i = g_nevents; i < count; i++) {
        UQK_TRY(hipEventCreate(&g_events[i]));
        g_nevents = i + 1;
    }
    return 0;
}

extern "C" int uqk_record(uint32_t index)
{
    if (index >= g_nevents) return (int)hipErrorInvalidValue;
    UQK_TRY(hipEventRecord(g_events[index], g_stream));
    return 0;
}

extern "C" int uqk_elapsed_ns(uint32_t first, uint32_t second, uint64_t *ns)
{
    if (first >= g_nevents || second >= g_nevents) return (int)hipErrorInvalidValue;
    float ms = 0.f;
    UQK_TRY(hipEventElapsedTime(&ms, g_events[first], g_events[second]));
    *ns = (uint64_t)((double)ms * 1e6 + 0.5);
    return 0;
}
