// Depthwise 3x3 / 5x5, stride 1 or 2 (code 15, qnn.c:807-983,
// depthwise_fixed.h, depthwise5.h), as an HBM-streaming band kernel.
//
// A block owns a band of output rows of one image and a slice of gs groups
// of 16 channels. It stages the band's padded input window, the NHWC bytes
// of its channel slice (the zero point at padding positions), straight from
// HBM into LDS with 16-byte global-to-LDS loads, all of them issued at once:
// consecutive lanes load consecutive 16-byte chunks of a pixel's slice and
// then of the next pixels, so every load instruction reads whole runs of
// the image row. The multiply-adds go to the matrix cores: one
// v_mfma_i32_16x16x64_i8 is 16 output pixels x 16 channels over four taps,
// its pixel operand the 16 channel bytes under a tap (one 16-byte LDS read,
// no transposes) and its weight operand block-diagonal (lane (channel c, tap
// slot s) holds w[tap][c] in byte c % 4 of word c / 4). The vector ALU is left
// with the requantisation.
//
// The staged window is [staged pixel][gs chunks of 16 bytes]; chunk g of
// staged pixel sp sits at position g ^ ((sp >> sws) & swm), chosen on the
// host so that the 16 pixels of an operand read (stride S pixels) fall in
// distinct 16-byte bank groups as far as the stride allows. Loads are
// arranged so that the lanes of an instruction write 1 KiB of LDS in order:
// lane l of instruction j fills position (j * 64 + l) of the window and
// fetches the logical chunk that belongs there.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"

struct DwBArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;           // [taps][C] signed int8 (the plan's layout)
    const int4 *epi;           // 32-byte records per channel
    const uint8_t *lut;
    int ih, iw, c, oh, ow, pt, pl, xz, yz, lo, hi;
    int images, band, bands, gs;   // output rows per block, bands per image, channel groups per block
    int cols_p;                    // staged columns: (ow - 1) * S + KS
    int win_bytes;                 // LDS bytes of the largest staged window (multiple of 1 KiB)
    int sws, swm;                  // chunk swizzle
    unsigned m_gs, m_cols, m_ow;   // udiv_magic of gs, cols_p, ow
};

template <int KS, int S, int EMODE>
__global__ __launch_bounds__(256) void k_dw_band(DwBArgs a)
{
    constexpr int T = KS * KS, NG = (T + 3) / 4;
    constexpr bool HI = (EMODE & 1) != 0, CORR = (EMODE & 2) != 0;
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int CB = a.gs * 16;
    // blockIdx.x = (slice * images + image) * bands + band
    const int per_slice = a.images * a.bands;
    const int slice = blockIdx.x / per_slice, nb = blockIdx.x - slice * per_slice;
    const int n = nb / a.bands, oyb = (nb - n * a.bands) * a.band;
    const int brows = min(a.band, a.oh - oyb);
    const int srows = (brows - 1) * S + KS;
    const int cb0 = slice * CB;
    int8_t *wts = smem + a.win_bytes;                       // [T][CB] weights of the slice
    int4 *recs = (int4 *)(wts + ((T * CB + 15) & ~15));     // [CB][2] records
    int8_t *lut_s = (int8_t *)(recs + 2 * CB);

    // Stage the window: position q = staged pixel sp * gs + physical chunk.
    {
        const int8_t *pad = (const int8_t *)g_pad_rows.b + (a.xz & 0xff) * 16;
        const int8_t *xim = a.x + (long)n * a.ih * a.iw * a.c + cb0;
        const uint32_t win = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)smem;
        const int chunks = srows * a.cols_p * a.gs, ninst = (chunks + 63) >> 6;
        const int iyb = oyb * S - a.pt;
        for (int j = wave; j < ninst; j += 4) {
            const int q = j * 64 + lane;
            const int sp = (int)udiv((unsigned)q, (unsigned)a.gs, a.m_gs), pg = q - sp * a.gs;
            const int r = (int)udiv((unsigned)sp, (unsigned)a.cols_p, a.m_cols), cc = sp - r * a.cols_p;
            const int gl = pg ^ ((sp >> a.sws) & a.swm);
            const int iy = iyb + r, ix = cc - a.pl;
            const bool in = q < chunks && (unsigned)iy < (unsigned)a.ih && (unsigned)ix < (unsigned)a.iw;
            lds_load16(in ? xim + ((long)iy * a.iw + ix) * a.c + gl * 16 : pad, win + j * 1024);
        }
    }
    // Weights, records and the post table of the slice (plain loads).
    for (int u = threadIdx.x; u < T * CB / 4; u += 256) {
        const int t = u / (CB / 4), cq = u - t * (CB / 4);
        ((int *)wts)[u] = *(const int *)(a.w + (long)t * a.c + cb0 + 4 * cq);
    }
    for (int u = threadIdx.x; u < 2 * CB; u += 256) recs[u] = a.epi[2 * cb0 + u];
    if (a.lut && threadIdx.x < 64) ((int *)lut_s)[threadIdx.x] = ((const int *)a.lut)[threadIdx.x];
    // Tap slot m of this lane: tap 4m + lg, its offset in staged pixels.
    int off[NG];
#pragma unroll
    for (int m = 0; m < NG; m++) {
        const int t = 4 * m + lg, ky = t / KS, kx = t - ky * KS;
        off[m] = t < T ? ky * a.cols_p + kx : 0;
    }
    wait_vm<0>();
    __syncthreads();

    const int npix = brows * a.ow, tiles = (npix + 15) >> 4, items = tiles * a.gs;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    int8_t *yim = a.y + ((long)n * a.oh + oyb) * a.ow * a.c + cb0;
    int gcur = -1;
    v4i B[NG];
    Epi e;
    for (int it = wave; it < items; it += 4) {
        const int g = it / tiles, tile = it - g * tiles;
        if (g != gcur) {
            gcur = g;
#pragma unroll
            for (int m = 0; m < NG; m++) {
                const int t = 4 * m + lg;
                const int wb = t < T ? (int)(uint8_t)wts[t * CB + g * 16 + lr] : 0;
                const int word = wb << (8 * (lr & 3)), at = lr >> 2;
                B[m] = (v4i){at == 0 ? word : 0, at == 1 ? word : 0, at == 2 ? word : 0, at == 3 ? word : 0};
            }
            e = load_epi(recs, g * 16 + lr);
        }
        // A row: band pixel p (clamped into the band for the tail tile).
        const int p = min(tile * 16 + lr, npix - 1);
        const int oy = (int)udiv((unsigned)p, (unsigned)a.ow, a.m_ow), ox = p - oy * a.ow;
        const int sp0 = oy * S * a.cols_p + ox * S;
        v4i A[NG];
#pragma unroll
        for (int m = 0; m < NG; m++) {
            const int sp = sp0 + off[m];
            const int ph = g ^ ((sp >> a.sws) & a.swm);
            A[m] = *(const v4i *)(smem + (sp * a.gs + ph) * 16);
        }
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < NG; m++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], B[m], acc, 0, 0, 0);
        // acc[i]: pixel tile*16 + 4*lg + i, channel g*16 + lr.
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[i], e, a.yz, vlo, vhi);
        if (a.lut) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
        }
        const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
        const int px = tile * 16 + lg * 4 + (lane & 3);
        if (px < npix) *(int *)(yim + (long)px * a.c + g * 16 + (lr & ~3)) = word;
    }
}

// Records as int4 pairs, read through the generic loader of uqk_device.h
// (load_epi takes a global or LDS int4 array alike).

static const int DW_LDS_MAX = 49152;     // per block: three blocks per CU

// LDS bytes besides the window: weights [T][gs*16], records, post table.
static size_t dw_fixed_bytes(int T, int gs)
{
    return (size_t)((T * gs * 16 + 15) & ~15) + (size_t)gs * 16 * 32 + 256;
}

// Bank groups hit by the 16 pixels (stride S) of an operand read under a
// swizzle: the largest number of lanes sharing one 16-byte bank group.
static int dw_conflicts(int gs, int S, int sws, int swm)
{
    int worst = 1;
    for (int g = 0; g < gs; g++)
        for (int base = 0; base < 64; base += 7) {
            int count[16] = {0};
            for (int p = 0; p < 16; p++) {
                const int sp = base + p * S;
                const int ph = g ^ ((sp >> sws) & swm);
                const int slot = (sp * gs + ph) & 15;
                if (++count[slot] > worst) worst = count[slot];
            }
        }
    return worst;
}

// Plan a layer once, when it is loaded: channel slice (groups of 16 per
// block), band of output rows, chunk swizzle. d->dwb[0] stays 0 when the
// layer does not fit.
extern "C" void uqk_dw_band_prepare(UQKSpatial *d)
{
    d->dwb[0] = d->dwb[1] = d->dwb[2] = d->dwb[3] = 0;
    const int ks = d->kh, s = d->sh;
    if (d->oc % 16 || d->ic != d->oc || d->kh != d->kw || (ks != 3 && ks != 5) || d->sh != d->sw ||
        (s != 1 && s != 2) || d->dh != 1 || d->dw != 1 || d->ow < 1 || d->oh < 1)
        return;
    const int G = d->oc / 16, T = ks * ks, cols_p = (d->ow - 1) * s + ks;
    double best = -1;
    int best_gs = 0, best_band = 0;
    for (int gs = G; gs >= 1; gs--) {
        if (G % gs) continue;
        const size_t fixed = dw_fixed_bytes(T, gs);
        const size_t row = (size_t)cols_p * gs * 16;
        if (fixed + (size_t)ks * row > DW_LDS_MAX) continue;
        int band = (int)(((DW_LDS_MAX - fixed) / row - ks) / s + 1);
        if (band > d->oh) band = d->oh;
        const int rows_p = (band - 1) * s + ks;
        const double amp = (double)rows_p / (band * s);
        const double seg = gs * 16 >= 128 ? 1.0 : gs * 16 / 128.0;
        if (seg / amp > best) {
            best = seg / amp;
            best_gs = gs;
            best_band = band;
        }
    }
    // The division magics are exact below 2^32 / divisor: staged positions
    // and band pixels stay far below that.
    if (best < 0 || (long)best_band * d->ow >= 65536) return;
    // Swizzle: the XOR must stay inside [0, gs), so its mask is below the
    // largest power of two dividing gs.
    int pow2 = 1;
    while (best_gs % (2 * pow2) == 0 && 2 * pow2 <= 16) pow2 *= 2;
    int bw = 99, bsws = 0, bswm = 0;
    for (int swm = 0; swm < pow2; swm = 2 * swm + 1)
        for (int sws = 0; sws < 8; sws++) {
            const int w = dw_conflicts(best_gs, s, sws, swm);
            if (w < bw) {
                bw = w;
                bsws = sws;
                bswm = swm;
            }
        }
    d->dwb[0] = best_gs;
    d->dwb[1] = best_band;
    d->dwb[2] = bsws;
    d->dwb[3] = bswm;
}

extern "C" int uqk_dw_band(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    if (d->dwb[0] <= 0) return (int)hipErrorInvalidValue;
    DwBArgs a;
    const int ks = d->kh, s = d->sh, T = ks * ks;
    a.gs = d->dwb[0];
    a.band = d->dwb[1];
    a.sws = d->dwb[2];
    a.swm = d->dwb[3];
    a.cols_p = (d->ow - 1) * s + ks;
    // Narrower bands for small batches, so that the grid still fills the chip.
    const long slices = d->oc / 16 / a.gs;
    while (a.band > 1 && (long)batches * slices * ((d->oh + a.band - 1) / a.band) < 768) a.band = (a.band + 1) / 2;
    a.bands = (d->oh + a.band - 1) / a.band;
    a.win_bytes = (int)((((size_t)(a.band - 1) * s + ks) * a.cols_p * a.gs * 16 + 1023) / 1024 * 1024);
    const size_t lds = (size_t)a.win_bytes + dw_fixed_bytes(T, a.gs);
    if (lds > DW_LDS_MAX) return (int)hipErrorInvalidValue;
    a.m_gs = udiv_magic((unsigned)a.gs);
    a.m_cols = udiv_magic((unsigned)a.cols_p);
    a.m_ow = udiv_magic((unsigned)d->ow);
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.c = d->oc; a.oh = d->oh; a.ow = d->ow; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.images = (int)batches;
    const unsigned long long blocks = (unsigned long long)batches * a.bands * (d->oc / 16 / a.gs);
    if (!blocks) return 0;
    if (blocks > 0x7fffffffULL) return (int)hipErrorInvalidValue;
    const int mode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0);
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    const dim3 grid((unsigned)blocks), block(256);
#define UQK_DWB(K, S)                                                                                          \
    do {                                                                                                       \
        switch (mode) {                                                                                        \
        case 0: hipExtLaunchKernelGGL((k_dw_band<K, S, 0>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a); break;  \
        case 1: hipExtLaunchKernelGGL((k_dw_band<K, S, 1>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a); break;  \
        case 2: hipExtLaunchKernelGGL((k_dw_band<K, S, 2>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a); break;  \
        default: hipExtLaunchKernelGGL((k_dw_band<K, S, 3>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a); break; \
        }                                                                                                      \
    } while (0)
    if (d->kh == 3 && d->sh == 1) UQK_DWB(3, 1);
    else if (d->kh == 3) UQK_DWB(3, 2);
    else if (d->sh == 1) UQK_DWB(5, 1);
    else UQK_DWB(5, 2);
#undef UQK_DWB
    return uqk_fail(hipGetLastError());
}
