// A 1x1 conv fused with the global mean over its output, for gfx950: the
// classifier head of MobileNet-style networks (code 14, 1x1 stride 1, then
// code 24 over the whole map; the reference runs them one after the other
// through its arena: qnn.c:1101-1169 / gemm.c:592-612 for the conv,
// qnn.c:184-198 for the mean). The conv's output is never written: each of
// an image's workgroups (two by default, each a contiguous share of the
// output channels) keeps the image's P <= 64 pixels of input in LDS,
// computes its output channels on the matrix cores, requantises each value
// exactly as the conv kernels do (its records, clamp and post table), and
// sums the int8 results of each channel over the image's pixels; the mean's
// own requantisation (uq_scale, zero points, clamp, as k_mean) then gives
// one byte per channel.
//
// Matrix cores: v_mfma_i32_32x32x32_i8 with the pixels as the MFMA rows (from
// LDS, 16 bytes per lane and K step) and 32 output channels as its columns
// (the weights, 16 bytes per lane and K step from L2), so a lane's 16 results
// share one channel, its record and its running sum: lane (fr, fh) holds
// channel fr of pixels 8g + 4fh + i. Items are 32-channel tiles, a
// contiguous range per wave, each over both 32-pixel tiles of the image; a
// lane adds its own pixels, then the lane holding the channel's other
// pixels (fh = 1) is added across the 32-lane halves.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int HM_WAVES = 8;            // waves per workgroup
constexpr int HM_MAXK = 8;             // K steps of 32 bytes: IC <= 256
constexpr int HM_MAXP = 64;            // pixels per image
// Workgroups per image by default. MobileNetV4-S's 960 channels (30 tiles of
// 32) in two parts leave each wave one or two tiles instead of three or four:
// its step 0.4228 -> 0.4199-0.4204 ms (one, three and six parts: 0.4228,
// 0.4220, 0.4236 ms; four: 0.4197-0.4204, with twice the input staging).
constexpr int HM_PARTS = 2;

struct HeadArgs {
    const int8_t *x;                   // [images][P][IC]
    int8_t *y;                         // [images][OC]
    const int8_t *w;                   // [oc_pad][kpad], zero past K
    const int4 *epi;                   // the conv's records, one per channel
    const uint8_t *lut;                // the conv's optional post table
    int P, IC, OC, kpad;
    int parts;                         // workgroups per image
    int yz, lo, hi;                    // the conv's output zero point and clamp
    int m_xz, m_yz, m_m, m_s;          // the mean's input/output zero points, multiplier, shift
};

template <bool HI, bool CORR>
__global__ __launch_bounds__(64 * HM_WAVES) void k_conv_mean(HeadArgs a)
{
    __shared__ __attribute__((aligned(16))) int8_t X[HM_MAXP * (256 + 16)];
    __shared__ __attribute__((aligned(16))) int8_t lut_s[256];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int fr = lane & 31, fh = lane >> 5;
    const int n = blockIdx.x / a.parts, part = blockIdx.x - n * a.parts;
    const int xs = a.IC + 16;                          // LDS row stride (16-byte pad: rows on distinct banks)

    // The image's pixels into LDS, 16 bytes per thread and step.
    const int8_t *xim = a.x + (long)n * a.P * a.IC;
    const int cpr = a.IC >> 4, chunks = a.P * cpr;
    for (int q = t; q < chunks; q += 64 * HM_WAVES) {
        const int p = q / cpr, c = q - p * cpr;
        *(v4i *)(X + p * xs + c * 16) = *(const v4i *)(xim + (long)p * a.IC + c * 16);
    }
    if (a.lut && t < 64) ((int *)lut_s)[t] = ((const int *)a.lut)[t];
    __syncthreads();

    // This workgroup's channel tiles [c0, c1), a contiguous share per wave.
    const int ks = a.IC >> 5, ctiles = a.OC >> 5;
    const int c0 = part * ctiles / a.parts, c1 = (part + 1) * ctiles / a.parts;
    const int i0 = c0 + wave * (c1 - c0) / HM_WAVES, i1 = c0 + (wave + 1) * (c1 - c0) / HM_WAVES;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    // Weight fragments of tile ct (channel ct*32 + fr, K bytes 32s + 16fh)
    // and its channel's record, loaded one tile ahead.
    auto load = [&](int ct, v4i (&w)[HM_MAXK], Epi &e) {
        const int8_t *wr = a.w + (long)(ct * 32 + fr) * a.kpad + fh * 16;
#pragma unroll
        for (int s = 0; s < HM_MAXK; s++)
            if (s < ks) w[s] = *(const v4i *)(wr + s * 32);
        e = load_epi(a.epi, ct * 32 + fr);
    };
    auto tile = [&](int ct, const v4i (&w)[HM_MAXK], const Epi &e) {
        int sum = 0;
#pragma unroll
        for (int pt = 0; pt < HM_MAXP / 32; pt++) {
            if (pt * 32 >= a.P) break;
            // Rows past the image read its last pixel; their results are not summed.
            const int8_t *sr = X + min(pt * 32 + fr, a.P - 1) * xs + fh * 16;
            v16i acc;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = 0;
#pragma unroll
            for (int s = 0; s < HM_MAXK; s++)
                if (s < ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(*(const v4i *)(sr + s * 32), w[s], acc, 0, 0, 0);
            // acc[4g + i]: pixel pt*32 + 8g + 4fh + i, channel ct*32 + fr.
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int v = conv_requant<HI, CORR>(acc[4 * g + i], e, a.yz, vlo, vhi);
                    if (a.lut) v = (int)lut_s[v + 128];
                    if (pt * 32 + 8 * g + 4 * fh + i < a.P) sum += v;
                }
        }
        // The channel's other pixels are in lane fr + 32.
        sum += __shfl_xor(sum, 32);
        if (fh == 0) {
            const int v = uq_scale(sum - a.P * a.m_xz, a.m_m, a.m_s) + a.m_yz;
            a.y[(long)n * a.OC + ct * 32 + fr] = (int8_t)min(max(v, -128), 127);
        }
    };
    v4i wa[HM_MAXK], wb[HM_MAXK];
    Epi ea, eb;
    if (i0 < i1) load(i0, wa, ea);
    for (int ct = i0; ct < i1; ct += 2) {
        if (ct + 1 < i1) load(ct + 1, wb, eb);
        tile(ct, wa, ea);
        if (ct + 1 >= i1) break;
        if (ct + 2 < i1) load(ct + 2, wa, ea);
        tile(ct + 1, wb, eb);
    }
}

// Whether a 1x1 conv (its descriptor) and the mean over its whole output
// fit the kernel: pointwise, IC a multiple of 32 up to 256, OC a multiple of
// 32, at most 64 pixels per image.
extern "C" int uqk_conv_mean_ok(const UQKSpatial *d)
{
    return d->mode == UQK_PW && d->kh == 1 && d->kw == 1 && d->sh == 1 && d->sw == 1 && d->pt == 0 && d->pl == 0 &&
           d->ic % 32 == 0 && d->ic <= 32 * HM_MAXK && d->oc % 32 == 0 && d->oc_pad >= d->oc && d->K == d->ic &&
           d->kpad >= d->ic && d->oh * d->ow <= HM_MAXP && d->oh * d->ow >= 1;
}

static uint64_t g_cm_launches;

// Launches of the fused conv + mean kernel since the library was loaded (a
// test hook; not part of the plan ABI).
extern "C" uint64_t uqk_conv_mean_launches(void) { return g_cm_launches; }

extern "C" int uqk_conv_mean(const UQKSpatial *d, const UQKMean *mean, const void *x, void *y, uint32_t images)
{
    if (!images) return 0;
    if (!uqk_conv_mean_ok(d) || images > 0x7fffffffU) return (int)hipErrorInvalidValue;
    HeadArgs a;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.P = d->oh * d->ow; a.IC = d->ic; a.OC = d->oc; a.kpad = d->kpad;
    a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.m_xz = mean->xz; a.m_yz = mean->yz; a.m_m = mean->m; a.m_s = mean->s;
    a.parts = mean->parts > 0 ? mean->parts : HM_PARTS;
    if (a.parts > (a.OC >> 5)) a.parts = a.OC >> 5;
    if ((unsigned long long)images * a.parts > 0x7fffffffULL) return (int)hipErrorInvalidValue;
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    const dim3 grid(images * a.parts), block(64 * HM_WAVES);
    switch ((d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0)) {
    case 0: hipExtLaunchKernelGGL((k_conv_mean<false, false>), grid, block, 0, st, e0, e1, 0u, a); break;
    case 1: hipExtLaunchKernelGGL((k_conv_mean<true, false>), grid, block, 0, st, e0, e1, 0u, a); break;
    case 2: hipExtLaunchKernelGGL((k_conv_mean<false, true>), grid, block, 0, st, e0, e1, 0u, a); break;
    default: hipExtLaunchKernelGGL((k_conv_mean<true, true>), grid, block, 0, st, e0, e1, 0u, a); break;
    }
    const int rc = uqk_fail(hipGetLastError());
    if (!rc) g_cm_launches++;
    return rc;
}
