// Stem conv fused with the 3x3 stride-2 conv that consumes its output, for
// gfx950 (two code-14 ops the reference runs one after the other through its
// arena: qnn.c:1101-1169 with the stem's RGB gather, qnn.c:990-1045, then
// the 3x3's column build). The stem's output never goes to HBM: a block
// computes the stem rows that a band of the second conv's output rows needs
// (the band's halo row is computed by both neighbouring blocks), keeps them
// in LDS, and runs the 3x3 from there.
//
// Per block (one image, SC_BR output rows of the second conv, four waves):
//   0  the input rows the band's stem rows touch go to LDS exactly as in
//      k_conv_stem (a 16-byte lead, each row followed by a 16-byte gap, rows
//      outside the image: all of it the stem's input zero point), so a stem
//      window is one unaligned run of LDS bytes; the stem-output stage S is
//      filled with the second conv's input zero point (its padding).
//   1  stem: items (stem row, 16-pixel block); one v_mfma_i32_16x16x64_i8
//      per 16 output channels with the stem weights as the MFMA rows, so a
//      lane holds four channels of one pixel: requantised (stem records and
//      post table) and written as one 4-byte word into S at the pixel's
//      padded column. S is [stem row][column + pl][32 channels].
//   2  3x3 stride 2 over S: groups of four 16-pixel row blocks of the band's
//      output; per 64-byte K step (two taps of 32 channels) one 16-byte LDS
//      read per lane (K past the 9 taps reads a valid tap; its weights are
//      zero); the weights as the MFMA rows, held in registers for the whole
//      phase; the requantised words of four row blocks transposed across
//      16-lane rows (rows_transpose4) into one 16-byte store per lane.
//   3  (optional) a 1x1 conv over 32 channels after the 3x3, whose input
//      is nothing else's: a lane's 32 channels of the 3x3's output (one
//      pixel per lane after phase 2's transpose) become the pixel operand of
//      v_mfma_i32_32x32x32_i8 (one v_permlane32_swap per register pair), the
//      1x1's weights its other operand, and only the 1x1's output is stored.
// Every epilogue uses its layer's own records and requantisation, so the
// bytes equal the separate launches'.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int SC_NT = 2;            // 32 channels in both layers (two 16-channel tiles)
constexpr int SC_C = 32;
constexpr int SC_LDS_MAX = 163840;

struct StemConvArgs {
    const int8_t *x;
    int8_t *y;
    // stem (code 14 in the stem form): weights [32][64] (16 bytes per kernel row)
    const int8_t *ws;
    const int4 *epis;
    const uint8_t *luts;
    int s_ih, s_iw, s_ic, s_kh, s_sh, s_sw, s_dh, s_pt, s_pl, s_xz, s_yz, s_lo, s_hi, s_oh, s_ow;
    // 3x3 stride-2 conv over 32 channels: weights [>= 32][kpad], k = tap * 32 + c
    const int8_t *wc;
    const int4 *epic;
    const uint8_t *lutc;
    int c_kpad, c_oh, c_ow, c_pt, c_pl, c_xz, c_yz, c_lo, c_hi;
    // geometry of a block
    int br, bands;             // output rows of the 3x3 per block, blocks per image
    int srows;                 // stem rows a band needs: (br - 1) * 2 + 3
    int in_rows;               // staged input rows: (srows - 1) * s_sh + (s_kh - 1) * s_dh + 1
    int rs;                    // staged input row stride: s_iw * s_ic + 16
    int cpr;                   // 16-byte pieces per staged row (the last is the gap)
    unsigned m_cpr, m_ow;      // udiv_magic(cpr), udiv_magic(c_ow)
    int cols;                  // columns of S: (c_ow - 1) * 2 + 3
    int o_s, o_es, o_ec, o_ls, o_lc, o_lp;   // LDS offsets: S, stem records, conv records, post tables
    // optional 1x1 conv over the 3x3's output (32 -> 32 channels): weights
    // [>= 32][p_kpad], its records, post table and requantisation variant
    const int8_t *wp;
    const int4 *epip;
    const uint8_t *lutp;
    int p_kpad, p_mode, p_yz, p_lo, p_hi;
};

// The 1x1 conv over 64 pixels of the 3x3's output, lane L holding the 32
// channels of pixel L as h0 (channels 0-15) and h1 (16-31): one
// v_permlane32_swap per register pair gives the two 32-pixel A operands of
// v_mfma_i32_32x32x32_i8 (rows: pixels, K: lanes < 32 channels 0-15, the
// others 16-31); the weights are its columns (lane: output channel
// lane & 31, K half lane >> 5), so a lane's 16 results share one channel and
// its record; a 4x4 byte transpose across lane quads gives each lane four
// channels of one pixel, stored as one word.
template <bool HI, bool CORR>
__device__ __forceinline__ void stem_pw(const StemConvArgs &a, const int (&h0)[4], const int (&h1)[4], const v4i &wpf,
                                        const Epi &ep, const int8_t *lut_p, int8_t *yg, int px0, int npx)
{
    const int lane = threadIdx.x & 63, fr = lane & 31, fh = lane >> 5;
    const int vlo = vgpr(a.p_lo), vhi = vgpr(a.p_hi);
    v4i A[2];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const auto sw = __builtin_amdgcn_permlane32_swap(h0[j], h1[j], false, false);
        A[0][j] = (int)sw[0];
        A[1][j] = (int)sw[1];
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        v16i acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0;
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[t], wpf, acc, 0, 0, 0);
        // acc[4g + i]: pixel px0 + 32t + 8g + 4fh + i, channel fr.
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = conv_requant<HI, CORR>(acc[4 * g + i], ep, a.p_yz, vlo, vhi);
                if (a.lutp) v[i] = lut_p[v[i] + 128];
            }
            const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
            const int px = px0 + 32 * t + 8 * g + 4 * fh + (lane & 3);
            if (px < npx) *(int *)(yg + __mul24(px, SC_C) + (fr & ~3)) = word;
        }
    }
}

// WPE: the waves per SIMD the register allocation must allow (1: no limit).
// Four let four blocks share a compute unit; the host takes that variant
// only when it compiled without spilling (uqk_stem_conv).
template <int EMS, int EMC, bool PW, int WPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) void k_stem_conv(StemConvArgs a)
{
    constexpr bool HS = EMS & 1, CS = EMS & 2, HC = EMC & 1, CC = EMC & 2;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t *S = smem + a.o_s;
    const int4 *es = (const int4 *)(smem + a.o_es), *ec = (const int4 *)(smem + a.o_ec);
    const int8_t *lut_s = smem + a.o_ls, *lut_c = smem + a.o_lc, *lut_p = smem + a.o_lp;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int n = blockIdx.x / a.bands, band = blockIdx.x - n * a.bands;
    const int r0 = band * a.br, brows = min(a.br, a.c_oh - r0);
    const int s0 = r0 * 2 - a.c_pt;                    // stem row of S row 0
    const int iy_base = s0 * a.s_sh - a.s_pt;          // input row of staged row 0

    // Stem weights (MFMA rows: channel nt*16 + lr, kernel row lg), the 3x3's
    // weights for all five K steps and the 1x1's, loaded while the block
    // stages.
    v4i wsf[SC_NT];
#pragma unroll
    for (int nt = 0; nt < SC_NT; nt++) wsf[nt] = *(const v4i *)(a.ws + (long)(nt * 16 + lr) * 64 + lg * 16);
    v4i wcf[SC_NT][5];
#pragma unroll
    for (int nt = 0; nt < SC_NT; nt++)
#pragma unroll
        for (int s = 0; s < 5; s++) wcf[nt][s] = *(const v4i *)(a.wc + (long)(nt * 16 + lr) * a.c_kpad + s * 64 + lg * 16);
    // The 1x1's weights (its MFMA columns: channel lane & 31, K half lane >> 5)
    // and its channel's record.
    v4i wpf = {0, 0, 0, 0};
    Epi ep = {};
    if (PW) {
        wpf = *(const v4i *)(a.wp + (long)(lane & 31) * a.p_kpad + (lane >> 5) * 16);
        ep = load_epi(a.epip, lane & 31);
    }

    // Phase 0.
    {
        const int sxz = (a.s_xz & 0xff) * 0x01010101, cxz = (a.c_xz & 0xff) * 0x01010101;
        const v4i sxv = {sxz, sxz, sxz, sxz}, cxv = {cxz, cxz, cxz, cxz};
        const int rowbytes = a.s_iw * a.s_ic, total = a.in_rows * a.cpr;
        const int8_t *xim = a.x + (long)n * a.s_ih * rowbytes;
        for (int c0 = tid; c0 < total; c0 += 4 * 256) {
            v4i v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + j * 256;
                const int r = (int)udiv((unsigned)c, (unsigned)a.cpr, a.m_cpr), k = c - r * a.cpr;
                const int iy = iy_base + r;
                v[j] = sxv;
                if (c < total && k < a.cpr - 1 && (unsigned)iy < (unsigned)a.s_ih)
                    v[j] = *(const v4i *)(xim + (long)iy * rowbytes + k * 16);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + j * 256;
                if (c < total) ((v4i *)smem)[1 + c] = v[j];
            }
        }
        if (tid == 0) ((v4i *)smem)[0] = sxv;
        for (int q = tid; q < a.srows * a.cols * (SC_C / 16); q += 256) ((v4i *)S)[q] = cxv;
        for (int i = tid; i < 2 * SC_C; i += 256) {
            ((int4 *)es)[i] = a.epis[i];
            ((int4 *)ec)[i] = a.epic[i];
        }
        if (tid < 64) {
            if (a.luts) ((int *)lut_s)[tid] = ((const int *)a.luts)[tid];
            if (a.lutc) ((int *)lut_c)[tid] = ((const int *)a.lutc)[tid];
            if (PW && a.lutp) ((int *)lut_p)[tid] = ((const int *)a.lutp)[tid];
        }
    }
    __syncthreads();

    // Phase 1: stem rows s0 .. s0 + srows - 1 (those inside the map).
    {
        const int vlo = vgpr(a.s_lo), vhi = vgpr(a.s_hi);
        Epi e[SC_NT][4];
#pragma unroll
        for (int nt = 0; nt < SC_NT; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) e[nt][i] = load_epi(es, nt * 16 + 4 * lg + i);
        const int ky = lg < a.s_kh ? lg : 0;
        const int step = a.s_sw * a.s_ic;
        const int rbs = (a.s_ow + 15) >> 4, items = a.srows * rbs;
        for (int item = wave; item < items; item += 4) {
            const int j = item / rbs, rb = item - j * rbs, s = s0 + j;
            if ((unsigned)s >= (unsigned)a.s_oh) continue;
            const int ox = min(rb * 16 + lr, a.s_ow - 1);
            const int off = 16 + (j * a.s_sh + ky * a.s_dh) * a.rs - a.s_pl * a.s_ic + __mul24(ox, step);
            const int *p = (const int *)(smem + (off & ~3));
            const int w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
            const unsigned sh = (unsigned)off;
            const v4i A = {(int)__builtin_amdgcn_alignbyte((unsigned)w1, (unsigned)w0, sh),
                           (int)__builtin_amdgcn_alignbyte((unsigned)w2, (unsigned)w1, sh),
                           (int)__builtin_amdgcn_alignbyte((unsigned)w3, (unsigned)w2, sh),
                           (int)__builtin_amdgcn_alignbyte((unsigned)w4, (unsigned)w3, sh)};
            // Columns past the 3x3's reach are not needed (nor stored).
            const bool keep = rb * 16 + lr < a.s_ow && rb * 16 + lr + a.c_pl < a.cols;
            int8_t *dst = S + ((j * a.cols) + rb * 16 + lr + a.c_pl) * SC_C + 4 * lg;
#pragma unroll
            for (int nt = 0; nt < SC_NT; nt++) {
                // acc[i]: channel nt*16 + 4*lg + i of pixel ox.
                const v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wsf[nt], A, (v4i){0, 0, 0, 0}, 0, 0, 0);
                int v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[i] = conv_requant<HS, CS>(acc[i], e[nt][i], a.s_yz, vlo, vhi);
                    if (a.luts) v[i] = lut_s[v[i] + 128];
                }
                if (keep) *(int *)(dst + nt * 16) = pack4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    __syncthreads();

    // Phase 2: the 3x3 stride 2 over S, four 16-pixel row blocks per item.
    {
        const int vlo = vgpr(a.c_lo), vhi = vgpr(a.c_hi);
        // K step s, lane group lg: 16 bytes at k = s*64 + lg*16 of tap k/32
        // (taps past 8 read tap 8: their weights are zero).
        int toff[5];
#pragma unroll
        for (int s = 0; s < 5; s++) {
            const int k = s * 64 + lg * 16, tap = min(k >> 5, 8), ky = tap / 3, kx = tap - ky * 3;
            toff[s] = (ky * a.cols + kx) * SC_C + ((k >> 4) & 1) * 16;
        }
        const int npx = brows * a.c_ow, groups = (npx + 63) >> 6;
        int8_t *ybase = a.y + ((long)n * a.c_oh + r0) * a.c_ow * SC_C;
        for (int g = wave; g < groups; g += 4) {
            v4i acc[4][SC_NT];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int px = min(g * 64 + rb * 16 + lr, npx - 1);
                const int rr = (int)udiv((unsigned)px, (unsigned)a.c_ow, a.m_ow), c = px - rr * a.c_ow;
                const int8_t *base = S + ((2 * rr) * a.cols + 2 * c) * SC_C;
#pragma unroll
                for (int nt = 0; nt < SC_NT; nt++) acc[rb][nt] = (v4i){0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < 5; s++) {
                    const v4i b = *(const v4i *)(base + toff[s]);
#pragma unroll
                    for (int nt = 0; nt < SC_NT; nt++)
                        acc[rb][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wcf[nt][s], b, acc[rb][nt], 0, 0, 0);
                }
            }
            // acc[rb][nt][i]: channel nt*16 + 4*lg + i of pixel g*64 + rb*16 + lr.
            int h[SC_NT][4];
#pragma unroll
            for (int nt = 0; nt < SC_NT; nt++) {
                Epi e[4];
#pragma unroll
                for (int i = 0; i < 4; i++) e[i] = load_epi(ec, nt * 16 + 4 * lg + i);
                int r[4];
#pragma unroll
                for (int rb = 0; rb < 4; rb++) {
                    int v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[i] = conv_requant<HC, CC>(acc[rb][nt][i], e[i], a.c_yz, vlo, vhi);
                        if (a.lutc) v[i] = lut_c[v[i] + 128];
                    }
                    r[rb] = pack4(v[0], v[1], v[2], v[3]);
                }
                rows_transpose4(r);
                // Lane (lr, lg) now holds the 16 channels of pixel g*64 + lg*16 + lr.
                const int px = g * 64 + lg * 16 + lr;
                if (!PW && px < npx) *(v4i *)(ybase + __mul24(px, SC_C) + nt * 16) = (v4i){r[0], r[1], r[2], r[3]};
#pragma unroll
                for (int q = 0; q < 4; q++) h[nt][q] = r[q];
            }
            if (PW) {
                switch (a.p_mode) {
                case 0: stem_pw<false, false>(a, h[0], h[1], wpf, ep, lut_p, ybase, g * 64, npx); break;
                case 1: stem_pw<true, false>(a, h[0], h[1], wpf, ep, lut_p, ybase, g * 64, npx); break;
                case 2: stem_pw<false, true>(a, h[0], h[1], wpf, ep, lut_p, ybase, g * 64, npx); break;
                default: stem_pw<true, true>(a, h[0], h[1], wpf, ep, lut_p, ybase, g * 64, npx); break;
                }
            }
        }
    }
}

// Whether a 1x1 conv over the 3x3's output fits phase 3: 32 -> 32 channels,
// stride 1, no padding or dilation, weights rows of 32 (or more, zero) bytes.
static int sc_pw_fits(const UQKSpatial *c, const UQKSpatial *p)
{
    return p->mode == UQK_PW && p->kh == 1 && p->kw == 1 && p->sh == 1 && p->sw == 1 && p->pt == 0 && p->pl == 0 &&
           p->ic == SC_C && p->oc == SC_C && p->oc_pad >= SC_C && p->K == SC_C && p->kpad >= SC_C &&
           p->ih == c->oh && p->iw == c->ow && p->oh == c->oh && p->ow == c->ow;
}

// Block geometry and LDS bytes; 0 when the pair does not fit the kernel.
static size_t sc_plan(const UQKSpatial *s, const UQKSpatial *c, int br, StemConvArgs *t)
{
    if (s->mode != UQK_STEM || s->oc != SC_C || s->oc_pad != SC_C || c->ic != SC_C || c->oc != SC_C ||
        c->kh != 3 || c->kw != 3 || c->sh != 2 || c->sw != 2 || c->dh != 1 || c->dw != 1 || c->K != 9 * SC_C ||
        c->kpad != 320 || c->mode == UQK_ROWS4 || c->mode == UQK_STEM || c->ih != s->oh || c->iw != s->ow ||
        c->pt < 0 || c->pt > 2 || c->pl < 0 || c->pl > 2 || c->oh < 1 || c->ow < 1)
        return 0;
    t->br = br;
    t->bands = (c->oh + br - 1) / br;
    t->srows = (br - 1) * 2 + 3;
    t->in_rows = (t->srows - 1) * s->sh + (s->kh - 1) * s->dh + 1;
    t->rs = s->iw * s->ic + 16;
    t->cpr = s->iw * s->ic / 16 + 1;
    t->cols = (c->ow - 1) * 2 + 3;
    size_t o = 16 + (size_t)t->in_rows * t->rs + 32;
    o = (o + 15) & ~(size_t)15;
    t->o_s = (int)o; o += (size_t)t->srows * t->cols * SC_C;
    t->o_es = (int)o; o += SC_C * 32;
    t->o_ec = (int)o; o += SC_C * 32;
    t->o_ls = (int)o; o += 256;
    t->o_lc = (int)o; o += 256;
    t->o_lp = (int)o; o += 256;
    return o <= (size_t)SC_LDS_MAX ? o : 0;
}

// Output rows of the 3x3 per block: on MobileNetV4-S at batch 256 three
// measured 0.468 ms per step, against 0.477 / 0.471 / 0.489 / 0.535 for two,
// four, six and eight (more rows recompute fewer halo stem rows but hold
// more LDS per block).
static const int SC_BR = 3;

extern "C" int uqk_stem_conv_ok(const UQKSpatial *s, const UQKSpatial *c, const UQKSpatial *p)
{
    StemConvArgs t;
    return uqk_conv_stem_ok(s) && sc_plan(s, c, SC_BR, &t) > 0 && (!p || sc_pw_fits(c, p));
}

static uint64_t g_sc_launches;

// Launch the four-waves-per-SIMD variant of a kernel instance when it needs
// no scratch memory (no spilled registers), else the unrestricted one; the
// choice is made once per instance.
template <int EMS, int EMC, bool PW>
static void sc_launch(dim3 grid, dim3 block, size_t lds, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                      const StemConvArgs &a)
{
    static int use4 = -1;
    if (use4 < 0) {
        hipFuncAttributes fa;
        use4 = hipFuncGetAttributes(&fa, (const void *)k_stem_conv<EMS, EMC, PW, 4>) == hipSuccess &&
               fa.localSizeBytes == 0;
    }
    if (use4) hipExtLaunchKernelGGL((k_stem_conv<EMS, EMC, PW, 4>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a);
    else hipExtLaunchKernelGGL((k_stem_conv<EMS, EMC, PW, 1>), grid, block, (uint32_t)lds, st, e0, e1, 0u, a);
}

// Launches of the fused stem kernel since the library was loaded (a test
// hook; not part of the plan ABI).
extern "C" uint64_t uqk_stem_conv_launches(void) { return g_sc_launches; }

extern "C" int uqk_stem_conv(const UQKSpatial *s, const UQKSpatial *c, const UQKSpatial *p, const void *x, void *y,
                             uint32_t images)
{
    if (!images) return 0;
    StemConvArgs a;
    const size_t lds = sc_plan(s, c, SC_BR, &a);
    if (!lds || !uqk_conv_stem_ok(s) || (p && !sc_pw_fits(c, p))) return (int)hipErrorInvalidValue;
    const unsigned long long blocks = (unsigned long long)images * a.bands;
    if (blocks > 0x7fffffffULL || (unsigned long long)s->ih * s->iw * s->ic > 0x7fffffffULL)
        return (int)hipErrorInvalidValue;
    a.x = (const int8_t *)x; a.y = (int8_t *)y;
    a.ws = (const int8_t *)s->w; a.epis = (const int4 *)s->epi; a.luts = (const uint8_t *)s->lut;
    a.s_ih = s->ih; a.s_iw = s->iw; a.s_ic = s->ic; a.s_kh = s->kh; a.s_sh = s->sh; a.s_sw = s->sw; a.s_dh = s->dh;
    a.s_pt = s->pt; a.s_pl = s->pl; a.s_xz = s->xz; a.s_yz = s->yz; a.s_lo = s->lo; a.s_hi = s->hi;
    a.s_oh = s->oh; a.s_ow = s->ow;
    a.wc = (const int8_t *)c->w; a.epic = (const int4 *)c->epi; a.lutc = (const uint8_t *)c->lut;
    a.c_kpad = c->kpad; a.c_oh = c->oh; a.c_ow = c->ow; a.c_pt = c->pt; a.c_pl = c->pl; a.c_xz = c->xz;
    a.c_yz = c->yz; a.c_lo = c->lo; a.c_hi = c->hi;
    a.m_cpr = udiv_magic((unsigned)a.cpr);
    a.m_ow = udiv_magic((unsigned)c->ow);
    a.wp = nullptr; a.epip = nullptr; a.lutp = nullptr;
    a.p_kpad = a.p_mode = a.p_yz = a.p_lo = a.p_hi = 0;
    if (p) {
        a.wp = (const int8_t *)p->w; a.epip = (const int4 *)p->epi; a.lutp = (const uint8_t *)p->lut;
        a.p_kpad = p->kpad; a.p_mode = (p->hi_shift ? 1 : 0) | (p->corr ? 2 : 0);
        a.p_yz = p->yz; a.p_lo = p->lo; a.p_hi = p->hi;
    }
    const int ems = (s->hi_shift ? 1 : 0) | (s->corr ? 2 : 0), emc = (c->hi_shift ? 1 : 0) | (c->corr ? 2 : 0);
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    const dim3 grid((unsigned)blocks), block(256);
#define SC_L(S, C)                                                                    \
    do {                                                                              \
        if (p) sc_launch<S, C, true>(grid, block, lds, st, e0, e1, a);                \
        else sc_launch<S, C, false>(grid, block, lds, st, e0, e1, a);                 \
    } while (0)
#define SC_EMC(S)                       \
    do {                                \
        switch (emc) {                  \
        case 0: SC_L(S, 0); break;      \
        case 1: SC_L(S, 1); break;      \
        case 2: SC_L(S, 2); break;      \
        default: SC_L(S, 3); break;     \
        }                               \
    } while (0)
    switch (ems) {
    case 0: SC_EMC(0); break;
    case 1: SC_EMC(1); break;
    case 2: SC_EMC(2); break;
    default: SC_EMC(3); break;
    }
#undef SC_EMC
#undef SC_L
    const int rc = uqk_fail(hipGetLastError());
    if (!rc) g_sc_launches++;
    return rc;
}
