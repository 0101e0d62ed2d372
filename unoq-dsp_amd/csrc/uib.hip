// Fused universal inverted bottleneck for gfx950, by bands of output rows:
//   [start depthwise, stride 1] -> 1x1 expand -> [depthwise, stride 1 or 2]
//   -> 1x1 project [-> residual add with the block input]
// (MobileNetV4's ExtraDW and the inverted bottlenecks with a stride-2
// depthwise; the reference runs these as three to five ops one after another
// through HBM: qnn.c:807-983 for the depthwise, qnn.c:1074-1246 for the 1x1
// convs, qnn.c:1248-1290 for the add). One workgroup of 16 waves takes one
// image's band of R output rows: it stages the input rows the band reaches,
// computes every intermediate row the band needs in LDS (the rows under the
// windows of two neighbouring bands are computed by both), and writes the
// band's output rows. Each phase is the arithmetic of the separate kernels
// (the layers' own operand bytes, records, requantisation and post tables),
// so the bytes are those of the unfused ops.
//
// Phases, separated by barriers:
//   0  input: with a start depthwise, its window planes ([Cin / 16] planes of
//      the padded rows the band reaches, 16 channels a position, padding at
//      the start depthwise's input zero point); without one, the input rows.
//      The depthwise window planes filled with its input zero point; the
//      layers' records, tap words, post tables and the add's tables; the
//      per-pixel position tables of each phase.
//   1  start depthwise (ib_dw_mode) into rows X1 [Pe][Cin + 16].
//   2  expand (ib_gemm, 32x32 tiles) of the Pe = rows x W pixels the band
//      needs, into the depthwise window planes at each pixel's padded
//      position (or, without a depthwise, into the rows D).
//   3  depthwise (ib_dw_mode) of the band's Po = rows x Wo output pixels,
//      window corners from a per-pixel table (so stride 2 is the same code),
//      into rows D [Po][Ce + 16].
//   4  project (16x16 or 32x32 tiles as in k_ib) with the fused add reading
//      the block input from the staged input (planes or rows); the output
//      staged in LDS over a region free by then, then 16-byte stores.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"
#include "ib_phases.h"

constexpr int UIB_LDS_MAX = 163840;

struct UibArgs {
    const int8_t *x;
    int8_t *y;
    int H, W, Ho, Wo, Cin, Ce, Cout;
    int R, bands;              // output rows per band, bands per image
    // start depthwise (k0 = 0: none): stride 1, pads p0t / p0l, X planes
    // cols0 = W + k0 - 1 positions wide
    int k0, p0t, p0l, cols0;
    const int *dw0;            // tap words [ky][k0 > 4 ? 2 : 1][Cin]
    const int4 *epi0;
    const uint8_t *lut0;
    int m0, yz0, lo0, hi0, xz0;
    const int8_t *we;          // expand weights [>= Ce][kpe]
    const int4 *epi_e;
    const uint8_t *lut_e;
    int kpe, e_mode, e_yz, e_lo, e_hi;
    // depthwise (k = 0: none): stride s, pads pt / pl, E planes cols_p wide
    int k, s, pt, pl, cols_p;
    const int *dww;            // tap words [ky][k > 4 ? 2 : 1][Ce]
    const int4 *epi_d;
    const uint8_t *lut_d;
    int d_mode, d_yz, d_lo, d_hi, d_xz;
    const int8_t *wp;          // project weights [>= Cout][kpp]
    const int4 *epi_p;
    const uint8_t *lut_p;
    int kpp, p_mode, p_yz, p_lo, p_hi;
    int has_add, add_x_first;
    const int *add_tab;
    int a_m, a_s, a_yz, a_lo, a_hi;
    long long a_c1, a_thr;     // the add's rescale as one multiply-add (s < 0)
    int a_hs;
    unsigned m_w, m_wo, m_cq, m_c0;   // udiv_magic(W), (Wo), (Cin / 16), (cols0)
    int xs, x1s, ds;           // LDS row strides: X rows, X1 rows, D rows
    int rec_lds;               // expand and depthwise records staged in LDS (else read from global memory)
    // LDS offsets: X1, E, D, records (start, expand, depthwise, project), add
    // tables, post tables, position tables (start, expand, depthwise, add),
    // tap words (start, depthwise)
    int o_x1, o_e, o_d, o_r0, o_re, o_rd, o_rp, o_at, o_lut, o_t0, o_te, o_td, o_ta, o_w0, o_wd;
};

template <int K0, int K>
__global__ __launch_bounds__(64 * IB_WAVES) void k_uib(UibArgs a)
{
    constexpr int NT = 64 * IB_WAVES;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t *X = smem, *X1 = smem + a.o_x1, *E = smem + a.o_e, *D = smem + a.o_d;
    int8_t *lut_s = smem + a.o_lut;
    const int *at = (const int *)(smem + a.o_at);
    int *t0 = (int *)(smem + a.o_t0), *te = (int *)(smem + a.o_te), *td = (int *)(smem + a.o_td);
    int *ta = (int *)(smem + a.o_ta);
    const int tid = threadIdx.x;
    const int n = blockIdx.x / a.bands, band = blockIdx.x - n * a.bands;
    const int r0 = band * a.R, rb = min(a.R, a.Ho - r0);
    // Rows of the expanded map the band needs (plane rows, padding included)
    // and those of them inside the map.
    const int ye_lo = K ? r0 * a.s - a.pt : r0, ye_hi = K ? (r0 + rb - 1) * a.s - a.pt + K - 1 : r0 + rb - 1;
    const int v_lo = max(ye_lo, 0), v_hi = min(ye_hi, a.H - 1);
    const int Pe = (v_hi - v_lo + 1) * a.W, Po = rb * a.Wo;
    const int planeE = (ye_hi - ye_lo + 1) * a.cols_p;
    const int plane0 = (v_hi - v_lo + K0) * a.cols0;   // rows v_lo - p0t .. v_hi - p0t + k0 - 1
    const int8_t *xim = a.x + (long)n * a.H * a.W * a.Cin;
    const int cq = a.Cin >> 4;

    // Phase 0.
    {
        if (K0) {
            // Plane position order, 16-channel group fastest: consecutive
            // lanes read consecutive 16-byte pieces of an input row.
            const int xzw = (a.xz0 & 0xff) * 0x01010101;
            const v4i xzv = {xzw, xzw, xzw, xzw};
            const int total = plane0 * cq;
            for (int q = tid; q < total; q += NT) {
                const int pos = (int)udiv((unsigned)q, (unsigned)cq, a.m_cq), g = q - pos * cq;
                const int j = (int)udiv((unsigned)pos, (unsigned)a.cols0, a.m_c0), c = pos - j * a.cols0;
                const int iy = v_lo - a.p0t + j, ix = c - a.p0l;
                v4i v = xzv;
                if ((unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
                    v = *(const v4i *)(xim + ((long)iy * a.W + ix) * a.Cin + g * 16);
                *(v4i *)(X + (g * plane0 + pos) * 16) = v;
            }
        } else {
            const int8_t *src = xim + (long)v_lo * a.W * a.Cin;
            for (int q = tid; q < Pe * cq; q += NT) {
                const int p = (int)udiv((unsigned)q, (unsigned)cq, a.m_cq), j = q - p * cq;
                *(v4i *)(X + p * a.xs + j * 16) = *(const v4i *)(src + (long)q * 16);
            }
        }
        if (K) {
            const int xzw = (a.d_xz & 0xff) * 0x01010101;
            const v4i xzv = {xzw, xzw, xzw, xzw};
            for (int q = tid; q < (a.Ce >> 4) * planeE; q += NT) ((v4i *)E)[q] = xzv;
        }
        if (a.rec_lds)
            for (int i = tid; i < 2 * a.Ce; i += NT) {
                ((int4 *)(smem + a.o_re))[i] = a.epi_e[i];
                if (K) ((int4 *)(smem + a.o_rd))[i] = a.epi_d[i];
            }
        for (int i = tid; i < 2 * a.Cout; i += NT) ((int4 *)(smem + a.o_rp))[i] = a.epi_p[i];
        if (K0) {
            for (int i = tid; i < 2 * a.Cin; i += NT) ((int4 *)(smem + a.o_r0))[i] = a.epi0[i];
            for (int i = tid; i < K0 * (K0 > 4 ? 2 : 1) * a.Cin; i += NT) ((int *)(smem + a.o_w0))[i] = a.dw0[i];
        }
        if (K)
            for (int i = tid; i < K * (K > 4 ? 2 : 1) * a.Ce; i += NT) ((int *)(smem + a.o_wd))[i] = a.dww[i];
        if (a.has_add)
            for (int i = tid; i < 512; i += NT) ((int *)(smem + a.o_at))[i] = a.add_tab[i];
        if (tid < 64) {
            if (a.lut_e) ((int *)lut_s)[tid] = ((const int *)a.lut_e)[tid];
            if (a.lut_d) ((int *)(lut_s + 256))[tid] = ((const int *)a.lut_d)[tid];
            if (a.lut_p) ((int *)(lut_s + 512))[tid] = ((const int *)a.lut_p)[tid];
            if (a.lut0) ((int *)(lut_s + 768))[tid] = ((const int *)a.lut0)[tid];
        }
        // Expanded pixel q (row v_lo + q / W): its start-depthwise window
        // corner in the X planes and its padded position in the E planes
        // (-1 past the columns any window reads).
        for (int q = tid; q < Pe; q += NT) {
            const int y = (int)udiv((unsigned)q, (unsigned)a.W, a.m_w), x = q - y * a.W;
            if (K0) t0[q] = y * a.cols0 + x;
            if (K) te[q] = x + a.pl < a.cols_p ? (y + v_lo - ye_lo) * a.cols_p + x + a.pl : -1;
        }
        // Output pixel p of the band: its window corner in the E planes, and
        // where the add finds the block input (a plane position or an X row).
        for (int p = tid; p < Po; p += NT) {
            const int oy = (int)udiv((unsigned)p, (unsigned)a.Wo, a.m_wo), ox = p - oy * a.Wo;
            if (K) td[p] = oy * a.s * a.cols_p + ox * a.s;
            if (a.has_add) ta[p] = K0 ? (r0 + oy - v_lo + a.p0t) * a.cols0 + ox + a.p0l : (r0 + oy - v_lo) * a.W + ox;
        }
    }
    __syncthreads();

    // Phase 1: start depthwise into X1.
    if constexpr (K0 > 0) {
        const DwPh g = {Pe, a.Cin, a.x1s, a.cols0, 0, a.yz0, a.lo0, a.hi0, (const int4 *)(smem + a.o_r0),
                        a.lut0 ? lut_s + 768 : nullptr};
        ib_dw_mode<K0>(a.m0, g, X, X1, t0, (const int *)(smem + a.o_w0), plane0);
        __syncthreads();
    }

    // Phase 2: expand.
    {
        const int8_t *src = K0 ? X1 : X;
        const int ss = K0 ? a.x1s : a.xs;
        const int4 *rec = a.rec_lds ? (const int4 *)(smem + a.o_re) : a.epi_e;
        v4i wfe[8];
        int wfe_ct = -1;
        if (K) {
            ib_gemm_mode<8>(a.e_mode, wfe, wfe_ct, a.we, a.kpe, a.Cin >> 5, src, ss, Pe, a.Ce >> 5, rec,
                            a.e_yz, a.e_lo, a.e_hi, a.lut_e ? lut_s : nullptr, [&](int p, int c, int word) {
                                const int pos = te[p];
                                if (pos >= 0) *(int *)(E + (__mul24(c >> 4, planeE) + pos) * 16 + (c & 15)) = word;
                            });
        } else {
            ib_gemm_mode<8>(a.e_mode, wfe, wfe_ct, a.we, a.kpe, a.Cin >> 5, src, ss, Pe, a.Ce >> 5, rec,
                            a.e_yz, a.e_lo, a.e_hi, a.lut_e ? lut_s : nullptr,
                            [&](int p, int c, int word) { *(int *)(D + __mul24(p, a.ds) + c) = word; });
        }
    }
    __syncthreads();

    // Phase 3: depthwise into D.
    if constexpr (K > 0) {
        const DwPh g = {Po, a.Ce, a.ds, a.cols_p, 0, a.d_yz, a.d_lo, a.d_hi,
                        a.rec_lds ? (const int4 *)(smem + a.o_rd) : a.epi_d, a.lut_d ? lut_s + 256 : nullptr};
        ib_dw_mode<K>(a.d_mode, g, E, D, td, (const int *)(smem + a.o_wd), planeE);
        __syncthreads();
    }

    // Phase 4: project (+ residual add) into the output stage, then out.
    // The add's rescale as in k_ib (one multiply-add, a_c1 / a_thr / a_hs).
    int8_t *S = K ? E : X1;
    const int *atab = at + (a.add_x_first ? 0 : 256), *btab = at + (a.add_x_first ? 256 : 0);
    auto project_sink = [&](int p, int c, int word) {
        if (a.has_add) {
            const int xr = K0 ? *(const int *)(X + (__mul24(c >> 4, plane0) + ta[p]) * 16 + (c & 15))
                              : *(const int *)(X + __mul24(ta[p], a.xs) + c);
            const int vlo = vgpr(a.a_lo), vhi = vgpr(a.a_hi);
            int z[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int sum = atab[sbyte(xr, i) + 128] + btab[sbyte(word, i) + 128];
                int r;
                if (a.a_s < 0) {
                    long long q = (long long)sum * a.a_m + a.a_c1;
                    if (q < a.a_thr) q -= 1LL << 31;
                    r = (int)(q >> 32) >> a.a_hs;
                } else {
                    r = (int)(((long long)(int)((unsigned)sum << a.a_s) * a.a_m + (1LL << 30)) >> 31);
                }
                z[i] = med3(r + a.a_yz, vlo, vhi);
            }
            word = pack4(z[0], z[1], z[2], z[3]);
        }
        *(int *)(S + __mul24(p, a.Cout) + c) = word;
    };
    const int i32 = (a.Cout >> 5) * ((Po + 31) >> 5), i16 = (a.Cout >> 4) * ((Po + 15) >> 4);
    if ((i32 + IB_WAVES - 1) / IB_WAVES * 16 <= (i16 + IB_WAVES - 1) / IB_WAVES * 4) {
        v4i wfp[16];
        int wfp_ct = -1;
        ib_gemm_mode<16>(a.p_mode, wfp, wfp_ct, a.wp, a.kpp, a.Ce >> 5, D, a.ds, Po, a.Cout >> 5,
                         (const int4 *)(smem + a.o_rp), a.p_yz, a.p_lo, a.p_hi, a.lut_p ? lut_s + 512 : nullptr,
                         project_sink);
    } else {
        ib_gemm16_mode<8>(a.p_mode, a.wp, a.kpp, (a.Ce + 63) >> 6, D, a.ds, Po, a.Cout >> 4,
                          (const int4 *)(smem + a.o_rp), a.p_yz, a.p_lo, a.p_hi, a.lut_p ? lut_s + 512 : nullptr,
                          project_sink);
    }
    __syncthreads();
    int8_t *yim = a.y + ((long)n * a.Ho + r0) * a.Wo * a.Cout;
    for (int q = tid; q < (Po * a.Cout) >> 4; q += NT) ((v4i *)yim)[q] = ((const v4i *)S)[q];
}

static size_t up16(size_t v) { return (v + 15) & ~(size_t)15; }

// LDS layout for bands of R output rows, with the expand and depthwise
// records in LDS or not; 0 when the block does not fit.
static size_t uib_layout(const UQKUib *f, int R, int rec_lds, UibArgs *t)
{
    const int K0 = f->k0, K = f->k, s = K ? f->s : 1;
    // Expanded rows a band needs, and those inside the map, at most.
    const int re = K ? (R - 1) * s + K : R;
    const int rv = re < f->H ? re : f->H;
    const size_t Pe = (size_t)rv * f->W, Po = (size_t)R * f->Wo;
    const int cols0 = f->W + K0 - 1;
    const int cols_p = K ? (f->Wo - 1) * s + K : 0;
    size_t o = 0;
    o += up16(K0 ? (size_t)(f->Cin / 16) * (rv + K0 - 1) * cols0 * 16 : Pe * (f->Cin + 16));   // X
    t->o_x1 = (int)o; o += up16(K0 ? Pe * (f->Cin + 16) : 0);
    t->o_e = (int)o; o += up16(K ? (size_t)(f->Ce / 16) * re * cols_p * 16 : 0);
    t->o_d = (int)o; o += up16((K ? Po : Pe) * (f->Ce + 16)) + 64;   // + the 16x16 project's K-tail over-read
    t->o_r0 = (int)o; o += K0 ? (size_t)f->Cin * 32 : 0;
    t->o_re = (int)o; o += rec_lds ? (size_t)f->Ce * 32 : 0;
    t->o_rd = (int)o; o += rec_lds && K ? (size_t)f->Ce * 32 : 0;
    t->o_rp = (int)o; o += (size_t)f->Cout * 32;
    t->o_at = (int)o; o += f->has_add ? 512 * 4 : 0;
    t->o_lut = (int)o; o += 4 * 256;
    t->o_t0 = (int)o; o += up16(K0 ? Pe * 4 : 0);
    t->o_te = (int)o; o += up16(K ? Pe * 4 : 0);
    t->o_td = (int)o; o += up16(K ? Po * 4 : 0);
    t->o_ta = (int)o; o += up16(f->has_add ? Po * 4 : 0);
    t->o_w0 = (int)o; o += up16(K0 ? (size_t)K0 * (K0 > 4 ? 2 : 1) * f->Cin * 4 : 0);
    t->o_wd = (int)o; o += up16(K ? (size_t)K * (K > 4 ? 2 : 1) * f->Ce * 4 : 0);
    // The output stage [Po][Cout] lies over the E planes, or over X1.
    const size_t stage = K ? (size_t)(t->o_d - t->o_e) : (size_t)(t->o_e - t->o_x1);
    if (Po * f->Cout > stage) return 0;
    t->cols0 = cols0;
    t->cols_p = cols_p;
    t->rec_lds = rec_lds;
    return o <= (size_t)UIB_LDS_MAX ? o : 0;
}

extern "C" size_t uqk_uib_plan(UQKUib *f)
{
    const int K0 = f->k0, K = f->k;
    f->R = 0;
    if (f->H < 1 || f->W < 1 || f->Ho < 1 || f->Wo < 1 || f->Cin % 32 || f->Ce % 32 || f->Cout % 32 ||
        f->Cin > 256 || f->Ce > 512 || (K0 != 0 && K0 != 3 && K0 != 5) || (K != 0 && K != 3 && K != 5) ||
        (!K0 && !K))
        return 0;
    if (K0 && (f->p0t < 0 || f->p0t >= K0 || f->p0l < 0 || f->p0l >= K0)) return 0;
    if (K) {
        if ((f->s != 1 && f->s != 2) || f->pt < 0 || f->pt >= K || f->pl < 0 || f->pl >= K) return 0;
        // Every output row's window reaches into the map; the map's height
        // and width are those the depthwise's own output follows from.
        if ((f->Ho - 1) * f->s - f->pt > f->H - 1 || (f->Wo - 1) * f->s - f->pl > f->W - 1) return 0;
    } else if (f->Ho != f->H || f->Wo != f->W) {
        return 0;
    }
    if (f->has_add && (f->Ho != f->H || f->Wo != f->W || f->Cin != f->Cout || (K && f->s != 1))) return 0;
    // The most rows per band that fit, with the expand and depthwise records
    // in LDS if they fit too (else read from L2 when a channel tile
    // changes).
    UibArgs t;
    for (int R = f->Ho; R >= 1; R--)
        for (int rec_lds = 1; rec_lds >= 0; rec_lds--) {
            const size_t lds = uib_layout(f, R, rec_lds, &t);
            if (lds) {
                f->R = R;
                f->rec_lds = rec_lds;
                return lds;
            }
        }
    return 0;
}

static uint64_t g_uib_launches;

// Launches of the banded bottleneck kernel since the library was loaded (a
// test hook; not part of the plan ABI).
extern "C" uint64_t uqk_uib_launches(void) { return g_uib_launches; }

template <int K0, int K>
static int uib_launch(const UibArgs &a, dim3 grid, size_t lds)
{
    static int ceiling_set;
    if (!ceiling_set) {
        const hipError_t e =
            hipFuncSetAttribute((const void *)k_uib<K0, K>, hipFuncAttributeMaxDynamicSharedMemorySize, UIB_LDS_MAX);
        if (e != hipSuccess) return uqk_fail(e);
        ceiling_set = 1;
    }
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    hipExtLaunchKernelGGL((k_uib<K0, K>), grid, dim3(64 * IB_WAVES), (uint32_t)lds, st, e0, e1, 0u, a);
    return uqk_fail(hipGetLastError());
}

extern "C" int uqk_uib(const UQKUib *f, const void *x, void *y, uint32_t images)
{
    if (!images) return 0;
    UibArgs a;
    UQKUib g = *f;
    const int R = f->R;
    if (R < 1 || R > f->Ho || !uqk_uib_plan(&g) || R > g.R) return (int)hipErrorInvalidValue;
    const size_t lds = uib_layout(f, R, f->rec_lds, &a);
    if (!lds) return (int)hipErrorInvalidValue;
    a.bands = (f->Ho + R - 1) / R;
    const unsigned long long blocks = (unsigned long long)images * a.bands;
    if (blocks > 0x7fffffffULL || (unsigned long long)f->H * f->W * f->Cin > 0x7fffffffULL)
        return (int)hipErrorInvalidValue;
    a.x = (const int8_t *)x; a.y = (int8_t *)y;
    a.H = f->H; a.W = f->W; a.Ho = f->Ho; a.Wo = f->Wo; a.Cin = f->Cin; a.Ce = f->Ce; a.Cout = f->Cout;
    a.R = R;
    a.k0 = f->k0; a.p0t = f->p0t; a.p0l = f->p0l;
    a.dw0 = (const int *)f->dw0; a.epi0 = (const int4 *)f->epi0; a.lut0 = (const uint8_t *)f->lut0;
    a.m0 = f->m0; a.yz0 = f->yz0; a.lo0 = f->lo0; a.hi0 = f->hi0; a.xz0 = f->xz0;
    a.we = (const int8_t *)f->we; a.epi_e = (const int4 *)f->epi_e; a.lut_e = (const uint8_t *)f->lut_e;
    a.kpe = f->kpe; a.e_mode = f->e_mode; a.e_yz = f->e_yz; a.e_lo = f->e_lo; a.e_hi = f->e_hi;
    a.k = f->k; a.s = f->k ? f->s : 1; a.pt = f->pt; a.pl = f->pl;
    a.dww = (const int *)f->dww; a.epi_d = (const int4 *)f->epi_d; a.lut_d = (const uint8_t *)f->lut_d;
    a.d_mode = f->d_mode; a.d_yz = f->d_yz; a.d_lo = f->d_lo; a.d_hi = f->d_hi; a.d_xz = f->d_xz;
    a.wp = (const int8_t *)f->wp; a.epi_p = (const int4 *)f->epi_p; a.lut_p = (const uint8_t *)f->lut_p;
    a.kpp = f->kpp; a.p_mode = f->p_mode; a.p_yz = f->p_yz; a.p_lo = f->p_lo; a.p_hi = f->p_hi;
    a.has_add = f->has_add; a.add_x_first = f->add_x_first; a.add_tab = (const int *)f->add_tab;
    a.a_m = f->a_m; a.a_s = f->a_s; a.a_yz = f->a_yz; a.a_lo = f->a_lo; a.a_hi = f->a_hi;
    a.a_c1 = a.a_thr = 0;
    a.a_hs = 0;
    if (f->has_add && f->a_s < 0) {
        const int nsh = -f->a_s;
        if (nsh > 31) return (int)hipErrorInvalidValue;
        a.a_c1 = (1LL << 30) + (1LL << (30 + nsh));
        a.a_thr = 1LL << (30 + nsh);
        a.a_hs = nsh - 1;
    }
    a.m_w = udiv_magic((unsigned)f->W); a.m_wo = udiv_magic((unsigned)f->Wo);
    a.m_cq = udiv_magic((unsigned)(f->Cin / 16)); a.m_c0 = udiv_magic((unsigned)a.cols0);
    a.xs = f->Cin + 16; a.x1s = f->Cin + 16; a.ds = f->Ce + 16;
    const dim3 grid((unsigned)blocks);
    int rc;
#define UIB_K(K0)                                                     \
    do {                                                              \
        switch (f->k) {                                               \
        case 0: rc = uib_launch<K0, 0>(a, grid, lds); break;          \
        case 3: rc = uib_launch<K0, 3>(a, grid, lds); break;          \
        default: rc = uib_launch<K0, 5>(a, grid, lds); break;         \
        }                                                             \
    } while (0)
    // Without a start depthwise the block has a depthwise (uqk_uib_plan).
    switch (f->k0) {
    case 0: rc = f->k == 3 ? uib_launch<0, 3>(a, grid, lds) : uib_launch<0, 5>(a, grid, lds); break;
    case 3: UIB_K(3); break;
    default: UIB_K(5); break;
    }
#undef UIB_K
    if (!rc) g_uib_launches++;
    return rc;
}
