// Fused inverted bottleneck for gfx950: 1x1 expand -> stride-1 depthwise ->
// 1x1 project [-> residual add with the block input], one workgroup of 16
// waves per image, every intermediate in LDS (the reference runs the three
// or four ops one after another through HBM: qnn.c:1074-1246 for the 1x1
// convs, qnn.c:807-983 for the depthwise, qnn.c:1248-1290 for the add).
// Each phase is the arithmetic of the separate kernels (same operand bytes,
// the same epilogue records, requantisation and post tables), so the bytes
// are identical; only the HBM round trips of the expanded tensors and three
// of the four launches go.
//
// Phases, separated by barriers:
//   0  the image's input rows, the three layers' records, the add and post
//      tables into LDS; the depthwise window planes filled with its input
//      zero point.
//   1  expand: 32x32 tiles on v_mfma_i32_32x32x32_i8 with the pixels as the
//      MFMA rows (from LDS) and the weights as its columns (16-byte loads
//      from HBM/L2), so that a lane's 16 results share one channel and its
//      requantisation record stays in registers while the wave's tiles share
//      a channel tile. A 4x4 byte transpose across each lane quad turns four
//      pixels of one channel into four channels of one pixel: 4-byte LDS
//      writes into the window plane of the channels' 16-channel group, at
//      the pixel's padded position.
//   2  depthwise on the matrix cores: 3x3 on 32x32 tiles, one
//      v_mfma_i32_32x32x32_i8 per tap (ib_dw3_32); 5x5 as in k_dw_mfma, per
//      16 pixels x 16 channels one v_mfma_i32_16x16x64_i8 per four taps. The
//      A rows are 16-byte reads of the window planes, B is block diagonal (a
//      lane's tap weight at its channel's byte). Output rows of Ce bytes
//      (padded by 16) in LDS.
//   3  project: 16x16 tiles on v_mfma_i32_16x16x64_i8 (finer work items for
//      the small maps) with the depthwise rows as the MFMA rows; the
//      residual add, if fused, per byte from the input rows still in LDS;
//      the output staged in LDS (over the window planes, free by then) and
//      copied out with 16-byte stores.
//
// LDS (bytes): X [P][Cin + 16] | E [Ce / 16][rows_p * cols_p][16] (later the
// output stage [P][Cout]) | D [P][Ce + 16] | records (expand, depthwise,
// project; 32 bytes per channel) | add tables [2][256] int32 | post tables
// [3][256] | padded window position of each pixel [P] int32 | depthwise tap
// words [ks][ks > 4 ? 2 : 1][Ce]. Rows padded by 16 bytes keep 32-row
// fragment reads off a single bank group.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"
#include "ib_phases.h"

constexpr int IB_LDS_MAX = 163840;

struct IbArgs {
    const int8_t *x;
    int8_t *y;
    int P, H, W, Cin, Ce, Cout, pt, pl;
    int rows_p, cols_p;        // depthwise window plane (padded map)
    int xs, ds;                // LDS row strides of X and D
    unsigned m_w;              // udiv_magic(W)
    unsigned m_cq;             // udiv_magic(Cin / 16)
    const int8_t *we;          // expand weights [>= Ce][kpe]
    const int4 *epi_e;
    const uint8_t *lut_e;
    int kpe, e_mode, e_yz, e_lo, e_hi;
    const int *dww;            // depthwise tap words [ky][k][Ce]
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
    int a_hs;                  // its high-word shift, -s - 1
    int ks;                    // depthwise kernel size
    int o_e, o_d, o_re, o_rd, o_rp, o_at, o_lut, o_po, o_tw;   // LDS offsets
};

template <int KS>
__global__ __launch_bounds__(64 * IB_WAVES) void k_ib(IbArgs a)
{
    constexpr int NT = 64 * IB_WAVES;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t *X = smem, *E = smem + a.o_e, *D = smem + a.o_d;
    int8_t *lut_s = smem + a.o_lut;
    const int *at = (const int *)(smem + a.o_at);
    int *padoff = (int *)(smem + a.o_po);
    const int tid = threadIdx.x;
    const long n = blockIdx.x;
    const int plane = a.rows_p * a.cols_p;
    const int *tw = (const int *)(smem + a.o_tw);

    // Phase 0.
    {
        const int8_t *xin = a.x + n * a.P * a.Cin;
        const int cq = a.Cin >> 4, chunks = a.P * cq;
        for (int q = tid; q < chunks; q += NT) {
            const int p = (int)udiv((unsigned)q, (unsigned)cq, a.m_cq), j = q - p * cq;
            *(v4i *)(X + p * a.xs + j * 16) = *(const v4i *)(xin + (long)q * 16);
        }
        const int xzw = (a.d_xz & 0xff) * 0x01010101;
        const v4i xzv = {xzw, xzw, xzw, xzw};
        for (int q = tid; q < (a.Ce >> 4) * plane; q += NT) ((v4i *)E)[q] = xzv;
        for (int i = tid; i < 2 * a.Ce; i += NT) {
            ((int4 *)(smem + a.o_re))[i] = a.epi_e[i];
            ((int4 *)(smem + a.o_rd))[i] = a.epi_d[i];
        }
        for (int i = tid; i < 2 * a.Cout; i += NT) ((int4 *)(smem + a.o_rp))[i] = a.epi_p[i];
        for (int i = tid; i < a.ks * (a.ks > 4 ? 2 : 1) * a.Ce; i += NT) ((int *)(smem + a.o_tw))[i] = a.dww[i];
        if (a.has_add)
            for (int i = tid; i < 512; i += NT) ((int *)(smem + a.o_at))[i] = a.add_tab[i];
        // Padded window position of each pixel.
        for (int p = tid; p < a.P; p += NT) {
            const int y = (int)udiv((unsigned)p, (unsigned)a.W, a.m_w), x = p - y * a.W;
            padoff[p] = (y + a.pt) * a.cols_p + x + a.pl;
        }
        if (tid < 64) {
            if (a.lut_e) ((int *)lut_s)[tid] = ((const int *)a.lut_e)[tid];
            if (a.lut_d) ((int *)(lut_s + 256))[tid] = ((const int *)a.lut_d)[tid];
            if (a.lut_p) ((int *)(lut_s + 512))[tid] = ((const int *)a.lut_p)[tid];
        }
    }
    __syncthreads();

    // Phase 1: expand into the window planes.
    v4i wfe[8];
    int wfe_ct = -1;
    ib_gemm_mode<8>(a.e_mode, wfe, wfe_ct, a.we, a.kpe, a.Cin >> 5, X, a.xs, a.P, a.Ce >> 5,
                    (const int4 *)(smem + a.o_re), a.e_yz, a.e_lo, a.e_hi, a.lut_e ? lut_s : nullptr,
                    [&](int p, int c, int word) {
                        *(int *)(E + (__mul24(c >> 4, plane) + padoff[p]) * 16 + (c & 15)) = word;
                    });
    __syncthreads();

    // Phase 2: depthwise into D.
    {
        const DwPh g = {a.P, a.Ce, a.ds, a.cols_p, a.pt * a.cols_p + a.pl, a.d_yz, a.d_lo, a.d_hi,
                        (const int4 *)(smem + a.o_rd), a.lut_d ? lut_s + 256 : nullptr};
        ib_dw_mode<KS>(a.d_mode, g, E, D, padoff, tw, plane);
    }
    __syncthreads();

    // Phase 3: project (+ residual add) into the output stage over E, then
    // out with 16-byte stores.
    // The add's rescale (qnn.c:61-83: rounding doubling high multiply, then
    // a rounding right shift by n = -s) as one multiply-add: for n >= 1,
    // floor((floor((v*m + 2^30) / 2^31) + 2^(n-1) - [h < 0]) / 2^n) =
    // floor((v*m + 2^30 + 2^(30+n) - [v*m < -2^30] * 2^31) / 2^(31+n)), whose
    // high word shifted by n - 1 is the result (a_c1, a_thr, a_hs from the
    // host); for s >= 0, (((v << s) * m + 2^30) >> 31).
    int8_t *S = E;
    const int *atab = at + (a.add_x_first ? 0 : 256), *btab = at + (a.add_x_first ? 256 : 0);
    auto project_sink = [&](int p, int c, int word) {
        if (a.has_add) {
            const int xr = *(const int *)(X + __mul24(p, a.xs) + c);
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
    // 32x32 tiles when they leave the busiest wave no more results per lane
    // than 16x16 tiles (16 per 32x32 item, 4 per 16x16 item), else 16x16:
    // on 14x14x96 outputs 21 items of 32x32 (two for some waves, 32 results)
    // against 78 of 16x16 (at most five, 20 results).
    const int i32 = (a.Cout >> 5) * ((a.P + 31) >> 5), i16 = (a.Cout >> 4) * ((a.P + 15) >> 4);
    if ((i32 + IB_WAVES - 1) / IB_WAVES * 16 <= (i16 + IB_WAVES - 1) / IB_WAVES * 4) {
        v4i wfp[16];
        int wfp_ct = -1;
        ib_gemm_mode<16>(a.p_mode, wfp, wfp_ct, a.wp, a.kpp, a.Ce >> 5, D, a.ds, a.P, a.Cout >> 5,
                         (const int4 *)(smem + a.o_rp), a.p_yz, a.p_lo, a.p_hi, a.lut_p ? lut_s + 512 : nullptr,
                         project_sink);
    } else {
        ib_gemm16_mode<8>(a.p_mode, a.wp, a.kpp, (a.Ce + 63) >> 6, D, a.ds, a.P, a.Cout >> 4,
                          (const int4 *)(smem + a.o_rp), a.p_yz, a.p_lo, a.p_hi, a.lut_p ? lut_s + 512 : nullptr,
                          project_sink);
    }
    __syncthreads();
    int8_t *yim = a.y + n * a.P * a.Cout;
    for (int q = tid; q < (a.P * a.Cout) >> 4; q += NT) ((v4i *)yim)[q] = ((const v4i *)S)[q];
}

// LDS layout of one workgroup (see the file header); 0 when the block does
// not fit this kernel: 32-multiple channel counts (K steps and tiles of
// 32), Cin <= 256, Ce <= 512, a 3x3 or 5x5 depthwise, the output stage
// within the window planes and the layout within the 160 KiB a workgroup
// can hold.
extern "C" size_t uqk_ib_lds(int P, int H, int W, int Cin, int Ce, int Cout, int ks, size_t *offsets)
{
    if (P < 1 || P != H * W || Cin % 32 || Ce % 32 || Cout % 32 || Cin > 256 || Ce > 512 || (ks != 3 && ks != 5))
        return 0;
    size_t o = 0, off[9];
    o += (size_t)P * (Cin + 16);                                        // X
    off[0] = o; o += (size_t)(Ce / 16) * (H + ks - 1) * (W + ks - 1) * 16; // E planes
    off[1] = o; o += (size_t)P * (Ce + 16);                             // D
    off[2] = o; o += (size_t)Ce * 32;                                   // expand records
    off[3] = o; o += (size_t)Ce * 32;                                   // depthwise records
    off[4] = o; o += (size_t)Cout * 32;                                 // project records
    off[5] = o; o += 512 * 4;                                           // add tables
    off[6] = o; o += 3 * 256;                                           // post tables
    off[7] = o; o += (size_t)P * 4;                                     // padded positions
    off[8] = o; o += (size_t)ks * (ks > 4 ? 2 : 1) * Ce * 4;            // depthwise tap words
    if (offsets) for (int i = 0; i < 9; i++) offsets[i] = off[i];
    // The output stage [P][Cout] lies over the window planes.
    if ((size_t)P * Cout > off[1] - off[0]) return 0;
    return o <= (size_t)IB_LDS_MAX ? o : 0;
}

static uint64_t g_ib_launches;   // successful launches, for tests that must know the fused kernel ran

// Launches of the fused bottleneck kernel since the library was loaded (a
// test hook; not part of the plan ABI).
extern "C" uint64_t uqk_ib_launches(void) { return g_ib_launches; }

extern "C" int uqk_ib(const UQKIb *f, const void *x, void *y, uint32_t images)
{
    if (!images) return 0;
    size_t off[9];
    const size_t lds = uqk_ib_lds(f->P, f->H, f->W, f->Cin, f->Ce, f->Cout, f->ks, off);
    if (!lds || images > 0x7fffffffu) return (int)hipErrorInvalidValue;
    IbArgs a;
    a.x = (const int8_t *)x; a.y = (int8_t *)y;
    a.P = f->P; a.H = f->H; a.W = f->W; a.Cin = f->Cin; a.Ce = f->Ce; a.Cout = f->Cout; a.pt = f->pt; a.pl = f->pl;
    a.rows_p = f->H + f->ks - 1; a.cols_p = f->W + f->ks - 1;
    a.xs = f->Cin + 16; a.ds = f->Ce + 16;
    a.m_w = udiv_magic((unsigned)f->W); a.m_cq = udiv_magic((unsigned)(f->Cin / 16));
    a.we = (const int8_t *)f->we; a.epi_e = (const int4 *)f->epi_e; a.lut_e = (const uint8_t *)f->lut_e;
    a.kpe = f->kpe; a.e_mode = f->e_mode; a.e_yz = f->e_yz; a.e_lo = f->e_lo; a.e_hi = f->e_hi;
    a.dww = (const int *)f->dww; a.epi_d = (const int4 *)f->epi_d; a.lut_d = (const uint8_t *)f->lut_d;
    a.d_mode = f->d_mode; a.d_yz = f->d_yz; a.d_lo = f->d_lo; a.d_hi = f->d_hi; a.d_xz = f->d_xz;
    a.wp = (const int8_t *)f->wp; a.epi_p = (const int4 *)f->epi_p; a.lut_p = (const uint8_t *)f->lut_p;
    a.kpp = f->kpp; a.p_mode = f->p_mode; a.p_yz = f->p_yz; a.p_lo = f->p_lo; a.p_hi = f->p_hi;
    a.has_add = f->has_add; a.add_x_first = f->add_x_first; a.add_tab = (const int *)f->add_tab;
    a.a_m = f->a_m; a.a_s = f->a_s; a.a_yz = f->a_yz; a.a_lo = f->a_lo; a.a_hi = f->a_hi;
    a.a_c1 = a.a_thr = 0;
    a.a_hs = 0;
    if (f->a_s < 0) {
        const int nsh = -f->a_s;
        if (nsh > 31) return (int)hipErrorInvalidValue;
        a.a_c1 = (1LL << 30) + (1LL << (30 + nsh));
        a.a_thr = 1LL << (30 + nsh);
        a.a_hs = nsh - 1;
    }
    a.o_e = (int)off[0]; a.o_d = (int)off[1]; a.o_re = (int)off[2]; a.o_rd = (int)off[3]; a.o_rp = (int)off[4];
    a.o_at = (int)off[5]; a.o_lut = (int)off[6]; a.o_po = (int)off[7]; a.o_tw = (int)off[8]; a.ks = f->ks;
    // The dynamic-LDS ceiling is raised once per kernel (a host call that
    // must not sit on every launch).
    static int ceiling_set[2];
    const int which = f->ks == 3 ? 0 : 1;
    if (!ceiling_set[which]) {
        const hipError_t e = which == 0 ? hipFuncSetAttribute((const void *)k_ib<3>,
                                                              hipFuncAttributeMaxDynamicSharedMemorySize, IB_LDS_MAX)
                                        : hipFuncSetAttribute((const void *)k_ib<5>,
                                                              hipFuncAttributeMaxDynamicSharedMemorySize, IB_LDS_MAX);
        if (e != hipSuccess) return uqk_fail(e);
        ceiling_set[which] = 1;
    }
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    const dim3 grid(images), block(64 * IB_WAVES);
    if (which == 0) hipExtLaunchKernelGGL(k_ib<3>, grid, block, (uint32_t)lds, st, e0, e1, 0u, a);
    else hipExtLaunchKernelGGL(k_ib<5>, grid, block, (uint32_t)lds, st, e0, e1, 0u, a);
    const int rc = uqk_fail(hipGetLastError());
    if (!rc) g_ib_launches++;
    return rc;
}
