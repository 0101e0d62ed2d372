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
#include <hip/hip_ext.h>
#include <type_traits>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"

static hipStream_t g_stream;      // stream of the next launch: g_main, or a side stream of a split batch
static hipStream_t g_main;        // compute (and the single-stream entry points)
static hipStream_t g_copy[2];     // host transfers of the pipelined batch: in, out
static hipEvent_t g_pipe_ev[8];   // pipeline hand-offs between the three streams
static hipStream_t g_side[UQK_MAX_SLICES - 1];   // compute streams of the other image slices
static hipEvent_t g_fork, g_join[UQK_MAX_SLICES - 1];
static int g_live_slices = 1;     // launches in flight side by side (image slices of one batch)
static int g_ready;
static int g_err;
static hipEvent_t *g_ev_start, *g_ev_stop;   // per-op timing events (profiling)
static uint32_t g_nevents;
static int g_timing;              // an op is being timed: its launches stamp its events
static uint32_t g_timed_op, g_timed_launches;

#define UQK_TRY(expr)                                  \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) {                        \
            g_err = (int)e_;                           \
            return (int)e_;                            \
        }                                              \
    } while (0)
#define UQK_LAUNCHED() UQK_TRY(hipGetLastError())

// Every kernel launch goes to g_stream. While an op is timed (uqk_time_begin
// .. uqk_time_end), its first launch stamps the op's start event and every
// launch its stop event with the dispatch's own start and end timestamps (the
// interval a kernel trace reports, without the gap an event record between
// kernels adds). The stream argument of the call sites is g_stream.
void uqk_next_launch(hipStream_t *stream, hipEvent_t *start, hipEvent_t *stop)
{
    *start = *stop = nullptr;
    if (g_timing) {
        *start = g_timed_launches ? nullptr : g_ev_start[g_timed_op];
        *stop = g_ev_stop[g_timed_op];
        g_timed_launches++;
    }
    *stream = g_stream;
}

int uqk_fail(hipError_t e)
{
    if (e != hipSuccess) g_err = (int)e;
    return (int)e;
}

int uqk_slices_live(void) { return g_live_slices; }

template <typename F, typename... Args>
static inline void uqk_launch(F kernel, dim3 grid, dim3 block, size_t lds, Args... args)
{
    hipStream_t stream;
    hipEvent_t start, stop;
    uqk_next_launch(&stream, &start, &stop);
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)lds, stream, start, stop, 0u, args...);
}
#define UQK_LAUNCH(kernel, grid, block, lds, stream, ...) uqk_launch(kernel, grid, block, lds, __VA_ARGS__)

// ---------------------------------------------------------------------------
// Implicit-GEMM convolution on v_mfma_i32_16x16x64_i8.
//
// A block is 4 waves; each wave owns RB x 16 output rows (pixels) and all
// NT x 16 output channels of the block's channel slice. Each lane supplies one
// 16-byte K slice of one row as the MFMA A operand (lane & 15 is the row,
// lane >> 4 the K slice); the B operand is the matching 16-byte K slice of the
// [oc_pad][kpad] weight matrix. A and B use the same lane -> K assignment, so
// the sum is independent of the hardware's K order inside an operand. The
// next K step's operands are loaded before the current step's MFMAs issue.
// The requantised bytes are staged in LDS and written as coalesced 16-byte
// row segments.
//
// Two A sources:
//   k_conv       pointwise rows read straight from HBM (MODE PW), or a
//                per-lane gather through a k -> (dy, dx, c) table (G16/G4/G1)
//   k_conv_rows  spatial convs: the block's input rows (with padding
//                materialised as xz) are staged once in LDS, and every lane
//                reads its K slices from there through a k -> LDS-offset table
// ---------------------------------------------------------------------------
struct ConvArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;
    const int4 *epi;
    const int4 *kmap;
    const int *delta;
    const uint8_t *lut;
    long M;
    int ih, iw, ic, icp, oh, ow, oc, kh, sh, sw, dh, pt, pl, xz, yz, lo, hi, K, kpad, ohw, corr, emode;
    int kw, dw, taps;
    int images, segs, row_groups, seg_rb, stem_rows;     // stem grid: segments, row blocks each, staged rows
    int stem_cpr;                                        // stem: 16-byte LDS chunks per staged row
    unsigned stem_cpr_magic;
    int tiles, cols, rows_max, tile_px;
    unsigned m_row, m_px;      // k_conv_rows staging: udiv_magic of items per staged row, per pixel
    // Fused residual add (k_conv only; res == nullptr when there is none).
    const int8_t *res;
    const int *add_tab;
    int add_m, add_s, add_yz, add_lo, add_hi, add_conv_a;
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


// Stage the block's per-channel records (columns n0 .. n0 + NT*16 - 1; the
// channels past OC reuse record 0) and the layer's 256-byte post table in
// LDS, so that the epilogue has no dependent global load. The caller's next
// barrier publishes them.
template <int NT>
__device__ __forceinline__ void stage_consts(const ConvArgs &a, int n0, int4 *epi_s, int8_t *lut_s)
{
    for (int t = threadIdx.x; t < 2 * NT * 16; t += 256) {
        const int col = n0 + (t >> 1);
        epi_s[t] = a.epi[2 * (col < a.oc ? col : 0) + (t & 1)];
    }
    if (a.lut && threadIdx.x < 64) ((int *)lut_s)[threadIdx.x] = ((const int *)a.lut)[threadIdx.x];
}

// The same constants in two halves for kernels whose operand loads are in
// flight at that point: consts_load issues the loads into registers (one
// record half and one table word per thread at most), consts_store
// writes them to LDS later, so no wait for them stalls the operand prefetch.
struct ConstRegs {
    int4 e;
    int l;
};

template <int NT>
__device__ __forceinline__ ConstRegs consts_load(const ConvArgs &a, int n0)
{
    static_assert(2 * NT * 16 <= 256, "one record half per thread");
    ConstRegs r = {{0, 0, 0, 0}, 0};
    const int t = threadIdx.x;
    if (t < 2 * NT * 16) {
        const int col = n0 + (t >> 1);
        r.e = a.epi[2 * (col < a.oc ? col : 0) + (t & 1)];
    }
    if (a.lut && t < 64) r.l = ((const int *)a.lut)[t];
    return r;
}

template <int NT>
__device__ __forceinline__ void consts_store(const ConvArgs &a, const ConstRegs &r, int4 *epi_s, int8_t *lut_s)
{
    const int t = threadIdx.x;
    if (t < 2 * NT * 16) epi_s[t] = r.e;
    if (a.lut && t < 64) ((int *)lut_s)[t] = r.l;
}

// Requantise a wave's RB*16 x NT*16 tile and store the valid rows
// [row_base, row_limit). The MFMA result gives a lane one channel (lane & 15)
// of four consecutive rows; the four bytes are packed into a word, and a 4x4
// byte transpose across each quad of lanes (two DPP quad permutes, two
// v_perm) turns that into one row x four channels per lane, stored as one
// dword. Needs OC % 4 == 0 (so a quad's channels are all valid or all not);
// other widths take byte stores.
// The residual add of op 18 on one word of four output bytes y and four
// residual bytes r: s = ta[first + 128] + tb[second + 128], then
// clamp(uq_scale(s, m, shift) + yz, lo, hi), first being the conv byte when
// the conv output is the add's operand a.
__device__ __forceinline__ int add_word(const ConvArgs &a, const int *tab, int y, int r)
{
    const int wa = a.add_conv_a ? y : r, wb = a.add_conv_a ? r : y;
    int z[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int s1 = tab[sbyte(wa, j) + 128] + tab[256 + sbyte(wb, j) + 128];
        z[j] = min(max(uq_scale(s1, a.add_m, a.add_s) + a.add_yz, a.add_lo), a.add_hi);
    }
    return pack4(z[0], z[1], z[2], z[3]);
}

// Residual words for a fused add, read before the K loop so that their
// latency hides behind it: the word of lane's transposed output position,
// row (rb*16 + 4*(lane >> 4) + (lane & 3)), channels n0 + nt*16 +
// (lane & 12) .. + 3. Used when OC % 4 == 0 (otherwise the epilogue's byte
// path reads the residual itself).
template <int RB, int NT>
__device__ __forceinline__ void load_residual(const ConvArgs &a, int (&rw)[RB][NT], long row_base, long row_limit,
                                              int n0, int lane)
{
    const bool words = a.res && (a.oc & 3) == 0;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const long row = row_base + rb * 16 + (lane >> 4) * 4 + (lane & 3);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int c = n0 + nt * 16 + (lane & 12);
            rw[rb][nt] = words && row < row_limit && c < a.oc ? *(const int *)(a.res + row * a.oc + c) : 0;
        }
    }
}

template <int RB, int NT, bool HI, bool CORR>
__device__ __forceinline__ void conv_store(const ConvArgs &a, const v4i (&acc)[RB][NT], int8_t *stage, int n0, int lane,
                                           long row_base, long row_limit, const int4 *epi_s, const int8_t *lut_s,
                                           const int *add_s, const int (&rw)[RB][NT])
{
    constexpr int R = RB * 16;
    constexpr int BN = NT * 16;
    constexpr int STRIDE = BN + 16;
    const int lr = lane & 15, lg = lane >> 4;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    const bool words = (a.oc & 3) == 0;
    const bool lut = a.lut != nullptr;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const Epi e = load_epi(epi_s, nt * 16 + lr);
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            int v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[rb][nt][i], e, a.yz, vlo, vhi);
            if (lut) {
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
            }
            if (words) {
                int t = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
                if (add_s) t = add_word(a, add_s, t, rw[rb][nt]);
                *(int *)(stage + (rb * 16 + lg * 4 + (lane & 3)) * STRIDE + nt * 16 + (lr & ~3)) = t;
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) stage[(rb * 16 + lg * 4 + i) * STRIDE + nt * 16 + lr] = (int8_t)v[i];
            }
        }
    }
    __syncthreads();
    const int ncols = min(BN, a.oc - n0);
    if ((a.oc & 15) == 0 && ncols == BN) {
        // The whole slice: NT 16-byte chunks per row, a compile-time split.
#pragma unroll
        for (int c = lane; c < R * NT; c += 64) {
            const int r = c / NT, cc = c - r * NT;
            const long row = row_base + r;
            if (row < row_limit)
                *(v4i *)(a.y + row * a.oc + n0 + cc * 16) = *(const v4i *)(&stage[r * STRIDE + cc * 16]);
        }
    } else if ((a.oc & 15) == 0) {
        const int cpr = ncols >> 4;
        for (int c = lane; c < R * cpr; c += 64) {
            const int r = c / cpr, cc = c - r * cpr;
            const long row = row_base + r;
            if (row < row_limit)
                *(v4i *)(a.y + row * a.oc + n0 + cc * 16) = *(const v4i *)(&stage[r * STRIDE + cc * 16]);
        }
    } else {
        for (int c = lane; c < R * ncols; c += 64) {
            const int r = c / ncols, cc = c - r * ncols;
            const long row = row_base + r;
            if (row < row_limit) {
                const long at = row * a.oc + n0 + cc;
                int v = stage[r * STRIDE + cc];
                if (add_s && !words) v = add_word(a, add_s, v, a.res[at]);
                a.y[at] = (int8_t)v;
            }
        }
    }
}


// Requantise and store a wave's tile computed with the channels as the MFMA
// rows (weights in the A operand, pixels in B): a lane holds channels
// nt*16 + 4*(lane >> 4) + i (i = 0..3) of pixel rb*16 + (lane & 15), packed
// into one word per (rb, nt). Per channel tile, the words of four row blocks
// go through rows_transpose4, after which row j of the wave holds all 16
// channels of one pixel of row block rb0 + j: one 16-byte store per lane, no
// LDS round trip. Only one tile's four channel records and four words are
// live at a time. Only the first NRB row blocks (at most RB) are
// requantised and stored. row_base is wave-uniform and rows are at most
// 2^24 apart within a wave, so the per-lane part of the address is a 24-bit
// multiply. Needs OC % 16 == 0.
template <int RB, int NT, bool HI, bool CORR, int NRB = RB>
__device__ __forceinline__ void conv_store_direct(const ConvArgs &a, const v4i (&acc)[RB][NT], int n0, int lane,
                                                  long row_base, long row_limit, const int4 *epi_s,
                                                  const int8_t *lut_s)
{
    static_assert(RB % 4 == 0 && NRB <= RB, "row blocks go through the transpose in fours");
    const int lr = lane & 15, lg = lane >> 4;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    const bool lut = a.lut != nullptr;
    int8_t *ybase = a.y + row_base * a.oc;
    const int rows_left = row_limit - row_base < (long)(NRB * 16) ? (int)(row_limit - row_base) : NRB * 16;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int cb = n0 + nt * 16;
        Epi e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) e[i] = load_epi(epi_s, nt * 16 + 4 * lg + i);
#pragma unroll
        for (int rb0 = 0; rb0 < NRB; rb0 += 4) {
            int r[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (rb0 + q >= NRB) {
                    r[q] = 0;
                    continue;
                }
                int v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[rb0 + q][nt][i], e[i], a.yz, vlo, vhi);
                if (lut) {
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
                }
                r[q] = pack4(v[0], v[1], v[2], v[3]);
            }
            rows_transpose4(r);
            const int prow = (rb0 + lg) * 16 + lr;
            if (prow < rows_left && cb < a.oc)
                *(v4i *)(ybase + __mul24(prow, a.oc) + cb) = (v4i){r[0], r[1], r[2], r[3]};
        }
    }
}

// One copy of the store per requantisation variant (emode = HI | CORR << 1).
template <int RB, int NT>
__device__ __forceinline__ void conv_epilogue(const ConvArgs &a, const v4i (&acc)[RB][NT], int8_t *stage, int n0,
                                              int lane, long row_base, long row_limit, const int4 *epi_s,
                                              const int8_t *lut_s, const int *add_s, const int (&rw)[RB][NT])
{
    switch (a.emode) {
    case 0: conv_store<RB, NT, false, false>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, add_s, rw); break;
    case 1: conv_store<RB, NT, true, false>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, add_s, rw); break;
    case 2: conv_store<RB, NT, false, true>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, add_s, rw); break;
    default: conv_store<RB, NT, true, true>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, add_s, rw); break;
    }
}

// The same with the requantisation variant fixed at compile time (EMODE =
// HI | CORR << 1), or chosen at run time when EMODE < 0. One variant per
// kernel keeps its register allocation to what that variant needs.
template <int RB, int NT, int EMODE>
__device__ __forceinline__ void conv_epilogue_em(const ConvArgs &a, const v4i (&acc)[RB][NT], int8_t *stage, int n0,
                                                 int lane, long row_base, long row_limit, const int4 *epi_s,
                                                 const int8_t *lut_s, const int *add_s, const int (&rw)[RB][NT])
{
    if constexpr (EMODE < 0)
        conv_epilogue<RB, NT>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, add_s, rw);
    else
        conv_store<RB, NT, (EMODE & 1) != 0, (EMODE & 2) != 0>(a, acc, stage, n0, lane, row_base, row_limit, epi_s,
                                                               lut_s, add_s, rw);
}

// Without a fused add.
template <int RB, int NT>
__device__ __forceinline__ void conv_epilogue(const ConvArgs &a, const v4i (&acc)[RB][NT], int8_t *stage, int n0,
                                              int lane, long row_base, long row_limit, const int4 *epi_s,
                                              const int8_t *lut_s)
{
    const int rw[RB][NT] = {};
    conv_epilogue<RB, NT>(a, acc, stage, n0, lane, row_base, row_limit, epi_s, lut_s, nullptr, rw);
}

// Copy K bytes [kc0, kc0 + kn) of a block's NT*16 weight rows (row stride
// kpad in the [oc_pad][kpad] matrix) to LDS with row stride wstride: 16-byte
// loads in K order (whole lines when kn == kpad, the slice then being one
// contiguous range), four per thread issued before the first LDS write.
template <int NT>
__device__ __forceinline__ void stage_weights(const int8_t *wslice, int kpad, int kc0, int kn, int wstride, int8_t *dst)
{
    const int cpr = kn >> 4, total = NT * 16 * cpr;
    for (int c0 = threadIdx.x; c0 < total; c0 += 4 * 256) {
        v4i v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = c0 + j * 256;
            if (c < total) {
                const int r = c / cpr, q = c - r * cpr;
                v[j] = *(const v4i *)(wslice + (long)r * kpad + kc0 + q * 16);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = c0 + j * 256;
            if (c < total) {
                const int r = c / cpr, q = c - r * cpr;
                *(v4i *)(dst + r * wstride + q * 16) = v[j];
            }
        }
    }
}

// Register-direct store of a k_conv tile computed with the channels as the
// MFMA rows: a lane holds channels nt*16 + 4*(lane >> 4) + i of pixel
// rb*16 + (lane & 15). Each (rb, nt) tile is requantised into one packed word
// per lane, one channel tile's records at a time; then the words of four
// tiles at a time go through rows_transpose4, after which lane (r, j) holds
// the 16 channels of pixel r of the group's tile j: one 16-byte store per
// lane. Needs OC % 16 == 0 and RB * NT a multiple of four.
template <int RB, int NT, bool HI, bool CORR>
__device__ __forceinline__ void conv_store_pairs(const ConvArgs &a, const v4i (&acc)[RB][NT], int n0, int lane,
                                                 long row_base, long row_limit, const int4 *epi_s,
                                                 const int8_t *lut_s)
{
    static_assert((RB * NT) % 4 == 0, "tiles go through the transpose in fours");
    const int lr = lane & 15, lg = lane >> 4;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    const bool lut = a.lut != nullptr;
    int words[RB][NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        Epi e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) e[i] = load_epi(epi_s, nt * 16 + 4 * lg + i);
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            int v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[rb][nt][i], e[i], a.yz, vlo, vhi);
            if (lut) {
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
            }
            words[rb][nt] = pack4(v[0], v[1], v[2], v[3]);
        }
    }
#pragma unroll
    for (int g = 0; g < RB * NT / 4; g++) {
        int r[4];
#pragma unroll
        for (int q = 0; q < 4; q++) r[q] = words[(g * 4 + q) / NT][(g * 4 + q) % NT];
        rows_transpose4(r);
        const int p = g * 4 + lg, rb = p / NT, nt = p - rb * NT;
        const long row = row_base + rb * 16 + lr;
        const int cb = n0 + nt * 16;
        if (row < row_limit && cb < a.oc) *(v4i *)(a.y + row * a.oc + cb) = (v4i){r[0], r[1], r[2], r[3]};
    }
}

// Operand ring depth of k_conv: as many K steps in flight as fit about 96
// registers, a power of two in [2, 8].
__host__ __device__ constexpr int conv_ring(int rb, int nt)
{
    return 96 / ((rb + nt) * 4) >= 8 ? 8 : 96 / ((rb + nt) * 4) >= 4 ? 4 : 2;
}

// K bytes of the block's weight slice staged in LDS at a time: all of kpad
// when NT*16 rows of kpad + 16 bytes fit 48 KiB, else the largest multiple
// of 64 * ring depth that fits (so every chunk starts on ring slot 0).
__host__ __device__ inline int conv_wchunk(int kpad, int rb, int nt)
{
    const int rows = nt * 16, budget = 49152;
    if (rows * (kpad + 16) <= budget) return kpad;
    const int unit = 64 * conv_ring(rb, nt);
    const int kc = (budget / rows - 16) / unit * unit;
    return kc < unit ? unit : kc;
}

// Dynamic LDS of k_conv: the staged weight chunk, or the output stage that
// reuses it after the K loop when that is larger.
__host__ __device__ inline size_t conv_lds(int kpad, int rb, int nt)
{
    const size_t w = (size_t)nt * 16 * (conv_wchunk(kpad, rb, nt) + 16);
    const size_t st = (size_t)4 * rb * 16 * (nt * 16 + 16);
    return w > st ? w : st;
}

// DIRECT: channels as the MFMA rows and the register-direct store
// (conv_store_pairs); instantiated without a fused add.
template <int RB, int NT, int MODE, int EMODE, bool ADD, bool DIRECT>
__global__ __launch_bounds__(256) void k_conv(ConvArgs a)
{
    static_assert(!(ADD && DIRECT), "the fused add goes through the LDS stage");
    constexpr int R = RB * 16;
    constexpr int STRIDE = NT * 16 + 16;
    constexpr int P = conv_ring(RB, NT);
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ __attribute__((aligned(4))) int8_t lut_s[256];
    __shared__ int4 epi_s[2 * NT * 16];
    __shared__ int add_s[ADD ? 512 : 1];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const long row0 = ((long)blockIdx.x * 4 + wave) * R;
    const int n0 = blockIdx.y * NT * 16;
    const int xzw = (a.xz & 0xff) * 0x01010101;

    const int8_t *base[RB];
    int iy0[RB], ix0[RB];
    bool valid[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const long row = row0 + rb * 16 + lr;
        valid[rb] = row < a.M;
        const long r = valid[rb] ? row : 0;
        if (MODE == UQK_PW) {
            base[rb] = a.x + r * a.ic;
            iy0[rb] = ix0[rb] = 0;
        } else {
            const long n = r / a.ohw;
            const int rem = (int)(r - n * a.ohw);
            const int oy = rem / a.ow, ox = rem - oy * a.ow;
            iy0[rb] = oy * a.sh - a.pt;
            ix0[rb] = ox * a.sw - a.pl;
            base[rb] = a.x + n * a.ih * a.iw * a.ic;
        }
    }

    // Pixel operand on a ring of P register slots: the loads of steps
    // s + 1 .. s + P - 1 are in flight while step s multiplies. The block's
    // weight slice (NT*16 rows, contiguous in the [oc_pad][kpad] matrix) is
    // staged in LDS once per K chunk with full-line loads and read from there
    // by all four waves; rows are padded by 16 bytes, so the 16 rows of a
    // 16-byte fragment read fall in distinct banks.
    const int steps = a.kpad >> 6;
    const int kc = conv_wchunk(a.kpad, RB, NT), wstride = kc + 16;
    v4i A[P][RB];
#pragma unroll
    for (int p = 0; p < P; p++) {
        if (p < steps) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                A[p][rb] = gather16<MODE>(a, base[rb], iy0[rb], ix0[rb], valid[rb], p * 64 + lg * 16, xzw);
        }
    }
    const ConstRegs consts = consts_load<NT>(a, n0);
    int rw[RB][NT] = {};
    if (ADD) load_residual<RB, NT>(a, rw, row0, a.M, n0, lane);
    v4i acc[RB][NT];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rb][nt] = (v4i){0, 0, 0, 0};
    const int8_t *wslice = a.w + (long)n0 * a.kpad;
    if (steps == 1) {
        // One K step: the weight fragments straight from global memory (a
        // staging round trip would only add a barrier).
        const int8_t *wrow = wslice + (long)lr * a.kpad + lg * 16;
        v4i B[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) B[nt] = *(const v4i *)(wrow + (long)nt * 16 * a.kpad);
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                acc[rb][nt] = DIRECT ? __builtin_amdgcn_mfma_i32_16x16x64_i8(B[nt], A[0][rb], acc[rb][nt], 0, 0, 0)
                                     : __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0][rb], B[nt], acc[rb][nt], 0, 0, 0);
    }
    for (int kc0 = 0; steps > 1 && kc0 < a.kpad; kc0 += kc) {
        const int kn = min(kc, a.kpad - kc0);
        if (kc0) __syncthreads();
        stage_weights<NT>(wslice, a.kpad, kc0, kn, wstride, smem);
        __syncthreads();
        const int s_begin = kc0 >> 6, s_end = (kc0 + kn) >> 6;
        const int8_t *wl = smem + lr * wstride + lg * 16;
        for (int s0 = s_begin; s0 < s_end; s0 += P) {
#pragma unroll
            for (int p = 0; p < P; p++) {
                const int s = s0 + p;
                if (s < s_end) {
                    v4i B[NT];
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) B[nt] = *(const v4i *)(wl + nt * 16 * wstride + (s - s_begin) * 64);
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
#pragma unroll
                        for (int rb = 0; rb < RB; rb++)
                            acc[rb][nt] = DIRECT
                                              ? __builtin_amdgcn_mfma_i32_16x16x64_i8(B[nt], A[p][rb], acc[rb][nt], 0, 0, 0)
                                              : __builtin_amdgcn_mfma_i32_16x16x64_i8(A[p][rb], B[nt], acc[rb][nt], 0, 0, 0);
                    if (s + P < steps) {
                        const int k1 = (s + P) * 64;
#pragma unroll
                        for (int rb = 0; rb < RB; rb++)
                            A[p][rb] = gather16<MODE>(a, base[rb], iy0[rb], ix0[rb], valid[rb], k1 + lg * 16, xzw);
                    }
                }
            }
        }
    }
    // ADD instances may also run layers without a fused add (the gather
    // modes have no ADD = false instance): the table and residual exist only
    // when a.res is set.
    const bool fused = ADD && a.res != nullptr;
    consts_store<NT>(a, consts, epi_s, lut_s);
    if (fused) {
        add_s[threadIdx.x] = a.add_tab[threadIdx.x];
        add_s[256 + threadIdx.x] = a.add_tab[256 + threadIdx.x];
    }
    __syncthreads();
    if constexpr (DIRECT) {
        conv_store_pairs<RB, NT, (EMODE & 1) != 0, (EMODE & 2) != 0>(a, acc, n0, lane, row0, a.M, epi_s, lut_s);
    } else {
        conv_epilogue_em<RB, NT, EMODE>(a, acc, smem + wave * R * STRIDE, n0, lane, row0, a.M, epi_s, lut_s,
                                        fused ? add_s : nullptr, rw);
    }
}

// Spatial conv with the block's input rows staged in LDS. A block covers up
// to 4*RB*16 consecutive output pixels of one image (a.tile_px: whole output
// rows where they fill the block well; tiles never straddle images); the
// staged region is the rows those pixels touch, full width, with
// out-of-image positions written as xz so the K loop has no bounds checks.
// WORDS: IC % 16 != 0. Each staged pixel holds icp = IC rounded up to four
// bytes (the extra channels are zero, and so are their weights), K counts
// icp-wide taps, and an A slice is four aligned 4-byte LDS reads.
template <int RB, int NT, bool WORDS, int EMODE, bool DIRECT>
__global__ __launch_bounds__(256) void k_conv_rows(ConvArgs a)
{
    constexpr int R = RB * 16;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ __attribute__((aligned(4))) int8_t lut_s[256];
    __shared__ int4 epi_s[2 * NT * 16];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int tile = blockIdx.x % a.tiles;
    const long n = blockIdx.x / a.tiles;
    const int n0 = blockIdx.y * NT * 16;
    const int p0 = tile * a.tile_px, pend = min(p0 + a.tile_px, a.ohw);   // tile_px <= BM
    const int oy_a = p0 / a.ow, oy_b = (pend - 1) / a.ow;
    const int rows = (oy_b - oy_a) * a.sh + (a.kh - 1) * a.dh + 1;
    const int rowbytes = a.cols * a.icp;
    const int tile_bytes = (a.rows_max * rowbytes + 15) & ~15;
    const int ndelta = WORDS ? a.K >> 2 : a.K >> 4;
    int8_t *xt = smem;
    int *dl = (int *)(smem + tile_bytes);
    constexpr int STRIDE = NT * 16 + 16;
    int8_t *stage = smem + tile_bytes + ((ndelta * 4 + 15) & ~15) + wave * R * STRIDE;

    const int iy_lo = oy_a * a.sh - a.pt;
    const int8_t *xim = a.x + n * a.ih * a.iw * a.ic;
    // Staging: each thread issues STAGE_U loads before its first LDS write,
    // so a block waits for about one HBM latency, not one per staged row.
    constexpr int STAGE_U = 4;
    // Staged item q -> (row, 16-byte piece) by multiply-high (q and the row
    // width are below 2^16). A piece never straddles pixels (IC % 16 == 0),
    // so its input byte is linear in the piece: b16 * 16 - pl * IC of the
    // input row, inside the image when that is in [0, IW * IC).
    if (!WORDS) {
        const int xzw = (a.xz & 0xff) * 0x01010101;
        const int cpr = rowbytes >> 4, total = rows * cpr;
        const int in_row = a.iw * a.ic, lead = a.pl * a.ic;
        const int8_t *xrow = xim + (long)iy_lo * in_row;
        for (int q0 = threadIdx.x; q0 < total; q0 += STAGE_U * 256) {
            v4i v[STAGE_U];
#pragma unroll
            for (int j = 0; j < STAGE_U; j++) {
                const int q = q0 + j * 256;
                const int r = (int)udiv((unsigned)q, (unsigned)cpr, a.m_row);
                const int off = ((q - __mul24(r, cpr)) << 4) - lead;
                const bool in = q < total && (unsigned)(iy_lo + r) < (unsigned)a.ih && (unsigned)off < (unsigned)in_row;
                v[j] = (v4i){xzw, xzw, xzw, xzw};
                if (in) v[j] = *(const v4i *)(xrow + __mul24(r, in_row) + off);
            }
#pragma unroll
            for (int j = 0; j < STAGE_U; j++)
                if (q0 + j * 256 < total) *(v4i *)(xt + (q0 + j * 256) * 16) = v[j];
        }
    } else {
        // One LDS word per item (a pixel's channels widened to icp bytes,
        // bytes past IC zero, padding positions the zero point).
        const int wpp = a.icp >> 2, wpr = a.cols * wpp, xzb = a.xz & 0xff, total = rows * wpr;
        for (int q0 = threadIdx.x; q0 < total; q0 += STAGE_U * 256) {
            int w[STAGE_U];
#pragma unroll
            for (int j = 0; j < STAGE_U; j++) {
                const int q = q0 + j * 256;
                const int r = (int)udiv((unsigned)q, (unsigned)wpr, a.m_row), wi = q - r * wpr;
                const int col = (int)udiv((unsigned)wi, (unsigned)wpp, a.m_px), cw = wi - col * wpp;
                const int iy = iy_lo + r, ix = col - a.pl;
                const bool in = q < total && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
                const int8_t *src = xim + (in ? ((long)iy * a.iw + ix) * a.ic : 0) + cw * 4;
                int word = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int b = cw * 4 + k < a.ic ? (in ? (int)(uint8_t)src[k] : xzb) : 0;
                    word |= b << (8 * k);
                }
                w[j] = word;
            }
#pragma unroll
            for (int j = 0; j < STAGE_U; j++)
                if (q0 + j * 256 < total) ((int *)xt)[q0 + j * 256] = w[j];
        }
    }
    for (int i = threadIdx.x; i < ndelta; i += 256) dl[i] = a.delta[i];
    stage_consts<NT>(a, n0, epi_s, lut_s);
    __syncthreads();

    int lbase[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int p = p0 + wave * R + rb * 16 + lr;
        const int pp = p < pend ? p : p0;
        const int oy = pp / a.ow, ox = pp - oy * a.ow;
        lbase[rb] = ((oy - oy_a) * a.sh * a.cols + ox * a.sw) * a.icp;
    }

    // Weights on a ring of P register slots (the pixel operand comes from
    // LDS): steps s + 1 .. s + P - 1 are in flight while step s multiplies.
    // (Staging them in LDS as k_conv does costs these blocks occupancy: the
    // pixel tile already holds most of the block's LDS.)
    constexpr int P = 48 / (NT * 4) >= 8 ? 8 : 48 / (NT * 4) >= 4 ? 4 : 2;
    const int8_t *wrow = a.w + (long)(n0 + lr) * a.kpad + lg * 16;
    const int steps = a.kpad >> 6;
    v4i B[P][NT];
#pragma unroll
    for (int p = 0; p < P; p++) {
        if (p < steps) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) B[p][nt] = *(const v4i *)(wrow + (long)nt * 16 * a.kpad + p * 64);
        }
    }
    v4i acc[RB][NT];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rb][nt] = (v4i){0, 0, 0, 0};
    for (int s0 = 0; s0 < steps; s0 += P) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int s = s0 + p;
            if (s >= steps) break;
            const int kg = s * 64 + lg * 16;
            // The K slice's LDS offsets are shared by the row blocks. Every
            // read is in the tile (every lbase is a pixel of the tile, slices
            // past K read offset 0) and used as read: the weights of slices
            // past K are zero, and rows past the tile are never stored.
            v4i A[RB];
            if (!WORDS) {
                const int d = dl[kg < a.K ? kg >> 4 : 0];
#pragma unroll
                for (int rb = 0; rb < RB; rb++) A[rb] = *(const v4i *)(xt + lbase[rb] + d);
            } else {
                const int w0 = kg >> 2;
                int d[4];
#pragma unroll
                for (int j = 0; j < 4; j++) d[j] = dl[kg < a.K && w0 + j < ndelta ? w0 + j : 0];
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    A[rb] = (v4i){*(const int *)(xt + lbase[rb] + d[0]), *(const int *)(xt + lbase[rb] + d[1]),
                                  *(const int *)(xt + lbase[rb] + d[2]), *(const int *)(xt + lbase[rb] + d[3])};
            }
            // DIRECT: channels as the MFMA rows, for the register-direct store.
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
                    acc[rb][nt] = DIRECT ? __builtin_amdgcn_mfma_i32_16x16x64_i8(B[p][nt], A[rb], acc[rb][nt], 0, 0, 0)
                                         : __builtin_amdgcn_mfma_i32_16x16x64_i8(A[rb], B[p][nt], acc[rb][nt], 0, 0, 0);
            if (s + P < steps) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) B[p][nt] = *(const v4i *)(wrow + (long)nt * 16 * a.kpad + (s + P) * 64);
            }
        }
    }
    const long img0 = n * a.ohw;
    if constexpr (DIRECT && RB % 4 == 0) {
        conv_store_direct<RB, NT, (EMODE & 1) != 0, (EMODE & 2) != 0>(a, acc, n0, lane, img0 + p0 + wave * R,
                                                                       img0 + pend, epi_s, lut_s);
    } else if constexpr (DIRECT) {
        conv_store_pairs<RB, NT, (EMODE & 1) != 0, (EMODE & 2) != 0>(a, acc, n0, lane, img0 + p0 + wave * R,
                                                                      img0 + pend, epi_s, lut_s);
    } else {
        const int rw[RB][NT] = {};
        conv_epilogue_em<RB, NT, EMODE>(a, acc, stage, n0, lane, img0 + p0 + wave * R, img0 + pend, epi_s, lut_s,
                                        nullptr, rw);
    }
}

// Row blocks G0 .. min(G0 + 4, NRB) - 1 of a stem wave: each lane's window
// (five aligned LDS words byte-aligned into its 16-byte K slice), one MFMA
// per channel tile, then the group's requantised store. The kernel runs its
// row blocks in these groups of four (the transpose's group), so only 16 NT
// accumulator registers are live (70 instead of 82 VGPRs at NT = 2).
template <int NT, int NRB, bool HI, bool CORR, int G0>
__device__ __forceinline__ void stem_group(const ConvArgs &a, const v4i (&B)[NT], const int8_t *smem, int wbase,
                                           int step, int ox0, int lane, int n0, long rbase, long rlimit,
                                           const int4 *epi_s, const int8_t *lut_s)
{
    constexpr int NG = NRB - G0 < 4 ? NRB - G0 : 4;
    const int lr = lane & 15;
    v4i acc[4][NT];
#pragma unroll
    for (int q = 0; q < NG; q++) {
        const int ox = min(ox0 + (G0 + q) * 16 + lr, a.ow - 1);
        const int off = wbase + __mul24(ox, step);
        const int *p = (const int *)(smem + (off & ~3));
        const int w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
        const unsigned sh = (unsigned)off;             // byte-align uses the low two bits
        const v4i A = {(int)__builtin_amdgcn_alignbyte((unsigned)w1, (unsigned)w0, sh),
                       (int)__builtin_amdgcn_alignbyte((unsigned)w2, (unsigned)w1, sh),
                       (int)__builtin_amdgcn_alignbyte((unsigned)w3, (unsigned)w2, sh),
                       (int)__builtin_amdgcn_alignbyte((unsigned)w4, (unsigned)w3, sh)};
        // Channels as the MFMA rows (weights in A), pixels as its columns.
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            acc[q][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(B[nt], A, (v4i){0, 0, 0, 0}, 0, 0, 0);
    }
    conv_store_direct<4, NT, HI, CORR, NG>(a, acc, n0, lane, rbase + G0 * 16, rlimit, epi_s, lut_s);
}

// Stem convolution (few input channels, kh <= 4, kw * IC <= 16, no column
// dilation). The K step is one kernel row per 16-lane group: lane group lg
// holds kernel row ky = lg, and its 16-byte K slice is the kw * IC
// contiguous input bytes that row covers (byte kx * IC + c; weights are zero
// past kw * IC and for lane groups past kh). A block is four waves on four
// consecutive output rows of one image; each wave covers one segment of its
// row, seg_rb row blocks of 16 pixels, with NRB >= seg_rb row blocks of
// registers (the rows past the segment are not stored). The input rows the block touches are copied into
// LDS with a 16-byte gap after each row and 16 bytes before the first; the
// gaps and the rows outside the image hold the input zero point, so padding
// columns and rows read as the zero point and every window is one unaligned
// run of LDS bytes: five aligned words and four byte-aligns per row block, no
// per-tap bounds test. The channels are the MFMA's rows, so the requantised
// bytes leave straight from registers (conv_store_direct).
template <int NT, int NRB, int EMODE>
__global__ __launch_bounds__(256) void k_conv_stem(ConvArgs a)
{
    constexpr bool HI = EMODE & 1, CORR = EMODE & 2;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ __attribute__((aligned(4))) int8_t lut_s[256];
    __shared__ int4 epi_s[2 * NT * 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    // blockIdx.x = (image * row_groups + row_group) * segments + segment
    const int seg = blockIdx.x % a.segs;
    const int rg = blockIdx.x / a.segs;
    const int n = rg / a.row_groups, oy0 = (rg - n * a.row_groups) * 4, oy = oy0 + wave;
    const bool row_ok = oy < a.oh;
    const int ox0 = seg * a.seg_rb * 16;
    const int n0 = blockIdx.y * NT * 16;
    const int xzw = (a.xz & 0xff) * 0x01010101;
    const v4i xzv = {xzw, xzw, xzw, xzw};
    const int rowbytes = a.iw * a.ic;                  // a multiple of 16 (host checked)
    const int rs = rowbytes + 16;                      // LDS row stride: the row and its gap
    const int iy_base = oy0 * a.sh - a.pt;             // input row of staged row 0
    const int8_t *xim = a.x + (long)n * a.ih * rowbytes;

    const int8_t *wrow = a.w + (long)(n0 + lr) * 64 + lg * 16;
    v4i B[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) B[nt] = *(const v4i *)(wrow + (long)nt * 16 * 64);

    // Stage: chunk c = r * cpr + j is 16-byte piece j of staged row r (the
    // last piece of a row is its gap), at LDS byte 16 + r * rs + 16 j. Four
    // loads per thread are in flight before the first LDS write.
    {
        const int cpr = a.stem_cpr, total = a.stem_rows * cpr;
        for (int c0 = threadIdx.x; c0 < total; c0 += 4 * 256) {
            v4i v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + j * 256;
                const int r = (int)udiv((unsigned)c, (unsigned)cpr, a.stem_cpr_magic), k = c - r * cpr;
                const int iy = iy_base + r;
                v[j] = xzv;
                if (c < total && k < cpr - 1 && (unsigned)iy < (unsigned)a.ih)
                    v[j] = *(const v4i *)(xim + (long)iy * rowbytes + k * 16);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + j * 256;
                if (c < total) ((v4i *)smem)[1 + c] = v[j];
            }
        }
        if (threadIdx.x == 0) ((v4i *)smem)[0] = xzv;
    }
    stage_consts<NT>(a, n0, epi_s, lut_s);

    // Staged row of this lane's kernel row (row 0 for lane groups past kh,
    // whose weights are zero) and the LDS byte of its window at pixel 0.
    const int ky = lg < a.kh ? lg : 0;
    const int wbase = 16 + (wave * a.sh + ky * a.dh) * rs - a.pl * a.ic;
    const int step = a.sw * a.ic;                      // window bytes between neighbouring pixels
    __syncthreads();
    // Output pixels of this wave: its output row, ox0 .. min(ox0 + seg_rb * 16, ow).
    const long rbase = ((long)n * a.oh + oy) * a.ow + ox0;
    const int send = min(ox0 + a.seg_rb * 16, a.ow);
    const long rlimit = row_ok ? ((long)n * a.oh + oy) * a.ow + send : rbase;
    stem_group<NT, NRB, HI, CORR, 0>(a, B, smem, wbase, step, ox0, lane, n0, rbase, rlimit, epi_s, lut_s);
    if constexpr (NRB > 4)
        stem_group<NT, NRB, HI, CORR, 4>(a, B, smem, wbase, step, ox0, lane, n0, rbase, rlimit, epi_s, lut_s);
}

// Dynamic LDS of k_conv_stem (a 16-byte lead, the staged rows each followed
// by a 16-byte gap, 32 bytes of slack for the last window's word reads), 0
// when the layer does not fit it: kh <= 4, no column dilation, kw * IC <= 16,
// left padding and the columns past the right edge each within 16 bytes,
// rows a multiple of 16 bytes, the stage at most 48 KiB, and OC a multiple
// of 16 (whole 16-byte stores).
static size_t stem_lds(const UQKSpatial *d)
{
    const int rowbytes = d->iw * d->ic;
    const int rows = 3 * d->sh + (d->kh - 1) * d->dh + 1;
    const int over = (d->ow - 1) * d->sw - d->pl + d->kw - d->iw;
    const size_t bytes = 16 + (size_t)rows * (rowbytes + 16) + 32;
    const bool fits = d->kh >= 1 && d->kh <= 4 && d->dw == 1 && d->kw * d->ic <= 16 && d->pl >= 0 &&
                      d->pl * d->ic <= 16 && (over > 0 ? over : 0) * d->ic <= 16 && rowbytes % 16 == 0 &&
                      d->oc % 16 == 0 && d->ow >= 1;
    return fits && bytes <= 49152 ? bytes : 0;
}

extern "C" int uqk_conv_stem_ok(const UQKSpatial *d) { return stem_lds(d) > 0; }

template <int RB, int NT>
static void launch_conv_mode(int mode, const ConvArgs &a, dim3 grid, size_t)
{
    const size_t lds = conv_lds(a.kpad, RB, NT);
    switch (mode) {
    case UQK_PW:
        // The common case: one kernel per requantisation variant and per
        // presence of a fused add.
#define UQK_PW_EM(ADD, DIR)                                                                                        \
    do {                                                                                                           \
        switch (a.emode) {                                                                                         \
        case 0: UQK_LAUNCH((k_conv<RB, NT, UQK_PW, 0, ADD, DIR>), grid, dim3(256), lds, g_stream, a); break;  \
        case 1: UQK_LAUNCH((k_conv<RB, NT, UQK_PW, 1, ADD, DIR>), grid, dim3(256), lds, g_stream, a); break;  \
        case 2: UQK_LAUNCH((k_conv<RB, NT, UQK_PW, 2, ADD, DIR>), grid, dim3(256), lds, g_stream, a); break;  \
        default: UQK_LAUNCH((k_conv<RB, NT, UQK_PW, 3, ADD, DIR>), grid, dim3(256), lds, g_stream, a); break; \
        }                                                                                                          \
    } while (0)
        // Register-direct stores when every store is a whole 16 bytes, the
        // tiles form whole groups of four and no add is fused (a padded
        // group, or the add applied per transposed word, measured slower
        // than the LDS stage).
        if (a.res) UQK_PW_EM(true, false);
        else if constexpr ((RB * NT) % 4 == 0) {
            if (a.oc % 16 == 0) UQK_PW_EM(false, true);
            else UQK_PW_EM(false, false);
        } else UQK_PW_EM(false, false);
#undef UQK_PW_EM
        break;
    case UQK_G16: UQK_LAUNCH((k_conv<RB, NT, UQK_G16, -1, true, false>), grid, dim3(256), lds, g_stream, a); break;
    case UQK_G4: UQK_LAUNCH((k_conv<RB, NT, UQK_G4, -1, true, false>), grid, dim3(256), lds, g_stream, a); break;
    default: UQK_LAUNCH((k_conv<RB, NT, UQK_G1, -1, true, false>), grid, dim3(256), lds, g_stream, a); break;
    }
}

template <int RB>
static void launch_conv_nt(int nt, int mode, const ConvArgs &a, dim3 grid, size_t lds)
{
    switch (nt) {
    case 2: launch_conv_mode<RB, 2>(mode, a, grid, lds); break;
    case 4: launch_conv_mode<RB, 4>(mode, a, grid, lds); break;
    case 6: launch_conv_mode<RB, 6>(mode, a, grid, lds); break;
    default: launch_conv_mode<RB, 8>(mode, a, grid, lds); break;
    }
}

// Whether k_conv_rows stores from registers (no LDS output stage): whole
// 16-byte stores, and row blocks (conv_store_direct) or channel tiles
// (conv_store_pairs) that go through the transpose in fours.
static bool rows_direct(int rb, int nt, int oc)
{
    return oc % 16 == 0 && (rb % 4 == 0 || (rb * nt) % 4 == 0);
}

template <int RB>
static void launch_rows_nt(int nt, int mode, const ConvArgs &a, dim3 grid, size_t lds)
{
    // Register-direct epilogue (no LDS output stage) as rows_direct decides;
    // uqk_conv picks rb = 4 only when OC % 16 == 0, and every even NT makes
    // two row blocks whole groups of four tiles.
#define UQK_ROWS_EM(NT, W, DIR)                                                                                 \
    do {                                                                                                        \
        switch (a.emode) {                                                                                      \
        case 0: UQK_LAUNCH((k_conv_rows<RB, NT, W, 0, DIR>), grid, dim3(256), lds, g_stream, a); break; \
        case 1: UQK_LAUNCH((k_conv_rows<RB, NT, W, 1, DIR>), grid, dim3(256), lds, g_stream, a); break; \
        case 2: UQK_LAUNCH((k_conv_rows<RB, NT, W, 2, DIR>), grid, dim3(256), lds, g_stream, a); break; \
        default: UQK_LAUNCH((k_conv_rows<RB, NT, W, 3, DIR>), grid, dim3(256), lds, g_stream, a); break; \
        }                                                                                                       \
    } while (0)
#define UQK_ROWS_DIR(NT, W)                                                                                     \
    do {                                                                                                        \
        if constexpr (RB % 4 == 0) UQK_ROWS_EM(NT, W, true);                                                    \
        else if (rows_direct(RB, NT, a.oc)) UQK_ROWS_EM(NT, W, true);                                           \
        else UQK_ROWS_EM(NT, W, false);                                                                         \
    } while (0)
#define UQK_ROWS_LAUNCH(NT)                                                                                     \
    do {                                                                                                        \
        if (mode == UQK_ROWS16) UQK_ROWS_DIR(NT, false);                                                        \
        else UQK_ROWS_DIR(NT, true);                                                                            \
    } while (0)
    switch (nt) {
    case 2: UQK_ROWS_LAUNCH(2); break;
    case 4: UQK_ROWS_LAUNCH(4); break;
    case 6: UQK_ROWS_LAUNCH(6); break;
    default: UQK_ROWS_LAUNCH(8); break;
    }
#undef UQK_ROWS_LAUNCH
#undef UQK_ROWS_DIR
#undef UQK_ROWS_EM
}

// Bytes of dynamic LDS the row-staged kernel needs for one layer.
// Output pixels per k_conv_rows tile: whole output rows when they fill at
// least 7/8 of the block's 64*rb pixels (then a tile's input rows overlap its
// neighbours' only by the kernel's halo), else 64*rb consecutive pixels.
// Sets *span to the most output rows one tile touches.
static int rows_tile(const UQKSpatial *d, int rb, int *span)
{
    const int bm = 4 * 16 * rb, rpt = bm / d->ow;
    if (rpt >= 1 && 8 * rpt * d->ow >= 7 * bm) {
        *span = rpt;
        return rpt * d->ow;
    }
    *span = (bm + d->ow - 2) / d->ow + 1;   // bm consecutive pixels from any column
    return bm;
}

// Dynamic LDS of k_conv_rows at rb row blocks per wave: the staged tile, the
// offset table and, unless the epilogue stores straight from registers
// (rb = 4, OC % 16 == 0), the output stage.
static size_t rows_lds(const UQKSpatial *d, int rb, bool with_stage = false)
{
    int span;
    rows_tile(d, rb, &span);
    const bool direct = !with_stage && rows_direct(rb, d->nt, d->oc);
    const int rows_max = (span - 1) * d->sh + (d->kh - 1) * d->dh + 1;
    const int cols = (d->ow - 1) * d->sw + (d->kw - 1) * d->dw + 1;
    const int ndelta = d->mode == UQK_ROWS16 ? d->K / 16 : d->K / 4;
    const int icp = d->mode == UQK_ROWS16 ? d->ic : (d->ic + 3) & ~3;
    return (size_t)((rows_max * cols * icp + 15) & ~15) + (size_t)((ndelta * 4 + 15) & ~15) +
           (direct ? 0 : (size_t)4 * 16 * rb * (16 * d->nt + 16));
}

extern "C" size_t uqk_conv_rows_lds(const UQKSpatial *d, int rb) { return rows_lds(d, rb); }

// Plan-time choice of the row-staged kernel: its two-row-block tile, counted
// with an output stage, within 64 KiB. Layers past that (wide K, such as a
// 3x3 over 128 channels at 80x80) measured faster as gathers (k_conv G16:
// 857 against 584 TOPS), so the register-direct epilogue's smaller footprint
// does not move them.
extern "C" int uqk_conv_rows_ok(const UQKSpatial *d) { return rows_lds(d, 2, true) <= 65536; }

static int conv_launch(const UQKSpatial *d, const void *x, void *y, uint32_t batches, const UQKAdd *add);

extern "C" int uqk_conv(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    return conv_launch(d, x, y, batches, nullptr);
}

extern "C" int uqk_conv_add_ok(const UQKSpatial *d)
{
    return d->mode == UQK_PW || d->mode == UQK_G16 || d->mode == UQK_G4 || d->mode == UQK_G1;
}

extern "C" int uqk_conv_add(const UQKSpatial *d, const void *x, void *y, uint32_t batches, const UQKAdd *add)
{
    if (!uqk_conv_add_ok(d) || !add || !add->res || !add->tables) return (int)hipErrorInvalidValue;
    return conv_launch(d, x, y, batches, add);
}

static int conv_launch(const UQKSpatial *d, const void *x, void *y, uint32_t batches, const UQKAdd *add)
{
    ConvArgs a;
    a.res = add ? (const int8_t *)add->res : nullptr;
    a.add_tab = add ? (const int *)add->tables : nullptr;
    a.add_m = add ? add->m : 0; a.add_s = add ? add->s : 0; a.add_yz = add ? add->yz : 0;
    a.add_lo = add ? add->lo : 0; a.add_hi = add ? add->hi : 0; a.add_conv_a = add ? add->conv_is_a : 0;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.kmap = (const int4 *)d->kmap;
    a.delta = (const int *)d->kmap;
    a.lut = (const uint8_t *)d->lut;
    a.M = (long)batches * d->oh * d->ow;
    a.ih = d->ih; a.iw = d->iw; a.ic = d->ic; a.oh = d->oh; a.ow = d->ow; a.oc = d->oc;
    a.icp = d->mode == UQK_ROWS4 ? (d->ic + 3) & ~3 : d->ic;
    a.kh = d->kh; a.sh = d->sh; a.sw = d->sw; a.dh = d->dh; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.K = d->K; a.kpad = d->kpad; a.ohw = d->oh * d->ow; a.corr = d->corr;
    a.emode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0);
    a.cols = (d->ow - 1) * d->sw + (d->kw - 1) * d->dw + 1;
    a.kw = d->kw; a.dw = d->dw; a.taps = d->kh * d->kw;
    if (a.M <= 0) return 0;
    if (!add && uqk_gemm_take(d, (uint64_t)a.M)) return uqk_gemm(d, x, y, batches);
    const int nchunks = d->oc_pad / (16 * d->nt);
    if (d->mode == UQK_STEM) {
        // A block is four output rows; each wave covers one segment of its
        // row, at most eight row blocks of 16 pixels (rows up to 128 pixels
        // are one segment, so each input row is staged once, and the
        // segments of longer rows share the row blocks evenly). The channel
        // slice covers up to 64 channels (NT = oc_pad / 16 when that is 1, 2
        // or 4).
        const int nt = d->oc_pad == 16 ? 1 : d->oc_pad == 32 ? 2 : 4;
        const int rbs = (d->ow + 15) / 16;
        a.images = (int)batches;
        a.segs = (rbs + 7) / 8;
        a.seg_rb = (rbs + a.segs - 1) / a.segs;
        a.row_groups = (d->oh + 3) / 4;
        a.stem_rows = 3 * d->sh + (d->kh - 1) * d->dh + 1;
        a.stem_cpr = d->iw * d->ic / 16 + 1;
        a.stem_cpr_magic = udiv_magic((unsigned)a.stem_cpr);
        const size_t lds = stem_lds(d);
        const unsigned long long items = (unsigned long long)batches * a.row_groups * a.segs;
        if (!lds || items > 0x7fffffffULL || (unsigned long long)d->ih * d->iw * d->ic > 0x7fffffffULL)
            return (int)hipErrorInvalidValue;
        dim3 grid((unsigned)items, (unsigned)(d->oc_pad / (16 * nt)));
        // Row blocks of registers per wave: seg_rb, at least four.
        const int nrb = a.seg_rb < 4 ? 4 : a.seg_rb;
#define UQK_STEM_EM(NT, NRB)                                                                               \
    do {                                                                                                   \
        switch (a.emode) {                                                                                 \
        case 0: UQK_LAUNCH((k_conv_stem<NT, NRB, 0>), grid, dim3(256), lds, g_stream, a); break;   \
        case 1: UQK_LAUNCH((k_conv_stem<NT, NRB, 1>), grid, dim3(256), lds, g_stream, a); break;   \
        case 2: UQK_LAUNCH((k_conv_stem<NT, NRB, 2>), grid, dim3(256), lds, g_stream, a); break;   \
        default: UQK_LAUNCH((k_conv_stem<NT, NRB, 3>), grid, dim3(256), lds, g_stream, a); break;  \
        }                                                                                                  \
    } while (0)
#define UQK_STEM_RB(NT)                                                                                    \
    do {                                                                                                   \
        switch (nrb) {                                                                                     \
        case 4: UQK_STEM_EM(NT, 4); break;                                                                 \
        case 5: UQK_STEM_EM(NT, 5); break;                                                                 \
        case 6: UQK_STEM_EM(NT, 6); break;                                                                 \
        case 7: UQK_STEM_EM(NT, 7); break;                                                                 \
        default: UQK_STEM_EM(NT, 8); break;                                                                \
        }                                                                                                  \
    } while (0)
        if (nt == 1) UQK_STEM_RB(1);
        else if (nt == 2) UQK_STEM_RB(2);
        else UQK_STEM_RB(4);
#undef UQK_STEM_RB
#undef UQK_STEM_EM
        UQK_LAUNCHED();
        return 0;
    }
    if (d->mode == UQK_ROWS16 || d->mode == UQK_ROWS4) {
        // Larger tiles stage fewer redundant input rows per output row.
        const int rb = d->nt <= 4 && d->oc % 16 == 0 && rows_lds(d, 4) <= 65536 ? 4 : 2;
        int span;
        a.tile_px = rows_tile(d, rb, &span);
        a.tiles = (a.ohw + a.tile_px - 1) / a.tile_px;
        a.rows_max = (span - 1) * d->sh + (d->kh - 1) * d->dh + 1;
        {
            // Staging divisors: items per staged row and per pixel (16-byte
            // chunks for ROWS16, words for ROWS4).
            const unsigned per_px = d->mode == UQK_ROWS16 ? (unsigned)d->ic / 16 : (unsigned)((d->ic + 3) & ~3) / 4;
            const unsigned per_row = (unsigned)a.cols * per_px;
            if ((unsigned long long)a.rows_max * per_row >= 65536ULL) return (int)hipErrorInvalidValue;
            a.m_row = udiv_magic(per_row);
            a.m_px = udiv_magic(per_px);
        }
        dim3 grid((unsigned)((long)batches * a.tiles), (unsigned)nchunks);
        if (rb == 4) launch_rows_nt<4>(d->nt, d->mode, a, grid, uqk_conv_rows_lds(d, rb));
        else launch_rows_nt<2>(d->nt, d->mode, a, grid, uqk_conv_rows_lds(d, rb));
    } else {
        // Narrower channel slices when the batch gives too few waves to keep
        // four per SIMD (1024 SIMDs): more slices re-read the (small) input
        // but hide the K loop's load latency. 8 -> 4 -> 2 and 6 -> 2 keep
        // oc_pad (a multiple of 16 * NT) a whole number of slices. The rows
        // of the image slices running side by side count together.
        int nt = d->nt;
        const long m_live = a.M * g_live_slices;
        const long row_waves = (m_live + 15) / 16;
        while (nt > 2 && row_waves * (d->oc_pad / (16 * nt)) < 4096) nt = nt == 8 ? 4 : 2;
        const int chunks = d->oc_pad / (16 * nt);
        // Two row blocks per wave only when that still gives every SIMD of
        // the chip several waves.
        const long waves2 = (m_live + 31) / 32 * chunks;
        const int rb = waves2 >= 8192 ? 2 : 1;
        const long rows = 4L * 16 * rb;
        dim3 grid((unsigned)((a.M + rows - 1) / rows), (unsigned)chunks);
        if (rb == 2) launch_conv_nt<2>(nt, d->mode, a, grid, 0);
        else launch_conv_nt<1>(nt, d->mode, a, grid, 0);
    }
    UQK_LAUNCHED();
    return 0;
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
    int groups, ih, iw, c, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl, xz, yz, lo, hi, ohw, is_max, corr;
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

template <int VEC, bool POOL, int KS>
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
    const int kh = KS ? KS : a.kh, kw = KS ? KS : a.kw;
#pragma unroll
    for (int ky = 0; ky < kh; ky++) {
        const int iy = oy * a.sh - a.pt + ky * a.dh;
        const bool rowin = iy >= 0 && iy < a.ih;
#pragma unroll
        for (int kx = 0; kx < kw; kx++) {
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
                load_vec<VEC>(a.w + (long)(ky * kw + kx) * a.c + c0, ww);
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
            v = uq_requant_affine(acc[j], load_epi(a.epi, c0 + j), a.corr, a.yz, a.lo, a.hi);
            if (a.lut) v = (int)(signed char)a.lut[v + 128];
        }
        out[j] = v;
    }
    store_vec<VEC>(a.y + pix * a.c + c0, out);
}

// Depthwise with an LDS input tile: a block covers a th x tw patch of output
// pixels for cg groups of 16 channels of one image. The input patch (halo and
// padding included, padding written as xz), the block's weights (four taps of
// one channel per word) and its epilogue records are staged in LDS once. Each
// thread produces 16 channels of one output pixel: per group of four taps it
// reads the four 16-byte tap vectors, transposes each 4x4 byte block with
// v_perm so that a word holds four taps of one channel, and accumulates with
// v_dot4 (int8 x int8 -> int32), i.e. 12 VALU ops per 16 tap-channel MACs.
struct DwTileArgs {
    const int8_t *x;
    int8_t *y;
    const int *wdot;
    const int4 *epi;
    const uint8_t *lut;
    int ih, iw, c, oh, ow, sh, sw, dh, dw, pt, pl, xz, yz, lo, hi, corr;
    int th, tw, cg, tiles_x, ith, itw;
};

__device__ __forceinline__ void transpose4x4(int x0, int x1, int x2, int x3, int &y0, int &y1, int &y2, int &y3)
{
    // perm(s0, s1, sel): byte i of the result is byte sel_i of {s0:s1}, with
    // indices 0-3 naming s1's bytes and 4-7 naming s0's.
    const int t0 = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x05010400u);
    const int t1 = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x07030602u);
    const int t2 = (int)__builtin_amdgcn_perm((unsigned)x3, (unsigned)x2, 0x05010400u);
    const int t3 = (int)__builtin_amdgcn_perm((unsigned)x3, (unsigned)x2, 0x07030602u);
    y0 = (int)__builtin_amdgcn_perm((unsigned)t2, (unsigned)t0, 0x05040100u);
    y1 = (int)__builtin_amdgcn_perm((unsigned)t2, (unsigned)t0, 0x07060302u);
    y2 = (int)__builtin_amdgcn_perm((unsigned)t3, (unsigned)t1, 0x05040100u);
    y3 = (int)__builtin_amdgcn_perm((unsigned)t3, (unsigned)t1, 0x07060302u);
}

template <int KS>
__global__ __launch_bounds__(256) void k_dw_tile(DwTileArgs a)
{
    constexpr int TAPS = KS * KS, G = (TAPS + 3) / 4;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int cb = a.cg * 16;
    const int xbytes = (a.ith * a.itw * cb + 15) & ~15;
    int8_t *xt = smem;
    int *wt = (int *)(smem + xbytes);
    int4 *et = (int4 *)(smem + xbytes + G * cb * 4);
    const int ty = blockIdx.x / a.tiles_x, tx = blockIdx.x - ty * a.tiles_x;
    const int c0 = blockIdx.y * cb;
    const long n = blockIdx.z;
    const int oy0 = ty * a.th, ox0 = tx * a.tw;
    const int iy0 = oy0 * a.sh - a.pt, ix0 = ox0 * a.sw - a.pl;
    const int8_t *xim = a.x + n * a.ih * a.iw * a.c + c0;
    const int xzw = (a.xz & 0xff) * 0x01010101;
    const int chunks = a.ith * a.itw * a.cg;
    for (int q = threadIdx.x; q < chunks; q += 256) {
        const int p = q / a.cg, g = q - p * a.cg;
        const int r = p / a.itw, col = p - r * a.itw;
        const int iy = iy0 + r, ix = ix0 + col;
        v4i v = {xzw, xzw, xzw, xzw};
        if (iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw) v = *(const v4i *)(xim + ((long)iy * a.iw + ix) * a.c + g * 16);
        *(v4i *)(xt + q * 16) = v;
    }
    const int wq = cb / 4;
    for (int q = threadIdx.x; q < G * wq; q += 256) {
        const int g = q / wq, k = q - g * wq;
        *(v4i *)(wt + g * cb + 4 * k) = *(const v4i *)(a.wdot + (long)g * a.c + c0 + 4 * k);
    }
    for (int q = threadIdx.x; q < 2 * cb; q += 256) et[q] = a.epi[2 * c0 + q];
    __syncthreads();
    const int work = a.th * a.tw * a.cg;
    for (int q = threadIdx.x; q < work; q += 256) {
        const int p = q / a.cg, gi = q - p * a.cg;
        const int py = p / a.tw, px = p - py * a.tw;
        const int oy = oy0 + py, ox = ox0 + px;
        if (oy >= a.oh || ox >= a.ow) continue;
        int acc[16];
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = 0;
        const int8_t *xp = xt + ((py * a.sh) * a.itw + px * a.sw) * cb + gi * 16;
#pragma unroll
        for (int g = 0; g < G; g++) {
            v4i X[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = 4 * g + j < TAPS ? 4 * g + j : 4 * g;
                const int ky = t / KS, kx = t - (t / KS) * KS;
                X[j] = *(const v4i *)(xp + ((ky * a.dh) * a.itw + kx * a.dw) * cb);
            }
            const v4i *W = (const v4i *)(wt + g * cb + gi * 16);
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const v4i w4 = W[qd];
                int y0, y1, y2, y3;
                transpose4x4(X[0][qd], X[1][qd], X[2][qd], X[3][qd], y0, y1, y2, y3);
                acc[4 * qd + 0] = __builtin_amdgcn_sdot4(y0, w4[0], acc[4 * qd + 0], false);
                acc[4 * qd + 1] = __builtin_amdgcn_sdot4(y1, w4[1], acc[4 * qd + 1], false);
                acc[4 * qd + 2] = __builtin_amdgcn_sdot4(y2, w4[2], acc[4 * qd + 2], false);
                acc[4 * qd + 3] = __builtin_amdgcn_sdot4(y3, w4[3], acc[4 * qd + 3], false);
            }
        }
        int out[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            int v = uq_requant_affine(acc[j], load_epi(et, gi * 16 + j), a.corr, a.yz, a.lo, a.hi);
            if (a.lut) v = (int)(signed char)a.lut[v + 128];
            out[j] = v;
        }
        store_vec<16>(a.y + ((n * a.oh + oy) * a.ow + ox) * a.c + c0 + gi * 16, out);
    }
}

// Depthwise 3x3 / 5x5, stride 1 or 2, no dilation, C % 4 == 0, on tap
// windows. A block covers TH output rows x 4*XW output columns x 4*CQ
// channels of one image. Its input rows are staged in LDS as windows: the
// word W[r][j][c] holds channel c of the four input columns S*j .. S*j + 3 of
// staged row r, so output column x (tile-relative) finds its first four taps
// of row r in window j = x and, for 5x5, its fifth tap in byte 0 of window
// x + 4/S. Windows are laid out [row][j / 4][channel % 4][channel / 4][j % 4]
// with CQ * 16 bytes of padding after each j / 4 block: a thread's four
// consecutive output columns of one channel are one 16-byte LDS read,
// neighbouring lanes (neighbouring channel quads) read neighbouring 16-byte
// blocks, and the padded stride (80 * CQ bytes) spreads the lanes of
// different column quads over distinct banks. Each
// thread computes 4 columns x 4 channels; per kernel row and channel that is
// four v_dot4 against the row's taps packed in a word (a zero weight on the
// unused lane of the word). The windows are built from the input rows with a
// 4x4 byte transpose (channel-major words of four columns) and v_alignbyte
// for the shifted starts. Requantisation uses the conv epilogue's records.
struct DwWinArgs {
    const int8_t *x;
    int8_t *y;
    const int4 *wrow;          // [ky][wk][C] words of four taps (C/4 int4 per row)
    const int4 *epi;
    const uint8_t *lut;
    int ih, iw, c, oh, ow, pt, pl, xz, yz, lo, hi;
    int th, xw, cq, tiles_x, tiles, ir, njq;
    int lcq;                   // log2(cq)
    int njq_magic, xw_magic;   // ceil(2^16 / njq), ceil(2^16 / xw): exact small quotients
};

template <int KS, int S, bool HI, bool CORR>
__global__ __launch_bounds__(256) void k_dw_win(DwWinArgs a)
{
    constexpr int NWK = KS > 4 ? 2 : 1;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int *W = (int *)smem;
    const int cb = 4 * a.cq;
    // LDS: windows | tap words [ky][wk][cb] | channel records [cb][2] | table
    const int jqs = 5 * cb;   // dwords per j / 4 block: 4 * cb data + 4 * cq padding
    int *wt = (int *)(smem + (size_t)a.ir * a.njq * jqs * 4);
    int4 *et = (int4 *)(wt + KS * NWK * cb);
    int8_t *lut_s = (int8_t *)(et + 2 * cb);
    const long n = blockIdx.x / a.tiles;
    const int tile = (int)(blockIdx.x - n * a.tiles);
    const int ty = tile / a.tiles_x, tx = tile - ty * a.tiles_x;
    const int c0 = blockIdx.y * cb;
    const int oy0 = ty * a.th, ox0 = tx * 4 * a.xw;
    const int iy0 = oy0 * S - a.pt, ix0 = ox0 * S - a.pl;
    const int8_t *xim = a.x + n * a.ih * a.iw * a.c + c0;
    const int xzw = (a.xz & 0xff) * 0x01010101;

    // This thread's output item: 4 columns x 4 channels.
    const int tid = threadIdx.x;
    const int cqi = tid & (a.cq - 1), rest = tid >> a.lcq;
    const int tyi = (rest * a.xw_magic) >> 16, xq = rest - tyi * a.xw;
    const bool live = tyi < a.th && oy0 + tyi < a.oh;
    const int cbase = c0 + 4 * cqi;

    // The block's tap words and channel records.
    for (int u = tid; u < KS * NWK * a.cq; u += 256) {
        const int row = u >> a.lcq, cqd = u & (a.cq - 1);
        *(v4i *)(wt + row * cb + 4 * cqd) = *(const v4i *)(a.wrow + ((long)row * a.c + c0) / 4 + cqd);
    }
    // Records as [half][channel % 4][channel / 4] int4s: lanes read 16-byte steps.
    for (int u = tid; u < 2 * cb; u += 256) {
        const int h = u >> (a.lcq + 2), rem = u & (cb - 1), i = rem >> a.lcq, cqd = rem & (a.cq - 1);
        et[u] = a.epi[2 * (c0 + 4 * cqd + i) + h];
    }

    // Stage windows: one unit = 4 consecutive windows x 4 channels of a row.
    const int units = a.ir * a.njq * a.cq;
    for (int u = tid; u < units; u += 256) {
        const int cqd = u & (a.cq - 1), r2 = u >> a.lcq;
        const int r = (r2 * a.njq_magic) >> 16, jq = r2 - r * a.njq;
        const int iy = iy0 + r;
        const bool rowin = (unsigned)iy < (unsigned)a.ih;
        const int8_t *src = xim + (rowin ? iy : 0) * a.iw * a.c + 4 * cqd;
        const int px0 = ix0 + S * 4 * jq;
        // Every load reads a valid pixel (padding positions re-read column 0)
        // and the padding value is selected afterwards: no branches.
        int P[4 * S + 4];
#pragma unroll
        for (int p = 0; p < 4 * S + 4; p++) {
            const int ix = px0 + p;
            const bool in = rowin && (unsigned)ix < (unsigned)a.iw;
            const int v = *(const int *)(src + (in ? ix : 0) * a.c);
            P[p] = in ? v : xzw;
        }
        int col[S + 1][4];   // col[g][i]: channel i over columns 4g .. 4g + 3
#pragma unroll
        for (int g = 0; g < S + 1; g++)
            transpose4x4(P[4 * g], P[4 * g + 1], P[4 * g + 2], P[4 * g + 3], col[g][0], col[g][1], col[g][2], col[g][3]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int w4[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int start = S * t;              // first column of window 4*jq + t
                const int g = start >> 2, sh = start & 3;
                w4[t] = sh ? (int)__builtin_amdgcn_alignbyte((unsigned)col[g + 1][i], (unsigned)col[g][i], (unsigned)sh)
                           : col[g][i];
            }
            *(v4i *)(W + ((long)r * a.njq + jq) * jqs + (i * a.cq + cqd) * 4) = (v4i){w4[0], w4[1], w4[2], w4[3]};
        }
    }
    if (a.lut && tid < 64) ((int *)lut_s)[tid] = ((const int *)a.lut)[tid];
    __syncthreads();
    if (!live) return;

    int acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0;
    // 5x5: one kernel row at a time keeps the register footprint small
    // enough for several waves per SIMD.
    constexpr int KU = KS > 4 ? 1 : KS;
#pragma unroll KU
    for (int ky = 0; ky < KS; ky++) {
        const int r = tyi * S + ky;
        const int *row = W + (long)r * a.njq * jqs + cqi * 4;
        const v4i w0 = *(const v4i *)(wt + (ky * NWK) * cb + 4 * cqi);
        const v4i w1 = *(const v4i *)(wt + (ky * NWK + NWK - 1) * cb + 4 * cqi);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const v4i win = *(const v4i *)(row + (long)xq * jqs + i * a.cq * 4);
#pragma unroll
            for (int t = 0; t < 4; t++) acc[t][i] = __builtin_amdgcn_sdot4(win[t], w0[i], acc[t][i], false);
            if (KS > 4) {
                int w2[4];
                if (S == 1) {
                    const v4i v = *(const v4i *)(row + (long)(xq + 1) * jqs + i * a.cq * 4);
                    w2[0] = v[0]; w2[1] = v[1]; w2[2] = v[2]; w2[3] = v[3];
                } else {
                    const int2 lo2 = *(const int2 *)(row + (long)xq * jqs + i * a.cq * 4 + 2);
                    const int2 hi2 = *(const int2 *)(row + (long)(xq + 1) * jqs + i * a.cq * 4);
                    w2[0] = lo2.x; w2[1] = lo2.y; w2[2] = hi2.x; w2[3] = hi2.y;
                }
#pragma unroll
                for (int t = 0; t < 4; t++) acc[t][i] = __builtin_amdgcn_sdot4(w2[t], w1[i], acc[t][i], false);
            }
        }
    }
    const int oy = oy0 + tyi;
    int8_t *yrow = a.y + ((n * a.oh + oy) * a.ow) * (long)a.c + cbase;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    Epi e[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int4 lo4 = et[i * a.cq + cqi], hi4 = et[cb + i * a.cq + cqi];
        e[i].bias = lo4.x; e[i].m = lo4.y; e[i].ls = lo4.z; e[i].T = lo4.w;
        e[i].c1 = (long long)(((unsigned long long)(unsigned)hi4.y << 32) | (unsigned)hi4.x);
        e[i].cthr = (long long)(((unsigned long long)(unsigned)hi4.w << 32) | (unsigned)hi4.z);
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ox = ox0 + 4 * xq + t;
        if (ox >= a.ow) break;
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[t][i], e[i], a.yz, vlo, vhi);
        if (a.lut) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
        }
        *(int *)(yrow + (long)ox * a.c) = pack4(v[0], v[1], v[2], v[3]);
    }
}

// Tile geometry for k_dw_win; returns the dynamic LDS bytes, 0 if unsuited.
static size_t dw_win_plan(const UQKSpatial *d, DwWinArgs *t)
{
    const int ks = d->kh, s = d->sh;
    if (d->oc % 4 || d->kh != d->kw || (ks != 3 && ks != 5) || d->sh != d->sw || (s != 1 && s != 2) ||
        d->dh != 1 || d->dw != 1)
        return 0;
    const int c4 = d->oc / 4;
    int cq = 1;
    while (cq < 16 && c4 % (2 * cq) == 0) cq *= 2;
    const int xq_all = (d->ow + 3) / 4;
    const int tiles_x = (xq_all + 7) / 8;
    const int xw = (xq_all + tiles_x - 1) / tiles_x;
    // Wide rows take four channel quads per block, narrow maps more.
    if (xw >= 4 && cq > 4) cq = 4;
    int th = 256 / (xw * cq);
    if (th < 1) return 0;
    if (th > d->oh) th = d->oh;
    t->th = th; t->xw = xw; t->cq = cq; t->tiles_x = tiles_x;
    t->ir = (th - 1) * s + ks;
    const int nj = 4 * xw + (ks > 4 ? 4 / s : 0);
    t->njq = (nj + 3) / 4;
    t->lcq = 0;
    while ((1 << t->lcq) < cq) t->lcq++;
    // (v * ceil(2^16 / d)) >> 16 == v / d for v < 2^16 / d; here v < 256 / cq
    // (items) and v < ir * njq (staging rows), both far below that bound.
    t->njq_magic = (65536 + t->njq - 1) / t->njq;
    t->xw_magic = (65536 + xw - 1) / xw;
    if (t->ir * t->njq >= 65536 / t->njq) return 0;
    const size_t bytes = (size_t)t->ir * t->njq * cq * 5 * 16 + (size_t)ks * (ks > 4 ? 2 : 1) * cq * 16 +
                         (size_t)cq * 4 * 32 + 256;
    return bytes <= 65536 ? bytes : 0;
}

extern "C" size_t uqk_dw_win_lds(const UQKSpatial *d)
{
    DwWinArgs t;
    return dw_win_plan(d, &t);
}

static int launch_dw_win(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    DwWinArgs a;
    const size_t lds = dw_win_plan(d, &a);
    if (!lds) return -1;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.wrow = (const int4 *)d->wdot;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.c = d->oc; a.oh = d->oh; a.ow = d->ow; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.tiles = (d->oh + a.th - 1) / a.th * a.tiles_x;
    const unsigned long long blocks = (unsigned long long)a.tiles * batches;
    if (blocks > 0x7fffffffULL) return -1;
    dim3 grid((unsigned)blocks, (unsigned)(d->oc / (4 * a.cq)));
    const int mode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0);
#define UQK_DWW(K, S)                                                                                        \
    do {                                                                                                     \
        switch (mode) {                                                                                      \
        case 0: UQK_LAUNCH((k_dw_win<K, S, false, false>), grid, dim3(256), lds, g_stream, a); break; \
        case 1: UQK_LAUNCH((k_dw_win<K, S, true, false>), grid, dim3(256), lds, g_stream, a); break;  \
        case 2: UQK_LAUNCH((k_dw_win<K, S, false, true>), grid, dim3(256), lds, g_stream, a); break;  \
        default: UQK_LAUNCH((k_dw_win<K, S, true, true>), grid, dim3(256), lds, g_stream, a); break;  \
        }                                                                                                    \
    } while (0)
    if (d->kh == 3 && d->sh == 1) UQK_DWW(3, 1);
    else if (d->kh == 3) UQK_DWW(3, 2);
    else if (d->sh == 1) UQK_DWW(5, 1);
    else UQK_DWW(5, 2);
#undef UQK_DWW
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Depthwise on the matrix cores (KS 3 or 5, stride 1 or 2, C % 16 == 0).
//
// One MFMA computes 16 output pixels x 16 channels over four taps: the K
// dimension is (tap, channel) with 16 channels per tap, the pixel operand of
// lane (pixel lr, slice lg) is the 16 channel bytes of the input pixel under
// tap 4m + lg (one 16-byte LDS read, NHWC as staged, no transposes), and the
// weight operand is block-diagonal: lane (channel lr, slice lg) holds
// w[tap 4m + lg][channel lr] in byte lr and zeros elsewhere. ceil(KS*KS / 4)
// MFMAs (7 for 5x5, 3 for 3x3) give the depthwise sums of a 16 x 16 tile;
// taps past KS*KS carry zero weights. The products and their sum are the
// signed int8 ones of the dot4 kernel, so the same records requantise them.
//
// A block is one band of output rows of one image (the whole map when its
// window fits 40 KiB of LDS) x GB groups of 16 channels (GB = 1, 2 or 4; more
// for small maps, whose images have few tiles): the padded input window the
// band's outputs need ((rows-1)*S + KS rows, (OW-1)*S + KS columns, padding
// as the zero point) is staged once in LDS, one plane per group, and the 4/GB
// waves of a group take 16-pixel tiles of the band's flattened output in turn
// (so 7x7 maps waste only the last tile's tail). Blocks are ordered channel
// groups outer, image and band inner, so the groups of one image share an XCD
// (and its L2) when the block count per group set is a multiple of 8.
// ---------------------------------------------------------------------------
struct DwMArgs {
    const int8_t *x;
    int8_t *y;
    const int *wdot;           // [ky][wk][C] words of four taps
    const int4 *epi;
    const uint8_t *lut;
    int ih, iw, c, oh, ow, pt, pl, xz, yz, lo, hi;
    int images, rows_p, cols_p;
    int band, bands;           // output rows per block, blocks per image and group set
    int lgb, lwg;              // log2 of channel groups per block, of waves per group
    unsigned m_cols, m_ow;     // udiv_magic(cols_p), udiv_magic(ow)
};

template <int KS, int S, bool HI, bool CORR>
__global__ __launch_bounds__(256) void k_dw_mfma(DwMArgs a)
{
    constexpr int T = KS * KS, NG = (T + 3) / 4, NWK = KS > 4 ? 2 : 1;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ __attribute__((aligned(4))) int8_t lut_s[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    // blockIdx.x = (group set * images + image) * bands + band
    const int per_set = a.images * a.bands;
    const int gblock = blockIdx.x / per_set, nb = blockIdx.x - gblock * per_set;
    const int n = nb / a.bands, oyb = (nb - n * a.bands) * a.band;   // first output row of the band
    const int brows = min(a.band, a.oh - oyb);
    const int gw = wave >> a.lwg, wsub = wave & ((1 << a.lwg) - 1);   // this wave's group, rank in it
    const int cblk = gblock << (a.lgb + 4), c0 = cblk + gw * 16;
    const int xzw = (a.xz & 0xff) * 0x01010101;
    const int plane = a.rows_p * a.cols_p;          // staged pixels per group (a full band)
    const int iyb = oyb * S - a.pt;                 // input row of staged row 0

    // Stage the band's padded window: item q = (staged pixel, group) with the
    // group fastest (one pixel's GB 16-byte chunks are contiguous in HBM);
    // staged pixel (r, cc) is input (iyb + r, cc - pl).
    {
        const int8_t *xim = a.x + (long)n * a.ih * a.iw * a.c + cblk;
        const int total = (((brows - 1) * S + KS) * a.cols_p) << a.lgb;
        for (int q0 = threadIdx.x; q0 < total; q0 += 4 * 256) {
            v4i v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int q = q0 + j * 256, sp = q >> a.lgb, gq = q & ((1 << a.lgb) - 1);
                const int r = (int)udiv((unsigned)sp, (unsigned)a.cols_p, a.m_cols), cc = sp - r * a.cols_p;
                const int iy = iyb + r, ix = cc - a.pl;
                const bool in = q < total && (unsigned)iy < (unsigned)a.ih && (unsigned)ix < (unsigned)a.iw;
                v[j] = (v4i){xzw, xzw, xzw, xzw};
                if (in) v[j] = *(const v4i *)(xim + ((long)iy * a.iw + ix) * a.c + gq * 16);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int q = q0 + j * 256;
                if (q < total) ((v4i *)smem)[(q & ((1 << a.lgb) - 1)) * plane + (q >> a.lgb)] = v[j];
            }
        }
    }
    if (a.lut && threadIdx.x < 64) ((int *)lut_s)[threadIdx.x] = ((const int *)a.lut)[threadIdx.x];

    // This lane's weight operands and tap offsets (LDS bytes from a pixel's
    // window corner); taps past T use offset 0 and zero weights.
    v4i B[NG];
    int off[NG];
#pragma unroll
    for (int m = 0; m < NG; m++) {
        const int t = 4 * m + lg;
        const int ky = t / KS, kx = t - ky * KS;
        int wb = 0;
        if (t < T) wb = (a.wdot[(ky * NWK + (kx >> 2)) * a.c + c0 + lr] >> (8 * (kx & 3))) & 0xff;
        const int word = wb << (8 * (lr & 3)), at = lr >> 2;
        B[m] = (v4i){at == 0 ? word : 0, at == 1 ? word : 0, at == 2 ? word : 0, at == 3 ? word : 0};
        off[m] = t < T ? (ky * a.cols_p + kx) * 16 : 0;
    }
    const Epi e = load_epi(a.epi, c0 + lr);
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    __syncthreads();

    const int npix = brows * a.ow, tiles = (npix + 15) >> 4;   // the band's output pixels
    int8_t *yim = a.y + ((long)n * a.oh + oyb) * a.ow * a.c + c0;
    const int8_t *pl = smem + (size_t)gw * plane * 16;
    for (int tile = wsub; tile < tiles; tile += 1 << a.lwg) {
        // A row: band pixel p (clamped into the band for the tail tile).
        const int p = min(tile * 16 + lr, npix - 1);
        const int oy = (int)udiv((unsigned)p, (unsigned)a.ow, a.m_ow), ox = p - oy * a.ow;   // oy within the band
        const int8_t *base = pl + (oy * S * a.cols_p + ox * S) * 16;
        v4i A[NG];
#pragma unroll
        for (int m = 0; m < NG; m++) A[m] = *(const v4i *)(base + off[m]);
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < NG; m++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], B[m], acc, 0, 0, 0);
        // acc[i]: pixel tile*16 + 4*lg + i, channel c0 + lr.
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[i], e, a.yz, vlo, vhi);
        if (a.lut) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
        }
        const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
        const int px = tile * 16 + lg * 4 + (lane & 3);
        if (px < npix) *(int *)(yim + (long)px * a.c + (lr & ~3)) = word;
    }
}

// Blocks of k_dw_mfma below which a launch splits its maps into more bands
// (four per compute unit of MI355X's 256).
constexpr long DWM_BLOCKS = 1024;

// Channel groups per block for a band of `band` output rows: enough tiles per
// wave on small maps (a 7x7 image has four), a whole number of blocks per
// image, the planes within 40 KiB.
static int dw_mfma_lgb(const UQKSpatial *d, int band, int rows_p, int cols_p)
{
    const int tiles = (band * d->ow + 15) / 16, groups = d->oc / 16;
    int lgb = tiles <= 4 ? 2 : tiles <= 16 ? 1 : 0;
    while (lgb && (groups % (1 << lgb) || ((size_t)rows_p * cols_p * 16 << lgb) > 40960)) lgb--;
    return lgb;
}

// Geometry of k_dw_mfma for a launch of `batches` images (0: only whether
// and how the layer fits); returns its dynamic LDS bytes, 0 if the layer
// does not suit it (then the dot4 window kernel runs it).
static size_t dw_mfma_plan(const UQKSpatial *d, DwMArgs *t, uint32_t batches)
{
    const int ks = d->kh, s = d->sh;
    if (!d->dwwin || d->oc % 16 || d->ic != d->oc || d->kh != d->kw || (ks != 3 && ks != 5) || d->sh != d->sw ||
        (s != 1 && s != 2) || d->dh != 1 || d->dw != 1)
        return 0;
    t->cols_p = (d->ow - 1) * s + ks;
    // Output rows per block: the whole map when its padded window fits 40
    // KiB, else the most rows whose window does (bands of the map). A launch
    // of fewer than DWM_BLOCKS blocks takes more, equal bands instead, as
    // many as it needs to reach DWM_BLOCKS while a band stages at most 1.25x
    // its rows' share of the input. Kernel time at batch 64: 56x56x96 5x5 s2
    // 13.4 us in bands of 20 and 8 rows (768 blocks), 11.8 in bands of 10;
    // 112x112x32 3x3 s1 19.4 us in bands of 20 (and 12, 768 blocks), 18.4-19.3
    // in eight of 14; a MobileNetV4-S step (launches of 2304 or more blocks)
    // 0.4240 ms with its 5x5 s2 layer in bands of 20 and 8 rows, 0.4252 in
    // equal bands of 14.
    const size_t row_bytes = (size_t)t->cols_p * 16;
    int band = d->oh;
    if ((size_t)((band - 1) * s + ks) * row_bytes > 40960) band = (int)((40960 / row_bytes - ks) / s + 1);
    if (band < 1 || (size_t)ks * row_bytes > 40960) return 0;
    const auto blocks_of = [&](int b, int nb) {
        return (long)batches * nb * ((d->oc / 16) >> dw_mfma_lgb(d, b, (b - 1) * s + ks, t->cols_p));
    };
    if (d->dw_rows > 0) {
        if (band > d->dw_rows) band = d->dw_rows;
    } else if (batches && blocks_of(band, (d->oh + band - 1) / band) < DWM_BLOCKS) {
        // 5x5 layers (25 taps per staged byte) take up to twice the blocks,
        // and of the band counts passed on the way the last that divides
        // the map exactly wins over a later uneven one: 64 x 56x56x96 5x5
        // s2 (28 output rows) 11.0-11.2 us in bands of 10 (3 bands, the old
        // rule), 9.3 in bands of 6 (5, uneven), 8.7-8.8 in bands of 7 (4);
        // 3x3 layers keep 1,024 blocks (112x112x32 3x3 s1: 18.0 us in bands
        // of 14, 18.6-18.9 in bands of 8 or 7).
        const long target = ks == 5 ? 2 * DWM_BLOCKS : DWM_BLOCKS;
        int nb = (d->oh + band - 1) / band;
        band = (d->oh + nb - 1) / nb;
        int pick = band;
        while (band > 1 && blocks_of(band, nb) < target) {
            const int nb2 = nb + 1, band2 = (d->oh + nb2 - 1) / nb2;
            if (((band2 - 1) * s + ks) * 4 > band2 * s * 5) break;
            nb = nb2;
            band = band2;
            if (d->oh % band == 0 || d->oh % pick != 0) pick = band;
        }
        band = pick;
    }
    t->band = band;
    t->bands = (d->oh + band - 1) / band;
    t->rows_p = (band - 1) * s + ks;
    const int lgb = dw_mfma_lgb(d, band, t->rows_p, t->cols_p);
    t->lgb = lgb;
    t->lwg = 2 - lgb;
    const size_t bytes = (size_t)t->rows_p * t->cols_p * 16 << lgb;
    if (bytes > 40960 || (long)band * d->ow >= 65536) return 0;
    t->m_cols = udiv_magic((unsigned)t->cols_p);
    t->m_ow = udiv_magic((unsigned)d->ow);
    return bytes;
}

static int launch_dw_mfma(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    DwMArgs a;
    const size_t lds = dw_mfma_plan(d, &a, batches);
    if (!lds) return -1;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.wdot = (const int *)d->wdot;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.c = d->oc; a.oh = d->oh; a.ow = d->ow; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.images = (int)batches;
    const unsigned long long blocks = (unsigned long long)batches * a.bands * (d->oc / 16 >> a.lgb);
    if (blocks > 0x7fffffffULL || batches == 0) return blocks ? -1 : 0;
    const int mode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0);
#define UQK_DWM(K, S)                                                                                           \
    do {                                                                                                        \
        switch (mode) {                                                                                         \
        case 0: UQK_LAUNCH((k_dw_mfma<K, S, false, false>), dim3((unsigned)blocks), dim3(256), lds, g_stream, a); break; \
        case 1: UQK_LAUNCH((k_dw_mfma<K, S, true, false>), dim3((unsigned)blocks), dim3(256), lds, g_stream, a); break;  \
        case 2: UQK_LAUNCH((k_dw_mfma<K, S, false, true>), dim3((unsigned)blocks), dim3(256), lds, g_stream, a); break;  \
        default: UQK_LAUNCH((k_dw_mfma<K, S, true, true>), dim3((unsigned)blocks), dim3(256), lds, g_stream, a); break;  \
        }                                                                                                       \
    } while (0)
    if (d->kh == 3 && d->sh == 1) UQK_DWM(3, 1);
    else if (d->kh == 3) UQK_DWM(3, 2);
    else if (d->sh == 1) UQK_DWM(5, 1);
    else UQK_DWM(5, 2);
#undef UQK_DWM
    UQK_LAUNCHED();
    return 0;
}

// Tile geometry for k_dw_tile; returns the dynamic LDS bytes, 0 if unsuited.
static size_t dw_tile_plan(const UQKSpatial *d, uint32_t batches, DwTileArgs *t)
{
    if (d->vec != 16 || d->kh != d->kw || (d->kh != 3 && d->kh != 5) || batches > 65535) return 0;
    const int groups = d->oc / 16;
    int cg = 1;
    for (int c = 4; c >= 1; c--)
        if (groups % c == 0) { cg = c; break; }
    const int npx = 256 / cg;
    const int tw = d->ow < 32 ? d->ow : 32;
    int th = npx / tw;
    if (th < 1) th = 1;
    if (th > d->oh) th = d->oh;
    t->th = th; t->tw = tw; t->cg = cg;
    t->tiles_x = (d->ow + tw - 1) / tw;
    t->ith = (th - 1) * d->sh + (d->kh - 1) * d->dh + 1;
    t->itw = (tw - 1) * d->sw + (d->kw - 1) * d->dw + 1;
    const int G = (d->kh * d->kw + 3) / 4;
    const size_t bytes = (size_t)((t->ith * t->itw * cg * 16 + 15) & ~15) + (size_t)G * cg * 16 * 4 + (size_t)cg * 16 * 32;
    return bytes <= 65536 ? bytes : 0;
}

static int launch_dw_tile(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    DwTileArgs a;
    const size_t lds = dw_tile_plan(d, batches, &a);
    if (!lds) return -1;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.wdot = (const int *)d->wdot;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.c = d->oc; a.oh = d->oh; a.ow = d->ow;
    a.sh = d->sh; a.sw = d->sw; a.dh = d->dh; a.dw = d->dw; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi; a.corr = d->corr;
    const int tiles_y = (d->oh + a.th - 1) / a.th;
    dim3 grid((unsigned)(tiles_y * a.tiles_x), (unsigned)(d->oc / (16 * a.cg)), batches);
    if (d->kh == 3) UQK_LAUNCH(k_dw_tile<3>, grid, dim3(256), lds, g_stream, a);
    else UQK_LAUNCH(k_dw_tile<5>, grid, dim3(256), lds, g_stream, a);
    UQK_LAUNCHED();
    return 0;
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
    a.corr = d->corr;
    const int vec = d->vec;
    a.groups = d->oc / vec;
    a.total = (long)batches * a.ohw * a.groups;
    if (a.total <= 0) return 0;
    dim3 grid((unsigned)((a.total + 255) / 256));
    const int ks = d->kh == d->kw && (d->kh == 3 || d->kh == 5) ? d->kh : 0;
#define UQK_WIN(V, P, K) UQK_LAUNCH((k_window<V, P, K>), grid, dim3(256), 0, g_stream, a)
#define UQK_WIN_KS(V, P) do { if (ks == 3) UQK_WIN(V, P, 3); else if (ks == 5) UQK_WIN(V, P, 5); else UQK_WIN(V, P, 0); } while (0)
    if (pool) {
        if (vec == 16) UQK_WIN_KS(16, true);
        else if (vec == 4) UQK_WIN_KS(4, true);
        else UQK_WIN_KS(1, true);
    } else {
        if (vec == 16) UQK_WIN_KS(16, false);
        else if (vec == 4) UQK_WIN_KS(4, false);
        else UQK_WIN_KS(1, false);
    }
#undef UQK_WIN_KS
#undef UQK_WIN
    UQK_LAUNCHED();
    return 0;
}

extern "C" int uqk_depthwise(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    if (!batches) return 0;
    if (d->dwwin) {
        // The band kernel by default for 3x3 stride 2 only (29.7 -> 19.8 us
        // at 64 x 112x112x64): the matrix-core window kernel measured faster
        // for 5x5 (12.8 / 14.2 against 15.2 / 17.7 us) and level for 3x3
        // stride 1.
        if (d->dwb[0] > 0 && (d->dwk == 0 || (d->dwk < 0 && d->kh == 3 && d->sh == 2)))
            return uqk_dw_band(d, x, y, batches);
        DwMArgs t;
        if (d->dwk != 2 && dw_mfma_plan(d, &t, 0)) return launch_dw_mfma(d, x, y, batches) < 0 ? (int)hipErrorInvalidValue : 0;
        return launch_dw_win(d, x, y, batches) < 0 ? (int)hipErrorInvalidValue : 0;
    }
    const int rc = launch_dw_tile(d, x, y, batches);
    if (rc >= 0) return rc;
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
    UQK_LAUNCH(k_add, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g_stream,
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

// Four channels per thread (one dword per pixel) when C % 4 == 0; the pixel
// loop is unrolled so that several loads are in flight.
__global__ __launch_bounds__(256) void k_mean4(const int8_t *x, int8_t *y, uint32_t batches, uint32_t pixels,
                                                uint32_t channels, int xz, int yz, int m, int s)
{
    const uint32_t groups = channels >> 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)batches * groups) return;
    const uint32_t n = (uint32_t)(idx / groups), g = (uint32_t)(idx - (uint64_t)n * groups);
    const int8_t *p = x + (uint64_t)n * pixels * channels + 4 * g;
    int sum[4] = {0, 0, 0, 0};
#pragma unroll 8
    for (uint32_t q = 0; q < pixels; q++) {
        const int w = *(const int *)(p + (uint64_t)q * channels);
#pragma unroll
        for (int j = 0; j < 4; j++) sum[j] += sbyte(w, j);
    }
    int v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = min(max(uq_scale(sum[j] - (int)pixels * xz, m, s) + yz, -128), 127);
    *(int *)(y + (uint64_t)n * channels + 4 * g) = pack4(v[0], v[1], v[2], v[3]);
}

extern "C" int uqk_mean(const void *x, void *y, uint32_t batches, uint32_t pixels, uint32_t channels,
                        int32_t xz, int32_t yz, int32_t m, int32_t shift)
{
    if (channels % 4 == 0) {
        const uint64_t total = (uint64_t)batches * (channels / 4);
        if (!total) return 0;
        UQK_LAUNCH(k_mean4, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g_stream,
                           (const int8_t *)x, (int8_t *)y, batches, pixels, channels, xz, yz, m, shift);
        UQK_LAUNCHED();
        return 0;
    }
    const uint64_t total = (uint64_t)batches * channels;
    if (!total) return 0;
    UQK_LAUNCH(k_mean, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g_stream,
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
    UQK_LAUNCH(k_lut, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g_stream,
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
        UQK_LAUNCH(k_resize<16>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
    else if (vec == 4)
        UQK_LAUNCH(k_resize<4>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
    else
        UQK_LAUNCH(k_resize<1>, grid, dim3(256), 0, g_stream, (const int8_t *)x, (int8_t *)y, total, groups, oh, ow, c, in_stride, (const uint32_t *)offsets);
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
    UQK_LAUNCH(k_window4, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g_stream,
                       (const int8_t *)x, (int8_t *)y, total, g, fill, in_bytes, out_bytes);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Row copies: destination row r (pitch dp) = row r of source 1 (w1 bytes at
// pitch s1) followed by row r of source 2 (w2 bytes at pitch s2, w2 may be
// 0). Concatenation (code 20), packing (19) and channel slices (26) are all
// this pattern. V-byte chunks (16, 4 or 1: whatever every pointer, pitch and
// width allows), one per thread; chunk q -> (row, chunk) by a 64-bit
// multiply-high, exact for q < 2^32.
// ---------------------------------------------------------------------------
struct Rows2 {
    int8_t *y;
    const int8_t *a, *b;
    uint64_t dp, s1, s2;       // pitches in bytes
    uint32_t c1, cpr;          // chunks of source 1 per row, chunks per destination row
    uint64_t magic;            // ceil(2^64 / cpr), 0 when cpr == 1
    uint64_t total;            // chunks
};

template <int V>
__global__ __launch_bounds__(256) void k_rows2(Rows2 g)
{
    typedef typename std::conditional<V == 16, v4i, typename std::conditional<V == 4, int, int8_t>::type>::type T;
    const uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= g.total) return;
    const uint64_t row = g.cpr == 1 ? q : __umul64hi(q, g.magic);
    const uint32_t c = (uint32_t)(q - row * g.cpr);
    T v;
    if (c < g.c1) v = *(const T *)(g.a + row * g.s1 + (uint64_t)c * V);
    else v = *(const T *)(g.b + row * g.s2 + (uint64_t)(c - g.c1) * V);
    *(T *)(g.y + row * g.dp + (uint64_t)c * V) = v;
}

extern "C" int uqk_rows2(void *y, uint64_t dp, const void *a, uint64_t s1, uint64_t w1, const void *b, uint64_t s2,
                         uint64_t w2, uint64_t rows)
{
    if (!rows || !(w1 + w2)) return 0;
    const uint64_t bits = (uint64_t)(uintptr_t)y | dp | (uint64_t)(uintptr_t)a | s1 | w1 |
                          (w2 ? ((uint64_t)(uintptr_t)b | s2 | w2) : 0);
    const int V = (bits & 15) == 0 ? 16 : (bits & 3) == 0 ? 4 : 1;
    Rows2 g;
    g.y = (int8_t *)y; g.a = (const int8_t *)a; g.b = (const int8_t *)b;
    g.dp = dp; g.s1 = s1; g.s2 = s2;
    g.c1 = (uint32_t)(w1 / V);
    g.cpr = (uint32_t)((w1 + w2) / V);
    g.magic = g.cpr == 1 ? 0 : ~0ULL / g.cpr + 1;
    g.total = rows * g.cpr;
    if (g.total >> 32) return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((g.total + 255) / 256));
    if (V == 16) UQK_LAUNCH(k_rows2<16>, grid, dim3(256), 0, g_stream, g);
    else if (V == 4) UQK_LAUNCH(k_rows2<4>, grid, dim3(256), 0, g_stream, g);
    else UQK_LAUNCH(k_rows2<1>, grid, dim3(256), 0, g_stream, g);
    UQK_LAUNCHED();
    return 0;
}

// Row gather with tables: the fused form of a concat along the last axis
// (code 20) of table lookups (code 22) of channel slices (code 26), such as
// YOLO's split -> SiLU tables -> concat chains, and of a pack of several
// outputs (code 19). Destination row r is the concatenation of up to
// UQK_GATHER_MAX segments; segment s copies `width` bytes of row r of its own
// source (any pitch) through its own 256-entry table or unchanged. Chunks of
// V bytes, one per thread, as k_rows2; the tables sit in LDS.
struct Gather {
    int8_t *y;
    uint64_t dp;
    const int8_t *src[UQK_GATHER_MAX];
    uint64_t stride[UQK_GATHER_MAX];
    const uint8_t *lut[UQK_GATHER_MAX];
    uint32_t flip[UQK_GATHER_MAX];
    uint32_t c0[UQK_GATHER_MAX + 1];   // segment s covers chunks [c0[s], c0[s + 1]) of a row
    uint32_t n, cpr;
    uint64_t magic;            // ceil(2^64 / cpr), 0 when cpr == 1
    uint64_t total;
};

template <int V>
__global__ __launch_bounds__(256) void k_gather(Gather g)
{
    typedef typename std::conditional<V == 16, v4i, typename std::conditional<V == 4, int, int8_t>::type>::type T;
    __shared__ uint8_t tab[UQK_GATHER_MAX][256];
    for (uint32_t s = 0; s < g.n; s++)
        if (g.lut[s]) tab[s][threadIdx.x] = g.lut[s][threadIdx.x ^ g.flip[s]];
    __syncthreads();
    const uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= g.total) return;
    const uint64_t row = g.cpr == 1 ? q : __umul64hi(q, g.magic);
    const uint32_t c = (uint32_t)(q - row * g.cpr);
    uint32_t s = 0;
    while (s + 1 < g.n && c >= g.c0[s + 1]) s++;
    T v = *(const T *)(g.src[s] + row * g.stride[s] + (uint64_t)(c - g.c0[s]) * V);
    if (g.lut[s]) {
        int w[V >= 4 ? V / 4 : 1];
        __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
        for (int k = 0; k < (V >= 4 ? V / 4 : 1); k++) {
            int word = 0;
#pragma unroll
            for (int j = 0; j < (V >= 4 ? 4 : 1); j++) word |= (int)tab[s][(w[k] >> (8 * j)) & 0xff] << (8 * j);
            w[k] = word;
        }
        __builtin_memcpy(&v, w, sizeof(T));
    }
    *(T *)(g.y + row * g.dp + (uint64_t)c * V) = v;
}

static uint64_t g_gather_launches;

// Launches of the row gather since the library was loaded (a test hook; not
// part of the plan ABI).
extern "C" uint64_t uqk_gather_launches(void) { return g_gather_launches; }

extern "C" int uqk_gather(void *y, uint64_t dp, const UQKSeg *segs, uint32_t n, uint64_t rows)
{
    if (n < 1 || n > UQK_GATHER_MAX) return (int)hipErrorInvalidValue;
    uint64_t bits = (uint64_t)(uintptr_t)y | dp, width = 0;
    for (uint32_t s = 0; s < n; s++) {
        bits |= (uint64_t)(uintptr_t)segs[s].src | segs[s].stride | segs[s].width;
        width += segs[s].width;
    }
    if (!rows || !width) return 0;
    const int V = (bits & 15) == 0 ? 16 : (bits & 3) == 0 ? 4 : 1;
    Gather g = {};
    g.y = (int8_t *)y;
    g.dp = dp;
    g.n = n;
    uint32_t at = 0;
    for (uint32_t s = 0; s < UQK_GATHER_MAX; s++) {
        g.c0[s] = at;
        if (s < n) {
            g.src[s] = (const int8_t *)segs[s].src;
            g.stride[s] = segs[s].stride;
            g.lut[s] = (const uint8_t *)segs[s].lut;
            g.flip[s] = segs[s].flip & 0xff;
            at += segs[s].width / V;
        }
    }
    g.c0[UQK_GATHER_MAX] = at;
    g.cpr = at;
    g.magic = g.cpr == 1 ? 0 : ~0ULL / g.cpr + 1;
    g.total = rows * g.cpr;
    if (g.total >> 32) return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((g.total + 255) / 256));
    if (V == 16) UQK_LAUNCH(k_gather<16>, grid, dim3(256), 0, g_stream, g);
    else if (V == 4) UQK_LAUNCH(k_gather<4>, grid, dim3(256), 0, g_stream, g);
    else UQK_LAUNCH(k_gather<1>, grid, dim3(256), 0, g_stream, g);
    UQK_LAUNCHED();
    g_gather_launches++;
    return 0;
}

// ---------------------------------------------------------------------------
// Permutation (code 10, graph.c:374-390) of rank <= 4 tensors, per image:
// out[i0,i1,i2,i3] = in[sum_d i_d * src_stride[d]], elements of 1 or 4 bytes.
// ---------------------------------------------------------------------------
struct Perm4 {
    uint32_t out[4];
    uint32_t src_stride[4];
};

template <typename T>
__global__ __launch_bounds__(256) void k_permute(const T *x, T *y, uint64_t total, uint32_t count, Perm4 g)
{
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const uint64_t img = idx / count;
    uint32_t r = (uint32_t)(idx - img * count), src = 0;
#pragma unroll
    for (int d = 3; d >= 0; d--) {
        const uint32_t o = r % g.out[d];
        r /= g.out[d];
        src += o * g.src_stride[d];
    }
    y[idx] = x[img * count + src];
}

extern "C" int uqk_permute(const void *x, void *y, uint32_t images, uint32_t rank, const uint32_t in_dims[4],
                           const uint32_t perm[4], uint32_t elem_bytes)
{
    Perm4 g;
    uint32_t stride[4] = {1, 1, 1, 1}, acc = 1, count = 1;
    for (int d = (int)rank - 1; d >= 0; d--) {
        stride[d] = acc;
        acc *= in_dims[d];
    }
    // Leading unit dimensions pad the permutation to rank 4.
    const uint32_t lead = 4 - rank;
    for (uint32_t d = 0; d < 4; d++) {
        g.out[d] = d < lead ? 1 : in_dims[perm[d - lead]];
        g.src_stride[d] = d < lead ? 0 : stride[perm[d - lead]];
        count *= g.out[d];
    }
    const uint64_t total = (uint64_t)count * images;
    if (!total) return 0;
    dim3 grid((unsigned)((total + 255) / 256));
    if (elem_bytes == 4)
        UQK_LAUNCH(k_permute<uint32_t>, grid, dim3(256), 0, g_stream, (const uint32_t *)x, (uint32_t *)y, total, count, g);
    else
        UQK_LAUNCH(k_permute<uint8_t>, grid, dim3(256), 0, g_stream, (const uint8_t *)x, (uint8_t *)y, total, count, g);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Elementwise product (uq_mul, qnn.c:111-116), 16 bytes per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_mul(const int8_t *a, const int8_t *b, int8_t *y, uint64_t count,
                                              int az, int bz, int yz, int m, int s, int lo, int hi)
{
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
                const int prod = (sbyte(va[q], j) - az) * (sbyte(vb[q], j) - bz);
                const int v = min(max(uq_scale(prod, m, s) + yz, lo), hi);
                word |= (v & 0xff) << (8 * j);
            }
            w[q] = word;
        }
        *(v4i *)(y + i0) = (v4i){w[0], w[1], w[2], w[3]};
    } else {
        for (uint64_t i = i0; i < count; i++) {
            const int prod = ((int)a[i] - az) * ((int)b[i] - bz);
            y[i] = (int8_t)min(max(uq_scale(prod, m, s) + yz, lo), hi);
        }
    }
}

extern "C" int uqk_mul(const void *a, const void *b, void *y, uint64_t count, const int32_t q[7])
{
    if (!count) return 0;
    const uint64_t threads = (count + 15) / 16;
    UQK_LAUNCH(k_mul, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g_stream,
                       (const int8_t *)a, (const int8_t *)b, (int8_t *)y, count, q[0], q[1], q[2], q[3], q[4], q[5], q[6]);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Batched int8 matmul (uq_bmm, qnn.c:117-153): z[h][r][c] =
// clamp(scale(sum_t (A[h][r][t] - az) * (B[h][t][c] - bz)) + yz). The sum is
// formed exactly in int32 (the loader bounds k * 255^2 * 2^max(s,0)).
// One 256-thread block per 32x32 output tile; K in slices of 32 staged in LDS
// as zero-point-shifted ints; each thread owns 4 rows of one column.
// ---------------------------------------------------------------------------
#define BMM_T 32
__global__ __launch_bounds__(256) void k_bmm(const int8_t *A, const int8_t *B, int8_t *Z, uint32_t m, uint32_t n,
                                              uint32_t k, uint32_t tiles_m, uint32_t tiles_n, uint32_t batches,
                                              uint64_t b_image_stride, int ta, int tb, int az, int bz, int yz,
                                              int mq, int s)
{
    __shared__ int As[BMM_T][BMM_T + 1], Bs[BMM_T][BMM_T + 1];
    uint32_t blk = blockIdx.x;
    const uint32_t tn = blk % tiles_n;
    blk /= tiles_n;
    const uint32_t tm = blk % tiles_m;
    const uint32_t mat = blk / tiles_m;           // image * batches + h
    const uint32_t img = mat / batches, h = mat - img * batches;
    const int8_t *a = A + (uint64_t)mat * m * k;
    const int8_t *b = B + img * b_image_stride + (uint64_t)h * k * n;
    const uint32_t row0 = tm * BMM_T, col0 = tn * BMM_T;
    const uint32_t tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
    int acc[4] = {0, 0, 0, 0};
    for (uint32_t k0 = 0; k0 < k; k0 += BMM_T) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t e = tid + 256 * j, hi = e >> 5, lo = e & 31;
            // A tile element (r, t): lanes walk the contiguous axis in memory.
            const uint32_t ra = ta ? lo : hi, ka = ta ? hi : lo;
            const uint32_t r = row0 + ra, t = k0 + ka;
            As[ra][ka] = (r < m && t < k) ? (int)a[ta ? (uint64_t)t * m + r : (uint64_t)r * k + t] - az : 0;
            const uint32_t tb_ = tb ? lo : hi, cb = tb ? hi : lo;
            const uint32_t c = col0 + cb, t2 = k0 + tb_;
            Bs[tb_][cb] = (c < n && t2 < k) ? (int)b[tb ? (uint64_t)c * k + t2 : (uint64_t)t2 * n + c] - bz : 0;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < BMM_T; kk++) {
            const int bv = Bs[kk][tx];
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] += As[ty * 4 + i][kk] * bv;
        }
        __syncthreads();
    }
    const uint32_t c = col0 + tx;
    if (c >= n) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t r = row0 + ty * 4 + i;
        if (r < m) Z[((uint64_t)mat * m + r) * n + c] = (int8_t)min(max(uq_scale(acc[i], mq, s) + yz, -128), 127);
    }
}

extern "C" int uqk_bmm(const void *a, const void *b, void *z, uint32_t images, uint32_t batches, uint32_t m,
                       uint32_t n, uint32_t k, const int32_t q[7])
{
    const uint32_t tiles_m = (m + BMM_T - 1) / BMM_T, tiles_n = (n + BMM_T - 1) / BMM_T;
    const uint64_t blocks = (uint64_t)tiles_m * tiles_n * batches * images;
    if (!blocks) return 0;
    if (blocks > 0x7fffffffULL) return (int)hipErrorInvalidValue;
    const uint64_t b_stride = (uint64_t)batches * k * n;
    UQK_LAUNCH(k_bmm, dim3((unsigned)blocks), dim3(256), 0, g_stream, (const int8_t *)a, (const int8_t *)b,
                       (int8_t *)z, m, n, k, tiles_m, tiles_n, batches, b_stride, q[5], q[6], q[0], q[1], q[2], q[3], q[4]);
    UQK_LAUNCHED();
    return 0;
}

// ---------------------------------------------------------------------------
// Exact int8 softmax (uq_softmax_exact, qnn.c:87-107): one wave per row.
// Row max and the Q12 sum of table exponentials are wave reductions; every
// lane then forms the same fixed-point reciprocal (three Newton-Raphson steps
// on the sum normalised to [1, 2)) and writes its own elements.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int high_mul(int a, int b)
{
    return (int)(((long long)a * (long long)b + (1LL << 30)) >> 31);
}

__global__ __launch_bounds__(256) void k_softmax(const int8_t *x, int8_t *y, uint64_t rows, uint32_t width,
                                                  const int *table)
{
    __shared__ int lut[256];
    lut[threadIdx.x] = table[threadIdx.x];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int8_t *src = x + row * width;
    int mx = -128;
    for (uint32_t j = lane; j < width; j += 64) mx = max(mx, (int)src[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
    unsigned sum = 0;
    for (uint32_t j = lane; j < width; j += 64) sum += ((unsigned)lut[mx - (int)src[j]] + 2048u) >> 12;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += (unsigned)__shfl_xor((int)sum, off, 64);
    const unsigned lead = (unsigned)__clz((int)sum), exponent = 35 - lead;
    const unsigned frac = (sum << lead) - 0x80000000u;
    const int half = (int)(((unsigned long long)frac + 0x80000000ull) >> 1);
    int r = 1515870810 + high_mul(half, -1010580540);
#pragma unroll
    for (int it = 0; it < 3; it++) {
        const int err = 536870912 - high_mul(half, r);
        r += high_mul(r, err) * 4;
    }
    const long long r2 = (long long)r * 2;
    r = r2 > 2147483647LL ? 2147483647 : (int)r2;
    int8_t *dst = y + row * width;
    for (uint32_t j = lane; j < width; j += 64) {
        const unsigned v = (unsigned)high_mul(r, lut[mx - (int)src[j]]);
        const unsigned rounded = exponent >= 32 ? 0u : (v + (1u << (exponent - 1))) >> exponent;
        dst[j] = (int8_t)(rounded > 255 ? 127 : (int)rounded - 128);
    }
}

// Table softmax (code 17, qnn.c:1082-1087): one wave per row; the 64-bit sum
// of Q24 table exponentials is a wave reduction, each element one exact
// 64-bit rounded division.
__global__ __launch_bounds__(256) void k_softmax_table(const int8_t *x, int8_t *y, uint64_t rows, uint32_t width,
                                                        const int *table, int lo, int hi)
{
    __shared__ int lut[256];
    lut[threadIdx.x] = table[threadIdx.x];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int8_t *src = x + row * width;
    int mx = -128;
    for (uint32_t j = lane; j < width; j += 64) mx = max(mx, (int)src[j]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
    unsigned long long sum = 0;
    for (uint32_t j = lane; j < width; j += 64) sum += (unsigned)lut[mx - (int)src[j]];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned lo32 = __shfl_xor((unsigned)sum, off, 64), hi32 = __shfl_xor((unsigned)(sum >> 32), off, 64);
        sum += ((unsigned long long)hi32 << 32) | lo32;
    }
    const unsigned long long half = sum / 2;
    int8_t *dst = y + row * width;
    for (uint32_t j = lane; j < width; j += 64) {
        const unsigned long long v = (unsigned long long)(unsigned)lut[mx - (int)src[j]] * 256ull;
        const int r = (int)((v + half) / sum) - 128;
        dst[j] = (int8_t)min(max(r, lo), hi);
    }
}

extern "C" int uqk_softmax_table(const void *x, void *y, uint64_t rows, uint32_t width, const void *table, int32_t lo,
                                 int32_t hi)
{
    if (!rows) return 0;
    UQK_LAUNCH(k_softmax_table, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, g_stream, (const int8_t *)x,
                       (int8_t *)y, rows, width, (const int *)table, lo, hi);
    UQK_LAUNCHED();
    return 0;
}

extern "C" int uqk_softmax(const void *x, void *y, uint64_t rows, uint32_t width, const void *table)
{
    if (!rows) return 0;
    UQK_LAUNCH(k_softmax, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, g_stream, (const int8_t *)x,
                       (int8_t *)y, rows, width, (const int *)table);
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

// Scratch of the no-allocation entry point (ug_enqueue_device_noalloc in
// graph.c): the intermediate activations of one call, laid out by graph.c.
// Each GPU holds its own copy of the array, at its own address, until the
// process ends. In host code the array's name is only a stand-in for the
// device symbol: its device address comes from hipGetSymbolAddress at init,
// with the device current, and host code uses that address only.
#define UQK_MAX_DEVICES 64
static __device__ __align__(256) uint8_t scratch[UQK_SCRATCH_BYTES];
static void *g_scratch[UQK_MAX_DEVICES];
static int g_device;

extern "C" void *uqk_scratch(size_t *bytes)
{
    if (!g_ready) return nullptr;
    if (bytes) *bytes = UQK_SCRATCH_BYTES;
    return g_scratch[g_device];
}

extern "C" int uqk_init(void)
{
    if (g_ready) return 0;
    int n = 0;
    UQK_TRY(hipGetDeviceCount(&n));
    if (n < 1) return (int)hipErrorNoDevice;
    UQK_TRY(hipGetDevice(&g_device));
    if (g_device < 0 || g_device >= UQK_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    if (!g_scratch[g_device]) {
        void *p = nullptr;
        UQK_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[g_device] = p;
    }
    // All streams at the default priority.
    UQK_TRY(hipStreamCreateWithFlags(&g_main, hipStreamNonBlocking));
    g_stream = g_main;
    UQK_TRY(hipStreamCreateWithFlags(&g_copy[0], hipStreamNonBlocking));
    UQK_TRY(hipStreamCreateWithFlags(&g_copy[1], hipStreamNonBlocking));
    for (int i = 0; i < 8; i++) UQK_TRY(hipEventCreateWithFlags(&g_pipe_ev[i], hipEventDisableTiming));
    for (int i = 0; i < UQK_MAX_SLICES - 1; i++) {
        UQK_TRY(hipStreamCreateWithFlags(&g_side[i], hipStreamNonBlocking));
        UQK_TRY(hipEventCreateWithFlags(&g_join[i], hipEventDisableTiming));
    }
    UQK_TRY(hipEventCreateWithFlags(&g_fork, hipEventDisableTiming));
    g_ready = 1;
    return 0;
}

// A batch split into image slices, one compute stream each: slice 0 on the
// main stream, slice k on side stream k - 1. split_fork orders the side
// streams after everything already queued on the main stream; split_use
// sends the following launches to one slice's stream (and tells the launch
// heuristics how many slices run side by side); split_join makes the main
// stream wait for the side streams, so that later work on it sees the whole
// batch.
extern "C" int uqk_split_fork(int slices)
{
    if (slices < 1 || slices > UQK_MAX_SLICES) return (int)hipErrorInvalidValue;
    UQK_TRY(hipEventRecord(g_fork, g_main));
    for (int k = 0; k < slices - 1; k++) UQK_TRY(hipStreamWaitEvent(g_side[k], g_fork, 0));
    return 0;
}

extern "C" void uqk_split_use(int slice, int slices)
{
    g_stream = slice > 0 ? g_side[slice - 1] : g_main;
    g_live_slices = slices;
}

extern "C" int uqk_split_join(int slices)
{
    g_stream = g_main;
    g_live_slices = 1;
    if (slices < 1 || slices > UQK_MAX_SLICES) return (int)hipErrorInvalidValue;
    for (int k = 0; k < slices - 1; k++) {
        UQK_TRY(hipEventRecord(g_join[k], g_side[k]));
        UQK_TRY(hipStreamWaitEvent(g_main, g_join[k], 0));
    }
    return 0;
}

// Stream ids for the pipelined transfers: 0 compute, 1 host-to-device,
// 2 device-to-host.
static hipStream_t stream_of(int id) { return id == 0 ? g_main : g_copy[id - 1]; }

extern "C" int uqk_copy_on(int stream, void *dst, const void *src, size_t bytes, int to_device)
{
    if (bytes)
        UQK_TRY(hipMemcpyAsync(dst, src, bytes, to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost,
                               stream_of(stream)));
    return 0;
}

extern "C" int uqk_pipe_record(int event, int stream)
{
    if (event < 0 || event >= 8) return (int)hipErrorInvalidValue;
    UQK_TRY(hipEventRecord(g_pipe_ev[event], stream_of(stream)));
    return 0;
}

extern "C" int uqk_pipe_wait(int stream, int event)
{
    if (event < 0 || event >= 8) return (int)hipErrorInvalidValue;
    UQK_TRY(hipStreamWaitEvent(stream_of(stream), g_pipe_ev[event], 0));
    return 0;
}

extern "C" int uqk_sync_all(void)
{
    UQK_TRY(hipStreamSynchronize(g_copy[0]));
    UQK_TRY(hipStreamSynchronize(g_main));
    UQK_TRY(hipStreamSynchronize(g_copy[1]));
    for (int k = 0; k < UQK_MAX_SLICES - 1; k++) UQK_TRY(hipStreamSynchronize(g_side[k]));
    return 0;
}

extern "C" void *uqk_host_alloc(size_t bytes)
{
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 16, hipHostMallocDefault) != hipSuccess) return nullptr;
    return p;
}

extern "C" void uqk_host_free(void *p)
{
    if (p) (void)hipHostFree(p);
}

// Whole-plan replay: capture what the host enqueues on the compute stream
// into a graph, instantiate it, and launch it as one submission.
extern "C" int uqk_capture_begin(void)
{
    UQK_TRY(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

extern "C" int uqk_capture_end(void **exec)
{
    hipGraph_t graph = nullptr;
    hipGraphExec_t e = nullptr;
    UQK_TRY(hipStreamEndCapture(g_stream, &graph));
    const hipError_t rc = hipGraphInstantiate(&e, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (rc != hipSuccess) {
        g_err = (int)rc;
        return (int)rc;
    }
    *exec = (void *)e;
    return 0;
}

extern "C" int uqk_graph_launch(void *exec)
{
    UQK_TRY(hipGraphLaunch((hipGraphExec_t)exec, g_stream));
    return 0;
}

extern "C" void uqk_graph_destroy(void *exec)
{
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
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
    UQK_TRY(hipStreamSynchronize(g_main));
    for (int k = 0; k < UQK_MAX_SLICES - 1; k++) UQK_TRY(hipStreamSynchronize(g_side[k]));
    return 0;
}

extern "C" int uqk_last_error(void) { return g_err; }

extern "C" int uqk_events(uint32_t count)
{
    if (count <= g_nevents) return 0;
    hipEvent_t *e0 = (hipEvent_t *)realloc(g_ev_start, sizeof(hipEvent_t) * count);
    if (!e0) return (int)hipErrorOutOfMemory;
    g_ev_start = e0;
    hipEvent_t *e1 = (hipEvent_t *)realloc(g_ev_stop, sizeof(hipEvent_t) * count);
    if (!e1) return (int)hipErrorOutOfMemory;
    g_ev_stop = e1;
    for (uint32_t i = g_nevents; i < count; i++) {
        UQK_TRY(hipEventCreate(&g_ev_start[i]));
        UQK_TRY(hipEventCreate(&g_ev_stop[i]));
        g_nevents = i + 1;
    }
    return 0;
}

// Time op `index`: its start event is recorded now on the stream and
// re-stamped by the op's first kernel; an op that launches no kernel (only
// copies, or nothing) gets its stop event recorded at uqk_time_end.
extern "C" int uqk_time_begin(uint32_t index)
{
    if (index >= g_nevents) return (int)hipErrorInvalidValue;
    UQK_TRY(hipEventRecord(g_ev_start[index], g_stream));
    g_timing = 1;
    g_timed_op = index;
    g_timed_launches = 0;
    return 0;
}

extern "C" int uqk_time_end(uint32_t index)
{
    g_timing = 0;
    if (index >= g_nevents) return (int)hipErrorInvalidValue;
    if (!g_timed_launches) UQK_TRY(hipEventRecord(g_ev_stop[index], g_stream));
    return 0;
}

extern "C" int uqk_op_ns(uint32_t index, uint64_t *ns)
{
    if (index >= g_nevents) return (int)hipErrorInvalidValue;
    float ms = 0.f;
    UQK_TRY(hipEventElapsedTime(&ms, g_ev_start[index], g_ev_stop[index]));
    *ns = (uint64_t)((double)ms * 1e6 + 0.5);
    return 0;
}
