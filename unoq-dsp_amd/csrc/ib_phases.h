// Phases shared by the fused bottleneck kernels (ib.hip, uib.hip) on gfx950:
// 1x1 GEMM phases over pixel rows in LDS on 32x32 and 16x16 matrix-core
// tiles, and depthwise phases over window planes in LDS on block-diagonal
// matrix-core tiles. A phase spreads its (channel tile, pixel tile) items
// over the workgroup's IB_WAVES waves, a contiguous range per wave, channel
// tile major; every result is requantised with its layer's own record and
// written through a sink or into LDS rows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "uqk_device.h"

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int IB_WAVES = 16;

// Fragments of a wave's weight tile: rows ct*32 + (lane & 31), the 16-byte
// K slice of each 32-byte step chosen by lane >> 5.
template <int MAXK>
__device__ __forceinline__ void ib_load_weights(v4i (&wf)[MAXK], const int8_t *w, int kp, int ks, int ct)
{
    const int lane = threadIdx.x & 63;
    const int8_t *wr = w + (long)(ct * 32 + (lane & 31)) * kp + (lane >> 5) * 16;
#pragma unroll
    for (int s = 0; s < MAXK; s++)
        if (s < ks) wf[s] = *(const v4i *)(wr + s * 32);
}

// This wave's range of (channel tile, pixel tile) items of a 1x1 phase.
__device__ __forceinline__ void ib_items(int ctiles, int P, int &i0, int &i1)
{
    const int wave = threadIdx.x >> 6, items = ctiles * ((P + 31) >> 5);
    i0 = wave * items / IB_WAVES;
    i1 = (wave + 1) * items / IB_WAVES;
}

// A 1x1 GEMM phase over the image's P pixels: pixel tiles of 32 (MFMA rows,
// rows of `src` in LDS with stride ss, clamped to P - 1 past the image) by
// channel tiles of 32 (columns: weights `w`, row stride kp, K = 32 * ks
// bytes). Each wave takes a contiguous range of (channel tile, pixel tile)
// items (ib_items), channel tile major, and reloads its weight fragments
// (wf, of channel tile `loaded`) and its channel's record (from `rec`, in
// LDS or global memory) only when the channel tile changes. `sink(p, c, word)` receives, per lane and for each
// of its four pixel groups, the requantised bytes of channels c .. c + 3 of
// pixel p (p < P only).
template <int MAXK, bool HI, bool CORR, bool LUT, typename Sink>
__device__ __forceinline__ void ib_gemm(v4i (&wf)[MAXK], int &loaded, const int8_t *w, int kp, int ks,
                                        const int8_t *src, int ss, int P, int ctiles, const int4 *rec, int yz,
                                        int lo, int hi, const int8_t *lut, Sink sink)
{
    const int lane = threadIdx.x & 63;
    const int fr = lane & 31, fh = lane >> 5;
    const int ptiles = (P + 31) >> 5;
    int i0, i1;
    ib_items(ctiles, P, i0, i1);
    const int vlo = vgpr(lo), vhi = vgpr(hi);
    Epi e = {};
    int have = -1;
    // (channel tile, pixel tile) of the item, stepped along without divisions.
    int ct = i0 / ptiles, pt = i0 - ct * ptiles;
    for (int item = i0; item < i1; item++, pt = pt + 1 < ptiles ? pt + 1 : 0, ct += pt == 0) {
        if (ct != loaded) {
            ib_load_weights<MAXK>(wf, w, kp, ks, ct);
            loaded = ct;
        }
        if (ct != have) {
            e = load_epi(rec, ct * 32 + fr);
            have = ct;
        }
        const int8_t *sr = src + __mul24(min(pt * 32 + fr, P - 1), ss) + fh * 16;
        v16i acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0;
#pragma unroll
        for (int s = 0; s < MAXK; s++)
            if (s < ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(*(const v4i *)(sr + s * 32), wf[s], acc, 0, 0, 0);
        // acc[4g + i]: pixel pt*32 + 8g + 4fh + i, channel ct*32 + fr.
        const int c = ct * 32 + (fr & ~3);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = conv_requant<HI, CORR>(acc[4 * g + i], e, yz, vlo, vhi);
                if (LUT) v[i] = lut[v[i] + 128];
            }
            const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
            const int p = pt * 32 + 8 * g + 4 * fh + (lane & 3);
            if (p < P) sink(p, c, word);
        }
    }
}

// ib_gemm with the requantisation variant (a wave-uniform mode) and the
// presence of a post table as template arguments.
template <int MAXK, typename Sink>
__device__ __forceinline__ void ib_gemm_mode(int mode, v4i (&wf)[MAXK], int &loaded, const int8_t *w, int kp,
                                             int ks, const int8_t *src, int ss, int P, int ctiles, const int4 *rec,
                                             int yz, int lo, int hi, const int8_t *lut, Sink sink)
{
#define IB_GEMM(H, C, L) ib_gemm<MAXK, H, C, L>(wf, loaded, w, kp, ks, src, ss, P, ctiles, rec, yz, lo, hi, lut, sink)
    switch (mode * 2 + (lut != nullptr)) {
    case 0: IB_GEMM(false, false, false); break;
    case 1: IB_GEMM(false, false, true); break;
    case 2: IB_GEMM(true, false, false); break;
    case 3: IB_GEMM(true, false, true); break;
    case 4: IB_GEMM(false, true, false); break;
    case 5: IB_GEMM(false, true, true); break;
    case 6: IB_GEMM(true, true, false); break;
    default: IB_GEMM(true, true, true); break;
    }
#undef IB_GEMM
}

// The project phase's GEMM, in 16x16 tiles on v_mfma_i32_16x16x64_i8 (finer
// items than 32x32 tiles: a 7x7 map has only two 32-pixel tiles): pixel
// tiles of 16 (rows of `src`, stride ss) by channel tiles of 16 (weights
// `w`, row stride kp, zero past the K bytes, so that the source bytes a K
// tail reads past its rows add nothing), K = 64 * ks bytes. Items as in
// ib_gemm. `sink(p, c, word)`: channels c .. c + 3 of pixel p.
template <int MAXK, bool HI, bool CORR, bool LUT, typename Sink>
__device__ __forceinline__ void ib_gemm16(const int8_t *w, int kp, int ks, const int8_t *src, int ss, int P,
                                          int ctiles, const int4 *rec, int yz, int lo, int hi, const int8_t *lut,
                                          Sink sink)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int ptiles = (P + 15) >> 4, items = ctiles * ptiles;
    const int i0 = wave * items / IB_WAVES, i1 = (wave + 1) * items / IB_WAVES;
    const int vlo = vgpr(lo), vhi = vgpr(hi);
    v4i wf[MAXK];
    Epi e = {};
    int loaded = -1;
    int ct = i0 / ptiles, pt = i0 - ct * ptiles;
    for (int item = i0; item < i1; item++, pt = pt + 1 < ptiles ? pt + 1 : 0, ct += pt == 0) {
        if (ct != loaded) {
            const int8_t *wr = w + (long)(ct * 16 + lr) * kp + lg * 16;
#pragma unroll
            for (int s = 0; s < MAXK; s++)
                if (s < ks) wf[s] = *(const v4i *)(wr + s * 64);
            e = load_epi(rec, ct * 16 + lr);
            loaded = ct;
        }
        const int8_t *sr = src + __mul24(min(pt * 16 + lr, P - 1), ss) + lg * 16;
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < MAXK; s++)
            if (s < ks) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i *)(sr + s * 64), wf[s], acc, 0, 0, 0);
        // acc[i]: pixel pt*16 + 4*lg + i, channel ct*16 + lr.
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = conv_requant<HI, CORR>(acc[i], e, yz, vlo, vhi);
            if (LUT) v[i] = lut[v[i] + 128];
        }
        const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
        const int p = pt * 16 + lg * 4 + (lane & 3);
        if (p < P) sink(p, ct * 16 + (lr & ~3), word);
    }
}

template <int MAXK, typename Sink>
__device__ __forceinline__ void ib_gemm16_mode(int mode, const int8_t *w, int kp, int ks, const int8_t *src, int ss,
                                               int P, int ctiles, const int4 *rec, int yz, int lo, int hi,
                                               const int8_t *lut, Sink sink)
{
#define IB_GEMM(H, C, L) ib_gemm16<MAXK, H, C, L>(w, kp, ks, src, ss, P, ctiles, rec, yz, lo, hi, lut, sink)
    switch (mode * 2 + (lut != nullptr)) {
    case 0: IB_GEMM(false, false, false); break;
    case 1: IB_GEMM(false, false, true); break;
    case 2: IB_GEMM(true, false, false); break;
    case 3: IB_GEMM(true, false, true); break;
    case 4: IB_GEMM(false, true, false); break;
    case 5: IB_GEMM(false, true, true); break;
    case 6: IB_GEMM(true, true, false); break;
    default: IB_GEMM(true, true, true); break;
    }
#undef IB_GEMM
}

// A depthwise phase over window planes in LDS: E holds C / 16 planes of
// `plane` positions of 16 channels (the padded map, `cols` positions a row);
// pos[p] less `corner` is the window's top-left position of output pixel p
// (p < P); the results go to rows of D (stride ds), requantised with the
// records `rec`, zero point yz, clamp [lo, hi] and, with LUT, the post table
// lut. Tap words tw[ky][KS > 4 ? 2 : 1][C] (four taps of a kernel row per
// word).
struct DwPh {
    int P, C, ds, cols, corner, yz, lo, hi;
    const int4 *rec;
    const int8_t *lut;
};

// Depthwise phase (any kernel size): items (16-channel group, 16-pixel
// tile), group major, a contiguous range per wave; per item one
// v_mfma_i32_16x16x64_i8 per four taps; the block-diagonal tap operands
// (from the tap words staged in LDS) and the channel's record are rebuilt
// when the group changes.
template <int KS, bool HI, bool CORR, bool LUT>
__device__ __forceinline__ void ib_dw(const DwPh &a, const int8_t *E, int8_t *D, const int *padoff, const int *tw,
                                      int plane)
{
    constexpr int T = KS * KS, NG = (T + 3) / 4, NWK = KS > 4 ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int tiles = (a.P + 15) >> 4, items = (a.C >> 4) * tiles;
    const int i0 = wave * items / IB_WAVES, i1 = (wave + 1) * items / IB_WAVES;
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    const int corner = a.corner;
    int off[NG];
#pragma unroll
    for (int m = 0; m < NG; m++) {
        const int t = 4 * m + lg, ky = t / KS, kx = t - ky * KS;
        off[m] = t < T ? (ky * a.cols + kx) * 16 : 0;
    }
    v4i B[NG];
    Epi e = {};
    int loaded = -1;
    // (group, tile) of the item, stepped along without divisions; gplane is
    // the group's window plane less the window corner.
    int g = i0 / tiles, t16 = i0 - g * tiles;
    const int8_t *gplane = E;
    for (int item = i0; item < i1; item++, t16 = t16 + 1 < tiles ? t16 + 1 : 0, g += t16 == 0) {
        if (g != loaded) {
            gplane = E + (g * plane - corner) * 16;
#pragma unroll
            for (int m = 0; m < NG; m++) {
                const int t = 4 * m + lg, ky = t / KS, kx = t - ky * KS;
                int wb = 0;
                if (t < T) wb = (tw[(ky * NWK + (kx >> 2)) * a.C + g * 16 + lr] >> (8 * (kx & 3))) & 0xff;
                const int word = wb << (8 * (lr & 3)), q = lr >> 2;
                B[m] = (v4i){q == 0 ? word : 0, q == 1 ? word : 0, q == 2 ? word : 0, q == 3 ? word : 0};
            }
            e = load_epi(a.rec, g * 16 + lr);
            loaded = g;
        }
        const int p = min(t16 * 16 + lr, a.P - 1);
        const int8_t *base = gplane + padoff[p] * 16;
        v4i acc = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < NG; m++)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(const v4i *)(base + off[m]), B[m], acc, 0, 0, 0);
        // acc[i]: pixel t16*16 + 4*lg + i, channel g*16 + lr.
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = conv_requant<HI, CORR>(acc[i], e, a.yz, vlo, vhi);
            if (LUT) v[i] = a.lut[v[i] + 128];
        }
        const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
        const int px = t16 * 16 + lg * 4 + (lane & 3);
        if (px < a.P) *(int *)(D + __mul24(px, a.ds) + g * 16 + (lr & ~3)) = word;
    }
}

// The 3x3 depthwise on 32x32 tiles (v_mfma_i32_32x32x32_i8, one per tap):
// 32 pixels (rows: 16-byte reads of the window planes of the tile's two
// 16-channel groups) by 32 channels (columns: block-diagonal, lane (channel
// n, half h) holds w[tap][n] in byte n % 16 of the half that contains n).
// A lane's 16 results share one channel, so one record per lane, and the
// epilogue is the expand's: 4x4 byte transposes into 4-byte writes of D.
// Items (32-channel tile, 32-pixel tile), channel tile major; the taps'
// operands and the record are rebuilt when the channel tile changes.
template <bool HI, bool CORR, bool LUT>
__device__ __forceinline__ void ib_dw3_32(const DwPh &a, const int8_t *E, int8_t *D, const int *padoff,
                                          const int *tw, int plane)
{
    const int lane = threadIdx.x & 63;
    const int fr = lane & 31, fh = lane >> 5;
    const int ptiles = (a.P + 31) >> 5;
    int i0, i1;
    ib_items(a.C >> 5, a.P, i0, i1);
    const int vlo = vgpr(a.lo), vhi = vgpr(a.hi);
    const int corner = a.corner;
    int off[9];
#pragma unroll
    for (int t = 0; t < 9; t++) off[t] = ((t / 3) * a.cols + t % 3) * 16;
    v4i B[9];
    Epi e = {};
    int loaded = -1;
    const int8_t *gplane = E;
    int ct = i0 / ptiles, pt = i0 - ct * ptiles;
    for (int item = i0; item < i1; item++, pt = pt + 1 < ptiles ? pt + 1 : 0, ct += pt == 0) {
        if (ct != loaded) {
            const int c = ct * 32 + fr, q = (fr & 15) >> 2;
            const bool mine = (fr >> 4) == fh;
#pragma unroll
            for (int t = 0; t < 9; t++) {
                const int wb = mine ? (tw[(t / 3) * a.C + c] >> (8 * (t % 3))) & 0xff : 0;
                const int word = wb << (8 * (fr & 3));
                B[t] = (v4i){q == 0 ? word : 0, q == 1 ? word : 0, q == 2 ? word : 0, q == 3 ? word : 0};
            }
            e = load_epi(a.rec, c);
            gplane = E + ((ct * 2 + fh) * plane - corner) * 16;
            loaded = ct;
        }
        const int8_t *base = gplane + padoff[min(pt * 32 + fr, a.P - 1)] * 16;
        v16i acc;
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0;
#pragma unroll
        for (int t = 0; t < 9; t++)
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(*(const v4i *)(base + off[t]), B[t], acc, 0, 0, 0);
        // acc[4g + i]: pixel pt*32 + 8g + 4fh + i, channel ct*32 + fr.
        const int c = ct * 32 + (fr & ~3);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = conv_requant<HI, CORR>(acc[4 * g + i], e, a.yz, vlo, vhi);
                if (LUT) v[i] = a.lut[v[i] + 128];
            }
            const int word = quad_transpose_bytes(pack4(v[0], v[1], v[2], v[3]), lane);
            const int px = pt * 32 + 8 * g + 4 * fh + (lane & 3);
            if (px < a.P) *(int *)(D + __mul24(px, a.ds) + c) = word;
        }
    }
}


// A depthwise phase with the requantisation variant (a wave-uniform mode)
// and the presence of a post table as template arguments: 3x3 on 32x32
// tiles, other sizes on 16x16x64 tiles.
template <int KS>
__device__ __forceinline__ void ib_dw_mode(int mode, const DwPh &g, const int8_t *E, int8_t *D, const int *pos,
                                           const int *tw, int plane)
{
#define IB_DW(H, C, L)                                          \
    do {                                                        \
        if (KS == 3) ib_dw3_32<H, C, L>(g, E, D, pos, tw, plane); \
        else ib_dw<KS, H, C, L>(g, E, D, pos, tw, plane);        \
    } while (0)
    switch (mode * 2 + (g.lut != nullptr)) {
    case 0: IB_DW(false, false, false); break;
    case 1: IB_DW(false, false, true); break;
    case 2: IB_DW(true, false, false); break;
    case 3: IB_DW(true, false, true); break;
    case 4: IB_DW(false, true, false); break;
    case 5: IB_DW(false, true, true); break;
    case 6: IB_DW(true, true, false); break;
    default: IB_DW(true, true, true); break;
    }
#undef IB_DW
}

