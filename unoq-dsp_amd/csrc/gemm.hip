// Large-tile int8 convolution GEMM for gfx950 (code 14 layers whose work is
// matrix-core bound: wide K and many output pixels).
//
// The layer is out[p][c] = requant(sum_k s[p][k] * w[c][k]) over the pixels
// p of the batch (implicit im2col: k = (ky, kx, ic), s = the signed input
// byte, or the input zero point in padding) and the output channels c; the
// reference computes the same sum on unsigned columns (qnn.c:1101-1169,
// gemm.c:592-612), whose +128 offset and K tail the load-time corrected bias
// absorbs (graph.c: prepare_spatial).
//
// Matrix cores: v_mfma_i32_32x32x32_i8, whose measured rate on MI355X is
// about 1.5x that of v_mfma_i32_16x16x64_i8. The weights are the MFMA rows
// (A operand) and the pixels its columns, so a lane's accumulator registers
// 4g .. 4g+3 hold four consecutive channels of one pixel: after
// requantisation two v_permlane32_swap per 32x32 tile give each lane 16
// consecutive channels of one pixel, one 16-byte store, with no LDS round
// trip for the output.
//
// Blocking: a block of NWP x NWC waves computes BP = NWP*WP pixels by
// BC = NWC*WC channels; each wave a WP x WC tile, (WP/32) * (WC/32)
// accumulators of 16 registers. K advances 64 bytes per stage: the block's
// pixel rows and weight rows for the stage (BP*64 + BC*64 bytes) are loaded
// from HBM/L2 with coalesced 16-byte loads into registers, written to one of
// two LDS buffers while the other buffer feeds the matrix cores, one barrier
// per stage. A staged row is 64 bytes as four 16-byte chunks, chunk c stored
// at position c ^ ((row >> 2) & 3): a fragment read (32 consecutive rows,
// one chunk) and a staging write (four rows, four chunks per 16 lanes) both
// touch 16 distinct 16-byte bank groups per 16 lanes. Each wave reads its
// (WP + WC) x 64 bytes per stage from LDS for WP*WC*64 MACs.
//
// Block order is XCD-aware: the hardware deals consecutive block ids to the
// eight XCDs in turn, so block id b is renumbered to put a contiguous range of
// output tiles (pixel tile major, channel tile minor) on each XCD; a pixel
// tile's input rows then come from HBM once per XCD and its channel tiles
// hit that XCD's L2.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include "uqk.h"
#include "uqk_device.h"
#include "uqk_internal.h"

typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;           // [oc_pad][kpad], k = (ky, kx, ic), zero past K
    const int4 *epi;           // 32-byte requantisation records, one per channel
    const uint8_t *lut;        // optional post table
    int M;                     // output pixels of the launch
    int K, kpad, oc, oc_pad;
    int ih, iw, ic, ow, ohw, kw, sh, sw, dh, dw, pt, pl;
    int xz, yz, lo, hi;
    int ctiles, nblocks;       // channel tiles; blocks launched
    int ntiles;                // output tiles of the launch
    int rotate;                // start each block's K walk at a different stage
};

// Position of logical 16-byte chunk c in staged row `row` of KS bytes (and,
// XOR being its own inverse, the logical chunk at position c): 64-byte rows
// as four chunks, c ^ ((row >> 2) & 3); 128-byte rows as eight chunks,
// c ^ ((row >> 1) & 7). Either way a fragment read (32 consecutive rows, one
// chunk) touches 16 distinct 16-byte bank groups per 16 lanes.
template <int KS>
__device__ __forceinline__ int swz(int row, int c)
{
    return KS == 64 ? c ^ ((row >> 2) & 3) : c ^ ((row >> 1) & 7);
}

// Requantisation records of a block's channels in LDS, one array per field.
struct EpiLds {
    int *m, *t, *b, *ls;
    long long *c1, *thr;
};

// Load records of channels c0 .. c0 + n - 1 (channels past OC reuse record
// 0; their outputs are not stored) into the LDS arrays, threads t, t + T, ...
template <int T>
__device__ __forceinline__ void load_records(const EpiLds &r, const int4 *epi, int c0, int n, int oc, int t)
{
    for (int j = t; j < n; j += T) {
        const int c = c0 + j < oc ? c0 + j : 0;
        const int4 e0 = epi[2 * c], e1 = epi[2 * c + 1];
        r.b[j] = e0.x; r.m[j] = e0.y; r.ls[j] = e0.z; r.t[j] = e0.w;
        r.c1[j] = (long long)(((unsigned long long)(unsigned)e1.y << 32) | (unsigned)e1.x);
        r.thr[j] = (long long)(((unsigned long long)(unsigned)e1.w << 32) | (unsigned)e1.z);
    }
}

// Requantise and store a wave's tile: lane (fr, fh) holds, in registers
// 4g .. 4g+3 of accumulator (ct, pt), channels ct*32 + 8g + 4fh + 0..3 of
// pixel pt*32 + fr (channels local to the block from cb, global from cg;
// pixel rows of the output from prow). Four channel words per pixel go
// through two v_permlane32_swap so that each lane stores 16 consecutive
// channels of one pixel. Rows at or past plimit and channels at or past OC
// (a multiple of 16) are not stored.
template <int PT, int CT, bool HI, bool CORR>
__device__ __forceinline__ void gemm_store(const v16i (&acc)[CT][PT], const EpiLds &r, const int8_t *lut_s, bool lut,
                                           int8_t *y, int oc, int yz, int lo, int hi, int cb, int cg, long prow,
                                           long plimit, int lane)
{
    const int fr = lane & 31, fh = lane >> 5;
    const int vlo = vgpr(lo), vhi = vgpr(hi);
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        int words[PT][4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int c = cb + ct * 32 + 8 * g + 4 * fh;
            const int4 m4 = *(const int4 *)&r.m[c], t4 = *(const int4 *)&r.t[c];
            const int4 b4 = *(const int4 *)&r.b[c], l4 = *(const int4 *)&r.ls[c];
            Epi e[4];
            const int mv[4] = {m4.x, m4.y, m4.z, m4.w}, tv[4] = {t4.x, t4.y, t4.z, t4.w};
            const int bv[4] = {b4.x, b4.y, b4.z, b4.w}, lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                e[i].m = mv[i];
                e[i].T = tv[i];
                e[i].bias = bv[i];
                e[i].ls = lv[i];
                e[i].c1 = r.c1[c + i];
                e[i].cthr = CORR ? r.thr[c + i] : 0;
            }
#pragma unroll
            for (int pt = 0; pt < PT; pt++) {
                int v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = conv_requant<HI, CORR>(acc[ct][pt][4 * g + i], e[i], yz, vlo, vhi);
                if (lut) {
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = lut_s[v[i] + 128];
                }
                words[pt][g] = pack4(v[0], v[1], v[2], v[3]);
            }
        }
        const int cgl = cg + ct * 32 + 16 * fh;
#pragma unroll
        for (int pt = 0; pt < PT; pt++) {
            const auto s02 = __builtin_amdgcn_permlane32_swap(words[pt][0], words[pt][2], false, false);
            const auto s13 = __builtin_amdgcn_permlane32_swap(words[pt][1], words[pt][3], false, false);
            const long p = prow + pt * 32 + fr;
            if (p < plimit && cgl < oc)
                *(v4i *)(y + p * oc + cgl) = (v4i){(int)s02[0], (int)s02[1], (int)s13[0], (int)s13[1]};
        }
    }
}

// IM2COL: the pixel operand gathered per stage from the input through the
// (ky, kx, ic) decomposition of k (IC % KS == 0, so a stage lies inside one
// tap); otherwise pointwise rows of IC bytes. NS: stages in the LDS ring;
// KS: K bytes per stage (64, or 128 so that every staged row is one whole
// 128-byte line, which halves the L2 requests per byte).
//
// TPB: output tiles per block. With TPB = 2 a block takes tiles 2b and 2b + 1
// (b its XCD-aware rank): once the first tile's last stage has been read,
// the second tile's first stage is issued before the first tile's epilogue,
// so that its latency and the block's start-up (records, address set-up)
// are paid once per two tiles.
template <int WP, int WC, int NWP, int NWC, int NS, int KS, bool IM2COL, int EMODE, int TPB>
__global__ __launch_bounds__(64 * NWP * NWC) void k_gemm(GemmArgs a)
{
    constexpr int NW = NWP * NWC, T = 64 * NW;
    constexpr int BP = WP * NWP, BC = WC * NWC;
    constexpr int PT = WP / 32, CT = WC / 32;
    constexpr int CPR = KS / 16, RPI = 1024 / KS;       // chunks per row, rows per staging instruction
    constexpr int NIX = BP / (RPI * NW), NIW = BC / (RPI * NW), NI = NIX + NIW;
    constexpr int STAGE = (BP + BC) * KS;
    constexpr bool HI = (EMODE & 1) != 0, CORR = (EMODE & 2) != 0;
    static_assert(KS == 64 || KS == 128, "stage depth");
    static_assert(NIX * RPI * NW == BP && NIW * RPI * NW == BC && NW % 2 == 0, "whole staging instructions per wave");
    static_assert(NS >= 2 && NS <= 6 && (NS - 1) * NI < 64, "stage ring");

    __shared__ __attribute__((aligned(1024))) int8_t ring[NS * STAGE];
    __shared__ __attribute__((aligned(16))) int r_m[TPB][BC], r_t[TPB][BC], r_b[TPB][BC], r_ls[TPB][BC];
    __shared__ __attribute__((aligned(16))) long long r_c1[TPB][BC], r_thr[TPB][BC];
    __shared__ __attribute__((aligned(16))) int8_t lut_s[256];

    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wp = wave % NWP, wc = wave / NWP;
    const int nb = a.nblocks, q8 = nb >> 3, r8 = nb & 7, xcd = (int)(blockIdx.x & 7);
    const int bid = xcd * q8 + min(xcd, r8) + (int)(blockIdx.x >> 3);
    // This block's tiles: bid * TPB + j for j < ntile.
    const int ntile = min(TPB, a.ntiles - bid * TPB);

    auto recs = [&](int j) { return EpiLds{r_m[j], r_t[j], r_b[j], r_ls[j], r_c1[j], r_thr[j]}; };
#pragma unroll
    for (int j = 0; j < TPB; j++)
        if (j < ntile) load_records<T>(recs(j), a.epi, (bid * TPB + j) % a.ctiles * BC, BC, a.oc, t);
    if (a.lut && t < 64) ((int *)lut_s)[t] = ((const int *)a.lut)[t];
    int lid = bid * TPB, p0 = 0, c0 = 0;

    // Staging: a stage is BP pixel rows then BC weight rows of KS bytes.
    // Wave w's instruction i fills stage bytes [j * 1024, j * 1024 + 1024)
    // with j = w + i * NW (instructions 0 .. NIX-1 pixel rows, the rest
    // weight rows); lane l writes 16 bytes at l * 16, i.e. row
    // j * RPI + l / CPR, physical chunk l % CPR, so it loads the logical
    // chunk at that position. The swizzle term depends on row bits that
    // i * NW * RPI (a multiple of 16) leaves alone, so each thread loads the
    // same logical chunk cq of all its rows.
    const int cq = swz<KS>(wave * RPI + lane / CPR, lane % CPR);
    const int8_t *pad = (const int8_t *)g_pad_rows.b + (a.xz & 0xff) * 16, *zero = (const int8_t *)g_pad_rows.b;
    const int8_t *xsrc[NIX];
    int iy0[NIX], ix0[NIX];
    const int8_t *wsrc[NIW];
    // The block's walk over the S stages of K starts at stage `rot` (the sum
    // does not depend on the order): blocks that run side by side then read
    // different weight and pixel lines at any one time instead of all
    // requesting the same lines of L2 together.
    const int S = (a.kpad + KS - 1) / KS;
    int rot = 0;
    // Tile `tile`'s origin and its staging sources.
    auto setup = [&](int tile) {
        lid = tile;
        p0 = lid / a.ctiles * BP;
        c0 = lid % a.ctiles * BC;
        rot = a.rotate ? lid % S : 0;
#pragma unroll
        for (int i = 0; i < NIX; i++) {
            const int p = min(p0 + (wave + i * NW) * RPI + lane / CPR, a.M - 1);
            if (IM2COL) {
                const int n = p / a.ohw, rem = p - n * a.ohw, oy = rem / a.ow, ox = rem - oy * a.ow;
                iy0[i] = oy * a.sh - a.pt;
                ix0[i] = ox * a.sw - a.pl;
                xsrc[i] = a.x + (long)n * a.ih * a.iw * a.ic + ((long)iy0[i] * a.iw + ix0[i]) * a.ic + cq * 16;
            } else {
                iy0[i] = ix0[i] = 0;
                xsrc[i] = a.x + (long)p * a.ic + cq * 16;
            }
        }
#pragma unroll
        for (int i = 0; i < NIW; i++)
            wsrc[i] = a.w + (long)min(c0 + (wave + (NIX + i) * NW) * RPI - BP + lane / CPR, a.oc_pad - 1) * a.kpad +
                      cq * 16;
    };
    setup(bid * TPB);
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)ring;
    auto issue = [&](int s, int buf) {
        const int ks = s + rot < S ? s + rot : s + rot - S;
        const int k0 = ks * KS;
        const uint32_t dst = ring_lds + buf * STAGE + wave * 1024;
        if (IM2COL) {
            const int tap = k0 / a.ic, tc = k0 - tap * a.ic;
            const int tky = tap / a.kw, tkx = tap - tky * a.kw;
            const int dy = tky * a.dh, dx = tkx * a.dw;
            const long off = ((long)dy * a.iw + dx) * a.ic + tc;
#pragma unroll
            for (int i = 0; i < NIX; i++) {
                const bool in = (unsigned)(iy0[i] + dy) < (unsigned)a.ih && (unsigned)(ix0[i] + dx) < (unsigned)a.iw;
                lds_load16(in ? xsrc[i] + off : pad, dst + i * NW * 1024);
            }
        } else {
            const bool in = k0 + cq * 16 < a.K;
#pragma unroll
            for (int i = 0; i < NIX; i++) lds_load16(in ? xsrc[i] + k0 : pad, dst + i * NW * 1024);
        }
        // Weight chunks past kpad (the last stage of a kpad that is not a
        // multiple of KS) are zero, so the pixel bytes they meet (the
        // zero-point row) add nothing.
        const bool win = k0 + cq * 16 < a.kpad;
#pragma unroll
        for (int i = 0; i < NIW; i++) lds_load16(win ? wsrc[i] + k0 : zero, dst + (NIX + i) * NW * 1024);
    };

    v16i acc[CT][PT];

    // Fragments of one 32-byte K half of a staged stage: lane (fr, fh)
    // takes logical chunk 2h + fh of weight row wc*WC + ct*32 + fr and of
    // pixel row wp*WP + pt*32 + fr.
    const int fr = lane & 31, fh = lane >> 5;
    auto read_frags = [&](int buf, int h, v4i (&wf)[CT], v4i (&xf)[PT]) {
        const int8_t *xs = ring + buf * STAGE, *ws = xs + BP * KS;
        const int c = 2 * h + fh;
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const int row = wc * WC + ct * 32 + fr;
            wf[ct] = *(const v4i *)(ws + row * KS + swz<KS>(row, c) * 16);
        }
#pragma unroll
        for (int pt = 0; pt < PT; pt++) {
            const int row = wp * WP + pt * 32 + fr;
            xf[pt] = *(const v4i *)(xs + row * KS + swz<KS>(row, c) * 16);
        }
    };
    auto mfmas = [&](const v4i (&wf)[CT], const v4i (&xf)[PT]) {
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int pt = 0; pt < PT; pt++)
                acc[ct][pt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[ct], xf[pt], acc[ct][pt], 0, 0, 0);
    };
    // Wait until this wave's loads of a stage have landed, `later` stages
    // (0 .. NS-1) having been issued after it.
    auto wait_stage = [&](int later) {
        if (later <= 0) wait_vm<0>();
        else if (later == 1) wait_vm<NI>();
        else if (later == 2) wait_vm<2 * NI>();
        else if (later == 3 || NS <= 4) wait_vm<3 * NI>();
        else if (later == 4 || NS <= 5) wait_vm<(NS > 4 ? 4 : 3) * NI>();
        else wait_vm<(NS > 5 ? 5 : 3) * NI>();
    };

    // Software pipeline over stages s = 0 .. S-1 (NS buffers, stage s in
    // buffer s % NS), each NH = KS / 32 K sub-steps: while the matrix cores
    // work through sub-step h, sub-step h + 1's fragments come from LDS
    // (two fragment sets in turn). Before the last sub-step of stage s the
    // block waits for stage s + 1 (issued NS - 1 stages earlier) and passes
    // a barrier, after which every wave has read all of stage s, so its
    // buffer is refilled with stage s + NS while that sub-step multiplies
    // and stage s + 1's first fragments are read.
    constexpr int NH = KS / 32;
    static_assert(NH % 2 == 0, "fragment sets alternate across stages");
#pragma unroll
    for (int s = 0; s < NS; s++)
        if (s < S) issue(s, s);
    for (int j = 0;;) {
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int pt = 0; pt < PT; pt++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[ct][pt][r] = 0;
    wait_stage(min(NS - 1, S - 1));
    __syncthreads();
    v4i wf[2][CT], xf[2][PT];
    read_frags(0, 0, wf[0], xf[0]);
    // The stages with a successor run in the loop and the last one after it.
    // Every pass through the loop body then ends the same way (barrier, next
    // stage's first fragment reads, last sub-step's multiplies), so the
    // compiler's LDS wait before each multiply covers only that sub-step's
    // own fragments. With the last stage inside the loop, the two ways out
    // of the last sub-step met at the multiplies and the wait there also
    // covered the reads just issued past the barrier: every stage stalled
    // on LDS latency with the matrix cores idle (46.4 against 43.7 us for a
    // 1x1 over 960 -> 1280 channels at 25088 pixels, 680 against 625-647 us
    // for the row-staged 3x3 below).
    for (int s = 0; s + 1 < S; s++) {
        const int buf = s % NS;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            if (h + 1 < NH) {
                read_frags(buf, h + 1, wf[(h + 1) & 1], xf[(h + 1) & 1]);
            } else {
                wait_stage(min(NS - 2, S - 2 - s));
                __syncthreads();
                if (s + NS < S) issue(s + NS, buf);
                read_frags((s + 1) % NS, 0, wf[0], xf[0]);
            }
            mfmas(wf[h & 1], xf[h & 1]);
        }
    }
#pragma unroll
    for (int h = 0; h < NH; h++) {
        if (h + 1 < NH) read_frags((S - 1) % NS, h + 1, wf[(h + 1) & 1], xf[(h + 1) & 1]);
        mfmas(wf[h & 1], xf[h & 1]);
    }

    // The next tile's first stage goes in before this tile's epilogue (after
    // a barrier: every wave has read the ring), its other stages after it.
    const int cp0 = p0, cc0 = c0, cur = j;
    const bool more = ++j < ntile;
    if (more) {
        __syncthreads();
        setup(bid * TPB + j);
        issue(0, 0);
    }
    gemm_store<PT, CT, HI, CORR>(acc, recs(cur), lut_s, a.lut != nullptr, a.y, a.oc, a.yz, a.lo, a.hi, wc * WC,
                                 cc0 + wc * WC, (long)cp0 + wp * WP, a.M, lane);
    if (!more) break;
#pragma unroll
    for (int s = 1; s < NS; s++)
        if (s < S) issue(s, s);
    }
}

// ---------------------------------------------------------------------------
// Row-staged implicit GEMM for stride-1, undilated convs over exactly 128
// input channels with at most 128 output channels (3x3 over 128 channels at
// 80x80, for instance): the im2col kernel above stages every tap's pixel rows
// again (nine times the input for a 3x3) and re-streams all weights for each
// 256-pixel tile. Here a block owns 512 consecutive output pixels of one
// image at a time (a tile) and stages the input rows those pixels touch, with
// the kernel's halo and padding (the zero point) around them, once per tile
// in LDS; each tap then reads its shifted window of those rows. The weights
// of one tap (128 channels x 128 bytes) stream through a three-stage ring.
// Blocks are persistent, one per CU, over a contiguous range of tiles: once
// a tile's last stage is read, the next tile's input rows and first weight
// stage are issued before the tile's epilogue runs, so that staging overlaps
// requantisation.
struct RowsArgs {
    const int8_t *x;
    int8_t *y;
    const int8_t *w;           // [oc_pad][kpad], k = (ky, kx, ic), kpad = kh * kw * 128
    const int4 *epi;
    const uint8_t *lut;
    int ih, iw, ow, ohw, kh, kw, pt, pl, oc, oc_pad, kpad, xz, yz, lo, hi;
    int cols;                  // staged columns: ow + kw - 1
    int tiles_per_image, tiles;
};

constexpr int RG_BP = 512, RG_BC = 128, RG_NS = 3, RG_NW = 8;
constexpr int RG_SLOTS = 832;                          // staged pixels (128 bytes each) per tile
constexpr int RG_NIN = RG_SLOTS / (8 * RG_NW);         // input staging instructions per wave
constexpr int RG_NIW = RG_BC * 128 / 1024 / RG_NW;     // weight instructions per wave per stage
static_assert(RG_NIN * 8 * RG_NW == RG_SLOTS, "whole staging instructions");

template <int EMODE>
__global__ __launch_bounds__(64 * RG_NW) void k_gemm_rows(RowsArgs a)
{
    constexpr int KS = 128, WP = 128, WC = 64, NWP = 4, NW = RG_NW, T = 64 * NW;
    constexpr int PT = WP / 32, CT = WC / 32, NS = RG_NS, NIW = RG_NIW, NH = KS / 32;
    constexpr int WSTAGE = RG_BC * KS;
    constexpr bool HI = (EMODE & 1) != 0, CORR = (EMODE & 2) != 0;

    __shared__ __attribute__((aligned(1024))) int8_t xin[RG_SLOTS * 128];
    __shared__ __attribute__((aligned(1024))) int8_t ring[NS * WSTAGE];
    __shared__ __attribute__((aligned(16))) int r_m[RG_BC], r_t[RG_BC], r_b[RG_BC], r_ls[RG_BC];
    __shared__ __attribute__((aligned(16))) long long r_c1[RG_BC], r_thr[RG_BC];
    __shared__ __attribute__((aligned(16))) int8_t lut_s[256];

    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wp = wave % NWP, wc = wave / NWP;
    const int fr = lane & 31, fh = lane >> 5;
    const int per = a.tiles / (int)gridDim.x, extra = a.tiles % (int)gridDim.x, b = (int)blockIdx.x;
    const int t_begin = b * per + min(b, extra), t_end = t_begin + per + (b < extra ? 1 : 0);
    if (t_begin >= t_end) return;

    const EpiLds recs = {r_m, r_t, r_b, r_ls, r_c1, r_thr};
    load_records<T>(recs, a.epi, 0, RG_BC, a.oc, t);
    if (a.lut && t < 64) ((int *)lut_s)[t] = ((const int *)a.lut)[t];

    const int8_t *pad = (const int8_t *)g_pad_rows.b + (a.xz & 0xff) * 16;
    const uint32_t xin_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)xin;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)ring;
    const int S = a.kh * a.kw;

    // Weight rows of the ring: instruction i of wave w fills rows
    // (w + i * NW) * 8 + lane / 8; the chunk a lane loads is the same for
    // all i (swizzle bits unchanged by i * NW * 8).
    const int cqw = swz<KS>(wave * 8 + lane / 8, lane % 8);
    const int8_t *wsrc[NIW];
#pragma unroll
    for (int i = 0; i < NIW; i++)
        wsrc[i] = a.w + (long)min((wave + i * NW) * 8 + lane / 8, a.oc_pad - 1) * a.kpad + cqw * 16;
    auto issue_w = [&](int s, int buf) {
        const uint32_t dst = ring_lds + buf * WSTAGE + wave * 1024;
#pragma unroll
        for (int i = 0; i < NIW; i++) lds_load16(wsrc[i] + s * KS, dst + i * NW * 1024);
    };
    // Tile geometry: image n, output pixels [pbeg, pend) of it, first output
    // row oy_a, staged rows (output rows spanned plus the kernel's halo).
    struct Tile {
        int n, pbeg, pend, oy_a, rows;
    };
    auto geom = [&](int tile) {
        Tile g;
        g.n = tile / a.tiles_per_image;
        g.pbeg = (tile - g.n * a.tiles_per_image) * RG_BP;
        g.pend = min(g.pbeg + RG_BP, a.ohw);
        g.oy_a = g.pbeg / a.ow;
        g.rows = (g.pend - 1) / a.ow - g.oy_a + a.kh;
        return g;
    };
    // Staged slot q = staged row r * cols + column c holds input pixel
    // (oy_a - pt + r, c - pl), or the zero point outside the image (and past
    // the tile's rows); its 16-byte chunks are swizzled by q as ring rows are.
    auto issue_in = [&](const Tile &g) {
        const int8_t *img = a.x + (long)g.n * a.ih * a.iw * 128;
        const int iyb = g.oy_a - a.pt;
        // Slots q, q + 64, ... of this lane (instruction i adds NW * 8), with
        // their staged row and column stepped along.
        int q = wave * 8 + lane / 8;
        int r = q / a.cols, c = q - r * a.cols;
#pragma unroll 1
        for (int i = 0; i < RG_NIN; i++) {
            const int iy = iyb + r, ix = c - a.pl;
            const int cq = swz<KS>(q, lane % 8);
            const bool in = r < g.rows && (unsigned)iy < (unsigned)a.ih && (unsigned)ix < (unsigned)a.iw;
            lds_load16(in ? img + ((long)iy * a.iw + ix) * 128 + cq * 16 : pad, xin_lds + (wave + i * NW) * 1024);
            q += NW * 8;
            c += NW * 8;
            while (c >= a.cols) {
                c -= a.cols;
                r++;
            }
        }
    };

    v16i acc[CT][PT];
    int qb[PT];
    auto read_frags = [&](int s, int h, v4i (&wf)[CT], v4i (&xf)[PT]) {
        const int ky = s / a.kw, kx = s - ky * a.kw, toff = ky * a.cols + kx;
        const int c = 2 * h + fh;
        const int8_t *ws = ring + (s % NS) * WSTAGE;
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            const int row = wc * WC + ct * 32 + fr;
            wf[ct] = *(const v4i *)(ws + row * KS + swz<KS>(row, c) * 16);
        }
#pragma unroll
        for (int pt = 0; pt < PT; pt++) {
            const int q = qb[pt] + toff;
            xf[pt] = *(const v4i *)(xin + q * KS + swz<KS>(q, c) * 16);
        }
    };
    auto mfmas = [&](const v4i (&wf)[CT], const v4i (&xf)[PT]) {
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int pt = 0; pt < PT; pt++)
                acc[ct][pt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[ct], xf[pt], acc[ct][pt], 0, 0, 0);
    };
    auto wait_stage = [&](int later) {
        if (later <= 0) wait_vm<0>();
        else if (later == 1) wait_vm<NIW>();
        else wait_vm<2 * NIW>();
    };

    // Load order per tile: input rows, weight stage 0, (the previous tile's
    // stores), weight stages 1 .. NS-1; the first wait then leaves only
    // stages 1 .. NS-1 outstanding.
    Tile g = geom(t_begin);
    issue_in(g);
#pragma unroll
    for (int s = 0; s < NS; s++)
        if (s < S) issue_w(s, s);
    for (int tile = t_begin;;) {
#pragma unroll
        for (int pt = 0; pt < PT; pt++) {
            const int o = min(g.pbeg + wp * WP + pt * 32 + fr, g.pend - 1);
            const int oy = o / a.ow, ox = o - oy * a.ow;
            qb[pt] = (oy - g.oy_a) * a.cols + ox;
        }
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int pt = 0; pt < PT; pt++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[ct][pt][r] = 0;
        wait_stage(min(NS - 1, S - 1));
        __syncthreads();
        v4i wf[2][CT], xf[2][PT];
        read_frags(0, 0, wf[0], xf[0]);
        for (int s = 0; s + 1 < S; s++) {
#pragma unroll
            for (int h = 0; h < NH; h++) {
                if (h + 1 < NH) {
                    read_frags(s, h + 1, wf[(h + 1) & 1], xf[(h + 1) & 1]);
                } else {
                    wait_stage(min(NS - 2, S - 2 - s));
                    __syncthreads();
                    if (s + NS < S) issue_w(s + NS, s % NS);
                    read_frags(s + 1, 0, wf[0], xf[0]);
                }
                mfmas(wf[h & 1], xf[h & 1]);
            }
        }
#pragma unroll
        for (int h = 0; h < NH; h++) {
            if (h + 1 < NH) read_frags(S - 1, h + 1, wf[(h + 1) & 1], xf[(h + 1) & 1]);
            mfmas(wf[h & 1], xf[h & 1]);
        }
        // Every wave has read the tile's rows and its last stages: the next
        // tile's rows and first stage go in before this tile's epilogue.
        __syncthreads();
        const Tile cur = g;
        const int next = tile + 1;
        if (next < t_end) {
            g = geom(next);
            issue_in(g);
            issue_w(0, 0);
        }
        const long prow = (long)cur.n * a.ohw;
        gemm_store<PT, CT, HI, CORR>(acc, recs, lut_s, a.lut != nullptr, a.y, a.oc, a.yz, a.lo, a.hi, wc * WC,
                                     wc * WC, prow + cur.pbeg + wp * WP, prow + cur.pend, lane);
        if (next >= t_end) break;
#pragma unroll
        for (int s = 1; s < NS; s++)
            if (s < S) issue_w(s, s);
        tile = next;
    }
}

static uint64_t g_launches;     // successful launches, for tests that must know which kernel ran
static int g_cus;               // compute units of the device (persistent grid sizes)

// Sets g_cus on first use; nonzero if the device cannot be queried.
static int cu_count(void)
{
    if (g_cus) return 0;
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1)
        return 1;
    g_cus = n;
    return 0;
}

// Launches of the large-tile GEMM since the library was loaded (a test hook;
// not part of the plan ABI).
extern "C" uint64_t uqk_gemm_launches(void) { return g_launches; }

template <int WP, int WC, int NWP, int NWC, int NS, int KS, bool IM2COL, int TPB>
static void launch_gemm_tpb(const GemmArgs &a, int emode, dim3 grid, dim3 block, hipStream_t st, hipEvent_t e0,
                            hipEvent_t e1)
{
    switch (emode) {
    case 0: hipExtLaunchKernelGGL((k_gemm<WP, WC, NWP, NWC, NS, KS, IM2COL, 0, TPB>), grid, block, 0, st, e0, e1, 0u, a); break;
    case 1: hipExtLaunchKernelGGL((k_gemm<WP, WC, NWP, NWC, NS, KS, IM2COL, 1, TPB>), grid, block, 0, st, e0, e1, 0u, a); break;
    case 2: hipExtLaunchKernelGGL((k_gemm<WP, WC, NWP, NWC, NS, KS, IM2COL, 2, TPB>), grid, block, 0, st, e0, e1, 0u, a); break;
    default: hipExtLaunchKernelGGL((k_gemm<WP, WC, NWP, NWC, NS, KS, IM2COL, 3, TPB>), grid, block, 0, st, e0, e1, 0u, a); break;
    }
}

// Two tiles per block when the launch has more tiles than the device has
// compute units (more than one round of blocks) and a block fills its
// compute unit (eight waves), else one: the four-wave configuration relies
// on two blocks per compute unit, whose LDS the second record buffer would
// no longer fit.
template <int WP, int WC, int NWP, int NWC, int NS, int KS, bool IM2COL>
static int launch_gemm(GemmArgs a, int emode, int tpb_forced)
{
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    const int tpb = tpb_forced == 1 || tpb_forced == 2 ? tpb_forced : a.ntiles > g_cus && NWP * NWC == 8 ? 2 : 1;
    a.nblocks = (a.ntiles + tpb - 1) / tpb;
    const dim3 grid((unsigned)a.nblocks), block(64 * NWP * NWC);
    if (tpb == 2) launch_gemm_tpb<WP, WC, NWP, NWC, NS, KS, IM2COL, 2>(a, emode, grid, block, st, e0, e1);
    else launch_gemm_tpb<WP, WC, NWP, NWC, NS, KS, IM2COL, 1>(a, emode, grid, block, st, e0, e1);
    const int rc = uqk_fail(hipGetLastError());
    if (!rc) g_launches++;
    return rc;
}

// Tile configurations (pixels x channels per block, waves, LDS stages of K
// bytes each):
//   0: 256 x 128, four waves of 128 x 64, three stages of 64 (78 KiB: two blocks per CU)
//   1: 256 x 256, eight waves of 128 x 64, three stages of 64 (104 KiB)
//   2: 256 x 128, eight waves of 64 x 64, three stages of 128 (148 KiB)
//   3: 256 x 256, eight waves of 128 x 64, two stages of 128 (136 KiB)
//   4: the row-staged kernel (k_gemm_rows), where the layer fits it
static const int g_tile_ks[4] = {64, 64, 128, 128};
static const int g_tile_bc[4] = {128, 256, 128, 256};

template <bool IM2COL>
static int launch_tile(int tile, const GemmArgs &a, int emode, int tpb)
{
    switch (tile) {
    case 1: return launch_gemm<128, 64, 2, 4, 3, 64, IM2COL>(a, emode, tpb);
    case 2: return launch_gemm<64, 64, 4, 2, 3, 128, IM2COL>(a, emode, tpb);
    case 3: return launch_gemm<128, 64, 2, 4, 2, 128, IM2COL>(a, emode, tpb);
    default: return launch_gemm<128, 64, 2, 2, 3, 64, IM2COL>(a, emode, tpb);
    }
}

static int gemm_im2col(const UQKSpatial *d) { return d->mode == UQK_G16 || d->mode == UQK_ROWS16; }

// Whether a layer fits the row-staged kernel: stride 1, no dilation, 128
// input channels (one 128-byte stage per tap), at most 128 output channels,
// at least three taps, and the rows that 512 consecutive output pixels of one
// image touch (plus the kernel's halo) within the staged slots. *cols: staged
// columns.
static int rows_fit(const UQKSpatial *d, int *cols)
{
    if (!gemm_im2col(d) || d->ic != 128 || d->sh != 1 || d->sw != 1 || d->dh != 1 || d->dw != 1) return 0;
    if (d->oc > RG_BC || d->oc % 16 || d->K != d->kh * d->kw * 128 || d->kpad != d->K || d->kh * d->kw < 3) return 0;
    const long c = (long)d->ow + d->kw - 1;
    long span = (RG_BP - 1 + d->ow - 1) / d->ow + 1;
    if (span > d->oh) span = d->oh;           /* a tile never leaves its image */
    if ((span + d->kh - 1) * c > RG_SLOTS) return 0;
    *cols = (int)c;
    return 1;
}


static int launch_rows(const UQKSpatial *d, const void *x, void *y, uint32_t batches, int cols, int emode)
{
    if (cu_count()) return uqk_fail(hipErrorInvalidDevice);
    RowsArgs a;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.ih = d->ih; a.iw = d->iw; a.ow = d->ow; a.ohw = d->oh * d->ow; a.kh = d->kh; a.kw = d->kw;
    a.pt = d->pt; a.pl = d->pl; a.oc = d->oc; a.oc_pad = d->oc_pad; a.kpad = d->kpad;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.cols = cols;
    a.tiles_per_image = (a.ohw + RG_BP - 1) / RG_BP;
    const uint64_t tiles = (uint64_t)batches * a.tiles_per_image;
    if (!tiles || tiles > 0x7fffffffULL) return (int)hipErrorInvalidValue;
    a.tiles = (int)tiles;
    const unsigned grid = (unsigned)(tiles < (uint64_t)g_cus ? tiles : (uint64_t)g_cus);
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    switch (emode) {
    case 0: hipExtLaunchKernelGGL(k_gemm_rows<0>, dim3(grid), dim3(64 * RG_NW), 0, st, e0, e1, 0u, a); break;
    case 1: hipExtLaunchKernelGGL(k_gemm_rows<1>, dim3(grid), dim3(64 * RG_NW), 0, st, e0, e1, 0u, a); break;
    case 2: hipExtLaunchKernelGGL(k_gemm_rows<2>, dim3(grid), dim3(64 * RG_NW), 0, st, e0, e1, 0u, a); break;
    default: hipExtLaunchKernelGGL(k_gemm_rows<3>, dim3(grid), dim3(64 * RG_NW), 0, st, e0, e1, 0u, a); break;
    }
    const int rc = uqk_fail(hipGetLastError());
    if (!rc) g_launches++;
    return rc;
}

extern "C" int uqk_gemm_ok(const UQKSpatial *d)
{
    if (d->oc % 16 || d->kpad % 64 || d->K < 256) return 0;
    if (d->mode == UQK_PW) return d->ic % 16 == 0;
    return gemm_im2col(d) && d->ic % 64 == 0 && d->K == d->kh * d->kw * d->ic && d->kpad == d->K;
}

// Tile configuration of a launch: 256 x 256 for layers over 128 channels
// (half the operand traffic per MAC of 256 x 128: 37.5 against 40.2 us for a
// 1x1 over 960 -> 1280 channels at 25088 pixels), else 256 x 128 with
// 128-byte stages where an im2col stage stays inside one tap (600 against
// 628 us for a 3x3 over 128 channels at 3.3M pixels). A forced
// configuration (d->gemm_tile) whose stages would straddle taps falls back
// to its 64-byte-stage shape.
static int gemm_tile(const UQKSpatial *d, uint64_t pixels)
{
    (void)pixels;
    int cols;
    const bool deep_ok = d->mode == UQK_PW || d->ic % 128 == 0;
    if (d->gemm_tile == 4 || (d->gemm_tile < 0 && rows_fit(d, &cols))) {
        if (rows_fit(d, &cols)) return 4;
    }
    int tile = d->gemm_tile >= 0 && d->gemm_tile < 4 ? d->gemm_tile : d->oc > 128 ? 1 : deep_ok ? 2 : 0;
    if (g_tile_ks[tile] == 128 && !deep_ok) tile -= 2;
    return tile;
}

extern "C" int uqk_gemm_take(const UQKSpatial *d, uint64_t pixels)
{
    if (d->gemm == 0 || !uqk_gemm_ok(d) || pixels >= 0x7fffffffULL) return 0;
    if (d->gemm == 1) return 1;
    // Also deep convs the general kernel would run on per-lane gathers (no
    // row staging within its LDS): a 3x3 stride-2 128 -> 128 conv at 40x40,
    // 64 images (K = 1,152, 25,600 pixels), 31.0 -> 16.3 us; smaller or
    // shallower ones (6,400 x 256 or 25,600 x 64 at K = 1,152, K = 576)
    // measured slower here.
    if (d->mode == UQK_G16 && d->K >= 1024 && pixels * (uint64_t)d->oc >= (1ULL << 21)) return 1;
    return d->K >= 512 && pixels * (uint64_t)d->oc >= (1ULL << 24);
}

extern "C" int uqk_gemm(const UQKSpatial *d, const void *x, void *y, uint32_t batches)
{
    const uint64_t pixels = (uint64_t)batches * d->oh * d->ow;
    if (!uqk_gemm_ok(d) || !pixels || pixels >= 0x7fffffffULL) return (int)hipErrorInvalidValue;
    GemmArgs a;
    a.x = (const int8_t *)x;
    a.y = (int8_t *)y;
    a.w = (const int8_t *)d->w;
    a.epi = (const int4 *)d->epi;
    a.lut = (const uint8_t *)d->lut;
    a.M = (int)pixels;
    a.K = d->K; a.kpad = d->kpad; a.oc = d->oc; a.oc_pad = d->oc_pad;
    a.ih = d->ih; a.iw = d->iw; a.ic = d->ic; a.ow = d->ow; a.ohw = d->oh * d->ow;
    a.kw = d->kw; a.sh = d->sh; a.sw = d->sw; a.dh = d->dh; a.dw = d->dw; a.pt = d->pt; a.pl = d->pl;
    a.xz = d->xz; a.yz = d->yz; a.lo = d->lo; a.hi = d->hi;
    a.rotate = 1;
    const int emode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0);
    const int tile = gemm_tile(d, pixels);
    if (tile == 4) {
        int cols = 0;
        rows_fit(d, &cols);
        return launch_rows(d, x, y, batches, cols, emode);
    }
    const int bp = 256, bc = g_tile_bc[tile];
    a.ctiles = (d->oc + bc - 1) / bc;
    const uint64_t tiles = (pixels + bp - 1) / bp * (uint64_t)a.ctiles;
    if (tiles > 0x7fffffffULL) return (int)hipErrorInvalidValue;
    a.ntiles = (int)tiles;
    if (cu_count()) return uqk_fail(hipErrorInvalidDevice);
    return d->mode != UQK_PW ? launch_tile<true>(tile, a, emode, d->gemm_tpb)
                             : launch_tile<false>(tile, a, emode, d->gemm_tpb);
}

// ---------------------------------------------------------------------------
// Matrix-core ceiling (a measurement hook, not part of the plan ABI): waves
// that issue v_mfma_i32_32x32x32_i8 on register operands, eight independent
// accumulators each, two waves per SIMD as in the GEMMs above, no memory
// traffic inside the loop (eight rotates per eight MFMAs vary the operands). Launched back to back for as long as a
// GEMM launch lasts, it gives the int8 rate the device sustains at the clock
// it holds under that load: the most any of the GEMMs could reach.
__device__ int uqk_ceiling_sink;   // external linkage, so the loop's result is not dead

__global__ __launch_bounds__(256) void k_mfma_ceiling(int iters)
{
    v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0;
    // Operand bytes from a multiplicative hash of the lane and block, rotated
    // by one bit after every round, so that the matrix cores see changing
    // data (their power, and so the clock the device holds, depends on it).
    v4i a, b;
    const unsigned seed = (threadIdx.x + 1u) * 0x9e3779b1u ^ (blockIdx.x + 1u) * 0x85ebca77u;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        a[k] = (int)(seed * (2u * k + 3u) + 0x27d4eb2fu * k);
        b[k] = (int)(seed * (2u * k + 7u) ^ 0x165667b1u * (k + 1u));
    }
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[j], 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            a[k] = (int)__builtin_rotateleft32((unsigned)a[k], 1);
            b[k] = (int)__builtin_rotateleft32((unsigned)b[k], 1);
        }
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[j][r];
    if (s == 0x7fffffff) uqk_ceiling_sink = s;    // keeps the loop; almost never stores
}

// Runs `warmup` untimed and `reps` timed launches of `iters` rounds on
// every SIMD (two blocks of four waves per compute unit) on the library
// stream and returns the sustained rate in *tops (10^12 int8 ops/s, two per
// multiply-accumulate) and the mean launch time in *us.
extern "C" int uqk_mfma_ceiling(int iters, int warmup, int reps, double *tops, double *us)
{
    if (iters < 1 || reps < 1 || warmup < 0 || !tops || !us) return (int)hipErrorInvalidValue;
    if (cu_count()) return uqk_fail(hipErrorInvalidDevice);
    hipStream_t st;
    hipEvent_t e0, e1;
    uqk_next_launch(&st, &e0, &e1);
    hipEvent_t t0, t1;
    if (hipEventCreate(&t0) != hipSuccess) return uqk_fail(hipErrorOutOfMemory);
    if (hipEventCreate(&t1) != hipSuccess) {
        (void)hipEventDestroy(t0);
        return uqk_fail(hipErrorOutOfMemory);
    }
    const dim3 grid((unsigned)(2 * g_cus)), block(256);
    int rc = 0;
    for (int i = 0; i < warmup && !rc; i++) {
        hipLaunchKernelGGL(k_mfma_ceiling, grid, block, 0, st, iters);
        rc = uqk_fail(hipGetLastError());
    }
    if (!rc) rc = uqk_fail(hipEventRecord(t0, st));
    for (int i = 0; i < reps && !rc; i++) {
        hipLaunchKernelGGL(k_mfma_ceiling, grid, block, 0, st, iters);
        rc = uqk_fail(hipGetLastError());
    }
    if (!rc) rc = uqk_fail(hipEventRecord(t1, st));
    if (!rc) rc = uqk_fail(hipEventSynchronize(t1));
    float ms = 0.f;
    if (!rc) rc = uqk_fail(hipEventElapsedTime(&ms, t0, t1));
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    if (rc) return rc;
    const double ops = 2.0 * 32 * 32 * 32 * 8 * (double)iters * 4 * grid.x * reps;
    *us = ms * 1e3 / reps;
    *tops = ops / (ms * 1e-3) / 1e12;
    return 0;
}
