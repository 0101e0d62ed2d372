/* Thin C ABI between the plain-C graph host (graph.c) and the gfx950 HIP
 * kernels (kernels.hip). Plain pointers and integers only: device pointers
 * are opaque `void *` on the host side. Every launcher enqueues on the
 * library's single HIP stream and returns 0 or a HIP error code. */
#ifndef UQK_H
#define UQK_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Spatial op descriptor shared by conv (code 14), depthwise (15) and pool (16).
 * Geometry is the qnn.c:12-16 parameter block; the device tables are built at
 * load time by graph.c:
 *   w    conv: [oc_pad][kpad] signed int8, k = (ky, kx, ic), zero beyond K
 *        depthwise: [taps][C] signed int8 (the plan's own layout)
 *   epi  32 bytes per channel: corrected bias folded for signed inputs
 *        (bias + 128*sum(w) [+ xz*tail weights]), multiplier, left shift,
 *        total right shift, and two int64 constants of the one-multiply
 *        requantisation (see epilogue_record in graph.c)
 *   wdot depthwise: [ceil(taps/4)][C] words of four taps per channel
 *   kmap conv gathers: int32 x4 per gather group {ky*dh, kx*dw, ic, 0}
 *   lut  optional fused 256-entry post table (uq_post) */
typedef struct {
    int32_t ih, iw, ic, oh, ow, oc;
    int32_t kh, kw, sh, sw, dh, dw, pt, pl;
    int32_t xz, yz, lo, hi;
    int32_t K, kpad, oc_pad, mode, nt, rb, is_max, vec, corr;
    int32_t hi_shift;          /* every shift in [-22, -1]: records fold bias and zero point into c1 */
    int32_t dwwin;             /* depthwise on tap windows (k_dw_win); wdot holds [ky][wk][C] tap words */
    int32_t gemm;              /* large-tile GEMM: -1 when the launch is large enough, 0 never, 1 whenever the shape fits */
    int32_t gemm_tile;         /* its tile configuration: -1 automatic, else 0..4 (gemm.hip) */
    int32_t gemm_tpb;          /* its output tiles per block: 0 automatic, else 1 or 2 */
    int32_t dwk;               /* depthwise kernel: -1 automatic, 0 band (dw.hip), 1 matrix-core window, 2 dot4 window */
    int32_t dw_rows;           /* matrix-core window depthwise: most output rows per block (0: automatic) */
    int32_t dwb[4];            /* band depthwise plan (uqk_dw_band_prepare): channel groups per block (0: the layer
                                * does not fit), output rows per block, chunk swizzle shift and mask */
    const void *w;
    const void *wdot;
    const void *epi;
    const void *kmap;
    const void *lut;
} UQKSpatial;

/* Conv A-operand sources: pointwise rows, per-lane gathers with 16/4/1-byte
 * granularity, LDS-staged input rows (16-byte slices, or 4-byte words over
 * channels padded to a multiple of four), or the stem form (at most four
 * kernel rows of kw * IC <= 16 contiguous input bytes each: the receptive
 * field is one 64-byte K step, 16 bytes per kernel row). */
enum { UQK_PW = 0, UQK_G16 = 1, UQK_G4 = 2, UQK_G1 = 3, UQK_ROWS16 = 4, UQK_ROWS4 = 5, UQK_STEM = 6 };

/* Dynamic LDS bytes of the tap-window depthwise kernel for a layer, 0 when
 * the layer's shape is outside it (needs C % 4 == 0, square 3x3 or 5x5,
 * stride 1 or 2, no dilation). */
size_t uqk_dw_win_lds(const UQKSpatial *d);

/* Band depthwise (dw.hip): 3x3/5x5, stride 1/2, C % 16 == 0. prepare fills
 * d->dwb once when the plan is loaded (reads the geometry fields); the launch
 * uses that plan (hipErrorInvalidValue if d->dwb[0] is 0). */
void uqk_dw_band_prepare(UQKSpatial *d);
int uqk_dw_band(const UQKSpatial *d, const void *x, void *y, uint32_t batches);

/* Fused inverted bottleneck (ib.hip: 1x1 expand -> stride-1 depthwise ->
 * 1x1 project [-> residual add with the block input]), one workgroup per
 * image. Device tables are the three layers' own prepared tables. */
typedef struct {
    int32_t P, H, W, Cin, Ce, Cout, ks, pt, pl;
    const void *we, *epi_e, *lut_e;
    int32_t kpe, e_mode, e_yz, e_lo, e_hi;
    const void *dww, *epi_d, *lut_d;
    int32_t d_mode, d_yz, d_lo, d_hi, d_xz;
    const void *wp, *epi_p, *lut_p;
    int32_t kpp, p_mode, p_yz, p_lo, p_hi;
    int32_t has_add, add_x_first;
    const void *add_tab;       /* the add's two 256-entry int32 tables */
    int32_t a_m, a_s, a_yz, a_lo, a_hi;
} UQKIb;

/* LDS bytes of the fused block for one image, 0 if the block does not fit
 * the kernel; offsets[9] receives the region offsets when non-null. */
size_t uqk_ib_lds(int P, int H, int W, int Cin, int Ce, int Cout, int ks, size_t *offsets);
int uqk_ib(const UQKIb *f, const void *x, void *y, uint32_t images);

/* Banded universal inverted bottleneck (uib.hip): [start depthwise, stride
 * 1] -> 1x1 expand -> [depthwise, stride 1 or 2] -> 1x1 project [-> residual
 * add with the block input], one workgroup per image and band of R output
 * rows. k0 / k: the depthwise kernel sizes (3 or 5; 0: absent, not both).
 * Tap words are the window form's [ky][k > 4 ? 2 : 1][C]. */
typedef struct {
    int32_t H, W, Ho, Wo, Cin, Ce, Cout;
    int32_t k0, p0t, p0l;
    const void *dw0, *epi0, *lut0;
    int32_t m0, yz0, lo0, hi0, xz0;
    const void *we, *epi_e, *lut_e;
    int32_t kpe, e_mode, e_yz, e_lo, e_hi;
    int32_t k, s, pt, pl;
    const void *dww, *epi_d, *lut_d;
    int32_t d_mode, d_yz, d_lo, d_hi, d_xz;
    const void *wp, *epi_p, *lut_p;
    int32_t kpp, p_mode, p_yz, p_lo, p_hi;
    int32_t has_add, add_x_first;
    const void *add_tab;
    int32_t a_m, a_s, a_yz, a_lo, a_hi;
    int32_t R;                 /* output rows per band: set by uqk_uib_plan */
    int32_t rec_lds;           /* expand and depthwise records in LDS: set by uqk_uib_plan */
} UQKUib;

/* Sets f->R to the most output rows per band whose workgroup fits in LDS
 * (and f->rec_lds: whether the expand and depthwise records fit in LDS too)
 * and returns that LDS size; 0 (and R = 0) when the block does not fit the
 * kernel (channel counts multiples of 32, Cin <= 256, Ce <= 512, pads within
 * the kernels, an add only at stride 1 with Cin == Cout). */
size_t uqk_uib_plan(UQKUib *f);
int uqk_uib(const UQKUib *f, const void *x, void *y, uint32_t images);

/* Stem conv fused with the 3x3 stride-2 conv over its 32-channel output
 * and, when p is not null, the 1x1 32 -> 32 conv over the 3x3's output
 * (stem.hip): whether the group fits, and its launch (images of the stem's
 * input to the last conv's output). */
int uqk_stem_conv_ok(const UQKSpatial *s, const UQKSpatial *c, const UQKSpatial *p);
int uqk_stem_conv(const UQKSpatial *s, const UQKSpatial *c, const UQKSpatial *p, const void *x, void *y,
                  uint32_t images);

/* Whether a conv layer fits the stem kernel (kh <= 4, kw * IC <= 16, no
 * column dilation, left and right padding within 16 bytes, input rows a
 * multiple of 16 bytes, its staged rows within 48 KiB, OC % 16 == 0). Reads
 * iw, ic, kh, kw, sh, sw, dh, dw, pl, ow and oc. */
int uqk_conv_stem_ok(const UQKSpatial *d);

/* Dynamic LDS bytes k_conv_rows needs for a layer at rb row blocks per wave. */
size_t uqk_conv_rows_lds(const UQKSpatial *d, int rb);
/* Whether a conv layer runs on k_conv_rows (chosen when the plan is loaded;
 * reads the fields uqk_conv_rows_lds reads). */
int uqk_conv_rows_ok(const UQKSpatial *d);

int uqk_init(void);
int uqk_device_count(void);
/* The no-allocation entry point's device scratch: a static array of
 * UQK_SCRATCH_BYTES per GPU, 256-byte aligned; its address on the device
 * that was current at uqk_init (NULL before it). */
#define UQK_SCRATCH_BYTES (64u << 20)
void *uqk_scratch(size_t *bytes);
void *uqk_malloc(size_t bytes);
void uqk_free(void *p);
int uqk_h2d(void *dst, const void *src, size_t bytes);        /* async on the stream */
int uqk_d2h(void *dst, const void *src, size_t bytes);        /* async on the stream */
int uqk_d2d(void *dst, const void *src, size_t bytes);        /* async on the stream */
int uqk_d2d_2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t height);
/* rows copies: y row r (pitch dp) = a row r (w1 bytes, pitch s1) then b row r
 * (w2 bytes, pitch s2; w2 may be 0). One kernel launch. */
int uqk_rows2(void *y, uint64_t dp, const void *a, uint64_t s1, uint64_t w1, const void *b, uint64_t s2, uint64_t w2,
              uint64_t rows);
/* Rows of up to UQK_GATHER_MAX segments, each `width` bytes per row from its own
 * source (row pitch `stride`), mapped through a 256-entry table (index byte
 * ^ flip) when `lut` is set: y row r = seg 0 | seg 1 | ... (pitch dp). */
#define UQK_GATHER_MAX 8
typedef struct {
    const void *src;
    uint64_t stride;
    uint32_t width;
    const void *lut;
    uint32_t flip;
} UQKSeg;
int uqk_gather(void *y, uint64_t dp, const UQKSeg *segs, uint32_t n, uint64_t rows);
uint64_t uqk_gather_launches(void);
int uqk_sync(void);
int uqk_last_error(void);

/* Pipelined host transfers: stream 0 computes, 1 copies host -> device, 2
 * device -> host (all at the default priority); events 0-7 hand work from
 * one stream to another. */
int uqk_copy_on(int stream, void *dst, const void *src, size_t bytes, int to_device);
int uqk_pipe_record(int event, int stream);
int uqk_pipe_wait(int stream, int event);
int uqk_sync_all(void);

/* Image slices of one batch on separate compute streams (at most
 * UQK_MAX_SLICES): split_fork orders the side streams after the main
 * stream's queued work, split_use(k, n) sends the following launches to
 * slice k's stream (n slices running side by side), split_join makes the
 * main stream wait for the side streams and current again. Two: the main
 * stream, the two transfer streams and one side stream are HIP's default
 * four hardware queues (more streams would share a queue, and more queues
 * measured far slower). uqk_sync waits for the main and side streams. */
#define UQK_MAX_SLICES 2
int uqk_split_fork(int slices);
void uqk_split_use(int slice, int slices);
int uqk_split_join(int slices);
void *uqk_host_alloc(size_t bytes);                   /* pinned (hipHostMalloc) */
void uqk_host_free(void *p);

/* Whole-plan graphs: capture the compute stream's submissions, replay them. */
int uqk_capture_begin(void);
int uqk_capture_end(void **exec);
int uqk_graph_launch(void *exec);
void uqk_graph_destroy(void *exec);

int uqk_conv(const UQKSpatial *d, const void *x, void *y, uint32_t batches);

/* Large-tile conv GEMM (gemm.hip): layers with OC % 16 == 0 and K >= 256
 * whose A operand is pointwise rows (UQK_PW) or an implicit im2col with
 * IC % 64 == 0 (UQK_G16 / UQK_ROWS16 weight layouts). uqk_gemm_ok: the
 * layer's shape fits; uqk_gemm_take: uqk_conv sends a launch of `pixels`
 * output pixels there (by d->gemm: wide K and many outputs, never, or
 * always). */
int uqk_gemm_ok(const UQKSpatial *d);
int uqk_gemm_take(const UQKSpatial *d, uint64_t pixels);
int uqk_gemm(const UQKSpatial *d, const void *x, void *y, uint32_t batches);

/* A residual add (op 18) applied in a conv's epilogue: y = add(conv(x), res)
 * (or add(res, conv(x)) when conv_is_a is 0), byte for byte the add op's
 * arithmetic on the conv's int8 output. res has the conv output's layout. */
typedef struct {
    const void *res;
    const void *tables;        /* the add's two 256-entry int32 tables (operand a, then b) */
    int32_t m, s, yz, lo, hi;
    int32_t conv_is_a;
} UQKAdd;

/* Whether uqk_conv_add takes a layer (the k_conv kernel modes). */
int uqk_conv_add_ok(const UQKSpatial *d);
int uqk_conv_add(const UQKSpatial *d, const void *x, void *y, uint32_t batches, const UQKAdd *add);

/* A 1x1 conv and the mean over its whole output (head.hip): y[n][c] =
 * mean(conv(x)[n][.][c]), the mean's parameters (op 24: input and output
 * zero points, multiplier, shift) in UQKMean. ok: whether the conv fits
 * (pointwise, IC % 32 == 0 and <= 256, OC % 32 == 0, at most 64 pixels). */
typedef struct {
    int32_t xz, yz, m, s;
    int32_t parts;             /* workgroups per image, each a share of the output channels (0: automatic) */
} UQKMean;
int uqk_conv_mean_ok(const UQKSpatial *d);
int uqk_conv_mean(const UQKSpatial *d, const UQKMean *mean, const void *x, void *y, uint32_t images);
int uqk_depthwise(const UQKSpatial *d, const void *x, void *y, uint32_t batches);
int uqk_pool(const UQKSpatial *d, const void *x, void *y, uint32_t batches);
int uqk_add(const void *a, const void *b, void *y, uint64_t count, const void *tables,
            int32_t m, int32_t shift, int32_t yz, int32_t lo, int32_t hi);
int uqk_mean(const void *x, void *y, uint32_t batches, uint32_t pixels, uint32_t channels,
             int32_t xz, int32_t yz, int32_t m, int32_t shift);
int uqk_lut(const void *x, void *y, uint64_t count, const void *table, uint32_t flip);
int uqk_resize(const void *x, void *y, uint32_t batches, uint32_t ih, uint32_t iw, uint32_t oh, uint32_t ow,
               uint32_t c, const void *offsets);
/* 4-D NHWC-order gather used by pad (code 23) and slice (code 26), per image:
 * out[i0,i1,i2,i3] = in[i0-o0, i1-o1, i2-o2, i3-o3] when inside `in`, else fill. */
int uqk_window4(const void *x, void *y, uint32_t images, const uint32_t in_dims[4], const uint32_t out_dims[4],
                const int32_t offset[4], int32_t fill);

/* Permutation (code 10) of a rank <= 4 tensor per image; z.d[i] = in_dims[perm[i]]. */
int uqk_permute(const void *x, void *y, uint32_t images, uint32_t rank, const uint32_t in_dims[4],
                const uint32_t perm[4], uint32_t elem_bytes);
/* Elementwise product (code 25), q = {az, bz, yz, m, shift, lo, hi}. */
int uqk_mul(const void *a, const void *b, void *y, uint64_t count, const int32_t q[7]);
/* Batched matmul (code 27) of images * batches matrices, a [m][k] ([k][m]
 * when q[5]), b [k][n] ([n][k] when q[6]), q = {az, bz, yz, m, shift, q5, q6}. */
int uqk_bmm(const void *a, const void *b, void *z, uint32_t images, uint32_t batches, uint32_t m, uint32_t n,
            uint32_t k, const int32_t q[7]);
/* Exact softmax (code 28) over rows of `width` bytes; table = 256 Q0.31 exponentials. */
int uqk_softmax(const void *x, void *y, uint64_t rows, uint32_t width, const void *table);

/* Table softmax (code 17) over rows of `width` bytes; table = 256 Q24 values. */
int uqk_softmax_table(const void *x, void *y, uint64_t rows, uint32_t width, const void *table, int32_t lo, int32_t hi);

/* Per-op timing: a start and a stop event for each of `count` ops. Between
 * time_begin(i) and time_end(i) the launches stamp op i's events with their
 * own dispatch timestamps (first kernel's start, last kernel's end); op_ns
 * reads the interval once the stream has passed it. */
int uqk_events(uint32_t count);
int uqk_time_begin(uint32_t index);
int uqk_time_end(uint32_t index);
int uqk_op_ns(uint32_t index, uint64_t *ns);

#ifdef __cplusplus
}
#endif
#endif
