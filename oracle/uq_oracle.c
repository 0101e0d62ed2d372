/* CPU restatement of the reference's INT8 NHWC vision path.
 *
 * TEST INFRASTRUCTURE ONLY. Tests, the smoke check and the benchmark's CPU
 * baseline leg load this file's library to check results against; the GPU
 * library never links or calls it.
 *
 * Every function follows the *generic* (macro-free) semantics of the
 * reference runtime; each cites the file:line it restates. Scalar loops on
 * purpose: clarity over speed. Parity of this restatement is pinned by the
 * tests in tests/test_oracle_*.py against the reference's own C build
 * (oracle/_ref), against closed forms and against brute-force numpy
 * formulations; see the header of each test for which function it pins.
 */
#include "uq_oracle.h"
#include <stdlib.h>
#include <string.h>

typedef struct { uint32_t magic, version, nt, no, arena_bytes, input, output, reserved; } Hdr;   /* graph.h:15 */
typedef struct { uint32_t offset, bytes, type, rank, d[4], flags, reserved[3]; } Ten;             /* graph.h:16 */
typedef struct { uint32_t code, a, b, out, p[4]; } Op;                                           /* graph.h:17 */

#define HEAD 20 /* qnn.h:9: q[0:20] header, then bias[OC], mult[OC], shift[OC] (qnn.c:12-16) */

/* qnn.c:61-83 (portable branch): left shift for positive exponents, rounded
 * doubling high multiply (v*m + 2^30) >> 31, then a rounding right shift with
 * ties away from zero. */
int32_t uqo_scale(int32_t v, int32_t m, int32_t shift)
{
    if (shift > 0) v = (int32_t)((uint32_t)v << shift);
    int64_t p = (int64_t)v * m;
    int32_t h = (int32_t)((p + ((int64_t)1 << 30)) >> 31);
    if (shift >= 0) return h;
    unsigned s = (unsigned)-shift;
    uint32_t mask = ((uint32_t)1 << s) - 1;
    int32_t base = h >> s;
    uint32_t rem = (uint32_t)h & mask;
    return base + (rem > ((mask >> 1) + (uint32_t)(h < 0)));
}

static int8_t clampi(int64_t v, int lo, int hi) { return (int8_t)(v < lo ? lo : v > hi ? hi : v); }

/* uq_post, qnn.c:162-173: y = table[y + 128] when the op names a LUT. */
static int8_t post(int8_t y, const uint8_t *lut) { return lut ? (int8_t)lut[(int)y + 128] : y; }

/* Packed conv weight, gemm.h:7-13: (n/4)*Kp*4 + (k/8)*32 + (n%4)*8 + k%8. */
static int packed_w(const int8_t *w, int n, int k, int kp)
{
    return w[(size_t)(n / 4) * kp * 4 + (size_t)(k / 8) * 32 + (n % 4) * 8 + k % 8];
}

/* Code 14 on one image block. Column build of qnn.c:1155-1169 (u = x + 128,
 * spatial pad and the K tail hold xz + 128), dot product of gemm.c:24-30 over
 * all Kp columns, then requantize qnn.c:734-738 and uq_post. */
static void conv_image(const Ten *a, const int8_t *x, const int8_t *w, int8_t *y, const int32_t *q, const uint8_t *lut)
{
    int kh = q[0], kw = q[1], sh = q[2], sw = q[3], dh = q[4], dw = q[5], pt = q[6], pl = q[7];
    int oh = q[10], ow = q[11], xz = q[12], yz = q[13], lo = q[14], hi = q[15];
    int ic = q[16], oc = q[17], kp = q[18];
    int nb = (int)a->d[0], ih = a->rank == 4 ? (int)a->d[1] : 1, iw = a->rank == 4 ? (int)a->d[2] : 1;
    int K = kh * kw * ic;
    const int32_t *bias = q + HEAD, *mult = bias + oc, *shift = mult + oc;
    int *col = malloc(sizeof(int) * (size_t)kp);
    for (int n = 0; n < nb; n++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++) {
                for (int k = 0; k < kp; k++) {
                    if (k >= K) { col[k] = xz + 128; continue; }
                    int t = k / ic, c = k % ic, ky = t / kw, kx = t % kw;
                    int sy = oy * sh - pt + ky * dh, sx = ox * sw - pl + kx * dw;
                    if (sy >= 0 && sx >= 0 && sy < ih && sx < iw)
                        col[k] = (int)x[(((size_t)n * ih + sy) * iw + sx) * ic + c] + 128;
                    else
                        col[k] = xz + 128;
                }
                int8_t *dst = y + (((size_t)n * oh + oy) * ow + ox) * oc;
                for (int c = 0; c < oc; c++) {
                    int64_t acc = 0;
                    for (int k = 0; k < kp; k++) acc += (int64_t)col[k] * packed_w(w, c, k, kp);
                    int32_t v = uqo_scale((int32_t)(acc + bias[c]), mult[c], shift[c]) + yz;
                    dst[c] = post(clampi(v, lo, hi), lut);
                }
            }
    free(col);
}

/* Codes 15 and 16 on one image block: the generic loop of qnn.c:1228-1245.
 * Depthwise starts at the corrected bias and adds (x+128)*w[t*C+c] per tap,
 * with xz+128 for padded taps (weights tflite.py:152-153, HWC order).
 * Average pooling sums valid taps and divides with a half-count nudge
 * (C division truncates); max pooling starts at -128. */
static void window_image(unsigned code, const Ten *a, const int8_t *x, const int8_t *w, int8_t *y, const int32_t *q, const uint8_t *lut)
{
    int kh = q[0], kw = q[1], sh = q[2], sw = q[3], dh = q[4], dw = q[5], pt = q[6], pl = q[7];
    int oh = q[10], ow = q[11], xz = q[12], yz = q[13], lo = q[14], hi = q[15];
    int ic = q[16], oc = q[17], is_max = q[19];
    int nb = (int)a->d[0], ih = (int)a->d[1], iw = (int)a->d[2];
    const int32_t *bias = q + HEAD, *mult = bias + oc, *shift = mult + oc;
    for (int n = 0; n < nb; n++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int c = 0; c < oc; c++) {
                    int64_t acc = code == 15 ? bias[c] : is_max ? -128 : 0;
                    int valid_count = 0;
                    for (int ky = 0; ky < kh; ky++)
                        for (int kx = 0; kx < kw; kx++) {
                            int sy = oy * sh - pt + ky * dh, sx = ox * sw - pl + kx * dw;
                            int valid = sy >= 0 && sx >= 0 && sy < ih && sx < iw;
                            int v = valid ? x[(((size_t)n * ih + sy) * iw + sx) * ic + c] : 0;
                            valid_count += valid;
                            if (code == 15) acc += (int64_t)((valid ? v : xz) + 128) * w[(ky * kw + kx) * oc + c];
                            else if (valid) { if (is_max) { if (v > acc) acc = v; } else acc += v; }
                        }
                    int64_t value = acc;
                    if (code == 15) value = (int64_t)uqo_scale((int32_t)acc, mult[c], shift[c]) + yz;
                    else if (!is_max) {
                        int32_t s = (int32_t)acc, half = valid_count / 2;
                        value = (s + (s > 0 ? half : -half)) / valid_count;
                    }
                    int8_t r = clampi(value, lo, hi);
                    y[(((size_t)n * oh + oy) * ow + ox) * oc + c] = code == 15 ? post(r, lut) : r;
                }
}

/* uq_add, qnn.c:175-183: two pre-scaled 256-entry tables, one requant. */
static void add_image(const int8_t *x, const int8_t *b, int8_t *y, uint32_t count, const int32_t *q)
{
    const int32_t *tx = q + 8, *tb = q + 264;
    for (uint32_t i = 0; i < count; i++) {
        int32_t sum = tx[(int)x[i] + 128] + tb[(int)b[i] + 128];
        y[i] = clampi((int64_t)uqo_scale(sum, q[0], q[1]) + q[2], q[3], q[4]);
    }
}

/* uq_mean, qnn.c:184-198: per (batch, channel) spatial sum minus count*xz. */
static void mean_image(const int8_t *x, int8_t *y, unsigned batches, unsigned channels, const int32_t *q)
{
    for (unsigned n = 0; n < batches; n++)
        for (unsigned c = 0; c < channels; c++) {
            int32_t sum = 0;
            for (int p = 0; p < q[0]; p++) sum += x[((size_t)n * q[0] + p) * channels + c];
            y[n * channels + c] = clampi((int64_t)uqo_scale(sum - q[0] * q[1], q[3], q[4]) + q[2], -128, 127);
        }
}

/* uq_mul, qnn.c:111-116: elementwise product of zero-point-shifted operands,
 * one requant, clamp to [q5, q6]. */
static void mul_image(const int8_t *x, const int8_t *b, int8_t *y, uint32_t count, const int32_t *q)
{
    for (uint32_t i = 0; i < count; i++) {
        int32_t prod = ((int32_t)x[i] - q[0]) * ((int32_t)b[i] - q[1]);
        y[i] = clampi((int64_t)uqo_scale(prod, q[3], q[4]) + q[2], q[5], q[6]);
    }
}

/* uq_bmm, qnn.c:117-153: for each of the d0 matrices, z[r][c] =
 * clamp(scale(sum_t (A[r][t] - q0) * (B[t][c] - q1), q3, q4) + q2). q5 = 1
 * reads A as [k][m], q6 = 1 reads B as [n][k]. The reference forms the same
 * exact integer sum from a u8 x i8 product and three correction terms
 * (qnn.c:142); the loader bounds it to int32 (graph.c:189). */
static void bmm_image(const Ten *a, const Ten *b, const Ten *z, const int8_t *x, const int8_t *w, int8_t *y, const int32_t *q)
{
    unsigned batches = z->d[0], m = z->d[1], n = z->d[2], k = a->d[q[5] ? 1 : 2];
    for (unsigned h = 0; h < batches; h++) {
        const int8_t *xa = x + (size_t)h * m * k, *wb = w + (size_t)h * k * n;
        for (unsigned r = 0; r < m; r++)
            for (unsigned c = 0; c < n; c++) {
                int64_t acc = 0;
                for (unsigned t = 0; t < k; t++) {
                    int av = xa[q[5] ? (size_t)t * m + r : (size_t)r * k + t];
                    int bv = wb[q[6] ? (size_t)c * k + t : (size_t)t * n + c];
                    acc += (int64_t)(av - q[0]) * (bv - q[1]);
                }
                y[((size_t)h * m + r) * n + c] = clampi((int64_t)uqo_scale((int32_t)acc, q[3], q[4]) + q[2], -128, 127);
            }
    }
    (void)b;
}

/* Code 17, qnn.c:1082-1087: per row of q[16] values, e_j = table[max - x_j]
 * (table = q[20..275], Q24 with table[0] = 2^24), y_j = round(256 e_j / S)
 * with S = sum e_j (64-bit, halves rounded up), minus 128, clamped to
 * [q14, q15]. */
static void softmax_table_image(const int8_t *x, int8_t *y, uint32_t bytes, const int32_t *q)
{
    uint32_t width = (uint32_t)q[16];
    const int32_t *table = q + HEAD;
    for (uint32_t base = 0; base < bytes; base += width) {
        int mx = -128;
        for (uint32_t j = 0; j < width; j++) if (x[base + j] > mx) mx = x[base + j];
        uint64_t sum = 0;
        for (uint32_t j = 0; j < width; j++) sum += (uint32_t)table[mx - x[base + j]];
        for (uint32_t j = 0; j < width; j++) {
            uint64_t v = (uint64_t)(uint32_t)table[mx - x[base + j]] * 256;
            int32_t r = (int32_t)((v + sum / 2) / sum) - 128;
            y[base + j] = clampi(r, q[14], q[15]);
        }
    }
}

/* Rounding doubling high multiply, qnn.c:61-70 with shift 0. */
static int32_t high_mul(int32_t a, int32_t b) { return uqo_scale(a, b, 0); }

/* uq_softmax_exact, qnn.c:87-107. Per row of q[0] values: e_j = lut[max - x_j]
 * (Q0.31 exponentials), S = sum of e_j rounded to Q12, 1/S by a fixed-point
 * Newton-Raphson iteration on S normalised to [1, 2) (gemmlowp's
 * one_over_one_plus_x_for_x_in_0_1: start 48/17 - 32/17 x, three steps
 * r += r (1 - x r)), then y_j = round(r e_j / 2^exponent) - 128, 127 on
 * overflow. */
static void softmax_image(const int8_t *x, int8_t *y, uint32_t bytes, const int32_t *q)
{
    uint32_t width = (uint32_t)q[0];
    const int32_t *lut = q + 1;
    for (uint32_t base = 0; base < bytes; base += width) {
        int mx = -128;
        for (uint32_t j = 0; j < width; j++) if (x[base + j] > mx) mx = x[base + j];
        uint32_t sum = 0;
        for (uint32_t j = 0; j < width; j++) sum += ((uint32_t)lut[mx - x[base + j]] + 2048u) >> 12;
        unsigned lead = 0;
        while (!(sum & (0x80000000u >> lead))) lead++;
        unsigned exponent = 35 - lead;
        uint32_t frac = (sum << lead) - 0x80000000u;              /* (S / 2^(31-lead) - 1) in Q0.32 */
        int32_t half = (int32_t)(((uint64_t)frac + 0x80000000u) >> 1); /* (1 + frac) / 2 in Q0.31 */
        int32_t r = 1515870810 + high_mul(half, -1010580540);     /* 48/17 - 32/17 * half, Q2.29 */
        for (int it = 0; it < 3; it++) {
            int32_t err = 536870912 - high_mul(half, r);         /* 1 - half * r, Q2.29 */
            r += high_mul(r, err) * 4;
        }
        int64_t r2 = (int64_t)r * 2;
        r = r2 > 2147483647 ? 2147483647 : (int32_t)r2;
        for (uint32_t j = 0; j < width; j++) {
            uint32_t v = (uint32_t)high_mul(r, lut[mx - x[base + j]]);
            uint32_t rounded = exponent >= 32 ? 0 : (v + (1u << (exponent - 1))) >> exponent;
            y[base + j] = (int8_t)(rounded > 255 ? 127 : (int)rounded - 128);
        }
    }
}

/* Code 10, graph.c:374-390: z[i0..] = a[...] with z->d[d] = a->d[p[d]], for
 * any element width (the two float NHWC/NCHW cases there are instances of
 * the same permutation). */
static void transpose_image(const Ten *a, const Ten *z, const uint8_t *x, uint8_t *y, const uint32_t *perm)
{
    unsigned w = a->type == 1 || a->type == 4 ? 4 : 1, rank = a->rank;
    size_t astride[4], count = 1;
    size_t acc = 1;
    for (int d = (int)rank - 1; d >= 0; d--) { astride[d] = acc; acc *= a->d[d]; }
    for (unsigned d = 0; d < rank; d++) count *= z->d[d];
    for (size_t e = 0; e < count; e++) {
        size_t rem = e, src = 0;
        for (int d = (int)rank - 1; d >= 0; d--) {
            size_t idx = rem % z->d[d];
            rem /= z->d[d];
            src += idx * astride[perm[d]];
        }
        memcpy(y + e * w, x + src * w, w);
    }
}

int uqo_run(const void *plan, uint32_t len, const void *input, uint32_t images,
            void *output, uint32_t snap_tensor, void *snap_out)
{
    const uint8_t *p = plan;
    Hdr h;
    if (!plan || len < sizeof h) return 10;
    memcpy(&h, p, sizeof h);
    if (h.magic != 0x55474e31u || h.nt == 0 || h.nt > 1024 || h.no == 0 || h.no > 512 || h.input >= h.nt || h.output >= h.nt) return 11;
    size_t meta = sizeof h + (size_t)h.nt * sizeof(Ten) + (size_t)h.no * sizeof(Op);
    if (len != meta + h.arena_bytes) return 12;
    Ten *ts = malloc(h.nt * sizeof(Ten));
    Op *ops = malloc(h.no * sizeof(Op));
    memcpy(ts, p + sizeof h, h.nt * sizeof(Ten));
    memcpy(ops, p + sizeof h + h.nt * sizeof(Ten), h.no * sizeof(Op));
    const uint8_t *arena = p + meta;
    int rc = 0;
    uint8_t **buf = calloc(h.nt, sizeof(uint8_t *));
    for (uint32_t i = 0; i < h.nt; i++) {
        if ((uint64_t)ts[i].offset + ts[i].bytes > h.arena_bytes) { rc = 13; goto done; }
        if (!ts[i].flags) buf[i] = calloc((size_t)images * ts[i].bytes + 1, 1);
    }
    memcpy(buf[h.input], input, (size_t)images * ts[h.input].bytes);
#define CONST(t) (arena + ts[t].offset)
    /* Image j of tensor t: activations are stacked, constants are shared. */
#define AT(t, j) (ts[t].flags ? CONST(t) : buf[t] + (size_t)(j) * ts[t].bytes)
    for (uint32_t i = 0; i < h.no && !rc; i++) {
        const Op *o = ops + i;
        const Ten *a = ts + o->a, *b = ts + o->b, *z = ts + o->out;
        if (z->flags) { rc = 15; break; }
        for (uint32_t j = 0; j < images && !rc; j++) {
            const int8_t *ap = (const int8_t *)AT(o->a, j), *bp = (const int8_t *)AT(o->b, j);
            int8_t *zp = (int8_t *)AT(o->out, j);
            switch (o->code) {
            case 17: softmax_table_image(ap, zp, a->bytes, (const int32_t *)CONST(o->p[0])); break;
            case 14: case 15: case 16: {
                const int32_t *q = (const int32_t *)CONST(o->p[0]);
                const uint8_t *lut = (o->code != 16 && o->p[1]) ? CONST(o->p[1] - 1) : NULL;
                if (o->code == 14) conv_image(a, ap, bp, zp, q, lut);
                else window_image(o->code, a, ap, bp, zp, q, lut);
                break;
            }
            case 18: add_image(ap, bp, zp, z->bytes, (const int32_t *)CONST(o->p[0])); break;
            case 24: mean_image(ap, zp, a->d[0], a->d[3], (const int32_t *)bp); break;
            case 5: memcpy(zp, ap, z->bytes); break;                                   /* graph.c:408 */
            case 10: transpose_image(a, z, (const uint8_t *)ap, (uint8_t *)zp, o->p); break;
            case 25: mul_image(ap, bp, zp, z->bytes, (const int32_t *)CONST(o->p[0])); break;
            case 27: bmm_image(a, b, z, ap, bp, zp, (const int32_t *)CONST(o->p[0])); break;
            case 28: softmax_image(ap, zp, z->bytes, (const int32_t *)bp); break;
            case 22: {                                                                 /* graph.c:331-341 */
                const uint8_t *table = (const uint8_t *)bp;
                unsigned flip = a->type == 3 ? 128 : 0;
                for (uint32_t k = 0; k < a->bytes; k++) zp[k] = (int8_t)table[(uint8_t)ap[k] ^ flip];
                break;
            }
            case 20: {                                                                 /* graph.c:347-355 */
                unsigned outer = 1, inner = 1, axis = o->p[0];
                for (unsigned d = 0; d < axis; d++) outer *= a->d[d];
                for (unsigned d = axis + 1; d < a->rank; d++) inner *= a->d[d];
                size_t ac = (size_t)a->d[axis] * inner, bc = (size_t)b->d[axis] * inner;
                for (unsigned r = 0; r < outer; r++) {
                    memcpy(zp + r * (ac + bc), ap + r * ac, ac);
                    memcpy(zp + r * (ac + bc) + ac, bp + r * bc, bc);
                }
                break;
            }
            case 21: {                                                                 /* graph.c:342-346 */
                const uint32_t *q = (const uint32_t *)bp;
                size_t c = a->d[3], stride = (size_t)a->d[1] * a->d[2] * c, off = 0;
                for (unsigned n = 0; n < a->d[0]; n++)
                    for (unsigned yy = 0; yy < z->d[1]; yy++)
                        for (unsigned xx = 0; xx < z->d[2]; xx++, off += c)
                            memcpy(zp + off, ap + n * stride + q[yy] + q[z->d[1] + xx], c);
                break;
            }
            case 23: {                                                                 /* graph.c:318-330 */
                const int32_t *q = (const int32_t *)bp;
                memset(zp, (int8_t)(int32_t)o->p[0], z->bytes);
                for (unsigned n = 0; n < a->d[0]; n++)
                    for (unsigned yy = 0; yy < a->d[1]; yy++)
                        for (unsigned xx = 0; xx < a->d[2]; xx++) {
                            size_t dst = ((((size_t)n + q[0]) * z->d[1] + yy + q[2]) * z->d[2] + xx + q[4]) * z->d[3] + q[6];
                            memcpy(zp + dst, ap + (((size_t)n * a->d[1] + yy) * a->d[2] + xx) * a->d[3], a->d[3]);
                        }
                break;
            }
            case 26: {                                                                 /* graph.c:306-313 */
                size_t stride[4] = {0}, step = 1, off = 0;
                unsigned idx[4] = {0}, last = a->rank - 1, span = z->d[last];
                for (int d = (int)a->rank - 1; d >= 0; d--) { stride[d] = step; off += o->p[d] * step; step *= a->d[d]; }
                for (size_t k = 0; k < z->bytes; k += span) {
                    memcpy(zp + k, ap + off, span);
                    for (int d = (int)last - 1; d >= 0; d--) {
                        off += stride[d];
                        if (++idx[d] < z->d[d]) break;
                        off -= idx[d] * stride[d];
                        idx[d] = 0;
                    }
                }
                break;
            }
            case 19: {                                                                 /* graph.c:356-360 */
                const uint32_t *list = (const uint32_t *)bp;
                size_t off = 0;
                for (unsigned k = 0; k < b->bytes / 4; k++) {
                    const Ten *t = ts + list[k];
                    memcpy(zp + off, AT(list[k], j), t->bytes);
                    off += t->bytes;
                }
                break;
            }
            default: rc = 19; /* outside the INT8 vision path restated here */
            }
        }
    }
    if (!rc) {
        for (uint32_t j = 0; j < images; j++)
            memcpy((uint8_t *)output + (size_t)j * ts[h.output].bytes, AT(h.output, j), ts[h.output].bytes);
        if (snap_tensor < h.nt && snap_out) {
            if (ts[snap_tensor].flags) memcpy(snap_out, CONST(snap_tensor), ts[snap_tensor].bytes);
            else memcpy(snap_out, buf[snap_tensor], (size_t)images * ts[snap_tensor].bytes);
        }
    }
done:
    for (uint32_t i = 0; i < h.nt; i++) free(buf[i]);
    free(buf); free(ts); free(ops);
    return rc;
}
