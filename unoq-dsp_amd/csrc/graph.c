/* Plain-C graph host of libuq_hip.so: plan validation, load-time preparation
 * of device tables, and an in-order executor that enqueues gfx950 kernels
 * through the thin C ABI of uqk.h.
 *
 * The plan format, the validation rules and their error codes are the
 * reference's interface (runtime/graph.c:50-262, runtime/qnn.c:209-252), so a
 * plan is accepted or rejected here exactly as the reference loader would,
 * with the same code; the checks run in the reference's order because the
 * first failing check decides the code. Execution differs by design: every
 * activation tensor owns a device buffer sized for a whole batch of stacked
 * images, constants are uploaded once, and each op is one kernel launch (or a
 * device copy) on one HIP stream.
 */
#include "uq_graph.h"
#include "uqk.h"
#include <stdlib.h>
#include <string.h>

#define UG_MAGIC 0x55474e31u
#define UG_MAX_T 1024u
#define UG_MAX_OP 512u
#define UG_MAX_PLAN (17u * 1024u * 1024u)
#define UG_ARENA (16u * 1024u * 1024u)
#define UG_MAX_WORK 2000000000ULL
#define UQ_HEAD 20
#define UQ_MAX_K 8192
#define UQ_MAX_C 2048

/* Record layouts of graph.h:15-17 (the plan ABI). */
typedef struct { uint32_t magic, version, nt, no, arena_bytes, input, output, reserved; } Header;
typedef struct { uint32_t offset, bytes, type, rank, d[4], flags, reserved[3]; } Tensor;
typedef struct { uint32_t code, a, b, out, p[4]; } Op;

/* A fused group (see find_groups): an inverted bottleneck run by one launch
 * (kind 0), a conv whose residual add runs in its epilogue (kind 1), a stem
 * conv, the 3x3 stride-2 conv over its output and optionally the 1x1 after
 * that (kind 2), a banded universal inverted bottleneck (kind 3), a 1x1
 * conv and the mean over its whole output (kind 4), a concat whose
 * operands' table lookups, inner concats and slices run inside its launch
 * (kind 5, find_gather), or a conv whose output only feeds a table lookup,
 * run with the two tables composed (kind 6, find_conv_lut). */
typedef struct {
    int kind;
    UQKIb desc;
    UQKUib ub;                       /* kind 3 */
    UQKAdd add;                      /* kind 1; add.res is set per launch */
    UQKMean mean;                    /* kind 4 */
    UQKSpatial sp;                   /* kind 6: the conv with the composed post table */
    /* kind 5: segments of the output rows (source tensor, byte offset in its
     * rows, bytes per row, table tensor or none, index flip) and the earlier
     * ops the launch stands in for, in plan order */
    uint32_t nseg, seg_src[4], seg_off[4], seg_width[4], seg_lut[4], seg_has_lut[4], seg_flip[4];
    uint32_t nelide, elide[10];
    uint32_t res;                    /* kind 1: tensor of the add's other operand */
    uint32_t first, nops, in, out;
    const uint8_t *last_in;          /* input pointer of the last fused launch */
    uint32_t last_images;            /* images of that launch, 0 if not run fused since */
    int last_ext;                    /* that launch read a caller buffer: inner tensors cannot be rebuilt */
} Group;

static struct {
    int ready, profile_enabled, stream_active, vision_only;
    Header h;
    Tensor ts[UG_MAX_T];
    Op ops[UG_MAX_OP];
    uint8_t *arena;              /* host copy of the plan arena */
    uint8_t *dev_arena;          /* device copy of the plan arena (constants) */
    uint8_t *dev_prep;           /* device pool of prepared per-op tables */
    uint8_t *act[UG_MAX_T];      /* device activation buffers, capacity images each */
    uint8_t *ptr[UG_MAX_T];      /* per-run tensor addresses */
    uint8_t bcast[UG_MAX_T];     /* constant read in a per-image operand slot: replicated per image */
    uint32_t capacity, last_images;
    UQKSpatial sp[UG_MAX_OP];
    uint64_t ticks[UG_MAX_OP + 2];
    uint64_t generation;         /* bumped whenever device buffers move (graphs must be re-captured) */
    /* Fused inverted-bottleneck groups: fuse_at[i] = group index + 1 when op i
     * starts one. A group's inner tensors reach HBM only when a snapshot asks
     * for them (materialize_group). */
    uint16_t fuse_at[UG_MAX_OP];
    uint16_t fuse_of_tensor[UG_MAX_T];   /* group index + 1 of an inner tensor */
    uint16_t elide[UG_MAX_OP];           /* group index + 1 of a gather (kind 5) that runs op i in its launch */
    int pack_rows;                       /* UQ_FUSE_GATHER=0 at load: a pack (op 19) copies tensor by tensor */
    uint8_t ext[UG_MAX_T];               /* G.ptr[t] is a caller buffer this run */
    /* fwd[i]: op i's output is used only by op i + 1, a reshape (code 5) to
     * the graph output; when that output is a caller buffer, op i writes
     * its bytes there directly and the reshape moves nothing. */
    uint8_t fwd[UG_MAX_OP];
    int slices;                          /* UQ_STREAMS at load: image slices of a batch, 0 = default */
    int split_open, split_n;             /* the last split batch's side stream is not joined yet */
    uint32_t split_images;               /* ... its image count, input and output addresses */
    const void *split_in, *split_out;
    uint32_t ngroups;
    Group groups[UG_MAX_OP / 2 + 1];
    uint8_t *pipe_in[2], *pipe_out[2]; /* device chunk buffers of the pipelined batch */
    uint64_t pipe_in_bytes, pipe_out_bytes;
    /* Activation snapshots unavailable: the last run kept its activations in
     * the shared scratch (ug_enqueue_device_noalloc), or a caller buffer it
     * was bound to has been freed. Cleared when a run binds pointers anew. */
    int snap_void;
    int prof_pending;                    /* a profiled batch is enqueued and its times not yet added */
    uint64_t scratch_generation;         /* generation and images of the scratch layout whose */
    uint32_t scratch_images;             /* ... per-image constant copies are in place */
} G;

static uint32_t width(uint32_t t) { return t == 1 || t == 4 ? 4 : t == 2 || t == 3 ? 1 : 0; }

static int same(const Tensor *a, const Tensor *b)
{
    if (a->type != b->type || a->rank != b->rank) return 0;
    for (uint32_t i = 0; i < a->rank; i++)
        if (a->d[i] != b->d[i]) return 0;
    return 1;
}

/* Scalar, last-axis vector, or equal shape (graph.c:33-40). */
static int broadcast(const Tensor *a, const Tensor *b)
{
    if (a->type != b->type || b->rank > a->rank) return 0;
    for (uint32_t i = 0; i < b->rank; i++)
        if (b->d[i] != 1 && b->d[i] != a->d[a->rank - b->rank + i]) return 0;
    if (b->bytes == width(b->type)) return 1;
    if (b->bytes == a->d[a->rank - 1] * width(b->type)) {
        for (uint32_t i = 0; i + 1 < b->rank; i++)
            if (b->d[i] != 1) return 0;
        return 1;
    }
    return same(a, b);
}

/* Host twin of the device requantiser, used only by the load-time bound
 * proof (qnn.c:246-249 needs the scaled endpoints). */
static int32_t scale_host(int32_t v, int32_t m, int shift)
{
    if (shift > 0) v = (int32_t)((uint32_t)v << shift);
    int64_t p = (int64_t)v * m;
    int32_t h = (int32_t)((p + ((int64_t)1 << 30)) >> 31);
    if (shift >= 0) return h;
    unsigned s = (unsigned)-shift;
    uint32_t mask = ((uint32_t)1 << s) - 1;
    return (h >> s) + (((uint32_t)h & mask) > ((mask >> 1) + (uint32_t)(h < 0)));
}

static int packed_weight(const int8_t *w, uint32_t n, uint32_t k, uint32_t kp)
{
    return w[(size_t)(n / 4) * kp * 4 + (size_t)(k / 8) * 32 + (n % 4) * 8 + k % 8];
}

/* Spatial-op rules of qnn.c:209-252 (codes 14-17), including the per-channel
 * int32 bound proof over unsigned inputs in [0, 255]. */
static int check_spatial(const Op *o, const Tensor *a, const Tensor *b, const Tensor *z, const Tensor *t,
                         const int32_t *q, const int8_t *w, uint64_t *work)
{
    if (a->type != 3 || z->type != 3 || !t->flags || t->type != 4 || t->bytes < UQ_HEAD * 4 ||
        ((o->code != 14 && o->code != 15) && o->p[1]) || o->p[2] || o->p[3])
        return 18;
    if (q[12] < -128 || q[12] > 127 || q[13] < -128 || q[13] > 127 || q[14] < -128 || q[15] > 127 || q[14] > q[15] ||
        q[19] < 0 || q[19] > 1)
        return 18;
    if (o->code == 17) {
        if (q[13] != -128 || q[14] != -128 || q[15] != 127 || a->rank != z->rank || a->bytes != z->bytes || !a->rank ||
            q[16] != (int32_t)a->d[a->rank - 1] || q[16] < 1 || q[16] > UQ_MAX_C || t->bytes != (UQ_HEAD + 256) * 4)
            return 18;
        for (unsigned i = 0; i < 256; i++)
            if (q[UQ_HEAD + i] < 0 || q[UQ_HEAD + i] > (1 << 24)) return 18;
        for (unsigned d = 0; d < a->rank; d++)
            if (a->d[d] != z->d[d]) return 18;
        if (q[UQ_HEAD] != (1 << 24)) return 18;
        *work += a->bytes;
        return 0;
    }
    if (a->rank != 4 || z->rank != 4 || a->d[0] != z->d[0] || q[16] != (int32_t)a->d[3] || q[17] != (int32_t)z->d[3] ||
        q[16] < 1 || q[16] > UQ_MAX_C || q[17] < 1 || q[17] > UQ_MAX_C)
        return 18;
    for (unsigned i = 0; i < 6; i++)
        if (q[i] < 1 || q[i] > 4096) return 18;
    for (unsigned i = 6; i < 12; i++)
        if (q[i] < 0 || q[i] > 4096) return 18;
    int64_t hh = (int64_t)a->d[1] + q[6] + q[8] - (int64_t)(q[0] - 1) * q[4] - 1;
    int64_t ww = (int64_t)a->d[2] + q[7] + q[9] - (int64_t)(q[1] - 1) * q[5] - 1;
    if (hh < 0 || ww < 0 || hh / q[2] + 1 != q[10] || ww / q[3] + 1 != q[11] || q[10] != (int32_t)z->d[1] ||
        q[11] != (int32_t)z->d[2])
        return 18;
    uint64_t area = (uint64_t)q[0] * q[1], rows = (uint64_t)z->d[0] * z->d[1] * z->d[2];
    if (o->code == 16) {
        if (q[16] != q[17] || q[12] != q[13] || q[4] != 1 || q[5] != 1 || area > 8192 || t->bytes != UQ_HEAD * 4) return 18;
        if (q[6] >= q[0] || q[7] >= q[1] || (q[10] - 1) * (int64_t)q[2] - q[6] >= a->d[1] ||
            (q[11] - 1) * (int64_t)q[3] - q[7] >= a->d[2])
            return 18;
        *work += rows * area * q[16];
        return 0;
    }
    uint64_t k = area * (o->code == 15 ? 1 : (uint64_t)q[16]);
    if (k > UQ_MAX_K || q[18] != (int32_t)((k + 7) & ~7ULL) || !b->flags || b->type != 3 ||
        t->bytes != (uint32_t)(UQ_HEAD + 3 * q[17]) * 4)
        return 18;
    if (o->code == 15) {
        if (q[16] != q[17] || b->bytes != area * q[17]) return 18;
    } else if (b->bytes != (uint32_t)((q[17] + 3) & ~3) * q[18])
        return 18;
    const int oc = q[17];
    for (int c = 0; c < oc; c++) {
        int shift = q[UQ_HEAD + 2 * oc + c], m = q[UQ_HEAD + oc + c];
        if (m < 0 || shift < -31 || shift > 15) return 18;
        int64_t lo = q[UQ_HEAD + c], hi = lo;
        unsigned terms = o->code == 15 ? (unsigned)k : (unsigned)q[18];
        for (unsigned j = 0; j < terms; j++) {
            int v = o->code == 15 ? w[j * oc + c] : packed_weight(w, (uint32_t)c, j, terms);
            if (v < 0) lo += 255 * v;
            else hi += 255 * v;
        }
        int64_t factor = (int64_t)1 << (shift > 0 ? shift : 0);
        if (lo * factor < INT32_MIN || hi * factor > INT32_MAX) return 18;
        if ((int64_t)scale_host((int32_t)lo, m, shift) + q[13] < INT32_MIN ||
            (int64_t)scale_host((int32_t)hi, m, shift) + q[13] > INT32_MAX)
            return 18;
    }
    *work += rows * k * q[17];
    return 0;
}

/* Structural validation of a whole plan: graph.c:50-216. Fills G.h/ts/ops. */
static int validate(const uint8_t *p, uint32_t len)
{
    Header *h = &G.h;
    if (!p || len < sizeof(Header)) return 10;
    memcpy(h, p, sizeof(Header));
    if (h->magic != UG_MAGIC || h->version < 1 || h->version > 3 || !h->nt || h->nt > UG_MAX_T || !h->no ||
        h->no > UG_MAX_OP || !h->arena_bytes || h->arena_bytes > UG_ARENA || h->input >= h->nt || h->output >= h->nt ||
        (h->version == 1 ? h->reserved != 0 : h->reserved > 1))
        return 11;
    uint32_t meta = (uint32_t)sizeof(Header) + h->nt * (uint32_t)sizeof(Tensor) + h->no * (uint32_t)sizeof(Op);
    if (len != meta + h->arena_bytes) return 12;
    memcpy(G.ts, p + sizeof(Header), h->nt * sizeof(Tensor));
    memcpy(G.ops, p + sizeof(Header) + h->nt * sizeof(Tensor), h->no * sizeof(Op));
    const uint8_t *arena = p + meta;
    static unsigned char defined[UG_MAX_T];
    static int birth[UG_MAX_T], death[UG_MAX_T];
    memset(defined, 0, sizeof defined);
    uint32_t end = 0;
    for (uint32_t i = 0; i < h->nt; i++) {
        Tensor *t = G.ts + i;
        uint32_t w = width(t->type);
        uint64_t count = 1;
        if (!w || t->rank > 4 || t->offset % 128 || (h->version < 3 && t->offset < end) || t->offset > h->arena_bytes ||
            t->flags > 1 || t->reserved[0] || t->reserved[1] || t->reserved[2])
            return 13;
        for (uint32_t d = 0; d < t->rank; d++) {
            if (!t->d[d] || t->d[d] > UG_ARENA) return 13;
            count *= t->d[d];
            if (count > UG_ARENA) return 13;
        }
        if (count * w != t->bytes || t->bytes > h->arena_bytes - t->offset) return 13;
        end = t->offset + t->bytes;
        defined[i] = (unsigned char)t->flags;
        birth[i] = -1;
        death[i] = t->flags ? (int)h->no : -1;
    }
    if (G.ts[h->input].flags) return 14;
    defined[h->input] = 1;
    uint64_t work = 0;
    int vision_only = 1, parallel_vision = 0;
    for (uint32_t i = 0; i < h->no; i++) {
        const Op *o = G.ops + i;
        if (o->code != 5 && o->code != 10 && (o->code < 14 || o->code > 28)) vision_only = 0;
        if (o->a >= h->nt || o->b >= h->nt || o->out >= h->nt || !defined[o->a] || defined[o->out]) return 15;
        const Tensor *a = G.ts + o->a, *b = G.ts + o->b, *z = G.ts + o->out;
        const uint32_t c = o->code;
        if (c == 1 || c == 6 || c == 8 || c == 9) {
            int integer = c == 6 || c == 9, packed = c == 8 || c == 9;
            if (packed && h->version < 2) return 16;
            if (!defined[o->b] || !b->flags || a->rank != 2 || b->rank != 2 || z->rank != 2 || a->d[1] != b->d[1] ||
                z->d[0] != a->d[0] || (packed ? ((z->d[1] + 3) / 4 * 4 != b->d[0]) : z->d[1] != b->d[0]))
                return 16;
            if (!integer && (a->type != 1 || b->type != 1 || z->type != 1)) return 16;
            if (integer && (a->type != 2 || b->type != 3 || z->type != 4 || a->d[1] > 8192 || o->p[0] > 255 ||
                            (int32_t)o->p[1] < -128 || (int32_t)o->p[1] > 127))
                return 16;
            if (integer && (o->p[3] != 1 || o->p[2] >= h->nt || !defined[o->p[2]] || !G.ts[o->p[2]].flags ||
                            G.ts[o->p[2]].type != 4 || G.ts[o->p[2]].bytes != z->d[1] * 4))
                return 16;
            if (c == 8 && (o->p[0] > 1 || o->p[1] || o->p[2] || o->p[3])) return 16;
            if (c == 9 && a->d[1] % 8) return 16;
            work += (uint64_t)a->d[0] * a->d[1] * z->d[1];
        } else if (c == 2 || c == 3) {
            if (!defined[o->b] || !same(a, z) || !broadcast(a, b) || (a->type != 1 && a->type != 4)) return 17;
            work += a->bytes / width(a->type);
        } else if (c == 4) {
            if (!same(a, z) || (a->type != 1 && a->type != 4)) return 18;
            work += a->bytes / 4;
        } else if (c == 5) {
            if (a->type != z->type || a->bytes != z->bytes) return 18;
            work += a->bytes;
        } else if (c == 7) {
            if (a->type != 4 || z->type != 1 || a->bytes != z->bytes) return 18;
            work += a->bytes / 4;
        } else if (c == 10) {
            if (a->rank != z->rank || a->type != z->type || a->bytes != z->bytes) return 18;
            unsigned seen = 0;
            for (unsigned d = 0; d < a->rank; d++) {
                unsigned q = o->p[d];
                if (q >= a->rank || (seen & (1u << q)) || z->d[d] != a->d[q]) return 18;
                seen |= 1u << q;
            }
            work += z->bytes;
        } else if (c == 11 || c == 12) {
            if (a->rank != 4 || a->type != 1 || z->type != 1 || !defined[o->b] || !b->flags || b->type != 4 || b->bytes != 48)
                return 18;
            int32_t q[12];
            memcpy(q, arena + b->offset, 48);
            for (unsigned d = 0; d < 6; d++)
                if (q[d] < 1 || q[d] > 4096) return 18;
            for (unsigned d = 6; d < 12; d++)
                if (q[d] < 0 || q[d] > 4096) return 18;
            int64_t hh = (int64_t)a->d[1] + q[6] + q[8] - (q[0] - 1) * (int64_t)q[4] - 1;
            int64_t ww = (int64_t)a->d[2] + q[7] + q[9] - (q[1] - 1) * (int64_t)q[5] - 1;
            if (hh < 0 || ww < 0 || hh / q[2] + 1 != q[10] || ww / q[3] + 1 != q[11]) return 18;
            uint64_t rows = (uint64_t)a->d[0] * q[10] * q[11], k = (uint64_t)q[0] * q[1] * a->d[3];
            if (c == 11) {
                if (z->rank != 2 || z->d[0] != rows || z->d[1] != k) return 18;
            } else if (z->rank != 4 || z->d[0] != a->d[0] || z->d[1] != (uint32_t)q[10] || z->d[2] != (uint32_t)q[11] ||
                       z->d[3] != a->d[3])
                return 18;
            work += rows * k;
        } else if (c == 13) {
            if (!same(a, z) || a->type != 1 || !a->rank) return 18;
            work += a->bytes / 4;
        } else if (c >= 14 && c <= 17) {
            if (h->version < 2 || o->p[0] >= h->nt || !defined[o->p[0]] || !defined[o->b]) return 18;
            const Tensor *t = G.ts + o->p[0];
            int rc = check_spatial(o, a, b, z, t, (const int32_t *)(arena + t->offset), (const int8_t *)(arena + b->offset), &work);
            if (rc) return rc;
            if (o->p[1]) {
                unsigned id = o->p[1] - 1;
                if (id >= h->nt || !G.ts[id].flags || G.ts[id].type != 2 || G.ts[id].bytes != 256) return 18;
                death[id] = (int)i;
                work += z->bytes;
            }
            if ((c == 14 || c == 15) && z->bytes >= 2048 && (uint64_t)z->d[0] * z->d[1] * z->d[2] >= 8) parallel_vision = 1;
        } else if (c == 18) {
            if (h->version < 2 || !defined[o->b] || a->type != 3 || !same(a, b) || !same(a, z) || o->p[0] >= h->nt || o->p[1] ||
                o->p[2] || o->p[3])
                return 18;
            const Tensor *t = G.ts + o->p[0];
            if (!t->flags || t->type != 4 || t->bytes != 520 * 4) return 18;
            const int32_t *q = (const int32_t *)(arena + t->offset);
            if (q[0] < 0 || q[1] < -31 || q[1] > 0 || q[2] < -128 || q[2] > 127 || q[3] < -128 || q[4] > 127 || q[3] > q[4] ||
                q[5] || q[6] || q[7])
                return 18;
            for (unsigned j = 8; j < 520; j++)
                if (q[j] < -267386880 || q[j] > 267386880) return 18;
            work += z->bytes;
        } else if (c == 19) {
            if (h->version < 2 || !b->flags || b->type != 4 || !b->bytes || b->bytes > 32 * 4 || b->bytes % 4 || z->type != 3 ||
                z->rank != 1 || o->p[0] || o->p[1] || o->p[2] || o->p[3])
                return 18;
            const uint32_t *list = (const uint32_t *)(arena + b->offset);
            uint64_t total = 0;
            if (list[0] != o->a) return 18;
            for (unsigned j = 0; j < b->bytes / 4; j++) {
                unsigned id = list[j];
                if (id >= h->nt || !defined[id] || (G.ts[id].type != 2 && G.ts[id].type != 3)) return 18;
                total += G.ts[id].bytes;
                death[id] = (int)i;
            }
            if (total != z->bytes) return 18;
            work += total;
        } else if (c == 20) {
            unsigned axis = o->p[0];
            if (h->version < 2 || !defined[o->b] || a->type != 3 || b->type != 3 || z->type != 3 || a->rank != b->rank ||
                a->rank != z->rank || axis >= a->rank || o->p[1] || o->p[2] || o->p[3])
                return 18;
            for (unsigned d = 0; d < a->rank; d++) {
                if (d == axis) {
                    if ((uint64_t)a->d[d] + b->d[d] != z->d[d]) return 18;
                } else if (a->d[d] != b->d[d] || a->d[d] != z->d[d])
                    return 18;
            }
            work += z->bytes;
        } else if (c == 21) {
            if (h->version < 2 || a->type != 3 || z->type != 3 || a->rank != 4 || z->rank != 4 || a->d[0] != z->d[0] ||
                a->d[3] != z->d[3] || !b->flags || b->type != 4 || b->bytes != (z->d[1] + z->d[2]) * 4 || o->p[0] || o->p[1] ||
                o->p[2] || o->p[3])
                return 18;
            const uint32_t *q = (const uint32_t *)(arena + b->offset);
            uint32_t row = a->d[2] * a->d[3], batch = a->d[1] * row;
            for (unsigned d = 0; d < z->d[1]; d++)
                if (q[d] >= batch || q[d] % row) return 18;
            for (unsigned d = 0; d < z->d[2]; d++)
                if (q[z->d[1] + d] >= row || q[z->d[1] + d] % a->d[3]) return 18;
            work += z->bytes;
        } else if (c == 22) {
            if (h->version < 2 || (a->type != 2 && a->type != 3) || (z->type != 2 && z->type != 3) || a->rank != z->rank ||
                a->bytes != z->bytes || !b->flags || b->type != 2 || b->bytes != 256 || o->p[0] || o->p[1] || o->p[2] || o->p[3])
                return 18;
            for (unsigned d = 0; d < a->rank; d++)
                if (a->d[d] != z->d[d]) return 18;
            work += z->bytes;
        } else if (c == 23) {
            if (h->version < 2 || a->type != 3 || z->type != 3 || a->rank != 4 || z->rank != 4 || !b->flags || b->type != 4 ||
                b->bytes != 32 || (int32_t)o->p[0] < -128 || (int32_t)o->p[0] > 127 || o->p[1] || o->p[2] || o->p[3])
                return 18;
            const int32_t *q = (const int32_t *)(arena + b->offset);
            for (unsigned d = 0; d < 4; d++)
                if (q[d * 2] < 0 || q[d * 2] > 4096 || q[d * 2 + 1] < 0 || q[d * 2 + 1] > 4096 ||
                    (uint64_t)a->d[d] + q[d * 2] + q[d * 2 + 1] != z->d[d])
                    return 18;
            work += z->bytes;
        } else if (c == 24) {
            if (h->version < 2 || a->type != 3 || z->type != 3 || a->rank != 4 || (z->rank != 2 && z->rank != 4) || !b->flags ||
                b->type != 4 || b->bytes != 20 || o->p[0] || o->p[1] || o->p[2] || o->p[3])
                return 18;
            if (z->d[0] != a->d[0] || z->d[z->rank - 1] != a->d[3] || (z->rank == 4 && (z->d[1] != 1 || z->d[2] != 1))) return 18;
            const int32_t *q = (const int32_t *)(arena + b->offset);
            if (q[0] < 1 || (uint64_t)a->d[1] * a->d[2] != (uint32_t)q[0] || q[1] < -128 || q[1] > 127 || q[2] < -128 ||
                q[2] > 127 || q[3] < 0 || q[4] < -31 || q[4] > 30)
                return 18;
            uint64_t bound = (uint64_t)q[0] * (q[1] >= 0 ? 128 + q[1] : 127 - q[1]);
            if ((bound << (q[4] > 0 ? q[4] : 0)) > 2147483520u) return 18;
            work += a->bytes;
        } else if (c == 25 || c == 27) {
            if (h->version < 2 || a->type != 3 || b->type != 3 || z->type != 3 || !defined[o->b] || o->p[0] >= h->nt || o->p[1] ||
                o->p[2] || o->p[3])
                return 18;
            const Tensor *t = G.ts + o->p[0];
            if (!t->flags || t->type != 4 || t->bytes != 28) return 18;
            const int32_t *q = (const int32_t *)(arena + t->offset);
            for (unsigned j = 0; j < 3; j++)
                if (q[j] < -128 || q[j] > 127) return 18;
            if (q[3] < 0 || q[4] < -31 || q[4] > 15) return 18;
            uint64_t k = 1;
            if (c == 25) {
                if (!same(a, b) || !same(a, z) || q[5] < -128 || q[6] > 127 || q[5] > q[6]) return 18;
                work += z->bytes;
            } else {
                if (a->rank != 3 || b->rank != 3 || z->rank != 3 || q[5] < 0 || q[5] > 1 || q[6] < 0 || q[6] > 1 ||
                    a->d[0] != b->d[0] || a->d[0] != z->d[0])
                    return 18;
                unsigned m = a->d[q[5] ? 2 : 1], n = b->d[q[6] ? 1 : 2];
                k = a->d[q[5] ? 1 : 2];
                if (k != b->d[q[6] ? 2 : 1] || k > 8192 || n > 2048 || z->d[1] != m || z->d[2] != n) return 18;
                work += (uint64_t)z->bytes * k;
            }
            if (k * 65025 * (1ULL << (q[4] > 0 ? q[4] : 0)) > 2147483520u) return 18;
        } else if (c == 26) {
            if (h->version < 2 || a->type != 3 || z->type != 3 || a->rank != z->rank || !a->rank) return 18;
            for (unsigned d = 0; d < 4; d++) {
                if (d >= a->rank) {
                    if (o->p[d]) return 18;
                } else if ((uint64_t)o->p[d] + z->d[d] > a->d[d])
                    return 18;
            }
            work += z->bytes;
        } else if (c == 28) {
            if (h->version < 2 || a->type != 3 || !same(a, z) || !a->rank || a->d[a->rank - 1] > 2048 || !b->flags ||
                b->type != 4 || b->bytes != 257 * 4 || o->p[0] || o->p[1] || o->p[2] || o->p[3])
                return 18;
            const int32_t *q = (const int32_t *)(arena + b->offset);
            if (q[0] != (int32_t)a->d[a->rank - 1] || q[1] != 2147483647) return 18;
            for (unsigned d = 2; d <= 256; d++)
                if (q[d] < 0 || q[d] > q[d - 1]) return 18;
            work += z->bytes;
        } else
            return 19;
        if (work > UG_MAX_WORK) return 20;
        death[o->a] = (int)i;
        death[o->b] = (int)i;
        birth[o->out] = (int)i;
        death[o->out] = (int)i;
        if ((c >= 14 && c <= 18) || c == 25 || c == 27) death[o->p[0]] = (int)i;
        if (c == 6 || c == 9) death[o->p[2]] = (int)i;
        defined[o->out] = 1;
    }
    G.vision_only = vision_only && parallel_vision;
    if (!defined[h->output]) return 21;
    if (h->version == 3) {
        death[h->output] = (int)h->no;
        for (unsigned x = 0; x < h->nt; x++) {
            if (G.ts[x].flags) {
                birth[x] = -1;
                death[x] = (int)h->no;
            }
            if (!defined[x]) return 15;
        }
        for (unsigned x = 0; x < h->nt; x++)
            for (unsigned y = x + 1; y < h->nt; y++) {
                int mem = G.ts[x].offset < G.ts[y].offset + G.ts[y].bytes && G.ts[y].offset < G.ts[x].offset + G.ts[x].bytes;
                int live = birth[x] <= death[y] && birth[y] <= death[x];
                if (mem && live) return 25;
            }
    }
    return 0;
}

/* Codes this library executes on the GPU: the INT8 vision path. */
static int supported(uint32_t code)
{
    switch (code) {
    case 5: case 10: case 14: case 15: case 16: case 17: case 18: case 19: case 20: case 21: case 22: case 23:
    case 24: case 25: case 26: case 27: case 28: return 1;
    default: return 0;
    }
}

static void release_device(void)
{
    for (uint32_t i = 0; i < UG_MAX_T; i++) {
        uqk_free(G.act[i]);
        G.act[i] = NULL;
    }
    uqk_free(G.dev_arena);
    uqk_free(G.dev_prep);
    G.dev_arena = G.dev_prep = NULL;
    for (int k = 0; k < 2; k++) {
        uqk_free(G.pipe_in[k]);
        uqk_free(G.pipe_out[k]);
        G.pipe_in[k] = G.pipe_out[k] = NULL;
    }
    G.pipe_in_bytes = G.pipe_out_bytes = 0;
    G.capacity = 0;
    G.last_images = 0;
    G.generation++;
}

static uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1) / m * m; }

/* N tile count per block (16 channels each): the least padded choice, or the
 * narrowest when each image has only a few output rows (FC-shaped layers,
 * where channel slices are the only source of parallelism). */
static int choose_nt(int oc, uint64_t rows_per_image)
{
    static const int opts[4] = {8, 6, 4, 2};
    if (rows_per_image <= 4) return 2;
    int best = 8, waste = 1 << 30;
    for (int i = 0; i < 4; i++) {
        int bn = 16 * opts[i], pad = (oc + bn - 1) / bn * bn - oc;
        if (pad < waste) { waste = pad; best = opts[i]; }
    }
    return best;
}

typedef struct { size_t w, epi, kmap, post, end; } Layout;

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

/* Kernel configuration of one conv (code 14): K padding, channel tile, and
 * the A-operand source. Spatial convs stage their input rows in LDS when the
 * tile fits in 64 KiB; otherwise lanes gather straight from HBM. */
typedef struct { int K, kpad, nt, oc_pad, mode, table_bytes, icp; } ConvPlan;

static ConvPlan conv_plan(const Op *o)
{
    const int32_t *q = (const int32_t *)(G.arena + G.ts[o->p[0]].offset);
    const Tensor *z = G.ts + o->out;
    ConvPlan c;
    int ic = q[16], oc = q[17];
    c.K = q[0] * q[1] * ic;
    c.icp = ic;
    c.kpad = (int)round_up((uint32_t)c.K, 64);
    c.nt = choose_nt(oc, (uint64_t)z->d[0] * z->d[1] * z->d[2]);
    c.oc_pad = (int)round_up((uint32_t)oc, (uint32_t)(16 * c.nt));
    int pointwise = q[0] == 1 && q[1] == 1 && q[2] == 1 && q[3] == 1 && !q[6] && !q[7] && !q[8] && !q[9];
    UQKSpatial st;
    memset(&st, 0, sizeof st);
    st.iw = (int)G.ts[o->a].d[2]; st.ic = ic; st.kh = q[0]; st.kw = q[1]; st.sh = q[2]; st.sw = q[3];
    st.dh = q[4]; st.dw = q[5]; st.pl = q[7]; st.ow = q[11]; st.oc = oc;
    if (G.ts[o->a].rank == 4 && uqk_conv_stem_ok(&st)) {
        /* Stem form: one 64-byte K step, 16 bytes per kernel row holding
         * that row's kw * IC contiguous input bytes; the channel slice spans
         * the padded OC when that is at most 64. */
        c.mode = UQK_STEM;
        c.K = 64;
        c.kpad = 64;
        int pad16 = (int)round_up((uint32_t)oc, 16);
        c.nt = pad16 <= 16 ? 1 : pad16 <= 32 ? 2 : 4;
        c.oc_pad = (int)round_up((uint32_t)oc, (uint32_t)(16 * c.nt));
        c.table_bytes = 16;
        return c;
    }
    if (pointwise && ic % 16 == 0) {
        c.mode = UQK_PW;
        c.table_bytes = 16;
        return c;
    }
    /* Row-staged modes: 16-byte K slices when IC % 16 == 0, otherwise taps
     * of icp = roundup(IC, 4) bytes (zero weights on the padded channels). */
    int icp = ic % 16 == 0 ? ic : (ic + 3) & ~3;
    int kw4 = q[0] * q[1] * icp;
    int rows_mode = ic % 16 == 0 ? UQK_ROWS16 : kw4 <= UQ_MAX_K ? UQK_ROWS4 : -1;
    if (rows_mode >= 0) {
        UQKSpatial t;
        memset(&t, 0, sizeof t);
        t.ow = q[11]; t.sw = q[3]; t.kh = q[0]; t.kw = q[1]; t.sh = q[2]; t.dh = q[4]; t.dw = q[5];
        t.ic = ic; t.K = kw4; t.nt = c.nt; t.mode = rows_mode;
        if (uqk_conv_rows_ok(&t)) {
            c.mode = rows_mode;
            c.icp = icp;
            c.K = kw4;
            c.kpad = (int)round_up((uint32_t)kw4, 64);
            c.table_bytes = (rows_mode == UQK_ROWS16 ? c.K / 16 : c.K / 4) * 4 + 16;
            return c;
        }
    }
    int group = ic % 16 == 0 ? 16 : ic % 4 == 0 ? 4 : 1;
    c.mode = group == 16 ? UQK_G16 : group == 4 ? UQK_G4 : UQK_G1;
    c.table_bytes = (c.K / group + 1) * 16;
    return c;
}

/* Sizes of one spatial op's prepared tables in the device pool. */
static Layout spatial_layout(const Op *o, size_t at)
{
    const int32_t *q = (const int32_t *)(G.arena + G.ts[o->p[0]].offset);
    Layout L = {at, at, at, at, at};
    int oc = q[17];
    if (o->code == 14) {
        ConvPlan c = conv_plan(o);
        L.w = at;
        L.epi = align256(L.w + (size_t)c.oc_pad * c.kpad);
        L.kmap = align256(L.epi + (size_t)oc * 32);
        L.post = align256(L.kmap + (size_t)c.table_bytes);   /* a composed post table (kind 6) */
        L.end = L.post + 256;
    } else if (o->code == 15) {
        /* Tap words: (taps + 3) / 4 groups for k_dw_tile, kh * 2 rows of one
         * or two words for k_dw_win; room for either. */
        int groups = (q[0] * q[1] + 3) / 4, rows = 2 * q[0];
        L.epi = at;
        L.w = align256(L.epi + (size_t)oc * 32);
        L.end = align256(L.w + (size_t)(groups > rows ? groups : rows) * oc * 4);
    }
    return L;
}

/* Per-channel epilogue record (32 bytes) for the single 64-bit multiply-add
 * form of requantisation used by the kernels. With v = acc + bias (int32,
 * exact by the load-time bound proof), n = max(-shift, 0), T = 31 + n:
 *   scale(v, m, shift) = ((v << max(shift, 0)) * m + c1 - corr) >> T
 *   c1   = 2^30 + (n ? 2^(30+n) : 0)
 *   corr = 2^31 when n > 0 and (v << ls) * m < -2^30, i.e. q < cthr = 2^(30+n)
 * The first rounding (v*m + 2^30) >> 31 and the ties-away rounding shift of
 * qnn.c:61-83 collapse into one floor because floor(floor(x/a)+b)/c) =
 * floor((x + a*b)/(a*c)) for integer b; the correction turns round-half-up
 * into ties-away for negative intermediates (the same identity the
 * reference's signed affine path relies on, qnn.c:284-296). */
static void epilogue_record(int32_t *e, int64_t bias, int32_t m, int32_t shift)
{
    int n = shift < 0 ? -shift : 0;
    int64_t c1 = ((int64_t)1 << 30) + (n ? ((int64_t)1 << (30 + n)) : 0);
    int64_t cthr = n ? ((int64_t)1 << (30 + n)) : INT64_MIN;
    e[0] = (int32_t)(uint32_t)(uint64_t)bias;
    e[1] = m;
    e[2] = shift > 0 ? shift : 0;
    e[3] = 31 + n;
    memcpy(e + 4, &c1, 8);
    memcpy(e + 6, &cthr, 8);
}

/* The conv record of layers whose every shift is in [-22, -1] (T in
 * [32, 53]): c1 also absorbs the corrected bias times m and the output zero
 * point times 2^T, so the kernel's one multiply-add gives the whole affine
 * value q = (acc + bias) * m + c1 + yz * 2^T. Summed mod 2^64: q itself fits
 * in int64 (|v * m| < 2^62, c1 <= 2^30 + 2^52, |yz * 2^T| <= 2^60) and the
 * multiply-add is exact mod 2^64. cthr moves by the same yz * 2^T. */
static void epilogue_record_hi(int32_t *e, int64_t bias, int32_t m, int32_t shift, int32_t yz)
{
    int n = -shift, T = 31 + n;
    uint64_t c1 = ((uint64_t)1 << 30) + ((uint64_t)1 << (30 + n)) + (uint64_t)bias * (uint64_t)(int64_t)m +
                  ((uint64_t)(int64_t)yz << T);
    int64_t cthr = ((int64_t)1 << (30 + n)) + (int64_t)yz * ((int64_t)1 << T);
    e[0] = (int32_t)(uint32_t)(uint64_t)bias;
    e[1] = m;
    e[2] = 0;
    e[3] = T;
    memcpy(e + 4, &c1, 8);
    memcpy(e + 6, &cthr, 8);
}

/* Build one spatial op's descriptor and host-side tables (graph-time work of
 * the reference's prepare step, qnn.c:388-501, re-targeted at the GPU). */
static void prepare_spatial(uint32_t i, const Layout *L, uint8_t *host_pool)
{
    const Op *o = G.ops + i;
    const Tensor *a = G.ts + o->a;
    const int32_t *q = (const int32_t *)(G.arena + G.ts[o->p[0]].offset);
    UQKSpatial *d = G.sp + i;
    memset(d, 0, sizeof *d);
    d->ih = (int32_t)a->d[1]; d->iw = (int32_t)a->d[2]; d->ic = q[16];
    d->oh = q[10]; d->ow = q[11]; d->oc = q[17];
    d->kh = q[0]; d->kw = q[1]; d->sh = q[2]; d->sw = q[3]; d->dh = q[4]; d->dw = q[5];
    d->pt = q[6]; d->pl = q[7];
    d->xz = q[12]; d->yz = q[13]; d->lo = q[14]; d->hi = q[15];
    d->corr = q[14] < q[13];
    d->is_max = o->code == 16 ? q[19] : 0;
    d->vec = d->oc % 16 == 0 ? 16 : d->oc % 4 == 0 ? 4 : 1;
    if (o->code != 16 && o->p[1]) d->lut = G.dev_arena + G.ts[o->p[1] - 1].offset;
    const int oc = q[17];
    const int32_t *bias = q + UQ_HEAD, *mult = bias + oc, *shift = mult + oc;
    d->dwwin = o->code == 15 && uqk_dw_win_lds(d) > 0;
    /* Large-tile GEMM policy (UQ_GEMM=0/1, UQ_GEMM_TILE=0..4 and
     * UQ_GEMM_TPB=1/2, tiles per block, at load time override the automatic
     * choice). */
    const char *ge = getenv("UQ_GEMM"), *gt = getenv("UQ_GEMM_TILE");
    d->gemm = ge && (!strcmp(ge, "0") || !strcmp(ge, "1")) ? atoi(ge) : -1;
    d->gemm_tile = gt && gt[0] >= '0' && gt[0] <= '4' && !gt[1] ? gt[0] - '0' : -1;
    const char *gp = getenv("UQ_GEMM_TPB");
    d->gemm_tpb = gp && (!strcmp(gp, "1") || !strcmp(gp, "2")) ? gp[0] - '0' : 0;
    /* Depthwise kernel (UQ_DW=band, mfma or win at load time overrides the
     * automatic choice). */
    const char *dk = getenv("UQ_DW");
    d->dwk = !dk ? -1 : !strcmp(dk, "band") ? 0 : !strcmp(dk, "mfma") ? 1 : !strcmp(dk, "win") ? 2 : -1;
    /* UQ_DW_ROWS=n at load time: at most n output rows per block of the
     * matrix-core window depthwise (0 or unset: its own choice). */
    const char *dr = getenv("UQ_DW_ROWS");
    d->dw_rows = dr && atoi(dr) > 0 ? atoi(dr) : 0;
    if (o->code == 15) uqk_dw_band_prepare(d);
    d->hi_shift = o->code == 14 || d->dwwin;
    for (int c = 0; c < oc; c++)
        if (shift[c] > -1 || shift[c] < -22) d->hi_shift = 0;
    const int8_t *w = (const int8_t *)(G.arena + G.ts[o->b].offset);
    if (o->code == 14) {
        ConvPlan cp = conv_plan(o);
        int K = cp.K, kp = q[18], kpad = cp.kpad, oc_pad = cp.oc_pad, ic = q[16], icp = cp.icp;
        int Klog = q[0] * q[1] * ic, rowk = q[1] * ic;
        d->K = K; d->kpad = kpad; d->oc_pad = oc_pad; d->nt = cp.nt; d->rb = 2; d->mode = cp.mode;
        int8_t *wt = (int8_t *)host_pool + L->w;
        int32_t *epi = (int32_t *)(host_pool + L->epi);
        int32_t *kmap = (int32_t *)(host_pool + L->kmap);
        memset(wt, 0, (size_t)oc_pad * kpad);
        for (int n = 0; n < oc; n++) {
            int64_t all = 0, tail = 0;
            for (int k = 0; k < kp; k++) {
                int v = packed_weight(w, (uint32_t)n, (uint32_t)k, (uint32_t)kp);
                all += v;
                /* Logical k = (tap, c) lands at tap * icp + c of the device
                 * row; in the stem form at ky * 16 + kx * IC + c. */
                if (k >= Klog) tail += v;
                else if (cp.mode == UQK_STEM) wt[(size_t)n * kpad + (k / rowk) * 16 + k % rowk] = (int8_t)v;
                else wt[(size_t)n * kpad + (k / ic) * icp + k % ic] = (int8_t)v;
            }
            /* u = s + 128 on every column; the K tail holds xz + 128. */
            int64_t b2 = (int64_t)bias[n] + 128 * all + (int64_t)q[12] * tail;
            if (d->hi_shift) epilogue_record_hi(epi + 8 * n, b2, mult[n], shift[n], q[13]);
            else epilogue_record(epi + 8 * n, b2, mult[n], shift[n]);
        }
        if (cp.mode == UQK_ROWS16 || cp.mode == UQK_ROWS4) {
            /* Slice -> byte offset inside the LDS row tile (full-width rows,
             * icp bytes per staged pixel). */
            int step = cp.mode == UQK_ROWS16 ? 16 : 4;
            int cols = (q[11] - 1) * q[3] + (q[1] - 1) * q[5] + 1;
            for (int g = 0; g < K / step; g++) {
                int k = g * step, t = k / icp, c = k % icp, ky = t / q[1], kx = t % q[1];
                kmap[g] = ((ky * q[4]) * cols + kx * q[5]) * icp + c;
            }
        } else if (cp.mode != UQK_PW && cp.mode != UQK_STEM) {
            int group = cp.mode == UQK_G16 ? 16 : cp.mode == UQK_G4 ? 4 : 1;
            for (int g = 0; g < K / group; g++) {
                int k = g * group, t = k / ic, c = k % ic, ky = t / q[1], kx = t % q[1];
                kmap[4 * g + 0] = ky * q[4];
                kmap[4 * g + 1] = kx * q[5];
                kmap[4 * g + 2] = c;
                kmap[4 * g + 3] = 0;
            }
        }
        d->w = G.dev_prep + L->w;
        d->epi = G.dev_prep + L->epi;
        d->kmap = G.dev_prep + L->kmap;
    } else if (o->code == 15) {
        int taps = q[0] * q[1], groups = (taps + 3) / 4;
        int32_t *epi = (int32_t *)(host_pool + L->epi);
        int8_t *wd = (int8_t *)host_pool + L->w;
        const int kh = q[0], kw = q[1], nwk = kw > 4 ? 2 : 1;
        for (int c = 0; c < oc; c++) {
            int64_t all = 0;
            for (int t = 0; t < taps; t++) all += w[t * oc + c];
            if (d->hi_shift) epilogue_record_hi(epi + 8 * c, (int64_t)bias[c] + 128 * all, mult[c], shift[c], q[13]);
            else epilogue_record(epi + 8 * c, (int64_t)bias[c] + 128 * all, mult[c], shift[c]);
            if (d->dwwin) {
                /* Kernel row ky, word k: taps kx = 4k .. 4k + 3 of the row
                 * (zero past kw), at [ky][k][C]. */
                for (int ky = 0; ky < kh; ky++)
                    for (int k = 0; k < nwk; k++)
                        for (int j = 0; j < 4; j++) {
                            int kx = 4 * k + j;
                            wd[(((size_t)ky * nwk + k) * oc + c) * 4 + j] = kx < kw ? w[(ky * kw + kx) * oc + c] : 0;
                        }
            } else {
                /* Four consecutive taps of one channel per 32-bit word, for dot4. */
                for (int g = 0; g < groups; g++)
                    for (int j = 0; j < 4; j++)
                        wd[((size_t)g * oc + c) * 4 + j] = 4 * g + j < taps ? w[(4 * g + j) * oc + c] : 0;
            }
        }
        d->w = G.dev_arena + G.ts[o->b].offset;
        d->wdot = G.dev_prep + L->w;
        d->epi = G.dev_prep + L->epi;
    }
}

static int enqueue_op(uint32_t i, uint32_t images);
static int settle(void);

/* Consumers of each activation tensor (operands a/b of every op, pack lists). */
static void count_users(uint16_t *users)
{
    memset(users, 0, sizeof(uint16_t) * UG_MAX_T);
    for (uint32_t i = 0; i < G.h.no; i++) {
        const Op *o = G.ops + i;
        users[o->a]++;
        if (o->b != o->a) users[o->b]++;
        if (o->code == 19) {
            const Tensor *lt = G.ts + o->b;
            const uint32_t *list = (const uint32_t *)(G.arena + lt->offset);
            for (uint32_t j = 0; j < lt->bytes / 4; j++) users[list[j]]++;
        }
    }
}

static int pointwise_conv(uint32_t i)
{
    const Op *o = G.ops + i;
    return o->code == 14 && G.sp[i].mode == UQK_PW && G.sp[i].kh == 1 && G.sp[i].kw == 1;
}

/* Fusable inverted bottlenecks: a 1x1 conv whose output feeds only a stride-1
 * depthwise (window form, same map size) whose output feeds only a 1x1 conv,
 * optionally followed by an add of that conv's output and the block input.
 * Inner tensors must be single-use activations, not the plan output; the map
 * must be one image per plan image (d0 == 1) and fit one workgroup's LDS.
 *
 * On unless UQ_FUSE_BOTTLENECK=0 at load time: on MobileNetV4-S at batch 256
 * the fused kernel (ib.hip, one image per workgroup) measured 0.487 against
 * 0.491 ms per step for the separate launches; the results are identical
 * either way. */
/* Conv + residual add: a conv run by k_conv whose output is used once, by
 * the next op, an add (op 18) of equal-sized operands; neither the conv
 * output nor anything else but the add's output is observable, so the add
 * can run in the conv's epilogue. */
static int find_conv_add(uint32_t i, const uint16_t *users)
{
    const Op *c = G.ops + i, *ad = G.ops + i + 1;
    if (c->code != 14 || ad->code != 18 || !uqk_conv_add_ok(G.sp + i)) return 0;
    const uint32_t t = c->out;
    if (users[t] != 1 || t == G.h.output || (ad->a != t && ad->b != t) || ad->a == ad->b) return 0;
    const uint32_t res = ad->a == t ? ad->b : ad->a;
    if (G.ts[res].bytes != G.ts[t].bytes || G.ts[ad->out].bytes != G.ts[t].bytes) return 0;
    if (G.ts[res].flags && !G.bcast[res]) return 0;
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 1;
    const int32_t *q = (const int32_t *)(G.arena + G.ts[ad->p[0]].offset);
    g->add.tables = G.dev_arena + G.ts[ad->p[0]].offset + 8 * 4;
    g->add.m = q[0]; g->add.s = q[1]; g->add.yz = q[2]; g->add.lo = q[3]; g->add.hi = q[4];
    g->add.conv_is_a = ad->a == t;
    g->res = res;
    g->first = i;
    g->nops = 2;
    g->in = c->a;
    g->out = ad->out;
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    G.fuse_of_tensor[t] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return 1;
}

/* A 1x1 conv whose output, used by nothing else, is averaged over the whole
 * map by the next op (MobileNet's classifier head) and that fits head.hip.
 * On unless UQ_FUSE_MEAN=0 at load time. */
/* A conv (op 14) whose output, used by nothing else and not the plan's,
 * feeds only the next op, a byte table lookup (op 22): the lookup's table
 * composed with the conv's own post table (or with the identity) becomes the
 * post table of one conv launch (the composition sits in the 256 bytes the
 * conv's device tables reserve for it). YOLO's detection heads. On unless
 * UQ_FUSE_LUT=0 at load time. */
static int find_conv_lut(uint32_t i, const uint16_t *users, uint8_t *pool, const Layout *layouts)
{
    const Op *c = G.ops + i, *l = G.ops + i + 1;
    if (c->code != 14 || l->code != 22 || l->a != c->out) return 0;
    const uint32_t t = c->out;
    if (users[t] != 1 || t == G.h.output || G.ts[t].flags || !G.ts[l->b].flags || G.ts[l->b].bytes < 256 ||
        width(G.ts[t].type) != 1)
        return 0;
    const uint8_t *table = G.arena + G.ts[l->b].offset;
    const uint8_t *own = c->p[1] ? G.arena + G.ts[c->p[1] - 1].offset : NULL;
    const uint32_t flip = G.ts[t].type == 3 ? 128u : 0u;
    uint8_t *post = pool + layouts[i].post;
    /* Index v + 128 of the conv's requantised value v: its output byte is
     * the own table's entry there, else the two's-complement byte of v. */
    for (uint32_t v = 0; v < 256; v++) {
        const uint32_t byte = own ? own[v] : (uint32_t)(uint8_t)(v - 128u);
        post[v] = table[byte ^ flip];
    }
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 6;
    g->sp = G.sp[i];
    g->sp.lut = G.dev_prep + layouts[i].post;
    g->first = i;
    g->nops = 2;
    g->in = c->a;
    g->out = l->out;
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    G.fuse_of_tensor[t] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return 1;
}

static int find_conv_mean(uint32_t i, const uint16_t *users)
{
    const Op *c = G.ops + i, *mn = G.ops + i + 1;
    if (c->code != 14 || mn->code != 24 || mn->a != c->out || !uqk_conv_mean_ok(G.sp + i)) return 0;
    const uint32_t t = c->out;
    if (users[t] != 1 || t == G.h.output || G.ts[t].rank != 4 || G.ts[t].d[0] != 1) return 0;
    const int32_t *q = (const int32_t *)(G.arena + G.ts[mn->b].offset);
    if (q[0] != G.sp[i].oh * G.sp[i].ow || (int)G.ts[t].d[3] != G.sp[i].oc) return 0;
    if (G.ts[mn->out].bytes != (uint32_t)G.sp[i].oc) return 0;
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 4;
    g->mean.xz = q[1]; g->mean.yz = q[2]; g->mean.m = q[3]; g->mean.s = q[4];
    /* UQ_MEAN_PARTS=n at load time: n workgroups per image (0 or unset:
     * automatic). */
    const char *pe = getenv("UQ_MEAN_PARTS");
    g->mean.parts = pe && atoi(pe) > 0 && atoi(pe) <= 8 ? atoi(pe) : 0;
    g->first = i;
    g->nops = 2;
    g->in = c->a;
    g->out = mn->out;
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    G.fuse_of_tensor[t] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return 1;
}

static uint32_t find_bottleneck(uint32_t i, const uint16_t *users)
{
    if (i + 2 >= G.h.no) return 0;
    const Op *e = G.ops + i, *d = G.ops + i + 1, *p = G.ops + i + 2;
    if (!pointwise_conv(i) || d->code != 15 || !pointwise_conv(i + 2)) return 0;
    const Tensor *x = G.ts + e->a;
    const UQKSpatial *se = G.sp + i, *sd = G.sp + i + 1, *sp = G.sp + i + 2;
    if (x->flags || x->rank != 4 || x->d[0] != 1 || e->a == G.h.input) return 0;
    if (d->a != e->out || p->a != d->out || !sd->dwwin || sd->sh != 1 || sd->sw != 1) return 0;
    if (sd->oh != se->oh || sd->ow != se->ow || sd->oc != se->oc || sp->ic != se->oc) return 0;
    if (users[e->out] != 1 || users[d->out] != 1 || e->out == G.h.output || d->out == G.h.output) return 0;
    if (se->ic % 16 || se->oc % 16 || sp->oc % 16) return 0;
    const int P = se->oh * se->ow;
    if (!uqk_ib_lds(P, se->oh, se->ow, se->ic, se->oc, sp->oc, sd->kh, NULL)) return 0;
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    UQKIb *f = &g->desc;
    f->P = P; f->H = se->oh; f->W = se->ow; f->Cin = se->ic; f->Ce = se->oc; f->Cout = sp->oc;
    f->ks = sd->kh; f->pt = sd->pt; f->pl = sd->pl;
    f->we = se->w; f->epi_e = se->epi; f->lut_e = se->lut; f->kpe = se->kpad;
    f->e_mode = (se->hi_shift ? 1 : 0) | (se->corr ? 2 : 0); f->e_yz = se->yz; f->e_lo = se->lo; f->e_hi = se->hi;
    f->dww = sd->wdot; f->epi_d = sd->epi; f->lut_d = sd->lut;
    f->d_mode = (sd->hi_shift ? 1 : 0) | (sd->corr ? 2 : 0); f->d_yz = sd->yz; f->d_lo = sd->lo; f->d_hi = sd->hi;
    f->d_xz = sd->xz;
    f->wp = sp->w; f->epi_p = sp->epi; f->lut_p = sp->lut; f->kpp = sp->kpad;
    f->p_mode = (sp->hi_shift ? 1 : 0) | (sp->corr ? 2 : 0); f->p_yz = sp->yz; f->p_lo = sp->lo; f->p_hi = sp->hi;
    g->first = i;
    g->nops = 3;
    g->in = e->a;
    g->out = p->out;
    if (i + 3 < G.h.no) {
        const Op *ad = G.ops + i + 3;
        const int ordered = ad->a == e->a && ad->b == p->out, swapped = ad->a == p->out && ad->b == e->a;
        const int32_t *q = ad->code == 18 ? (const int32_t *)(G.arena + G.ts[ad->p[0]].offset) : NULL;
        /* The fused add takes shifts in [-31, 31] (its rescale as one
         * multiply-add); others leave the add to its own launch. */
        if (q && (ordered || swapped) && users[p->out] == 1 && p->out != G.h.output && se->ic == sp->oc &&
            q[1] >= -31 && q[1] <= 31) {
            f->has_add = 1;
            f->add_x_first = ordered;
            f->add_tab = G.dev_arena + G.ts[ad->p[0]].offset + 8 * 4;
            f->a_m = q[0]; f->a_s = q[1]; f->a_yz = q[2]; f->a_lo = q[3]; f->a_hi = q[4];
            g->nops = 4;
            g->out = ad->out;
        }
    }
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    G.fuse_of_tensor[e->out] = G.fuse_of_tensor[d->out] = (uint16_t)(G.ngroups + 1);
    if (g->nops == 4) G.fuse_of_tensor[p->out] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return g->nops;
}

/* Universal inverted bottlenecks by bands of output rows (uib.hip): a
 * stride-1 depthwise whose output keeps the map size and feeds only a 1x1
 * conv (the start depthwise), then [a depthwise of stride 1 or 2], then a
 * 1x1 conv, optionally followed by an add of the block input; or a 1x1 conv,
 * a stride-2 depthwise and a 1x1 conv (k_ib takes the stride-1 form). The
 * depthwise layers in window form; inner tensors single-use activations,
 * not the plan output; one image per plan image.
 *
 * By default only blocks whose whole map fits one workgroup (one band) run
 * fused: on MobileNetV4-S at batch 256 that fuses the 14x14 ExtraDW block
 * (0.437 against 0.457 ms per step unfused), while the banded forms measured
 * slower than their separate launches (the 28x28 block in five bands of
 * three rows, 0.471 ms with it; the 7x7 ExtraDW block in two bands, 0.463).
 * UQ_FUSE_UIB=2 at load time fuses banded blocks too, =0 none. */
static uint32_t find_uib(uint32_t i, const uint16_t *users, int bands_ok)
{
    UQKUib u;
    memset(&u, 0, sizeof u);
    uint32_t j = i;
    const Tensor *x = G.ts + G.ops[i].a;
    if (x->flags || x->rank != 4 || x->d[0] != 1 || G.ops[i].a == G.h.input) return 0;
    if (G.ops[j].code == 15) {
        const UQKSpatial *d = G.sp + j;
        if (!d->dwwin || d->sh != 1 || d->sw != 1 || d->oh != d->ih || d->ow != d->iw || d->oc != d->ic) return 0;
        u.k0 = d->kh; u.p0t = d->pt; u.p0l = d->pl;
        u.dw0 = d->wdot; u.epi0 = d->epi; u.lut0 = d->lut;
        u.m0 = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0); u.yz0 = d->yz; u.lo0 = d->lo; u.hi0 = d->hi; u.xz0 = d->xz;
        j++;
    }
    if (j + 1 >= G.h.no || !pointwise_conv(j) || G.ops[j].a != (j > i ? G.ops[j - 1].out : G.ops[i].a)) return 0;
    const UQKSpatial *se = G.sp + j;
    if (u.k0 && (se->ih != G.sp[i].oh || se->iw != G.sp[i].ow || se->ic != G.sp[i].oc)) return 0;
    u.H = se->ih; u.W = se->iw; u.Cin = se->ic; u.Ce = se->oc;
    u.we = se->w; u.epi_e = se->epi; u.lut_e = se->lut; u.kpe = se->kpad;
    u.e_mode = (se->hi_shift ? 1 : 0) | (se->corr ? 2 : 0); u.e_yz = se->yz; u.e_lo = se->lo; u.e_hi = se->hi;
    j++;
    if (G.ops[j].code == 15) {
        const UQKSpatial *d = G.sp + j;
        if (!d->dwwin || d->sh != d->sw || d->ih != u.H || d->iw != u.W || d->ic != u.Ce || d->oc != u.Ce ||
            G.ops[j].a != G.ops[j - 1].out)
            return 0;
        u.k = d->kh; u.s = d->sh; u.pt = d->pt; u.pl = d->pl;
        u.dww = d->wdot; u.epi_d = d->epi; u.lut_d = d->lut;
        u.d_mode = (d->hi_shift ? 1 : 0) | (d->corr ? 2 : 0); u.d_yz = d->yz; u.d_lo = d->lo; u.d_hi = d->hi;
        u.d_xz = d->xz;
        u.Ho = d->oh; u.Wo = d->ow;
        j++;
    } else {
        u.Ho = u.H; u.Wo = u.W;
    }
    if (j >= G.h.no || !pointwise_conv(j) || G.ops[j].a != G.ops[j - 1].out) return 0;
    if (!u.k0 && (!u.k || u.s == 1)) return 0;
    const UQKSpatial *sp = G.sp + j;
    if (sp->ih != u.Ho || sp->iw != u.Wo || sp->ic != u.Ce) return 0;
    u.Cout = sp->oc;
    u.wp = sp->w; u.epi_p = sp->epi; u.lut_p = sp->lut; u.kpp = sp->kpad;
    u.p_mode = (sp->hi_shift ? 1 : 0) | (sp->corr ? 2 : 0); u.p_yz = sp->yz; u.p_lo = sp->lo; u.p_hi = sp->hi;
    for (uint32_t k = i; k < j; k++)
        if (users[G.ops[k].out] != 1 || G.ops[k].out == G.h.output) return 0;
    uint32_t nops = j - i + 1, out = G.ops[j].out;
    if (j + 1 < G.h.no && G.ops[j + 1].code == 18) {
        const Op *ad = G.ops + j + 1;
        const uint32_t xin = G.ops[i].a;
        const int ordered = ad->a == xin && ad->b == out, swapped = ad->a == out && ad->b == xin;
        const int32_t *q = (const int32_t *)(G.arena + G.ts[ad->p[0]].offset);
        /* The fused add takes shifts in [-31, 31] (its rescale as one
         * multiply-add); others leave the add to its own launch. */
        if ((ordered || swapped) && users[out] == 1 && out != G.h.output && u.Cin == u.Cout && u.Ho == u.H &&
            u.Wo == u.W && q[1] >= -31 && q[1] <= 31) {
            u.has_add = 1;
            u.add_x_first = ordered;
            u.add_tab = G.dev_arena + G.ts[ad->p[0]].offset + 8 * 4;
            u.a_m = q[0]; u.a_s = q[1]; u.a_yz = q[2]; u.a_lo = q[3]; u.a_hi = q[4];
            nops++;
            out = ad->out;
        }
    }
    if (!uqk_uib_plan(&u)) return 0;
    if (bands_ok < 2 && u.R < u.Ho) return 0;
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 3;
    g->ub = u;
    g->first = i;
    g->nops = nops;
    g->in = G.ops[i].a;
    g->out = out;
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    for (uint32_t k = i; k + 1 < i + nops; k++) G.fuse_of_tensor[G.ops[k].out] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return nops;
}

/* Stem + 3x3 stride 2 [+ 1x1]: a stem conv (the stem form, 32 output
 * channels) whose output, used by nothing else, is the input of the next op,
 * a 3x3 stride-2 conv over those 32 channels that fits stem.hip; and when
 * the op after that is a 1x1 32 -> 32 conv over the 3x3's output, used by
 * nothing else either, that conv too. On unless UQ_FUSE_STEM=0 at load
 * time (UQ_FUSE_STEM=2: stem and 3x3 only). Returns the ops taken. */
static int find_stem_conv(uint32_t i, const uint16_t *users, int with_pw)
{
    const Op *s = G.ops + i, *c = G.ops + i + 1;
    if (s->code != 14 || c->code != 14 || c->a != s->out) return 0;
    const uint32_t t = s->out;
    if (users[t] != 1 || t == G.h.output || G.ts[s->a].rank != 4 || G.ts[s->a].d[0] != 1) return 0;
    if (!uqk_stem_conv_ok(G.sp + i, G.sp + i + 1, NULL)) return 0;
    const Op *p = i + 2 < G.h.no ? G.ops + i + 2 : NULL;
    const int pw = with_pw && p && p->code == 14 && p->a == c->out && users[c->out] == 1 && c->out != G.h.output &&
                   uqk_stem_conv_ok(G.sp + i, G.sp + i + 1, G.sp + i + 2);
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 2;
    g->first = i;
    g->nops = pw ? 3 : 2;
    g->in = s->a;
    g->out = pw ? p->out : c->out;
    G.fuse_at[i] = (uint16_t)(G.ngroups + 1);
    G.fuse_of_tensor[t] = (uint16_t)(G.ngroups + 1);
    if (pw) G.fuse_of_tensor[c->out] = (uint16_t)(G.ngroups + 1);
    G.ngroups++;
    return (int)g->nops;
}

/* Row gathers (kind 5): a concat along the last axis (op 20) of int8/uint8
 * rows whose operands are single-use table lookups (op 22), or single-use
 * concats along the last axis (nested, up to four segments) of such lookups
 * or plain tensors; a lookup
 * whose input is a single-use slice of the last axis only (op 26) reads the
 * slice's source directly. One launch (uqk_gather) writes the concat's rows
 * from the sources through the tables, in place of the lookups, the inner
 * concat and those slices. YOLO's C3k2 blocks (split, two SiLU tables,
 * concat, concat with the bottleneck output) drop four launches each, its
 * SPPF block (three chained concats of pooled maps) two. On
 * unless UQ_FUSE_GATHER=0 at load time. */
static int rows_like(const Tensor *t, const Tensor *z)
{
    if (t->flags || t->rank != z->rank || t->rank < 1 || t->rank > 4 || width(t->type) != 1) return 0;
    for (uint32_t d = 0; d + 1 < t->rank; d++)
        if (t->d[d] != z->d[d]) return 0;
    return 1;
}

static int gather_operand(Group *g, uint32_t t, int depth, const uint16_t *users, const uint32_t *prod,
                          const uint8_t *taken)
{
    const Tensor *z = G.ts + G.ops[g->first].out;
    const uint32_t r = z->rank;
    if (!rows_like(G.ts + t, z)) return 0;
    const uint32_t j = prod[t] ? prod[t] - 1 : UG_MAX_OP;
    const int inner = j < UG_MAX_OP && !taken[j] && users[t] == 1 && t != G.h.output && t != G.h.input;
    if (inner && depth < 3 && G.ops[j].code == 20 && G.ops[j].p[0] == r - 1 && G.ops[j].a != G.ops[j].b &&
        g->nelide < 10) {
        const uint32_t mark = g->nseg, em = g->nelide;
        g->elide[g->nelide++] = j;
        if (gather_operand(g, G.ops[j].a, depth + 1, users, prod, taken) &&
            gather_operand(g, G.ops[j].b, depth + 1, users, prod, taken))
            return 1;
        g->nseg = mark;
        g->nelide = em;
    }
    if (g->nseg >= 4) return 0;
    const uint32_t k = g->nseg;
    g->seg_src[k] = t;
    g->seg_off[k] = 0;
    g->seg_width[k] = G.ts[t].d[r - 1];
    g->seg_has_lut[k] = 0;
    g->seg_lut[k] = g->seg_flip[k] = 0;
    if (inner && G.ops[j].code == 22 && rows_like(G.ts + G.ops[j].a, z) && g->nelide < 10) {
        const uint32_t s = G.ops[j].a;
        g->elide[g->nelide++] = j;
        g->seg_src[k] = s;
        g->seg_width[k] = G.ts[s].d[r - 1];
        g->seg_has_lut[k] = 1;
        g->seg_lut[k] = G.ops[j].b;
        g->seg_flip[k] = G.ts[s].type == 3 ? 128u : 0u;
        /* A single-use slice of the last axis: read its source. */
        const uint32_t i = prod[s] ? prod[s] - 1 : UG_MAX_OP;
        if (i < UG_MAX_OP && !taken[i] && G.ops[i].code == 26 && users[s] == 1 && s != G.h.output &&
            s != G.h.input && rows_like(G.ts + G.ops[i].a, z) && g->nelide < 10) {
            const Tensor *x = G.ts + G.ops[i].a, *y = G.ts + s;
            int ok = 1;
            for (uint32_t d = 0; d + 1 < r; d++)
                if (G.ops[i].p[d] != 0) ok = 0;
            if (ok && (uint64_t)G.ops[i].p[r - 1] + y->d[r - 1] <= x->d[r - 1]) {
                g->elide[g->nelide++] = i;
                g->seg_src[k] = G.ops[i].a;
                g->seg_off[k] = G.ops[i].p[r - 1];
            }
        }
    }
    g->nseg++;
    return 1;
}

static int find_gather(uint32_t k, const uint16_t *users, const uint32_t *prod, uint8_t *taken)
{
    const Op *o = G.ops + k;
    if (o->code != 20 || taken[k] || o->a == o->b) return 0;
    const Tensor *z = G.ts + o->out;
    if (z->flags || width(z->type) != 1 || o->p[0] != z->rank - 1) return 0;
    Group *g = &G.groups[G.ngroups];
    memset(g, 0, sizeof *g);
    g->kind = 5;
    g->first = k;
    g->nops = 1;
    if (!gather_operand(g, o->a, 0, users, prod, taken) || !gather_operand(g, o->b, 0, users, prod, taken) ||
        !g->nelide)
        return 0;
    uint64_t w = 0;
    for (uint32_t s = 0; s < g->nseg; s++) w += g->seg_width[s];
    if (w != z->d[z->rank - 1]) return 0;
    /* Plan order, for rebuilding the inner tensors. */
    for (uint32_t a = 0; a < g->nelide; a++)
        for (uint32_t b = a + 1; b < g->nelide; b++)
            if (g->elide[b] < g->elide[a]) {
                const uint32_t t = g->elide[a];
                g->elide[a] = g->elide[b];
                g->elide[b] = t;
            }
    g->in = g->seg_src[0];
    g->out = o->out;
    G.fuse_at[k] = (uint16_t)(G.ngroups + 1);
    taken[k] = 1;
    for (uint32_t e = 0; e < g->nelide; e++) {
        G.elide[g->elide[e]] = (uint16_t)(G.ngroups + 1);
        G.fuse_of_tensor[G.ops[g->elide[e]].out] = (uint16_t)(G.ngroups + 1);
        taken[g->elide[e]] = 1;
    }
    G.ngroups++;
    return 1;
}

static void find_groups(uint8_t *pool, const Layout *layouts)
{
    static uint16_t users[UG_MAX_T];
    memset(G.fuse_at, 0, sizeof G.fuse_at);
    memset(G.fuse_of_tensor, 0, sizeof G.fuse_of_tensor);
    memset(G.elide, 0, sizeof G.elide);
    G.ngroups = 0;
    count_users(users);
    const char *streams = getenv("UQ_STREAMS");
    G.slices = streams ? atoi(streams) : 0;
    if (G.slices > UQK_MAX_SLICES) G.slices = UQK_MAX_SLICES;
    const char *env = getenv("UQ_FUSE_BOTTLENECK");
    const int bottleneck = !(env && !strcmp(env, "0"));
    const char *senv = getenv("UQ_FUSE_STEM");
    const int stem = !(senv && !strcmp(senv, "0")), stem_pw = !(senv && !strcmp(senv, "2"));
    const char *menv = getenv("UQ_FUSE_MEAN");
    const int conv_mean = !(menv && !strcmp(menv, "0"));
    const char *lenv = getenv("UQ_FUSE_LUT");
    const int conv_lut = !(lenv && !strcmp(lenv, "0"));
    const char *uenv = getenv("UQ_FUSE_UIB");
    const int uib = !uenv ? 1 : !strcmp(uenv, "0") ? 0 : !strcmp(uenv, "2") ? 2 : 1;
    for (uint32_t i = 0; i + 1 < G.h.no; i++) {
        uint32_t n = stem ? (uint32_t)find_stem_conv(i, users, stem_pw) : 0;
        if (!n && uib) n = find_uib(i, users, uib);
        if (!n && bottleneck) n = find_bottleneck(i, users);
        if (!n && find_conv_add(i, users)) n = 2;
        if (!n && conv_mean && find_conv_mean(i, users)) n = 2;
        if (!n && conv_lut && find_conv_lut(i, users, pool, layouts)) n = 2;
        if (n) i += n - 1;
    }
    const char *genv = getenv("UQ_FUSE_GATHER");
    G.pack_rows = genv && !strcmp(genv, "0");
    if (!G.pack_rows) {
        static uint32_t prod[UG_MAX_T];
        static uint8_t taken[UG_MAX_OP];
        memset(prod, 0, sizeof prod);
        memset(taken, 0, sizeof taken);
        for (uint32_t i = 0; i < G.h.no; i++) prod[G.ops[i].out] = i + 1;
        for (uint32_t gi = 0; gi < G.ngroups; gi++)
            for (uint32_t k = 0; k < G.groups[gi].nops; k++) taken[G.groups[gi].first + k] = 1;
        /* Last concat first, so that the outermost concat of a chain takes
         * the inner ones. */
        for (uint32_t k = G.h.no; k-- > 0 && G.ngroups < UG_MAX_OP / 2;) find_gather(k, users, prod, taken);
    }
    memset(G.fwd, 0, sizeof G.fwd);
    for (uint32_t i = 1; i < G.h.no; i++) {
        const Op *r = G.ops + i, *p = G.ops + i - 1;
        const uint32_t t = r->a;
        if (r->code != 5 || r->out != G.h.output || p->out != t || users[t] != 1 || t == G.h.input ||
            G.ts[t].flags || G.ts[r->out].flags || G.ts[t].bytes != G.ts[r->out].bytes)
            continue;
        int grouped = 0;
        for (uint32_t g = 0; g < G.ngroups; g++)
            if (i - 1 >= G.groups[g].first && i - 1 < G.groups[g].first + G.groups[g].nops) grouped = 1;
        if (!grouped) G.fwd[i - 1] = 1;
    }
}

/* Write a fused group's inner tensors after a fused run (for snapshots): its
 * ops again, one by one, from the input the fused launch read, into the
 * library's own buffers. */
static int materialize_group(uint32_t t)
{
    const uint32_t gi = G.fuse_of_tensor[t];
    if (!gi) return 0;
    Group *g = &G.groups[gi - 1];
    if (!g->last_images) return 0;
    if (g->last_ext) return 22;
    if (g->kind == 5) {
        /* The ops the gather stood in for, from their inputs (the library's
         * own buffers, unchanged since). */
        int rc = 0;
        for (uint32_t e = 0; e < g->nelide; e++) G.ptr[G.ops[g->elide[e]].out] = G.act[G.ops[g->elide[e]].out];
        for (uint32_t e = 0; e < g->nelide && !rc; e++) rc = enqueue_op(g->elide[e], g->last_images);
        if (!rc) rc = uqk_sync();
        g->last_images = 0;
        return rc ? 24 : 0;
    }
    uint8_t *saved_in = G.ptr[g->in];
    G.ptr[g->in] = (uint8_t *)g->last_in;
    for (uint32_t k = 0; k < g->nops; k++) G.ptr[G.ops[g->first + k].out] = G.act[G.ops[g->first + k].out];
    int rc = 0;
    for (uint32_t k = 0; k < g->nops && !rc; k++) rc = enqueue_op(g->first + k, g->last_images);
    G.ptr[g->in] = saved_in;
    if (!rc) rc = uqk_sync();
    g->last_images = 0;
    return rc ? 24 : 0;
}

static int prepare_device(void)
{
    if (uqk_init()) return 24;
    G.dev_arena = uqk_malloc(G.h.arena_bytes);
    if (!G.dev_arena) return 24;
    size_t at = 0;
    static Layout layouts[UG_MAX_OP];
    for (uint32_t i = 0; i < G.h.no; i++) {
        const Op *o = G.ops + i;
        if (o->code == 14 || o->code == 15 || o->code == 16) {
            layouts[i] = spatial_layout(o, at);
            at = layouts[i].end;
        }
    }
    uint8_t *host_pool = calloc(at + 256, 1);
    if (!host_pool) return 24;
    G.dev_prep = uqk_malloc(at + 256);
    if (!G.dev_prep) { free(host_pool); return 24; }
    for (uint32_t i = 0; i < G.h.no; i++) {
        const Op *o = G.ops + i;
        if (o->code == 14 || o->code == 15 || o->code == 16) prepare_spatial(i, layouts + i, host_pool);
    }
    find_groups(host_pool, layouts);
    int rc = uqk_h2d(G.dev_arena, G.arena, G.h.arena_bytes);
    if (!rc) rc = uqk_h2d(G.dev_prep, host_pool, at + 256);
    if (!rc) rc = uqk_sync();
    free(host_pool);
    if (!rc) rc = uqk_events(G.h.no);
    return rc ? 24 : 0;
}

int ug_load(const void *blob, uint32_t len)
{
    if (G.split_open) {
        (void)settle();
        (void)uqk_sync();
    }
    G.ready = 0;
    G.profile_enabled = 0;
    G.stream_active = 0;
    release_device();
    int rc = validate((const uint8_t *)blob, len);
    if (rc) return rc;
    for (uint32_t i = 0; i < G.h.no; i++)
        if (!supported(G.ops[i].code)) return 19;
    /* Operands read image by image (every `a` except a pack list head, and
     * the `b` of add, concat, mul and bmm). The loader lets a constant fill
     * such a slot; it then gets one copy per image so that every kernel can
     * step through stacked images uniformly. */
    memset(G.bcast, 0, sizeof G.bcast);
    for (uint32_t i = 0; i < G.h.no; i++) {
        const Op *o = G.ops + i;
        if (o->code != 19 && G.ts[o->a].flags) G.bcast[o->a] = 1;
        if ((o->code == 18 || o->code == 20 || o->code == 25 || o->code == 27) && G.ts[o->b].flags) G.bcast[o->b] = 1;
    }
    free(G.arena);
    G.arena = malloc(G.h.arena_bytes);
    if (!G.arena) return 24;
    uint32_t meta = (uint32_t)sizeof(Header) + G.h.nt * (uint32_t)sizeof(Tensor) + G.h.no * (uint32_t)sizeof(Op);
    memcpy(G.arena, (const uint8_t *)blob + meta, G.h.arena_bytes);
    rc = prepare_device();
    if (rc) {
        release_device();
        return rc;
    }
    memset(G.ticks, 0, sizeof G.ticks);
    G.ready = 1;
    return 0;
}

uint32_t ug_input_bytes(void) { return G.ready ? G.ts[G.h.input].bytes : 0; }
uint32_t ug_output_bytes(void) { return G.ready ? G.ts[G.h.output].bytes : 0; }
uint32_t ug_op_count(void) { return G.ready ? G.h.no : 0; }

static int ensure_capacity(uint32_t images)
{
    if (images <= G.capacity) return 0;
    if (settle() || uqk_sync()) return 24;
    for (uint32_t t = 0; t < G.h.nt; t++) {
        uqk_free(G.act[t]);
        G.act[t] = NULL;
    }
    G.capacity = 0;
    G.generation++;
    for (uint32_t t = 0; t < G.h.nt; t++) {
        if (G.ts[t].flags && !G.bcast[t]) continue;
        G.act[t] = uqk_malloc((size_t)images * G.ts[t].bytes);
        if (!G.act[t]) return 24;
        if (G.ts[t].flags)
            for (uint32_t k = 0; k < images; k++)
                if (uqk_d2d(G.act[t] + (size_t)k * G.ts[t].bytes, G.dev_arena + G.ts[t].offset, G.ts[t].bytes)) return 24;
    }
    G.capacity = images;
    return 0;
}

/* Enqueue ops [i0, i1) of the plan for `images` stacked images on the
 * current stream, launching fused groups in place of their ops (not while
 * per-op profiling is on, and not on a caller's input buffer). Tensor
 * addresses come from G.ptr. Returns the op after the last one enqueued (a
 * group that starts before i1 runs whole). */
/* Whether a gather (kind 5) runs fused this time: not while per-op
 * profiling is on, and only from the library's own buffers, which still
 * hold the same bytes if a snapshot later asks for an inner tensor. */
static int gather_fused(const Group *g)
{
    if (G.profile_enabled) return 0;
    for (uint32_t s = 0; s < g->nseg; s++)
        if (G.ext[g->seg_src[s]]) return 0;
    return 1;
}

static int gather_launch(Group *g, uint32_t images)
{
    UQKSeg segs[4];
    const Tensor *z = G.ts + g->out;
    uint64_t rows = images;
    for (uint32_t d = 0; d + 1 < z->rank; d++) rows *= z->d[d];
    for (uint32_t s = 0; s < g->nseg; s++) {
        const Tensor *t = G.ts + g->seg_src[s];
        segs[s].src = G.ptr[g->seg_src[s]] + g->seg_off[s];
        segs[s].stride = t->d[t->rank - 1];
        segs[s].width = g->seg_width[s];
        segs[s].lut = g->seg_has_lut[s] ? G.ptr[g->seg_lut[s]] : NULL;
        segs[s].flip = g->seg_flip[s];
    }
    return uqk_gather(G.ptr[g->out], z->d[z->rank - 1], segs, g->nseg, rows);
}

static int enqueue_range(uint32_t i0, uint32_t i1, uint32_t images, uint32_t *next)
{
    uint32_t i = i0;
    for (; i < i1; i++) {
        if (G.elide[i] && gather_fused(&G.groups[G.elide[i] - 1])) continue;
        const uint32_t g = G.fuse_at[i];
        if (g && G.groups[g - 1].kind == 5) {
            Group *grp = &G.groups[g - 1];
            if (gather_fused(grp)) {
                const int rc = gather_launch(grp, images);
                if (rc) return rc;
                grp->last_in = G.ptr[grp->in];
                grp->last_images = images;
                grp->last_ext = 0;
                continue;
            }
            grp->last_images = 0;
            const int rc = enqueue_op(i, images);
            if (rc) return rc;
            continue;
        }
        /* Groups of kinds 0, 1 and 3 run fused only when the buffers they read
         * are the library's own, which still hold the same bytes if a
         * snapshot later asks for an inner tensor (materialize_group). The
         * stem group (kind 2) reads the plan input, a caller buffer on the
         * device entry points: it runs fused on it, and its inner tensor's
         * snapshot is then unavailable (22). */
        if (g && !G.profile_enabled &&
            (G.groups[g - 1].kind == 2 ||
             (!G.ext[G.groups[g - 1].in] && (G.groups[g - 1].kind != 1 || !G.ext[G.groups[g - 1].res])))) {
            Group *grp = &G.groups[g - 1];
            int rc;
            if (grp->kind == 0) {
                rc = uqk_ib(&grp->desc, G.ptr[grp->in], G.ptr[grp->out], images);
            } else if (grp->kind == 3) {
                rc = uqk_uib(&grp->ub, G.ptr[grp->in], G.ptr[grp->out], images);
            } else if (grp->kind == 6) {
                rc = uqk_conv(&grp->sp, G.ptr[grp->in], G.ptr[grp->out], images * G.ts[G.ops[i].a].d[0]);
            } else if (grp->kind == 4) {
                rc = uqk_conv_mean(G.sp + i, &grp->mean, G.ptr[grp->in], G.ptr[grp->out],
                                   images * G.ts[G.ops[i].a].d[0]);
            } else if (grp->kind == 1) {
                grp->add.res = G.ptr[grp->res];
                rc = uqk_conv_add(G.sp + i, G.ptr[grp->in], G.ptr[grp->out], images * G.ts[G.ops[i].a].d[0],
                                  &grp->add);
            } else {
                rc = uqk_stem_conv(G.sp + i, G.sp + i + 1, grp->nops == 3 ? G.sp + i + 2 : NULL, G.ptr[grp->in],
                                   G.ptr[grp->out], images);
            }
            if (rc) return rc;
            grp->last_in = G.ptr[grp->in];
            grp->last_images = images;
            grp->last_ext = G.ext[grp->in];
            i += grp->nops - 1;
            continue;
        }
        if (g) G.groups[g - 1].last_images = 0;
        int rc = enqueue_op(i, images);
        if (rc) return rc;
    }
    *next = i;
    return 0;
}

/* Images per slice below which a batch runs on one stream. */
#define UQ_SLICE_MIN 64

/* Number of image slices a batch of `images` runs as: UQ_STREAMS (1 or 2)
 * when set at load, else 2 from 2 * UQ_SLICE_MIN images for plans of at
 * least four ops. Two slices measured 5% faster than one on MobileNetV4-S at
 * batch 256, whose layers are mostly latency-bound launches of a few hundred
 * workgroups; a plan of one large conv only loses half of each grid. */
static int slice_count(uint32_t images)
{
    if (G.profile_enabled) return 1;
    int n = G.slices;
    if (n <= 0) n = G.h.no >= 4 ? 2 : 1;
    while (n > 1 && images / (uint32_t)n < UQ_SLICE_MIN) n--;
    return n;
}

/* Join the side stream of the last split batch into the library stream, if
 * it may still hold work of that batch (see enqueue_ops). Every entry point
 * that puts other work on the library stream, reads results or changes
 * buffers calls this first. */
static int settle(void)
{
    if (!G.split_open) return 0;
    G.split_open = 0;
    return uqk_split_join(G.split_n) ? 24 : 0;
}

/* Enqueue the whole plan. A large batch runs as image slices on separate
 * compute streams, op by op in turn, so that the launches of one slice
 * overlap the latency and tail of the other's: every op works image by
 * image, and each slice sees the batch's buffers offset by its first image
 * (shared constants are not offset). Each slice keeps its own address table
 * across ops, since internal copies alias their source (enqueue_op, code 5).
 * Afterwards G.ptr is slice 0's table, the addresses of the whole batch.
 *
 * The side stream is not joined back at the end: the next identical batch
 * (same slices, image count, input and output buffers) continues on each
 * stream, where each slice reads and writes the same images as before, so
 * the two streams drift apart and one slice's bandwidth-bound layers overlap
 * the other's latency-bound ones. Anything else settles first (the side
 * stream joins the library stream; uqk_sync waits for both). */
static int finish_profile(void);

static int enqueue_ops(uint32_t images)
{
    const int n = slice_count(images);
    int rc = 0;
    uint32_t next = 0;
    if (n == 1) {
        if (settle()) return 24;
        /* Each profiled batch re-stamps the same per-op events: the one
         * before it is counted first. */
        if (G.profile_enabled) {
            if (finish_profile()) return 24;
            G.prof_pending = 1;
        }
        return enqueue_range(0, G.h.no, images, &next);
    }
    const int cont = G.split_open && G.split_n == n && G.split_images == images &&
                     G.split_in == G.ptr[G.h.input] && G.split_out == G.ptr[G.h.output];
    if (!cont && (settle() || uqk_split_fork(n))) return 24;
    G.split_open = 1;
    G.split_n = n;
    G.split_images = images;
    G.split_in = G.ptr[G.h.input];
    G.split_out = G.ptr[G.h.output];
    static uint8_t *tab[UQK_MAX_SLICES][UG_MAX_T];
    uint32_t first[UQK_MAX_SLICES + 1];
    for (int k = 0; k <= n; k++) first[k] = (uint32_t)((uint64_t)images * (uint32_t)k / (uint32_t)n);
    for (int k = 0; k < n; k++)
        for (uint32_t t = 0; t < G.h.nt; t++)
            tab[k][t] = G.ts[t].flags && !G.bcast[t] ? G.ptr[t] : G.ptr[t] + (size_t)first[k] * G.ts[t].bytes;
    const size_t tb = sizeof(uint8_t *) * G.h.nt;
    for (uint32_t i = 0; i < G.h.no && !rc; i = next) {
        for (int k = n - 1; k >= 0 && !rc; k--) {
            memcpy(G.ptr, tab[k], tb);
            uqk_split_use(k, n);
            rc = enqueue_range(i, i + 1, first[k + 1] - first[k], &next);
            memcpy(tab[k], G.ptr, tb);
        }
    }
    uqk_split_use(0, 1);
    memcpy(G.ptr, tab[0], tb);
    /* Fused groups record the input and image count of the whole batch. */
    for (uint32_t g = 0; g < G.ngroups; g++)
        if (G.groups[g].last_images) {
            G.groups[g].last_in = G.ptr[G.groups[g].in];
            G.groups[g].last_images = images;
        }
    return rc;
}

static int launch_op(uint32_t i, uint32_t images);

/* Enqueue op i; while profiling, with its kernels stamping the op's timing
 * events. */
static int enqueue_op(uint32_t i, uint32_t images)
{
    if (!G.profile_enabled) return launch_op(i, images);
    int rc = uqk_time_begin(i);
    if (!rc) rc = launch_op(i, images);
    int rc2 = uqk_time_end(i);
    return rc ? rc : rc2;
}

static int launch_op(uint32_t i, uint32_t images)
{
    const uint8_t *A = G.arena;
    if (G.fwd[i] && G.ext[G.ops[i + 1].out]) {
        G.ptr[G.ops[i].out] = G.ptr[G.ops[i + 1].out];
        G.ext[G.ops[i].out] = 1;
    }
    {
        const Op *o = G.ops + i;
        const Tensor *a = G.ts + o->a, *b = G.ts + o->b, *z = G.ts + o->out;
        void *zp = G.ptr[o->out];
        const void *ap = G.ptr[o->a], *bp = G.ptr[o->b];
        int rc = 0;
        switch (o->code) {
        case 14: rc = uqk_conv(G.sp + i, ap, zp, images * a->d[0]); break;
        case 15: rc = uqk_depthwise(G.sp + i, ap, zp, images * a->d[0]); break;
        case 16: rc = uqk_pool(G.sp + i, ap, zp, images * a->d[0]); break;
        case 18: {
            const int32_t *q = (const int32_t *)(A + G.ts[o->p[0]].offset);
            rc = uqk_add(ap, bp, zp, (uint64_t)images * z->bytes, G.dev_arena + G.ts[o->p[0]].offset + 8 * 4,
                         q[0], q[1], q[2], q[3], q[4]);
            break;
        }
        case 24: {
            const int32_t *q = (const int32_t *)(A + b->offset);
            rc = uqk_mean(ap, zp, images * a->d[0], (uint32_t)q[0], a->d[3], q[1], q[2], q[3], q[4]);
            break;
        }
        case 5:
            /* Every tensor is written once (graph.c:72 forbids redefinition),
             * so an internal copy can alias its source instead of moving bytes
             * (in every image slice); a copy into a caller buffer moves them
             * unless the producer already wrote there (fwd). */
            if (!G.ext[o->out]) {
                G.ptr[o->out] = (uint8_t *)G.ptr[o->a];
                G.ext[o->out] = G.ext[o->a];
            } else if (zp != ap)
                rc = uqk_d2d(zp, ap, (size_t)images * z->bytes);
            break;
        case 22: rc = uqk_lut(ap, zp, (uint64_t)images * a->bytes, bp, a->type == 3 ? 128u : 0u); break;
        case 10: rc = uqk_permute(ap, zp, images, a->rank, a->d, o->p, width(a->type)); break;
        case 17: {
            const int32_t *q = (const int32_t *)(A + G.ts[o->p[0]].offset);
            const uint32_t w = (uint32_t)q[16];
            rc = uqk_softmax_table(ap, zp, (uint64_t)images * (z->bytes / w), w,
                                   G.dev_arena + G.ts[o->p[0]].offset + UQ_HEAD * 4, q[14], q[15]);
            break;
        }
        case 25: rc = uqk_mul(ap, bp, zp, (uint64_t)images * z->bytes, (const int32_t *)(A + G.ts[o->p[0]].offset)); break;
        case 27: {
            const int32_t *q = (const int32_t *)(A + G.ts[o->p[0]].offset);
            rc = uqk_bmm(ap, bp, zp, images, z->d[0], z->d[1], z->d[2], a->d[q[5] ? 1 : 2], q);
            break;
        }
        case 28: {
            const uint32_t w = a->d[a->rank - 1];
            rc = uqk_softmax(ap, zp, (uint64_t)images * (z->bytes / w), w, G.dev_arena + b->offset + 4);
            break;
        }
        case 20: {
            uint64_t outer = images, inner = 1;
            uint32_t axis = o->p[0];
            for (uint32_t d = 0; d < axis; d++) outer *= a->d[d];
            for (uint32_t d = axis + 1; d < a->rank; d++) inner *= a->d[d];
            size_t ac = (size_t)a->d[axis] * inner, bc = (size_t)b->d[axis] * inner;
            rc = uqk_rows2(zp, ac + bc, ap, ac, ac, bp, bc, bc, outer);
            break;
        }
        case 21: rc = uqk_resize(ap, zp, images * a->d[0], a->d[1], a->d[2], z->d[1], z->d[2], a->d[3], bp); break;
        case 23: {
            const int32_t *q = (const int32_t *)(A + b->offset);
            int32_t off[4] = {q[0], q[2], q[4], q[6]};
            rc = uqk_window4(ap, zp, images, a->d, z->d, off, (int32_t)(int8_t)(int32_t)o->p[0]);
            break;
        }
        case 26: {
            uint32_t in[4] = {1, 1, 1, 1}, out[4] = {1, 1, 1, 1};
            int32_t off[4] = {0, 0, 0, 0};
            uint32_t lead = 4 - a->rank;
            for (uint32_t d = 0; d < a->rank; d++) {
                in[lead + d] = a->d[d];
                out[lead + d] = z->d[d];
                off[lead + d] = -(int32_t)o->p[d];
            }
            /* A slice of the last axis only, inside it, is a row copy (other
             * windows fill positions outside the input). */
            if (in[0] == out[0] && in[1] == out[1] && in[2] == out[2] && !off[0] && !off[1] && !off[2] &&
                off[3] <= 0 && (int64_t)out[3] - off[3] <= (int64_t)in[3])
                rc = uqk_rows2(zp, out[3], (const uint8_t *)ap - off[3], in[3], out[3], NULL, 0, 0,
                               (uint64_t)images * in[0] * in[1] * in[2]);
            else
                rc = uqk_window4(ap, zp, images, in, out, off, 0);
            break;
        }
        case 19: {
            const uint32_t *list = (const uint32_t *)(A + b->offset);
            const uint32_t nl = b->bytes / 4;
            /* Two to UQK_GATHER_MAX activations: one row gather, a row per
             * image (UQ_FUSE_GATHER=0: a copy per tensor). */
            UQKSeg segs[UQK_GATHER_MAX];
            int one = nl >= 2 && nl <= UQK_GATHER_MAX && !G.pack_rows;
            for (uint32_t j = 0; j < nl && one; j++) {
                const Tensor *t = G.ts + list[j];
                if (t->flags) one = 0;
                segs[j] = (UQKSeg){G.ptr[list[j]], t->bytes, t->bytes, NULL, 0};
            }
            if (one) {
                rc = uqk_gather(zp, z->bytes, segs, nl, images);
                break;
            }
            size_t off = 0;
            for (uint32_t j = 0; j < b->bytes / 4 && !rc; j++) {
                const Tensor *t = G.ts + list[j];
                if (t->flags) {
                    for (uint32_t k = 0; k < images && !rc; k++)
                        rc = uqk_d2d((uint8_t *)zp + (size_t)k * z->bytes + off, G.ptr[list[j]], t->bytes);
                } else
                    rc = uqk_rows2((uint8_t *)zp + off, z->bytes, G.ptr[list[j]], t->bytes, t->bytes, NULL, 0, 0,
                                   images);
                off += t->bytes;
            }
            break;
        }
        default: rc = 19;
        }
        if (rc) return rc;
    }
    return 0;
}

static void bind_pointers(const void *d_in, void *d_out)
{
    G.snap_void = 0;
    for (uint32_t t = 0; t < G.h.nt; t++) {
        G.ptr[t] = G.ts[t].flags && !G.bcast[t] ? G.dev_arena + G.ts[t].offset : G.act[t];
        G.ext[t] = 0;
    }
    if (d_in) {
        G.ptr[G.h.input] = (uint8_t *)d_in;
        G.ext[G.h.input] = 1;
    }
    if (d_out && G.h.output != G.h.input && !G.ts[G.h.output].flags) {
        G.ptr[G.h.output] = (uint8_t *)d_out;
        G.ext[G.h.output] = 1;
    }
}

/* Copy the output tensor to a caller buffer when it was not produced there. */
static int deliver_output_device(void *d_out, uint32_t images)
{
    const Tensor *t = G.ts + G.h.output;
    if (G.ptr[G.h.output] == (uint8_t *)d_out) return 0;
    if (t->flags) {
        for (uint32_t k = 0; k < images; k++)
            if (uqk_d2d((uint8_t *)d_out + (size_t)k * t->bytes, G.ptr[G.h.output], t->bytes)) return 24;
        return 0;
    }
    return uqk_d2d(d_out, G.ptr[G.h.output], (size_t)images * t->bytes) ? 24 : 0;
}

/* Add the per-op times of the pending profiled batch (if any) to the
 * counters: one run per profiled batch. */
static int finish_profile(void)
{
    if (!G.profile_enabled || !G.prof_pending) return 0;
    G.prof_pending = 0;
    if (uqk_sync()) return 24;
    uint64_t total = 0;
    for (uint32_t i = 0; i < G.h.no; i++) {
        uint64_t ns = 0;
        if (uqk_op_ns(i, &ns)) return 24;
        G.ticks[2 + i] += ns;
        total += ns;
    }
    G.ticks[0]++;
    G.ticks[1] += total;
    return 0;
}

static int fail(int rc)
{
    G.ready = 0;
    return rc;
}

int ug_run_batch(const void *input, uint64_t ni, void *output, uint64_t no, uint32_t images)
{
    if (!G.ready || !input || !output || !images || ni != (uint64_t)images * ug_input_bytes() ||
        no != (uint64_t)images * ug_output_bytes())
        return 22;
    if (settle() || ensure_capacity(images)) return fail(24);
    bind_pointers(NULL, NULL);
    if (uqk_h2d(G.ptr[G.h.input], input, ni)) return fail(24);
    /* The copy back runs on the library stream: it needs both slices. */
    if (enqueue_ops(images) || settle()) return fail(24);
    const Tensor *t = G.ts + G.h.output;
    if (t->flags) {
        if (uqk_sync()) return fail(24);
        for (uint32_t k = 0; k < images; k++) memcpy((uint8_t *)output + (size_t)k * t->bytes, G.arena + t->offset, t->bytes);
    } else {
        if (uqk_d2h(output, G.ptr[G.h.output], no)) return fail(24);
        if (uqk_sync()) return fail(24);
    }
    G.last_images = images;
    return finish_profile() ? fail(24) : 0;
}

int ug_run(const void *input, uint32_t ni, void *output, uint32_t no)
{
    if (!G.ready || !input || !output || ni != ug_input_bytes() || no != ug_output_bytes()) return 22;
    return ug_run_batch(input, ni, output, no, 1);
}

int ug_enqueue_device(const void *d_input, void *d_output, uint32_t images)
{
    if (!G.ready || !d_input || !d_output || !images) return 22;
    if (ensure_capacity(images)) return fail(24);
    bind_pointers(d_input, d_output);
    if (enqueue_ops(images)) return fail(24);
    /* A copy of the output on the library stream needs the whole batch. */
    if (G.ptr[G.h.output] != (uint8_t *)d_output && settle()) return fail(24);
    if (deliver_output_device(d_output, images)) return fail(24);
    G.last_images = images;
    return 0;
}

/* Tensors that take a scratch slot in a no-allocation run: activations other
 * than the caller's input (and the caller's output, when the output is an
 * activation distinct from the input), and constants replicated per image. */
static int scratch_tensor(uint32_t t)
{
    const Tensor *x = G.ts + t;
    if (x->flags && !G.bcast[t]) return 0;
    if (t == G.h.input) return 0;
    if (t == G.h.output && G.h.output != G.h.input && !x->flags) return 0;
    return 1;
}

int ug_enqueue_device_noalloc(const void *d_input, void *d_output, uint32_t images)
{
    if (!G.ready || !d_input || !d_output || !images) return 22;
    size_t cap = 0;
    uint8_t *base = uqk_scratch(&cap);
    if (!base) return 24;
    static size_t off[UG_MAX_T];
    size_t need = 0;
    for (uint32_t t = 0; t < G.h.nt; t++) {
        off[t] = 0;
        if (!scratch_tensor(t)) continue;
        off[t] = need;
        need += ((size_t)images * G.ts[t].bytes + 255) & ~(size_t)255;
        if (need > cap) return 22;
    }
    /* Per-image copies of constants in per-image operand slots, made once
     * per scratch layout; earlier work that may still read the scratch
     * (the other image slice of the last batch) finishes first. */
    const int fresh = G.scratch_generation != G.generation || G.scratch_images != images;
    if (fresh && settle()) return fail(24);
    G.snap_void = 1;
    for (uint32_t t = 0; t < G.h.nt; t++) {
        G.ext[t] = 0;
        if (scratch_tensor(t)) G.ptr[t] = base + off[t];
        else G.ptr[t] = G.ts[t].flags ? G.dev_arena + G.ts[t].offset : NULL;
    }
    if (fresh) {
        G.scratch_generation = G.generation;
        G.scratch_images = 0;
        for (uint32_t t = 0; t < G.h.nt; t++)
            if (G.ts[t].flags && G.bcast[t])
                for (uint32_t k = 0; k < images; k++)
                    if (uqk_d2d(G.ptr[t] + (size_t)k * G.ts[t].bytes, G.dev_arena + G.ts[t].offset, G.ts[t].bytes))
                        return fail(24);
        G.scratch_images = images;
    }
    G.ptr[G.h.input] = (uint8_t *)d_input;
    G.ext[G.h.input] = 1;
    if (G.h.output != G.h.input && !G.ts[G.h.output].flags) {
        G.ptr[G.h.output] = (uint8_t *)d_output;
        G.ext[G.h.output] = 1;
    }
    if (enqueue_ops(images)) return fail(24);
    if (G.ptr[G.h.output] != (uint8_t *)d_output && settle()) return fail(24);
    if (deliver_output_device(d_output, images)) return fail(24);
    G.last_images = 0;
    for (uint32_t g = 0; g < G.ngroups; g++) G.groups[g].last_images = 0;
    return 0;
}

int ug_synchronize(void)
{
    if (uqk_sync()) return fail(24);
    G.split_open = 0;                    /* both streams are idle */
    return finish_profile() ? fail(24) : 0;
}

int ug_run_device(const void *d_input, void *d_output, uint32_t images)
{
    int rc = ug_enqueue_device(d_input, d_output, images);
    if (rc) return rc;
    return ug_synchronize();
}

/* Chunked host-buffer batch with transfers overlapped with compute: chunk k's
 * host-to-device copy runs on the copy-in stream while chunk k-1 computes and
 * chunk k-2's results copy back on the copy-out stream. Two device buffers
 * per direction; events order reuse (a slot's input is overwritten only after
 * the chunk that read it finished, its output only after its copy-back). */
int ug_run_batch_pipelined(const void *input, uint64_t ni, void *output, uint64_t no, uint32_t images, uint32_t chunk)
{
    if (!G.ready || !input || !output || !images || ni != (uint64_t)images * ug_input_bytes() ||
        no != (uint64_t)images * ug_output_bytes())
        return 22;
    if (settle()) return fail(24);
    const Tensor *t = G.ts + G.h.output;
    /* Auto: chunks of at least 256 images (smaller launches underfill the
     * chip, which costs more than the overlap gains), pipelined from 512. */
    if (!chunk) chunk = images >= 512 ? ((images + 7) / 8 > 256 ? (images + 7) / 8 : 256) : images;
    if (chunk > images) chunk = images;
    /* Profiling records per-op events on the compute stream, and a constant
     * output needs no device work: both take the single-stream path. */
    if (G.profile_enabled || t->flags || chunk == images) return ug_run_batch(input, ni, output, no, images);
    const uint64_t ib = ug_input_bytes(), ob = ug_output_bytes();
    if (ensure_capacity(chunk)) return fail(24);
    if (G.pipe_in_bytes < (uint64_t)chunk * ib || G.pipe_out_bytes < (uint64_t)chunk * ob) {
        if (uqk_sync_all()) return fail(24);
        for (int k = 0; k < 2; k++) {
            uqk_free(G.pipe_in[k]);
            uqk_free(G.pipe_out[k]);
            G.pipe_in[k] = uqk_malloc((size_t)chunk * ib);
            G.pipe_out[k] = uqk_malloc((size_t)chunk * ob);
            if (!G.pipe_in[k] || !G.pipe_out[k]) return fail(24);
        }
        G.pipe_in_bytes = (uint64_t)chunk * ib;
        G.pipe_out_bytes = (uint64_t)chunk * ob;
        G.generation++;
    }
    /* events: 0/1 input slot loaded, 2/3 slot computed, 4/5 output slot copied back */
    const uint32_t chunks = (images + chunk - 1) / chunk;
    uint32_t last = chunk;
    for (uint32_t k = 0; k < chunks; k++) {
        const int slot = (int)(k & 1);
        const uint32_t nk = (k + 1) * chunk <= images ? chunk : images - k * chunk;
        const uint8_t *src = (const uint8_t *)input + (size_t)k * chunk * ib;
        uint8_t *dst = (uint8_t *)output + (size_t)k * chunk * ob;
        if (k >= 2 && uqk_pipe_wait(1, 2 + slot)) return fail(24);
        if (uqk_copy_on(1, G.pipe_in[slot], src, (size_t)nk * ib, 1) || uqk_pipe_record(slot, 1)) return fail(24);
        if (uqk_pipe_wait(0, slot)) return fail(24);
        if (k >= 2 && uqk_pipe_wait(0, 4 + slot)) return fail(24);
        bind_pointers(G.pipe_in[slot], G.pipe_out[slot]);
        /* The chunk's completion event is recorded on the library stream:
         * join the side stream first. */
        if (enqueue_ops(nk) || settle() || deliver_output_device(G.pipe_out[slot], nk)) return fail(24);
        if (uqk_pipe_record(2 + slot, 0)) return fail(24);
        if (uqk_pipe_wait(2, 2 + slot)) return fail(24);
        if (uqk_copy_on(2, dst, G.pipe_out[slot], (size_t)nk * ob, 0) || uqk_pipe_record(4 + slot, 2)) return fail(24);
        last = nk;
    }
    if (uqk_sync_all()) return fail(24);
    /* Snapshots see the last chunk's tensors. */
    G.last_images = last;
    return 0;
}

void *ug_host_alloc(uint64_t bytes)
{
    if (uqk_init()) return NULL;
    return uqk_host_alloc((size_t)bytes);
}

int ug_host_free(void *p)
{
    uqk_host_free(p);
    return 0;
}

/* ---- Bridge ABI: the reference's host session (runtime/bridge.c:99-185) ---
 * One session at a time over the library's single model. Mode 0 ("rpc") runs
 * each ug_infer through ug_run. Mode 1 ("mailbox", the persistent-worker
 * pipeline of the DSP host) keeps the per-call path short instead: pinned
 * staging buffers and one captured graph of the whole plan, replayed per
 * call. */
typedef struct {
    int pipeline;
    uint32_t ni, no;
    uint8_t *h_in, *h_out;      /* pinned staging (mailbox mode) */
    uint8_t *d_in, *d_out;      /* device buffers of one image (mailbox mode) */
    void *graph;
    uint64_t generation;
} Session;

static Session *g_session;

static void session_release(Session *s)
{
    uqk_graph_destroy(s->graph);
    uqk_host_free(s->h_in);
    uqk_host_free(s->h_out);
    uqk_free(s->d_in);
    uqk_free(s->d_out);
    free(s);
}

void ug_close(void *ptr)
{
    Session *s = ptr;
    if (!s || s != g_session) return;
    (void)settle();
    (void)uqk_sync();
    session_release(s);
    g_session = NULL;
}

void *ug_open_mode(const void *plan, uint32_t bytes, int pipeline, int *error)
{
    if (!error) return NULL;
    *error = 1;
    if (!plan || bytes > UG_MAX_PLAN || pipeline < 0 || pipeline > 1) return NULL;
    if (g_session) {
        *error = 1001;
        return NULL;
    }
    int rc = ug_load(plan, bytes);
    if (rc) {
        *error = rc;
        return NULL;
    }
    uint32_t ni = ug_input_bytes(), no = ug_output_bytes();
    if (!ni || !no || ni > 4u * 1024 * 1024 || no > 4u * 1024 * 1024) {
        /* bridge.c:117 reports the loader's (zero) code for oversized I/O. */
        *error = 0;
        return NULL;
    }
    Session *s = calloc(1, sizeof *s);
    if (!s) {
        *error = 1002;
        return NULL;
    }
    s->pipeline = pipeline;
    s->ni = ni;
    s->no = no;
    if (pipeline) {
        s->h_in = uqk_host_alloc(ni);
        s->h_out = uqk_host_alloc(no);
        s->d_in = uqk_malloc(ni);
        s->d_out = uqk_malloc(no);
        if (!s->h_in || !s->h_out || !s->d_in || !s->d_out) {
            session_release(s);
            *error = 1002;
            return NULL;
        }
    }
    g_session = s;
    *error = 0;
    return s;
}

void *ug_open(const void *plan, uint32_t bytes, int *error) { return ug_open_mode(plan, bytes, 0, error); }

/* Capture the whole plan for one image on the session's device buffers. */
static int session_capture(Session *s)
{
    uqk_graph_destroy(s->graph);
    s->graph = NULL;
    if (ensure_capacity(1)) return 24;
    bind_pointers(s->d_in, s->d_out);
    if (uqk_capture_begin()) return 24;
    int rc = enqueue_ops(1);
    if (!rc) rc = deliver_output_device(s->d_out, 1);
    void *exec = NULL;
    int end = uqk_capture_end(&exec);
    if (rc || end) {
        uqk_graph_destroy(exec);
        return 24;
    }
    s->graph = exec;
    s->generation = G.generation;
    return 0;
}

int ug_infer(void *ptr, const void *in, uint32_t ni, void *out, uint32_t no)
{
    Session *s = ptr;
    if (!s || s != g_session || !in || !out || ni != s->ni || no != s->no) return 1003;
    if (!s->pipeline || G.profile_enabled || G.ts[G.h.output].flags) return ug_run(in, ni, out, no);
    if (!G.ready || ug_input_bytes() != ni || ug_output_bytes() != no) return 22;
    if (settle()) return fail(24);
    if ((!s->graph || s->generation != G.generation) && session_capture(s)) return fail(24);
    memcpy(s->h_in, in, ni);
    if (uqk_h2d(s->d_in, s->h_in, ni) || uqk_graph_launch(s->graph) || uqk_d2h(s->h_out, s->d_out, no) || uqk_sync())
        return fail(24);
    memcpy(out, s->h_out, no);
    /* The captured run bound the tensors to this session's buffers. */
    bind_pointers(s->d_in, s->d_out);
    G.last_images = 1;
    return 0;
}

int ug_snapshot_tensor(void *ptr, uint32_t index, void *out, uint32_t bytes)
{
    Session *s = ptr;
    if (!s || s != g_session || s->pipeline || !out || !bytes || bytes > 4u * 1024 * 1024) return 1003;
    return ug_snapshot(index, out, bytes);
}

int ug_profile_control(void *ptr, uint32_t command, void *out, uint32_t bytes)
{
    Session *s = ptr;
    if (!s || s != g_session || !out || (bytes != 130 * 8 && bytes != (UG_MAX_OP + 2) * 8) || command > 2) return 1003;
    return ug_profile(command, out, bytes);
}

int ug_snapshot_images(uint32_t index, void *out, uint64_t bytes)
{
    if (!G.ready || index >= G.h.nt || !out) return 22;
    const Tensor *t = G.ts + index;
    if (t->flags) {
        if (bytes != t->bytes) return 22;
        memcpy(out, G.arena + t->offset, t->bytes);
        return 0;
    }
    if (G.snap_void || !G.last_images || bytes != (uint64_t)G.last_images * t->bytes) return 22;
    if (settle()) return fail(24);
    const int mrc = materialize_group(index);
    if (mrc) return mrc == 22 ? 22 : fail(24);
    if (uqk_d2h(out, G.ptr[index], bytes) || uqk_sync()) return fail(24);
    return 0;
}

int ug_snapshot(uint32_t index, void *out, uint32_t bytes)
{
    if (!G.ready || index >= G.h.nt || !out || bytes != G.ts[index].bytes) return 22;
    const Tensor *t = G.ts + index;
    if (t->flags) {
        memcpy(out, G.arena + t->offset, bytes);
        return 0;
    }
    if (G.snap_void) return 22;
    if (!G.last_images) {
        memcpy(out, G.arena + t->offset, bytes); /* arena contents before any run */
        return 0;
    }
    if (settle()) return fail(24);
    const int mrc = materialize_group(index);
    if (mrc) return mrc == 22 ? 22 : fail(24);
    if (uqk_d2h(out, G.ptr[index], bytes) || uqk_sync()) return fail(24);
    return 0;
}

int ug_profile(uint32_t command, void *out, uint32_t bytes)
{
    if (!G.ready || command > 2 || !out || (bytes != sizeof(G.ticks) && !(G.h.no <= 128 && bytes == 130 * 8))) return 22;
    if (command == 2 && finish_profile()) return fail(24);
    if (command == 1) memset(G.ticks, 0, sizeof G.ticks);
    if (command < 2) {
        G.profile_enabled = (int)command;
        G.prof_pending = 0;
    }
    memcpy(out, G.ticks, bytes);
    return 0;
}

int ug_stream_begin(void)
{
    if (G.stream_active) return 24;
    if (!G.ready) return 22;
    if (G.vision_only && G.h.reserved) G.stream_active = 1;
    return 0;
}

int ug_stream_end(void)
{
    if (!G.stream_active) return 0;
    G.stream_active = 0;
    return 0;
}

void *ug_device_alloc(uint64_t bytes)
{
    if (uqk_init()) return NULL;
    return uqk_malloc((size_t)bytes);
}

int ug_device_free(void *d)
{
    (void)settle();
    /* A run bound to this buffer (input, output or an alias of either) can
     * no longer be snapshotted, and the next batch must not continue its
     * side stream on it. */
    if (d && G.ready) {
        for (uint32_t t = 0; t < G.h.nt; t++)
            if (G.ext[t] && G.ptr[t] == (uint8_t *)d) G.snap_void = 1;
        if (G.split_in == d || G.split_out == d) G.split_in = G.split_out = NULL;
    }
    uqk_free(d);
    return 0;
}

int ug_device_upload(void *d_dst, const void *src, uint64_t bytes)
{
    if (uqk_init() || settle() || uqk_h2d(d_dst, src, (size_t)bytes) || uqk_sync()) return 24;
    return 0;
}

int ug_device_download(void *dst, const void *d_src, uint64_t bytes)
{
    if (uqk_init() || settle() || uqk_d2h(dst, d_src, (size_t)bytes) || uqk_sync()) return 24;
    return 0;
}
