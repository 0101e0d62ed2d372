/* .uqmodel bundle reader for the GPU library (plain C).
 *
 * Container format of the reference (src/unoq_dsp/bundle.py:18-19, 66-141):
 *   "UQMODEL\0" | u32 version = 1 | u32 manifest bytes | u32 plan bytes |
 *   32-byte SHA-256(manifest || plan) | manifest (JSON) | plan
 * The manifest is metadata for the Python API; running needs only the plan,
 * so this reader checks the header, lengths and checksum, the plan header
 * rules of bundle.py:25-32 (plan versions 2 and 3 only), and hands the plan to
 * ug_load, which applies the full validation of graph.c.
 */
#include "uq_graph.h"
#include <string.h>

/* SHA-256 (FIPS 180-4). Round constants: the first 32 bits of the fractional
 * parts of the cube roots of the first 64 primes; initial state: the same for
 * the square roots of the first 8 primes. */
static const uint32_t K256[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

static uint32_t rotr(uint32_t x, unsigned n) { return (x >> n) | (x << (32 - n)); }

static void sha256_block(uint32_t h[8], const uint8_t *p)
{
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K256[i] + w[i];
        uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        k = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
}

void uq_sha256(const void *data, uint64_t len, uint8_t out[32])
{
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au, 0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    const uint8_t *p = data;
    uint64_t full = len / 64;
    for (uint64_t i = 0; i < full; i++) sha256_block(h, p + 64 * i);
    uint8_t tail[128] = {0};
    uint64_t rest = len - 64 * full;
    memcpy(tail, p + 64 * full, (size_t)rest);
    tail[rest] = 0x80;
    uint64_t blocks = rest + 9 <= 64 ? 1 : 2;
    uint64_t bits = len * 8;
    for (int i = 0; i < 8; i++) tail[64 * blocks - 1 - i] = (uint8_t)(bits >> (8 * i));
    for (uint64_t i = 0; i < blocks; i++) sha256_block(h, tail + 64 * i);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(h[i] >> 8);
        out[4 * i + 3] = (uint8_t)h[i];
    }
}

#define HEADER_BYTES 52u
#define MAX_MANIFEST (4u * 1024u * 1024u)
#define MAX_PLAN (17u * 1024u * 1024u)

static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

int ug_bundle_plan(const void *file, uint64_t len, const void **plan, uint32_t *plan_len)
{
    const uint8_t *p = file;
    if (!p || len < HEADER_BYTES) return 30;
    uint32_t version = rd32(p + 8), nm = rd32(p + 12), np = rd32(p + 16);
    if (memcmp(p, "UQMODEL\0", 8) != 0 || version != 1 || nm < 1 || nm > MAX_MANIFEST || np < 32 || np > MAX_PLAN) return 30;
    if (len != (uint64_t)HEADER_BYTES + nm + np) return 30;
    uint8_t digest[32];
    uq_sha256(p + HEADER_BYTES, (uint64_t)nm + np, digest);
    if (memcmp(digest, p + 20, 32) != 0) return 31;
    const uint8_t *q = p + HEADER_BYTES + nm;
    uint32_t pv = rd32(q + 4);
    if (rd32(q) != 0x55474e31u || (pv != 2 && pv != 3)) return 32;
    if (plan) *plan = q;
    if (plan_len) *plan_len = np;
    return 0;
}

int ug_load_bundle(const void *file, uint64_t len)
{
    const void *plan;
    uint32_t np;
    int rc = ug_bundle_plan(file, len, &plan, &np);
    if (rc) return rc;
    return ug_load(plan, np);
}
