/*
 * gq_oracle.c -- CPU restatement of gguf-rs's quantized dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
 * Nothing in the product library links or calls this file.
 *
 * Compiled with -O2 -ffp-contract=off: Rust never fuses a*b-c into an FMA,
 * and the dequantized values must come out bit-identical to the reference.
 * Citations are into the reference crate (src/...).
 *
 * Pinning (how each function is checked, in tests/test_oracle.py):
 *   f16<->f32        exhaustive over 65536 patterns vs numpy float16.
 *   Q8_0             q8_0.rs:109-170 known answers + brute-force fp64 dot.
 *   get_scale_min_k4 q4_k.rs:228-241 known-answer vectors + bit-packing
 *                    round trip over all 64x64 (sc, m) pairs.
 *   Q4_K / Q5_K      closed-form dequant (numpy), q4_k.rs:243-259 fused ==
 *                    dequant-then-dot, fp64 brute-force dot.
 *   Q6_K             closed-form element mapping (numpy, written from the
 *                    ggml layout independently), q6_k.rs:147-164.
 *   Q8_K             q8_k.rs:97-138 invariants (bsums, zero block, padding,
 *                    round-trip bound).
 *   per-32 Q8 pack   model/mod.rs:574-583 restated in numpy.
 *   IQ3_XXS          parity unpinned: the reference has no implementation
 *                    (quant/mod.rs:7, :38-41).  This is a restatement of
 *                    ggml's published dequantize_row_iq3_xxs; its codebook is
 *                    a placeholder unless the caller installs the real one.
 */
#define _GNU_SOURCE  /* sched_getaffinity */
#include "gq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ types */

size_t gqo_block_size(int t) {
    switch (t) {
    case GQO_F32: case GQO_F16: case GQO_BF16: return 1;
    case GQO_Q8_0: return 32;
    case GQO_Q4_K: case GQO_Q5_K: case GQO_Q6_K: case GQO_Q8_K: case GQO_IQ3_XXS: return 256;
    default: return 0;
    }
}

size_t gqo_block_bytes(int t) {
    switch (t) {
    case GQO_F32: return 4;
    case GQO_F16: case GQO_BF16: return 2;
    case GQO_Q8_0: return 34;
    case GQO_Q4_K: return 144;
    case GQO_Q5_K: return 176;
    case GQO_Q6_K: return 210;
    case GQO_Q8_K: return 292;
    case GQO_IQ3_XXS: return 98;
    default: return 0;
    }
}

size_t gqo_type_size(int t, size_t n) {
    size_t bs = gqo_block_size(t);
    if (!bs) return 0;
    return ((n + bs - 1) / bs) * gqo_block_bytes(t);
}

/* ------------------------------------------------------------- f16 <-> f32 */

/* IEEE binary16 -> binary32, exact (what half::f16::to_f32 computes). */
float gqo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (half::f16::from_f32). */
uint16_t gqo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffff;
    if (exp == 0xff) /* inf / nan (keep a quiet payload bit for nan) */
        return sign | 0x7c00 | (man ? (0x200 | (man >> 13)) : 0);
    int e = (int)exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign; /* below half the smallest subnormal */
        man |= 0x800000;
        int shift = 14 - e; /* 14..24 */
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return sign | (uint16_t)hm;
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1fff;
    uint16_t out = sign | (uint16_t)(e << 10) | (uint16_t)hm;
    if (rem > 0x1000 || (rem == 0x1000 && (hm & 1))) out++; /* carry may bump exp: correct */
    return out;
}

static inline float rd_f16(const uint8_t *p) { return gqo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* -------------------------------------------------------------------- Q8_0 */

/* q8_0.rs:14-51 */
int gqo_dequant_q8_0(const uint8_t *data, size_t nbytes, size_t n, float *out) {
    size_t nb = (n + 31) / 32;
    if (nbytes < nb * 34) return GQO_ESHORT;
    size_t o = 0;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * 34;
        float scale = rd_f16(blk);
        size_t cnt = (b == nb - 1) ? n - b * 32 : 32;
        for (size_t i = 0; i < cnt; i++) out[o++] = scale * (float)(int8_t)blk[2 + i];
    }
    return 0;
}

/* q8_0.rs:58-90: per block sequential sum of q*x, then acc += scale*block_dot */
int gqo_dot_q8_0(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res) {
    size_t nb = (n + 31) / 32;
    if (nbytes < nb * 34) return GQO_ESHORT;
    float acc = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * 34;
        float scale = rd_f16(blk);
        size_t start = b * 32;
        size_t cnt = n - start < 32 ? n - start : 32;
        float bd = 0.0f;
        for (size_t i = 0; i < cnt; i++) bd += (float)(int8_t)blk[2 + i] * x[start + i];
        acc += scale * bd;
    }
    *res = acc;
    return 0;
}

/* -------------------------------------------------------------------- Q4_K */

/* q4_k.rs:26-35 */
void gqo_get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* q4_k.rs:37-91 (also the Q5_K variant, q5_k.rs:41-99, when qh != NULL) */
static void dequant_k4_block(const uint8_t *blk, const uint8_t *qh, const uint8_t *qs, float *y) {
    float d = rd_f16(blk), dmin = rd_f16(blk + 2);
    const uint8_t *scales = blk + 4;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc0, m0, sc1, m1s;
        gqo_get_scale_min_k4(is, scales, &sc0, &m0);
        float d1 = d * (float)sc0, m1 = dmin * (float)m0;
        gqo_get_scale_min_k4(is + 1, scales, &sc1, &m1s);
        float d2 = d * (float)sc1, m2 = dmin * (float)m1s;
        const uint8_t *q = qs + j / 2;
        for (int l = 0; l < 32; l++) {
            int hb = qh ? (((qh[l] >> is) & 1) << 4) : 0;
            y[j + l] = d1 * (float)((q[l] & 0xF) + hb) - m1;
        }
        for (int l = 0; l < 32; l++) {
            int hb = qh ? (((qh[l] >> (is + 1)) & 1) << 4) : 0;
            y[j + 32 + l] = d2 * (float)((q[l] >> 4) + hb) - m2;
        }
        is += 2;
    }
}

static int dequant_k4(const uint8_t *data, size_t nbytes, size_t n, float *out, int q5) {
    size_t bb = q5 ? 176 : 144;
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * bb) return GQO_ESHORT;
    float tmp[256];
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * bb;
        dequant_k4_block(blk, q5 ? blk + 16 : NULL, blk + (q5 ? 48 : 16), tmp);
        size_t cnt = n - b * 256 < 256 ? n - b * 256 : 256;
        memcpy(out + b * 256, tmp, cnt * sizeof(float));
    }
    return 0;
}

int gqo_dequant_q4_k(const uint8_t *d, size_t nb, size_t n, float *o) { return dequant_k4(d, nb, n, o, 0); }
int gqo_dequant_q5_k(const uint8_t *d, size_t nb, size_t n, float *o) { return dequant_k4(d, nb, n, o, 1); }

/* dot_q4_k_group (q4_k.rs:152-203) / dot_q5_k_group (q5_k.rs:249-317): an
 * 8-lane f32 accumulator, lane k takes ((d1*lo - m1)*x_lo) then
 * ((d2*hi - m2)*x_hi) for each of the 4 byte-octets, then a sequential
 * horizontal sum.  Out-of-range x lanes read as 0.0 (load_f32x8_partial). */
static float dot_k4_group(float d1, float m1, float d2, float m2, const uint8_t *qs,
                          const uint8_t *qh, int sh1, int sh2, const float *x, size_t avail) {
    float sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t base = 0; base < 32; base += 8) {
        for (int k = 0; k < 8; k++) {
            uint8_t q = qs[base + k];
            int h1 = qh ? (((qh[base + k] >> sh1) & 1) << 4) : 0;
            int h2 = qh ? (((qh[base + k] >> sh2) & 1) << 4) : 0;
            float lo = (float)((q & 0xF) | h1);
            float hi = (float)((q >> 4) | h2);
            float xl = (base + k < avail) ? x[base + k] : 0.0f;
            float xh = (32 + base + k < avail) ? x[32 + base + k] : 0.0f;
            float t = d1 * lo;
            t = t - m1;
            sum[k] = sum[k] + t * xl;
            float u = d2 * hi;
            u = u - m2;
            sum[k] = sum[k] + u * xh;
        }
    }
    float s = 0.0f; /* arr.iter().sum(): sequential */
    for (int k = 0; k < 8; k++) s += sum[k];
    return s;
}

/* q4_k.rs:95-147, q5_k.rs:189-247 */
static int dot_k4(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res, int q5) {
    size_t bb = q5 ? 176 : 144;
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * bb) return GQO_ESHORT;
    float acc = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * bb;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *scales = blk + 4;
        const uint8_t *qh = q5 ? blk + 16 : NULL;
        const uint8_t *qs = blk + (q5 ? 48 : 16);
        size_t bo = b * 256;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc0, m0, sc1, m1s;
            gqo_get_scale_min_k4(is, scales, &sc0, &m0);
            float d1 = d * (float)sc0, m1 = dmin * (float)m0;
            gqo_get_scale_min_k4(is + 1, scales, &sc1, &m1s);
            float d2 = d * (float)sc1, m2 = dmin * (float)m1s;
            size_t off = bo + j;
            size_t avail = n > off ? n - off : 0;
            acc += dot_k4_group(d1, m1, d2, m2, qs + j / 2, qh, is, is + 1, avail ? x + off : x, avail);
            is += 2;
        }
    }
    *res = acc;
    return 0;
}

int gqo_dot_q4_k(const uint8_t *d, size_t nb, const float *x, size_t n, float *r) { return dot_k4(d, nb, x, n, r, 0); }
int gqo_dot_q5_k(const uint8_t *d, size_t nb, const float *x, size_t n, float *r) { return dot_k4(d, nb, x, n, r, 1); }

/* -------------------------------------------------------------------- Q6_K */

/* q6_k.rs:25-32 */
static inline void quads(const uint8_t *ql, const uint8_t *qh, int l, int q[4]) {
    uint8_t h = qh[l];
    q[0] = ((ql[l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
    q[1] = ((ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
    q[2] = ((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
    q[3] = ((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
}

/* q6_k.rs:34-77: y = (d * sc) * q */
int gqo_dequant_q6_k(const uint8_t *data, size_t nbytes, size_t n, float *out) {
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * 210) return GQO_ESHORT;
    float tmp[256];
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * 210;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = rd_f16(blk + 208);
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            for (int l = 0; l < 32; l++) {
                int is = l / 16, q[4];
                quads(ql, qh, l, q);
                tmp[h * 128 + l] = d * (float)sc[h * 8 + is] * (float)q[0];
                tmp[h * 128 + l + 32] = d * (float)sc[h * 8 + is + 2] * (float)q[1];
                tmp[h * 128 + l + 64] = d * (float)sc[h * 8 + is + 4] * (float)q[2];
                tmp[h * 128 + l + 96] = d * (float)sc[h * 8 + is + 6] * (float)q[3];
            }
        }
        size_t cnt = n - b * 256 < 256 ? n - b * 256 : 256;
        memcpy(out + b * 256, tmp, cnt * sizeof(float));
    }
    return 0;
}

/* q6_k.rs:82-131: acc += ((d*sc)*q)*x, one scalar accumulator, element order
 * (h, l, quad). */
int gqo_dot_q6_k(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res) {
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * 210) return GQO_ESHORT;
    float acc = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * 210;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = rd_f16(blk + 208);
        size_t bo = b * 256;
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            size_t yh = bo + h * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16, q[4];
                quads(ql, qh, l, q);
                for (int k = 0; k < 4; k++) {
                    size_t idx = yh + l + 32 * k;
                    if (idx < n) {
                        float t = d * (float)sc[h * 8 + is + 2 * k];
                        t = t * (float)q[k];
                        acc += t * x[idx];
                    } else {
                        acc += 0.0f;
                    }
                }
            }
        }
    }
    *res = acc;
    return 0;
}

/* ----------------------------------------------------------------- IQ3_XXS */

/* The reference has no IQ3_XXS arithmetic (quant/mod.rs:7,38-41); this is a
 * restatement of ggml's published dequantize_row_iq3_xxs:
 *   block: f16 d | qs[64] grid indices | 8 x u32 aux (per 32 elements):
 *   aux bits 0..27 = four 7-bit sign indices, bits 28..31 = scale s;
 *   db = d * (0.5 + s) * 0.5;
 *   signs7 -> 8 sign bits via even parity: ksigns[i] = i | (popcount(i)&1)<<7;
 *   for each of 4 groups of 8: two grid entries (4 magnitude bytes each),
 *   y[j] = db * mag[j] * (sign bit j ? -1 : 1).
 * The codebook ggml ships (iq3xxs_grid) is not available here; the default
 * below is a deterministic placeholder over ggml's magnitude alphabet
 * {4,12,20,28,36,44,52,62}.  gqo_set_iq3xxs_grid installs another table.
 * Parity unpinned. */
static uint32_t g_iq3_grid[256];
static int g_iq3_init = 0;

static void iq3_default_grid(uint32_t *g) {
    static const uint8_t mags[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t h = i * 0x9E3779B1u;
        h ^= h >> 15;
        uint32_t e = 0;
        for (int k = 0; k < 4; k++) e |= (uint32_t)mags[(h >> (3 * k)) & 7] << (8 * k);
        g[i] = e;
    }
}

static const uint32_t *iq3_grid(void) {
    if (!g_iq3_init) { iq3_default_grid(g_iq3_grid); g_iq3_init = 1; }
    return g_iq3_grid;
}

void gqo_set_iq3xxs_grid(const uint32_t *grid) {
    if (grid) memcpy(g_iq3_grid, grid, sizeof(g_iq3_grid));
    else iq3_default_grid(g_iq3_grid);
    g_iq3_init = 1;
}
void gqo_get_iq3xxs_grid(uint32_t *grid) { memcpy(grid, iq3_grid(), sizeof(g_iq3_grid)); }

static inline uint8_t ksign(uint32_t i) {
    return (uint8_t)(i | ((uint32_t)(__builtin_popcount(i) & 1) << 7));
}

static void dequant_iq3_block(const uint8_t *blk, float *y) {
    const uint32_t *grid = iq3_grid();
    float d = rd_f16(blk);
    const uint8_t *qs = blk + 2;
    const uint8_t *sas = blk + 2 + 64;
    for (int ib = 0; ib < 8; ib++) {
        uint32_t aux = (uint32_t)sas[4 * ib] | ((uint32_t)sas[4 * ib + 1] << 8) |
                       ((uint32_t)sas[4 * ib + 2] << 16) | ((uint32_t)sas[4 * ib + 3] << 24);
        float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            uint8_t signs = ksign((aux >> (7 * l)) & 127);
            uint32_t g1 = grid[qs[8 * ib + 2 * l]], g2 = grid[qs[8 * ib + 2 * l + 1]];
            for (int j = 0; j < 4; j++) {
                float m1 = (float)((g1 >> (8 * j)) & 0xff), m2 = (float)((g2 >> (8 * j)) & 0xff);
                y[32 * ib + 8 * l + j] = db * m1 * ((signs >> j) & 1 ? -1.0f : 1.0f);
                y[32 * ib + 8 * l + j + 4] = db * m2 * ((signs >> (j + 4)) & 1 ? -1.0f : 1.0f);
            }
        }
    }
}

int gqo_dequant_iq3_xxs(const uint8_t *data, size_t nbytes, size_t n, float *out) {
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * 98) return GQO_ESHORT;
    float tmp[256];
    for (size_t b = 0; b < nb; b++) {
        dequant_iq3_block(data + b * 98, tmp);
        size_t cnt = n - b * 256 < 256 ? n - b * 256 : 256;
        memcpy(out + b * 256, tmp, cnt * sizeof(float));
    }
    return 0;
}

/* The reference's generic dot_row fallback (quant/mod.rs:76-80):
 * dequant then sequential sum of w*x. */
int gqo_dot_iq3_xxs(const uint8_t *data, size_t nbytes, const float *x, size_t n, float *res) {
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * 98) return GQO_ESHORT;
    float tmp[256], acc = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        dequant_iq3_block(data + b * 98, tmp);
        size_t cnt = n - b * 256 < 256 ? n - b * 256 : 256;
        for (size_t i = 0; i < cnt; i++) acc += tmp[i] * x[b * 256 + i];
    }
    *res = acc;
    return 0;
}

/* ------------------------------------------------------------- dispatchers */

int gqo_dequant(int t, const uint8_t *d, size_t nb, size_t n, float *o) {
    switch (t) {
    case GQO_Q8_0: return gqo_dequant_q8_0(d, nb, n, o);
    case GQO_Q4_K: return gqo_dequant_q4_k(d, nb, n, o);
    case GQO_Q5_K: return gqo_dequant_q5_k(d, nb, n, o);
    case GQO_Q6_K: return gqo_dequant_q6_k(d, nb, n, o);
    case GQO_IQ3_XXS: return gqo_dequant_iq3_xxs(d, nb, n, o);
    default: return GQO_EDTYPE;
    }
}

/* quant/mod.rs:65-83 */
int gqo_dot_row(int t, const uint8_t *d, size_t nb, const float *x, size_t n, float *r) {
    switch (t) {
    case GQO_Q8_0: return gqo_dot_q8_0(d, nb, x, n, r);
    case GQO_Q4_K: return gqo_dot_q4_k(d, nb, x, n, r);
    case GQO_Q5_K: return gqo_dot_q5_k(d, nb, x, n, r);
    case GQO_Q6_K: return gqo_dot_q6_k(d, nb, x, n, r);
    case GQO_IQ3_XXS: return gqo_dot_iq3_xxs(d, nb, x, n, r);
    default: return GQO_EDTYPE;
    }
}

/* -------------------------------------------------------------------- Q8_K */

/* q8_k.rs:49-91 */
void gqo_quantize_row_q8_k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums) {
    size_t nb = (n + 255) / 256;
    memset(qs, 0, nb * 256);
    for (size_t b = 0; b < nb; b++) {
        size_t s = b * 256, e = s + 256 < n ? s + 256 : n;
        float amax = 0.0f, mx = 0.0f;
        for (size_t i = s; i < e; i++) {
            float av = fabsf(x[i]);
            if (av > amax) { amax = av; mx = x[i]; }
        }
        d[b] = 0.0f;
        if (amax > 0.0f) {
            float iscale = -127.0f / mx;
            for (size_t i = s; i < e; i++) {
                int r = (int)roundf(iscale * x[i]);
                qs[i] = (int8_t)(r < 127 ? r : 127);
            }
            d[b] = 1.0f / iscale;
        }
        for (int g = 0; g < 16; g++) {
            int16_t acc = 0;
            for (int k = 0; k < 16; k++) acc = (int16_t)(acc + qs[b * 256 + g * 16 + k]);
            bsums[b * 16 + g] = acc;
        }
    }
}

/* q5_k.rs:126-184 */
int gqo_dot_q5_k_q8k(const uint8_t *data, size_t nbytes, size_t n, const float *dx8,
                     const int8_t *xq, const int16_t *bsums, float *res) {
    size_t nb = (n + 255) / 256;
    if (nbytes < nb * 176) return GQO_ESHORT;
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = data + b * 176;
        float d = rd_f16(blk), dmin = rd_f16(blk + 2);
        const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
        const int8_t *xb = xq + b * 256;
        const int16_t *bs = bsums + b * 16;
        int32_t acc_pos = 0, acc_min = 0;
        for (int is = 0; is < 8; is++) {
            uint8_t sc, m;
            gqo_get_scale_min_k4(is, scales, &sc, &m);
            int32_t pos = 0;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = qs[32 * (is / 2) + l];
                int nib = (is % 2 == 0) ? (byte & 0xF) : (byte >> 4);
                int hi = ((qh[l] >> is) & 1) << 4;
                pos += (nib | hi) * (int32_t)xb[32 * is + l];
            }
            int32_t ms = (int32_t)bs[2 * is] + (int32_t)bs[2 * is + 1];
            acc_pos += (int32_t)sc * pos;
            acc_min += (int32_t)m * ms;
        }
        float t1 = d * (float)acc_pos;
        float t2 = dmin * (float)acc_min;
        sumf += dx8[b] * (t1 - t2);
    }
    *res = sumf;
    return 0;
}

/* ------------------------------------------------------- per-32 Q8 pack */

/* KvDtype::Q8_0::pack (model/mod.rs:574-583): scale = amax/127 (1.0 for an
 * all-zero block), stored as f16; q = clamp(round(x / scale), -127, 127)
 * with the f32 (unrounded) scale. */
void gqo_quantize_q8_32(const float *x, size_t n, uint16_t *scale_f16, int8_t *q) {
    size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        size_t s = b * 32, e = s + 32 < n ? s + 32 : n;
        float amax = 0.0f;
        for (size_t i = s; i < e; i++) amax = fmaxf(amax, fabsf(x[i]));
        float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        scale_f16[b] = gqo_f32_to_f16(scale);
        for (size_t i = s; i < e; i++) {
            float r = roundf(x[i] / scale);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            q[i] = (int8_t)r;
        }
        for (size_t i = e; i < s + 32; i++) q[i] = 0;
    }
}

/* ------------------------------------------------------------ matmul_into */

typedef struct {
    int dtype;
    const uint8_t *w;
    size_t nbytes, in_dim, r0, r1, batch;
    const float *x;
    float *out;
    int rc;
} job_t;

static void *matvec_job(void *p) {
    job_t *j = (job_t *)p;
    size_t rb = gqo_type_size(j->dtype, j->in_dim);
    for (size_t r = j->r0; r < j->r1 && !j->rc; r++) {
        size_t off = r * rb;
        if (off + rb > j->nbytes) { j->rc = GQO_ESHORT; break; }
        j->rc = gqo_dot_row(j->dtype, j->w + off, j->nbytes - off, j->x, j->in_dim, &j->out[r]);
    }
    return NULL;
}

/* nthreads 0: the cores this process may run on (rayon's default pool),
 * capped by GQO_MAX_THREADS (default 16, the GPU box's CPU share). */
static int hw_threads(int n) {
    if (n > 0) return n;
    cpu_set_t set;
    int c = sched_getaffinity(0, sizeof set, &set) == 0 ? CPU_COUNT(&set) : (int)sysconf(_SC_NPROCESSORS_ONLN);
    const char *e = getenv("GQO_MAX_THREADS");
    int cap = e && atoi(e) > 0 ? atoi(e) : 16;
    if (c > cap) c = cap;
    return c > 0 ? c : 1;
}

static int run_jobs(job_t *proto, size_t rows, int nthreads, void *(*fn)(void *)) {
    int nt = hw_threads(nthreads);
    if ((size_t)nt > rows) nt = rows ? (int)rows : 1;
    pthread_t th[256];
    job_t jobs[256];
    if (nt > 256) nt = 256;
    size_t per = (rows + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        jobs[t] = *proto;
        jobs[t].r0 = (size_t)t * per < rows ? (size_t)t * per : rows;
        jobs[t].r1 = jobs[t].r0 + per < rows ? jobs[t].r0 + per : rows;
        jobs[t].rc = 0;
        if (nt == 1) fn(&jobs[t]);
        else pthread_create(&th[t], NULL, fn, &jobs[t]);
    }
    int rc = 0;
    for (int t = 0; t < nt; t++) {
        if (nt > 1) pthread_join(th[t], NULL);
        if (jobs[t].rc && !rc) rc = jobs[t].rc;
    }
    return rc;
}

/* Rows through the per-format float dot (quant::dot_row), row-parallel:
 * the non-Q5_K branch of WeightMap::matmul_into (model/mod.rs:396-402) and
 * the per-row dots of ffn_gate_up (cpu_path.rs:222-229). */
int gqo_matmul_rows(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                    float *out, size_t out_dim, int nthreads) {
    if (!gqo_block_size(dtype) || dtype == GQO_F32 || dtype == GQO_F16 || dtype == GQO_BF16)
        return GQO_EDTYPE;
    job_t p = {dtype, w, nbytes, in_dim, 0, 0, 0, x, out, 0};
    return run_jobs(&p, out_dim, nthreads, matvec_job);
}

typedef struct {
    const uint8_t *w;
    size_t nbytes, in_dim, r0, r1;
    const float *d8;
    const int8_t *q8;
    const int16_t *bs;
    float *out;
    int rc;
} q8k_job;

static void *q8k_rows_job(void *p) {
    q8k_job *j = (q8k_job *)p;
    size_t rb = gqo_type_size(GQO_Q5_K, j->in_dim);
    for (size_t r = j->r0; r < j->r1 && !j->rc; r++) {
        size_t off = r * rb;
        if (off + rb > j->nbytes) { j->rc = GQO_ESHORT; break; }
        j->rc = gqo_dot_q5_k_q8k(j->w + off, j->nbytes - off, j->in_dim, j->d8, j->q8, j->bs,
                                 &j->out[r]);
    }
    return NULL;
}

/* model/mod.rs:362-403: Q5_K quantizes x to Q8_K once (q8_k.rs:49-91) and
 * runs dot_q5_k_q8k (q5_k.rs:126-184) per row (model/mod.rs:381-394);
 * every other type takes quant::dot_row. */
int gqo_matmul_into(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                    float *out, size_t out_dim, int nthreads) {
    if (dtype != GQO_Q5_K) return gqo_matmul_rows(dtype, w, nbytes, x, in_dim, out, out_dim, nthreads);
    size_t nb = (in_dim + 255) / 256;
    float *d8 = (float *)malloc(sizeof(float) * (nb ? nb : 1));
    int8_t *q8 = (int8_t *)malloc(nb ? nb * 256 : 1);
    int16_t *bs = (int16_t *)malloc(sizeof(int16_t) * (nb ? nb * 16 : 1));
    gqo_quantize_row_q8_k(x, in_dim, d8, q8, bs);
    int nt = hw_threads(nthreads);
    if ((size_t)nt > out_dim) nt = out_dim ? (int)out_dim : 1;
    if (nt > 256) nt = 256;
    pthread_t th[256];
    q8k_job jobs[256];
    size_t per = (out_dim + nt - 1) / nt;
    for (int t = 0; t < nt; t++) {
        size_t r0 = (size_t)t * per < out_dim ? (size_t)t * per : out_dim;
        size_t r1 = r0 + per < out_dim ? r0 + per : out_dim;
        q8k_job j = {w, nbytes, in_dim, r0, r1, d8, q8, bs, out, 0};
        jobs[t] = j;
        if (nt == 1) q8k_rows_job(&jobs[t]);
        else pthread_create(&th[t], NULL, q8k_rows_job, &jobs[t]);
    }
    int rc = 0;
    for (int t = 0; t < nt; t++) {
        if (nt > 1) pthread_join(th[t], NULL);
        if (jobs[t].rc && !rc) rc = jobs[t].rc;
    }
    free(d8);
    free(q8);
    free(bs);
    return rc;
}

/* cpu_backend.rs:38-65 */
int gqo_matmul_dequant(int dtype, const uint8_t *w, size_t nbytes, const float *x, size_t in_dim,
                       float *out, size_t out_dim) {
    if (dtype != GQO_Q8_0 && dtype != GQO_Q4_K && dtype != GQO_Q5_K && dtype != GQO_Q6_K)
        return GQO_EDTYPE;
    size_t rb = gqo_type_size(dtype, in_dim);
    for (size_t r = 0; r < out_dim; r++) {
        size_t off = r * rb;
        if (off > nbytes) return GQO_ESHORT;
        int rc = gqo_dot_row(dtype, w + off, nbytes - off, x, in_dim, &out[r]);
        if (rc) return rc;
    }
    return 0;
}

/* model/mod.rs:446-456: dequant row once, then per token a sequential sum */
int gqo_matmul_batch_rows(int dtype, const uint8_t *w, size_t nbytes, const float *x,
                          size_t in_dim, size_t batch, size_t r0, size_t r1, float *rowmajor) {
    size_t rb = gqo_type_size(dtype, in_dim);
    if (!rb) return GQO_EDTYPE;
    float *wr = (float *)malloc(in_dim * sizeof(float));
    int rc = 0;
    for (size_t r = r0; r < r1 && !rc; r++) {
        size_t off = r * rb;
        if (off + rb > nbytes) { rc = GQO_ESHORT; break; }
        rc = gqo_dequant(dtype, w + off, rb, in_dim, wr);
        if (rc) break;
        for (size_t t = 0; t < batch; t++) {
            const float *xt = x + t * in_dim;
            float s = 0.0f;
            for (size_t i = 0; i < in_dim; i++) s += wr[i] * xt[i];
            rowmajor[(r - r0) * batch + t] = s;
        }
    }
    free(wr);
    return rc;
}

static void *batch_job(void *p) {
    job_t *j = (job_t *)p;
    if (j->r1 > j->r0)
        j->rc = gqo_matmul_batch_rows(j->dtype, j->w, j->nbytes, j->x, j->in_dim, j->batch, j->r0,
                                      j->r1, j->out + j->r0 * j->batch);
    return NULL;
}

/* model/mod.rs:414-464 */
int gqo_matmul_batch_into(int dtype, const uint8_t *w, size_t nbytes, const float *x,
                          size_t in_dim, size_t batch, float *out, size_t out_dim, int nthreads) {
    float *rm = (float *)malloc(out_dim * batch * sizeof(float));
    if (!rm) return GQO_ESHORT;
    job_t p = {dtype, w, nbytes, in_dim, 0, 0, batch, x, rm, 0};
    int rc = run_jobs(&p, out_dim, nthreads, batch_job);
    if (!rc)
        for (size_t r = 0; r < out_dim; r++)
            for (size_t t = 0; t < batch; t++) out[t * out_dim + r] = rm[r * batch + t];
    free(rm);
    return rc;
}

/* ------------------------------------------------------------------ MoE */

void gqo_moe_route(const float *logits, int T, int E, int k, int *ids, float *w) {
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t)t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; e++) mx = l[e] > mx ? l[e] : mx;
        float sum = 0.0f;
        for (int e = 0; e < E; e++) sum += expf(l[e] - mx);
        unsigned char taken[4096] = {0};
        for (int s = 0; s < k; s++) {
            int best = -1;
            for (int e = 0; e < E; e++)
                if (!taken[e] && (best < 0 || l[e] > l[best])) best = e;
            taken[best] = 1;
            ids[t * k + s] = best;
            w[t * k + s] = expf(l[best] - mx) / sum;
        }
    }
}

static float silu(float g) { return g / (1.0f + expf(-g)); }

int gqo_moe_ffn(int dtype, const uint8_t *gate, const uint8_t *up, const uint8_t *down, int E,
                int H, int F, const float *x, int T, int k, const int *ids, const float *w,
                float *out, int nthreads) {
    const size_t rb_h = gqo_type_size(dtype, (size_t)H), rb_f = gqo_type_size(dtype, (size_t)F);
    float *g = (float *)malloc(sizeof(float) * F), *u = (float *)malloc(sizeof(float) * F);
    float *h = (float *)malloc(sizeof(float) * F), *y = (float *)malloc(sizeof(float) * H);
    int rc = 0;
    for (int t = 0; t < T && !rc; t++) {
        float *o = out + (size_t)t * H;
        for (int i = 0; i < H; i++) o[i] = 0.0f;
        for (int s = 0; s < k && !rc; s++) {
            const int e = ids[t * k + s];
            if (e < 0 || e >= E) { rc = GQO_ERANGE; break; }
            const uint8_t *ge = gate + (size_t)e * F * rb_h, *ue = up + (size_t)e * F * rb_h;
            const uint8_t *de = down + (size_t)e * H * rb_f;
            rc = gqo_matmul_into(dtype, ge, (size_t)F * rb_h, x + (size_t)t * H, H, g, F, nthreads);
            if (!rc) rc = gqo_matmul_into(dtype, ue, (size_t)F * rb_h, x + (size_t)t * H, H, u, F, nthreads);
            if (rc) break;
            for (int i = 0; i < F; i++) h[i] = silu(g[i]) * u[i];
            rc = gqo_matmul_into(dtype, de, (size_t)H * rb_f, h, F, y, H, nthreads);
            if (rc) break;
            const float ws = w[t * k + s];
            for (int i = 0; i < H; i++) o[i] += ws * y[i];
        }
    }
    free(g); free(u); free(h); free(y);
    return rc;
}

/* --------------------------------------------------------------- decode */

/* cpu_path.rs:67-74: sum of squares (sequential), rms = sqrt(ss/n + eps),
 * out = w * x / rms */
static void rms_norm(const float *x, const float *w, int n, float eps, float *out) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    float rms = sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = w[i] * x[i] / rms;
}

/* cpu_path.rs:99-133 (freq_scale = 1) */
static void rope(float *q, float *k, int n_heads, int n_kv, int hd, float theta, int pos) {
    int half = hd / 2;
    float *sn = (float *)malloc(sizeof(float) * half), *cs = (float *)malloc(sizeof(float) * half);
    for (int d = 0; d < half; d++) {
        float freq = (float)pos * 1.0f / powf(theta, 2.0f * (float)d / (float)hd);
        sn[d] = sinf(freq);
        cs[d] = cosf(freq);
    }
    for (int pass = 0; pass < 2; pass++) {
        float *v = pass ? k : q;
        int nh = pass ? n_kv : n_heads;
        for (int h = 0; h < nh; h++) {
            float *p = v + (size_t)h * hd;
            for (int d = 0; d < half; d++) {
                float x0 = p[d], x1 = p[d + half];
                p[d] = x0 * cs[d] - x1 * sn[d];
                p[d + half] = x0 * sn[d] + x1 * cs[d];
            }
        }
    }
    free(sn);
    free(cs);
}

/* gqo_f16_to_f32 tabulated over all 65536 patterns (same values). */
static float g_f16_tab[65536];
static pthread_once_t g_f16_once = PTHREAD_ONCE_INIT;
static void f16_tab_init(void) {
    for (uint32_t i = 0; i < 65536; i++) g_f16_tab[i] = gqo_f16_to_f32((uint16_t)i);
}
static const float *f16_table(void) {
    pthread_once(&g_f16_once, f16_tab_init);
    return g_f16_tab;
}

typedef struct {
    const float *q, *kall, *vall;
    float *att;
    int n, hd, kvd, group, h0, h1;
} attn_job;

static void *attn_worker(void *p) {
    attn_job *j = (attn_job *)p;
    const int hd = j->hd, kvd = j->kvd, n = j->n;
    float *sc = (float *)malloc(sizeof(float) * n);
    const float sq = sqrtf((float)hd);
    for (int h = j->h0; h < j->h1; h++) {
        const int kh = h / j->group;
        const float *qh = j->q + (size_t)h * hd;
        for (int t = 0; t < n; t++) {
            const float *kt = j->kall + (size_t)t * kvd + (size_t)kh * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; d++) dot += qh[d] * kt[d];
            sc[t] = dot / sq;
        }
        float mx = -INFINITY;
        for (int t = 0; t < n; t++) mx = sc[t] > mx ? sc[t] : mx;
        for (int t = 0; t < n; t++) sc[t] = expf(sc[t] - mx);
        float sum = 0.0f;
        for (int t = 0; t < n; t++) sum += sc[t];
        for (int t = 0; t < n; t++) sc[t] /= sum;
        for (int t = 0; t < n; t++) {
            const float *vt = j->vall + (size_t)t * kvd + (size_t)kh * hd;
            for (int d = 0; d < hd; d++) j->att[h * hd + d] += sc[t] * vt[d];
        }
    }
    free(sc);
    return NULL;
}

int gqo_decode_step(const gqo_model *m, int token, int pos, float *logits, int nthreads) {
    const int H = m->hidden, hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv_heads;
    const int kvd = nkv * hd, F = m->ffn, group = nh / nkv, n = pos + 1;
    float *x = (float *)malloc(sizeof(float) * H), *xn = (float *)malloc(sizeof(float) * H);
    float *q = (float *)malloc(sizeof(float) * nh * hd), *k = (float *)malloc(sizeof(float) * kvd);
    float *v = (float *)malloc(sizeof(float) * kvd), *att = (float *)malloc(sizeof(float) * nh * hd);
    float *proj = (float *)malloc(sizeof(float) * H), *act = (float *)malloc(sizeof(float) * F);
    float *g = (float *)malloc(sizeof(float) * F), *u = (float *)malloc(sizeof(float) * F);
    float *kall = (float *)malloc(sizeof(float) * (size_t)n * kvd);
    float *vall = (float *)malloc(sizeof(float) * (size_t)n * kvd);
    int rc = 0;
    if (m->kv_q8 && (kvd % 32 || kvd > 32768)) rc = -1;
    memcpy(x, m->embd + (size_t)token * H, sizeof(float) * H);
    for (int L = 0; L < m->n_layers && !rc; L++) {
        const int *lt = m->layer_types ? m->layer_types + 7 * L : NULL;
        const int tq = lt ? lt[0] : m->attn_type, tk = lt ? lt[1] : m->attn_type;
        const int tv = lt ? lt[2] : m->attn_type, to = lt ? lt[3] : m->attn_type;
        const int tg = lt ? lt[4] : m->gate_up_type, tu = lt ? lt[5] : m->gate_up_type;
        const int td = lt ? lt[6] : m->down_type;
        rms_norm(x, m->attn_norm[L], H, m->eps, xn);
        rc |= gqo_matmul_into(tq, m->wq[L], gqo_type_size(tq, H) * nh * hd, xn, H, q, nh * hd, nthreads);
        rc |= gqo_matmul_into(tk, m->wk[L], gqo_type_size(tk, H) * kvd, xn, H, k, kvd, nthreads);
        rc |= gqo_matmul_into(tv, m->wv[L], gqo_type_size(tv, H) * kvd, xn, H, v, kvd, nthreads);
        rope(q, k, nh, nkv, hd, m->theta, pos);
        const float *tab = f16_table();
        if (m->kv_q8) {
            /* KvDtype::Q8_0: pack (model/mod.rs:574-583) the new row, unpack
             * (:595-602) every row up to pos. */
            const int nb = kvd / 32;
            const size_t rowb = (size_t)nb * 34;
            uint8_t *kc = (uint8_t *)m->kcache[L], *vc = (uint8_t *)m->vcache[L];
            uint16_t sc[2][1024];
            int8_t qq[2][32768];
            gqo_quantize_q8_32(k, (size_t)kvd, sc[0], qq[0]);
            gqo_quantize_q8_32(v, (size_t)kvd, sc[1], qq[1]);
            for (int b = 0; b < nb; b++) {
                uint8_t *kb = kc + (size_t)pos * rowb + 34 * b, *vb = vc + (size_t)pos * rowb + 34 * b;
                kb[0] = (uint8_t)sc[0][b]; kb[1] = (uint8_t)(sc[0][b] >> 8);
                vb[0] = (uint8_t)sc[1][b]; vb[1] = (uint8_t)(sc[1][b] >> 8);
                memcpy(kb + 2, qq[0] + 32 * b, 32);
                memcpy(vb + 2, qq[1] + 32 * b, 32);
            }
            for (size_t t = 0; t < (size_t)n; t++)
                for (int b = 0; b < nb; b++) {
                    const uint8_t *kb = kc + t * rowb + 34 * b, *vb = vc + t * rowb + 34 * b;
                    const float ks = tab[kb[0] | (kb[1] << 8)], vs = tab[vb[0] | (vb[1] << 8)];
                    for (int e = 0; e < 32; e++) {
                        kall[t * kvd + 32 * b + e] = (float)(int8_t)kb[2 + e] * ks;
                        vall[t * kvd + 32 * b + e] = (float)(int8_t)vb[2 + e] * vs;
                    }
                }
        } else {
            uint16_t *kc = m->kcache[L], *vc = m->vcache[L];
            for (int i = 0; i < kvd; i++) {
                kc[(size_t)pos * kvd + i] = gqo_f32_to_f16(k[i]);
                vc[(size_t)pos * kvd + i] = gqo_f32_to_f16(v[i]);
            }
            for (size_t i = 0; i < (size_t)n * kvd; i++) {
                kall[i] = tab[kc[i]];
                vall[i] = tab[vc[i]];
            }
        }
        /* attention_into (cpu_path.rs:141-194); heads are independent and
         * are computed on separate threads (same arithmetic per head). */
        for (int i = 0; i < nh * hd; i++) att[i] = 0.0f;
        attn_job aj = {q, kall, vall, att, n, hd, kvd, group, 0, 0};
        int nt = hw_threads(nthreads);
        if (nt > nh) nt = nh;
        pthread_t th[256];
        attn_job jobs[256];
        int per = (nh + nt - 1) / nt;
        for (int t = 0; t < nt; t++) {
            jobs[t] = aj;
            jobs[t].h0 = t * per < nh ? t * per : nh;
            jobs[t].h1 = (t + 1) * per < nh ? (t + 1) * per : nh;
            pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
        }
        for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
        rc |= gqo_matmul_into(to, m->wo[L], gqo_type_size(to, nh * hd) * H, att, nh * hd, proj, H, nthreads);
        for (int i = 0; i < H; i++) x[i] += proj[i];
        rms_norm(x, m->ffn_norm[L], H, m->eps, xn);
        /* ffn_gate_up (cpu_path.rs:200-232): quant::dot_row per row for
         * every type (no Q8_K branch, unlike matmul_into) */
        rc |= gqo_matmul_rows(tg, m->wgate[L], gqo_type_size(tg, H) * F, xn, H, g, F, nthreads);
        rc |= gqo_matmul_rows(tu, m->wup[L], gqo_type_size(tu, H) * F, xn, H, u, F, nthreads);
        for (int i = 0; i < F; i++) act[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        rc |= gqo_matmul_into(td, m->wdown[L], gqo_type_size(td, F) * H, act, F, proj, H, nthreads);
        for (int i = 0; i < H; i++) x[i] += proj[i];
    }
    /* logits == NULL: a prompt position whose logits nobody reads (the
     * batch path's non-final rows); the head is skipped. */
    if (!rc && logits) {
        rms_norm(x, m->output_norm, H, m->eps, xn);
        rc = gqo_matmul_into(m->head_type, m->lm_head, gqo_type_size(m->head_type, H) * m->vocab,
                             xn, H, logits, m->vocab, nthreads);
    }
    free(x); free(xn); free(q); free(k); free(v); free(att); free(proj); free(act);
    free(g); free(u); free(kall); free(vall);
    return rc;
}

/* sampler.rs:120-131 */
size_t gqo_argmax(const float *xs, size_t n) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (xs[i] > bv) { bv = xs[i]; best = i; }
    return best;
}
