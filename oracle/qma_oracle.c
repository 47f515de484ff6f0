/*
 * qma_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY) for the quantized
 * MoE expert-matmul path of the qma reference engine.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file, as the checker and as the timed CPU baseline.  The GPU library
 * (qwen-mobile-agent_amd/csrc) does not link or call it.
 *
 * Restates, function by function, the reference's scalar/NEON arithmetic.
 * NEON vector ops are restated lane by lane:
 *   vdotq_s32(acc, a, b)   lane j += sum_{t<4} a[4j+t]*b[4j+t]   (int32, exact)
 *   vfmaq_n_f32(acc, v, s) lane j  = fmaf(v[j], s, acc[j])        (fused)
 *   vaddvq_f32(v)          (v0+v1)+(v2+v3)                         (FADDP order)
 *   vcvtaq_s32_f32         round half away from zero, saturating, NaN -> 0
 * Build flags: -O2 -ffp-contract=off (no fusion other than explicit fmaf).
 */
#include "qma_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32                                                             */
/* ------------------------------------------------------------------------ */

/* Exact fp16 -> fp32, restating the portable branch of half_to_float
   (qma.h:107-124; the aarch64 FCVT branch at qma.h:102-105 is exact too). */
float orc_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t f;
    if (exp == 0) {
        if (man == 0) {
            f = sign;
        } else {
            exp = 127 - 15 + 1;
            while (!(man & 0x400u)) { man <<= 1; exp--; }
            man &= 0x3ffu;
            f = sign | (exp << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        f = sign | 0x7f800000u | (man << 13);
    } else {
        f = sign | ((exp + (127 - 15)) << 23) | (man << 13);
    }
    float r;
    memcpy(&r, &f, 4);
    return r;
}

/* fp32 -> fp16, IEEE round-to-nearest-even (the build's synthetic-weight
   quantizers use it; the GPU side uses the hardware RNE conversion). */
uint16_t orc_float_to_half(float x)
{
    uint32_t f;
    memcpy(&f, &x, 4);
    uint32_t sign = (f >> 16) & 0x8000u;
    uint32_t ex = (f >> 23) & 0xffu;
    uint32_t man = f & 0x7fffffu;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0));
    int32_t e = (int32_t)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t out = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) out++;   /* carries into exp */
    return (uint16_t)out;
}

/* ------------------------------------------------------------------------ */
/* Q4_K / Q6_K formats                                                       */
/* ------------------------------------------------------------------------ */

/* 6-bit scale/min unpack: q8k.c:22-30 (same indexing as quants.c:18-26). */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quants.c:29-47 */
void orc_dequant_q4k(const void *blocks, float *y, int64_t k)
{
    const orc_block_q4k *x = (const orc_block_q4k *)blocks;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *q = x[i].qs;
        const float d = orc_half_to_float(x[i].d);
        const float mn = orc_half_to_float(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < ORC_QK_K; j += 64) {
            orc_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = mn * m;
            orc_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = mn * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* quants.c:50-75 */
void orc_dequant_q6k(const void *blocks, float *y, int64_t k)
{
    const orc_block_q6k *x = (const orc_block_q6k *)blocks;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_half_to_float(x[i].d);
        const uint8_t *ql = x[i].ql;
        const uint8_t *qh = x[i].qh;
        const int8_t *sc = x[i].scales;
        for (int n = 0; n < ORC_QK_K; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* fp32 dequantize-then-dot: quants.c:80-105 */
float orc_dot_q4k_f32(const void *row, const float *x, int n)
{
    const orc_block_q4k *W = (const orc_block_q4k *)row;
    const int nb = n / ORC_QK_K;
    float acc = 0.0f;
    for (int i = 0; i < nb; i++) {
        const uint8_t *q = W[i].qs;
        const float d = orc_half_to_float(W[i].d);
        const float mn = orc_half_to_float(W[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < ORC_QK_K; j += 64) {
            orc_scale_min_k4(is + 0, W[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = mn * m;
            orc_scale_min_k4(is + 1, W[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = mn * m;
            const float *xp = x + (size_t)i * ORC_QK_K + j;
            float s1 = 0, s2 = 0;
            for (int l = 0; l < 32; ++l) {
                s1 += (d1 * (q[l] & 0xF) - m1) * xp[l];
                s2 += (d2 * (q[l] >> 4) - m2) * xp[l + 32];
            }
            acc += s1 + s2;
            q += 32;
            is += 2;
        }
    }
    return acc;
}

/* fp32 dequantize-then-dot: quants.c:108-133 */
float orc_dot_q6k_f32(const void *row, const float *x, int n)
{
    const orc_block_q6k *W = (const orc_block_q6k *)row;
    const int nb = n / ORC_QK_K;
    float acc = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float d = orc_half_to_float(W[i].d);
        const uint8_t *ql = W[i].ql;
        const uint8_t *qh = W[i].qh;
        const int8_t *sc = W[i].scales;
        const float *xp = x + (size_t)i * ORC_QK_K;
        for (int n2 = 0; n2 < ORC_QK_K; n2 += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                acc += d * sc[is + 0] * q1 * xp[l + 0];
                acc += d * sc[is + 2] * q2 * xp[l + 32];
                acc += d * sc[is + 4] * q3 * xp[l + 64];
                acc += d * sc[is + 6] * q4 * xp[l + 96];
            }
            xp += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
    return acc;
}

/* ------------------------------------------------------------------------ */
/* Q8_K activation quantization and int8 dots                                */
/* ------------------------------------------------------------------------ */

/* vcvtaq_s32_f32: round to nearest, ties away from zero, saturating. */
static int32_t cvta_s32(float v)
{
    if (v != v) return 0;
    if (v >= 2147483647.5f) return INT32_MAX;
    if (v <= -2147483648.5f) return INT32_MIN;
    return (int32_t)roundf(v);
}

/* quantize_row_q8k: q8k.c:34-85.  amax follows vmaxq_f32 (NaN propagates). */
void orc_q8k_quant(const float *x, int n, int8_t *xq, float *xd, int16_t *xsum)
{
    const int nb = n / ORC_QK_K;
    for (int i = 0; i < nb; i++) {
        const float *xs = x + (size_t)i * ORC_QK_K;
        int8_t *q = xq + (size_t)i * ORC_QK_K;
        int16_t *sp = xsum + (size_t)i * (ORC_QK_K / 16);
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK_K; j++) {
            const float a = fabsf(xs[j]);
            if (a != a || amax != amax) amax = NAN;
            else if (a > amax) amax = a;
        }
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        xd[i] = s;
        const float inv = 1.0f / s;
        for (int j = 0; j < ORC_QK_K; j += 16) {
            int32_t sum = 0;
            for (int t = 0; t < 16; t++) {
                int32_t v = cvta_s32(xs[j + t] * inv);
                if (v > 127) v = 127;
                if (v < -127) v = -127;
                q[j + t] = (int8_t)v;
                sum += v;
            }
            sp[j / 16] = (int16_t)sum;
        }
    }
}

/* dot_q4_K_q8k: q8k.c:89-131, restated lane by lane. */
static float q4k_dot_row(const orc_block_q4k *b, const int8_t *xq,
                         const float *xd, const int16_t *xsum, int cols)
{
    const int nb = cols / ORC_QK_K;
    float total = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float d = orc_half_to_float(b[i].d);
        const float mn = orc_half_to_float(b[i].dmin);
        const float xd_blk = xd[i];
        const uint8_t *q = b[i].qs;
        const int8_t *xp = xq + (size_t)i * ORC_QK_K;
        const int16_t *sp = xsum + (size_t)i * (ORC_QK_K / 16);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float bias = 0.0f;
        int is = 0;
        for (int g = 0; g < 4; g++) {
            uint8_t s1, m1, s2, m2;
            orc_scale_min_k4(is + 0, b[i].scales, &s1, &m1);
            orc_scale_min_k4(is + 1, b[i].scales, &s2, &m2);
            const float d1 = d * s1, mm1 = mn * m1;
            const float d2 = d * s2, mm2 = mn * m2;
            int32_t pn[4], ph[4];
            for (int j = 0; j < 4; j++) {
                int32_t a = 0, h = 0;
                for (int t = 0; t < 4; t++) {
                    a += (q[4 * j + t] & 0xF) * xp[4 * j + t];
                    h += (q[4 * j + t] >> 4) * xp[32 + 4 * j + t];
                }
                for (int t = 0; t < 4; t++) {
                    a += (q[16 + 4 * j + t] & 0xF) * xp[16 + 4 * j + t];
                    h += (q[16 + 4 * j + t] >> 4) * xp[48 + 4 * j + t];
                }
                pn[j] = a;
                ph[j] = h;
            }
            const float sx0 = (float)(sp[0] + sp[1]);
            const float sx1 = (float)(sp[2] + sp[3]);
            const float f1 = d1 * xd_blk, f2 = d2 * xd_blk;
            for (int j = 0; j < 4; j++) acc[j] = fmaf((float)pn[j], f1, acc[j]);
            for (int j = 0; j < 4; j++) acc[j] = fmaf((float)ph[j], f2, acc[j]);
            bias += (mm1 * sx0 + mm2 * sx1) * xd_blk;
            q += 32;
            xp += 64;
            sp += 4;
            is += 2;
        }
        total += ((acc[0] + acc[1]) + (acc[2] + acc[3])) - bias;
    }
    return total;
}

/* dot_q6_K_q8k: q8k.c:210-262, restated lane by lane (integer, exact). */
static float q6k_dot_row(const orc_block_q6k *b, const int8_t *xq,
                         const float *xd, int cols, int32_t *isum_out)
{
    const int nb = cols / ORC_QK_K;
    float total = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float d = orc_half_to_float(b[i].d);
        const float xd_blk = xd[i];
        const uint8_t *ql = b[i].ql;
        const uint8_t *qh = b[i].qh;
        const int8_t *sc = b[i].scales;
        const int8_t *xp = xq + (size_t)i * ORC_QK_K;
        int32_t acc[4] = {0, 0, 0, 0};
        for (int j = 0; j < 2; j++) {
            uint8_t raw[8][16];
            for (int t = 0; t < 16; t++) {
                const uint8_t l0 = ql[t], l1 = ql[16 + t], l2 = ql[32 + t], l3 = ql[48 + t];
                const uint8_t h0 = qh[t], h1 = qh[16 + t];
                raw[0][t] = (uint8_t)((l0 & 0xF) | ((h0 & 3) << 4));
                raw[1][t] = (uint8_t)((l1 & 0xF) | ((h1 & 3) << 4));
                raw[2][t] = (uint8_t)((l2 & 0xF) | (((h0 & 0xC) >> 2) << 4));
                raw[3][t] = (uint8_t)((l3 & 0xF) | (((h1 & 0xC) >> 2) << 4));
                raw[4][t] = (uint8_t)((l0 >> 4) | (((h0 & 0x30) >> 4) << 4));
                raw[5][t] = (uint8_t)((l1 >> 4) | (((h1 & 0x30) >> 4) << 4));
                raw[6][t] = (uint8_t)((l2 >> 4) | (((h0 & 0xC0) >> 6) << 4));
                raw[7][t] = (uint8_t)((l3 >> 4) | (((h1 & 0xC0) >> 6) << 4));
            }
            for (int g = 0; g < 8; g++) {
                for (int lane = 0; lane < 4; lane++) {
                    int32_t p = 0;
                    for (int t = 0; t < 4; t++)
                        p += ((int32_t)raw[g][4 * lane + t] - 32) * xp[16 * g + 4 * lane + t];
                    acc[lane] += p * (int32_t)sc[g];
                }
            }
            ql += 64;
            qh += 32;
            sc += 8;
            xp += 128;
        }
        const int32_t isum = acc[0] + acc[1] + acc[2] + acc[3];
        if (isum_out) isum_out[i] = isum;
        total += d * xd_blk * (float)isum;
    }
    return total;
}

/* qma_q8k_dot dispatch: q8k.c:305-316 (unknown wtype -> 0.0f). */
float orc_q8k_dot(const void *row, int wtype, const int8_t *xq,
                  const float *xd, const int16_t *xsum, int n)
{
    if (wtype == ORC_TYPE_Q4_K)
        return q4k_dot_row((const orc_block_q4k *)row, xq, xd, xsum, n);
    if (wtype == ORC_TYPE_Q6_K)
        return q6k_dot_row((const orc_block_q6k *)row, xq, xd, n, NULL);
    return 0.0f;
}

/* dot_q4_K_gateup_q8k: q8k.c:140-207.  Per row the arithmetic and its
   association are those of dot_q4_K_q8k (q8k.c:194-203 vs 123-128). */
void orc_q8k_gateup(const void *g, const void *u, const int8_t *xq,
                    const float *xd, const int16_t *xsum, int n,
                    float *gate, float *up)
{
    *gate = q4k_dot_row((const orc_block_q4k *)g, xq, xd, xsum, n);
    *up = q4k_dot_row((const orc_block_q4k *)u, xq, xd, xsum, n);
}

/* Integer intermediates of q8k.c:117-120: Plo (sub-block 2g) and Phi
   (sub-block 2g+1) as full 32-lane int32 sums. */
void orc_q4k_subsums(const void *row, const int8_t *xq, int n, int32_t *P)
{
    const orc_block_q4k *b = (const orc_block_q4k *)row;
    const int nb = n / ORC_QK_K;
    for (int i = 0; i < nb; i++) {
        for (int g = 0; g < 4; g++) {
            const uint8_t *q = b[i].qs + 32 * g;
            const int8_t *xp = xq + (size_t)i * ORC_QK_K + 64 * g;
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (q[l] & 0xF) * xp[l];
                hi += (q[l] >> 4) * xp[32 + l];
            }
            P[8 * i + 2 * g] = lo;
            P[8 * i + 2 * g + 1] = hi;
        }
    }
}

/* Integer intermediate of q8k.c:259: the per-super-block int32 sum. */
void orc_q6k_blocksums(const void *row, const int8_t *xq, int n, int32_t *S)
{
    const int nb = n / ORC_QK_K;
    float *ones = (float *)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
    for (int i = 0; i < nb; i++) ones[i] = 1.0f;
    q6k_dot_row((const orc_block_q6k *)row, xq, ones, n, S);
    free(ones);
}

/* ------------------------------------------------------------------------ */
/* CPU pool following pool_run (nn.c:139-175)                                */
/* ------------------------------------------------------------------------ */

typedef void (*orc_job_fn)(void *arg, int i0, int i1);

static struct {
    pthread_t th[16];
    int n;
    orc_job_fn fn;
    void *arg;
    int n_items;
    int chunk;
    int cursor;
    int gen;
    int done;
    int stop;
    pthread_mutex_t mu;
    pthread_cond_t cv;
} g_pool = {.n = 0, .mu = PTHREAD_MUTEX_INITIALIZER, .cv = PTHREAD_COND_INITIALIZER};

static int g_pool_want = 1;

static void *pool_worker(void *p)
{
    (void)p;
    int my_gen = 0;
    for (;;) {
        pthread_mutex_lock(&g_pool.mu);
        while (g_pool.gen == my_gen && !g_pool.stop) pthread_cond_wait(&g_pool.cv, &g_pool.mu);
        if (g_pool.stop) {
            pthread_mutex_unlock(&g_pool.mu);
            break;
        }
        my_gen = g_pool.gen;
        pthread_mutex_unlock(&g_pool.mu);
        for (;;) {
            const int i = __atomic_fetch_add(&g_pool.cursor, g_pool.chunk, __ATOMIC_RELAXED);
            if (i >= g_pool.n_items) break;
            const int i1 = i + g_pool.chunk < g_pool.n_items ? i + g_pool.chunk : g_pool.n_items;
            g_pool.fn(g_pool.arg, i, i1);
        }
        pthread_mutex_lock(&g_pool.mu);
        g_pool.done++;
        if (g_pool.done == g_pool.n) pthread_cond_broadcast(&g_pool.cv);
        pthread_mutex_unlock(&g_pool.mu);
    }
    return NULL;
}

static void pool_stop(void)
{
    if (g_pool.n == 0) return;
    pthread_mutex_lock(&g_pool.mu);
    g_pool.stop = 1;
    pthread_cond_broadcast(&g_pool.cv);
    pthread_mutex_unlock(&g_pool.mu);
    for (int i = 0; i < g_pool.n; i++) pthread_join(g_pool.th[i], NULL);
    g_pool.n = 0;
    g_pool.stop = 0;
}

void orc_pool_set_threads(int n)
{
    if (n < 1) n = 1;
    if (n > 16) n = 16;          /* nn.c:141-142 */
    g_pool_want = n;
}

int orc_pool_threads(void) { return g_pool_want; }

static void pool_ensure(void)
{
    if (g_pool.n == g_pool_want) return;
    pool_stop();
    if (g_pool_want <= 1) return;
    g_pool.gen = 0;
    for (int i = 0; i < g_pool_want; i++) pthread_create(&g_pool.th[i], NULL, pool_worker, NULL);
    g_pool.n = g_pool_want;
}

/* pool_run (nn.c:158-175): serial when n_items < workers; chunked cursor. */
static void pool_run(orc_job_fn fn, void *arg, int n_items)
{
    if (n_items <= 0) return;
    pool_ensure();
    const int n_active = g_pool.n > 0 ? g_pool.n : 1;
    if (n_active == 1 || n_items < n_active) {
        fn(arg, 0, n_items);
        return;
    }
    g_pool.fn = fn;
    g_pool.arg = arg;
    g_pool.n_items = n_items;
    g_pool.chunk = n_items / (n_active * 8) + 1;
    __atomic_store_n(&g_pool.cursor, 0, __ATOMIC_RELAXED);
    pthread_mutex_lock(&g_pool.mu);
    g_pool.done = 0;
    g_pool.gen++;
    pthread_cond_broadcast(&g_pool.cv);
    while (g_pool.done != g_pool.n) pthread_cond_wait(&g_pool.cv, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

/* ------------------------------------------------------------------------ */
/* matmul driver (nn.c:261-345, q8k branch)                                  */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t *W;
    float *out;
    int n_in, n_out, T, wtype;
    size_t wrow;
    const int8_t *xq;
    const float *xd;
    const int16_t *xs;
} mm_job;

static void mm_worker(void *arg, int i0, int i1)
{
    const mm_job *c = (const mm_job *)arg;
    for (int r = i0; r < i1; r++) {
        const uint8_t *wr = c->W + (size_t)r * c->wrow;
        for (int t = 0; t < c->T; t++) {
            c->out[(size_t)t * c->n_out + r] =
                orc_q8k_dot(wr, c->wtype, c->xq + (size_t)t * c->n_in,
                            c->xd + (size_t)t * (c->n_in / ORC_QK_K),
                            c->xs + (size_t)t * (c->n_in / 16), c->n_in);
        }
    }
}

void orc_matmul_q8k(const float *x, const void *W, int n_in, int n_out,
                    int T, int wtype, float *out)
{
    int8_t *xq = (int8_t *)malloc((size_t)T * n_in);
    float *xd = (float *)malloc(sizeof(float) * (size_t)T * (n_in / ORC_QK_K));
    int16_t *xs = (int16_t *)malloc(sizeof(int16_t) * (size_t)T * (n_in / 16));
    for (int t = 0; t < T; t++)
        orc_q8k_quant(x + (size_t)t * n_in, n_in, xq + (size_t)t * n_in,
                      xd + (size_t)t * (n_in / ORC_QK_K), xs + (size_t)t * (n_in / 16));
    const size_t bs = wtype == ORC_TYPE_Q4_K ? sizeof(orc_block_q4k) : sizeof(orc_block_q6k);
    mm_job c = {(const uint8_t *)W, out, n_in, n_out, T, wtype,
                (size_t)(n_in / ORC_QK_K) * bs, xq, xd, xs};
    pool_run(mm_worker, &c, n_out);
    free(xq);
    free(xd);
    free(xs);
}

/* ------------------------------------------------------------------------ */
/* MoE FFN (nn.c:383-707, q8k semantics)                                     */
/* ------------------------------------------------------------------------ */

static size_t q4k_row_bytes(int n) { return (size_t)(n / ORC_QK_K) * sizeof(orc_block_q4k); }
static size_t row_bytes(int n, int t)
{
    return (size_t)(n / ORC_QK_K) * (t == ORC_TYPE_Q4_K ? sizeof(orc_block_q4k) : sizeof(orc_block_q6k));
}

/* Router: nn.c:514-536.  The optional bias is the synthetic skew of the
   prefill workload, added to each logit after the dot (not in the reference). */
void orc_moe_route(const orc_moe_layer *L, const float *xp, int *sel, float *w,
                   float *logits_out)
{
    const int E = L->n_expert, N = L->n_embd;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    float mx = -1e30f;
    for (int e = 0; e < E; e++) {
        const float *gi = L->gate_inp + (size_t)e * N;
        float s = 0;
        for (int i = 0; i < N; i++) s += gi[i] * xp[i];
        if (L->router_bias) s += L->router_bias[e];
        logits[e] = s;
        if (logits_out) logits_out[e] = s;
        if (s > mx) mx = s;
    }
    float sum = 0;
    for (int e = 0; e < E; e++) {
        logits[e] = expf(logits[e] - mx);
        sum += logits[e];
    }
    for (int e = 0; e < E; e++) logits[e] /= sum;
    for (int k = 0; k < L->n_used; k++) {
        int best = 0;
        float bv = -1e30f;
        for (int e = 0; e < E; e++)
            if (logits[e] > bv) {
                bv = logits[e];
                best = e;
            }
        sel[k] = best;
        w[k] = bv;
        logits[best] = -1e30f;
    }
    float ws = 0;
    for (int k = 0; k < L->n_used; k++) ws += w[k];
    for (int k = 0; k < L->n_used; k++) w[k] /= ws;
    free(logits);
}

/* gate/up + SwiGLU of one expert for one token (nn.c:423-432). */
void orc_moe_expert_h(const uint8_t *ge, const uint8_t *ue, int n_embd, int n_ff,
                      const int8_t *xq, const float *xd, const int16_t *xsum, float *h)
{
    const size_t gu_row = q4k_row_bytes(n_embd);
    for (int i = 0; i < n_ff; i++) {
        float g, u;
        orc_q8k_gateup(ge + (size_t)i * gu_row, ue + (size_t)i * gu_row, xq, xd, xsum,
                       n_embd, &g, &u);
        h[i] = (g / (1.0f + expf(-g))) * u;
    }
}

/* moe_expert_one_q8k: nn.c:412-439 (acc += we * down . Q8_K(h)). */
static void expert_one(const orc_moe_layer *L, const uint8_t *ge, const uint8_t *ue,
                       const uint8_t *de, int de_type, const int8_t *xq,
                       const float *xd, const int16_t *xsum, float we, float *acc)
{
    const int N = L->n_embd, F = L->n_ff;
    float *h = (float *)malloc(sizeof(float) * (size_t)F);
    int8_t *gq = (int8_t *)malloc((size_t)F);
    float *gd = (float *)malloc(sizeof(float) * (size_t)(F / ORC_QK_K));
    int16_t *gs = (int16_t *)malloc(sizeof(int16_t) * (size_t)(F / 16));
    orc_moe_expert_h(ge, ue, N, F, xq, xd, xsum, h);
    orc_q8k_quant(h, F, gq, gd, gs);
    const size_t dn_row = row_bytes(F, de_type);
    for (int i = 0; i < N; i++)
        acc[i] += we * orc_q8k_dot(de + (size_t)i * dn_row, de_type, gq, gd, gs, F);
    free(h);
    free(gq);
    free(gd);
    free(gs);
}

/* Shared-expert gate of moe_shared_q8k (nn.c:452-454): uses the Q8_K
   dequantised x, (w * xq) * xd, serial order, then a sigmoid. */
float orc_moe_shared_gate(const float *wsh, const int8_t *xq, const float *xd, int n_embd)
{
    float gs = 0;
    for (int i = 0; i < n_embd; i++) gs += wsh[i] * xq[i] * xd[i / ORC_QK_K];
    return 1.0f / (1.0f + expf(-gs));
}

/* moe_shared_q8k: nn.c:446-473 */
static void shared_one(const orc_moe_layer *L, const int8_t *xq, const float *xd,
                       const int16_t *xsum, float *acc)
{
    const float gs = orc_moe_shared_gate(L->gate_inp_shexp, xq, xd, L->n_embd);
    expert_one(L, L->gate_shexp, L->up_shexp, L->down_shexp, L->t_down_shexp, xq, xd, xsum,
               gs, acc);
}

typedef struct {
    const orc_moe_layer *L;
    const int *sel;
    const float *w;
    const int8_t *xq;
    const float *xd;
    const int16_t *xs;
    float *pacc;
} xpar_job;

/* moe_xpar_worker: nn.c:652-707 (mmap addressing, nn.c:668-674). */
static void xpar_worker(void *arg, int b, int e)
{
    const xpar_job *xa = (const xpar_job *)arg;
    const orc_moe_layer *L = xa->L;
    const int N = L->n_embd, F = L->n_ff, K = L->n_used;
    const size_t ge_bytes = (size_t)F * q4k_row_bytes(N);
    const size_t dn = (size_t)N * row_bytes(F, L->t_down_exps);
    for (int id = b; id < e; id++) {
        const int t = id / K, k = id % K;
        const int ex = xa->sel[(size_t)t * K + k];
        const float we = xa->w[(size_t)t * K + k];
        float *acc = xa->pacc + (size_t)id * N;
        expert_one(L, L->gate_exps + (size_t)ex * ge_bytes, L->up_exps + (size_t)ex * ge_bytes,
                   L->down_exps + (size_t)ex * dn, L->t_down_exps, xa->xq + (size_t)t * N,
                   xa->xd + (size_t)t * (N / ORC_QK_K), xa->xs + (size_t)t * (N / 16), we, acc);
    }
}

/* moe_ffn: nn.c:509-649 (q8k branch) with routing given.  Deviation from
   the reference: the per-pair partials start at zero (nn.c:604 mallocs them
   uninitialised and accumulates into them). */
void orc_moe_ffn_routed(const orc_moe_layer *L, const float *x, float *out, int T,
                        const int *sel, const float *w)
{
    const int N = L->n_embd, K = L->n_used;
    int8_t *xq = (int8_t *)malloc((size_t)T * N);
    float *xd = (float *)malloc(sizeof(float) * (size_t)T * (N / ORC_QK_K));
    int16_t *xs = (int16_t *)malloc(sizeof(int16_t) * (size_t)T * (N / 16));
    memset(out, 0, sizeof(float) * (size_t)N * T);
    for (int t = 0; t < T; t++)
        orc_q8k_quant(x + (size_t)t * N, N, xq + (size_t)t * N, xd + (size_t)t * (N / ORC_QK_K),
                      xs + (size_t)t * (N / 16));
    float *pacc = (float *)calloc((size_t)T * K * N, sizeof(float));
    xpar_job xa = {L, sel, w, xq, xd, xs, pacc};
    pool_run(xpar_worker, &xa, T * K);
    for (int t = 0; t < T; t++) {
        float *acc = out + (size_t)t * N;
        for (int k = 0; k < K; k++) {
            const float *part = pacc + ((size_t)t * K + k) * N;
            for (int i = 0; i < N; i++) acc[i] += part[i];
        }
        shared_one(L, xq + (size_t)t * N, xd + (size_t)t * (N / ORC_QK_K), xs + (size_t)t * (N / 16),
                   acc);
    }
    free(pacc);
    free(xq);
    free(xd);
    free(xs);
}

void orc_moe_ffn(const orc_moe_layer *L, const float *x, float *out, int T)
{
    const int K = L->n_used;
    int *sel = (int *)malloc(sizeof(int) * (size_t)T * K);
    float *w = (float *)malloc(sizeof(float) * (size_t)T * K);
    for (int t = 0; t < T; t++)
        orc_moe_route(L, x + (size_t)t * L->n_embd, sel + (size_t)t * K, w + (size_t)t * K, NULL);
    orc_moe_ffn_routed(L, x, out, T, sel, w);
    free(sel);
    free(w);
}

/* ---- the fp32 twins, taken when QMA_NOQ8K is set or q8k is unavailable
   (nn.c:585): no activation quantisation, dequantise-then-dot throughout. */

/* h = silu(gate . x) * (up . x) on fp32 x, the first loop of moe_expert_one
   (nn.c:395-400) and of moe_shared (nn.c:480-484). */
void orc_moe_expert_h_f32(const uint8_t *ge, const uint8_t *ue, int n_embd, int n_ff, const float *x,
                          float *h)
{
    const size_t gu_row = q4k_row_bytes(n_embd);
    for (int i = 0; i < n_ff; i++) {
        const float g = orc_dot_q4k_f32(ge + (size_t)i * gu_row, x, n_embd);
        const float u = orc_dot_q4k_f32(ue + (size_t)i * gu_row, x, n_embd);
        h[i] = (g / (1.0f + expf(-g))) * u;
    }
}

/* acc[i] += we * down_i . h over fp32 h (nn.c:401-406, 485-490) */
static void down_f32(const uint8_t *de, int de_type, int n_embd, int n_ff, const float *h, float we,
                     float *acc)
{
    const size_t dn_row = row_bytes(n_ff, de_type);
    for (int i = 0; i < n_embd; i++) {
        const float y = de_type == ORC_TYPE_Q4_K ? orc_dot_q4k_f32(de + (size_t)i * dn_row, h, n_ff)
                                                 : orc_dot_q6k_f32(de + (size_t)i * dn_row, h, n_ff);
        acc[i] += we * y;
    }
}

/* the shared gate of moe_shared (nn.c:477-479): fp32 x, serial sum, sigmoid */
float orc_moe_shared_gate_f32(const float *wsh, const float *x, int n_embd)
{
    float gs = 0;
    for (int i = 0; i < n_embd; i++) gs += wsh[i] * x[i];
    return 1.0f / (1.0f + expf(-gs));
}

/* moe_ffn with q8k off (nn.c:576-629): the router as in the q8k branch, one
   moe_expert_one per (token, slot) into a zeroed partial, the partials
   summed in slot order, then moe_shared added. */
void orc_moe_ffn_f32(const orc_moe_layer *L, const float *x, float *out, int T)
{
    const int N = L->n_embd, F = L->n_ff, K = L->n_used;
    const size_t ge_bytes = (size_t)F * q4k_row_bytes(N);
    const size_t dn = (size_t)N * row_bytes(F, L->t_down_exps);
    int *sel = (int *)malloc(sizeof(int) * (size_t)K);
    float *w = (float *)malloc(sizeof(float) * (size_t)K);
    float *h = (float *)malloc(sizeof(float) * (size_t)F);
    float *part = (float *)malloc(sizeof(float) * (size_t)N);
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * N;
        float *acc = out + (size_t)t * N;
        orc_moe_route(L, xt, sel, w, NULL);
        memset(acc, 0, sizeof(float) * (size_t)N);
        for (int k = 0; k < K; k++) {
            const int ex = sel[k];
            orc_moe_expert_h_f32(L->gate_exps + (size_t)ex * ge_bytes, L->up_exps + (size_t)ex * ge_bytes, N, F,
                                 xt, h);
            memset(part, 0, sizeof(float) * (size_t)N);
            down_f32(L->down_exps + (size_t)ex * dn, L->t_down_exps, N, F, h, w[k], part);
            for (int i = 0; i < N; i++) acc[i] += part[i];
        }
        const float gs = orc_moe_shared_gate_f32(L->gate_inp_shexp, xt, N);
        orc_moe_expert_h_f32(L->gate_shexp, L->up_shexp, N, F, xt, h);
        down_f32(L->down_shexp, L->t_down_shexp, N, F, h, gs, acc);
    }
    free(sel);
    free(w);
    free(h);
    free(part);
}

/* Layer stack of the decode workload: x <- moe_l(x) + x for each layer, the
   residual add of qma_eval (nn.c:2252) with the non-FFN parts of the layer
   left out. */
void orc_moe_stack(const orc_moe_layer *layers, int n_layer, float *x)
{
    const int N = layers[0].n_embd;
    float *out = (float *)malloc(sizeof(float) * (size_t)N);
    for (int l = 0; l < n_layer; l++) {
        orc_moe_ffn(&layers[l], x, out, 1);
        for (int i = 0; i < N; i++) x[i] = out[i] + x[i];
    }
    free(out);
}

/* ------------------------------------------------------------------------ */
/* synthetic inputs                                                          */
/* ------------------------------------------------------------------------ */

uint64_t orc_splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* splitmix64 -> Box-Muller in double, rounded once to fp32. */
void orc_fill_normal(uint64_t seed, int64_t n, float mean, float std, float *out)
{
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const uint64_t a = orc_splitmix64(&s), b = orc_splitmix64(&s);
        const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)((double)mean + (double)std * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std * r * sin(two_pi * u2));
    }
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* fp32 -> Q4_K, the build's own quantizer: per 32-lane sub-block an
   asymmetric [min(0,lo), hi] range on 4 bits, 6-bit scales/mins against
   fp16 super-scales.  Byte layout inverts orc_scale_min_k4 / quants.c:29-47. */
void orc_quantize_q4k(const float *x, int64_t n, void *out)
{
    orc_block_q4k *y = (orc_block_q4k *)out;
    const int64_t nb = n / ORC_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * ORC_QK_K;
        float scale[8], minv[8], maxs = 0.0f, maxm = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = xb[32 * j];
            for (int l = 0; l < 32; l++) {
                const float v = xb[32 * j + l];
                if (v < lo) lo = v;
                if (v > hi) hi = v;
            }
            if (hi < lo) hi = lo;
            scale[j] = (hi - lo) / 15.0f;
            minv[j] = -lo;
            if (scale[j] > maxs) maxs = scale[j];
            if (minv[j] > maxm) maxm = minv[j];
        }
        const uint16_t dh = orc_float_to_half(maxs / 63.0f);
        const uint16_t mh = orc_float_to_half(maxm / 63.0f);
        const float dq = orc_half_to_float(dh), mq = orc_half_to_float(mh);
        uint8_t sc[8], mm[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = dq > 0.0f ? (uint8_t)clampf(roundf(scale[j] / dq), 0.0f, 63.0f) : 0;
            mm[j] = mq > 0.0f ? (uint8_t)clampf(roundf(minv[j] / mq), 0.0f, 63.0f) : 0;
        }
        y[i].d = dh;
        y[i].dmin = mh;
        for (int j = 0; j < 4; j++) {
            y[i].scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            y[i].scales[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
            y[i].scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mm[j + 4] & 0xF) << 4));
        }
        memset(y[i].qs, 0, sizeof(y[i].qs));
        for (int j = 0; j < 8; j++) {
            const float ds = dq * (float)sc[j];
            const float dm = mq * (float)mm[j];
            for (int l = 0; l < 32; l++) {
                uint8_t q = 0;
                if (ds > 0.0f) {
                    const float t = xb[32 * j + l] + dm;
                    q = (uint8_t)clampf(roundf(t / ds), 0.0f, 15.0f);
                }
                const int g = j / 2;
                if (j & 1) y[i].qs[32 * g + l] |= (uint8_t)(q << 4);
                else y[i].qs[32 * g + l] |= q;
            }
        }
    }
}

/* fp32 -> Q6_K, the build's own quantizer: symmetric 6-bit values in
   [-31, 31] per 16-lane group, int8 group scales against an fp16
   super-scale.  Byte layout inverts quants.c:50-75. */
void orc_quantize_q6k(const float *x, int64_t n, void *out)
{
    orc_block_q6k *y = (orc_block_q6k *)out;
    const int64_t nb = n / ORC_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * ORC_QK_K;
        float sf[16], maxs = 0.0f;
        for (int g = 0; g < 16; g++) {
            float a = 0.0f;
            for (int l = 0; l < 16; l++) {
                const float v = fabsf(xb[16 * g + l]);
                if (v > a) a = v;
            }
            sf[g] = a / 31.0f;
            if (sf[g] > maxs) maxs = sf[g];
        }
        const uint16_t dh = orc_float_to_half(maxs / 127.0f);
        const float dq = orc_half_to_float(dh);
        int8_t sc[16];
        for (int g = 0; g < 16; g++)
            sc[g] = dq > 0.0f ? (int8_t)clampf(roundf(sf[g] / dq), -128.0f, 127.0f) : 0;
        memset(y[i].ql, 0, sizeof(y[i].ql));
        memset(y[i].qh, 0, sizeof(y[i].qh));
        for (int e = 0; e < 256; e++) {
            const int g = e / 16;
            const float ds = dq * (float)sc[g];
            int q = 0;
            if (ds > 0.0f) q = (int)clampf(roundf(xb[e] / ds), -32.0f, 31.0f);
            const uint8_t u = (uint8_t)(q + 32);
            const int half = e / 128, r = e % 128, Q = r / 32, l = r % 32;
            const int qli = 64 * half + (Q & 1) * 32 + l;
            if (Q < 2) y[i].ql[qli] |= (uint8_t)(u & 0xF);
            else y[i].ql[qli] |= (uint8_t)((u & 0xF) << 4);
            y[i].qh[32 * half + l] |= (uint8_t)(((u >> 4) & 3) << (2 * Q));
        }
        for (int g = 0; g < 16; g++) y[i].scales[g] = sc[g];
        y[i].d = dh;
    }
}

/* ---------------------------------------------------------------------- */
/* Sampler (src/sampler.c): repeat penalty, temperature, top-k candidates,  */
/* top-p and the seeded draw.                                              */
/* ---------------------------------------------------------------------- */

/* xorshift64* step, sampler.c:9-14 */
static uint64_t orc_rng_next(uint64_t *s)
{
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return *s * 0x2545F4914F6CDD1DULL;
}

typedef struct {
    float p;
    int id;
} orc_cand;

/* descending by value; the order of equal values is qsort's (sampler.c:28-33) */
static int orc_cand_cmp(const void *a, const void *b)
{
    const orc_cand *x = (const orc_cand *)a, *y = (const orc_cand *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return 0;
}

static void orc_heap_down(orc_cand *c, int k, int j)
{
    for (;;) {
        const int lc = 2 * j + 1, rc = lc + 1;
        int mn = j;
        if (lc < k && c[lc].p < c[mn].p) mn = lc;
        if (rc < k && c[rc].p < c[mn].p) mn = rc;
        if (mn == j) break;
        const orc_cand t = c[j];
        c[j] = c[mn];
        c[mn] = t;
        j = mn;
    }
}

/* sampler_candidates, sampler.c:36-97: penalty per occurrence in
   last_tokens, then logits / temp, then the k largest by a min-heap over
   (logit, id) in index order, sorted descending. */
int orc_sampler_candidates(int n_vocab, const float *logits, const orc_sampler *s, int *ids, float *lgs,
                           int max_k)
{
    const int n = n_vocab;
    const float *l = logits;
    float *buf = NULL;
    if (s->repeat_penalty != 1.0f || s->temp > 0.0f) {
        buf = (float *)malloc(sizeof(float) * (size_t)n);
        if (!buf) return 0;
        memcpy(buf, logits, sizeof(float) * (size_t)n);
        if (s->repeat_penalty != 1.0f) {
            for (int i = 0; i < s->n_last; i++) {
                const int id = s->last_tokens[i];
                if (id >= 0 && id < n) {
                    if (buf[id] < 0.0f) buf[id] *= s->repeat_penalty;
                    else buf[id] /= s->repeat_penalty;
                }
            }
        }
        if (s->temp > 0.0f)
            for (int i = 0; i < n; i++) buf[i] /= s->temp;
        l = buf;
    }
    int k = s->top_k;
    if (k < 1) k = 1;
    if (k > n) k = n;
    if (k > max_k) k = max_k;
    orc_cand *c = (orc_cand *)malloc(sizeof(orc_cand) * (size_t)(k > 0 ? k : 1));
    if (!c) {
        free(buf);
        return 0;
    }
    for (int i = 0; i < k; i++) {
        c[i].p = l[i];
        c[i].id = i;
    }
    for (int i = k / 2 - 1; i >= 0; i--) orc_heap_down(c, k, i);
    for (int i = k; i < n; i++) {
        if (l[i] > c[0].p) {
            c[0].p = l[i];
            c[0].id = i;
            orc_heap_down(c, k, 0);
        }
    }
    qsort(c, (size_t)k, sizeof(orc_cand), orc_cand_cmp);
    for (int i = 0; i < k; i++) {
        ids[i] = c[i].id;
        lgs[i] = c[i].p;
    }
    free(c);
    free(buf);
    return k;
}

/* sampler_pick, sampler.c:100-134: masked candidates carry <= -1e29; greedy
   at temp <= 0; softmax over the live candidates (double sum), top-p cut,
   one xorshift64* draw, cumulative pick; the pick joins last_tokens (64). */
int orc_sampler_pick(orc_sampler *s, const int *ids, float *lgs, int n, float top_p)
{
    if (n <= 0) return 0;
    int first_live = -1;
    for (int i = 0; i < n; i++)
        if (lgs[i] > -1e29f) {
            first_live = i;
            break;
        }
    if (first_live < 0) return ids[0];
    if (s->temp <= 0.0f) return ids[first_live];
    float mx = lgs[first_live];
    for (int i = first_live; i < n; i++)
        if (lgs[i] > -1e29f && lgs[i] > mx) mx = lgs[i];
    double z = 0.0;
    for (int i = first_live; i < n; i++)
        if (lgs[i] > -1e29f) {
            const float p = expf(lgs[i] - mx);
            lgs[i] = p;
            z += p;
        }
    const float inv = (float)(1.0 / z);
    for (int i = first_live; i < n; i++)
        if (lgs[i] > -1e29f) lgs[i] *= inv;
    float acc = 0.0f;
    int kept = first_live;
    for (int i = first_live; i < n; i++) {
        if (lgs[i] <= -1e29f) continue;
        acc += lgs[i];
        kept = i + 1;
        if (acc >= top_p) break;
    }
    const uint64_t r = orc_rng_next(&s->seed);
    const float rv = (float)((r >> 11) * (1.0 / 9007199254740992.0));
    float cum = 0.0f;
    int pick = ids[kept - 1];
    for (int i = first_live; i < kept; i++) {
        if (lgs[i] <= -1e29f) continue;
        cum += lgs[i];
        if (rv < cum) {
            pick = ids[i];
            break;
        }
    }
    if (s->n_last < 64) {
        s->last_tokens[s->n_last++] = pick;
    } else {
        memmove(s->last_tokens, s->last_tokens + 1, 63 * sizeof(int));
        s->last_tokens[63] = pick;
    }
    return pick;
}
