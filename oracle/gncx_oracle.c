/*
 * gncx_oracle.c -- CPU restatement of GNC-X's quantized linear-algebra path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library, which fails loudly instead of falling back to the CPU.
 *
 * All line citations refer to csrc/gncx_llm_kernels.cpp of the reference.
 * The reference's SIMD branches (SSSE3/AVX2, selected by -march=native on any
 * x86-64 host with AVX2) fix the float association restated here; integer
 * parts are exact, so only FMA contraction separates these bits from a
 * reference build.
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   fp16/bf16 decode        all 65536 codes vs IEEE (numpy float16)
 *   block dequantisation    closed forms + reference embedding decoders
 *                           (golden fixtures) + one-hot probes of the dots
 *   Q8 activation quant     known answers (zero block, +-amax, ties-to-even)
 *                           + bits recovered from the reference's Q8_0 matvec
 *   dots / matvec / matbatch  float64 brute force, special cases, golden
 *   rmsnorm / rope / attn   closed forms (pos 0, window 1, equal keys) + golden
 *   swiglu / softcap        golden fixtures + closed forms
 */
#include "gncx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---- row-parallel driver ---------------------------------------------- */

/* Output rows are split into contiguous chunks, one pthread each, as the
 * reference's pool splits them (cpp:169-208).  Every row is computed by
 * exactly one thread with the same scalar arithmetic, so the result does not
 * depend on the thread count.  Threads: $ORC_THREADS, else the online CPUs,
 * at most 16. */
typedef void (*orc_rows_fn)(void* ctx, int32_t m0, int32_t m1);

typedef struct {
    orc_rows_fn fn;
    void* ctx;
    int32_t m0, m1;
} orc_chunk;

static void* orc_chunk_main(void* p) {
    const orc_chunk* c = (const orc_chunk*)p;
    c->fn(c->ctx, c->m0, c->m1);
    return NULL;
}

int32_t orc_threads(void) {
    const char* e = getenv("ORC_THREADS");
    long t = e && e[0] ? strtol(e, NULL, 10) : sysconf(_SC_NPROCESSORS_ONLN);
    if (t < 1) t = 1;
    if (t > 16) t = 16;
    return (int32_t)t;
}

static void orc_parallel_rows(int32_t n, int32_t min_rows, orc_rows_fn fn, void* ctx) {
    int32_t t = orc_threads();
    if (min_rows < 1) min_rows = 1;
    if (t > n / min_rows) t = n / min_rows;
    if (t <= 1) {
        fn(ctx, 0, n);
        return;
    }
    orc_chunk chunks[16];
    pthread_t tid[16];
    int started[16];
    const int32_t per = (n + t - 1) / t;
    for (int32_t i = 0; i < t; ++i) {
        chunks[i].fn = fn;
        chunks[i].ctx = ctx;
        chunks[i].m0 = i * per < n ? i * per : n;
        chunks[i].m1 = (i + 1) * per < n ? (i + 1) * per : n;
        started[i] = i > 0 && pthread_create(&tid[i], NULL, orc_chunk_main, &chunks[i]) == 0;
        if (i > 0 && !started[i]) fn(ctx, chunks[i].m0, chunks[i].m1);
    }
    fn(ctx, chunks[0].m0, chunks[0].m1);
    for (int32_t i = 1; i < t; ++i)
        if (started[i]) pthread_join(tid[i], NULL);
}

/* ---- scalar decoders ------------------------------------------------- */

/* cpp:85-112 -- exact IEEE half -> float, subnormals normalised. */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int32_t  e    = (h >> 10) & 0x1f;
    uint32_t m    = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* value = m * 2^-24; renormalise the mantissa */
            int32_t shift = 0;
            while ((m & 0x400u) == 0) { m <<= 1; ++shift; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((uint32_t)(e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* cpp:114-119 */
float orc_bf16_to_fp32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Byte sizes of the packed blocks (cpp:266-297). */
size_t orc_row_bytes(int32_t type, int32_t k) {
    switch (type) {
    case ORC_Q4_0: return (size_t)(k / 32) * 18;
    case ORC_Q8_0: return (size_t)(k / 32) * 34;
    case ORC_Q4_K: return (size_t)(k / 256) * 144;
    case ORC_Q6_K: return (size_t)(k / 256) * 210;
    case ORC_BF16: return (size_t)k * 2;
    default:       return 0;
    }
}

/* cpp:1112-1120 -- 6-bit scale/min unpack of a Q4_K super-block. */
static void k4_scale_min(int j, const uint8_t* s, int* sc, int* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* ---- activation quantisation ----------------------------------------- */

/* cpp:955-995: per 32 values amax, inv = 127/amax, q = nearbyint(x*inv),
 * d = amax/127, plus the whole/low-16/high-16 sums of q.  amax == 0 gives an
 * all-zero block with d = 0. */
void orc_quantize_act_q8(const float* x, int32_t k, orc_act_q8* out) {
    const int32_t nb = k / 32;
    for (int32_t b = 0; b < nb; ++b) {
        const float* src = x + (size_t)b * 32;
        orc_act_q8* blk = out + b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float a = fabsf(src[i]);
            if (a > amax) amax = a;
        }
        if (amax == 0.0f) {
            memset(blk, 0, sizeof(*blk));
            continue;
        }
        const float inv = 127.0f / amax;
        blk->d = amax / 127.0f;
        int32_t lo = 0, hi = 0;
        for (int i = 0; i < 16; ++i) {
            int8_t a = (int8_t)nearbyintf(src[i] * inv);
            int8_t c = (int8_t)nearbyintf(src[i + 16] * inv);
            blk->qs[i] = a;
            blk->qs[i + 16] = c;
            lo += a;
            hi += c;
        }
        blk->sum_lo16 = lo;
        blk->sum_hi16 = hi;
        blk->sum = lo + hi;
    }
}

/* ---- block dequantisation -------------------------------------------- */

void orc_dequant_row(int32_t type, const uint8_t* row, int32_t k, float* out) {
    if (type == ORC_Q4_0) {
        /* element j = d*((qs[j]&15)-8), j+16 = d*((qs[j]>>4)-8): the pairing
         * of cpp:1023-1030 and cpp:1057-1062. */
        for (int32_t b = 0; b < k / 32; ++b) {
            const uint8_t* blk = row + (size_t)b * 18;
            const float d = orc_fp16_to_fp32(rd16(blk));
            for (int j = 0; j < 16; ++j) {
                out[b * 32 + j]      = d * (float)((blk[2 + j] & 15) - 8);
                out[b * 32 + j + 16] = d * (float)((blk[2 + j] >> 4) - 8);
            }
        }
    } else if (type == ORC_Q8_0) {
        /* cpp:707-714 (embedding decoder, scale_factor 1). */
        for (int32_t b = 0; b < k / 32; ++b) {
            const uint8_t* blk = row + (size_t)b * 34;
            const float d = orc_fp16_to_fp32(rd16(blk));
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
        }
    } else if (type == ORC_Q4_K) {
        /* cpp:1127-1178: chunk c holds qs[32c..32c+31]; low nibbles are
         * elements 64c+l (sub-block 2c), high nibbles 64c+32+l (2c+1);
         * w = (d*sc)*q - dmin*m. */
        for (int32_t sb = 0; sb < k / 256; ++sb) {
            const uint8_t* blk = row + (size_t)sb * 144;
            const float d = orc_fp16_to_fp32(rd16(blk));
            const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
            const uint8_t* sc = blk + 4;
            const uint8_t* qs = blk + 16;
            float* y = out + (size_t)sb * 256;
            for (int c = 0; c < 4; ++c) {
                int s1, m1, s2, m2;
                k4_scale_min(2 * c, sc, &s1, &m1);
                k4_scale_min(2 * c + 1, sc, &s2, &m2);
                const float d1 = d * (float)s1, dm1 = dmin * (float)m1;
                const float d2 = d * (float)s2, dm2 = dmin * (float)m2;
                for (int l = 0; l < 32; ++l) {
                    y[64 * c + l]      = d1 * (float)(qs[32 * c + l] & 15) - dm1;
                    y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - dm2;
                }
            }
        }
    } else if (type == ORC_Q6_K) {
        /* cpp:734-759 (embedding decoder, scale_factor 1): w = (d*sc)*q. */
        for (int32_t sb = 0; sb < k / 256; ++sb) {
            const uint8_t* blk = row + (size_t)sb * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            const float d = orc_fp16_to_fp32(rd16(blk + 208));
            float* y = out + (size_t)sb * 256;
            for (int h = 0; h < 2; ++h) {
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l]      = d * (float)sc[is + 0] * (float)q1;
                    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
                y += 128;
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
    } else if (type == ORC_BF16) {
        for (int32_t j = 0; j < k; ++j) out[j] = orc_bf16_to_fp32(rd16(row + 2 * (size_t)j));
    }
}

/* ---- per-row dots (the matvec inner loops) ---------------------------- */

/* cpp:1362-1382 with the dot of cpp:1021-1065: blocks whose activation
 * scale is zero are skipped. */
static float dot_row_q4_0(const uint8_t* row, const orc_act_q8* act, int32_t k) {
    float acc = 0.0f;
    for (int32_t b = 0; b < k / 32; ++b) {
        const orc_act_q8* a = act + b;
        if (a->d == 0.0f) continue;
        const uint8_t* blk = row + (size_t)b * 18;
        const float ws = orc_fp16_to_fp32(rd16(blk));
        int32_t dot = 0;
        for (int j = 0; j < 16; ++j)
            dot += (blk[2 + j] & 15) * a->qs[j] + (blk[2 + j] >> 4) * a->qs[j + 16];
        const int32_t folded = dot - 8 * a->sum;
        acc += (float)folded * (ws * a->d);
    }
    return acc;
}

/* cpp:1413-1431 with the dot of cpp:1070-1107 (no zero skip). */
static float dot_row_q8_0(const uint8_t* row, const orc_act_q8* act, int32_t k, int skip_zero) {
    float acc = 0.0f;
    for (int32_t b = 0; b < k / 32; ++b) {
        const orc_act_q8* a = act + b;
        if (skip_zero && a->d == 0.0f) continue;
        const uint8_t* blk = row + (size_t)b * 34;
        const float ws = orc_fp16_to_fp32(rd16(blk));
        int32_t dot = 0;
        for (int j = 0; j < 32; ++j) dot += (int8_t)blk[2 + j] * a->qs[j];
        acc += (float)dot * (ws * a->d);
    }
    return acc;
}

/* cpp:1127-1205 (SIMD branch): one super-block's contribution. */
static float dot256_q4_k(const uint8_t* blk, const orc_act_q8* act) {
    const float d = orc_fp16_to_fp32(rd16(blk));
    const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* q = blk + 16;
    float total = 0.0f;
    for (int c = 0; c < 4; ++c) {
        int s1, m1, s2, m2;
        k4_scale_min(2 * c, sc, &s1, &m1);
        k4_scale_min(2 * c + 1, sc, &s2, &m2);
        const orc_act_q8* lo = act + 2 * c;
        const orc_act_q8* hi = act + 2 * c + 1;
        int32_t dlo = 0, dhi = 0;
        for (int l = 0; l < 32; ++l) {
            dlo += (q[l] & 15) * lo->qs[l];
            dhi += (q[l] >> 4) * hi->qs[l];
        }
        const float d1 = d * (float)s1, dm1 = dmin * (float)m1;
        const float d2 = d * (float)s2, dm2 = dmin * (float)m2;
        total += lo->d * (d1 * (float)dlo - dm1 * (float)lo->sum)
               + hi->d * (d2 * (float)dhi - dm2 * (float)hi->sum);
        q += 32;
    }
    return total;
}

/* cpp:1211-1321 (SIMD branch): four lane accumulators, one per 32-row group
 * of a 128-half, reduced as (l0+l1)+(l2+l3) and scaled by d at the end. */
static float dot256_q6_k(const uint8_t* blk, const orc_act_q8* act) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = orc_fp16_to_fp32(rd16(blk + 208));
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int h = 0; h < 2; ++h) {
        const orc_act_q8* a = act + 4 * h;
        for (int is = 0; is < 2; ++is) {
            int32_t dot[4] = {0, 0, 0, 0};
            for (int l = 16 * is; l < 16 * is + 16; ++l) {
                const int q1 = (ql[l] & 15) | (((qh[l] >> 0) & 3) << 4);
                const int q2 = (ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4);
                const int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                const int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
                dot[0] += q1 * a[0].qs[l];
                dot[1] += q2 * a[1].qs[l];
                dot[2] += q3 * a[2].qs[l];
                dot[3] += q4 * a[3].qs[l];
            }
            for (int g = 0; g < 4; ++g) {
                const int32_t s = is == 0 ? a[g].sum_lo16 : a[g].sum_hi16;
                const float f = a[g].d * (float)sc[is + 2 * g];
                lane[g] += (float)(dot[g] - 32 * s) * f;
            }
        }
        ql += 64;
        qh += 32;
        sc += 8;
    }
    return d * ((lane[0] + lane[1]) + (lane[2] + lane[3]));
}

/* cpp:1432-1461: BF16 row in fp32, four SSE lanes then s0+s1+s2+s3. */
static float dot_row_bf16(const uint8_t* row, const float* x, int32_t k) {
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int32_t j = 0;
    for (; j + 3 < k; j += 4)
        for (int i = 0; i < 4; ++i)
            lane[i] += orc_bf16_to_fp32(rd16(row + 2 * (size_t)(j + i))) * x[j + i];
    float acc = lane[0] + lane[1] + lane[2] + lane[3];
    for (; j < k; ++j) acc += orc_bf16_to_fp32(rd16(row + 2 * (size_t)j)) * x[j];
    return acc;
}

float orc_dot_row(int32_t type, const uint8_t* row, const orc_act_q8* act, int32_t k,
                  const float* x_fp32) {
    switch (type) {
    case ORC_Q4_0: return dot_row_q4_0(row, act, k);
    case ORC_Q8_0: return dot_row_q8_0(row, act, k, 0);
    case ORC_Q4_K: {
        /* cpp:1383-1397: row_acc += per-super-block total */
        float acc = 0.0f;
        for (int32_t sb = 0; sb < k / 256; ++sb) acc += dot256_q4_k(row + (size_t)sb * 144, act + sb * 8);
        return acc;
    }
    case ORC_Q6_K: {
        float acc = 0.0f;
        for (int32_t sb = 0; sb < k / 256; ++sb) acc += dot256_q6_k(row + (size_t)sb * 210, act + sb * 8);
        return acc;
    }
    case ORC_BF16: return dot_row_bf16(row, x_fp32, k);
    default: return 0.0f;
    }
}

/* ---- matvec / matbatch / lm_head -------------------------------------- */

typedef struct {
    int32_t type;
    const uint8_t* w;
    const float* x;
    const orc_act_q8* act;
    int32_t k;
    size_t rb;
    float* y;
} mv_ctx;

static void mv_rows(void* p, int32_t m0, int32_t m1) {
    const mv_ctx* c = (const mv_ctx*)p;
    for (int32_t m = m0; m < m1; ++m) c->y[m] = orc_dot_row(c->type, c->w + (size_t)m * c->rb, c->act, c->k, c->x);
}

/* cpp:1327-1471.  Unknown types leave y untouched (cpp:1362-1462). */
void orc_matvec(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y) {
    if (type != ORC_Q4_0 && type != ORC_Q8_0 && type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_BF16)
        return;
    orc_act_q8* act = (orc_act_q8*)malloc(sizeof(orc_act_q8) * (size_t)(k / 32 > 0 ? k / 32 : 1));
    orc_quantize_act_q8(x, k, act);
    mv_ctx c = {type, w, x, act, k, orc_row_bytes(type, k), y};
    orc_parallel_rows(n, 64, mv_rows, &c);
    free(act);
}

typedef struct {
    int32_t type;
    const uint8_t* w;
    const float* x;
    const orc_act_q8* act;
    int32_t b, k, n;
    size_t rb;
    float* y;
} mb_ctx;

static void mb_rows(void* p, int32_t m0, int32_t m1);

/* cpp:1495-1692.  Each token row is quantised on its own (cpp:1506-1510);
 * the per-type inner loops differ from matvec in association and in which
 * zero-scale blocks they skip, and are restated as such. */
void orc_matbatch(int32_t type, const uint8_t* w, const float* x, int32_t b, int32_t k,
                  int32_t n, float* y) {
    if (type != ORC_Q4_0 && type != ORC_Q8_0 && type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_BF16)
        return;
    const int32_t nb = k / 32;
    orc_act_q8* act = (orc_act_q8*)malloc(sizeof(orc_act_q8) * (size_t)nb * (size_t)(b > 0 ? b : 1));
    for (int32_t t = 0; t < b; ++t) orc_quantize_act_q8(x + (size_t)t * k, k, act + (size_t)t * nb);
    mb_ctx c = {type, w, x, act, b, k, n, orc_row_bytes(type, k), y};
    orc_parallel_rows(n, 4, mb_rows, &c);
    free(act);
}

static void mb_rows(void* p, int32_t m0, int32_t m1) {
    const mb_ctx* c = (const mb_ctx*)p;
    const int32_t type = c->type, b = c->b, k = c->k, n = c->n, nb = k / 32;
    const orc_act_q8* act = c->act;
    const float* x = c->x;
    float* y = c->y;
    for (int32_t m = m0; m < m1; ++m) {
        const uint8_t* row = c->w + (size_t)m * c->rb;
        for (int32_t t = 0; t < b; ++t) {
            const orc_act_q8* a = act + (size_t)t * nb;
            float acc = 0.0f;
            if (type == ORC_Q4_0) {
                acc = dot_row_q4_0(row, a, k);                          /* cpp:1517-1542 */
            } else if (type == ORC_Q8_0) {
                acc = dot_row_q8_0(row, a, k, 1);                       /* cpp:1631-1655 */
            } else if (type == ORC_Q6_K) {
                for (int32_t sb = 0; sb < k / 256; ++sb)                 /* cpp:1611-1630 */
                    acc += dot256_q6_k(row + (size_t)sb * 210, a + sb * 8);
            } else if (type == ORC_Q4_K) {
                /* cpp:1543-1610: per chunk, sum_t built from the non-zero
                 * halves, then accs[t] += sum_t. */
                for (int32_t sb = 0; sb < k / 256; ++sb) {
                    const uint8_t* blk = row + (size_t)sb * 144;
                    const float d = orc_fp16_to_fp32(rd16(blk));
                    const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
                    const uint8_t* q = blk + 16;
                    for (int c = 0; c < 4; ++c) {
                        int s1, m1, s2, m2;
                        k4_scale_min(2 * c, blk + 4, &s1, &m1);
                        k4_scale_min(2 * c + 1, blk + 4, &s2, &m2);
                        const float d1 = d * (float)s1, dm1 = dmin * (float)m1;
                        const float d2 = d * (float)s2, dm2 = dmin * (float)m2;
                        const orc_act_q8* lo = a + sb * 8 + 2 * c;
                        const orc_act_q8* hi = lo + 1;
                        float sum_t = 0.0f;
                        if (lo->d != 0.0f) {
                            int32_t dot = 0;
                            for (int l = 0; l < 32; ++l) dot += (q[l] & 15) * lo->qs[l];
                            sum_t += lo->d * (d1 * (float)dot - dm1 * (float)lo->sum);
                        }
                        if (hi->d != 0.0f) {
                            int32_t dot = 0;
                            for (int l = 0; l < 32; ++l) dot += (q[l] >> 4) * hi->qs[l];
                            sum_t += hi->d * (d2 * (float)dot - dm2 * (float)hi->sum);
                        }
                        acc += sum_t;
                        q += 32;
                    }
                }
            } else { /* BF16, cpp:1656-1676: sequential fp32 over j */
                const float* xt = x + (size_t)t * k;
                for (int32_t j = 0; j < k; ++j) acc += orc_bf16_to_fp32(rd16(row + 2 * (size_t)j)) * xt[j];
            }
            y[(size_t)t * n + m] = acc;
        }
    }
}

/* cpp:1713-1732: matvec on the tied embedding, then optional tanh softcap. */
void orc_lm_head(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t vocab,
                 float softcap, float* y) {
    orc_matvec(type, w, x, k, vocab, y);
    if (softcap > 0.0f) {
        const float inv = 1.0f / softcap;
        for (int32_t v = 0; v < vocab; ++v) y[v] = tanhf(y[v] * inv) * softcap;
    }
}

/* ---- norms, rope, attention, activations ------------------------------ */

/* Sum of squares as the reference forms it: four fp32 lanes (i mod 4) over
 * the multiple-of-4 prefix, lanes added in double, double tail
 * (cpp:803-823 and cpp:912-925). */
static double sumsq_ref(const float* v, int32_t n) {
    float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int32_t i = 0;
    for (; i + 3 < n; i += 4)
        for (int j = 0; j < 4; ++j) lane[j] += v[i + j] * v[i + j];
    double s = (double)lane[0] + (double)lane[1] + (double)lane[2] + (double)lane[3];
    for (; i < n; ++i) s += (double)v[i] * (double)v[i];
    return s;
}

/* cpp:789-833 (the out_tokens == NULL fast path). */
void orc_rmsnorm(const float* x, const float* gamma, int32_t dim, float eps, float* out) {
    const double s = sumsq_ref(x, dim);
    const float inv = 1.0f / sqrtf((float)(s / dim) + eps);
    for (int32_t i = 0; i < dim; ++i) out[i] = x[i] * inv * gamma[i];
}

/* cpp:895-953: per head, in place; gamma may be NULL. */
void orc_rmsnorm_heads(float* v, const float* gamma, int32_t n_heads, int32_t head_dim, float eps) {
    for (int32_t h = 0; h < n_heads; ++h) {
        float* x = v + (size_t)h * head_dim;
        const double s = sumsq_ref(x, head_dim);
        const float inv = 1.0f / sqrtf((float)(s / head_dim) + eps);
        for (int32_t i = 0; i < head_dim; ++i) x[i] = gamma ? x[i] * inv * gamma[i] : x[i] * inv;
    }
}

/* cpp:1779-1796: theta_i = pos / (base^(2i/hd) [* factor_i]). */
void orc_rope_table(int32_t pos, int32_t head_dim, float freq_base, const float* freq_factors,
                    float* cos_t, float* sin_t) {
    for (int32_t i = 0; i < head_dim / 2; ++i) {
        float freq = 1.0f / powf(freq_base, (float)(2 * i) / (float)head_dim);
        if (freq_factors != NULL && freq_factors[i] != 0.0f) freq /= freq_factors[i];
        const float angle = (float)pos * freq;
        cos_t[i] = cosf(angle);
        sin_t[i] = sinf(angle);
    }
}

/* cpp:1797-1862: NEOX rotate-half on pairs (i, i + hd/2). */
void orc_rope(float* q, float* k, const float* freq_factors, int32_t n_heads, int32_t n_kv_heads,
              int32_t head_dim, int32_t pos, float freq_base) {
    float cs[512], sn[512];
    const int32_t half = head_dim / 2;
    orc_rope_table(pos, head_dim, freq_base, freq_factors, cs, sn);
    for (int pass = 0; pass < 2; ++pass) {
        float* v = pass == 0 ? q : k;
        const int32_t nh = pass == 0 ? n_heads : n_kv_heads;
        if (v == NULL) continue;
        for (int32_t h = 0; h < nh; ++h) {
            float* x = v + (size_t)h * head_dim;
            for (int32_t i = 0; i < half; ++i) {
                const float x1 = x[i], x2 = x[i + half];
                x[i]        = x1 * cs[i] - x2 * sn[i];
                x[i + half] = x2 * cs[i] + x1 * sn[i];
            }
        }
    }
}

/* q.k as the reference's SSE loop forms it (cpp:1925-1946): two 4-lane
 * accumulators over steps of 8, added lane-wise, reduced (l0+l1)+(l2+l3),
 * scalar tail. */
static float qk_dot_ref(const float* q, const float* k, int32_t hd) {
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
    int32_t d = 0;
    for (; d + 7 < hd; d += 8)
        for (int i = 0; i < 4; ++i) {
            a0[i] += q[d + i] * k[d + i];
            a1[i] += q[d + 4 + i] * k[d + 4 + i];
        }
    float c[4];
    for (int i = 0; i < 4; ++i) c[i] = a0[i] + a1[i];
    float dot = (c[0] + c[1]) + (c[2] + c[3]);
    for (; d < hd; ++d) dot += q[d] * k[d];
    return dot;
}

/* cpp:1887-1994: write K/V at pos, then per head a two-pass softmax over
 * the window [max(0, pos-sw+1), pos]; kv head = h / (n_heads/n_kv_heads). */
/* One query head of one position: scores over the window [t0, pos], the
 * max-shifted exponentials, and V weighted by exp / (sum + 1e-12).  sc holds
 * at least pos - t0 + 1 floats.  Shared by the single step and the batched
 * prefill below, so both give the same bits. */
static void attn_head(const float* qh, const float* k_cache, const float* v_cache, int32_t kvh, int32_t t0,
                      int32_t t1, int32_t kv_dim, int32_t head_dim, float scale, float* sc, float* oh) {
    const int32_t win = t1 - t0;
    float mx = -1e30f;
    for (int32_t t = t0; t < t1; ++t) {
        const float* kt = k_cache + (size_t)t * kv_dim + (size_t)kvh * head_dim;
        const float s = qk_dot_ref(qh, kt, head_dim) * scale;
        sc[t - t0] = s;
        if (s > mx) mx = s;
    }
    float sum = 0.0f;
    for (int32_t i = 0; i < win; ++i) {
        const float e = expf(sc[i] - mx);
        sc[i] = e;
        sum += e;
    }
    const float inv = 1.0f / (sum + 1e-12f);
    for (int32_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
    for (int32_t t = t0; t < t1; ++t) {
        const float w = sc[t - t0] * inv;
        const float* vt = v_cache + (size_t)t * kv_dim + (size_t)kvh * head_dim;
        for (int32_t d = 0; d < head_dim; ++d) oh[d] += w * vt[d];
    }
}

static int32_t attn_window_start(int32_t pos, int32_t sliding_window) {
    return sliding_window > 0 ? (pos - sliding_window + 1 > 0 ? pos - sliding_window + 1 : 0) : 0;
}

void orc_attention_step(const float* q, const float* k_new, const float* v_new, float* k_cache,
                        float* v_cache, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                        int32_t head_dim, float scale, int32_t sliding_window, int32_t write_kv,
                        float* out) {
    const int32_t kv_dim = n_kv_heads * head_dim;
    if (write_kv && k_new != NULL && v_new != NULL) {
        memcpy(k_cache + (size_t)pos * kv_dim, k_new, sizeof(float) * (size_t)kv_dim);
        memcpy(v_cache + (size_t)pos * kv_dim, v_new, sizeof(float) * (size_t)kv_dim);
    }
    const int32_t group = n_heads / n_kv_heads;
    const int32_t t0 = attn_window_start(pos, sliding_window);
    const int32_t t1 = pos + 1;
    const int32_t win = t1 - t0;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(win > 0 ? win : 1));
    for (int32_t h = 0; h < n_heads; ++h)
        attn_head(q + (size_t)h * head_dim, k_cache, v_cache, h / group, t0, t1, kv_dim, head_dim, scale, sc,
                  out + (size_t)h * head_dim);
    free(sc);
}

/* The streamer's prefill attention loop (lua/gncx_streamer.lua:1079-1109):
 * token i of the batch attends at position pos0 + i over K/V rows that are
 * already in the caches (rows pos0 .. pos0 + b - 1 written by the caller).
 * Each (token, head) is attn_head, as in b consecutive orc_attention_step
 * calls with write_kv; the (token, head) pairs run in parallel. */
typedef struct {
    const float *q, *k_cache, *v_cache;
    float* out;
    int32_t pos0, n_heads, group, kv_dim, head_dim, window;
    float scale;
} attn_pf_ctx;

static void attn_pf_rows(void* p, int32_t m0, int32_t m1) {
    const attn_pf_ctx* c = (const attn_pf_ctx*)p;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(c->pos0 + m1 / c->n_heads + 1));
    for (int32_t m = m0; m < m1; ++m) {
        const int32_t i = m / c->n_heads, h = m % c->n_heads;
        const int32_t pos = c->pos0 + i;
        const size_t row = (size_t)i * c->n_heads * c->head_dim + (size_t)h * c->head_dim;
        attn_head(c->q + row, c->k_cache, c->v_cache, h / c->group, attn_window_start(pos, c->window), pos + 1,
                  c->kv_dim, c->head_dim, c->scale, sc, c->out + row);
    }
    free(sc);
}

void orc_attention_prefill(const float* q, const float* k_cache, const float* v_cache, int32_t pos0, int32_t b,
                           int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                           int32_t sliding_window, float* out) {
    if (b <= 0) return;
    attn_pf_ctx c = {q, k_cache, v_cache, out, pos0, n_heads, n_heads / n_kv_heads, n_kv_heads * head_dim,
                     head_dim, sliding_window, scale};
    orc_parallel_rows(b * n_heads, 8, attn_pf_rows, &c);
}

/* cpp:2038-2052 */
void orc_swiglu(const float* gate, const float* up, int32_t n, float* out) {
    for (int32_t i = 0; i < n; ++i) {
        const float x = gate[i];
        out[i] = x / (1.0f + expf(-x)) * up[i];
    }
}

/* cpp:842-889: the 4-phase telemetry encode of v[dim].  Tokens are written
 * as packed words phase | d << 8 | |residual| << 16 (the 4-byte
 * GNCXCompactToken of cpp:267-271 read little-endian); returns the quant
 * scale.  r_k is the repunit of k ones (cpp:61-83). */
float orc_encode_4phase(const float* v, int32_t dim, int32_t layer_k, uint32_t* tokens) {
    const int32_t k = layer_k < 0 ? 0 : (layer_k > 17 ? 17 : layer_k);
    int64_t r_k = 1;
    for (int32_t i = 0; i < k; ++i) r_k = r_k * 10 + 1;
    float max_abs = 1e-9f;
    for (int32_t j = 0; j < dim; ++j) {
        const float a = fabsf(v[j]);
        if (a > max_abs) max_abs = a;
    }
    const float target = (float)(9 * r_k);
    const float to_int = target / max_abs;
    const float inv_rk = 1.0f / (float)r_k;
    const float half_rk = (float)(r_k >> 1);
    for (int32_t j = 0; j < dim; ++j) {
        const int64_t val = (int64_t)nearbyintf(v[j] * to_int);
        const int64_t av = val >= 0 ? val : -val;
        int32_t d = (int32_t)(((float)av + half_rk) * inv_rk);
        if (d > 9) d = 9;
        const int64_t anchor = (int64_t)d * r_k;
        const int64_t res = val - (val >= 0 ? anchor : -anchor);
        const uint32_t ares = (uint16_t)(res >= 0 ? res : -res);
        const uint32_t phase = (val >= 0 ? 2u : 0u) | (res >= 0 ? 1u : 0u);
        tokens[j] = phase | ((uint32_t)d << 8) | (ares << 16);
    }
    return max_abs / target;
}

/* cpp:2018-2033: tanh-approximated GELU of gate times up, with the
 * reference's constants and association. */
void orc_geglu(const float* gate, const float* up, int32_t n, float* out) {
    const float c = 0.7978845608028654f;
    for (int32_t i = 0; i < n; ++i) {
        const float x = gate[i];
        const float inner = c * (x + 0.044715f * x * x * x);
        out[i] = 0.5f * x * (1.0f + tanhf(inner)) * up[i];
    }
}

/* cpp:693-780: one embedding row, times scale_factor folded into d. */
void orc_fetch_embedding(int32_t type, const uint8_t* table, int32_t token, int32_t dim,
                         float scale, float* out) {
    const uint8_t* row = table + (size_t)token * orc_row_bytes(type, dim);
    if (type == ORC_Q8_0) {
        for (int32_t b = 0; b < dim / 32; ++b) {
            const uint8_t* blk = row + (size_t)b * 34;
            const float d = orc_fp16_to_fp32(rd16(blk)) * scale;
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
        }
    } else if (type == ORC_Q6_K) {
        for (int32_t sb = 0; sb < dim / 256; ++sb) {
            const uint8_t* blk = row + (size_t)sb * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            const float d = orc_fp16_to_fp32(rd16(blk + 208)) * scale;
            float* y = out + (size_t)sb * 256;
            for (int h = 0; h < 2; ++h) {
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l]      = d * (float)sc[is + 0] * (float)q1;
                    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
                y += 128;
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
    } else if (type == ORC_BF16) {
        for (int32_t j = 0; j < dim; ++j) out[j] = orc_bf16_to_fp32(rd16(row + 2 * (size_t)j)) * scale;
    }
}
