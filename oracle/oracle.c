/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle of the paged decode path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / the timed CPU baseline; the
 * product path (dendrite_amd) never calls it.
 *
 * It restates ReferenceBackend::decode / decode_batch
 * (crates/dendrite-core/src/attention/backend.rs:206-283):
 *   - gather the K/V of every block of the table in order (backend.rs:228-233),
 *     skipping BlockId::INVALID entries (cache/block.rs:11);
 *   - concatenate along the token axis (backend.rs:241-242);
 *   - expand KV heads to query heads with candle's Tensor::repeat, i.e. tile:
 *     query head h reads KV head h % num_kv_heads (backend.rs:245-252), or the
 *     interleaved h / (num_heads/num_kv_heads) mapping of model/layer.rs:321-340;
 *   - scores = q . K^T * scale with scale = AttentionConfig.scale (an f32,
 *     backend.rs:37) used as f64 (backend.rs:214, 255-256);
 *   - softmax over the tokens (backend.rs:259) and probs . V (backend.rs:262);
 *   - an empty table gives zeros (backend.rs:218-222, 235-238).
 * Page layout: Page tensor [2][num_kv_heads][16][head_dim]
 * (crates/dendrite-core/src/cache/paged.rs:57, 90-94).  Token count per page:
 * 16 except each sequence's last page, which holds last_page_len tokens
 * (1..16, 0 read as 16 like PageTable::last_page_len, cache/paged.rs:384-390).
 * KV formats (quantization/fp8.rs:29-53, quantization/mod.rs:47-141) are
 * decoded with the OCP FP8 E4M3 ("FN") and OCP MX v1.0 E8M0 closed forms.
 *
 * Modes:
 *   oracle_decode        f64 arithmetic on exactly dequantised inputs — the
 *                        parity reference;
 *   oracle_decode_candle f32 in candle's op order with materialised
 *                        gather/concat and tiled copies — the timed CPU
 *                        baseline ("ReferenceBackend-equivalent C
 *                        restatement"), and a streaming f32 variant that
 *                        skips the materialisation for large configs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_PAGE 16
#define OR_INVALID 0xFFFFFFFFu

enum { F16 = 0, BF16 = 1, F32 = 2, FP8 = 3, MX = 4 };

/* ---------------------------------------------------------- element codecs */

/* OCP E4M3 "FN": bias 7, no infinities, S.1111.111 is NaN, max 448,
 * subnormals m * 2^-9.  fp8.rs:39-52 states the same range. */
double oracle_e4m3(uint8_t b) {
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    double v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexp((double)m, -9);
    else v = ldexp(1.0 + m / 8.0, e - 7);
    return s ? -v : v;
}

/* OCP MX E8M0: 2^(e - 127), e = 255 is NaN. */
double oracle_e8m0(uint8_t e) { return e == 255 ? NAN : ldexp(1.0, (int)e - 127); }

/* Both decodings for every byte, filled when the library loads, so the
 * element reads below look values up instead of recomputing them. */
static double dec_e4m3[256], dec_e8m0[256];
__attribute__((constructor)) static void fill_decode_tables(void) {
    for (int c = 0; c < 256; ++c) {
        dec_e4m3[c] = oracle_e4m3((uint8_t)c);
        dec_e8m0[c] = oracle_e8m0((uint8_t)c);
    }
}

/* ------------------------------------------------ quantise-on-write oracle
 * The page write rule (dh_pool_write_pages_device), restated from the format
 * definitions: E4M3 "FN" encodes a float as the nearest finite code value
 * (searched over the code table), ties to the even code, |x| >= 448
 * saturating to +-448 (fp8.rs:39-52 states that range); block scales as the
 * benchmark configurations define them: FP8 amax / 448 per (page, K|V, head),
 * 1 for amax 0; MXFP8 2^(floor(log2 amax) - 8) per 32 along head_dim
 * (quantization/mod.rs:96-97), as E8M0 clamped to 2^-127 .. 2^127. */
double oracle_f16(uint16_t h);

static double e4m3_tab[127];
static int e4m3_tab_init = 0;

uint8_t oracle_e4m3_encode(float x) {
    if (!e4m3_tab_init) {
        for (int c = 0; c < 127; ++c) e4m3_tab[c] = oracle_e4m3((uint8_t)c);
        e4m3_tab_init = 1;
    }
    if (x != x) return 0x7F;
    const uint8_t s = signbit(x) ? 0x80 : 0x00;
    const double a = fabs((double)x);
    if (a >= 448.0) return s | 0x7E;
    int best = 0;
    double bd = a;
    for (int c = 1; c < 127; ++c) {
        const double dd = fabs(e4m3_tab[c] - a);
        if (dd < bd || (dd == bd && (c & 1) == 0)) {
            best = c;
            bd = dd;
        }
    }
    return (uint8_t)(s | best);
}

/* Nearest bfloat16 (ties to the even pattern) of a finite float. */
static uint16_t bf16_nearest(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t lo = u & 0xFFFF0000u, hi = lo + 0x10000u;
    float flo, fhi;
    memcpy(&flo, &lo, 4);
    memcpy(&fhi, &hi, 4);
    const double dl = fabs((double)x - flo), dh = fabs((double)fhi - x);
    if (dl < dh || (dl == dh && ((lo >> 16) & 1) == 0)) return (uint16_t)(lo >> 16);
    return (uint16_t)(hi >> 16);
}

/* Nearest IEEE half (ties to the even pattern; from 65520 on, infinity) of
 * a finite float, by bisection over the ordered finite patterns. */
static uint16_t f16_nearest(float x) {
    const uint16_t s = signbit(x) ? 0x8000 : 0x0000;
    const double a = fabs((double)x);
    if (a >= 65520.0) return s | 0x7C00;
    int lo = 0, hi = 0x7BFF;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (oracle_f16((uint16_t)mid) <= a) lo = mid;
        else hi = mid - 1;
    }
    if (lo == 0x7BFF) return s | 0x7BFF;
    const double dl = a - oracle_f16((uint16_t)lo), dh = oracle_f16((uint16_t)(lo + 1)) - a;
    if (dl < dh || (dl == dh && (lo & 1) == 0)) return (uint16_t)(s | lo);
    return (uint16_t)(s | (lo + 1));
}

/* src: n pages of [2][hkv][16][d] floats; data / scales: the pool records. */
int oracle_write_pages(uint32_t fmt, uint32_t hkv, uint32_t d, const float* src, uint32_t n, uint8_t* data,
                       uint8_t* scales) {
    const size_t block = (size_t)OR_PAGE * d, nblk = (size_t)2 * hkv;
    for (size_t i = 0; i < n; ++i) {
        for (size_t b = 0; b < nblk; ++b) {
            const float* x = src + (i * nblk + b) * block;
            const size_t e0 = (i * nblk + b) * block;
            if (fmt == F32) {
                memcpy(data + e0 * 4, x, block * 4);
            } else if (fmt == BF16) {
                for (size_t e = 0; e < block; ++e) {
                    const uint16_t h = bf16_nearest(x[e]);
                    memcpy(data + (e0 + e) * 2, &h, 2);
                }
            } else if (fmt == F16) {
                for (size_t e = 0; e < block; ++e) {
                    const uint16_t h = f16_nearest(x[e]);
                    memcpy(data + (e0 + e) * 2, &h, 2);
                }
            } else if (fmt == FP8) {
                float amax = 0.f;
                for (size_t e = 0; e < block; ++e) amax = fmaxf(amax, fabsf(x[e]));
                const float sc = amax > 0.f ? amax / 448.0f : 1.0f;
                for (size_t e = 0; e < block; ++e) data[e0 + e] = oracle_e4m3_encode(x[e] / sc);
                memcpy(scales + (i * nblk + b) * 4, &sc, 4);
            } else if (fmt == MX) {
                for (size_t g = 0; g < block; g += 32) {
                    float amax = 0.f;
                    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(x[g + k]));
                    int se = -127;
                    if (amax > 0.f) {
                        int ex;
                        frexpf(amax, &ex);                 /* amax in [2^(ex-1), 2^ex) */
                        se = ex - 1 - 8;
                        se = se < -127 ? -127 : (se > 127 ? 127 : se);
                    }
                    scales[(i * nblk + b) * (block / 32) + g / 32] = (uint8_t)(se + 127);
                    const float inv = ldexpf(1.0f, -se);
                    for (int k = 0; k < 32; ++k) data[e0 + g + k] = oracle_e4m3_encode(x[g + k] * inv);
                }
            } else {
                return -1;
            }
        }
    }
    return 0;
}

double oracle_bf16(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

double oracle_f16(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexp((double)m, -24);
    else v = ldexp(1.0 + m / 1024.0, e - 15);
    return s ? -v : v;
}

static size_t elem_bytes(uint32_t fmt) {
    return fmt == F32 ? 4 : (fmt == F16 || fmt == BF16) ? 2 : 1;
}

static size_t scale_rec_bytes(uint32_t fmt, uint32_t hkv, uint32_t d) {
    if (fmt == FP8) return (size_t)2 * hkv * 4;
    if (fmt == MX) return (size_t)2 * hkv * OR_PAGE * (d / 32);
    return 0;
}

typedef struct {
    const uint8_t* data;     /* compact pages, page_map[id] -> row */
    const uint8_t* scales;
    const uint32_t* page_map;
    uint32_t num_pool_pages;
    uint32_t fmt, hkv, d;
    size_t page_bytes, scale_bytes;
} pool_view;

/* Dequantised element (plane, head, token, dim) of a page row. */
static double kv_elem(const pool_view* pv, uint32_t row, uint32_t plane, uint32_t head, uint32_t tok,
                      uint32_t dim) {
    const size_t idx = (((size_t)plane * pv->hkv + head) * OR_PAGE + tok) * pv->d + dim;
    const uint8_t* p = pv->data + (size_t)row * pv->page_bytes;
    switch (pv->fmt) {
        case F32: { float f; memcpy(&f, p + idx * 4, 4); return f; }
        case BF16: { uint16_t h; memcpy(&h, p + idx * 2, 2); return oracle_bf16(h); }
        case F16: { uint16_t h; memcpy(&h, p + idx * 2, 2); return oracle_f16(h); }
        case FP8: {
            float sc;
            memcpy(&sc, pv->scales + (size_t)row * pv->scale_bytes + ((size_t)plane * pv->hkv + head) * 4, 4);
            return dec_e4m3[p[idx]] * (double)sc;
        }
        default: {
            const uint32_t G = pv->d / 32;
            const uint8_t e = pv->scales[(size_t)row * pv->scale_bytes +
                                         (((size_t)plane * pv->hkv + head) * OR_PAGE + tok) * G + dim / 32];
            return dec_e4m3[p[idx]] * dec_e8m0[e];
        }
    }
}

static double q_elem(const void* q, uint32_t q_dtype, size_t idx) {
    if (q_dtype == F32) return ((const float*)q)[idx];
    if (q_dtype == BF16) return oracle_bf16(((const uint16_t*)q)[idx]);
    return oracle_f16(((const uint16_t*)q)[idx]);
}

/* Token runs of one sequence: rows of its pages and the token count of each.
 * Returns the number of pages, or -1 when a page is absent from the view. */
static int seq_pages(const pool_view* pv, const uint32_t* indptr, const uint32_t* indices,
                     const int32_t* lpl, uint32_t b, uint32_t* rows, int* ntok) {
    int n = 0;
    for (uint32_t k = indptr[b]; k < indptr[b + 1]; ++k) {
        const uint32_t id = indices[k];
        if (id == OR_INVALID) continue;
        if (id >= pv->num_pool_pages || pv->page_map[id] == OR_INVALID) return -1;
        rows[n] = pv->page_map[id];
        ntok[n] = OR_PAGE;
        ++n;
    }
    if (n > 0 && lpl) {
        int L = lpl[b];
        ntok[n - 1] = (L <= 0 || L > OR_PAGE) ? OR_PAGE : L;
    }
    return n;
}

static uint32_t kv_head_of(uint32_t h, uint32_t hq, uint32_t hkv, uint32_t gqa) {
    return gqa == 0 ? h % hkv : h / (hq / hkv);
}

/* f64 parity oracle.  out: [n_seq][hq][d] doubles for the sequences listed in
 * seqs (or all batch sequences when seqs is NULL).  Returns 0, or -1 when a
 * referenced page is absent. */
int oracle_decode(const void* data, const void* scales, const uint32_t* page_map,
                  uint32_t num_pool_pages, uint32_t fmt, uint32_t hkv, uint32_t d, const void* q,
                  uint32_t q_dtype, uint32_t hq, float scale, uint32_t gqa, const uint32_t* indptr,
                  const uint32_t* indices, const int32_t* last_page_len, uint32_t batch,
                  const uint32_t* seqs, uint32_t n_seq, double* out, int threads) {
    pool_view pv = {(const uint8_t*)data, (const uint8_t*)scales, page_map, num_pool_pages, fmt, hkv, d,
                    (size_t)2 * hkv * OR_PAGE * d * elem_bytes(fmt), scale_rec_bytes(fmt, hkv, d)};
    const uint32_t ns = seqs ? n_seq : batch;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(| : bad)
    for (uint32_t si = 0; si < ns; ++si) {
        const uint32_t b = seqs ? seqs[si] : si;
        const uint32_t np = indptr[b + 1] - indptr[b];
        uint32_t* rows = (uint32_t*)malloc((np + 1) * sizeof(uint32_t));
        int* ntok = (int*)malloc((np + 1) * sizeof(int));
        const int n = seq_pages(&pv, indptr, indices, last_page_len, b, rows, ntok);
        if (n < 0) {
            bad = 1;
            free(rows);
            free(ntok);
            continue;
        }
        int T = 0;
        for (int i = 0; i < n; ++i) T += ntok[i];
        double* s = (double*)malloc(((size_t)T + 1) * sizeof(double));
        /* K and V of one KV head, dequantised once for the query heads that
         * share it (the same values kv_elem gives, in token order). */
        double* kd = (double*)malloc(((size_t)T * d + 1) * sizeof(double));
        double* vd = (double*)malloc(((size_t)T * d + 1) * sizeof(double));
        double* qd = (double*)malloc((size_t)d * sizeof(double));
        for (uint32_t kh = 0; kh < hkv; ++kh) {
            int t = 0;
            for (int i = 0; i < n; ++i)
                for (int j = 0; j < ntok[i]; ++j, ++t)
                    for (uint32_t k = 0; k < d; ++k) {
                        kd[(size_t)t * d + k] = kv_elem(&pv, rows[i], 0, kh, j, k);
                        vd[(size_t)t * d + k] = kv_elem(&pv, rows[i], 1, kh, j, k);
                    }
            for (uint32_t h = 0; h < hq; ++h) {
                if (kv_head_of(h, hq, hkv, gqa) != kh) continue;
                double* o = out + ((size_t)si * hq + h) * d;
                memset(o, 0, d * sizeof(double));
                if (T == 0) continue;
                const size_t qb = ((size_t)b * hq + h) * d;
                double mx = -INFINITY;
                for (uint32_t k = 0; k < d; ++k) qd[k] = q_elem(q, q_dtype, qb + k);
                /* four tokens' dot products side by side, each summed over
                 * k in order (the same sums as one token at a time) */
                for (t = 0; t + 4 <= T; t += 4) {
                    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
                    const double* k0 = kd + (size_t)t * d;
                    for (uint32_t k = 0; k < d; ++k) {
                        a0 += qd[k] * k0[k];
                        a1 += qd[k] * k0[d + k];
                        a2 += qd[k] * k0[2 * d + k];
                        a3 += qd[k] * k0[3 * d + k];
                    }
                    s[t] = a0 * (double)scale;
                    s[t + 1] = a1 * (double)scale;
                    s[t + 2] = a2 * (double)scale;
                    s[t + 3] = a3 * (double)scale;
                }
                for (; t < T; ++t) {
                    double acc = 0.0;
                    for (uint32_t k = 0; k < d; ++k) acc += qd[k] * kd[(size_t)t * d + k];
                    s[t] = acc * (double)scale;
                }
                for (t = 0; t < T; ++t)
                    if (s[t] > mx) mx = s[t];
                double den = 0.0;
                for (t = 0; t < T; ++t) {
                    s[t] = exp(s[t] - mx);
                    den += s[t];
                }
                for (t = 0; t < T; ++t) {
                    const double w = s[t] / den;
                    for (uint32_t k = 0; k < d; ++k) o[k] += w * vd[(size_t)t * d + k];
                }
            }
        }
        free(kd);
        free(vd);
        free(qd);
        free(s);
        free(rows);
        free(ntok);
    }
    return bad ? -1 : 0;
}

/* f32 CPU baseline in candle's op order.  materialise != 0: per sequence,
 * gather + concat K/V to [hkv][T][d] f32, tile to [hq][T][d], then per head
 * scores (f32 dot), scale, softmax, probs . V — the copies of backend.rs:
 * 241-252 included.  materialise == 0: the same arithmetic reading pages in
 * place (streaming variant for configurations whose materialised copies do
 * not fit).  out: [n_seq][hq][d] floats.  Returns 0 or -1. */
int oracle_decode_candle(const void* data, const void* scales, const uint32_t* page_map,
                         uint32_t num_pool_pages, uint32_t fmt, uint32_t hkv, uint32_t d,
                         const void* q, uint32_t q_dtype, uint32_t hq, float scale, uint32_t gqa,
                         const uint32_t* indptr, const uint32_t* indices,
                         const int32_t* last_page_len, uint32_t batch, const uint32_t* seqs,
                         uint32_t n_seq, float* out, int threads, int materialise) {
    pool_view pv = {(const uint8_t*)data, (const uint8_t*)scales, page_map, num_pool_pages, fmt, hkv, d,
                    (size_t)2 * hkv * OR_PAGE * d * elem_bytes(fmt), scale_rec_bytes(fmt, hkv, d)};
    const uint32_t ns = seqs ? n_seq : batch;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(| : bad)
    for (uint32_t si = 0; si < ns; ++si) {
        const uint32_t b = seqs ? seqs[si] : si;
        const uint32_t np = indptr[b + 1] - indptr[b];
        uint32_t* rows = (uint32_t*)malloc((np + 1) * sizeof(uint32_t));
        int* ntok = (int*)malloc((np + 1) * sizeof(int));
        const int n = seq_pages(&pv, indptr, indices, last_page_len, b, rows, ntok);
        if (n < 0) {
            bad = 1;
            free(rows);
            free(ntok);
            continue;
        }
        int T = 0;
        for (int i = 0; i < n; ++i) T += ntok[i];
        float* qf = (float*)malloc((size_t)hq * d * sizeof(float));
        for (size_t k = 0; k < (size_t)hq * d; ++k) qf[k] = (float)q_elem(q, q_dtype, (size_t)b * hq * d + k);
        float* s = (float*)malloc(((size_t)T + 1) * sizeof(float));
        float *kc = NULL, *vc = NULL, *kt = NULL, *vt = NULL;
        if (materialise && T > 0) {
            kc = (float*)malloc((size_t)hkv * T * d * sizeof(float));
            vc = (float*)malloc((size_t)hkv * T * d * sizeof(float));
            for (uint32_t h = 0; h < hkv; ++h) {
                int t = 0;
                for (int i = 0; i < n; ++i)
                    for (int j = 0; j < ntok[i]; ++j, ++t)
                        for (uint32_t k = 0; k < d; ++k) {
                            kc[((size_t)h * T + t) * d + k] = (float)kv_elem(&pv, rows[i], 0, h, j, k);
                            vc[((size_t)h * T + t) * d + k] = (float)kv_elem(&pv, rows[i], 1, h, j, k);
                        }
            }
            kt = (float*)malloc((size_t)hq * T * d * sizeof(float));
            vt = (float*)malloc((size_t)hq * T * d * sizeof(float));
            for (uint32_t h = 0; h < hq; ++h) {
                const uint32_t kh = kv_head_of(h, hq, hkv, gqa);
                memcpy(kt + (size_t)h * T * d, kc + (size_t)kh * T * d, (size_t)T * d * sizeof(float));
                memcpy(vt + (size_t)h * T * d, vc + (size_t)kh * T * d, (size_t)T * d * sizeof(float));
            }
        }
        for (uint32_t h = 0; h < hq; ++h) {
            float* o = out + ((size_t)si * hq + h) * d;
            memset(o, 0, d * sizeof(float));
            if (T == 0) continue;
            const uint32_t kh = kv_head_of(h, hq, hkv, gqa);
            const float* qv = qf + (size_t)h * d;
            float mx = -INFINITY;
            for (int t = 0, i = 0; i < n; ++i)
                for (int j = 0; j < ntok[i]; ++j, ++t) {
                    float acc = 0.f;
                    if (materialise) {
                        const float* kr = kt + ((size_t)h * T + t) * d;
                        for (uint32_t k = 0; k < d; ++k) acc += qv[k] * kr[k];
                    } else {
                        for (uint32_t k = 0; k < d; ++k) acc += qv[k] * (float)kv_elem(&pv, rows[i], 0, kh, j, k);
                    }
                    s[t] = acc * scale;
                    if (s[t] > mx) mx = s[t];
                }
            float den = 0.f;
            for (int t = 0; t < T; ++t) {
                s[t] = expf(s[t] - mx);
                den += s[t];
            }
            for (int t = 0; t < T; ++t) s[t] /= den;
            for (int t = 0, i = 0; i < n; ++i)
                for (int j = 0; j < ntok[i]; ++j, ++t) {
                    if (materialise) {
                        const float* vr = vt + ((size_t)h * T + t) * d;
                        for (uint32_t k = 0; k < d; ++k) o[k] += s[t] * vr[k];
                    } else {
                        for (uint32_t k = 0; k < d; ++k) o[k] += s[t] * (float)kv_elem(&pv, rows[i], 1, kh, j, k);
                    }
                }
        }
        free(kc); free(vc); free(kt); free(vt);
        free(s); free(qf); free(rows); free(ntok);
    }
    return bad ? -1 : 0;
}

/* merge_attention_outputs, crates/dendrite-ffi/src/flashinfer/cascade.rs:
 * 116-124, in f32 exactly as written there (natural log). */
void oracle_merge(float o1, float lse1, float o2, float lse2, float* o, float* lse) {
    const float m = lse1 > lse2 ? lse1 : lse2;
    const float e1 = expf(lse1 - m), e2 = expf(lse2 - m);
    const float sum = e1 + e2;
    *o = (o1 * e1 + o2 * e2) / sum;
    *lse = m + logf(sum);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
