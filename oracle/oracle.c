/*
 * CPU oracle for the candle-moe fused-MoE hot path -- TEST INFRASTRUCTURE.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this file's library; the product never does. See oracle.h for what each
 * function restates and what pins it.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: */
/* as easy as 1, 2, 3", SC11). Multipliers and Weyl constants are the   */
/* published ones of that paper.                                        */
/* ------------------------------------------------------------------ */
static inline void philox_round(uint32_t c[4], const uint32_t k[2]) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k[0];
    const uint32_t n2 = hi0 ^ c[3] ^ k[1];
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
}

void om_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
    uint32_t k[2] = {key[0], key[1]};
    for (int r = 0; r < 10; ++r) {
        if (r) { k[0] += 0x9E3779B9u; k[1] += 0xBB67AE85u; }
        philox_round(c, k);
    }
    memcpy(out, c, sizeof(c));
}

/* Block b of stream s under seed: counter {b_lo, b_hi, s_lo, s_hi},
 * key {seed_lo, seed_hi}; its 4 words give 4 normals via two Box-Muller
 * transforms evaluated in f64. */
void om_fill_normal(float* out, size_t n, uint64_t seed, uint64_t stream, float mean, float std_) {
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const size_t nblk = (n + 3) / 4;
#pragma omp parallel for schedule(static)
    for (long long b = 0; b < (long long)nblk; ++b) {
        const uint32_t ctr[4] = {(uint32_t)b, (uint32_t)((uint64_t)b >> 32),
                                 (uint32_t)stream, (uint32_t)(stream >> 32)};
        uint32_t r[4];
        om_philox4x32_10(ctr, key, r);
        double z[4];
        for (int h = 0; h < 2; ++h) {
            const double u1 = ((double)r[2 * h] + 0.5) * (1.0 / 4294967296.0);
            const double u2 = ((double)r[2 * h + 1] + 0.5) * (1.0 / 4294967296.0);
            const double rad = sqrt(-2.0 * log(u1));
            const double th = 6.283185307179586476925286766559 * u2;
            z[2 * h] = rad * cos(th);
            z[2 * h + 1] = rad * sin(th);
        }
        for (int i = 0; i < 4; ++i) {
            const size_t o = (size_t)b * 4 + i;
            if (o < n) out[o] = (float)((double)mean + (double)std_ * z[i]);
        }
    }
}

/* ------------------------------------------------------------------ */
/* dtype helpers                                                       */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16, round to nearest even, with subnormals and overflow to inf. */
static inline uint16_t f32_to_f16(float f) {
    const uint32_t u = f2u(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (au < 0x38800000u) {                                   /* below 2^-14: subnormal */
        /* value = au as float; subnormal unit 2^-24 */
        const float a = u2f(au);
        /* exact: a * 2^24 is representable in f32 for these inputs; rint is RNE */
        const float s = a * 16777216.0f;
        const uint32_t m = (uint32_t)rintf(s);
        return (uint16_t)(sign | m);
    }
    uint32_t e = ((au >> 23) - 112u) << 10;
    uint32_t m = (au >> 13) & 0x3ffu;
    uint32_t rest = au & 0x1fffu;
    uint32_t h = e | m;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}
static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)m * (1.0f / 16777216.0f);
        return (sign ? -v : v);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float rnd(float v, int dtype) {
    if (dtype == OM_BF16) return bf16_to_f32(f32_to_bf16(v));
    if (dtype == OM_F16) return f16_to_f32(f32_to_f16(v));
    return v;
}

void om_f32_to_dtype(const float* in, void* out, size_t n, int dtype) {
    if (dtype == OM_F32) { memcpy(out, in, n * 4); return; }
    uint16_t* o = (uint16_t*)out;
    for (size_t i = 0; i < n; ++i) o[i] = dtype == OM_BF16 ? f32_to_bf16(in[i]) : f32_to_f16(in[i]);
}

void om_dtype_to_f32(const void* in, float* out, size_t n, int dtype) {
    if (dtype == OM_F32) { memcpy(out, in, n * 4); return; }
    const uint16_t* s = (const uint16_t*)in;
    for (size_t i = 0; i < n; ++i) out[i] = dtype == OM_BF16 ? bf16_to_f32(s[i]) : f16_to_f32(s[i]);
}

/* Convert n elements starting at src (element offset off) to f32. */
static void load_row(const void* src, size_t off, int n, int dtype, float* dst) {
    if (dtype == OM_F32) { memcpy(dst, (const float*)src + off, (size_t)n * 4); return; }
    const uint16_t* s = (const uint16_t*)src + off;
    if (dtype == OM_BF16) {
        for (int i = 0; i < n; ++i) dst[i] = u2f((uint32_t)s[i] << 16);
        return;
    }
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        const __m128i h = _mm_loadu_si128((const __m128i*)(s + i));
        _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(h));
    }
    for (; i < n; ++i) dst[i] = f16_to_f32(s[i]);
}

/* ------------------------------------------------------------------ */
/* Router                                                              */
/* ------------------------------------------------------------------ */
/* Stable descending selection: candle's arg_sort (descending) keeps the
 * lower index first among equal values; the reference kernel breaks ties
 * the same way (/root/reference/kernels/topk_softmax.cu:236-243). */
static void select_topk(const float* p, int E, int k, int t, int T,
                        float* w, uint32_t* idx, uint32_t* tei, unsigned char* used) {
    memset(used, 0, (size_t)E);
    for (int j = 0; j < k; ++j) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (used[e]) continue;
            if (best < 0 || p[e] > p[best]) best = e;
        }
        used[best] = 1;
        w[(size_t)t * k + j] = p[best];
        idx[(size_t)t * k + j] = (uint32_t)best;
        tei[(size_t)t * k + j] = (uint32_t)((long long)j * T + t);
    }
}

static int topk_impl(const float* logits, int T, int E, int k, float* w, uint32_t* idx,
                     uint32_t* tei, int literal) {
    if (k < 1 || k > E || E < 1 || T < 0) return -1;
#pragma omp parallel
    {
        float* p = (float*)malloc(sizeof(float) * (size_t)E);
        unsigned char* used = (unsigned char*)malloc((size_t)E);
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            const float* row = logits + (size_t)t * E;
            float m = row[0];
            for (int e = 1; e < E; ++e) if (row[e] > m) m = row[e];
            if (literal) {
                float s = 0.f;
                for (int e = 0; e < E; ++e) { p[e] = expf(row[e] - m); s = s + p[e]; }
                for (int e = 0; e < E; ++e) p[e] = p[e] / s;
            } else {
                double s = 0.0;
                for (int e = 0; e < E; ++e) {
                    const float d = row[e] - m;
                    p[e] = (float)exp((double)d);
                    s += (double)p[e];
                }
                const float S = (float)s;
                for (int e = 0; e < E; ++e) p[e] = p[e] / S;
            }
            select_topk(p, E, k, t, T, w, idx, tei, used);
        }
        free(p);
        free(used);
    }
    return 0;
}

int om_topk_softmax(const float* logits, int T, int E, int k, float* w, uint32_t* idx, uint32_t* tei) {
    return topk_impl(logits, T, E, k, w, idx, tei, 0);
}

int om_topk_softmax_f32lit(const float* logits, int T, int E, int k, float* w, uint32_t* idx,
                           uint32_t* tei) {
    return topk_impl(logits, T, E, k, w, idx, tei, 1);
}

/* ------------------------------------------------------------------ */
/* Grouping (preprocessing)                                            */
/* ------------------------------------------------------------------ */
void om_preprocess(const uint32_t* idx, const float* w, int T, int k, int E, int32_t* offsets,
                   int32_t* sorted_tok, float* sorted_w, int32_t* sorted_pair) {
    const long long P = (long long)T * k;
    int32_t* cnt = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    for (long long p = 0; p < P; ++p) if (idx[p] < (uint32_t)E) cnt[idx[p]]++;
    int32_t sum = 0, mx = 0;
    for (int e = 0; e < E; ++e) {
        offsets[e] = sum;
        if (cnt[e] > mx) mx = cnt[e];
        sum += cnt[e];
    }
    offsets[E] = sum;
    offsets[E + 1] = mx;
    for (int e = 0; e < E; ++e) cnt[e] = offsets[e];
    for (long long p = 0; p < P; ++p) {
        const uint32_t e = idx[p];
        if (e >= (uint32_t)E) continue;
        const int32_t pos = cnt[e]++;
        if (sorted_tok) sorted_tok[pos] = (int32_t)(p / k);
        if (sorted_w) sorted_w[pos] = w ? w[p] : 0.f;
        if (sorted_pair) sorted_pair[pos] = (int32_t)p;
    }
    free(cnt);
}

/* ------------------------------------------------------------------ */
/* MoE                                                                 */
/* ------------------------------------------------------------------ */
/* f32 activations (reference kernels/common.cuh:116-138; candle's f32
 * unary ops silu = v / (1 + exp(-v)), gelu = tanh approximation). */
static inline float act_f32(float v, int act) {
    if (act == OM_GELU) {
        const float c = 0.7978845608028654f; /* sqrt(2/pi) */
        return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
    if (act == OM_RELU) return v > 0.f ? v : 0.f;
    return v / (1.0f + expf(-v));
}

/* candle's f16/bf16 SiLU is v / (1 + exp(-v)) with every op rounded to
 * the dtype; GELU and ReLU are computed in f32 and rounded once. */
static inline float act_dtype(float v, int act, int dtype) {
    if (dtype == OM_F32) return act_f32(v, act);
    if (act == OM_SILU) {
        const float ex = rnd(expf(-v), dtype);
        const float den = rnd(1.0f + ex, dtype);
        return rnd(v / den, dtype);
    }
    return rnd(act_f32(v, act), dtype);
}

static inline double act_f64(double v, int act) {
    if (act == OM_GELU) {
        const double c = 0.79788456080286535588; /* sqrt(2/pi) */
        return 0.5 * v * (1.0 + tanh(c * (v + 0.044715 * v * v * v)));
    }
    if (act == OM_RELU) return v > 0.0 ? v : 0.0;
    return v / (1.0 + exp(-v));
}

#define RB 16 /* rows per block: each weight row is converted once per block */

typedef struct {
    int32_t tok;   /* token id */
    int32_t slot;  /* j */
    int32_t orow;  /* output row */
} pair_t;

int om_fused_moe(const void* x, const void* gate, const void* up, const void* down, const float* w,
                 const uint32_t* idx, const double* out_init, double* out, int T, int H, int I, int E,
                 int k, int act, int moe_type, int dtype, int mode, const int32_t* rows, int n_rows,
                 int nthreads) {
    if (T < 0 || H < 1 || I < 1 || E < 1 || k < 1) return -1;
    if (moe_type != OM_QWEN3 && moe_type != OM_NOMIC) return -2;
    if (moe_type == OM_QWEN3 && !down) return -3;
    if (dtype < 0 || dtype > 2 || act < 0 || act > 2) return -4;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    const int NR = rows ? n_rows : T;
    /* token -> output row */
    int32_t* omap = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T > 0 ? T : 1));
    for (int t = 0; t < T; ++t) omap[t] = rows ? -1 : t;
    if (rows) for (int r = 0; r < n_rows; ++r) if (rows[r] >= 0 && rows[r] < T) omap[rows[r]] = r;
    for (long long i = 0; i < (long long)NR * H; ++i) out[i] = out_init ? out_init[i] : 0.0;

    /* For every expert in ascending order, its pairs in ascending (t, j)
     * order: the row-major nonzero() order of /root/reference/tests/moe_tests.rs:168-170. */
    pair_t* pl = (pair_t*)malloc(sizeof(pair_t) * ((size_t)T * k + 1));
    const int cand = (mode == OM_MODE_CANDLE);
    const int f32acc = (mode == OM_MODE_F32ACC);
    const int f32p = cand || f32acc; /* f32 accumulators (else f64) */
    const size_t x_es = (size_t)H;
    for (int e = 0; e < E; ++e) {
        int np = 0;
        for (int t = 0; t < T; ++t) {
            if (omap[t] < 0) continue;
            for (int j = 0; j < k; ++j)
                if (idx[(size_t)t * k + j] == (uint32_t)e) { pl[np].tok = t; pl[np].slot = j; pl[np].orow = omap[t]; ++np; }
        }
        if (!np) continue;
        /* expert MLP outputs (already scaled by the routing weight) */
        double* yw = (double*)malloc(sizeof(double) * (size_t)np * H);
        const size_t gI = (size_t)e * H * I; /* gate/up expert offset */
        const size_t dI = (size_t)e * I * H; /* down expert offset */
        const int nblk = (np + RB - 1) / RB;
#pragma omp parallel
        {
            float* xr = (float*)malloc(sizeof(float) * (size_t)RB * H);
            float* wrow = (float*)malloc(sizeof(float) * (size_t)(H > I ? H : I));
            float* ga = (float*)malloc(sizeof(float) * (size_t)RB * I);
            float* ua = (float*)malloc(sizeof(float) * (size_t)RB * I);
            float* ya = (float*)malloc(sizeof(float) * (size_t)RB * H);
            double* gd = (double*)malloc(sizeof(double) * (size_t)RB * I);
            double* ud = (double*)malloc(sizeof(double) * (size_t)RB * I);
            double* yd = (double*)malloc(sizeof(double) * (size_t)RB * H);
#pragma omp for schedule(dynamic, 1)
            for (int b = 0; b < nblk; ++b) {
                const int r0 = b * RB;
                const int nb = np - r0 < RB ? np - r0 : RB;
                for (int r = 0; r < nb; ++r) load_row(x, (size_t)pl[r0 + r].tok * x_es, H, dtype, xr + (size_t)r * H);
                if (f32p) {
                    memset(ga, 0, sizeof(float) * (size_t)nb * I);
                    memset(ua, 0, sizeof(float) * (size_t)nb * I);
                } else {
                    for (size_t i = 0; i < (size_t)nb * I; ++i) gd[i] = ud[i] = 0.0;
                }
                /* gate (and up for Qwen3): [nb,H] x [H,I], f32 (candle) or f64 */
                for (int kk = 0; kk < H; ++kk) {
                    load_row(gate, gI + (size_t)kk * I, I, dtype, wrow);
                    for (int r = 0; r < nb; ++r) {
                        const float xv = xr[(size_t)r * H + kk];
                        if (f32p) { float* a = ga + (size_t)r * I; for (int n = 0; n < I; ++n) a[n] = a[n] + xv * wrow[n]; }
                        else { double* a = gd + (size_t)r * I; for (int n = 0; n < I; ++n) a[n] += (double)xv * (double)wrow[n]; }
                    }
                    if (moe_type == OM_QWEN3) {
                        load_row(up, gI + (size_t)kk * I, I, dtype, wrow);
                        for (int r = 0; r < nb; ++r) {
                            const float xv = xr[(size_t)r * H + kk];
                            if (f32p) { float* a = ua + (size_t)r * I; for (int n = 0; n < I; ++n) a[n] = a[n] + xv * wrow[n]; }
                            else { double* a = ud + (size_t)r * I; for (int n = 0; n < I; ++n) a[n] += (double)xv * (double)wrow[n]; }
                        }
                    }
                }
                /* activation (and SwiGLU product) -> intermediate h, in ga / gd */
                for (int r = 0; r < nb; ++r) {
                    for (int n = 0; n < I; ++n) {
                        const size_t o = (size_t)r * I + n;
                        if (cand) {
                            const float g = rnd(ga[o], dtype);
                            const float a = act_dtype(g, act, dtype);
                            ga[o] = (moe_type == OM_QWEN3) ? rnd(a * rnd(ua[o], dtype), dtype) : a;
                        } else if (f32acc) {
                            const float a = act_f32(ga[o], act);
                            ga[o] = rnd((moe_type == OM_QWEN3) ? a * ua[o] : a, dtype);
                        } else {
                            const double a = act_f64(gd[o], act);
                            gd[o] = (moe_type == OM_QWEN3) ? a * ud[o] : a;
                        }
                    }
                }
                /* projection back to H */
                if (f32p) memset(ya, 0, sizeof(float) * (size_t)nb * H);
                else for (size_t i = 0; i < (size_t)nb * H; ++i) yd[i] = 0.0;
                if (moe_type == OM_QWEN3) {
                    /* y = h [nb,I] x down[e] [I,H] */
                    for (int i = 0; i < I; ++i) {
                        load_row(down, dI + (size_t)i * H, H, dtype, wrow);
                        for (int r = 0; r < nb; ++r) {
                            if (f32p) { const float hv = ga[(size_t)r * I + i]; float* a = ya + (size_t)r * H; for (int n = 0; n < H; ++n) a[n] = a[n] + hv * wrow[n]; }
                            else { const double hv = gd[(size_t)r * I + i]; double* a = yd + (size_t)r * H; for (int n = 0; n < H; ++n) a[n] += hv * (double)wrow[n]; }
                        }
                    }
                } else {
                    /* y = h [nb,I] x up[e]^T, up[e] is [H,I]: y[n] = sum_i h[i] * up[e][n][i] */
                    for (int n = 0; n < H; ++n) {
                        load_row(up, gI + (size_t)n * I, I, dtype, wrow);
                        for (int r = 0; r < nb; ++r) {
                            if (f32p) { const float* hv = ga + (size_t)r * I; float s = 0.f; for (int i = 0; i < I; ++i) s = s + hv[i] * wrow[i]; ya[(size_t)r * H + n] = s; }
                            else { const double* hv = gd + (size_t)r * I; double s = 0.0; for (int i = 0; i < I; ++i) s += hv[i] * (double)wrow[i]; yd[(size_t)r * H + n] = s; }
                        }
                    }
                }
                /* scale by the routing weight cast to the activation dtype
                 * (/root/reference/tests/moe_tests.rs:177-183) */
                for (int r = 0; r < nb; ++r) {
                    const pair_t* pp = &pl[r0 + r];
                    const float wf = w[(size_t)pp->tok * k + pp->slot];
                    double* dst = yw + (size_t)(r0 + r) * H;
                    if (cand) {
                        const float wd = rnd(wf, dtype);
                        for (int n = 0; n < H; ++n) dst[n] = (double)rnd(rnd(ya[(size_t)r * H + n], dtype) * wd, dtype);
                    } else if (f32acc) {
                        for (int n = 0; n < H; ++n) dst[n] = (double)(ya[(size_t)r * H + n] * wf);
                    } else {
                        for (int n = 0; n < H; ++n) dst[n] = yd[(size_t)r * H + n] * (double)wf;
                    }
                }
            }
            free(xr); free(wrow); free(ga); free(ua); free(ya); free(gd); free(ud); free(yd);
        }
        /* index_add in pair order (/root/reference/tests/moe_tests.rs:185) */
        for (int r = 0; r < np; ++r) {
            double* o = out + (size_t)pl[r].orow * H;
            const double* s = yw + (size_t)r * H;
            if (cand) for (int n = 0; n < H; ++n) o[n] = (double)rnd((float)o[n] + (float)s[n], dtype);
            else if (f32acc) for (int n = 0; n < H; ++n) o[n] = (double)((float)o[n] + (float)s[n]);
            else for (int n = 0; n < H; ++n) o[n] += s[n];
        }
        free(yw);
    }
    /* f32 accumulation: the output is rounded to the dtype once, at the end */
    if (f32acc) for (long long i = 0; i < (long long)NR * H; ++i) out[i] = (double)rnd((float)out[i], dtype);
    free(pl);
    free(omap);
    return 0;
}

/* ------------------------------------------------------------------ */
/* FP8 expert weights: OCP 8-bit floating point e4m3 (E4M3FN of the    */
/* OCP OFP8 specification, v1.0): 1 sign, 4 exponent (bias 7) and 3    */
/* mantissa bits, no infinities, S.1111.111 is NaN, largest finite 448. */
/* The product format (candle_moe_quantize_fp8) adds one f32 scale per  */
/* output channel; it has no counterpart in the reference.             */
/* ------------------------------------------------------------------ */
float om_e4m3_decode(uint8_t c) {
    const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);             /* subnormal: m/8 * 2^(1-7) */
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);   /* normal: (1 + m/8) * 2^(e-7) */
    return s ? -v : v;
}

/* Nearest e4m3 value, ties to the even code (round to nearest even); |x| at
 * or above 448 saturates to +-448, NaN gives 0x7F; the sign of a zero result
 * is kept. Written as a search over the 127 finite magnitudes (monotone in
 * the code), not by bit manipulation. */
static uint8_t e4m3_encode_tab(float x, const double* mag) {
    if (isnan(x)) return 0x7f;
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    const double a = fabs((double)x);
    if (a >= 448.0) return sign | 0x7e;
    int lo = 0, hi = 0x7e; /* largest code with value <= a */
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (mag[mid] <= a) lo = mid; else hi = mid - 1;
    }
    const double d0 = a - mag[lo], d1 = mag[lo + 1] - a; /* exact in f64 */
    int c = lo;
    if (d1 < d0 || (d1 == d0 && (lo & 1))) c = lo + 1;
    return sign | (uint8_t)c;
}

static void e4m3_magnitudes(double mag[128]) {
    for (int c = 0; c < 128; ++c) mag[c] = c < 0x7f ? (double)om_e4m3_decode((uint8_t)c) : INFINITY;
}

uint8_t om_e4m3_encode(float x) {
    double mag[128];
    e4m3_magnitudes(mag);
    return e4m3_encode_tab(x, mag);
}

void om_quantize_fp8(const void* w, int dtype, int E, int K, int N, int kn, uint8_t* q, float* scales) {
    double mag[128];
    e4m3_magnitudes(mag);
    const size_t slab = (size_t)K * N;
    float* ws = (float*)malloc(sizeof(float) * (slab > 0 ? slab : 1));
    for (int e = 0; e < E; ++e) {
        load_row(w, (size_t)e * slab, (int)slab, dtype, ws); /* the expert's weights as f32 */
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; ++n) {
            float amax = 0.0f;
            for (int k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(ws[kn ? (size_t)k * N + n : (size_t)n * K + k]));
            const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
            scales[(size_t)e * N + n] = sc;
            uint8_t* Q = q + ((size_t)e * N + n) * K;
            for (int k = 0; k < K; ++k) Q[k] = e4m3_encode_tab(ws[kn ? (size_t)k * N + n : (size_t)n * K + k] / sc, mag);
        }
    }
    free(ws);
}

void om_dequantize_fp8(const uint8_t* q, const float* scales, size_t rows, int K, float* out) {
    float dec[256];
    for (int c = 0; c < 256; ++c) dec[c] = om_e4m3_decode((uint8_t)c);
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < (long long)rows; ++r)
        for (int k = 0; k < K; ++k) out[r * K + k] = dec[q[r * K + k]] * scales[r];
}
