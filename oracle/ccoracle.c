/* ccoracle.c — CPU restatement of the reference's batched ragged decode pass.
 *
 * TEST INFRASTRUCTURE ONLY (see ccoracle.h): the parity checker and the timed
 * CPU baseline, never a product path. Build: oracle/Makefile.
 *
 * Paths cited are relative to the reference checkout (l-wn/ChatTorrent).
 * Arithmetic is plain IEEE f32 in the order the reference's WGSL writes it;
 * the build passes -ffp-contract=off so no `a*b + c` is fused. Where WGSL
 * leaves an order to the implementation (vec4 `dot`, `exp`, `sqrt`, `/`),
 * the choice made here is stated; those results are tolerance-level parity.
 */
#include "ccoracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ f16 --- */

/* web/f16.js:21-40 half(): f32 -> half bits, nearest-even, ±65504 clamp,
 * NaN kept (0x7e00 | sign), ±inf clamped to ±65504. */
uint16_t orc_half_bits(float x) {
    uint32_t b = f2u(x);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t exp = (b >> 23) & 0xffu;
    uint32_t man = b & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (man ? 0x7e00u : 0x7bffu));
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7bffu);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t h = m >> shift;
        uint32_t rest = m & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rest > mid || (rest == mid && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    if (h > 0x7bffu) h = 0x7bffu;
    return (uint16_t)(sign | h);
}

/* web/f16.js:47-58 buildTable(): every half's exact value. */
float orc_half_value(uint16_t h) {
    uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

void orc_to_f16(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_half_bits(x[i]);
}

void orc_from_f16(const uint16_t* h, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_half_value(h[i]);
}

/* web/model/kernels.js:1356-1383 round_f16: integer-only RNE to an f16 value
 * kept as f32; past 65504 clamps, NaN is left as it is; below 2^-14 the
 * value is rounded on the 2^-24 grid with round() (ties to even). */
void orc_round_f16(float* a, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        uint32_t b = f2u(a[i]);
        uint32_t sign = b & 0x80000000u, m = b & 0x7fffffffu;
        if (m > 0x7f800000u) continue;
        if (m > 0x477fe000u) { a[i] = u2f(sign | 0x477fe000u); continue; }
        if (m < 0x38800000u) {
            float q = rintf(u2f(m) * 16777216.0f) / 16777216.0f;
            a[i] = u2f(sign | f2u(q));
            continue;
        }
        uint32_t rest = m & 0x1fffu, r = m & ~0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (r & 0x2000u))) r += 0x2000u;
        a[i] = u2f(sign | r);
    }
}

/* ------------------------------------------------------- synthetic inputs --- */
/* Counter-based generator shared bit for bit with the device generators
 * (chattorrent_amd/csrc/synth.hip). splitmix64 finaliser, keyed by
 * (seed, stream, index). */
static inline uint64_t smix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_rng(uint64_t seed, uint64_t stream, uint64_t i) {
    return smix(smix(seed ^ (stream * 0xD1B54A32D192ED03ull)) + i);
}

/* orc_rng with the (seed, stream) key computed once: rng_at(key_of(s, t), i)
 * == orc_rng(s, t, i). */
static inline uint64_t key_of(uint64_t seed, uint64_t stream) {
    return smix(seed ^ (stream * 0xD1B54A32D192ED03ull));
}
static inline uint64_t rng_at(uint64_t key, uint64_t i) { return smix(key + i); }

/* Irwin-Hall sum of four 16-bit uniforms, centred: std 37837.2. */
static inline int64_t ih4(uint64_t r) {
    return (int64_t)(r & 0xffffu) + (int64_t)((r >> 16) & 0xffffu)
         + (int64_t)((r >> 32) & 0xffffu) + (int64_t)(r >> 48) - 131070;
}

/* int8 weight ~ clamp(round(N(0, 40)), ±127), integer-exact: q = S*277/2^18. */
static inline int8_t gen_code(uint64_t r) {
    int64_t q = (ih4(r) * 277 + 131072) >> 18;
    if (q > 127) q = 127;
    if (q < -127) q = -127;
    return (int8_t)q;
}

uint16_t orc_gen_scale_f16(uint64_t seed, uint64_t stream, uint64_t i, double lo, double hi) {
    uint64_t u = orc_rng(seed, stream, i) >> 40;                /* 24 bits */
    double v = lo + (hi - lo) * ((double)u * (1.0 / 16777216.0));
    return orc_half_bits((float)v);
}

/* A q8 tensor [N, K]: codes and one f16 scale ~U(1e-4, 4e-4) per `group`
 * values along K. Scales use stream ^ 0x5ca1e. */
void orc_gen_q8(uint64_t seed, uint64_t stream, int64_t N, int64_t K, int group,
                int8_t* codes, uint16_t* scales_f16) {
    int64_t ng = (K + group - 1) / group;
    const uint64_t kc = key_of(seed, stream);
    #pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++) {
        for (int64_t k = 0; k < K; k++) codes[n * K + k] = gen_code(rng_at(kc, (uint64_t)(n * K + k)));
        for (int64_t g = 0; g < ng; g++)
            scales_f16[n * ng + g] = orc_gen_scale_f16(seed, stream ^ 0x5ca1eull, (uint64_t)(n * ng + g), 1e-4, 4e-4);
    }
}

/* f16 values ~N(0, 1) (Irwin-Hall approximation). */
void orc_gen_normal_f16(uint64_t seed, uint64_t stream, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; i++) {
        double x = (double)ih4(orc_rng(seed, stream, (uint64_t)i)) * (1.0 / 37837.2);
        out[i] = orc_half_bits((float)x);
    }
}

void orc_gen_ids(uint64_t seed, uint64_t stream, int64_t n, int vocab, int32_t* out) {
    for (int64_t i = 0; i < n; i++)
        out[i] = (int32_t)(((orc_rng(seed, stream, (uint64_t)i) >> 32) * (uint64_t)vocab) >> 32);
}


/* Random int8 KV rows for a chat (`key`) and tokens t0 .. t0+tokens-1:
 * codes uniform in [-127, 127], one f16 scale ~U(0.005, 0.02) per
 * (token, kv head), widened to f32. Generator index of a row:
 * base = ((key << 24) + t) * nKV + head; code d at base*D + d; the scale at
 * base in stream ^ 0x5ca1e. */
void orc_gen_kv(uint64_t seed, uint64_t stream, uint64_t key, int t0, int tokens, int nKV,
                int D, int8_t* codes, float* scales) {
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; t++)
        for (int n = 0; n < nKV; n++) {
            uint64_t base = ((key << 24) + (uint64_t)(t0 + t)) * (uint64_t)nKV + (uint64_t)n;
            for (int d = 0; d < D; d++) {
                uint64_t r = orc_rng(seed, stream, base * (uint64_t)D + (uint64_t)d);
                codes[((int64_t)t * nKV + n) * D + d] = (int8_t)((int)((r >> 8) % 255u) - 127);
            }
            scales[(int64_t)t * nKV + n] =
                orc_half_value(orc_gen_scale_f16(seed, stream ^ 0x5ca1eull, base, 0.005, 0.02));
        }
}

/* The rows orc_gen_kv generates for a chat (`key`), tokens 0..tokens-1,
 * written straight into a paged cache in the reference's row layout
 * (web/model/kernels.js:999-1022: D/4 code words, then the f32 scale once per
 * 32-value block; row at ((pages[t/page]*nKV + n)*page + t%page)*RW). The
 * same bits as orc_gen_kv followed by a row-by-row copy; this form only
 * saves the full-depth parity tests the copy. */
void orc_fill_kv_paged(uint64_t seed, uint64_t stream, uint64_t key, int tokens, int nKV, int D,
                       int page, const uint32_t* pages, uint32_t* cache) {
    const int QB = D < 32 ? D : 32, nb = D / QB, RW = D / 4 + nb;
    const uint64_t kc = key_of(seed, stream);
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; t++)
        for (int n = 0; n < nKV; n++) {
            uint64_t base = (key << 24) + (uint64_t)t;
            base = base * (uint64_t)nKV + (uint64_t)n;
            uint32_t* row = cache + (((int64_t)pages[t / page] * nKV + n) * page + t % page) * RW;
            uint8_t* bytes = (uint8_t*)row;
            for (int d = 0; d < D; d++) {
                uint64_t r = rng_at(kc, base * (uint64_t)D + (uint64_t)d);
                bytes[d] = (uint8_t)(int8_t)((int)((r >> 8) % 255u) - 127);
            }
            const uint32_t sb = f2u(orc_half_value(orc_gen_scale_f16(seed, stream ^ 0x5ca1eull, base, 0.005, 0.02)));
            for (int b = 0; b < nb; b++) row[D / 4 + b] = sb;
        }
}

/* ---------------------------------------------------------------- kernels --- */

/* web/model/kernels.js:449-501 matmul_gemv_q8 (and :588-751, which give every
 * row the same arithmetic). Y[M,N] = X[M,K] . W[N,K]^T, W int8 with one f32
 * scale per `group` along K. LANES = group/4 lanes split each group by u32
 * word: lane l accumulates acc += S[g] * dot(x4, q4) over its words
 * g*LANES + l, groups in increasing order; then a pairwise tree over lanes
 * (s = LANES/2 .. 1). WGSL's vec4 dot order is the implementation's; here it
 * is ((x0*q0 + x1*q1) + x2*q2) + x3*q3. */
void orc_matmul_q8(const float* X, int M, int K, const int8_t* W, const float* S,
                   int N, int group, float* Y) {
    const int L = group / 4, K4 = K / 4, ng = (K + group - 1) / group;
    const int64_t per = (int64_t)ng * 4 * L;           /* padded K, lane-major per group */
    float* xt = (float*)calloc((size_t)M * per, sizeof(float));
    for (int m = 0; m < M; m++)
        for (int g = 0; g < ng; g++)
            for (int l = 0; l < L; l++) {
                int w = g * L + l;
                if (w >= K4) continue;
                for (int j = 0; j < 4; j++)
                    xt[m * per + (g * 4 + j) * L + l] = X[(int64_t)m * K + 4 * w + j];
            }
    /* Columns go in blocks of NB, each block's dequantised weights held while
     * every row streams past them (a row's activations are read once per
     * block, not per column); within a block, CB columns advance together as
     * independent chains. Each output keeps the sequence above. */
    enum { NB = 16, CB = 4 };
    const int nblk = (N + NB - 1) / NB;
    #pragma omp parallel
    {
        float* wt = (float*)malloc((size_t)NB * per * sizeof(float));
        float* acc = (float*)malloc((size_t)CB * L * sizeof(float));
        #pragma omp for schedule(dynamic, 1)
        for (int blk = 0; blk < nblk; blk++) {
            const int n0 = blk * NB, nn = N - n0 < NB ? N - n0 : NB;
            for (int c = 0; c < nn; c++)
                for (int g = 0; g < ng; g++)
                    for (int l = 0; l < L; l++) {
                        int w = g * L + l;
                        for (int j = 0; j < 4; j++)
                            wt[c * per + (g * 4 + j) * L + l] =
                                w < K4 ? (float)W[(int64_t)(n0 + c) * K + 4 * w + j] : 0.0f;
                    }
            for (int m = 0; m < M; m++) {
                const float* xm = xt + m * per;
                for (int c0 = 0; c0 < nn; c0 += CB) {
                    const int cn = nn - c0 < CB ? nn - c0 : CB;
                    for (int i = 0; i < CB * L; i++) acc[i] = 0.0f;
                    for (int g = 0; g < ng; g++) {
                        const float* x0 = xm + (g * 4 + 0) * L;
                        const float* x1 = xm + (g * 4 + 1) * L;
                        const float* x2 = xm + (g * 4 + 2) * L;
                        const float* x3 = xm + (g * 4 + 3) * L;
                        const int full = (g + 1) * L <= K4;
                        for (int c = 0; c < cn; c++) {
                            const float s = S[(int64_t)(n0 + c0 + c) * ng + g];
                            const float* wc = wt + (int64_t)(c0 + c) * per + (g * 4) * L;
                            const float *w0 = wc, *w1 = wc + L, *w2 = wc + 2 * L, *w3 = wc + 3 * L;
                            float* a = acc + c * L;
                            if (full && L == 8) {       /* group 32: one 8-lane vector */
                                for (int l = 0; l < 8; l++) {
                                    float d = ((x0[l] * w0[l] + x1[l] * w1[l]) + x2[l] * w2[l]) + x3[l] * w3[l];
                                    a[l] += s * d;
                                }
                            } else if (full) {
                                for (int l = 0; l < L; l++) {
                                    float d = ((x0[l] * w0[l] + x1[l] * w1[l]) + x2[l] * w2[l]) + x3[l] * w3[l];
                                    a[l] += s * d;
                                }
                            } else {
                                for (int l = 0; l < L; l++) {
                                    if (g * L + l >= K4) continue;      /* partial last group */
                                    float d = ((x0[l] * w0[l] + x1[l] * w1[l]) + x2[l] * w2[l]) + x3[l] * w3[l];
                                    a[l] += s * d;
                                }
                            }
                        }
                    }
                    for (int c = 0; c < cn; c++) {
                        float* a = acc + c * L;
                        for (int st = L / 2; st > 0; st >>= 1)
                            for (int l = 0; l < st; l++) a[l] += a[l + st];
                        Y[(int64_t)m * N + n0 + c0 + c] = a[0];
                    }
                }
            }
        }
        free(wt);
        free(acc);
    }
    free(xt);
}

/* web/model/kernels.js:895-917 gather_embed_nopos_q8: out[t,h] =
 * f32(q[v*H + h]) * S[v*nGroup + h/group]. */
void orc_gather_embed_q8(const int32_t* ids, int T, int H, const int8_t* wte,
                         const float* S, int group, float* out) {
    const int ng = (H + group - 1) / group;
    for (int t = 0; t < T; t++) {
        int64_t v = ids[t];
        for (int h = 0; h < H; h++)
            out[(int64_t)t * H + h] = (float)wte[v * H + h] * S[v * ng + h / group];
    }
}

/* web/model/kernels.js:930-976 rmsnorm: 256 threads sum x*x over h = tid,
 * tid+256, ...; a pairwise tree (s = 128 .. 1); scale = 1/sqrt(sum/H + eps);
 * y = x*scale*w. */
void orc_rmsnorm(const float* x, const float* w, float* y, int T, int H, float eps) {
    float part[256];
    for (int t = 0; t < T; t++) {
        const float* xr = x + (int64_t)t * H;
        for (int tid = 0; tid < 256; tid++) {
            float ss = 0.0f;
            for (int h = tid; h < H; h += 256) { float v = xr[h]; ss += v * v; }
            part[tid] = ss;
        }
        for (int s = 128; s > 0; s >>= 1)
            for (int tid = 0; tid < s; tid++) part[tid] += part[tid + s];
        float scale = 1.0f / sqrtf(part[0] / (float)H + eps);
        for (int h = 0; h < H; h++) y[(int64_t)t * H + h] = xr[h] * scale * w[h];
    }
}

/* web/model/kernels.js:2000-2014 llama3Scale (HF _compute_llama3_parameters).
 * s = {factor, low_freq_factor, high_freq_factor, original_max_positions}. */
static double llama3_scale(double f0, const double* s) {
    const double PI = 3.14159265358979323846;
    double wavelen = (2.0 * PI) / f0;
    double lowW = s[3] / s[1], highW = s[3] / s[2];
    if (wavelen < highW) return f0;
    if (wavelen > lowW) return f0 / s[0];
    double smooth = (s[3] / wavelen - s[1]) / (s[2] - s[1]);
    return smooth * f0 + (1.0 - smooth) * (f0 / s[0]);
}

/* web/model/kernels.js:2016-2045 ropeTable: cos/sin in f64, rounded to f32
 * once, laid out [pos][pair] with the two interleaved. inv_freq =
 * theta^(-(2i)/rot), optionally llama3-rescaled. */
void orc_rope_table(int rot, double theta, const double* scaling, int cap, float* tbl) {
    const int half = rot / 2;
    for (int i = 0; i < half; i++) {
        double inv = pow(theta, -(2.0 * i) / (double)rot);
        if (scaling) inv = llama3_scale(inv, scaling);
        for (int pos = 0; pos < cap; pos++) {
            double ang = (double)pos * inv;
            tbl[((int64_t)pos * half + i) * 2] = (float)cos(ang);
            tbl[((int64_t)pos * half + i) * 2 + 1] = (float)sin(ang);
        }
    }
}

/* web/model/kernels.js:1093-1129 rope, dense case (pages = [0], page = T):
 * buf [nH, T, D]; channel i pairs with i + rot/2; a*c - b*s, b*c + a*s. */
void orc_rope(float* buf, int nH, int T, int rot, int D, int T_past, const float* tbl) {
    const int half = rot / 2;
    for (int h = 0; h < nH; h++)
        for (int t = 0; t < T; t++) {
            float* row = buf + ((int64_t)h * T + t) * D;
            for (int i = 0; i < half; i++) {
                int64_t k = ((int64_t)(T_past + t) * half + i) * 2;
                float c = tbl[k], s = tbl[k + 1];
                float a = row[i], b = row[i + half];
                row[i] = a * c - b * s;
                row[i + half] = b * c + a * s;
            }
        }
}

/* web/model/kernels.js:1024-1073 store_kv. src [T_new, nKV*D] f32. For each
 * (token, kv head, block of QB = min(32, D)): RoPE (channels < rot) from the
 * table, amax, scale = amax/127, inv = scale > 0 ? 1/scale : 0,
 * q = clamp(round(x*inv), ±127) packed four to a word low byte first, then
 * the f32 scale. Row at ((pages[t/page]*nKV + n)*page + t%page)*RW,
 * RW = D/4 + D/QB words. */
void orc_store_kv(const float* src, uint32_t* cache, int T_new, int T_past, int page,
                  int nKV, int D, int rot, const uint32_t* pages, const float* tbl) {
    const int QB = D < 32 ? D : 32, nb = D / QB, RW = D / 4 + nb, half = rot / 2;
    float x[32];
    for (int tn = 0; tn < T_new; tn++)
        for (int n = 0; n < nKV; n++)
            for (int b = 0; b < nb; b++) {
                const int t = T_past + tn;
                const float* s = src + (int64_t)tn * nKV * D + (int64_t)n * D;
                float amax = 0.0f;
                for (int j = 0; j < QB; j++) {
                    int c = b * QB + j;
                    float v = s[c];
                    if (c < rot) {
                        int i = c % half;
                        int64_t k = ((int64_t)t * half + i) * 2;
                        float cs = tbl[k], sn = tbl[k + 1];
                        float a = s[i], o = s[i + half];
                        v = c < half ? a * cs - o * sn : o * cs + a * sn;
                    }
                    x[j] = v;
                    amax = fmaxf(amax, fabsf(v));
                }
                float scale = amax / 127.0f;
                float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
                int64_t at = (((int64_t)pages[t / page] * nKV + n) * page + t % page) * RW;
                for (int w = 0; w < QB / 4; w++) {
                    uint32_t word = 0;
                    for (int j = 0; j < 4; j++) {
                        float q = rintf(x[4 * w + j] * inv);
                        if (q > 127.0f) q = 127.0f;
                        if (q < -127.0f) q = -127.0f;
                        word |= ((uint32_t)(int32_t)q & 0xffu) << (8 * j);
                    }
                    cache[at + b * (QB / 4) + w] = word;
                }
                cache[at + D / 4 + b] = f2u(scale);
            }
}

/* web/model/kernels.js:1140-1178 qk_scores_gqa: per block,
 * s = sum_w dot(q4, k4) (dot order as in orc_matmul_q8); sum += s * scale_b;
 * score = sum * (1/sqrt(D)). Q is [nH, T_q, D]; rows r0 .. r0+T_new-1.
 * Every score is that sequence of f32 operations; the loops only visit them
 * by kv head and token, so each K row is read once for the group x T_new
 * query rows that share it (one lane each). */
void orc_qk_scores(const float* Q, const uint32_t* K, float* scores, int T_new, int T_act,
                   int page, int D, int nH, int group, const uint32_t* pages, int r0, int T_q) {
    const int QB = D < 32 ? D : 32, nb = D / QB, RW = D / 4 + nb, nKV = nH / group;
    const int G = group * T_new, TB = 64;
    const int nblk = (T_act + TB - 1) / TB;
    const float sc = 1.0f / sqrtf((float)D);
    /* qt[kvh][i][g]: lane g = (h - kvh*group) * T_new + tn */
    float* qt = (float*)malloc((size_t)nKV * D * G * sizeof(float));
    for (int h = 0; h < nH; h++)
        for (int tn = 0; tn < T_new; tn++) {
            const int kvh = h / group, g = (h - kvh * group) * T_new + tn;
            const float* q = Q + ((int64_t)h * T_q + r0 + tn) * D;
            for (int i = 0; i < D; i++) qt[((int64_t)kvh * D + i) * G + g] = q[i];
        }
    #pragma omp parallel
    {
        float* sum = (float*)malloc((size_t)G * sizeof(float));
        float* s = (float*)malloc((size_t)G * sizeof(float));
        float kf[512];
        #pragma omp for collapse(2) schedule(dynamic, 1)
        for (int kvh = 0; kvh < nKV; kvh++)
            for (int blk = 0; blk < nblk; blk++) {
                const float* qk = qt + (int64_t)kvh * D * G;
                const int t1 = blk * TB + TB < T_act ? blk * TB + TB : T_act;
                for (int ta = blk * TB; ta < t1; ta++) {
                    int64_t at = (((int64_t)pages[ta / page] * nKV + kvh) * page + ta % page) * RW;
                    const int8_t* k8 = (const int8_t*)(K + at);
                    for (int i = 0; i < D; i++) kf[i] = (float)k8[i];
                    for (int g = 0; g < G; g++) sum[g] = 0.0f;
                    for (int b = 0; b < nb; b++) {
                        for (int g = 0; g < G; g++) s[g] = 0.0f;
                        for (int w = 0; w < QB / 4; w++) {
                            const int i = b * QB + 4 * w;
                            const float k0 = kf[i], k1 = kf[i + 1], k2 = kf[i + 2], k3 = kf[i + 3];
                            const float *q0 = qk + (int64_t)i * G, *q1 = q0 + G, *q2 = q1 + G, *q3 = q2 + G;
                            for (int g = 0; g < G; g++) {
                                float d = (((q0[g] * k0) + q1[g] * k1) + q2[g] * k2) + q3[g] * k3;
                                s[g] += d;
                            }
                        }
                        const float scale = u2f(K[at + D / 4 + b]);
                        for (int g = 0; g < G; g++) sum[g] += s[g] * scale;
                    }
                    for (int g = 0; g < G; g++) {
                        const int h = kvh * group + g / T_new, tn = g % T_new;
                        scores[((int64_t)h * T_new + tn) * T_act + ta] = sum[g] * sc;
                    }
                }
            }
        free(sum);
        free(s);
    }
    free(qt);
}

/* web/model/kernels.js:1188-1253 causal_softmax: exact three passes over a
 * row with 256 threads (strided partials, pairwise trees): max over
 * k <= T_past + i, exp(s - max) in place and its sum, then divide; masked
 * columns become exact zeros. */
void orc_causal_softmax(float* scores, int T_new, int T_act, int T_past, int nH) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int h = 0; h < nH; h++)
        for (int i = 0; i < T_new; i++) {
            float red[256];
            float* row = scores + ((int64_t)h * T_new + i) * T_act;
            const int limit = T_past + i;
            for (int tid = 0; tid < 256; tid++) {
                float m = -1e30f;
                for (int k = tid; k < T_act; k += 256) if (k <= limit) m = fmaxf(m, row[k]);
                red[tid] = m;
            }
            for (int s = 128; s > 0; s >>= 1)
                for (int tid = 0; tid < s; tid++) red[tid] = fmaxf(red[tid], red[tid + s]);
            const float row_max = red[0];
            for (int tid = 0; tid < 256; tid++) {
                float acc = 0.0f;
                for (int k = tid; k < T_act; k += 256)
                    if (k <= limit) { float e = expf(row[k] - row_max); row[k] = e; acc += e; }
                red[tid] = acc;
            }
            for (int s = 128; s > 0; s >>= 1)
                for (int tid = 0; tid < s; tid++) red[tid] += red[tid + s];
            const float total = red[0];
            for (int k = 0; k < T_act; k++) row[k] = k > limit ? 0.0f : row[k] / total;
        }
}

/* web/model/kernels.js:1264-1310 attn_av_gqa: out[h, r0+tn, d] =
 * sum_i p_i * (q_i,d * scale_i,d/QB), tokens in order. Each channel's sum is
 * that sequence; the loops walk (kv head, 32 channels) and then the tokens,
 * so each V row is dequantised once for all the query rows of its group. */
void orc_attn_av(const float* scores, const uint32_t* V, float* out, int T_new, int T_act,
                 int page, int D, int nH, int group, const uint32_t* pages, int r0, int T_q) {
    const int QB = D < 32 ? D : 32, RW = D / 4 + D / QB, nKV = nH / group;
    const int G = group * T_new, DC = D < 32 ? D : 32, nch = D / DC;
    #pragma omp parallel
    {
        float* sum = (float*)malloc((size_t)G * DC * sizeof(float));
        float vq[32];
        #pragma omp for collapse(2) schedule(dynamic, 1)
        for (int kvh = 0; kvh < nKV; kvh++)
            for (int c = 0; c < nch; c++) {
                const int d0 = c * DC;
                for (int j = 0; j < G * DC; j++) sum[j] = 0.0f;
                for (int i = 0; i < T_act; i++) {
                    int64_t r = (((int64_t)pages[i / page] * nKV + kvh) * page + i % page) * RW;
                    const int8_t* q8 = (const int8_t*)(V + r);
                    for (int d = 0; d < DC; d++) vq[d] = (float)q8[d0 + d] * u2f(V[r + D / 4 + (d0 + d) / QB]);
                    for (int g = 0; g < G; g++) {
                        const int h = kvh * group + g / T_new, tn = g % T_new;
                        const float pi = scores[((int64_t)h * T_new + tn) * T_act + i];
                        float* sg = sum + (int64_t)g * DC;
                        for (int d = 0; d < DC; d++) sg[d] += pi * vq[d];
                    }
                }
                for (int g = 0; g < G; g++) {
                    const int h = kvh * group + g / T_new, tn = g % T_new;
                    for (int d = 0; d < DC; d++) out[((int64_t)h * T_q + r0 + tn) * D + d0 + d] = sum[g * DC + d];
                }
            }
        free(sum);
    }
}

/* web/model/kernels.js:1513-1529 silu_mul: scale = 1/(1 + exp(-g));
 * out = g * scale * up. */
void orc_silu_mul(const float* g, const float* u, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float scale = 1.0f / (1.0f + expf(-g[i]));
        out[i] = g[i] * scale * u[i];
    }
}

/* web/model/kernels.js:1334-1346 add_inplace. */
void orc_add_inplace(float* a, const float* b, int64_t n) {
    for (int64_t i = 0; i < n; i++) a[i] = a[i] + b[i];
}

/* web/model/kernels.js:1453-1507 topk_stage / topkRows :2129-2144: the top M
 * (value, index) pairs of a row, best first: larger value, then lower index.
 * The staged bitonic selection returns exactly this set in this order. */
void orc_topk(const float* row, int V, int M, float* vals, uint32_t* ids) {
    for (int m = 0; m < M; m++) { vals[m] = -INFINITY; ids[m] = 0xffffffffu; }
    /* better(): kernels.js:1466-1468 — larger value, or equal and lower index.
     * The padding the kernel uses is (-inf, 0xffffffff). */
#define BETTER(av, ai, bv, bi) ((av) > (bv) || ((av) == (bv) && (ai) < (bi)))
    for (int i = 0; i < V; i++) {
        float v = row[i];
        if (!BETTER(v, (uint32_t)i, vals[M - 1], ids[M - 1])) continue;
        int j = M - 1;
        while (j > 0 && BETTER(v, (uint32_t)i, vals[j - 1], ids[j - 1])) {
            vals[j] = vals[j - 1]; ids[j] = ids[j - 1]; j--;
        }
        vals[j] = v;
        ids[j] = (uint32_t)i;
    }
#undef BETTER
}
