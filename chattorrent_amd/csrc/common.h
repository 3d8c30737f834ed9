// Shared device/host definitions for the MI355X (gfx950) decode pass.
//
// Layouts used throughout (one wave = 64 lanes; MFMA = v_mfma_f32_16x16x32_f16):
//   * MFMA operand fragment: a 16 x 32 tile, lane l holds row (l % 16), k-block
//     (l / 16) as 8 consecutive f16 (one uint4). The k permutation inside a
//     fragment is free as long as both operands share it.
//   * Result fragment: lane l holds rows 4*(l/16) + r (r = 0..3) of column l % 16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CC_WAVE 64

// ---------------------------------------------------------------- f32 bits ---
__host__ __device__ static inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ static inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// web/model/kernels.js:1356-1383 round_f16: nearest-even to an f16 value kept
// as f32, ±65504 clamp, NaN unchanged, integer ops except the exact 2^24 grid
// rounding below 2^-14.
__host__ __device__ static inline float round_f16_value(float a) {
    uint32_t b = f2u(a);
    uint32_t sign = b & 0x80000000u, m = b & 0x7fffffffu;
    if (m > 0x7f800000u) return a;
    if (m > 0x477fe000u) return u2f(sign | 0x477fe000u);
    if (m < 0x38800000u) {
        float q = __builtin_rintf(u2f(m) * 16777216.0f) / 16777216.0f;
        return u2f(sign | f2u(q));
    }
    uint32_t rest = m & 0x1fffu, r = m & ~0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (r & 0x2000u))) r += 0x2000u;
    return u2f(sign | r);
}

// web/f16.js:21-40 half(): f32 -> half bits (nearest-even, ±65504 clamp).
__host__ __device__ static inline uint16_t half_bits(float x) {
    uint32_t b = f2u(x);
    uint32_t sign = (b >> 16) & 0x8000u, exp = (b >> 23) & 0xffu, man = b & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (man ? 0x7e00u : 0x7bffu));
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7bffu);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t mm = man | 0x800000u;
        int shift = 14 - e;
        uint32_t h = mm >> shift;
        uint32_t rest = mm & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rest > mid || (rest == mid && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    if (h > 0x7bffu) h = 0x7bffu;
    return (uint16_t)(sign | h);
}

// Exact value of an f16 bit pattern.
__host__ __device__ static inline float half_value(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) return u2f(f2u((float)m * 5.9604644775390625e-08f) | sign);
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

// ------------------------------------------------------ synthetic generator ---
// Shared bit for bit with the CPU oracle's generator (splitmix64 keyed by
// (seed, stream, index)); see the generator notes in synth.hip.
__host__ __device__ static inline uint64_t smix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ static inline uint64_t cc_rng(uint64_t seed, uint64_t stream, uint64_t i) {
    return smix(smix(seed ^ (stream * 0xD1B54A32D192ED03ull)) + i);
}
__host__ __device__ static inline int64_t ih4(uint64_t r) {
    return (int64_t)(r & 0xffffu) + (int64_t)((r >> 16) & 0xffffu)
         + (int64_t)((r >> 32) & 0xffffu) + (int64_t)(r >> 48) - 131070;
}
__host__ __device__ static inline int gen_code(uint64_t r) {
    int64_t q = (ih4(r) * 277 + 131072) >> 18;
    if (q > 127) q = 127;
    if (q < -127) q = -127;
    return (int)q;
}
__host__ __device__ static inline uint16_t gen_scale_f16(uint64_t seed, uint64_t stream, uint64_t i,
                                                         double lo, double hi) {
    uint64_t u = cc_rng(seed, stream, i) >> 40;
    double v = lo + (hi - lo) * ((double)u * (1.0 / 16777216.0));
    return half_bits((float)v);
}

// ------------------------------------------------------------------- MFMA ---
__device__ static inline float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Eight int8 codes stored with a +128 bias (byte = q ^ 0x80) -> eight exact
// f16 values: the byte u placed under exponent 0x64 is 1024 + u; subtracting
// 1152 leaves q = u - 128 exactly.
__device__ static inline half8_t dequant8_biased(uint32_t lo, uint32_t hi) {
    const uint32_t k64 = 0x64646464u;
    uint32_t a0 = __builtin_amdgcn_perm(k64, lo, 0x07010700u);   // bytes: u0, 64, u1, 64
    uint32_t a1 = __builtin_amdgcn_perm(k64, lo, 0x07030702u);
    uint32_t a2 = __builtin_amdgcn_perm(k64, hi, 0x07010700u);
    uint32_t a3 = __builtin_amdgcn_perm(k64, hi, 0x07030702u);
    const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    half2_t h0 = __builtin_bit_cast(half2_t, a0) - off;
    half2_t h1 = __builtin_bit_cast(half2_t, a1) - off;
    half2_t h2 = __builtin_bit_cast(half2_t, a2) - off;
    half2_t h3 = __builtin_bit_cast(half2_t, a3) - off;
    half8_t r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
}

// x ≈ hi + lo with hi = f16(x) (nearest-even) and lo = f16(x - hi); the
// difference x - hi is exact in f32, so hi + lo carries ~22 significant bits
// while lo stays a normal f16 (|x| >= 2^-3; below that lo's absolute step is
// 2^-24). Attention's Q operand uses it: its values are of order 1 and its
// scores are sums of such products, where that step is below f32 rounding.
// The matmul operands use split_hilo_x, attention's P.V split_hilo2.
// x is made opaque first: when x is a product, the compiler may otherwise fold
// the multiply into the f16 conversion (v_fma_mix, one rounding) for one use
// of hi and convert the f32 product (two roundings) for another, and the two
// differ by an f16 ulp about once in 2^13 values — hi + lo is then off by it.
__device__ static inline void split_hilo(float x, _Float16& hi, _Float16& lo) {
    asm("" : "+v"(x));
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// The scaled split the matmul operands use: hi = f16(x)
// and lo = f16((x - hi) * 2^11). The remainder is below half an f16 step of
// hi, so lo scaled by 2^11 is of x's own magnitude and stays a normal f16 for
// every |x| >= 2^-14 (an unscaled lo is subnormal below |x| = 2^-3 and keeps
// fewer bits). The matmuls multiply lo's products by 2^-11, exactly, with the
// weight fragment scaled by HILO_LO_WEIGHT. |x - hi| * 2^11 <= 2^15 for every
// finite f16 hi.
constexpr float HILO_LO_SHIFT = 2048.0f;
constexpr float HILO_LO_WEIGHT = 1.0f / 2048.0f;
__device__ static inline void split_hilo_x(float x, _Float16& hi, _Float16& lo) {
    asm("" : "+v"(x));
    hi = (_Float16)x;
    lo = (_Float16)((x - (float)hi) * HILO_LO_SHIFT);
}

// Eight dequantised weights scaled by 2^-11 (exact: |q| <= 127 integers), the
// fragment the scaled lo half multiplies.
__device__ static inline half8_t lo_weight8(half8_t b) {
    const _Float16 w = (_Float16)HILO_LO_WEIGHT;
    const half8_t s = {w, w, w, w, w, w, w, w};
    return b * s;
}

// Attention's P.V operand: two values x = p * s_v as hi = f16(x)
// (nearest-even) and lo = f16(x - hi), packed as two f16 pairs; x - hi is
// exact in f32 (one v_fma_mix from hi's f16 value). Attention forms p
// times 2^PV_SHIFT_LOG2 (2^8, folded into the softmax's exponent, and taken off
// again, exactly, when a wave writes its partial), so lo is a normal f16 for
// p * s_v >= 2^-11 (22 significant bits) and below that its absolute step
// is 2^-32 of p * s_v, under f32 rounding of the page's sum; both halves
// multiply the same V fragment into one accumulator. p is formed as
// exp2(s - (max - 8)); with |max| < PV_MAX_SCORE (log2 units) the rounding
// of max - 8 keeps p below 256.1, so p * s stays in the f16 range for V
// scales up to PV_SCALE_MAX (|V| <= 32385). A row meeting a page with a
// larger (or non-finite) V scale, or a running max beyond that bound, drops
// the shift from that page on (its O and running sum times 2^-8, exactly).
// (Truncating the pair with v_cvt_pkrtz saves two instructions but biases
// every lo toward zero, and the bias adds up over a long softmax sum.)
constexpr float PV_SHIFT_LOG2 = 8.0f;
constexpr float PV_UNSHIFT = 1.0f / 256.0f;
constexpr float PV_SCALE_MAX = 255.0f;
constexpr float PV_MAX_SCORE = 4096.0f;
__device__ static inline void split_hilo2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    asm("" : "+v"(x0), "+v"(x1));
    const f2_t x = {x0, x1};
    const half2_t h = __builtin_convertvector(x, half2_t);
    const f2_t r = {__builtin_fmaf((float)h[0], -1.0f, x0), __builtin_fmaf((float)h[1], -1.0f, x1)};
    const half2_t l = __builtin_convertvector(r, half2_t);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, l);
}

__device__ static inline float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ static inline float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
