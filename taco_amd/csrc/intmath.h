// Exact integer helpers shared by the gfx950 kernels and a host test build (g++). Every function
// is the exact value of the integer rule it names (crates/hardshell/src/int.rs); the divisions
// avoid generic 128-bit division, which the GPU compiler expands into a bit-serial loop.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HS_HD __host__ __device__ __forceinline__
#else
#define HS_HD inline
#endif

namespace hs {

typedef __int128 i128;
typedef unsigned __int128 u128;

HS_HD int clz64(uint64_t x) { return x ? __builtin_clzll(x) : 64; }

HS_HD int clz128(u128 x) {
    const uint64_t hi = (uint64_t)(x >> 64);
    return hi ? __builtin_clzll(hi) : 64 + clz64((uint64_t)x);
}

// floor((p + 2^(s-1)) / 2^s) for |p| < 2^63 (int.rs:110-124; for s >= 64 the exact result is
// 0). Never overflows: the low s bits round separately.
HS_HD int64_t shift_round64(int64_t p, uint32_t s) {
    if (s == 0) return p;
    if (s >= 64) return 0;
    const uint64_t r = (uint64_t)p & (((uint64_t)1 << s) - 1);
    const uint64_t up = (r + ((uint64_t)1 << (s - 1))) >> s;
    return (p >> s) + (int64_t)up;
}

// rescale(x, m, s) for |x| < 2^32: the product is exact in i64.
HS_HD int64_t rescale_small(int64_t x, int32_t m, uint32_t s) { return shift_round64(x * (int64_t)m, s); }

// shift_round (int.rs:110-124) of an i128 with the rule's largest shift: s = 0 keeps p, a
// shift above max_shift gives 0.
HS_HD i128 shift_round128(i128 p, uint32_t s, uint32_t max_shift) {
    if (s == 0) return p;
    if (s > max_shift) return 0;
    const u128 half = (u128)1 << (s - 1);
    return (i128)((u128)p + half) >> s;
}

// rescale (int.rs:63-67) for any i64 x.
HS_HD i128 rescale_full(int64_t x, int32_t m, uint32_t s) { return shift_round128((i128)x * (i128)m, s, 95); }

HS_HD int64_t clamp64(int64_t x, int64_t lo, int64_t hi) {
    int64_t u = x < hi ? x : hi;
    return u > lo ? u : lo;
}

HS_HD int64_t clamp128(i128 x, int64_t lo, int64_t hi) {
    i128 u = x < (i128)hi ? x : (i128)hi;
    return (int64_t)(u > (i128)lo ? u : (i128)lo);
}

// floor_div (int.rs) for b > 0.
HS_HD int64_t floor_div64(int64_t a, int64_t b) {
    int64_t q = a / b, r = a % b;
    return (r != 0 && r < 0) ? q - 1 : q;
}

// isqrt_u128 (int.rs:213-233): the exact floor square root, digit by digit from the highest
// even bit at or below the top bit of x.
HS_HD u128 isqrt128(u128 x) {
    if (x == 0) return 0;
    u128 bit = (u128)1 << ((127 - clz128(x)) & ~1);
    u128 rem = x, res = 0;
    while (bit != 0) {
        if (rem >= res + bit) {
            rem -= res + bit;
            res = (res >> 1) + bit;
        } else {
            res >>= 1;
        }
        bit >>= 2;
    }
    return res;
}

// isqrt128 for x < 2^100 from a double-precision estimate, then corrected exactly: the result
// is the floor square root whatever the estimate (the loops step to it), and the estimate is
// within one of it (correctly rounded conversion and square root, root < 2^50).
HS_HD uint64_t isqrt_est(u128 x) {
    if (x >> 100) return (uint64_t)isqrt128(x);
    const double dx = (double)(uint64_t)(x >> 64) * 18446744073709551616.0 + (double)(uint64_t)x;
    uint64_t r = (uint64_t)__builtin_sqrt(dx);
    while ((u128)r * r > x) r--;
    while ((u128)(r + 1) * (r + 1) <= x) r++;
    return r;
}

// floor(2^64 / s) for s >= 2: 2^64 - 1 = q s + r, so 2^64 = q s + r + 1.
HS_HD uint64_t div_2p64(uint64_t s) {
    const uint64_t q = ~(uint64_t)0 / s;
    const uint64_t r = ~(uint64_t)0 - q * s;
    return r + 1 == s ? q + 1 : q;
}

// floor(x / d) for d >= 1: long division over the four 32-bit limbs (each step divides a
// value below d * 2^32 <= 2^64).
HS_HD u128 div_u128_u32(u128 x, uint32_t d) {
    u128 q = 0;
    uint64_t rem = 0;
    for (int i = 3; i >= 0; i--) {
        const uint64_t cur = (rem << 32) | (uint64_t)(uint32_t)(x >> (32 * i));
        const uint64_t qi = cur / d;
        rem = cur - qi * d;
        q |= (u128)qi << (32 * i);
    }
    return q;
}

// floor((u1 * 2^64 + u0) / v) for u1 < v (the quotient fits 64 bits): the two-digit long
// division with normalized 32-bit digits of H. S. Warren, Hacker's Delight, 2nd ed., 9-4
// ("divlu"), with 64-bit words.
HS_HD uint64_t div_u128_u64(uint64_t u1, uint64_t u0, uint64_t v) {
    const uint64_t b = (uint64_t)1 << 32;
    const int s = clz64(v);
    v <<= s;
    const uint64_t vn1 = v >> 32, vn0 = v & 0xffffffffu;
    const uint64_t un32 = s ? (u1 << s) | (u0 >> (64 - s)) : u1;
    const uint64_t un10 = u0 << s;
    const uint64_t un1 = un10 >> 32, un0 = un10 & 0xffffffffu;
    uint64_t q1 = un32 / vn1, rhat = un32 - q1 * vn1;
    while (q1 >= b || q1 * vn0 > b * rhat + un1) {
        q1--;
        rhat += vn1;
        if (rhat >= b) break;
    }
    const uint64_t un21 = un32 * b + un1 - q1 * v;
    uint64_t q0 = un21 / vn1;
    rhat = un21 - q0 * vn1;
    while (q0 >= b || q0 * vn0 > b * rhat + un0) {
        q0--;
        rhat += vn1;
        if (rhat >= b) break;
    }
    return q1 * b + q0;
}

// The reciprocal of FreqTable::from_weights' quotient: floor(spare * 2^64 / W) for
// spare < W (W >= 2^32 > spare in the coder).
HS_HD uint64_t coder_frac(uint64_t spare, uint64_t W) { return div_u128_u64(spare, 0, W); }

// floor(w * spare / W) for w <= W (freq.rs:103-149): a plain u64 division when W < 2^32 (then
// w * spare < 2^64), else the 64-bit reciprocal frac = floor(spare 2^64 / W) and one correction
// (the estimate is at most one below the quotient).
HS_HD uint64_t quotient(uint64_t w, uint64_t spare, uint64_t W, uint64_t frac) {
    if (W < ((uint64_t)1 << 32)) return (w * spare) / W;
    uint64_t est = (uint64_t)(((u128)w * frac) >> 64);
    const u128 num = (u128)w * spare;
    if (num - (u128)est * W >= W) est++;
    return est;
}

// shift_round(t * g, s) for 64 <= s <= 126 from the high word of the product only:
// floor((P + 2^(s-1)) / 2^s) = floor((P_hi + 2^(s-65)) / 2^(s-64)) for s >= 65 (the low word
// cannot carry the floor across an integer), and P_hi + [P_lo >= 2^63] for s = 64. |t g| < 2^126.
HS_HD int64_t shift_round_hi(int64_t t, int64_t g, uint32_t s) {
    const i128 p = (i128)t * (i128)g;
    const int64_t hi = (int64_t)(p >> 64);
    if (s == 64) return hi + (int64_t)((uint64_t)p >> 63);
    const uint32_t u = s - 64;
    return (hi + ((int64_t)1 << (u - 1))) >> u;
}

// The LayerNorm element rule in single precision for 8-bit outputs with |beta| <= 256:
// clamp(floor(X + 1/2) + beta, +-127) for X = c inv m gamma 2^-s, from y = c k + b with
// k = float(inv m 2^-s) gamma (two roundings) and b = 1/2 + beta (exact), one fused
// multiply-add. |y - (X + b)| <= 3.0001 2^-24 |X| + 2^-24 |y|. y is clamped to [-126.5, 127.5]:
// inside, |X| < 458 and the error is below 1575 2^-24 < 2^-13, so floor(y) is exact when y lies
// at least 2^-13 from an integer, and it lies in [-127, 127] (no output clamp); outside, y has
// the sign and size of X + b (relative error below 2^-21), so floor(X + b) is at least 127 or at
// most -127 and the output clamp gives the floor of the clamped y, whose fraction is 1/2.
// |k| <= 2^110 keeps y finite or an infinity of the sign of c k (never NaN). Returns false
// (declines) near an integer; *out is then unused.
HS_HD bool ln_elem_f32(int32_t c, float k, float b, int32_t *out) {
    const float y = fmaf((float)c, k, b);
    const float yc = fminf(fmaxf(y, -126.5f), 127.5f);
    const float fl = floorf(yc);
    const float f = yc - fl;
    *out = (int32_t)fl;
    return fabsf(f - 0.5f) <= 0.5f - 0x1p-13f;
}

// floor((c inv gamma m + 2^(s - 1)) / 2^s) (the LayerNorm element rule, layernorm.rs:66-108,
// s <= 126) in double precision, with kr = ldexp((double)inv * m, -s) of the row:
// v = fma(c kr, gamma, 1/2). The roundings (inv to double, inv m, c kr, the fma) keep
// |v - (z + 1/2)| <= 4 2^-53 (|z| + 1) < 2^-20 for |v| <= 2^30 (z the exact quotient), so
// floor(v) is floor(z + 1/2) when v lies at least 2^-20 from an integer. Adding 1.5 2^52 rounds
// v to the nearest integer r (exact for |v| <= 2^30; r is the low word of the sum's encoding) and
// dl = v - r is exact, so floor(v) = r - [dl < 0]. Returns false (f unset) when the distance test
// fails: the caller then takes the integer rule. |f| <= 2^30.
HS_HD bool ln_elem_f64(int32_t c, double kr, double gamma, int32_t *f) {
    const double v = fma((double)c * kr, gamma, 0.5);
    const double t = v + 6755399441055744.0;
    const double dl = v - (t - 6755399441055744.0);
    if (!(fabs(v) <= 1073741824.0 && fabs(dl) >= 0x1p-20)) return false;
    uint64_t bits;
    memcpy(&bits, &t, sizeof bits);
    *f = (int32_t)(uint32_t)bits - (dl < 0.0 ? 1 : 0);
    return true;
}

// floor(a / d) for d >= 1 and |a| < 2^52, from inv_d = 1.0 / d (rounded to double). For d >= 2
// the product a inv_d lies within |a / d| 2^-51 < 1/2 of a / d (d = 1 is exact), so its floor is
// within one of the quotient; the exact remainder a - q d then corrects it (|q d| <= |a| + d).
HS_HD int64_t floor_div_est(int64_t a, int64_t d, double inv_d) {
    int64_t q = (int64_t)__builtin_floor((double)a * inv_d);
    const int64_t r = a - q * d;
    if (r < 0) q--;
    else if (r >= d) q++;
    return q;
}

// floor(x / n) for n >= 1 when the quotient is below 2^62, from inv_n = 1.0 / n. The double
// estimate of x / n carries a relative error below 2^-50 (x to double, the product), so it is
// within 2^12 of the quotient; the remainder x - q1 n then has |x - q1 n| < 2^13 n < 2^45 and is
// exact in 64-bit two's complement arithmetic, and floor_div_est finishes the quotient.
HS_HD uint64_t div_u128_est(u128 x, uint32_t n, double inv_n) {
    const double dx = (double)(uint64_t)(x >> 64) * 18446744073709551616.0 + (double)(uint64_t)x;
    const uint64_t q1 = (uint64_t)(dx * inv_n);
    const int64_t r = (int64_t)((uint64_t)x - q1 * (uint64_t)n);
    return (uint64_t)((int64_t)q1 + floor_div_est(r, n, inv_n));
}

// floor(2^k / r) for k <= 62 and 1 <= r < 2^53: the correctly rounded double quotient is within
// 2^k 2^-53 of 2^k / r, so for k <= 52 its truncation is within one of the quotient, and the
// exact remainder corrects it; larger k take the integer division.
HS_HD uint64_t pow2_div_est(uint32_t k, uint64_t r) {
    const int64_t num = (int64_t)1 << k;
    if (k > 52) return (uint64_t)num / r;
    int64_t q = (int64_t)((double)num / (double)r);
    const int64_t rem = num - q * (int64_t)r;
    if (rem < 0) q--;
    else if (rem >= (int64_t)r) q++;
    return (uint64_t)q;
}

// The LayerNorm scale of a row (layernorm.rs:188-256): inv = floor(2^k / isqrt(var 2^(2j) + eps))
// with var = floor(sq / n). k <= 48 and the root is below 2^64, so the division is in u64.
HS_HD uint64_t ln_inv(u128 sq, uint32_t n, uint32_t k, uint32_t j, uint64_t eps) {
    const u128 var = div_u128_u32(sq, n);
    const uint64_t r = isqrt_est((var << (2 * j)) + (u128)eps);
    return ((uint64_t)1 << k) / (r > 0 ? r : 1);
}

// ln_inv for rows of the residual stream: sq < n 2^62 (every |x - mean| < 2^31), so var < 2^62,
// var 2^(2j) + eps < 2^100 for j <= 18, and the root is below 2^50; the divisions take the
// estimate-and-correct forms above (inv_n = 1.0 / n). Equal to ln_inv on that domain.
HS_HD uint64_t ln_inv_est(u128 sq, uint32_t n, uint32_t k, uint32_t j, uint64_t eps, double inv_n) {
    const uint64_t var = div_u128_est(sq, n, inv_n);
    const uint64_t r = isqrt_est(((u128)var << (2 * j)) + (u128)eps);
    return pow2_div_est(k, r > 0 ? r : 1);
}

// The softmax weight p = floor(e 2^P / S) (softmax.rs:78-104) of a table entry e <= S, e < 2^31,
// S < 2^53, P <= 30, exactly and without a branch. The row gives R = 2^P / S rounded once and
// sp = -S 2^-P (exact). n = round(e R) comes from one fused multiply-add (adding 1.5 2^52 rounds
// to an integer, the low word of the sum); |e R - e 2^P / S| <= 2^P 2^-53, so
// |n - e 2^P / S| < 1/2 + 2^-23 and n is p or p + 1. p = n - 1 exactly when e 2^P < n S: the sign
// of fma(n, sp, e) = (e 2^P - n S) 2^-P rounded once, since every operand is exact (n is
// w - 1.5 2^52 exactly, S < 2^53, e < 2^31), a rounding keeps the sign of a nonzero value and an
// exact zero gives +0. The sign word shifted arithmetically is -1 or 0.
// The attention output byte clamp(rescale_full(v, m, s), +-127) (attention.rs:36-46, int.rs:63-67)
// of v = hi 2^16 + lo, the pairwise sums of the four digit-plane products, for
// |hi|, |lo| <= 2^30 + 2^22 and 48 <= s <= 63, in i64: with A = hi m and B = lo m + 2^(s-1)
// (|A| < 2^61.01, |B| < 2^63), v m + 2^(s-1) = A 2^16 + B, and
// floor((A 2^16 + B) / 2^s) = floor((A + floor(B / 2^16)) / 2^(s-16)) (A is an integer, and
// floor(floor(z) / n) = floor(z / n)); C = A + (B >> 16) stays below 2^61.02, so its high word
// shifted by s - 48 is the quotient, an i32.
HS_HD int32_t attn_out_planes(int32_t hi, int32_t lo, int32_t m, uint32_t s) {
    const int64_t b = (int64_t)lo * m + ((int64_t)1 << (s - 1));
    const int64_t c = (int64_t)hi * m + (b >> 16);
    const int32_t r = (int32_t)(c >> 32) >> (s - 48);
    return r < -127 ? -127 : (r > 127 ? 127 : r);
}

HS_HD double softmax_sp(uint64_t S, int P) { return -ldexp((double)S, -P); }
HS_HD uint32_t softmax_p_of(uint32_t e, double R, double sp) {
    const double ed = (double)e;
    const double w = fma(ed, R, 6755399441055744.0);
    const double r = fma(w - 6755399441055744.0, sp, ed);
    uint64_t wb, rb;
    memcpy(&wb, &w, sizeof wb);
    memcpy(&rb, &r, sizeof rb);
    return (uint32_t)wb + (uint32_t)((int32_t)(rb >> 32) >> 31);
}

}  // namespace hs
