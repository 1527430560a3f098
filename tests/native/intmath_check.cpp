// Host build of taco_amd/csrc/intmath.h against plain unsigned __int128 arithmetic (libgcc's
// exact division) and the digit-by-digit square root of the rule: edge cases and seeded
// random cases. Prints "ok <n>" or the first mismatch and exits 1.
#include <cstdio>
#include <cstdlib>
#include <initializer_list>

#include "../../taco_amd/csrc/intmath.h"

using hs::i128;
using hs::u128;

static uint64_t sm_state = 0x1234567;
static uint64_t next() {  // splitmix64
    uint64_t z = (sm_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static uint64_t rnd_bits() {  // random value with a random bit length
    const int b = (int)(next() % 65);
    return b == 0 ? 0 : (b == 64 ? next() : next() & ((1ull << b) - 1));
}

static u128 isqrt_ref(u128 x) {  // bitwise from 2^126 as int.rs
    u128 bit = (u128)1 << 126;
    while (bit > x) bit >>= 2;
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

#define CHECK(cond, ...)                   \
    do {                                   \
        if (!(cond)) {                     \
            std::printf(__VA_ARGS__);      \
            std::printf("\n");             \
            return 1;                      \
        }                                  \
    } while (0)

int main(int argc, char **argv) {
    const long n = argc > 1 ? std::atol(argv[1]) : 200000;
    long count = 0;
    // div_2p64
    const uint64_t edge[] = {2, 3, 4, 5, 7, 1ull << 32, (1ull << 32) + 1, (1ull << 63), (1ull << 63) + 1,
                             ~0ull, ~0ull - 1, 1000000007ull, 1ull << 40};
    for (uint64_t s : edge) {
        CHECK(hs::div_2p64(s) == (uint64_t)(((u128)1 << 64) / s), "div_2p64 %llu", (unsigned long long)s);
        count++;
    }
    for (long i = 0; i < n; i++) {
        uint64_t s = rnd_bits();
        if (s < 2) s = 2;
        CHECK(hs::div_2p64(s) == (uint64_t)(((u128)1 << 64) / s), "div_2p64 %llu", (unsigned long long)s);
        count++;
    }
    // div_u128_u32
    for (long i = 0; i < n; i++) {
        const u128 x = ((u128)rnd_bits() << 64) | rnd_bits();
        uint32_t d = (uint32_t)rnd_bits();
        if (d == 0) d = 1 + (uint32_t)(next() % 1000);
        CHECK(hs::div_u128_u32(x, d) == x / d, "div_u128_u32");
        count++;
    }
    // div_u128_u64 (u1 < v)
    for (long i = 0; i < n; i++) {
        uint64_t v = rnd_bits();
        if (v == 0) v = 1;
        const uint64_t u1 = v == 1 ? 0 : next() % v, u0 = (i & 1) ? next() : rnd_bits();
        const u128 want = (((u128)u1 << 64) | u0) / v;
        CHECK(hs::div_u128_u64(u1, u0, v) == (uint64_t)want, "div_u128_u64 %llu %llu %llu",
              (unsigned long long)u1, (unsigned long long)u0, (unsigned long long)v);
        count++;
    }
    for (uint64_t v : edge) {
        for (uint64_t u1 : {(uint64_t)0, (uint64_t)1, v - 1, v / 2}) {
            if (u1 >= v) continue;
            for (uint64_t u0 : {(uint64_t)0, ~(uint64_t)0, (uint64_t)1 << 63}) {
                const u128 want = (((u128)u1 << 64) | u0) / v;
                CHECK(hs::div_u128_u64(u1, u0, v) == (uint64_t)want, "div_u128_u64 edge");
                count++;
            }
        }
    }
    // coder_frac and quotient against the exact floor(w * spare / W)
    for (long i = 0; i < n; i++) {
        const uint64_t spare = next() >> 32;
        uint64_t W = rnd_bits();
        if (W <= spare) W = spare + 1 + (next() >> 8);
        const uint64_t w = W == 0 ? 0 : next() % (W + 1);
        const uint64_t frac = W >= (1ull << 32) ? hs::coder_frac(spare, W) : 0;
        if (W >= (1ull << 32))
            CHECK(frac == (uint64_t)((((u128)spare) << 64) / W), "coder_frac");
        CHECK(hs::quotient(w, spare, W, frac) == (uint64_t)(((u128)w * spare) / W), "quotient");
        count++;
    }
    // isqrt128
    for (long i = 0; i < n; i++) {
        const int sh = (int)(next() % 128);
        const u128 x = (((u128)next() << 64) | next()) >> sh;
        const u128 r = hs::isqrt128(x);
        CHECK(r == isqrt_ref(x), "isqrt128");
        CHECK(r * r <= x && (r + 1) * (r + 1) > x, "isqrt128 bound");
        count++;
    }
    for (u128 x : {(u128)0, (u128)1, (u128)2, (u128)3, (u128)4, ~(u128)0, (u128)1 << 126, ((u128)1 << 126) - 1}) {
        CHECK(hs::isqrt128(x) == isqrt_ref(x), "isqrt128 edge");
        count++;
    }
    // isqrt_est (double estimate + exact correction) against the bitwise root
    for (long i = 0; i < n; i++) {
        const int sh = (int)(next() % 128);
        const u128 x = (((u128)next() << 64) | next()) >> sh;
        CHECK((u128)hs::isqrt_est(x) == isqrt_ref(x), "isqrt_est");
        count++;
    }
    for (int b = 0; b < 127; b++)
        for (int dlt = -2; dlt <= 2; dlt++) {
            const u128 base = (u128)1 << b;
            const u128 r = isqrt_ref(base);
            const u128 x = (dlt < 0 && base < (u128)(-dlt)) ? 0 : base + dlt;
            const u128 sqv = r * r + dlt;  // around perfect squares too
            CHECK((u128)hs::isqrt_est(x) == isqrt_ref(x), "isqrt_est pow2");
            if (dlt >= -1 || r * r >= 2) CHECK((u128)hs::isqrt_est(sqv) == isqrt_ref(sqv), "isqrt_est square");
            count += 2;
        }
    // shift_round_hi against the i128 rule (|t g| < 2^126, 64 <= s <= 126)
    for (long i = 0; i < n; i++) {
        const int tb = (int)(next() % 63), gb = (int)(next() % 63);
        int64_t t = (int64_t)(next() >> (64 - tb)), gg = (int64_t)(next() >> (64 - gb));
        if (next() & 1) t = -t;
        if (next() & 1) gg = -gg;
        const uint32_t sh = 64 + (uint32_t)(next() % 63);
        const i128 want = hs::shift_round128((i128)t * (i128)gg, sh, 126);
        CHECK((i128)hs::shift_round_hi(t, gg, sh) == want, "shift_round_hi %lld %lld %u", (long long)t, (long long)gg, sh);
        count++;
    }
    // ln_inv against the u128 form
    for (long i = 0; i < n / 4; i++) {
        const u128 sq = ((u128)(next() >> (next() % 64)) << (next() % 12)) * (1 + next() % 3);
        const uint32_t nn = 1 + (uint32_t)(next() % 4096), k = (uint32_t)(next() % 49), j = (uint32_t)(next() % 17);
        const uint64_t eps = 1 + (next() >> (2 + next() % 62));
        const u128 var = sq / nn;
        const u128 root = isqrt_ref((var << (2 * j)) + eps);
        const uint64_t want = (uint64_t)(((u128)1 << k) / root);
        CHECK(hs::ln_inv(sq, nn, k, j, eps) == want, "ln_inv");
        count++;
    }
    // the estimate-and-correct divisions of the LayerNorm row scale against exact division
    auto floor_ref = [](int64_t a, int64_t d) { return a >= 0 ? a / d : -((-a + d - 1) / d); };
    for (long i = 0; i < n; i++) {
        int64_t a = (int64_t)(next() >> (12 + next() % 52));  // |a| < 2^52
        if (next() & 1) a = -a;
        const int64_t d = (next() & 3) == 0 ? 1 + (int64_t)(next() % 8) : 1 + (int64_t)(next() % (1u << 22));
        const int64_t near = (next() & 1) ? (a / d) * d + (int64_t)(next() % 3) - 1 : a;  // next to multiples
        for (int64_t v : {a, near}) {
            if (v >= ((int64_t)1 << 52) || v <= -((int64_t)1 << 52)) continue;
            CHECK(hs::floor_div_est(v, d, 1.0 / (double)d) == floor_ref(v, d), "floor_div_est %lld %lld",
                  (long long)v, (long long)d);
            count++;
        }
    }
    for (long i = 0; i < n; i++) {  // x < n 2^62, the quotient below 2^62
        const uint32_t nn = (next() & 3) == 0 ? 1 + (uint32_t)(next() % 4) : 1 + (uint32_t)(next() % 4096);
        const u128 lim = (u128)nn << 62;
        u128 x = (((u128)next() << 64) | next()) % lim;
        if ((next() & 7) == 0) x = lim - 1 - (u128)(next() % 4);
        if ((next() & 7) == 1) x = (x / nn) * nn + (next() % 2);  // exact multiples and one past
        if (x >= lim) x = lim - 1;
        CHECK((u128)hs::div_u128_est(x, nn, 1.0 / (double)nn) == x / nn, "div_u128_est");
        count++;
    }
    for (long i = 0; i < n; i++) {
        const uint32_t k = (uint32_t)(next() % 63);
        uint64_t r = 1 + (next() >> (11 + next() % 53));  // 1 .. 2^53
        if ((next() & 7) == 0) r = (uint64_t)1 << (next() % 53);
        if (r >= ((uint64_t)1 << 53)) r = ((uint64_t)1 << 53) - 1;
        CHECK(hs::pow2_div_est(k, r) == ((uint64_t)1 << k) / r, "pow2_div_est %u %llu", k, (unsigned long long)r);
        count++;
    }
    for (long i = 0; i < n / 4; i++) {  // ln_inv_est equals ln_inv on rows of the residual stream
        const uint32_t nn = 1 + (uint32_t)(next() % 4096), k = (uint32_t)(next() % 49), j = (uint32_t)(next() % 17);
        const u128 lim = (u128)nn << 62;
        u128 sq = ((((u128)next() << 64) | next()) >> (next() % 128)) % lim;
        if ((next() & 7) == 0) sq = lim - 1;
        const uint64_t eps = (next() & 3) == 0 ? 0 : 1 + (next() >> (2 + next() % 62));
        CHECK(hs::ln_inv_est(sq, nn, k, j, eps, 1.0 / (double)nn) == hs::ln_inv(sq, nn, k, j, eps), "ln_inv_est");
        count++;
    }
    // ln_elem_f64 against floor((c inv gamma m + 2^(s-1)) / 2^s) in i128 (|product| < 2^126):
    // every value it returns is exact; it may only decline.
    auto exact_ln = [](int32_t c, uint64_t inv, int32_t g, int32_t m, uint32_t s) -> i128 {
        const i128 p = (i128)c * (i128)inv * (i128)g * (i128)m;
        return s == 0 ? p : (p + ((i128)1 << (s - 1))) >> s;
    };
    long declined = 0, taken = 0;
    auto check_ln = [&](int32_t c, uint64_t inv, int32_t g, int32_t m, uint32_t s) -> bool {
        const double kr = std::ldexp((double)inv * (double)m, -(int)s);
        int32_t f = 0;
        if (!hs::ln_elem_f64(c, kr, (double)g, &f)) {
            declined++;
            return true;
        }
        taken++;
        return (i128)f == exact_ln(c, inv, g, m, s);
    };
    for (long i = 0; i < n; i++) {
        // the fold's range: |c| < 2^31, inv < 2^64, |gamma| < 2^15, m < 2^31, |product| < 2^126
        const int32_t c = (int32_t)(next() >> (33 + next() % 31)) * ((next() & 1) ? -1 : 1);
        const int32_t g = (int32_t)(next() % 65535) - 32767;
        const int32_t m = (int32_t)(next() >> (33 + next() % 31));
        uint64_t inv = rnd_bits();
        const int lc = 64 - hs::clz64((uint64_t)(c < 0 ? -(int64_t)c : c)), lg = 16, lm = 64 - hs::clz64((uint64_t)m);
        const int room = 125 - lc - lg - lm;
        if (room < 64) inv = room <= 0 ? 0 : inv & ((1ull << room) - 1);
        const uint32_t s = (uint32_t)(next() % 127);
        CHECK(check_ln(c, inv, g, m, s), "ln_elem_f64 c %d inv %llu g %d m %d s %u", c, (unsigned long long)inv, g, m, s);
        count++;
    }
    // adversarial: quotients exactly on and just beside a half (p = k 2^s + 2^(s-1) + delta)
    for (uint32_t s = 1; s <= 63; s++)
        for (long k = -70; k <= 70; k += 7)
            for (int delta = -3; delta <= 3; delta++) {
                const i128 p = (i128)k * ((i128)1 << s) + ((i128)1 << (s - 1)) + delta;
                if (p <= 0 || p >= ((i128)1 << 64)) continue;
                CHECK(check_ln(1, (uint64_t)p, 1, 1, s), "ln_elem_f64 half s %u k %ld d %d", s, k, delta);
                CHECK(check_ln(-1, (uint64_t)p, 1, 1, s), "ln_elem_f64 -half s %u k %ld d %d", s, k, delta);
                CHECK(check_ln(1, (uint64_t)p, -1, 1, s), "ln_elem_f64 -g half s %u k %ld d %d", s, k, delta);
                count += 3;
            }
    CHECK(taken > n / 2, "ln_elem_f64 declined too often (%ld of %ld)", declined, declined + taken);
    // ln_elem_f32 against clamp(floor((c inv gamma m + 2^(s-1)) / 2^s) + beta, +-127) in i128 for
    // |beta| <= 256, with k and b formed as the kernel forms them: every value it returns is exact.
    long declined32 = 0, taken32 = 0;
    auto check_ln32 = [&](int32_t c, uint64_t inv, int32_t g, int32_t m, uint32_t s, int32_t beta) -> bool {
        const float krf = (float)std::ldexp((double)inv * (double)m, -(int)s);
        int32_t y = 0;
        if (!hs::ln_elem_f32(c, krf * (float)g, 0.5f + (float)beta, &y)) {
            declined32++;
            return true;
        }
        taken32++;
        i128 want = exact_ln(c, inv, g, m, s) + beta;
        want = want < -127 ? -127 : (want > 127 ? 127 : want);
        return (i128)y == want;
    };
    for (long i = 0; i < n; i++) {
        const int32_t c = (int32_t)(next() >> (33 + next() % 31)) * ((next() & 1) ? -1 : 1);
        const int32_t g = (int32_t)(next() % 65535) - 32767;
        const int32_t m = (int32_t)(next() >> (33 + next() % 31)) * ((next() & 1) ? -1 : 1);
        uint64_t inv = rnd_bits();
        const int lc = 64 - hs::clz64((uint64_t)(c < 0 ? -(int64_t)c : c)), lg = 16;
        const int lm = 64 - hs::clz64((uint64_t)(m < 0 ? -(int64_t)m : m));
        const int room = 125 - lc - lg - lm;
        if (room < 64) inv = room <= 0 ? 0 : inv & ((1ull << room) - 1);
        const uint32_t s = (uint32_t)(next() % 127);
        const int32_t beta = (int32_t)(next() % 513) - 256;
        CHECK(check_ln32(c, inv, g, m, s, beta), "ln_elem_f32 c %d inv %llu g %d m %d s %u beta %d", c,
              (unsigned long long)inv, g, m, s, beta);
        count++;
    }
    // outputs near the clamp and quotients on and beside a half
    for (uint32_t s = 1; s <= 63; s++)
        for (long k = -400; k <= 400; k += 13)
            for (int delta = -3; delta <= 3; delta++) {
                const i128 p = (i128)k * ((i128)1 << s) + ((i128)1 << (s - 1)) + delta;
                if (p <= 0 || p >= ((i128)1 << 64)) continue;
                for (int32_t beta : {-256, -130, -1, 0, 1, 127, 256}) {
                    CHECK(check_ln32(1, (uint64_t)p, 1, 1, s, beta), "ln_elem_f32 half s %u k %ld d %d b %d", s, k, delta, beta);
                    CHECK(check_ln32(-1, (uint64_t)p, 1, 1, s, beta), "ln_elem_f32 -half s %u k %ld d %d b %d", s, k, delta, beta);
                    count += 2;
                }
            }
    CHECK(taken32 > n / 2, "ln_elem_f32 declined too often (%ld of %ld)", declined32, declined32 + taken32);
    // softmax_p_of: floor(e 2^P / S) for e <= S, e < 2^31, S < 2^53, P <= 30; random rows and
    // entries on, just below and just above the multiples of S / 2^P
    auto check_p = [&](uint32_t e, uint64_t S, int P) -> bool {
        const double R = ldexp(1.0 / (double)S, P);
        const uint64_t want = (uint64_t)(((u128)e << P) / S);
        return hs::softmax_p_of(e, R, hs::softmax_sp(S, P)) == (uint32_t)want;
    };
    for (long i = 0; i < 4 * n; i++) {
        const int bits = 1 + (int)(next() % 52);
        uint64_t S = next() & ((1ull << bits) - 1);
        if (S == 0) S = 1;
        const int P = (int)(next() % 31);
        const uint64_t emax = S < 0x7FFFFFFFull ? S : 0x7FFFFFFFull;
        uint32_t e;
        if (i % 2) {
            e = (uint32_t)(next() % (emax + 1));
        } else {  // near the first e with floor(e 2^P / S) >= q
            const uint64_t q = next() % (((u128)emax << P) / S + 1);
            const u128 e0 = ((u128)q * S + ((u128)1 << P) - 1) >> P;
            const int delta = (int)(next() % 3) - 1;
            const i128 ev = (i128)e0 + delta;
            e = (uint32_t)(ev < 0 ? 0 : (ev > (i128)emax ? emax : (uint64_t)ev));
        }
        CHECK(check_p(e, S, P), "softmax_p_of e %u S %llu P %d", e, (unsigned long long)S, P);
        count++;
    }
    for (int P = 0; P <= 30; P++)
        for (uint64_t S : {1ull, 2ull, 3ull, 0x7FFFFFFFull, 0x80000000ull, 0xFFFFFFFFull, 0x100000001ull,
                           255ull * 0x7FFFFFFFull, (1ull << 53) - 1}) {
            const uint64_t emax = S < 0x7FFFFFFFull ? S : 0x7FFFFFFFull;
            for (uint64_t e : {(uint64_t)0, (uint64_t)1, emax / 2, emax - 1, emax}) {
                if (e > emax) continue;
                CHECK(check_p((uint32_t)e, S, P), "softmax_p_of edge e %llu S %llu P %d", (unsigned long long)e,
                      (unsigned long long)S, P);
                count++;
            }
        }
    // attn_out_planes: clamp(rescale_full(hi 2^16 + lo, m, s), +-127) for |hi|, |lo| <= 2^30 + 2^22,
    // 48 <= s <= 63; random planes and values on, just below and just above the rounding steps
    const int64_t PL = (1ll << 30) + (1ll << 22);
    auto check_out = [&](int64_t v, int32_t m, uint32_t s) -> bool {
        const int64_t hi = v >> 16, lo = v - (hi << 16);  // lo in [0, 2^16)
        if (hi > PL || hi < -PL) return true;           // outside the domain
        const int64_t want = hs::clamp128(hs::rescale_full(v, m, s), -127, 127);
        return hs::attn_out_planes((int32_t)hi, (int32_t)lo, m, s) == (int32_t)want;
    };
    for (long i = 0; i < 2 * n; i++) {
        const uint32_t s = 48 + (uint32_t)(next() % 16);
        const int32_t m = (int32_t)(uint32_t)next();
        const int64_t hi = (int64_t)(next() % (2 * PL + 1)) - PL, lo = (int64_t)(next() % (2 * PL + 1)) - PL;
        const int64_t want = hs::clamp128(hs::rescale_full(hi * 65536 + lo, m, s), -127, 127);
        CHECK(hs::attn_out_planes((int32_t)hi, (int32_t)lo, m, s) == (int32_t)want, "attn_out_planes %lld %lld %d %u",
              (long long)hi, (long long)lo, m, s);
        count++;
    }
    for (long i = 0; i < n; i++) {  // v m + 2^(s-1) beside a multiple of 2^s, |q| <= 200
        const uint32_t s = 48 + (uint32_t)(next() % 16);
        int32_t m = (int32_t)(uint32_t)(next() >> (next() % 32));
        if (m == 0) m = 1;
        if (next() & 1) m = -m;
        const i128 q = (i128)(int64_t)(next() % 401) - 200;
        const i128 num = q * ((i128)1 << s) - ((i128)1 << (s - 1));  // v m = num at the step
        const i128 am = m < 0 ? -(i128)m : (i128)m;
        const i128 v0 = (num >= 0 ? (num + am - 1) / am : -((-num) / am)) * (m < 0 ? -1 : 1);
        for (int d = -2; d <= 2; d++) {
            const i128 v = v0 + d;
            if (v > ((i128)1 << 46) || v < -((i128)1 << 46)) continue;
            CHECK(check_out((int64_t)v, m, s), "attn_out_planes step v %lld m %d s %u", (long long)v, m, s);
            count++;
        }
    }
    std::printf("ok %ld\n", count);
    return 0;
}
