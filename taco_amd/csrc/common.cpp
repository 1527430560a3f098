#include "common.h"

#include <cstdlib>
#include <cstring>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

namespace hs {

namespace {
thread_local std::string g_msg;
thread_local int g_code = 0;

inline uint32_t rotr(uint32_t x, unsigned n) { return (x >> n) | (x << (32 - n)); }

const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
    0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
    0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
    0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
    0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
    0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
    0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
    0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
    0xc67178f2};

void compress(uint32_t h[8], const uint8_t blk[64]) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = (uint32_t)blk[4 * i] << 24 | (uint32_t)blk[4 * i + 1] << 16 |
               (uint32_t)blk[4 * i + 2] << 8 | blk[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = hh + S1 + ch + K256[i] + w[i];
        uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
}  // namespace

hs_status fail(hs_status st, int code, const std::string &msg) {
    g_msg = msg;
    g_code = code;
    return st;
}

void clear_error() {
    g_msg.clear();
    g_code = 0;
}

namespace {

#if defined(__x86_64__)
// The same compression with the x86 SHA extensions (sha256rnds2 runs two rounds on the state
// split as ABEF / CDGH; sha256msg1 / sha256msg2 extend the message schedule four words at a time).
__attribute__((target("sha,sse4.1,ssse3"))) void compress_ni(uint32_t h[8], const uint8_t *data, size_t nblk) {
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
    __m128i t = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[0]), 0xB1);  // C D A B
    __m128i s1 = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[4]), 0x1B);  // E F G H
    __m128i s0 = _mm_alignr_epi8(t, s1, 8);                                         // A B E F
    s1 = _mm_blend_epi16(s1, t, 0xF0);                                              // C D G H
    for (size_t b = 0; b < nblk; b++, data += 64) {
        const __m128i save0 = s0, save1 = s1;
        __m128i w[4];
        for (int q = 0; q < 16; q++) {
            if (q < 4) {
                w[q] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i *)(data + 16 * q)), bswap);
            } else {
                __m128i x = _mm_sha256msg1_epu32(w[(q - 4) & 3], w[(q - 3) & 3]);
                x = _mm_add_epi32(x, _mm_alignr_epi8(w[(q - 1) & 3], w[(q - 2) & 3], 4));
                w[q & 3] = _mm_sha256msg2_epu32(x, w[(q - 1) & 3]);
            }
            const __m128i wk = _mm_add_epi32(w[q & 3], _mm_loadu_si128((const __m128i *)&K256[4 * q]));
            s1 = _mm_sha256rnds2_epu32(s1, s0, wk);
            s0 = _mm_sha256rnds2_epu32(s0, s1, _mm_shuffle_epi32(wk, 0x0E));
        }
        s0 = _mm_add_epi32(s0, save0);
        s1 = _mm_add_epi32(s1, save1);
    }
    t = _mm_shuffle_epi32(s0, 0x1B);             // F E B A
    s1 = _mm_shuffle_epi32(s1, 0xB1);            // D C H G
    s0 = _mm_blend_epi16(t, s1, 0xF0);           // D C B A
    s1 = _mm_alignr_epi8(s1, t, 8);              // H G F E
    _mm_storeu_si128((__m128i *)&h[0], s0);
    _mm_storeu_si128((__m128i *)&h[4], s1);
}

// HS_SHA256_PORTABLE=1 selects the portable compression (for tests of both forms).
bool have_sha_ni() {
    static const bool yes = !std::getenv("HS_SHA256_PORTABLE") && __builtin_cpu_supports("sha") &&
                            __builtin_cpu_supports("sse4.1") && __builtin_cpu_supports("ssse3");
    return yes;
}
#endif

void compress_blocks(uint32_t h[8], const uint8_t *data, size_t nblk) {
#if defined(__x86_64__)
    if (have_sha_ni()) {
        compress_ni(h, data, nblk);
        return;
    }
#endif
    for (size_t b = 0; b < nblk; b++) compress(h, data + 64 * b);
}

}  // namespace

void sha256(const uint8_t *data, size_t len, uint8_t out[32]) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    size_t i = len / 64 * 64;
    compress_blocks(h, data, len / 64);
    uint8_t tail[128] = {0};
    const size_t rest = len - i;
    std::memcpy(tail, data + i, rest);
    tail[rest] = 0x80;
    const size_t tl = rest + 9 <= 64 ? 64 : 128;
    const uint64_t bits = (uint64_t)len * 8;
    for (int b = 0; b < 8; b++) tail[tl - 1 - b] = (uint8_t)(bits >> (8 * b));
    compress_blocks(h, tail, tl / 64);
    for (int k = 0; k < 8; k++)
        for (int b = 0; b < 4; b++) out[4 * k + b] = (uint8_t)(h[k] >> (24 - 8 * b));
}

}  // namespace hs

extern "C" const char *hs_last_error_message(void) { return hs::g_msg.c_str(); }
extern "C" int hs_last_error_code(void) { return hs::g_code; }
