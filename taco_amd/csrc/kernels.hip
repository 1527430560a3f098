// gfx950 (CDNA4, MI355X) kernels of the HardShell forward pass. Integer only; every result is
// the exact value of the reference CPU rule it cites (crates/hardshell/src/...). No atomics: all
// reductions are fixed-order wave/LDS trees, so results do not depend on scheduling.
#include <hip/hip_runtime.h>

#include "intmath.h"
#include "kernels.h"

namespace hs {

typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int32_t RES = (1 << 30) - 1;             // gpt2/mod.rs:116
constexpr int64_t SCORE_LIMIT = (int64_t)1 << 40;  // gpt2/mod.rs:119

// ---- wave reductions (wave64) -------------------------------------------------------------

__device__ __forceinline__ int64_t wave_max64(int64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        int64_t u = __shfl_xor(v, o, 64);
        v = u > v ? u : v;
    }
    return v;
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// =============================================================================================
// Int8 GEMM on MFMA: C[m][n] = sum_k A[m][k] * W[n][k] (both operands K-contiguous, "NT"),
// exact int32 (|C| <= 2^30 for K <= 2^16, crates/hardshell/src/kernels.rs:24-29), with the
// requantize epilogue of the op fused (crates/hardshell/src/gpt2/ops.rs:107-176).
//
// Tile 128 x 128 x 64, 256 threads = 4 waves in 2 x 2; each wave owns 64 x 64 = 4 x 4 tiles of
// v_mfma_i32_16x16x64_i8. Operands go global -> registers -> LDS (double buffered, one
// barrier per k-step); the next k-tile's global loads are in flight during the MFMAs.
// =============================================================================================

constexpr int LDS_STRIDE = GEMM_BK + 16;  // bytes per LDS row: 64 data + 16 pad (bank spread)

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) int8_t sA[2][GEMM_BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) int8_t sW[2][GEMM_BN * LDS_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-aware tile order: workgroup L runs on XCD L % 8, and XCD x takes the x-th contiguous
    // chunk of a grouped order (groups of `group` M-tiles, N outermost inside a group), so an
    // A row-tile stays in one XCD's L2 while the W tiles stream past it.
    int mt, nt;
    {
        const int gm = (g.m + GEMM_BM - 1) / GEMM_BM, gn = (g.n + GEMM_BN - 1) / GEMM_BN;
        const int T = gm * gn, L = blockIdx.x, x = L & 7, k = L >> 3;
        const int q = T >> 3, r = T & 7;
        const int p = x * q + (x < r ? x : r) + k;
        const int G = g.group, grp = p / (G * gn), in = p - grp * G * gn;
        const int gs = gm - grp * G < G ? gm - grp * G : G;
        nt = in / gs;
        mt = grp * G + in % gs;
    }
    const int m0 = mt * GEMM_BM, n0 = nt * GEMM_BN;
    const int K = g.k_pad, nk = K / GEMM_BK;
    const int8_t *A = g.a + (size_t)m0 * K;
    const int8_t *W = g.w + (size_t)n0 * K;

    // Each thread moves two 16-byte chunks of each 128 x 64 tile: chunk c -> row c / 4,
    // column 16 * (c % 4).
    const int c0 = tid, c1 = tid + 256;
    const int r0 = c0 >> 2, q0 = (c0 & 3) * 16, r1 = c1 >> 2, q1 = (c1 & 3) * 16;
    v4i ra0, ra1, rw0, rw1;
    auto gload = [&](int kt) {
        const int kk = kt * GEMM_BK;
        ra0 = *(const v4i *)(A + (size_t)r0 * K + kk + q0);
        ra1 = *(const v4i *)(A + (size_t)r1 * K + kk + q1);
        rw0 = *(const v4i *)(W + (size_t)r0 * K + kk + q0);
        rw1 = *(const v4i *)(W + (size_t)r1 * K + kk + q1);
    };
    auto sstore = [&](int st) {
        *(v4i *)(&sA[st][r0 * LDS_STRIDE + q0]) = ra0;
        *(v4i *)(&sA[st][r1 * LDS_STRIDE + q1]) = ra1;
        *(v4i *)(&sW[st][r0 * LDS_STRIDE + q0]) = rw0;
        *(v4i *)(&sW[st][r1 * LDS_STRIDE + q1]) = rw1;
    };

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};

    gload(0);
    sstore(0);
    __syncthreads();
    const int frow = lane & 15, fk = (lane >> 4) * 16;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        v4i af[4], bf[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            af[i] = *(const v4i *)(&sA[cur][(wm * 64 + i * 16 + frow) * LDS_STRIDE + fk]);
#pragma unroll
        for (int j = 0; j < 4; j++)
            bf[j] = *(const v4i *)(&sW[cur][(wn * 64 + j * 16 + frow) * LDS_STRIDE + fk]);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds C[4 * (lane / 16) + e][lane % 16] of each 16 x 16 tile.
    if (EPI == (int)Epi::LogitsCompact) {
        // logit = clamp(rescale(acc, m[n], s), +-2^40) (ops.rs:229-234), stored as the largest
        // logit of this wave's 64 columns (per row) and min(tilemax - logit, cap16) per logit.
        // The table index min(max - l, len - 1) is recovered exactly from them, because
        // max - l = (max - tilemax) + (tilemax - l) and cap16 >= len - 1.
        const int tile_n0 = n0 + wn * 64;
        int32_t mlt[4];
        bool okn[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = tile_n0 + j * 16 + (lane & 15);
            okn[j] = n < g.n;
            mlt[j] = okn[j] ? g.mult[n] : 0;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + e;
                int64_t l[4], mx = INT64_MIN;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    l[j] = okn[j] ? clamp64(rescale_small(acc[i][j][e], mlt[j], g.shift), -SCORE_LIMIT,
                                            SCORE_LIMIT)
                                  : INT64_MIN;
                    mx = l[j] > mx ? l[j] : mx;
                }
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {  // the 16 lanes that hold this row
                    const int64_t u = __shfl_xor(mx, o, 64);
                    mx = u > mx ? u : mx;
                }
                if (m < g.m) {
                    if ((lane & 15) == 0 && tile_n0 < g.n) g.tmax[(size_t)m * g.tmax_ld + tile_n0 / 64] = mx;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (!okn[j]) continue;
                        const int64_t dd = mx - l[j];
                        ((uint16_t *)g.out)[(size_t)m * g.ldo + tile_n0 + j * 16 + (lane & 15)] =
                            (uint16_t)(dd < g.cap16 ? dd : g.cap16);
                    }
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + wn * 64 + j * 16 + (lane & 15);
        if (n >= g.n) continue;
        int32_t bias = 0, mult = 0;
        if (EPI == (int)Epi::Act || EPI == (int)Epi::Residual || EPI == (int)Epi::Gelu) bias = g.bias[n];
        if (EPI != (int)Epi::Raw) mult = g.mult[n];
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + e;
                if (m >= g.m) continue;
                const int32_t a = acc[i][j][e];
                const size_t o = (size_t)m * g.ldo + n;
                if (EPI == (int)Epi::Raw) {
                    ((int32_t *)g.out)[o] = a;
                } else if (EPI == (int)Epi::Act) {  // ops.rs:123-130
                    const int64_t y = rescale_small((int64_t)a + bias, mult, g.shift);
                    ((int8_t *)g.out)[o] = (int8_t)clamp64(y, -127, 127);
                } else if (EPI == (int)Epi::Residual) {  // ops.rs:131-145
                    const int64_t y = clamp64(rescale_small((int64_t)a + bias, mult, g.shift),
                                              -SCORE_LIMIT, SCORE_LIMIT);
                    int32_t *x = (int32_t *)g.out + o;
                    *x = (int32_t)clamp64((int64_t)*x + y, -RES, RES);
                } else if (EPI == (int)Epi::Gelu) {  // ops.rs:146-154, gelu.rs:58-62
                    const int64_t y = clamp64(rescale_small((int64_t)a + bias, mult, g.shift),
                                              -g.gelu_off, g.gelu_off - 1);
                    ((int8_t *)g.out)[o] = g.gelu[y + g.gelu_off];
                } else {  // Logits: ops.rs:229-234
                    ((int64_t *)g.out)[o] =
                        clamp64(rescale_small(a, mult, g.shift), -SCORE_LIMIT, SCORE_LIMIT);
                }
            }
        }
    }
}

hipError_t launch_gemm(Epi epi, const GemmArgs &ga, hipStream_t stream) {
    GemmArgs g = ga;
    if (g.m <= 0 || g.n <= 0) return hipSuccess;
    const int gm = (g.m + GEMM_BM - 1) / GEMM_BM, gn = (g.n + GEMM_BN - 1) / GEMM_BN;
    if (g.group == 0) g.group = gemm_group(g.m);
    if (g.group < 1 || g.group > gm) return hipErrorInvalidValue;
    dim3 grid(gm * gn);
    switch (epi) {
        case Epi::Raw: hipLaunchKernelGGL(k_gemm<0>, grid, dim3(256), 0, stream, g); break;
        case Epi::Act: hipLaunchKernelGGL(k_gemm<1>, grid, dim3(256), 0, stream, g); break;
        case Epi::Residual: hipLaunchKernelGGL(k_gemm<2>, grid, dim3(256), 0, stream, g); break;
        case Epi::Gelu: hipLaunchKernelGGL(k_gemm<3>, grid, dim3(256), 0, stream, g); break;
        case Epi::Logits: hipLaunchKernelGGL(k_gemm<4>, grid, dim3(256), 0, stream, g); break;
        case Epi::LogitsCompact: hipLaunchKernelGGL(k_gemm<5>, grid, dim3(256), 0, stream, g); break;
    }
    return hipGetLastError();
}

// =============================================================================================
// Embedding (reference.rs:208-221): x = clamp(rescale(wte[tok]) + rescale(wpe[pos]), -R, R).
// =============================================================================================

__global__ void k_embed(const RowInfo *rows, const int8_t *wte, int wte_ld, const int8_t *wpe,
                        const int32_t *embed_m, int embed_s, const int32_t *pos_m, int pos_s,
                        int d, int32_t *x) {
    const int r = blockIdx.x, j = blockIdx.y * blockDim.x + threadIdx.x;
    if (j >= d) return;
    const RowInfo ri = rows[r];
    const int64_t v = rescale_small(wte[(size_t)ri.token * wte_ld + j], embed_m[ri.token], embed_s) +
                      rescale_small(wpe[(size_t)ri.pos * d + j], pos_m[ri.pos], pos_s);
    x[(size_t)r * d + j] = (int32_t)clamp64(v, -RES, RES);
}

hipError_t launch_embed(const RowInfo *rows, int n_rows, const int8_t *wte, int wte_ld,
                        const int8_t *wpe, const int32_t *embed_m, int embed_s,
                        const int32_t *pos_m, int pos_s, int d, int32_t *x, hipStream_t stream) {
    dim3 grid(n_rows, (d + 255) / 256);
    hipLaunchKernelGGL(k_embed, grid, dim3(256), 0, stream, rows, wte, wte_ld, wpe, embed_m,
                       embed_s, pos_m, pos_s, d, x);
    return hipGetLastError();
}

// =============================================================================================
// Integer LayerNorm (crates/hardshell/src/layernorm.rs:201-256), one workgroup per row:
// mean = floor(sum / n); var = floor(sum (x - mean)^2 / n) in u128; inv = 2^K / isqrt(var *
// 2^2J + eps); y = rescale_wide((x - mean) * inv * gamma, m, s) + beta (or the one-rounding form
// with beta_frac); out = clamp(y, -127, 127).
// =============================================================================================

__device__ __forceinline__ u128 wave_sum128(u128 v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t lo = __shfl_xor((uint64_t)v, o, 64);
        const uint64_t hi = __shfl_xor((uint64_t)(v >> 64), o, 64);
        v += ((u128)hi << 64) | lo;
    }
    return v;
}

// One wave per row, four rows per workgroup, no LDS and no barriers: the row sum, then the sum
// of squares of c = x - mean (|c| < 2^32, so a square fits u64 and each lane carries into a
// high word), and the per-row inv of ln_inv (no 128-bit division). The product c * inv * gamma
// * m is formed as (c * inv) * (gamma * m): the reference's bounds (|t| < 2^95, |m| < 2^31,
// layernorm.rs:31-39) keep it below 2^126, so its wrapping product never wraps and the two
// forms are the same integer. When max|c| * inv < 2^63 (exact test), c * inv is an i64.
__global__ __launch_bounds__(256) void k_layernorm(LnArgs a, int n_rows) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    const int d = a.d;
    const int src = a.src ? a.src[row] : row;
    const int32_t *x = a.x + (size_t)src * d;
    int64_t sum = 0;
    for (int j = lane; j < d; j += 64) sum += x[j];
    sum = wave_sum64(sum);
    const int64_t mean = floor_div64(sum, d);
    uint64_t lo = 0, hi = 0, cmax = 0;
    for (int j = lane; j < d; j += 64) {
        const int64_t c = (int64_t)x[j] - mean;
        const uint64_t u = c < 0 ? (uint64_t)(-c) : (uint64_t)c;
        const uint64_t v = u * u;
        lo += v;
        hi += lo < v;
        cmax = u > cmax ? u : cmax;
    }
    const u128 sq = wave_sum128(((u128)hi << 64) | lo);
    cmax = (uint64_t)wave_max64((int64_t)cmax);
    const uint64_t inv = ln_inv(sq, (uint32_t)d, (uint32_t)a.k, (uint32_t)a.j, a.eps);
    const bool small = (u128)cmax * inv < ((u128)1 << 63);
    int8_t *out = a.out + (size_t)row * a.ldo;
    for (int j = lane; j < d; j += 64) {
        const int64_t c = (int64_t)x[j] - mean;
        const i128 cinv = small ? (i128)(c * (int64_t)inv) : (i128)c * (i128)(u128)inv;
        const i128 p = cinv * (i128)a.gm[j];
        i128 y;
        if (a.beta_frac == 0) {
            y = shift_round128(p, a.s, 126) + (i128)a.beta[j];
        } else {
            const i128 cb = (i128)a.beta[j] << (a.s - a.beta_frac);
            y = shift_round128(p + cb, a.s, 126);
        }
        out[j] = (int8_t)clamp128(y, -127, 127);
    }
}

hipError_t launch_layernorm(const LnArgs &a, int n_rows, hipStream_t stream) {
    if (n_rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_layernorm, dim3((n_rows + 3) / 4), dim3(256), 0, stream, a, n_rows);
    return hipGetLastError();
}

// =============================================================================================
// K and V of each row into the cache at the row's position (reference.rs:246-252).
// Cache layout of one layer: [slot][head][position][hd].
// =============================================================================================

__global__ void k_kv_store(const RowInfo *rows, const int8_t *qkv, int d, int n_head, int hd,
                           int n_ctx, int8_t *kc, int8_t *vc) {
    const int r = blockIdx.x, c = blockIdx.y * blockDim.x + threadIdx.x;
    if (c >= d) return;
    const RowInfo ri = rows[r];
    const int h = c / hd, cc = c - h * hd;
    const size_t o = (((size_t)ri.slot * n_head + h) * n_ctx + ri.pos) * hd + cc;
    kc[o] = qkv[(size_t)r * 3 * d + d + c];
    vc[o] = qkv[(size_t)r * 3 * d + 2 * d + c];
}

hipError_t launch_kv_store(const RowInfo *rows, int n_rows, const int8_t *qkv, int d, int n_head,
                           int hd, int n_ctx, int8_t *kc, int8_t *vc, hipStream_t stream) {
    dim3 grid(n_rows, (d + 255) / 256);
    hipLaunchKernelGGL(k_kv_store, grid, dim3(256), 0, stream, rows, qkv, d, n_head, hd, n_ctx,
                       kc, vc);
    return hipGetLastError();
}

// =============================================================================================
// Causal integer attention (reference.rs:254-283, softmax.rs:78-104): one wave per (row, head)
// over the keys 0..pos of the row's slot. Three passes over the keys: the max score, the sum of
// the table entries, then p = floor(e * 2^P / S) and sum p * v in i64. Dots with v_dot4_i32_i8.
// =============================================================================================

__device__ __forceinline__ int32_t dot_key(const int *q4, const int8_t *k, int hd) {
    int32_t s = 0;
    const int *k4 = (const int *)k;
    for (int c = 0; c < hd / 4; c++) s = __builtin_amdgcn_sdot4(q4[c], k4[c], s, false);
    return s;
}

__global__ __launch_bounds__(256) void k_attend(AttnArgs a, int n_tasks) {
    __shared__ __attribute__((aligned(16))) int s_q[4][64];  // hd <= 256 bytes per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int task = blockIdx.x * 4 + wave;
    const bool valid = task < n_tasks;
    const int r = valid ? task / a.n_head : 0, h = valid ? task % a.n_head : 0;
    const int hd = a.hd;
    int slot, keys;
    if (a.rows) {
        slot = a.rows[r].slot;
        keys = a.keys ? (int)a.keys[r] : a.rows[r].pos + 1;
    } else {
        slot = r;
        keys = (int)a.keys[r];
    }
    keys = keys < 1 ? 1 : (keys > a.ctx_cap ? a.ctx_cap : keys);  // never read past the cache
    if (valid && lane < hd / 4) s_q[wave][lane] = ((const int *)(a.q + (size_t)r * a.ldq + h * hd))[lane];
    __syncthreads();
    if (!valid) return;
    const int *q4 = s_q[wave];
    const size_t base = ((size_t)slot * a.n_head + h) * a.ctx_cap * hd;
    const int8_t *K = a.kc + base, *V = a.vc + base;
    const int last = a.exp_len - 1;

    // pass 1: M = max score
    int64_t mx = INT64_MIN;
    for (int j = lane; j < keys; j += 64) {
        const int64_t s = clamp64(rescale_small(dot_key(q4, K + (size_t)j * hd, hd), a.score_m,
                                                a.score_s), -SCORE_LIMIT, SCORE_LIMIT);
        mx = s > mx ? s : mx;
    }
    mx = wave_max64(mx);
    // pass 2: S = sum e_j
    int64_t sum = 0;
    for (int j = lane; j < keys; j += 64) {
        const int64_t s = clamp64(rescale_small(dot_key(q4, K + (size_t)j * hd, hd), a.score_m,
                                                a.score_s), -SCORE_LIMIT, SCORE_LIMIT);
        const int64_t dd = mx - s;
        sum += a.exp_table[dd < last ? dd : last];
    }
    sum = wave_sum64(sum);
    // pass 3: p_j and the weighted sum of the values (c = lane + 64 t)
    int64_t acc[4] = {0, 0, 0, 0};
    for (int j0 = 0; j0 < keys; j0 += 64) {
        const int j = j0 + lane;
        uint64_t p = 0;
        if (j < keys) {
            const int64_t s = clamp64(rescale_small(dot_key(q4, K + (size_t)j * hd, hd), a.score_m,
                                                    a.score_s), -SCORE_LIMIT, SCORE_LIMIT);
            const int64_t dd = mx - s;
            const uint64_t e = (uint64_t)a.exp_table[dd < last ? dd : last];
            p = (e << a.softmax_p) / (uint64_t)sum;
        }
        const int cnt = keys - j0 < 64 ? keys - j0 : 64;
        for (int jj = 0; jj < cnt; jj++) {
            const int64_t pj = (int64_t)__shfl(p, jj, 64);
            const int8_t *v = V + (size_t)(j0 + jj) * hd;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int c = lane + 64 * t;
                if (c < hd) acc[t] += pj * (int64_t)v[c];
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int c = lane + 64 * t;
        if (c < hd)
            a.out[(size_t)r * a.ldo + h * hd + c] =
                (int8_t)clamp128(rescale_full(acc[t], a.out_m, a.out_s), -127, 127);
    }
}

hipError_t launch_attend(const AttnArgs &a, int n_rows, hipStream_t stream) {
    const int tasks = n_rows * a.n_head;
    if (tasks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_attend, dim3((tasks + 3) / 4), dim3(256), 0, stream, a, tasks);
    return hipGetLastError();
}

// =============================================================================================
// Prefill attention on MFMA (head_dim 64). One workgroup = one group of <= 64 rows x one head;
// wave w owns rows 16w .. 16w + 15. Three passes over the keys in blocks of 64, recomputing
// S = Q K^T with v_mfma_i32_16x16x64_i8 (exact i32): (1) the row max of the scores, (2) the sum
// of the table entries, (3) p = floor(e 2^P / S) and sum_j p_j v_j. The PV product splits p into
// four balanced signed base-256 digits (crates/hardshell/src/gpt2/attention.rs:36-46), so it is
// four exact i8 MFMA products: |sum_j d_j v_j| <= 2^16 * 128 * 127 < 2^31.
// =============================================================================================

constexpr int AT_ST = 80;  // LDS row stride in bytes (64 + 16)

__global__ __launch_bounds__(256) void k_attend_mfma(AttnArgs a, const AttnGroup *groups) {
    __shared__ __attribute__((aligned(16))) int8_t sQ[64 * AT_ST];
    __shared__ __attribute__((aligned(16))) int8_t sK[64 * AT_ST];
    __shared__ __attribute__((aligned(16))) int8_t sVt[64 * AT_ST];
    __shared__ __attribute__((aligned(16))) int8_t sP[4][64 * AT_ST];
    const AttnGroup G = groups[blockIdx.x];
    const int h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int nk = G.pos0 + G.count;  // keys 0 .. nk - 1, never past the cache
    nk = nk > a.ctx_cap ? a.ctx_cap : nk;
    const size_t base = ((size_t)G.slot * a.n_head + h) * a.ctx_cap * 64;
    const int last = a.exp_len - 1;
    {
        const int r = tid >> 2, c = (tid & 3) * 16;
        v4i v = {0, 0, 0, 0};
        if (r < G.count) v = *(const v4i *)(a.q + (size_t)(G.first + r) * a.ldq + h * 64 + c);
        *(v4i *)&sQ[r * AT_ST + c] = v;
    }
    __syncthreads();
    const v4i qf = *(const v4i *)&sQ[(16 * w + (lane & 15)) * AT_ST + (lane >> 4) * 16];
    // this lane's rows (e = 0..3) and their positions
    int row[4], posr[4];
    bool valid[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        row[e] = 16 * w + 4 * (lane >> 4) + e;
        valid[e] = row[e] < G.count;
        posr[e] = G.pos0 + row[e];
    }
    auto load_k = [&](int kb) {
        const int key = kb * 64 + (tid >> 2), c = (tid & 3) * 16;
        v4i v = {0, 0, 0, 0};
        if (key < nk) v = *(const v4i *)(a.kc + base + (size_t)key * 64 + c);
        *(v4i *)&sK[(tid >> 2) * AT_ST + c] = v;
    };
    auto load_vt = [&](int kb) {
        const int kl = tid >> 2, key = kb * 64 + kl, c = (tid & 3) * 16;
        v4i v = {0, 0, 0, 0};
        if (key < nk) v = *(const v4i *)(a.vc + base + (size_t)key * 64 + c);
        const int8_t *b = (const int8_t *)&v;
#pragma unroll
        for (int i = 0; i < 16; i++) sVt[(c + i) * AT_ST + kl] = b[i];
    };
    auto qk = [&](v4i s[4]) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const v4i kf = *(const v4i *)&sK[(t * 16 + (lane & 15)) * AT_ST + (lane >> 4) * 16];
            s[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qf, kf, v4i{0, 0, 0, 0}, 0, 0, 0);
        }
    };
    auto score = [&](int32_t dot) {
        return clamp64(rescale_small(dot, a.score_m, a.score_s), -SCORE_LIMIT, SCORE_LIMIT);
    };
    const int nkb = (nk + 63) / 64;
    // pass 1: the row max. The score clamp(rescale(dot)) is monotone in the dot (its direction
    // is the sign of score_m), so the largest score is the score of the largest or of the
    // smallest dot.
    int32_t dmax[4] = {INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
    int32_t dmin[4] = {INT32_MAX, INT32_MAX, INT32_MAX, INT32_MAX};
    for (int kb = 0; kb < nkb; kb++) {
        load_k(kb);
        __syncthreads();
        v4i s[4];
        qk(s);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int key = kb * 64 + t * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (key <= posr[e]) {
                    dmax[e] = s[t][e] > dmax[e] ? s[t][e] : dmax[e];
                    dmin[e] = s[t][e] < dmin[e] ? s[t][e] : dmin[e];
                }
        }
        __syncthreads();
    }
    int64_t mx[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const int32_t u = __shfl_xor(dmax[e], o, 64), v = __shfl_xor(dmin[e], o, 64);
            dmax[e] = u > dmax[e] ? u : dmax[e];
            dmin[e] = v < dmin[e] ? v : dmin[e];
        }
        const int64_t a0 = score(dmax[e]), a1 = score(dmin[e]);
        mx[e] = a0 > a1 ? a0 : a1;  // rows past the group's count: unused
    }
    int64_t sum[4] = {0, 0, 0, 0};
    for (int kb = 0; kb < nkb; kb++) {  // pass 2: the sum of the table entries
        load_k(kb);
        __syncthreads();
        v4i s[4];
        qk(s);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int key = kb * 64 + t * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (valid[e] && key <= posr[e]) {
                    const int64_t dd = mx[e] - score(s[t][e]);
                    sum[e] += a.exp_table[dd < last ? dd : last];
                }
        }
        __syncthreads();
    }
    uint64_t frac[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sum[e] += __shfl_xor(sum[e], o, 64);
        // floor(2^64 / S) for S >= 2; S = 1 divides exactly
        frac[e] = sum[e] >= 2 ? div_2p64((uint64_t)sum[e]) : 0;
    }
    v4i acc[4][4];  // [digit plane][channel tile]
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[k][c] = v4i{0, 0, 0, 0};
    for (int kb = 0; kb < nkb; kb++) {  // pass 3: p and the digit-plane PV products
        load_k(kb);
        load_vt(kb);
        __syncthreads();
        v4i s[4];
        qk(s);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int key = kb * 64 + t * 16 + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int64_t p = 0;
                if (valid[e] && key <= posr[e]) {
                    const int64_t dd = mx[e] - score(s[t][e]);
                    const uint64_t num = (uint64_t)a.exp_table[dd < last ? dd : last] << a.softmax_p;
                    const uint64_t S = (uint64_t)sum[e];
                    uint64_t q = num;
                    if (S >= 2) {
                        q = __umul64hi(num, frac[e]);  // q <= floor(num / S) <= q + 1
                        if (num - q * S >= S) q++;
                    }
                    p = (int64_t)q;
                }
                int64_t rest = p;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int64_t dg = ((rest + 128) & 255) - 128;
                    sP[k][row[e] * AT_ST + t * 16 + (lane & 15)] = (int8_t)dg;
                    rest = (rest - dg) >> 8;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const v4i af = *(const v4i *)&sP[k][(16 * w + (lane & 15)) * AT_ST + (lane >> 4) * 16];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const v4i bf = *(const v4i *)&sVt[(c * 16 + (lane & 15)) * AT_ST + (lane >> 4) * 16];
                acc[k][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, acc[k][c], 0, 0, 0);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (!valid[e]) continue;
            const int64_t o = (int64_t)acc[0][c][e] + ((int64_t)acc[1][c][e] << 8) +
                              ((int64_t)acc[2][c][e] << 16) + ((int64_t)acc[3][c][e] << 24);
            a.out[(size_t)(G.first + row[e]) * a.ldo + h * 64 + c * 16 + (lane & 15)] =
                (int8_t)clamp128(rescale_full(o, a.out_m, a.out_s), -127, 127);
        }
}

hipError_t launch_attend_groups(const AttnArgs &a, const AttnGroup *groups, int n_groups,
                                hipStream_t stream) {
    if (n_groups <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_attend_mfma, dim3(n_groups, a.n_head), dim3(256), 0, stream, a, groups);
    return hipGetLastError();
}

// =============================================================================================
// The coder op: logits -> weights (logits.rs:62-72) -> the interval of FreqTable::from_weights
// (crates/taco-coder/src/freq.rs:103-149) for an Encode(token) or Decode(target) query.
// One workgroup per row; thread t owns the symbols [t * chunk, (t + 1) * chunk).
// f_i = 1 + floor(w_i * spare / W) with an exact quotient: a 64-bit reciprocal of W and one
// correction step (W >= 2^32), or a plain u64 division (W < 2^32).
// =============================================================================================


__global__ __launch_bounds__(256) void k_coder(CoderArgs a) {
    __shared__ int64_t s_i64[256];
    __shared__ uint64_t s_u64[256];
    __shared__ uint32_t s_idx[256];
    __shared__ uint64_t s_W, s_frac;
    __shared__ uint32_t s_largest;
    const int row = blockIdx.x, tid = threadIdx.x;
    const int V = a.vocab;
    const int chunk = (V + 255) / 256;
    const int j0 = tid * chunk, j1 = min(V, j0 + chunk);
    const int64_t *l = a.logits + (size_t)row * a.ld;
    const int last = a.table_len - 1;

    // pass 1: the largest logit
    int64_t mx = INT64_MIN;
    for (int j = j0; j < j1; j++) mx = l[j] > mx ? l[j] : mx;
    s_i64[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s_i64[tid] = s_i64[tid + o] > s_i64[tid] ? s_i64[tid + o] : s_i64[tid];
        __syncthreads();
    }
    const int64_t M = s_i64[0];
    __syncthreads();
    // pass 2: W = sum w and the largest weight (the lowest id on a tie)
    uint64_t W = 0, best = 0;
    uint32_t bidx = 0xFFFFFFFFu;
    for (int j = j0; j < j1; j++) {
        const int64_t dd = M - l[j];
        const uint64_t w = a.table[dd < last ? dd : last];
        if (a.weights) a.weights[(size_t)row * V + j] = w;
        W += w;
        if (bidx == 0xFFFFFFFFu || w > best) {
            best = w;
            bidx = j;
        }
    }
    s_u64[tid] = W;
    s_i64[tid] = (int64_t)best;
    s_idx[tid] = bidx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) {
            s_u64[tid] += s_u64[tid + o];
            const uint64_t b0 = (uint64_t)s_i64[tid], b1 = (uint64_t)s_i64[tid + o];
            const uint32_t i0 = s_idx[tid], i1 = s_idx[tid + o];
            // the larger weight wins; on a tie the lower index (a strided tree does not keep
            // the lower slot on the lower indices, so compare them)
            if (i0 == 0xFFFFFFFFu || (i1 != 0xFFFFFFFFu && (b1 > b0 || (b1 == b0 && i1 < i0)))) {
                s_i64[tid] = (int64_t)b1;
                s_idx[tid] = i1;
            }
        }
        __syncthreads();
    }
    if (tid == 0) {
        uint64_t Wt = s_u64[0];
        uint32_t largest = s_idx[0];
        if (Wt == 0) {  // every weight 0: every weight is 1 (freq.rs:119-123)
            Wt = (uint64_t)V;
            largest = 0;
        }
        const uint64_t total = (uint64_t)1 << a.bits;
        const uint64_t spare = total - (uint64_t)V;
        s_W = Wt;
        s_largest = largest;
        s_frac = Wt >= ((uint64_t)1 << 32) ? coder_frac(spare, Wt) : 0;
    }
    __syncthreads();
    const uint64_t Wt = s_W, frac = s_frac;
    const bool all_zero = s_u64[0] == 0;
    const uint32_t largest = s_largest;
    const uint64_t total = (uint64_t)1 << a.bits, spare = total - (uint64_t)V;
    const uint32_t kind = a.queries ? a.queries[2 * row] : 0;
    const uint32_t value = a.queries ? a.queries[2 * row + 1] : 0;
    // pass 3: the sum of f over the chunk, and over the symbols below the encode token
    uint64_t F = 0, Fbelow = 0, ftok = 0;
    for (int j = j0; j < j1; j++) {
        const int64_t dd = M - l[j];
        const uint64_t w = all_zero ? 1 : a.table[dd < last ? dd : last];
        const uint64_t f = 1 + quotient(w, spare, Wt, frac);
        F += f;
        if (kind == 0 && (uint32_t)j < value) Fbelow += f;
        if (kind == 0 && (uint32_t)j == value) ftok = f;
    }
    __syncthreads();
    s_u64[tid] = F;
    __syncthreads();
    if (tid == 0) {  // exclusive scan of the chunk sums, in order
        uint64_t run = 0;
        for (int t = 0; t < 256; t++) {
            const uint64_t v = s_u64[t];
            s_u64[t] = run;
            run += v;
        }
        s_W = run;  // sum of all f
    }
    __syncthreads();
    const uint64_t base = s_u64[tid];
    const uint64_t Q = s_W;
    const uint64_t rem = total - Q;
    uint64_t *out = a.intervals ? a.intervals + 3 * (size_t)row : nullptr;
    if (!out) return;
    if (kind == 0) {
        // start = sum_{j < tok} f_j (+ rem if the largest is below tok); the owner writes it
        const uint32_t tok = value;
        if ((int)tok >= j0 && (int)tok < j1) {
            const uint64_t start = base + Fbelow + (largest < tok ? rem : 0);
            const uint64_t freq = ftok + (largest == tok ? rem : 0);
            out[0] = tok;
            out[1] = start;
            out[2] = freq;
        }
        return;
    }
    // Decode: the largest i with start_i <= target; starts increase with i.
    const uint64_t target = value;
    uint64_t run = base;
    int cand = -1;
    uint64_t cstart = 0, cfreq = 0;
    for (int j = j0; j < j1; j++) {
        const int64_t dd = M - l[j];
        const uint64_t w = all_zero ? 1 : a.table[dd < last ? dd : last];
        const uint64_t f = 1 + quotient(w, spare, Wt, frac);
        const uint64_t start = run + ((uint32_t)j > largest ? rem : 0);
        run += f;
        if (start <= target) {
            cand = j;
            cstart = start;
            cfreq = f + ((uint32_t)j == largest ? rem : 0);
        } else {
            break;
        }
    }
    __syncthreads();
    s_i64[tid] = cand;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s_i64[tid] = s_i64[tid + o] > s_i64[tid] ? s_i64[tid + o] : s_i64[tid];
        __syncthreads();
    }
    if (cand >= 0 && cand == s_i64[0]) {
        out[0] = (uint64_t)cand;
        out[1] = cstart;
        out[2] = cfreq;
    }
}

hipError_t launch_coder(const CoderArgs &a, int n_rows, hipStream_t stream) {
    if (n_rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_coder, dim3(n_rows), dim3(256), 0, stream, a);
    return hipGetLastError();
}


// =============================================================================================
// The coder op over compact logits. One workgroup per row, one coalesced pass over the row: the
// table index d_j = min(M - l_j, len - 1) of every symbol goes into a histogram in LDS (and a
// second one for the symbols below an Encode token), so the quotients floor(table[d] * spare /
// W) are computed once per table entry, not once per symbol:
//   W = sum_d cnt[d] table[d];  sum f = V + sum_d cnt[d] q[d];  sum_{j<tok} f = tok + sum_d
//   cnt_lo[d] q[d].  largest = the first symbol whose weight is table[0] (d <= d0).
// A Decode query needs the starts in symbol order: an ordered block scan over the row.
// =============================================================================================

__device__ __forceinline__ int64_t block_max64(int64_t v, int64_t *s, int tid) {
    s[tid] = v;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s[tid] = s[tid + o] > s[tid] ? s[tid + o] : s[tid];
        __syncthreads();
    }
    v = s[0];
    __syncthreads();
    return v;
}

__device__ __forceinline__ uint64_t block_sum64(uint64_t v, uint64_t *s, int tid) {
    s[tid] = v;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) s[tid] += s[tid + o];
        __syncthreads();
    }
    v = s[0];
    __syncthreads();
    return v;
}

// Reductions over a 256-thread block through wave shuffles and one LDS slot per wave.
__device__ __forceinline__ int64_t block_max64w(int64_t v, int64_t *s4, int tid) {
    v = wave_max64(v);
    if ((tid & 63) == 0) s4[tid >> 6] = v;
    __syncthreads();
    int64_t r = s4[0];
#pragma unroll
    for (int w = 1; w < 4; w++) r = s4[w] > r ? s4[w] : r;
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint64_t block_sum64w(uint64_t v, uint64_t *s4, int tid) {
    v = (uint64_t)wave_sum64((int64_t)v);
    if ((tid & 63) == 0) s4[tid >> 6] = v;
    __syncthreads();
    const uint64_t r = s4[0] + s4[1] + s4[2] + s4[3];
    __syncthreads();
    return r;
}

// One row per workgroup. The histogram counts the symbols of each table index d < zcut (the
// bins with a nonzero weight); with V < 2^16 the count and the count below the Encode token
// share one u32 (low and high half), else they are two arrays. Symbols with d >= zcut have
// weight 0, f = 1 and no share of the spare, and need no count.
__global__ __launch_bounds__(256) void k_coder_compact(CompactCoderArgs a) {
    extern __shared__ uint32_t hist[];
    __shared__ int64_t s_i[256];
    __shared__ uint64_t s_u[256];
    __shared__ uint64_t s_frac;
    const int row = blockIdx.x, tid = threadIdx.x;
    const int V = a.vocab, len = a.table_len, last = len - 1;
    const int zc = a.zcut;
    const bool packed = V < 65536;
    const uint16_t *d16 = a.d16 + (size_t)row * a.ld16;
    const int64_t *tm = a.tmax + (size_t)row * a.ntiles;
    const uint32_t kind = a.queries ? a.queries[2 * row] : 0;
    const uint32_t value = a.queries ? a.queries[2 * row + 1] : 0;
    const uint32_t tok = kind == 0 ? value : 0;  // Encode token (0: no symbol below)

    int64_t mx = INT64_MIN;
    for (int t = tid; t < a.ntiles; t += 256) mx = tm[t] > mx ? tm[t] : mx;
    const int64_t M = block_max64w(mx, s_i, tid);
    for (int d = tid; d < (packed ? zc : 2 * zc); d += 256) hist[d] = 0;
    if (a.weights) {  // the weights themselves (run_weights)
        for (int j = tid; j < V; j += 256) {
            const int64_t dd = M - tm[j >> 6] + d16[j];
            a.weights[(size_t)row * V + j] = a.table[dd < last ? dd : last];
        }
    }
    __syncthreads();

    // One pass: 8 consecutive symbols per thread and step (one 16-byte load; the 8 share a
    // 64-column tile). A group whose tile max is zcut or more below M has only weight-0 symbols.
    int64_t first = INT64_MAX;  // the first symbol with weight table[0] (d <= d0 < zcut)
    for (int g0 = tid * 8; g0 < V; g0 += 256 * 8) {
        const int64_t base64 = M - tm[g0 >> 6];
        if (base64 >= zc) continue;
        const uint4 raw = *(const uint4 *)(d16 + g0);
        const uint16_t *dv = (const uint16_t *)&raw;
        const int base = (int)base64;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = g0 + q;
            const int dd = base + (int)dv[q];
            if (j < V && dd < zc) {  // then dd <= last: d = dd
                if (packed) {
                    atomicAdd(&hist[dd], (uint32_t)j < tok ? 0x10001u : 1u);
                } else {
                    atomicAdd(&hist[dd], 1u);
                    if ((uint32_t)j < tok) atomicAdd(&hist[zc + dd], 1u);
                }
                if (dd <= a.d0 && j < first) first = j;
            }
        }
    }
    __syncthreads();
    const int64_t largest = -block_max64w(-first, s_i, tid);

    uint64_t W = 0;
    for (int d = tid; d < zc; d += 256) {
        const uint32_t c = packed ? (hist[d] & 0xffffu) : hist[d];
        W += (uint64_t)c * a.table[d];
    }
    W = block_sum64w(W, s_u, tid);
    const uint64_t total = (uint64_t)1 << a.bits, spare = total - (uint64_t)V;
    if (tid == 0) s_frac = W >= ((uint64_t)1 << 32) ? coder_frac(spare, W) : 0;
    __syncthreads();
    const uint64_t frac = s_frac;
    uint64_t S = 0, Slo = 0;
    for (int d = tid; d < zc; d += 256) {
        const uint32_t h = hist[d];
        const uint32_t c = packed ? (h & 0xffffu) : h, clo = packed ? (h >> 16) : hist[zc + d];
        if (!c) continue;
        const uint64_t q = quotient(a.table[d], spare, W, frac);
        S += (uint64_t)c * q;
        Slo += (uint64_t)clo * q;
    }
    S = block_sum64w(S, s_u, tid);
    Slo = block_sum64w(Slo, s_u + 8, tid);
    const uint64_t rem = total - ((uint64_t)V + S);
    uint64_t *out = a.intervals ? a.intervals + 3 * (size_t)row : nullptr;
    if (!out) return;
    if (kind == 0) {
        if (tid == 0) {
            const int64_t dt = M - tm[tok >> 6] + d16[tok];
            const uint64_t f = 1 + quotient(a.table[dt < last ? dt : last], spare, W, frac);
            out[0] = tok;
            out[1] = (uint64_t)tok + Slo + ((int64_t)tok > largest ? rem : 0);
            out[2] = f + ((int64_t)tok == largest ? rem : 0);
        }
        return;
    }
    // Decode: the largest i with start_i <= target, in symbol order, 2048 symbols per step.
    const uint64_t target = value;
    uint64_t run = 0;
    int64_t cand = -1;
    uint64_t cstart = 0, cfreq = 0;
    for (int b = 0; b < V; b += 2048) {
        uint64_t f[8];
        uint64_t local = 0;
        const int j0 = b + tid * 8;
        if (j0 < V) {
            const uint4 raw = *(const uint4 *)(d16 + j0);
            const uint16_t *dv = (const uint16_t *)&raw;
            const int64_t base = M - tm[j0 >> 6];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int j = j0 + q;
                f[q] = 0;
                if (j < V) {
                    const int64_t dd = base + dv[q];
                    const int d = (int)(dd < last ? dd : last);
                    f[q] = 1 + quotient(a.table[d], spare, W, frac) + (j == largest ? rem : 0);
                    local += f[q];
                }
            }
        }
        s_u[tid] = local;
        __syncthreads();
        if (tid == 0) {  // exclusive scan of the 256 partial sums, in order
            uint64_t acc = run;
            for (int t = 0; t < 256; t++) {
                const uint64_t v = s_u[t];
                s_u[t] = acc;
                acc += v;
            }
            s_i[0] = (int64_t)acc;
        }
        __syncthreads();
        uint64_t start = s_u[tid];
        const uint64_t next_run = (uint64_t)s_i[0];
        __syncthreads();
        if (j0 < V) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int j = j0 + q;
                if (j >= V) break;
                if (start <= target) {
                    cand = j;
                    cstart = start;
                    cfreq = f[q];
                }
                start += f[q];
            }
        }
        run = next_run;
    }
    const int64_t best = block_max64(cand, s_i, tid);
    if (cand >= 0 && cand == best) {
        out[0] = (uint64_t)cand;
        out[1] = cstart;
        out[2] = cfreq;
    }
}

hipError_t launch_coder_compact(const CompactCoderArgs &a, int n_rows, hipStream_t stream) {
    if (n_rows <= 0) return hipSuccess;
    const size_t lds = (a.vocab < 65536 ? 1 : 2) * sizeof(uint32_t) * (size_t)a.zcut;
    static size_t allowed = 0;  // raise the dynamic LDS limit once per size
    if (lds > allowed) {
        hipError_t e = hipFuncSetAttribute((const void *)k_coder_compact,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        allowed = lds;
    }
    hipLaunchKernelGGL(k_coder_compact, dim3(n_rows), dim3(256), lds, stream, a);
    return hipGetLastError();
}

}  // namespace hs
