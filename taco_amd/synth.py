"""Seeded synthetic workloads for the fold benchmark: GPT-2-shape integer models in .hsm layout
with uniform int8 weights, and Zipf(1.1) token streams.

The recipe: int8 weights uniform in [-127, 127] as (splitmix64 % 255) - 127 (the generator of
crates/hardshell/tests/common/mod.rs:16-50); per-row rescale multipliers uniform in
[2^30, 2^31) (ADR 0004 section 6); shifts s = 30 + round(log2(sigma_in / sigma_target)) with
targets 40 for i8 activations, 8000 for the GELU input, 768 for scores and logits and 2^14 for
the residual; LayerNorm K = 48, J = 8, eps = 2^43, gamma uniform in [2^13, 2^15), beta in
[-16, 16]; exponent tables round(2^30 exp(-i/256)) and round(2^40 exp(-i/256)) with 8,192
entries; a 65,536-entry GELU table; a vocabulary of fixed-width 4-byte tokens (id i is the
little-endian u32 of i; the last id is <|endoftext|>). Every float step uses +, -, *, / only
(no libm), so the model bytes are the same on every machine; the Zipf weights use the C
library's pow.
"""

from __future__ import annotations

import hashlib
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from fractions import Fraction
from typing import List

import numpy as np

from .hsm_writer import HsmWriter

MASK = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


@dataclass(frozen=True)
class Dims:
    n_layer: int
    n_head: int
    d_model: int
    d_ff: int
    vocab: int = 50_257
    n_ctx: int = 1024


GPT2_SMALL = Dims(12, 12, 768, 3072)
GPT2_MEDIUM = Dims(24, 16, 1024, 4096)
GPT2_XL = Dims(48, 25, 1600, 6400)


def splitmix_block(state0: int, start: int, n: int) -> np.ndarray:
    """Outputs start .. start+n of the splitmix64 stream whose state is `state0` before the
    first call (output i uses the state state0 + (i + 1) * GAMMA)."""
    z = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z *= np.uint64(GAMMA)
        z += np.uint64(state0 & MASK)
        z ^= z >> np.uint64(30)
        z *= np.uint64(0xBF58476D1CE4E5B9)
        z ^= z >> np.uint64(27)
        z *= np.uint64(0x94D049BB133111EB)
        z ^= z >> np.uint64(31)
    return z


class Stream:
    """A splitmix64 stream consumed in order, generated in vectorised blocks."""

    def __init__(self, seed: int):
        self.state0 = seed & MASK
        self.n = 0

    def take(self, n: int) -> np.ndarray:
        out = splitmix_block(self.state0, self.n, n)
        self.n += n
        return out

    def next(self) -> int:
        return int(self.take(1)[0])


_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        _POOL = ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1))
    return _POOL


def _uniform_i8(s: Stream, shape) -> np.ndarray:
    """(next_u64 % 255) - 127 for each element, in stream order. Output i depends only on its
    stream index, so chunks are generated on a thread pool (numpy releases the GIL)."""
    n = int(np.prod(shape))
    out = np.empty(n, np.int8)
    step = 1 << 22
    base = s.n

    def fill(i):
        z = splitmix_block(s.state0, base + i, min(step, n - i))
        z %= np.uint64(255)
        out[i:i + len(z)] = z.astype(np.int16) - 127

    list(_pool().map(fill, range(0, n, step)))
    s.n += n
    return out.reshape(shape)


def _uniform_int(s: Stream, n: int, lo: int, hi: int, dtype) -> np.ndarray:
    """Uniform integers in [lo, hi) (hi - lo < 2^63)."""
    z = s.take(n)
    return (np.int64(lo) + (z % np.uint64(hi - lo)).astype(np.int64)).astype(dtype)


def shift_for(sigma_in_sq: Fraction, target: int) -> int:
    """30 + round(log2(sigma_in / target)), exactly, from sigma_in^2."""
    return 30 + _round_log2_sq(Fraction(sigma_in_sq) / (target * target))


def _round_log2_sq(r: Fraction) -> int:
    """round(log2(sqrt(r))): the k with 2^(2k-1) <= r < 2^(2k+1)."""
    k = 0
    while r >= Fraction(2) ** (2 * k + 1):
        k += 1
    while r < Fraction(2) ** (2 * k - 1):
        k -= 1
    return k


LN2 = 0.6931471805599453


def det_exp(x: float) -> float:
    """exp with basic operations only (range reduction by ln 2, Taylor series): the form of
    crates/hardshell/tests/common/mod.rs:61-78."""
    if x < -700.0:
        return 0.0
    k = round(x / LN2)
    r = x - k * LN2
    term, total = 1.0, 1.0
    for i in range(1, 22):
        term = term * r / float(i)
        total += term
    return total * (2.0 ** k)


def gelu(x: float) -> float:
    c = 0.7978845608028654
    u = c * (x + 0.044715 * x * x * x)
    if u > 20.0:
        t = 1.0
    elif u < -20.0:
        t = -1.0
    else:
        e = det_exp(2.0 * u)
        t = (e - 1.0) / (e + 1.0)
    return 0.5 * x * (1.0 + t)


def _rust_round(v: float) -> int:
    """f64::round: half away from zero."""
    f = int(v)
    r = v - f
    if r >= 0.5:
        f += 1
    elif r <= -0.5:
        f -= 1
    return f


def gelu_table_wide() -> np.ndarray:
    # input unit 1/4000, output unit 1/10240 (i16 entries)
    out = np.empty(65536, np.int16)
    for i, q in enumerate(range(-32768, 32768)):
        out[i] = max(-32767, min(32767, _rust_round(gelu(q / 4000.0) * 10240.0)))
    return out


def gelu_table() -> np.ndarray:
    # input unit 1/4000 (GELU input sigma 8000 is 2.0), output unit 1/40
    out = np.empty(65536, np.int8)
    for i, q in enumerate(range(-32768, 32768)):
        out[i] = max(-127, min(127, _rust_round(gelu(q / 4000.0) * 40.0)))
    return out


def exp_tables(length: int = 8192):
    a = np.array([_rust_round(2.0 ** 30 * det_exp(-i / 256.0)) for i in range(length)], np.int32)
    l = np.array([_rust_round(2.0 ** 40 * det_exp(-i / 256.0)) for i in range(length)], np.uint64)
    return a, l


def vocabulary(vocab: int) -> List[bytes]:
    return [int(i).to_bytes(4, "little") for i in range(vocab - 1)] + [b"<|endoftext|>"]


SIGMA_W_SQ = Fraction(255 * 255 - 1, 12)  # uniform [-127, 127]: variance 5418.67
SIGMA_ACT_SQ = Fraction(1600 * 1600)       # i8 model activations times weights


def build_model(dims: Dims, seed: int = 0x7AC0_5EED, wide: bool = False, table_len: int = 8192,
                score_target: int = 768, beta_max: int = 16, residual_target: int = 1 << 14,
                score_mult: int = 0) -> bytes:
    """The synthetic model. wide=True makes a model-file version 2 model: an i16 GELU table
    (output unit 1/10240), a 16-bit ln_f (target 10240) and ln_beta_frac = 8 (beta in units of
    2^-8, uniform in [-4096, 4096]); the shifts that read those activations are 8 larger.
    table_len sets the length of both exponent tables; score_target the typical attention score
    (larger targets give smaller score shifts); beta_max the LayerNorm beta range [-beta_max,
    beta_max] in output units; residual_target the typical residual update (larger targets give
    the residual products shifts below 31, the general rescale form); score_mult, when nonzero,
    replaces every layer's attention score multiplier (after drawing it, so the rest of the model
    stays the same), e.g. a negative one."""
    d, f, V, C, L, H = dims.d_model, dims.d_ff, dims.vocab, dims.n_ctx, dims.n_layer, dims.n_head
    hd = d // H
    s = Stream(seed)
    w = HsmWriter(n_layer=L, n_head=H, d_model=d, d_ff=f, vocab_size=V, n_ctx=C, eot_token=V - 1,
                  ln_k=48, ln_j=8, ln_eps=1 << 43, softmax_p=30)
    w.set_vocabulary(vocabulary(V))
    frac = 8 if wide else 0
    if wide:
        w.ln_f_bits = 16
        w.ln_beta_frac = frac

    def mult(n):
        return _uniform_int(s, n, 1 << 30, 1 << 31, np.int64).astype(np.int32)

    def bias(n):
        return _uniform_int(s, n, -(1 << 16), (1 << 16) + 1, np.int32)

    # gamma uniform in [2^13, 2^15): E[gamma^2] = (a^2 + ab + b^2) / 3
    a_, b_ = 1 << 13, 1 << 15
    gamma_sq = Fraction(a_ * a_ + a_ * b_ + b_ * b_, 3)

    def layernorm(prefix, target=40):
        w.add_tensor(prefix + ".g", _uniform_int(s, d, 1 << 13, 1 << 15, np.int16))
        w.add_tensor(prefix + ".b", _uniform_int(s, d, -(beta_max << frac), (beta_max << frac) + 1, np.int32))
        w.add_tensor(prefix + ".rescale", mult(1), shift_for(Fraction(2) ** 80 * gamma_sq, target))

    def linear(prefix, rows, cols, target, in_scale=1):
        w.add_tensor(prefix + ".w", _uniform_i8(s, (rows, cols)))
        w.add_tensor(prefix + ".b", bias(rows))
        w.add_tensor(prefix + ".rescale", mult(rows), shift_for(SIGMA_ACT_SQ * cols * in_scale ** 2, target))

    w.add_tensor("wte", _uniform_i8(s, (V, d)))
    w.add_tensor("wte.rescale_embed", mult(V), shift_for(SIGMA_W_SQ, 1 << 14))
    w.add_tensor("wte.rescale_logits", mult(V), shift_for(SIGMA_ACT_SQ * d * (65536 if wide else 1), 768))
    w.add_tensor("wpe", _uniform_i8(s, (C, d)))
    w.add_tensor("wpe.rescale", mult(C), shift_for(SIGMA_W_SQ, 1 << 14))
    table = gelu_table_wide() if wide else gelu_table()
    for l in range(L):
        p = f"h.{l}"
        layernorm(p + ".ln_1")
        linear(p + ".attn.c_attn", 3 * d, d, 40)
        sm = mult(1)
        if score_mult:
            sm = np.array([score_mult], np.int32)
        w.add_tensor(p + ".attn.score.rescale", sm, shift_for(SIGMA_ACT_SQ * hd, score_target))
        w.add_tensor(p + ".attn.out.rescale", mult(1), shift_for(Fraction(2) ** 60 * 1600, 40))
        linear(p + ".attn.c_proj", d, d, residual_target)
        layernorm(p + ".ln_2")
        linear(p + ".mlp.c_fc", f, d, 8000)
        w.add_tensor(p + ".mlp.gelu", table)
        linear(p + ".mlp.c_proj", d, f, residual_target, 256 if wide else 1)
    layernorm("ln_f", 10240 if wide else 40)
    ae, le = exp_tables(table_len)
    w.add_tensor("attn_exp", ae)
    w.add_tensor("logits_exp", le)
    return w.finish()


def zipf_tokens(n: int, vocab: int = 50_257, s_exp: float = 1.1, seed: int = 0x21FF) -> np.ndarray:
    """n Zipf(s) token ids over the vocab - 1 ids that are not <|endoftext|>: rank r (1-based)
    has probability proportional to r^-s, from a u64 CDF table and next_u64 % total; a seeded
    Fisher-Yates permutation maps rank to id."""
    k = vocab - 1
    # r ** -s with the C library's pow (correctly rounded in the image's glibc), one by one
    wts = np.array([int(2.0 ** 52 * (float(r) ** -s_exp)) for r in range(1, k + 1)], np.uint64)
    cdf = np.cumsum(wts, dtype=np.uint64)
    total = int(cdf[-1])
    st = Stream(seed)
    perm = np.arange(k, dtype=np.uint32)
    z = st.take(k - 1)
    for idx, i in enumerate(range(k - 1, 0, -1)):
        j = int(z[idx] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    x = st.take(n) % np.uint64(total)
    ranks = np.searchsorted(cdf, x, side="right")
    return perm[ranks].astype(np.uint32)


def sha256_tokens(t: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(t, dtype="<u4").tobytes()).hexdigest()
