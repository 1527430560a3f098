"""ctypes wrapper of the oracle (oracle/liboracle.so). Test infrastructure only: the tests, the
smoke check and the CPU-baseline leg of bench.py use it as the checker."""

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle.so is not built: run oracle/build.py")
        L = C.CDLL(path)
        P = C.c_void_p
        u8p, u32p, u64p = C.POINTER(C.c_uint8), C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)
        L.or_model_load.restype = P
        L.or_model_load.argtypes = [P, C.c_size_t]
        L.or_model_free.argtypes = [P]
        L.or_model_dims.argtypes = [P, P]
        L.or_session_new.restype = P
        L.or_session_new.argtypes = [P, C.c_uint32]
        L.or_session_free.argtypes = [P]
        L.or_session_start_block.argtypes = [P, P]
        L.or_session_step.argtypes = [P, C.c_uint32, P]
        L.or_session_position.restype = C.c_uint32
        L.or_session_position.argtypes = [P]
        L.or_session_probe.argtypes = [P, C.c_uint32, P, P, P, P, P]
        L.or_fast_window_intervals.argtypes = [P, P, C.c_size_t, C.c_size_t, P]
        L.or_fast_window_weights.argtypes = [P, P, C.c_size_t, C.c_size_t, P]
        L.or_fold_payloads.argtypes = [P, P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, P,
                                       C.c_size_t, P]
        L.or_matmul_i8.argtypes = [P, C.c_size_t, P, C.c_size_t, C.c_size_t, P]
        L.or_freq_from_weights.argtypes = [P, C.c_size_t, C.c_uint32, P]
        L.or_freq_interval.argtypes = [P, C.c_size_t, C.c_uint32, C.c_uint32, P, P]
        L.or_freq_find.argtypes = [P, C.c_size_t, C.c_uint32, C.c_uint64, P, P, P]
        L.or_encode_script.restype = C.c_size_t
        L.or_encode_script.argtypes = [P, C.c_size_t, P, C.c_size_t]
        L.or_decoder_new.restype = P
        L.or_decoder_new.argtypes = [P, C.c_size_t]
        L.or_decoder_free.argtypes = [P]
        L.or_decoder_target.restype = C.c_uint64
        L.or_decoder_target.argtypes = [P, C.c_uint32]
        L.or_decoder_decode_interval.argtypes = [P, C.c_uint64, C.c_uint64, C.c_uint32]
        L.or_decoder_decode_bit.argtypes = [P, C.c_uint32]
        L.or_encode_block.restype = C.c_size_t
        L.or_encode_block.argtypes = [P, C.c_uint32, P, C.c_size_t, C.c_size_t, P, C.c_size_t]
        L.or_decode_block.restype = C.c_long
        L.or_decode_block.argtypes = [P, C.c_uint32, P, C.c_size_t, P, C.c_size_t]
        L.or_build_model.restype = C.c_size_t
        L.or_build_model.argtypes = [P, C.c_uint64, C.c_size_t, C.c_int, P, C.c_size_t]
        L.or_rescale.argtypes = [C.c_int64, C.c_int32, C.c_uint8, P, P]
        L.or_rescale_wide.argtypes = [C.c_int64, C.c_uint64, C.c_int32, C.c_uint8, P, P]
        L.or_rescale_clamp.restype = C.c_int64
        L.or_rescale_clamp.argtypes = [C.c_int64, C.c_int32, C.c_uint8, C.c_int64, C.c_int64]
        L.or_floor_div.restype = C.c_int64
        L.or_floor_div.argtypes = [C.c_int64, C.c_int64]
        L.or_isqrt_u128.restype = C.c_uint64
        L.or_isqrt_u128.argtypes = [C.c_uint64, C.c_uint64]
        L.or_layernorm.argtypes = [P, C.c_size_t, P, P, C.c_int32, C.c_uint8, C.c_uint8,
                                   C.c_uint8, C.c_uint8, C.c_uint64, C.c_int, P]
        L.or_softmax.argtypes = [P, C.c_size_t, P, C.c_size_t, C.c_uint8, P]
        L.or_logits_to_weights.argtypes = [P, C.c_size_t, P, C.c_size_t, P]
        L.or_linear_act_ref.argtypes = [P, P, P, P, C.c_uint8, C.c_size_t, C.c_size_t, C.c_size_t,
                                         P]
        L.or_attend_decode_ref.argtypes = [P, P, P, P, C.c_size_t, C.c_size_t, C.c_size_t,
                                            C.c_size_t, C.c_int32, C.c_uint8, C.c_int32, C.c_uint8,
                                            P, C.c_size_t, C.c_uint8, P]
        L.or_mix_stats.argtypes = [P, C.c_size_t, C.c_uint32, P]
        L.or_mix_state_new.restype = P
        L.or_mix_state_free.argtypes = [P]
        L.or_mix_state_predict.argtypes = [P, P, P]
        L.or_mix_state_mix_stats.restype = C.c_uint32
        L.or_mix_state_mix_stats.argtypes = [P, C.c_uint64, C.c_uint64, C.c_uint32]
        L.or_mix_state_mix.argtypes = [P, P, C.c_size_t]
        L.or_mix_state_observe.argtypes = [P, C.c_uint32]
        L.or_logistic_tables.argtypes = [P, P]
        L.or_encode_mixed_block.restype = C.c_size_t
        L.or_encode_mixed_block.argtypes = [P, C.c_uint32, P, C.c_size_t, P, C.c_size_t]
        L.or_decode_mixed_block.restype = C.c_long
        L.or_decode_mixed_block.argtypes = [P, C.c_uint32, P, C.c_size_t, P, C.c_size_t]
        L.or_mix_record.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, P, P, P]
        L.or_mix_apply.argtypes = [P, C.c_size_t, C.c_uint32, C.c_uint32]
        _lib = L
    return _lib


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _i128(hi, lo):
    v = (int(hi) << 64) | int(lo)
    return v


def rescale(x, m, s):
    hi, lo = C.c_int64(), C.c_uint64()
    lib().or_rescale(x, m, s, C.byref(hi), C.byref(lo))
    return _i128(hi.value, lo.value)


def rescale_wide(x, m, s):
    x &= (1 << 128) - 1
    xhi = x >> 64
    if xhi >= 1 << 63:
        xhi -= 1 << 64
    hi, lo = C.c_int64(), C.c_uint64()
    lib().or_rescale_wide(xhi, x & ((1 << 64) - 1), m, s, C.byref(hi), C.byref(lo))
    return _i128(hi.value, lo.value)


def build_model(dims, seed, calib_len, wide=False):
    d = np.asarray(dims, dtype=np.uint32)
    n = lib().or_build_model(ptr(d), seed, calib_len, int(wide), None, 0)
    out = np.zeros(n, dtype=np.uint8)
    lib().or_build_model(ptr(d), seed, calib_len, int(wide), ptr(out), n)
    return out.tobytes()


def tiny_dims():
    return (2, 4, 64, 256, 300, 64)


class Model:
    def __init__(self, data: bytes):
        self._buf = np.frombuffer(data, dtype=np.uint8).copy()
        self.h = lib().or_model_load(ptr(self._buf), len(self._buf))
        if not self.h:
            raise ValueError("the oracle could not read the model")
        d = np.zeros(8, dtype=np.uint32)
        lib().or_model_dims(self.h, ptr(d))
        (self.n_layer, self.n_head, self.d_model, self.d_ff, self.vocab, self.n_ctx, self.eot,
         wide) = (int(v) for v in d)
        self.wide = bool(wide)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None


class Session:
    """The reference session (crates/hardshell/src/gpt2/reference.rs)."""

    def __init__(self, model: Model, overlap: int = 0):
        self.model = model
        self.h = lib().or_session_new(model.h, overlap)
        self.w = np.zeros(model.vocab, dtype=np.uint64)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_session_free(self.h)
            self.h = None

    def start_block(self):
        if lib().or_session_start_block(self.h, ptr(self.w)) != 0:
            raise ValueError("start_block refused")
        return self.w.copy()

    def step(self, token):
        if lib().or_session_step(self.h, int(token), ptr(self.w)) != 0:
            raise ValueError("step refused")
        return self.w.copy()

    def position(self):
        return lib().or_session_position(self.h)

    def probe(self, token):
        d = self.model.d_model
        xe = np.zeros(d, np.int32)
        ln1 = np.zeros(d, np.int8)
        qkv = np.zeros(3 * d, np.int8)
        att = np.zeros(d, np.int8)
        xb = np.zeros(d, np.int32)
        if lib().or_session_probe(self.h, int(token), ptr(xe), ptr(ln1), ptr(qkv), ptr(att),
                                  ptr(xb)) != 0:
            raise ValueError("step refused")
        return dict(x_embed=xe, ln1=ln1, qkv=qkv, att=att, x_block0=xb)


def freq_from_weights(w, bits):
    w = np.ascontiguousarray(w, dtype=np.uint64)
    out = np.zeros(len(w), dtype=np.uint64)
    if lib().or_freq_from_weights(ptr(w), len(w), bits, ptr(out)) != 0:
        raise ValueError("from_weights refused")
    return out


def logits_to_weights(logits, table):
    """weights_of (crates/hardshell/src/logits.rs:62-72): table[min(max - l, len - 1)]."""
    l = np.ascontiguousarray(logits, dtype=np.int64)
    t = np.ascontiguousarray(table, dtype=np.uint64)
    w = np.zeros(len(l), np.uint64)
    if lib().or_logits_to_weights(ptr(l), len(l), ptr(t), len(t), ptr(w)) != 0:
        raise ValueError("weights refused")
    return w


MIX_NONE = 0xFFFFFFFF
MIX_PLAIN = 0xFFFFFFFE


def mix_stats(w, p):
    """Pass 1 of taco_match::Mixer::mix: (sum of w, w[p] or 0, the first index of the largest
    weight or 0)."""
    w = np.ascontiguousarray(w, dtype=np.uint64)
    out = np.zeros(4, np.uint64)
    lib().or_mix_stats(ptr(w), len(w), p, ptr(out))
    return int(out[0]) | (int(out[1]) << 64), int(out[2]), int(out[3])


def mix_record(total, wp, q):
    """(k, m, w'[p]) of rule 5; ValueError for a q outside 1..=65535 or w[p] > total."""
    k, m, wpm = C.c_uint32(), C.c_uint32(), C.c_uint64()
    e = lib().or_mix_record(total & ((1 << 64) - 1), total >> 64, wp, q, C.byref(k), C.byref(m),
                            C.byref(wpm))
    if e:
        raise ValueError(f"mix record refused ({e})")
    return k.value, m.value, wpm.value


def mix_apply(w, p, q):
    """The weights of Mixer::mix(w, p) with the mixer's probability q of p (p = MIX_NONE: no
    prediction)."""
    w = np.array(w, dtype=np.uint64)
    e = lib().or_mix_apply(ptr(w), len(w), p, q)
    if e:
        raise ValueError(f"mix refused ({e})")
    return w


class MixState:
    """The match model and the mixer of one block, mixer rule version 1 (crates/taco/src/mix.rs)."""

    def __init__(self):
        self.h = lib().or_mix_state_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_mix_state_free(self.h)
            self.h = None

    def predict(self):
        """(token, length) of the match model, or None."""
        t, n = C.c_uint32(), C.c_uint32()
        return (t.value, n.value) if lib().or_mix_state_predict(self.h, C.byref(t), C.byref(n)) else None

    def mix_stats(self, total, predicted, top):
        """q for the model's prediction from the statistics of the GPT-2 weights (0: none)."""
        return lib().or_mix_state_mix_stats(self.h, total, predicted, top)

    def mix(self, w):
        """Mixer::mix of the weights with the model's prediction."""
        w = np.array(w, dtype=np.uint64)
        if lib().or_mix_state_mix(self.h, ptr(w), len(w)) != 0:
            raise ValueError("mix refused")
        return w

    def observe(self, token):
        lib().or_mix_state_observe(self.h, token)


def logistic_tables():
    sq = np.zeros(8191, np.uint16)
    st = np.zeros(65536, np.int16)
    lib().or_logistic_tables(ptr(sq), ptr(st))
    return sq, st


def encode_mixed_block(model, tokens, overlap=0):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    cap = 16 + 8 * len(t)
    out = np.zeros(cap, np.uint8)
    n = lib().or_encode_mixed_block(model.h, overlap, ptr(t), len(t), ptr(out), cap)
    if n == (1 << 64) - 1:
        raise ValueError("encode failed")
    return out[:n].tobytes()


def decode_mixed_block(model, payload, overlap=0, cap=1 << 20):
    p = np.frombuffer(payload, np.uint8).copy()
    out = np.zeros(cap, np.uint32)
    n = lib().or_decode_mixed_block(model.h, overlap, ptr(p), len(p), ptr(out), cap)
    if n < 0:
        raise ValueError("decode failed")
    return out[:n].copy()


def freq_interval(w, bits, symbol):
    w = np.ascontiguousarray(w, dtype=np.uint64)
    s, f = C.c_uint64(), C.c_uint64()
    if lib().or_freq_interval(ptr(w), len(w), bits, symbol, C.byref(s), C.byref(f)) != 0:
        raise ValueError("interval refused")
    return s.value, f.value


def freq_find(w, bits, target):
    w = np.ascontiguousarray(w, dtype=np.uint64)
    sym, s, f = C.c_uint32(), C.c_uint64(), C.c_uint64()
    if lib().or_freq_find(ptr(w), len(w), bits, target, C.byref(sym), C.byref(s),
                          C.byref(f)) != 0:
        raise ValueError("find refused")
    return sym.value, s.value, f.value


def encode_script(ops):
    a = np.ascontiguousarray(np.asarray(ops, dtype=np.uint64).reshape(-1, 4))
    n = lib().or_encode_script(ptr(a), len(a), None, 0)
    out = np.zeros(max(n, 1), dtype=np.uint8)
    lib().or_encode_script(ptr(a), len(a), ptr(out), n)
    return out[:n].tobytes()


class Decoder:
    def __init__(self, data: bytes):
        self._b = np.frombuffer(data, dtype=np.uint8).copy() if data else np.zeros(1, np.uint8)
        self.h = lib().or_decoder_new(ptr(self._b), len(data))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_decoder_free(self.h)

    def target(self, bits):
        return lib().or_decoder_target(self.h, bits)

    def decode_interval(self, start, freq, bits):
        if lib().or_decoder_decode_interval(self.h, start, freq, bits) != 0:
            raise ValueError("target not in interval")

    def decode_bit(self, p1):
        return bool(lib().or_decoder_decode_bit(self.h, p1))


def encode_block(model, tokens, overlap=0, stop=None):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    stop = (1 << 64) - 1 if stop is None else stop
    cap = 16 + 8 * len(t)
    out = np.zeros(cap, np.uint8)
    n = lib().or_encode_block(model.h, overlap, ptr(t), len(t), stop, ptr(out), cap)
    if n == (1 << 64) - 1:
        return None
    return out[:n].tobytes()


def decode_block(model, payload, overlap=0, cap=1 << 20):
    p = np.frombuffer(payload, np.uint8).copy()
    out = np.zeros(cap, np.uint32)
    n = lib().or_decode_block(model.h, overlap, ptr(p), len(p), ptr(out), cap)
    if n < 0:
        raise ValueError("decode failed")
    return out[:n].copy()


def fast_window_intervals(model, tokens, chunk=32):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.zeros((len(t), 3), np.uint64)
    if lib().or_fast_window_intervals(model.h, ptr(t), len(t), chunk, ptr(out)) != 0:
        raise ValueError("window refused")
    return out


def fast_window_weights(model, tokens, chunk=32):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.zeros((len(t), model.vocab), np.uint64)
    if lib().or_fast_window_weights(model.h, ptr(t), len(t), chunk, ptr(out)) != 0:
        raise ValueError("window refused")
    return out


def fold_payloads(model, tokens, count, n, chunk=32, threads=1):
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    cap = 16 + 8 * n
    out = np.zeros(count * cap, np.uint8)
    lens = np.zeros(count, np.uint64)
    if lib().or_fold_payloads(model.h, ptr(t), count, n, chunk, threads, ptr(out), cap,
                              ptr(lens)) != 0:
        raise ValueError("fold refused")
    return [out[w * cap: w * cap + int(lens[w])].tobytes() for w in range(count)]


def matmul_i8(w, x):
    w = np.ascontiguousarray(w, dtype=np.int8)
    x = np.ascontiguousarray(x, dtype=np.int8)
    rows, cols = w.shape
    n = x.shape[0]
    out = np.zeros((n, rows), np.int32)
    lib().or_matmul_i8(ptr(w), rows, ptr(x), n, cols, ptr(out))
    return out


def linear_act_ref(w, a, bias, mult, shift):
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    bias = np.ascontiguousarray(bias, dtype=np.int32)
    mult = np.ascontiguousarray(mult, dtype=np.int32)
    n, k = w.shape
    m = a.shape[0]
    out = np.zeros((m, n), np.int8)
    lib().or_linear_act_ref(ptr(w), ptr(a), ptr(bias), ptr(mult), shift, m, n, k, ptr(out))
    return out


def attend_decode_ref(q, kc, vc, ctx, score_m, score_s, out_m, out_s, table, p):
    q = np.ascontiguousarray(q, dtype=np.int8)
    kc = np.ascontiguousarray(kc, dtype=np.int8)
    vc = np.ascontiguousarray(vc, dtype=np.int8)
    ctx = np.ascontiguousarray(ctx, dtype=np.uint32)
    table = np.ascontiguousarray(table, dtype=np.int32)
    b, h, hd = q.shape
    cap = kc.shape[2]
    out = np.zeros((b, h * hd), np.int8)
    lib().or_attend_decode_ref(ptr(q), ptr(kc), ptr(vc), ptr(ctx), b, h, hd, cap, score_m,
                               score_s, out_m, out_s, ptr(table), len(table), p, ptr(out))
    return out
