"""Python mirror of the hardshell-cuda API (crates/hardshell-cuda/src/lib.rs:36-43) over the C ABI
of libhardshell_hip.so (include/hardshell_hip.h): HipDevice, HipModel, HipBatch, HipSession
and the op-level entry points. Errors mirror crates/hardshell-cuda/src/error.rs:9-51.

The native library is required: importing this module never falls back to a CPU path, and
every call fails loudly if libhardshell_hip.so is missing."""

from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Iterable, List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhardshell_hip.so")

HS_OK, HS_NO_DEVICE, HS_DEVICE_ERROR, HS_UNSUPPORTED, HS_MODEL_ERROR, HS_BAD_SLOT, \
    HS_LENGTH_MISMATCH, HS_INVALID_ARGUMENT = range(8)

MODEL_ERRORS = {
    1: "InvalidShape", 2: "LengthMismatch", 3: "DotTooLong", 4: "BadMagic",
    5: "UnsupportedVersion", 6: "Truncated", 7: "HeaderNotUtf8", 8: "HeaderJson",
    9: "InvalidHeader", 10: "Layout", 11: "NonZeroPadding", 12: "Vocabulary",
    13: "MissingTensor", 14: "UnexpectedTensor", 15: "TensorMismatch", 16: "TokenOutOfRange",
    17: "InvalidOverlap", 18: "BadTruncate", 19: "TooLarge", 20: "Unsupported",
}


class HipError(Exception):
    def __init__(self, status: int, code: int, message: str):
        super().__init__(message)
        self.status, self.code, self.message = status, code, message


class NoDevice(HipError):
    pass


class DeviceError(HipError):
    pass


class Unsupported(HipError):
    pass


class ModelError(HipError):
    @property
    def kind(self) -> str:
        return MODEL_ERRORS.get(self.code, str(self.code))


class BadSlot(HipError):
    pass


class LengthMismatch(HipError):
    pass


_ERRORS = {HS_NO_DEVICE: NoDevice, HS_DEVICE_ERROR: DeviceError, HS_UNSUPPORTED: Unsupported,
           HS_MODEL_ERROR: ModelError, HS_BAD_SLOT: BadSlot, HS_LENGTH_MISMATCH: LengthMismatch,
           HS_INVALID_ARGUMENT: HipError}


class _Input(C.Structure):
    _fields_ = [("slot", C.c_uint32), ("token", C.c_uint32)]


# The mixed coder op of the logs profile (crates/hardshell-cuda/src/mixed.rs).
HS_MIX_NONE = 0xFFFFFFFF   # a mixed table without a prediction
HS_MIX_PLAIN = 0xFFFFFFFE  # the table of GPT-2 alone


class MixStats(C.Structure):
    """MixStats (mixed.rs:36-49): total = sum w, predicted = w[p], top = the largest."""
    _fields_ = [("total", C.c_uint64), ("predicted", C.c_uint64), ("top", C.c_uint32),
                ("pad", C.c_uint32)]


MIXER_FN = C.CFUNCTYPE(C.c_uint32, C.c_void_p, C.c_size_t, C.POINTER(MixStats))


def _mixer(fn):
    """A C callback over fn(input, stats) -> q; an exception gives q = 0 (refused)."""
    def call(_user, i, st):
        try:
            return int(fn(int(i), st.contents))
        except Exception:  # noqa: BLE001 - the library reports the bad q
            return 0
    return MIXER_FN(call)


class _Query(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("value", C.c_uint32)]


class _Interval(C.Structure):
    _fields_ = [("symbol", C.c_uint64), ("start", C.c_uint64), ("freq", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "taco_amd/libhardshell_hip.so is not built (run `python -c 'import __graft_entry__ as g; "
                "g.build()'`); there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        P, S, U32, U64 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64
        L.hs_last_error_message.restype = C.c_char_p
        L.hs_last_error_code.restype = C.c_int
        L.hs_version.restype = C.c_char_p
        L.hs_device_open.argtypes = [C.c_int, C.POINTER(P)]
        L.hs_device_close.argtypes = [P]
        L.hs_device_name.argtypes = [P, C.c_char_p, S]
        L.hs_device_memory.argtypes = [P, C.POINTER(S), C.POINTER(S)]
        L.hs_model_load.argtypes = [P, P, S, C.POINTER(P)]
        L.hs_model_free.argtypes = [P]
        L.hs_model_hash.argtypes = [P, P]
        for f in ("vocab", "n_ctx", "eot"):
            getattr(L, "hs_model_" + f).restype = U32
            getattr(L, "hs_model_" + f).argtypes = [P]
        L.hs_model_is_wide.argtypes = [P]
        L.hs_model_weight_bytes.restype = U64
        L.hs_model_weight_bytes.argtypes = [P]
        L.hs_model_cache_bytes_per_slot.restype = U64
        L.hs_model_cache_bytes_per_slot.argtypes = [P]
        L.hs_batch_new.argtypes = [P, S, S, C.POINTER(P)]
        L.hs_batch_free.argtypes = [P]
        L.hs_batch_set_overlap.argtypes = [P, U32]
        for f in ("slots", "max_rows"):
            getattr(L, "hs_batch_" + f).restype = S
            getattr(L, "hs_batch_" + f).argtypes = [P]
        L.hs_batch_gpu_bytes.restype = U64
        L.hs_batch_gpu_bytes.argtypes = [P]
        for f in ("position", "stream_len", "room"):
            getattr(L, "hs_batch_" + f).restype = S
            getattr(L, "hs_batch_" + f).argtypes = [P, S]
        L.hs_batch_reset.argtypes = [P, S]
        L.hs_batch_run_weights.argtypes = [P, P, S, P]
        L.hs_batch_run_coded.argtypes = [P, P, P, S, U32, P]
        L.hs_batch_step.argtypes = [P, P, S]
        L.hs_batch_weights.argtypes = [P, S, P]
        L.hs_batch_truncate.argtypes = [P, S, S]
        L.hs_op_gemm_i8.argtypes = [P, P, P, S, S, S, P]
        L.hs_op_gemm_requant_i8.argtypes = [P, P, P, P, P, C.c_uint8, S, S, S, P]
        L.hs_op_gemm_i8_split.argtypes = [P, P, P, S, S, S, C.c_uint32, P]
        L.hs_op_gemm_i8_i16.argtypes = [P, P, P, S, S, S, C.c_uint32, P]
        L.hs_op_gemm_requant_i8_dev.argtypes = [P, P, P, P, P, C.c_uint8, S, S, S, P, P]
        L.hs_op_gemm_layout.argtypes = [S, S, S, C.POINTER(S), C.POINTER(S), C.POINTER(S)]
        L.hs_op_gemm_layout.restype = None
        L.hs_op_attend_decode_dev.argtypes = [P, P, P, P, P, S, S, S, S, C.c_int32, C.c_uint8,
                                              C.c_int32, C.c_uint8, P, S, C.c_uint8, P, P]
        L.hs_op_attend_decode_dev_noalloc.argtypes = L.hs_op_attend_decode_dev.argtypes
        L.hs_read_bw.argtypes = [P, S, S, C.POINTER(C.c_uint64)]
        L.hs_probe_issue.argtypes = [P, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]
        L.hs_model_load_with.argtypes = [P, P, S, P, C.POINTER(P)]
        L.hs_batch_run_without_readback.argtypes = [P, P, S]
        L.hs_device_kernel_resources.argtypes = [P, P, P, P, P, S, C.POINTER(S)]
        L.hs_device_alloc.argtypes = [P, S, C.POINTER(P)]
        L.hs_device_free.argtypes = [P, P]
        L.hs_device_upload.argtypes = [P, P, P, S]
        L.hs_device_download.argtypes = [P, P, P, S]
        L.hs_device_synchronize.argtypes = [P]
        L.hs_device_copy.argtypes = [P, P, P, S]
        L.hs_op_gemm_requant_gpu_ns.argtypes = [P, P, P, P, P, C.c_uint8, S, S, S, P, S,
                                                C.POINTER(U64)]
        L.hs_op_attend_decode_gpu_ns.argtypes = [P, P, P, P, P, S, S, S, S, C.c_int32,
                                                 C.c_uint8, C.c_int32, C.c_uint8, P, S,
                                                 C.c_uint8, P, S, C.POINTER(U64)]
        L.hs_op_attend_decode_sets_gpu_ns.argtypes = [P, P, P, P, S, P, S, S, S, S, C.c_int32,
                                                      C.c_uint8, C.c_int32, C.c_uint8, P, S,
                                                      C.c_uint8, P, C.POINTER(U64)]
        L.hs_batch_set_profiling.argtypes = [P, C.c_int]
        L.hs_batch_profile.restype = S
        L.hs_batch_profile.argtypes = [P, P, P, P, P, S, C.c_int]
        L.hs_batch_model.restype = P
        L.hs_batch_model.argtypes = [P]
        L.hs_model_validate.argtypes = [P, S, P]
        L.hs_op_coder.argtypes = [P, P, S, S, P, S, P, U32, P]
        L.hs_batch_run_coded_mixed.argtypes = [P, P, P, P, S, U32, MIXER_FN, P, P]
        L.hs_batch_run_coded_dual.argtypes = [P, P, P, P, S, U32, MIXER_FN, P, P, P]
        L.hs_op_mixed_coder.argtypes = [P, P, S, S, P, P, U32, MIXER_FN, P, P, P]
        L.hs_op_mixed_coder_logits.argtypes = [P, P, S, S, P, S, P, P, U32, MIXER_FN, P, P, P]
        _lib = L
    return _lib


def _check(status: int):
    if status != HS_OK:
        L = lib()
        msg = L.hs_last_error_message().decode(errors="replace")
        raise _ERRORS.get(status, HipError)(status, L.hs_last_error_code(), msg)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def version() -> str:
    return lib().hs_version().decode()


class HipDevice:
    """CudaDevice (crates/hardshell-cuda/src/device.rs:29-74)."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        _check(lib().hs_device_open(ordinal, C.byref(h)))
        self.h = h

    @classmethod
    def open(cls, ordinal: int = 0) -> "HipDevice":
        return cls(ordinal)

    def name(self) -> str:
        buf = C.create_string_buffer(256)
        _check(lib().hs_device_name(self.h, buf, 256))
        return buf.value.decode()

    def memory(self) -> Tuple[int, int]:
        f, t = C.c_size_t(), C.c_size_t()
        _check(lib().hs_device_memory(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def close(self):
        if getattr(self, "h", None):
            lib().hs_device_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


class HipModel:
    """CudaModel (crates/hardshell-cuda/src/model.rs:242-398)."""

    def __init__(self, dev: HipDevice, data: bytes, loaded: Optional["HipModel"] = None):
        self.dev = dev  # the device outlives the model
        buf = np.frombuffer(data, dtype=np.uint8)
        h = C.c_void_p()
        if loaded is None:
            _check(lib().hs_model_load(dev.h, _ptr(buf), len(buf), C.byref(h)))
        else:
            _check(lib().hs_model_load_with(dev.h, _ptr(buf), len(buf), loaded.h, C.byref(h)))
        self.h = h

    @classmethod
    def load(cls, dev: HipDevice, data: bytes) -> "HipModel":
        return cls(dev, data)

    @classmethod
    def load_with(cls, dev: HipDevice, data: bytes, loaded: "HipModel") -> "HipModel":
        """CudaModel::load_with (model.rs:259-349): reuses the parse of `loaded` when the bytes
        are its file."""
        return cls(dev, data, loaded)

    def hash(self) -> bytes:
        out = np.zeros(32, np.uint8)
        lib().hs_model_hash(self.h, _ptr(out))
        return out.tobytes()

    def vocab_size(self) -> int:
        return lib().hs_model_vocab(self.h)

    def n_ctx(self) -> int:
        return lib().hs_model_n_ctx(self.h)

    def eot_token(self) -> int:
        return lib().hs_model_eot(self.h)

    def is_wide(self) -> bool:
        return bool(lib().hs_model_is_wide(self.h))

    def weight_bytes(self) -> int:
        return lib().hs_model_weight_bytes(self.h)

    def cache_bytes_per_slot(self) -> int:
        return lib().hs_model_cache_bytes_per_slot(self.h)

    def free(self):
        if getattr(self, "h", None):
            lib().hs_model_free(self.h)
            self.h = None

    def __del__(self):
        self.free()


@dataclass(frozen=True)
class CoderInterval:
    """CoderInterval (crates/hardshell-cuda/src/batch.rs:49-58)."""
    symbol: int
    start: int
    freq: int
    is_last: bool


ENCODE, DECODE = 0, 1


def _inputs(inputs: Sequence[Tuple[int, int]]) -> np.ndarray:
    a = np.asarray(inputs, dtype=np.uint32).reshape(-1, 2)
    return np.ascontiguousarray(a)


class HipBatch:
    """CudaBatch (crates/hardshell-cuda/src/batch.rs:237-476)."""

    def __init__(self, model: HipModel, slots: int, max_rows: int):
        self.model = model
        h = C.c_void_p()
        _check(lib().hs_batch_new(model.h, slots, max_rows, C.byref(h)))
        self.h = h
        self.vocab = model.vocab_size()

    def set_overlap(self, k: int):
        _check(lib().hs_batch_set_overlap(self.h, k))

    def slots(self) -> int:
        return lib().hs_batch_slots(self.h)

    def max_rows(self) -> int:
        return lib().hs_batch_max_rows(self.h)

    def gpu_bytes(self) -> int:
        return lib().hs_batch_gpu_bytes(self.h)

    def position(self, slot: int) -> int:
        return lib().hs_batch_position(self.h, slot)

    def reset(self, slot: int):
        lib().hs_batch_reset(self.h, slot)

    def run_without_readback(self, inputs) -> None:
        """CudaBatch::run_without_readback (batch.rs:478-484)."""
        a = _inputs(inputs)
        _check(lib().hs_batch_run_without_readback(self.h, _ptr(a), len(a)))

    def run_weights(self, inputs) -> np.ndarray:
        a = _inputs(inputs)
        out = np.zeros((len(a), self.vocab), np.uint64)
        _check(lib().hs_batch_run_weights(self.h, _ptr(a), len(a), _ptr(out)))
        return out

    def run_coded_raw(self, inputs, queries, freq_bits: int = 32) -> np.ndarray:
        """The intervals as an [n, 3] u64 array (symbol, start, freq)."""
        a = _inputs(inputs)
        q = np.ascontiguousarray(np.asarray(queries, dtype=np.uint32).reshape(-1, 2))
        if len(q) != len(a):
            raise LengthMismatch(HS_LENGTH_MISMATCH, 0,
                                 f"length mismatch: expected {len(a)}, found {len(q)}")
        out = np.zeros((len(a), 3), np.uint64)
        _check(lib().hs_batch_run_coded(self.h, _ptr(a), _ptr(q), len(a), freq_bits, _ptr(out)))
        return out

    def run_coded(self, inputs, queries, freq_bits: int = 32) -> List[CoderInterval]:
        raw = self.run_coded_raw(inputs, queries, freq_bits)
        return [CoderInterval(int(s), int(st), int(f), int(s) + 1 == self.vocab) for s, st, f in raw]

    def run_coded_mixed(self, inputs, queries, tables, freq_bits, mixer) -> np.ndarray:
        """CudaBatch::run_coded_mixed: tables[i] is HS_MIX_PLAIN, HS_MIX_NONE or the predicted
        token; mixer(i, stats) -> q. The intervals as an [n, 3] u64 array."""
        a = _inputs(inputs)
        q = np.ascontiguousarray(np.asarray(queries, dtype=np.uint32).reshape(-1, 2))
        t = np.ascontiguousarray(np.asarray(tables, dtype=np.uint32))
        out = np.zeros((len(a), 3), np.uint64)
        cb = _mixer(mixer)
        _check(lib().hs_batch_run_coded_mixed(self.h, _ptr(a), _ptr(q), _ptr(t), len(a), freq_bits,
                                              cb, None, _ptr(out)))
        return out

    def run_coded_dual(self, inputs, tokens, predictions, freq_bits, mixer):
        """CudaBatch::run_coded_dual: (plain, mixed) intervals as two [n, 3] u64 arrays;
        predictions[i] is a token or HS_MIX_NONE."""
        a = _inputs(inputs)
        tk = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        pr = np.ascontiguousarray(np.asarray(predictions, dtype=np.uint32))
        plain = np.zeros((len(a), 3), np.uint64)
        mixed = np.zeros((len(a), 3), np.uint64)
        cb = _mixer(mixer)
        _check(lib().hs_batch_run_coded_dual(self.h, _ptr(a), _ptr(tk), _ptr(pr), len(a), freq_bits,
                                             cb, None, _ptr(plain), _ptr(mixed)))
        return plain, mixed

    def step(self, inputs):
        a = _inputs(inputs)
        _check(lib().hs_batch_step(self.h, _ptr(a), len(a)))

    def weights(self, slot: int) -> np.ndarray:
        out = np.zeros(self.vocab, np.uint64)
        _check(lib().hs_batch_weights(self.h, slot, _ptr(out)))
        return out

    def stream_len(self, slot: int) -> int:
        return lib().hs_batch_stream_len(self.h, slot)

    def room(self, slot: int) -> int:
        return lib().hs_batch_room(self.h, slot)

    def truncate(self, slot: int, length: int):
        _check(lib().hs_batch_truncate(self.h, slot, length))

    def free(self):
        if getattr(self, "h", None):
            lib().hs_batch_free(self.h)
            self.h = None

    def __del__(self):
        self.free()


class HipSession:
    """CudaSession (crates/hardshell-cuda/src/session.rs:20-91): a batch of one slot with the
    API shape of hardshell::gpt2::Session."""

    def __init__(self, model: HipModel, overlap: int = 0, max_rows: int = 64):
        self.batch = HipBatch(model, 1, max_rows)
        if overlap:
            self.batch.set_overlap(overlap)
        self.eot = model.eot_token()

    def start_block(self) -> np.ndarray:
        self.batch.reset(0)
        return self.batch.run_weights([(0, self.eot)])[0]

    def step(self, token: int) -> np.ndarray:
        return self.batch.run_weights([(0, token)])[0]

    def step_many(self, tokens: Iterable[int]) -> np.ndarray:
        return self.batch.run_weights([(0, t) for t in tokens])

    def position(self) -> int:
        return self.batch.position(0)


def matmul_i8(dev: HipDevice, w: np.ndarray, a: np.ndarray) -> np.ndarray:
    """ops.rs:142-161: out[i][r] = w[r] . a[i], exact i32."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    n, k = w.shape
    m = a.shape[0]
    out = np.zeros((m, n), np.int32)
    _check(lib().hs_op_gemm_i8(dev.h, _ptr(w), _ptr(a), m, n, k, _ptr(out)))
    return out


def matmul_i8_split(dev: HipDevice, w: np.ndarray, a: np.ndarray, splits: int) -> np.ndarray:
    """ops.rs:163-184: matmul_i8 with K in `splits` slices whose partials are summed."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    n, k = w.shape
    m = a.shape[0]
    out = np.zeros((m, n), np.int32)
    _check(lib().hs_op_gemm_i8_split(dev.h, _ptr(w), _ptr(a), m, n, k, splits, _ptr(out)))
    return out


def matmul_i8_i16(dev: HipDevice, w: np.ndarray, a: np.ndarray, splits: int = 1) -> np.ndarray:
    """ops.rs:220-282: out[i][r] = w[r] . a[i] for i16 activations, exact i64."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int16)
    n, k = w.shape
    m = a.shape[0]
    out = np.zeros((m, n), np.int64)
    _check(lib().hs_op_gemm_i8_i16(dev.h, _ptr(w), _ptr(a), m, n, k, splits, _ptr(out)))
    return out


def gemm_requant_i8(dev: HipDevice, w, a, bias, mult, shift: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    bias = np.ascontiguousarray(bias, dtype=np.int32)
    mult = np.ascontiguousarray(mult, dtype=np.int32)
    n, k = w.shape
    m = a.shape[0]
    out = np.zeros((m, n), np.int8)
    _check(lib().hs_op_gemm_requant_i8(dev.h, _ptr(w), _ptr(a), _ptr(bias), _ptr(mult), shift,
                                       m, n, k, _ptr(out)))
    return out


def kernel_resources(dev: HipDevice):
    """CudaDevice::kernel_resources (device.rs:65-74): (name, registers, private bytes, static
    LDS bytes) of each main kernel."""
    cap = 64
    names = (C.c_char * (64 * cap))()
    regs, priv, lds = (np.zeros(cap, np.int32) for _ in range(3))
    n = C.c_size_t()
    _check(lib().hs_device_kernel_resources(dev.h, names, _ptr(regs), _ptr(priv), _ptr(lds), cap,
                                            C.byref(n)))
    raw = bytes(names)
    return [(raw[64 * i:64 * i + 64].split(b"\0")[0].decode(), int(regs[i]), int(priv[i]), int(lds[i]))
            for i in range(min(n.value, cap))]


def read_bw(dev: HipDevice, nbytes: int, reps: int) -> float:
    """read_gpu_ns (crates/hardshell-cuda/src/ops.rs:328-335) as bytes per second: a streaming
    kernel reads a device buffer of nbytes, reps times."""
    ns = C.c_uint64()
    _check(lib().hs_read_bw(dev.h, nbytes, reps, C.byref(ns)))
    return nbytes * reps / (ns.value * 1e-9)


def probe_issue(dev: HipDevice, op: int, waves_per_simd: int, iters: int) -> int:
    """hs_probe_issue: the GPU ns of one launch of `iters` rounds of op on every SIMD."""
    ns = C.c_uint64()
    _check(lib().hs_probe_issue(dev.h, op, waves_per_simd, iters, C.byref(ns)))
    return ns.value


def gemm_layout(m: int, n: int, k: int) -> Tuple[int, int, int]:
    a, b, c = C.c_size_t(), C.c_size_t(), C.c_size_t()
    lib().hs_op_gemm_layout(m, n, k, C.byref(a), C.byref(b), C.byref(c))
    return a.value, b.value, c.value


def gemm_pack(x: np.ndarray, rows_pad: int, k_pad: int) -> np.ndarray:
    """An i8 operand [rows, k] in the layout of the _dev GEMM entries: k_pad / 64 panels of
    rows_pad rows x 64 bytes, zero padded (hs_op_gemm_layout)."""
    rows, k = x.shape
    p = np.zeros((rows_pad, k_pad), np.int8)
    p[:rows, :k] = x
    return np.ascontiguousarray(p.reshape(rows_pad, k_pad // 64, 64).transpose(1, 0, 2))


def mixed_intervals_of_weights(dev: HipDevice, weights: np.ndarray, queries, predictions,
                               freq_bits: int, mixer):
    """mixed_intervals_of_weights (mixed.rs:160-233): the statistics [rows, 3] (total,
    predicted, top) and the intervals [rows, 3] of the mixed tables of given weights."""
    w = np.ascontiguousarray(weights, dtype=np.uint64)
    rows, vocab = w.shape
    q = np.ascontiguousarray(np.asarray(queries, dtype=np.uint32).reshape(-1, 2))
    pr = np.ascontiguousarray(np.asarray(predictions, dtype=np.uint32))
    stats = (MixStats * rows)()
    out = np.zeros((rows, 3), np.uint64)
    cb = _mixer(mixer)
    _check(lib().hs_op_mixed_coder(dev.h, _ptr(w), rows, vocab, _ptr(q), _ptr(pr), freq_bits, cb,
                                   None, C.cast(stats, C.c_void_p), _ptr(out)))
    st = np.array([[s.total, s.predicted, s.top] for s in stats], dtype=np.uint64).reshape(rows, 3)
    return st, out


def mixed_coder_logits(dev: HipDevice, logits: np.ndarray, table: np.ndarray, queries, tables,
                       freq_bits: int, mixer):
    """The mixed coder op on given i64 logits [rows, vocab] and a logits table (the compact
    form for tables of at most 16,384 entries): statistics [rows, 3] and intervals [rows, 3]."""
    logits = np.ascontiguousarray(logits, dtype=np.int64)
    table = np.ascontiguousarray(table, dtype=np.uint64)
    rows, vocab = logits.shape
    q = np.ascontiguousarray(np.asarray(queries, dtype=np.uint32).reshape(-1, 2))
    t = np.ascontiguousarray(np.asarray(tables, dtype=np.uint32))
    stats = (MixStats * rows)()
    out = np.zeros((rows, 3), np.uint64)
    cb = _mixer(mixer)
    _check(lib().hs_op_mixed_coder_logits(dev.h, _ptr(logits), rows, vocab, _ptr(table), len(table),
                                          _ptr(q), _ptr(t), freq_bits, cb, None,
                                          C.cast(stats, C.c_void_p), _ptr(out)))
    st = np.array([[s.total, s.predicted, s.top] for s in stats], dtype=np.uint64).reshape(rows, 3)
    return st, out


def coder(dev: HipDevice, logits: np.ndarray, table: np.ndarray, queries, freq_bits: int = 32
          ) -> np.ndarray:
    """The coder op on given i64 logits [rows, vocab]: (symbol, start, freq) per row."""
    logits = np.ascontiguousarray(logits, dtype=np.int64)
    table = np.ascontiguousarray(table, dtype=np.uint64)
    q = np.ascontiguousarray(np.asarray(queries, dtype=np.uint32).reshape(-1, 2))
    rows, vocab = logits.shape
    out = np.zeros((rows, 3), np.uint64)
    _check(lib().hs_op_coder(dev.h, _ptr(logits), rows, vocab, _ptr(table), len(table), _ptr(q),
                             freq_bits, _ptr(out)))
    return out
