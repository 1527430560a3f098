"""The fold/unfold harness over libtaco_hip.so (include/taco_hip.h): the role of the reference's
taco crate on this path (crates/taco/src/gpu_fold.rs, gpu_unfold.rs, codec.rs), and the .taco
container of the text profile (crates/taco-format/src/writer.rs:245-288)."""

from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional, Sequence

import numpy as np

from . import hip

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtaco_hip.so")
_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        hip.lib()  # the backend first (libtaco_hip.so links it)
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("taco_amd/libtaco_hip.so is not built; there is no CPU fallback")
        L = C.CDLL(LIB_PATH)
        P, S = C.c_void_p, C.c_size_t
        L.tc_fold_blocks.argtypes = [P, C.c_uint32, P, P, S, P, P, S, P]
        L.tc_unfold_blocks.argtypes = [P, C.c_uint32, P, P, S, P, S, P]
        L.tc_container_build.restype = S
        L.tc_container_build.argtypes = [P, P, S, C.c_uint32, C.c_uint32, P, P, P, P, S]
        L.tc_tokenizer_new.argtypes = [P, P, S, C.c_uint32, P, S, C.POINTER(P)]
        L.tc_tokenizer_for_model.argtypes = [P, C.POINTER(P)]
        L.tc_tokenizer_free.argtypes = [P]
        L.tc_tokenizer_free.restype = None
        L.tc_tokenize.argtypes = [P, P, S, P, S, C.POINTER(S)]
        L.tc_pretokenize.argtypes = [P, S, P, S]
        L.tc_pretokenize.restype = S
        L.tc_fold_bytes.argtypes = [P, P, P, S, C.c_uint32, C.c_uint32, P, S, C.POINTER(S)]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


NO_PAYLOAD = (1 << 64) - 1


def fold_blocks(batch: hip.HipBatch, blocks: Sequence[np.ndarray], overlap: int = 0,
                stop: Optional[Sequence[int]] = None) -> List[Optional[bytes]]:
    """The payload of each block of tokens (None if the encoder stopped at `stop`)."""
    toks = np.ascontiguousarray(np.concatenate([np.asarray(b, np.uint32) for b in blocks])
                                if blocks else np.zeros(0, np.uint32), dtype=np.uint32)
    offs = np.zeros(len(blocks) + 1, np.uint64)
    offs[1:] = np.cumsum([len(b) for b in blocks])
    cap = 16 + 5 * max([len(b) for b in blocks] + [1])
    out = np.zeros(max(1, len(blocks) * cap), np.uint8)
    lens = np.zeros(max(1, len(blocks)), np.uint64)
    st = None if stop is None else np.ascontiguousarray(stop, dtype=np.uint64)
    hip._check(lib().tc_fold_blocks(batch.h, overlap, _p(toks), _p(offs), len(blocks),
                                    None if st is None else _p(st), _p(out), cap, _p(lens)))
    res: List[Optional[bytes]] = []
    for b in range(len(blocks)):
        n = int(lens[b])
        if n == NO_PAYLOAD:
            res.append(None)
        else:
            if n > cap:
                raise RuntimeError("payload larger than its buffer")
            res.append(out[b * cap: b * cap + n].tobytes())
    return res


def unfold_blocks(batch: hip.HipBatch, payloads: Sequence[bytes], overlap: int = 0,
                  cap: int = 1 << 16) -> List[np.ndarray]:
    data = np.frombuffer(b"".join(payloads) or b"\0", np.uint8).copy()
    offs = np.zeros(len(payloads) + 1, np.uint64)
    offs[1:] = np.cumsum([len(p) for p in payloads])
    toks = np.zeros(max(1, len(payloads) * cap), np.uint32)
    counts = np.zeros(max(1, len(payloads)), np.uint64)
    hip._check(lib().tc_unfold_blocks(batch.h, overlap, _p(data), _p(offs), len(payloads),
                                      _p(toks), cap, _p(counts)))
    return [toks[b * cap: b * cap + int(counts[b])].copy() for b in range(len(payloads))]


def container(model_hash: bytes, original: bytes, block_size: int, overlap: int,
              payloads: Sequence[Optional[bytes]]) -> bytes:
    """Container::build with Block::choose_smallest(len, coded, None) for each block: coded if
    the payload is strictly smaller than the block's original bytes, else raw."""
    count = (len(original) + block_size - 1) // block_size
    if len(payloads) != count:
        raise ValueError("one payload (or None) per block")
    kinds = np.zeros(max(1, count), np.uint8)
    parts, offs = [], [0]
    for b, p in enumerate(payloads):
        orig = min(block_size, len(original) - b * block_size)
        if p is not None and len(p) < orig:
            kinds[b] = 1
            parts.append(p)
        offs.append(offs[-1] + (len(p) if kinds[b] == 1 else 0))
    blob = np.frombuffer(b"".join(parts) or b"\0", np.uint8)
    offa = np.asarray(offs, np.uint64)
    mh = np.frombuffer(model_hash, np.uint8)
    orig = np.frombuffer(original or b"\0", np.uint8)
    # 104-byte header, 5 bytes per block, and stored blocks no larger than the original bytes
    cap = 104 + 5 * count + len(original)
    out = np.empty(cap, np.uint8)
    n = lib().tc_container_build(_p(mh), _p(orig), len(original), block_size, overlap, _p(kinds),
                                 _p(blob), _p(offa), _p(out), cap)
    if n == 0:
        raise ValueError("the container was refused")
    if n > cap:
        raise RuntimeError("the container is larger than its bound")
    return out[:n].tobytes()


def token_bytes(tokens: np.ndarray) -> bytes:
    """The original bytes of a stream of fixed-width 4-byte tokens (id -> its LE u32)."""
    return np.ascontiguousarray(tokens, dtype="<u4").tobytes()


class Tokenizer:
    """crates/taco/src/tokenizer (Tokenizer::new / for_vocabulary / encode) over tc_tokenizer."""

    def __init__(self, h):
        self.h = h

    @classmethod
    def from_parts(cls, tokens: Sequence[bytes], eot: Optional[int], merges) -> "Tokenizer":
        blob = np.frombuffer(b"".join(tokens) or b"\0", np.uint8).copy()
        offs = np.zeros(len(tokens) + 1, np.uint64)
        offs[1:] = np.cumsum([len(t) for t in tokens])
        pairs = np.ascontiguousarray(np.asarray(merges, np.uint32).reshape(-1, 2)) if len(merges) else np.zeros((1, 2), np.uint32)
        h = C.c_void_p()
        hip._check(lib().tc_tokenizer_new(_p(blob), _p(offs), len(tokens),
                                          0xFFFFFFFF if eot is None else eot, _p(pairs), len(merges),
                                          C.byref(h)))
        return cls(h)

    @classmethod
    def for_model(cls, model: hip.HipModel) -> "Tokenizer":
        h = C.c_void_p()
        hip._check(lib().tc_tokenizer_for_model(model.h, C.byref(h)))
        return cls(h)

    def encode(self, data: bytes) -> np.ndarray:
        buf = np.frombuffer(data or b"\0", np.uint8)
        out = np.zeros(max(1, len(data)), np.uint32)
        n = C.c_size_t()
        hip._check(lib().tc_tokenize(self.h, _p(buf), len(data), _p(out), len(out), C.byref(n)))
        return out[:n.value].copy()

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.tc_tokenizer_free(self.h)
            self.h = None


def pieces(text: bytes) -> List[bytes]:
    """The GPT-2 pre-tokenizer pieces of well-formed UTF-8 text (tokenizer/pretokenize.rs)."""
    buf = np.frombuffer(text or b"\0", np.uint8)
    ends = np.zeros(max(1, len(text)), np.uint64)
    n = lib().tc_pretokenize(_p(buf), len(text), _p(ends), len(ends))
    if n == (1 << 64) - 1:
        raise ValueError("not well-formed UTF-8")
    out, s = [], 0
    for e in ends[:n]:
        out.append(text[s:int(e)])
        s = int(e)
    return out


def fold_bytes(batch: hip.HipBatch, tokenizer: Tokenizer, data: bytes, block_size: int,
               overlap: int = 0) -> bytes:
    """The byte-level fold of the text profile (crates/taco/src/fold.rs:502-565) without zstd
    candidates: the .taco container of data."""
    buf = np.frombuffer(data or b"\0", np.uint8)
    cap = 256 + 6 * len(data)
    out = np.zeros(cap, np.uint8)
    n = C.c_size_t()
    hip._check(lib().tc_fold_bytes(batch.h, tokenizer.h, _p(buf), len(data), block_size, overlap,
                                   _p(out), cap, C.byref(n)))
    return out[:n.value].tobytes()
