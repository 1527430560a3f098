"""A .hsm writer (the layout of crates/hardshell/src/hsm/writer.rs:76-156): compact JSON in
schema order, the header-length fixed point, space padding of the header, align-64 sections with
zero padding. Used to write synthetic models; pinned by rewriting conformance/tiny.hsm to the
same bytes (tests/test_host.py)."""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np

_DTYPES = {np.dtype(np.int8): "i8", np.dtype(np.int16): "i16", np.dtype(np.int32): "i32",
           np.dtype(np.uint64): "u64"}


def _align64(x: int) -> int:
    return (x + 63) & ~63


class HsmWriter:
    def __init__(self, *, n_layer: int, n_head: int, d_model: int, d_ff: int, vocab_size: int,
                 n_ctx: int, eot_token: int, ln_k: int, ln_j: int, ln_eps: int, softmax_p: int,
                 architecture: str = "gpt2"):
        self.model = dict(architecture=architecture, n_layer=n_layer, n_head=n_head,
                          d_model=d_model, d_ff=d_ff, vocab_size=vocab_size, n_ctx=n_ctx,
                          eot_token=eot_token)
        self.constants = [("ln_k", ln_k), ("ln_j", ln_j), ("ln_eps", ln_eps),
                          ("softmax_p", softmax_p)]
        self.ln_f_bits: Optional[int] = None
        self.ln_beta_frac: Optional[int] = None
        self.vocabulary: List[bytes] = []
        self.merges: List[Tuple[int, int]] = []
        self.tensors: List[Tuple[str, np.ndarray, Optional[int]]] = []

    def set_vocabulary(self, tokens: Sequence[bytes]):
        self.vocabulary = list(tokens)

    def set_merges(self, pairs: Sequence[Tuple[int, int]]):
        self.merges = list(pairs)

    def add_tensor(self, name: str, data: np.ndarray, shift: Optional[int] = None):
        if data.dtype not in _DTYPES:
            raise ValueError(f"dtype {data.dtype} is not a .hsm dtype")
        self.tensors.append((name, np.ascontiguousarray(data), shift))

    def _header(self, header_len: int, vocab_len: int, merges_len: int) -> str:
        m = self.model
        parts = [f'"architecture":"{m["architecture"]}"']
        for k in ("n_layer", "n_head", "d_model", "d_ff", "vocab_size", "n_ctx", "eot_token"):
            parts.append(f'"{k}":{m[k]}')
        consts = [f'"{k}":{v}' for k, v in self.constants]
        if self.ln_f_bits is not None:
            consts.append(f'"ln_f_bits":{self.ln_f_bits}')
        if self.ln_beta_frac is not None:
            consts.append(f'"ln_beta_frac":{self.ln_beta_frac}')
        parts.append('"constants":{' + ",".join(consts) + "}")
        voff = _align64(16 + header_len)
        out = ['{"model":{' + ",".join(parts) + "}",
               f'"vocabulary":{{"offset":{voff},"length":{vocab_len}}}']
        cursor = voff + vocab_len
        if merges_len:
            moff = _align64(cursor)
            out.append(f'"merges":{{"offset":{moff},"length":{merges_len}}}')
            cursor = moff + merges_len
        ts = []
        for name, data, shift in self.tensors:
            off = _align64(cursor)
            shape = ",".join(str(d) for d in data.shape)
            t = (f'{{"name":"{name}","dtype":"{_DTYPES[data.dtype]}","shape":[{shape}],'
                 f'"offset":{off},"length":{data.nbytes}')
            if shift is not None:
                t += f',"shift":{shift}'
            ts.append(t + "}")
            cursor = off + data.nbytes
        out.append('"tensors":[' + ",".join(ts) + "]")
        return ",".join(out) + "}"

    def finish(self) -> bytes:
        vb = bytearray()
        for t in self.vocabulary:
            vb += len(t).to_bytes(2, "little") + t
        mb = bytearray()
        for l, r in self.merges:
            mb += int(l).to_bytes(4, "little") + int(r).to_bytes(4, "little")
        header_len = 0
        while True:
            js = self._header(header_len, len(vb), len(mb)).encode()
            if len(js) <= header_len:
                break
            header_len = len(js)
        v2 = self.ln_f_bits is not None or self.ln_beta_frac is not None or any(
            n.endswith(".mlp.gelu") and d.dtype == np.int16 for n, d, _ in self.tensors)
        head = bytearray(b"HSHLMDL\0")
        head += (2 if v2 else 1).to_bytes(4, "little") + header_len.to_bytes(4, "little")
        head += js + b" " * (header_len - len(js))
        # one zero-filled buffer, each section copied to its aligned offset (the padding is the
        # zeros left between sections)
        pos = _align64(len(head)) + len(vb)
        if mb:
            pos = _align64(pos) + len(mb)
        offsets = []
        for _, data, _ in self.tensors:
            pos = _align64(pos)
            offsets.append(pos)
            pos += data.nbytes
        out = np.zeros(pos, np.uint8)
        out[:len(head)] = np.frombuffer(bytes(head), np.uint8)
        cur = _align64(len(head))
        out[cur:cur + len(vb)] = np.frombuffer(bytes(vb), np.uint8)
        if mb:
            cur = _align64(cur + len(vb))
            out[cur:cur + len(mb)] = np.frombuffer(bytes(mb), np.uint8)
        for off, (_, data, _) in zip(offsets, self.tensors):
            out[off:off + data.nbytes] = data.reshape(-1).view(np.uint8)
        return out.tobytes()
