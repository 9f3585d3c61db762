"""ctypes loader for the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


class G3Info(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "context_length", "embedding_length", "block_count", "feed_forward_length", "head_count",
        "head_count_kv", "head_dim", "value_dim", "vocab_size", "sliding_window")] + \
        [("rms_epsilon", C.c_float), ("global_rope_base", C.c_float), ("local_rope_base", C.c_float),
         ("eos_id", C.c_uint32), ("bos_id", C.c_uint32)]


class G3Taps(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "xn", "q_proj", "k_proj", "v_proj", "q_att", "keys", "values", "history", "att")] + \
        [("hist_cap", C.c_uint32)]


_libs = {}


def lib(path: str | None = None):
    """The oracle library at `path` (default: the built liboracle.so). Other paths load
    variants compiled from patched copies of vrt_oracle.c (the wiring tests' mutants)."""
    path = path or LIB_PATH
    L = _libs.get(path)
    if L is None:
        if path == LIB_PATH and not os.path.exists(path):
            build()
        L = C.CDLL(path)
        P, F, U32, U64, I = C.c_void_p, C.c_float, C.c_uint32, C.c_uint64, C.c_int
        sig = {
            "or_f32_to_f16": (C.c_uint16, [F]),
            "or_f16_to_f32": (F, [C.c_uint16]),
            "or_f32_to_f16_rne": (C.c_uint16, [F]),
            "or_f32_to_f16_rne_n": (None, [P, U64, P]),
            "or_f32_to_bf16_rne": (C.c_uint16, [F]),
            "or_f32_to_bf16_rne_n": (None, [P, U64, P]),
            "or_bf16_to_f32": (F, [C.c_uint16]),
            "or_q8_quantize_a": (None, [P, U64, U32, P]),
            "or_q8_quantize_b": (None, [P, U64, U32, P]),
            "or_q8_dequant": (None, [P, U64, P]),
            "or_q8_matvec_lanes": (None, [P, P, P, U32, U64, U32]),
            "or_q8_matvec_f64": (None, [P, P, P, U32, U64]),
            "or_gelu_tanh": (F, [F]),
            "or_gelu_mul": (None, [P, P, U32]),
            "or_argmax": (None, [P, U64, P, P]),
            "or_rms_norm_into": (None, [P, P, P, U32, F]),
            "or_rms_norm_inplace": (None, [P, P, U32, F]),
            "or_rms_norm_heads": (None, [P, P, U32, U32, F]),
            "or_rope_inv_freq": (None, [U32, F, P]),
            "or_rope_table": (None, [P, U32, U32, P, P]),
            "or_apply_rope": (None, [P, U32, U32, P, P]),
            "or_attention": (I, [P, P, P, U32, U32, U32, F, P]),
            "or_g3_open": (P, [C.c_char_p, U32, C.c_char_p, C.c_size_t]),
            "or_g3_close": (None, [P]),
            "or_g3_get_info": (None, [P, P]),
            "or_g3_reset": (None, [P]),
            "or_g3_decode": (I, [P, U32, U32, I, P, P, P, P]),
            "or_g3_generate": (I, [P, P, U32, U32, P, P]),
            "or_g3_error": (C.c_char_p, [P]),
            "or_g3_set_kv_f16": (None, [P, I]),
            "or_g3_set_kv_format": (None, [P, I]),
            "or_g3_set_taps": (None, [P, P]),
            "or_num_threads": (I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _libs[path] = L
    return L


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def f32_to_f16(x: float) -> int:
    return int(lib().or_f32_to_f16(C.c_float(x)))


def f32_to_f16_rne(x: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits of float32 values, round to nearest even (the fp16 KV rounding)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().or_f32_to_f16_rne_n(_p(a), a.size, _p(out))
    return out


def f16_to_f32(h: int) -> float:
    return float(lib().or_f16_to_f32(C.c_uint16(h)))


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """bfloat16 bits of float32 values, round to nearest even (the bf16 KV rounding)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_rne_n(_p(a), a.size, _p(out))
    return out


def bf16_to_f32(h: int) -> float:
    return float(lib().or_bf16_to_f32(C.c_uint16(h)))


def quantize(w: np.ndarray, variant: str = "a") -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    out = np.empty(w.size // 32 * 34, dtype=np.uint8)
    fn = lib().or_q8_quantize_a if variant == "a" else lib().or_q8_quantize_b
    fn(_p(w), w.size // 32, 32, _p(out))
    return out


def dequant(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(blocks.size // 34 * 32, dtype=np.float32)
    lib().or_q8_dequant(_p(blocks), blocks.size // 34, _p(out))
    return out


def matvec_lanes(w: np.ndarray, x: np.ndarray, rows: int, lanes: int = 8) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib().or_q8_matvec_lanes(_p(w), _p(x), _p(y), x.size, rows, lanes)
    return y


def matvec_f64(w: np.ndarray, x: np.ndarray, rows: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float64)
    lib().or_q8_matvec_f64(_p(w), _p(x), _p(y), x.size, rows)
    return y


def gelu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.array(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    lib().or_gelu_mul(_p(g), _p(u), g.size)
    return g


def argmax(v: np.ndarray):
    v = np.ascontiguousarray(v, dtype=np.float32)
    i, val = C.c_uint32(), C.c_float()
    lib().or_argmax(_p(v), v.size, C.byref(i), C.byref(val))
    return int(i.value), float(val.value)


def rms_norm_into(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_rms_norm_into(_p(x), _p(w), _p(out), x.size, C.c_float(eps))
    return out


def rms_norm_inplace(x, w, eps=1e-6):
    v = np.array(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().or_rms_norm_inplace(_p(v), _p(w), v.size, C.c_float(eps))
    return v


def rms_norm_heads(x, w, heads, eps=1e-6):
    v = np.array(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().or_rms_norm_heads(_p(v), _p(w), heads, w.size, C.c_float(eps))
    return v


def rope_inv_freq(head_dim, theta):
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().or_rope_inv_freq(head_dim, C.c_float(theta), _p(out))
    return out


def rope_table(inv, pos):
    inv = np.ascontiguousarray(inv, dtype=np.float32)
    c = np.empty_like(inv)
    s = np.empty_like(inv)
    lib().or_rope_table(_p(inv), inv.size, pos, _p(c), _p(s))
    return c, s


def apply_rope(x, heads, head_dim, c, s):
    v = np.array(x, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32)
    s = np.ascontiguousarray(s, dtype=np.float32)
    lib().or_apply_rope(_p(v), heads, head_dim, _p(c), _p(s))
    return v


def attention(q, keys, values, heads, head_dim, scale):
    q = np.ascontiguousarray(q, dtype=np.float32)
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(heads * head_dim, dtype=np.float32)
    rc = lib().or_attention(_p(q), _p(keys), _p(values), keys.shape[0], heads, head_dim, C.c_float(scale), _p(out))
    if rc:
        raise RuntimeError("Gemma 3 attention softmax failed")
    return out


class Model:
    """The whole-model oracle (src/gemma3.cpp executor restated) over a GGUF file."""

    def __init__(self, path: str, lanes: int = 8, lib_path: str | None = None, kv_f16: bool = False,
                 kv_bf16: bool = False):
        self.L = lib(lib_path)
        err = C.create_string_buffer(512)
        self.h = self.L.or_g3_open(str(path).encode(), lanes, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())
        if kv_f16:
            self.L.or_g3_set_kv_f16(self.h, 1)
        if kv_bf16:
            self.L.or_g3_set_kv_format(self.h, 2)
        info = G3Info()
        self.L.or_g3_get_info(self.h, C.byref(info))
        self.info = info

    def close(self):
        if self.h:
            self.L.or_g3_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reset(self):
        self.L.or_g3_reset(self.h)

    def decode(self, token: int, pos: int, want_logits: bool = True, logits: bool = False):
        d = self.info.embedding_length
        hidden = np.empty(d, dtype=np.float32)
        lg = np.empty(self.info.vocab_size, dtype=np.float32) if logits else None
        ai, av = C.c_uint32(), C.c_float()
        rc = self.L.or_g3_decode(self.h, token, pos, 1 if want_logits else 0, _p(hidden),
                                 _p(lg) if lg is not None else None, C.byref(ai), C.byref(av))
        if rc:
            raise RuntimeError(self.L.or_g3_error(self.h).decode())
        return dict(hidden=hidden, logits=lg, index=int(ai.value) if want_logits else None,
                    value=float(av.value) if want_logits else None)

    def decode_taps(self, token: int, pos: int, hist_cap: int, want_logits: bool = False):
        """decode() that also returns the attention sub-path's intermediates of every block
        (or_g3_set_taps): xn, q_proj, k_proj, v_proj, q_att, att, and keys/values [L, history, hd]
        oldest first (at most hist_cap rows per block), history [L]."""
        i = self.info
        nl, d, hd, qd = i.block_count, i.embedding_length, i.head_dim, i.head_count * i.head_dim
        t = dict(xn=np.zeros((nl, d), np.float32), q_proj=np.zeros((nl, qd), np.float32),
                 k_proj=np.zeros((nl, hd), np.float32), v_proj=np.zeros((nl, hd), np.float32),
                 q_att=np.zeros((nl, qd), np.float32), att=np.zeros((nl, qd), np.float32),
                 keys=np.zeros((nl, hist_cap, hd), np.float32), values=np.zeros((nl, hist_cap, hd), np.float32),
                 history=np.zeros(nl, np.uint32))
        taps = G3Taps(**{k: a.ctypes.data for k, a in t.items()}, hist_cap=hist_cap)
        self.L.or_g3_set_taps(self.h, C.byref(taps))
        try:
            r = self.decode(token, pos, want_logits=want_logits)
        finally:
            self.L.or_g3_set_taps(self.h, None)
        r.update(t)
        return r

    def generate(self, prompt, max_new: int):
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(max_new, 1), dtype=np.uint32)
        n = C.c_uint32()
        rc = self.L.or_g3_generate(self.h, _p(pr), pr.size, max_new, _p(out), C.byref(n))
        if rc:
            raise RuntimeError(self.L.or_g3_error(self.h).decode())
        return out[: n.value].copy()


def num_threads() -> int:
    return int(lib().or_num_threads())
