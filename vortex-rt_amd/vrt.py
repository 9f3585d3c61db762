"""ctypes binding of libvrt_hip.so (include/vrt_hip.h) for tests and the bench.

Loads the in-tree build (_build/libvrt_hip.so) and raises if it is missing: there is no
fallback path. Device memory is owned by DeviceBuffer objects (vrt_alloc / vrt_free).
"""
from __future__ import annotations

import ctypes as C
import weakref
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "_build", "libvrt_hip.so")

VRT_OK, VRT_ERR_INVALID, VRT_ERR_HIP, VRT_ERR_STATE, VRT_ERR_NUMERIC = 0, 1, 2, 3, 4
MEM_DEVICE, MEM_HOST = 0, 1
OPT_USE_GRAPH = 1
OPT_PERSISTENT = 2
OPT_QUERY_PERSISTENT = 3
OPT_TRACE = 4
OPT_KV_F16 = 5
OPT_KV_BF16 = 12
OPT_TEAM = 6
OPT_QUERY_TEAM = 7
OPT_FUSION = 8
OPT_Q8_LANES = 9
OPT_QUERY_Q8_LANES = 10
OPT_QUERY_TEAM_POSITIONS = 11
OPT_QUERY_TEAM_CHUNKED = 13


class VrtError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class ArgmaxResult(C.Structure):
    _fields_ = [("index", C.c_uint32), ("value", C.c_float)]


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("device_index", C.c_uint32),
                ("vendor_id", C.c_uint32), ("device_id", C.c_uint32), ("subgroup_size", C.c_uint32),
                ("compute_units", C.c_uint32), ("fp16", C.c_uint32), ("int8", C.c_uint32),
                ("storage8", C.c_uint32), ("storage16", C.c_uint32), ("device_local_bytes", C.c_uint64),
                ("l2_bytes", C.c_uint64)]


class G3Config(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "context_length", "embedding_length", "block_count", "feed_forward_length", "head_count",
        "head_count_kv", "head_dim", "value_dim", "vocab_size", "sliding_window")] + \
        [("rms_epsilon", C.c_float), ("global_rope_base", C.c_float), ("local_rope_base", C.c_float)]


class G3Layer(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                          "ffn_down")] + \
        [(n, C.c_void_p) for n in ("attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm",
                                   "post_ffw_norm")]


class G3Desc(C.Structure):
    _fields_ = [("config", G3Config), ("arena", C.c_void_p), ("arena_bytes", C.c_uint64),
                ("token_embd", C.c_uint64), ("output_norm", C.c_void_p), ("layers", C.POINTER(G3Layer)),
                ("eos_token_id", C.c_uint32)]


# Every symbol include/vrt_hip.h declares, with its ctypes signature.
_P, _U32, _U64, _I, _F = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float
SIGNATURES = {
    "vrt_last_error": (C.c_char_p, []),
    "vrt_ctx_create": (_I, [C.c_char_p, C.POINTER(_P)]),
    "vrt_ctx_destroy": (_I, [_P]),
    "vrt_ctx_info": (_I, [_P, C.POINTER(DeviceInfo)]),
    "vrt_alloc": (_I, [_P, _U64, _U32, C.POINTER(_P)]),
    "vrt_free": (_I, [_P, _P]),
    "vrt_memcpy": (_I, [_P, _P, _P, _U64]),
    "vrt_memset": (_I, [_P, _P, _I, _U64]),
    "vrt_sync": (_I, [_P]),
    "vrt_stream": (_I, [_P, C.POINTER(_P)]),
    "vrt_event_create": (_I, [_P, C.POINTER(_P)]),
    "vrt_event_record": (_I, [_P, _P]),
    "vrt_event_elapsed_ms": (_I, [_P, _P, C.POINTER(_F)]),
    "vrt_event_destroy": (_I, [_P]),
    "vrt_q8_matvec": (_I, [_P, _P, _U64, _U32, _P, _P, _U32, _U32]),
    "vrt_q8_matvec_multi": (_I, [_P, _P, _U64, _U32, _P, _P, _U32, _P, _P]),
    "vrt_q8_ffn": (_I, [_P, _P, _U64, _U32, _U32, _U32, _U32, _U32, _U32, _P, _P, _U64, _P]),
    "vrt_q8_ffn_noalloc": (_I, [_P, _P, _U64, _U32, _U32, _U32, _U32, _U32, _U32, _P, _P]),
    "vrt_gelu_mul": (_I, [_P, _P, _P, _U32]),
    "vrt_argmax": (_I, [_P, _P, _U32, _P]),
    "vrt_q8_quantize": (_I, [_P, _P, _U64, _U32, _P]),
    "vrt_q8_dequantize": (_I, [_P, _P, _U64, _P]),
    "vrt_g3_create": (_I, [_P, C.POINTER(G3Desc), C.POINTER(_P)]),
    "vrt_g3_destroy": (_I, [_P]),
    "vrt_g3_reset": (_I, [_P]),
    "vrt_g3_decode": (_I, [_P, _U32, _U32, _U32, C.POINTER(ArgmaxResult), _P]),
    "vrt_g3_prefill": (_I, [_P, _P, _U32, _U32, C.POINTER(ArgmaxResult), _P]),
    "vrt_g3_logits": (_I, [_P, _P, _U32]),
    "vrt_g3_generate": (_I, [_P, _P, _U32, _U32, _P, C.POINTER(_U32)]),
    "vrt_g3_start": (_I, [_P, _P, _U32, _U32]),
    "vrt_g3_step": (_I, [_P, _U32]),
    "vrt_g3_collect": (_I, [_P, _P, C.POINTER(_U32)]),
    "vrt_g3_forced": (_I, [_P, _P, _U32, _U32, _P]),
    "vrt_g3_set_option": (_I, [_P, _U32, _U32]),
    "vrt_g3_get_option": (_I, [_P, _U32, C.POINTER(_U32)]),
    "vrt_g3_time_lm_head": (_I, [_P, _U32, C.POINTER(_F)]),
    "vrt_g3_read_trace": (_I, [_P, _P, _U64, C.POINTER(_U32), C.POINTER(_U32)]),
    "vrt_g3_read_exchange": (_I, [_P, _U32, _P, _U64, C.POINTER(_U64)]),
    "vrt_g3_batch_create": (_I, [_P, _U32, _U32, C.POINTER(_P)]),
    "vrt_g3_batch_destroy": (_I, [_P]),
    "vrt_g3_batch_reset": (_I, [_P, _U32]),
    "vrt_g3_batch_step": (_I, [_P, _P, _P, _U32, _P]),
    "vrt_g3_batch_position": (_I, [_P, _U32, C.POINTER(_U32)]),
    "vrt_g3_batch_logits": (_I, [_P, _U32, _P, _U32]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != VRT_OK:
        raise VrtError(rc, lib().vrt_last_error().decode(errors="replace"))


def ptr(a):
    if a is None:
        return None
    if isinstance(a, DeviceBuffer):
        return a.ptr
    if isinstance(a, int):
        return a
    return a.ctypes.data_as(C.c_void_p).value


class Context:
    """VulkanContext replacement (include/vortexrt/vulkan_context.hpp:43-60)."""

    def __init__(self, selector: str = ""):
        h = C.c_void_p()
        check(lib().vrt_ctx_create(selector.encode(), C.byref(h)))
        self.h = h.value
        info = DeviceInfo()
        check(lib().vrt_ctx_info(self.h, C.byref(info)))
        self.info = info
        self._children = weakref.WeakSet()   # executors and buffers: released before the context

    def close(self):
        if getattr(self, "h", None):
            for c in list(getattr(self, "_children", ())):
                c.close()
            lib().vrt_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def sync(self):
        check(lib().vrt_sync(self.h))

    def alloc(self, nbytes: int, kind: int = MEM_DEVICE) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes, kind)

    def upload(self, arr: np.ndarray, kind: int = MEM_DEVICE) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(self, arr.nbytes, kind)
        b.write(arr)
        return b

    def event(self):
        h = C.c_void_p()
        check(lib().vrt_event_create(self.h, C.byref(h)))
        return h.value

    def record(self, ev):
        check(lib().vrt_event_record(self.h, ev))

    @staticmethod
    def elapsed_ms(a, b) -> float:
        ms = C.c_float()
        check(lib().vrt_event_elapsed_ms(a, b, C.byref(ms)))
        return float(ms.value)


class DeviceBuffer:
    """Buffer replacement (include/vortexrt/buffer.hpp:11-42)."""

    def __init__(self, ctx: Context, nbytes: int, kind: int = MEM_DEVICE):
        self.ctx, self.nbytes, self.kind = ctx, int(nbytes), kind
        p = C.c_void_p()
        check(lib().vrt_alloc(ctx.h, self.nbytes, kind, C.byref(p)))
        self.ptr = p.value
        ctx._children.add(self)

    def write(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(lib().vrt_memcpy(self.ctx.h, self.ptr + offset, ptr(arr), arr.nbytes))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(lib().vrt_memcpy(self.ctx.h, ptr(out), self.ptr + offset, out.nbytes))
        return out

    def close(self):
        self.free()

    def free(self):
        if getattr(self, "ptr", None):
            lib().vrt_free(self.ctx.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- kernels ------------------------------------------------------------------------------

def q8_matvec(ctx, w: DeviceBuffer, off: int, x: DeviceBuffer, y: DeviceBuffer, k: int, rows: int, w_bytes=None):
    check(lib().vrt_q8_matvec(ctx.h, w.ptr, w.nbytes if w_bytes is None else w_bytes, off, x.ptr, y.ptr, k, rows))


def q8_matvec_multi(ctx, w: DeviceBuffer, offs, dims, k: int, x: DeviceBuffer, y: DeviceBuffer):
    o = np.asarray(offs, dtype=np.uint32)
    d = np.asarray(dims, dtype=np.uint32)
    check(lib().vrt_q8_matvec_multi(ctx.h, w.ptr, w.nbytes, len(o), ptr(o), ptr(d), k, x.ptr, y.ptr))


def q8_ffn(ctx, w, gate_off, up_off, down_off, k, ffn, out, x, ws, y):
    check(lib().vrt_q8_ffn(ctx.h, w.ptr, w.nbytes, gate_off, up_off, down_off, k, ffn, out, x.ptr, ws.ptr, ws.nbytes,
                           y.ptr))


def q8_ffn_noalloc(ctx, w, gate_off, up_off, down_off, k, ffn, out, x, y):
    """vrt_q8_ffn on the library's static per-device workspace (no allocation)."""
    check(lib().vrt_q8_ffn_noalloc(ctx.h, w.ptr, w.nbytes, gate_off, up_off, down_off, k, ffn, out, x.ptr, y.ptr))


def gelu_mul(ctx, gate: DeviceBuffer, up: DeviceBuffer, n: int):
    check(lib().vrt_gelu_mul(ctx.h, gate.ptr, up.ptr, n))


def argmax(ctx, x: DeviceBuffer, n: int, out: DeviceBuffer):
    check(lib().vrt_argmax(ctx.h, x.ptr, n, out.ptr))


def q8_quantize(ctx, x: DeviceBuffer, n: int, variant: int, out: DeviceBuffer):
    check(lib().vrt_q8_quantize(ctx.h, x.ptr, n, variant, out.ptr))


def q8_dequantize(ctx, blocks: DeviceBuffer, nblocks: int, out: DeviceBuffer):
    check(lib().vrt_q8_dequantize(ctx.h, blocks.ptr, nblocks, out.ptr))


# ---- Gemma 3 executor ----------------------------------------------------------------------

class Gemma3:
    """Executor over a GGUF file: parses it (gguf.py), uploads the tensor-data section as the
    device arena and builds the vrt_g3 executor (Gemma3Model's device half)."""

    def __init__(self, ctx: Context, path: str):
        import gguf as G
        self.ctx = ctx
        f = G.GgufFile.open(path)
        self.file = f
        if f.meta_str("general.architecture") != "gemma3":
            raise RuntimeError("Gemma3Model requires general.architecture=gemma3")

        def req(key):
            v = f.meta_u64(key)
            if v is None or v > 0xFFFFFFFF:
                raise RuntimeError("Missing/invalid Gemma 3 metadata: " + key)
            return v

        cfg = G3Config()
        cfg.context_length = req("gemma3.context_length")
        cfg.embedding_length = req("gemma3.embedding_length")
        cfg.block_count = req("gemma3.block_count")
        cfg.feed_forward_length = req("gemma3.feed_forward_length")
        cfg.head_count = req("gemma3.attention.head_count")
        cfg.head_count_kv = req("gemma3.attention.head_count_kv")
        cfg.head_dim = req("gemma3.attention.key_length")
        cfg.value_dim = req("gemma3.attention.value_length")
        eps = f.meta_f64("gemma3.attention.layer_norm_rms_epsilon")
        if eps is None:
            raise RuntimeError("Missing Gemma 3 metadata: gemma3.attention.layer_norm_rms_epsilon")
        cfg.rms_epsilon = eps
        sw = f.meta_u64("gemma3.attention.sliding_window")
        cfg.sliding_window = sw if sw is not None and sw <= 0xFFFFFFFF else 0
        rb = f.meta_f64("gemma3.rope.freq_base")
        cfg.global_rope_base = rb if rb is not None and np.isfinite(rb) and rb > 0 else 1.0e6
        cfg.local_rope_base = 1.0e4
        emb = f.tensors.get("token_embd.weight")
        if emb is None or emb.type != 8 or len(emb.dims) != 2 or emb.dims[0] != cfg.embedding_length:
            raise RuntimeError("Unsupported token_embd.weight layout")
        cfg.vocab_size = emb.dims[1]
        self.config = cfg
        self.eos = f.meta_u64("tokenizer.ggml.eos_token_id")
        self.eos = 1 if self.eos is None else self.eos
        data = f.data_view()
        self.arena = DeviceBuffer(ctx, len(data))
        # upload in chunks from the memory map
        chunk = 64 << 20
        arr = np.frombuffer(data, dtype=np.uint8)
        for o in range(0, len(arr), chunk):
            part = np.ascontiguousarray(arr[o:o + chunk])
            check(lib().vrt_memcpy(ctx.h, self.arena.ptr + o, ptr(part), part.nbytes))
        self._keep = []

        def f32(name):
            t = f.tensors.get(name)
            if t is None:
                raise RuntimeError("Missing Gemma 3 tensor: " + name)
            a = f.read_f32(name)
            self._keep.append(a)
            return ptr(a)

        layers = (G3Layer * cfg.block_count)()
        for l in range(cfg.block_count):
            p = f"blk.{l}."
            Ly = layers[l]
            for fld, nm in (("attn_q", "attn_q"), ("attn_k", "attn_k"), ("attn_v", "attn_v"),
                            ("attn_output", "attn_output"), ("ffn_gate", "ffn_gate"), ("ffn_up", "ffn_up"),
                            ("ffn_down", "ffn_down")):
                t = f.tensors.get(p + nm + ".weight")
                if t is None or t.type != 8:
                    raise RuntimeError("Missing Gemma 3 tensor: " + p + nm + ".weight")
                setattr(Ly, fld, t.offset)
            for fld, nm in (("attn_norm", "attn_norm"), ("attn_q_norm", "attn_q_norm"),
                            ("attn_k_norm", "attn_k_norm"), ("post_attention_norm", "post_attention_norm"),
                            ("ffn_norm", "ffn_norm"), ("post_ffw_norm", "post_ffw_norm")):
                setattr(Ly, fld, f32(p + nm + ".weight"))
        desc = G3Desc()
        desc.config = cfg
        desc.arena = self.arena.ptr
        desc.arena_bytes = len(data)
        desc.token_embd = emb.offset
        desc.output_norm = f32("output_norm.weight")
        desc.layers = layers
        desc.eos_token_id = self.eos
        h = C.c_void_p()
        check(lib().vrt_g3_create(ctx.h, C.byref(desc), C.byref(h)))
        self.h = h.value
        self.kv_f16 = False    # 16-bit KV entries (fp16 or bf16)
        self._batches = weakref.WeakSet()   # batched decoders over this executor: closed first
        ctx._children.add(self)
        self._keep.clear()

    def close(self):
        if getattr(self, "h", None):
            for b in list(getattr(self, "_batches", ())):
                b.close()
            check(lib().vrt_g3_destroy(self.h))
            self.h = None
        if getattr(self, "arena", None) is not None:
            self.arena.free()
            self.arena = None

    def __del__(self):
        self.close()

    def set_graph(self, on: bool):
        check(lib().vrt_g3_set_option(self.h, OPT_USE_GRAPH, 1 if on else 0))

    def set_persistent(self, on: bool):
        """Persistent decode kernel (default when available) or the multi-kernel step."""
        check(lib().vrt_g3_set_option(self.h, OPT_PERSISTENT, 1 if on else 0))

    def set_team(self, on: bool):
        """Phase-team persistent kernel for positions below its limit (default on)."""
        check(lib().vrt_g3_set_option(self.h, OPT_TEAM, 1 if on else 0))

    def team_available(self) -> bool:
        return lib().vrt_g3_set_option(self.h, OPT_QUERY_TEAM, 0) == VRT_OK

    def team_enabled(self) -> bool:
        """Whether steps may run on the team kernel (set_team; it runs them when also available)."""
        return bool(self.get_option(OPT_TEAM))

    def team_positions(self) -> int:
        """Steps at positions below this run on the team kernel (0: unavailable)."""
        return self.get_option(OPT_QUERY_TEAM_POSITIONS)

    def team_chunked_from(self) -> int:
        """Team-kernel steps from this position on run its chunked-history variant."""
        return self.get_option(OPT_QUERY_TEAM_CHUNKED)

    def set_trace(self, on: bool):
        check(lib().vrt_g3_set_option(self.h, OPT_TRACE, 1 if on else 0))

    def get_option(self, option: int) -> int:
        v = C.c_uint32()
        check(lib().vrt_g3_get_option(self.h, option, C.byref(v)))
        return int(v.value)

    def set_fusion(self, on: bool):
        """Projection fusion (default on); off runs the unfused multi-kernel sequence."""
        check(lib().vrt_g3_set_option(self.h, OPT_FUSION, 1 if on else 0))

    def set_q8_lanes(self, lanes: int):
        """Row-slot width request of the projections: 0 (auto), 8, 16, 32 or 64."""
        check(lib().vrt_g3_set_option(self.h, OPT_Q8_LANES, lanes))

    def q8_lanes(self) -> int:
        """Lanes per row the embedding-width projections run with."""
        return self.get_option(OPT_QUERY_Q8_LANES)

    def set_kv_f16(self, on: bool):
        """fp16 KV cache (keys and values rounded to fp16 as they enter it); resets the cache.
        Off: fp32 entries."""
        if on:
            check(lib().vrt_g3_set_option(self.h, OPT_KV_F16, 1))
        else:
            self.set_kv_format("f32")
        self.kv_f16 = bool(on)

    def set_kv_bf16(self, on: bool):
        """bf16 KV cache (keys and values rounded to bfloat16 as they enter it); resets the
        cache. Off: fp32 entries."""
        if on:
            check(lib().vrt_g3_set_option(self.h, OPT_KV_BF16, 1))
        else:
            self.set_kv_format("f32")
        self.kv_f16 = bool(on)

    def set_kv_format(self, fmt: str):
        """KV cache entries "f32", "f16" or "bf16" (resets the cache when it changes)."""
        if fmt == "f16":
            check(lib().vrt_g3_set_option(self.h, OPT_KV_F16, 1))
        elif fmt == "bf16":
            check(lib().vrt_g3_set_option(self.h, OPT_KV_BF16, 1))
        elif fmt == "f32":
            check(lib().vrt_g3_set_option(self.h, OPT_KV_F16, 0))
            check(lib().vrt_g3_set_option(self.h, OPT_KV_BF16, 0))
        else:
            raise ValueError(f"unknown KV format {fmt!r}")
        self.kv_f16 = fmt != "f32"

    def kv_format(self) -> str:
        if self.get_option(OPT_KV_BF16):
            return "bf16"
        return "f16" if self.get_option(OPT_KV_F16) else "f32"

    def read_trace(self) -> np.ndarray:
        """[nwg, slots] s_memrealtime ticks (100 MHz) of the last persistent launch's first step."""
        nwg, slots = C.c_uint32(), C.c_uint32()
        buf = np.zeros(1 << 20, dtype=np.uint64)
        check(lib().vrt_g3_read_trace(self.h, ptr(buf), buf.size, C.byref(nwg), C.byref(slots)))
        return buf[: nwg.value * slots.value].reshape(nwg.value, slots.value).copy()

    def read_exchange(self, which: int):
        """(values, tags) of a persistent-kernel exchange buffer (0 qkv, 1 partials, 2 o, 3 g, 4 f, 5 argmax)."""
        buf = np.zeros(1 << 20, dtype=np.uint64)
        n = C.c_uint64()
        check(lib().vrt_g3_read_exchange(self.h, which, ptr(buf), buf.size, C.byref(n)))
        w = buf[: n.value]
        return (w & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32), (w >> np.uint64(32)).astype(np.uint32)

    def persistent_available(self) -> bool:
        return lib().vrt_g3_set_option(self.h, OPT_QUERY_PERSISTENT, 0) == VRT_OK

    def reset(self):
        check(lib().vrt_g3_reset(self.h))

    def decode(self, token: int, pos: int, top_k: int = 1, hidden: bool = False):
        r = ArgmaxResult()
        hbuf = np.empty(self.config.embedding_length, dtype=np.float32) if hidden else None
        check(lib().vrt_g3_decode(self.h, token, pos, top_k, C.byref(r), ptr(hbuf)))
        return (int(r.index), float(r.value)), hbuf

    def prefill(self, tokens, top_k: int = 1, hidden: bool = False):
        """Batched prefill of positions 0..n-1; returns ((index, value), hidden or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        r = ArgmaxResult()
        hbuf = np.empty(self.config.embedding_length, dtype=np.float32) if hidden else None
        check(lib().vrt_g3_prefill(self.h, ptr(t), t.size, top_k, C.byref(r), ptr(hbuf)))
        return (int(r.index), float(r.value)), hbuf

    def logits(self) -> np.ndarray:
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        check(lib().vrt_g3_logits(self.h, ptr(out), out.size))
        return out

    def generate(self, prompt, max_new: int) -> np.ndarray:
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(1, max_new), dtype=np.uint32)
        n = C.c_uint32()
        check(lib().vrt_g3_generate(self.h, ptr(pr), pr.size, max_new, ptr(out), C.byref(n)))
        return out[: n.value].copy()

    def start(self, prompt, max_new: int):
        pr = np.ascontiguousarray(prompt, dtype=np.uint32)
        self._gen_max = max_new
        check(lib().vrt_g3_start(self.h, ptr(pr), pr.size, max_new))

    def step(self, n: int):
        check(lib().vrt_g3_step(self.h, n))

    def collect(self) -> np.ndarray:
        out = np.empty(max(1, self._gen_max), dtype=np.uint32)
        n = C.c_uint32()
        check(lib().vrt_g3_collect(self.h, ptr(out), C.byref(n)))
        return out[: n.value].copy()

    def forced(self, tokens, first_logit_step: int):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros(t.size, dtype=np.dtype([("index", np.uint32), ("value", np.float32)]))
        check(lib().vrt_g3_forced(self.h, ptr(t), t.size, first_logit_step, ptr(out)))
        return out

    def time_lm_head(self, iters: int) -> float:
        us = C.c_float()
        check(lib().vrt_g3_time_lm_head(self.h, iters, C.byref(us)))
        return float(us.value)


class Gemma3Batch:
    """Batched greedy decode over independent sequences that share a Gemma3 executor's weights
    (vrt_g3_batch_*): each sequence has its own KV cache and position."""

    def __init__(self, model: "Gemma3", max_seqs: int, max_ctx: int):
        self.h = None
        self.model = model
        self.max_seqs = max_seqs
        h = C.c_void_p()
        check(lib().vrt_g3_batch_create(model.h, max_seqs, max_ctx, C.byref(h)))
        self.h = h.value
        model._batches.add(self)

    def close(self):
        if getattr(self, "h", None):
            check(lib().vrt_g3_batch_destroy(self.h))
            self.h = None

    def __del__(self):
        self.close()

    def reset(self, seq=None):
        check(lib().vrt_g3_batch_reset(self.h, 0xFFFFFFFF if seq is None else seq))

    def position(self, seq: int) -> int:
        p = C.c_uint32()
        check(lib().vrt_g3_batch_position(self.h, seq, C.byref(p)))
        return p.value

    def step(self, seqs, tokens):
        """One step: sequence seqs[i] consumes tokens[i]; returns (indices, values)."""
        s = np.ascontiguousarray(seqs, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        if s.size != t.size:
            raise ValueError("seqs and tokens differ in length")
        out = np.zeros(s.size, dtype=np.dtype([("index", np.uint32), ("value", np.float32)]))
        check(lib().vrt_g3_batch_step(self.h, ptr(s), ptr(t), s.size, ptr(out)))
        return out["index"].copy(), out["value"].copy()

    def logits(self, row: int) -> np.ndarray:
        out = np.empty(self.model.config.vocab_size, dtype=np.float32)
        check(lib().vrt_g3_batch_logits(self.h, row, ptr(out), out.size))
        return out

    def generate(self, prompts, max_new: int, starts=None, eos=None):
        """Continuous batching: sequence i joins at step starts[i] (default 0), feeds its prompt
        one token per step, then its own greedy tokens, until max_new tokens or EOS. Returns the
        generated ids per sequence."""
        n = len(prompts)
        if n > self.max_seqs:
            raise ValueError("more prompts than sequences")
        starts = [0] * n if starts is None else list(starts)
        feed = [list(np.asarray(p, dtype=np.uint32)) for p in prompts]
        gen = [[] for _ in range(n)]
        done = [False] * n
        for i in range(n):
            self.reset(i)
        step = 0
        while not all(done):
            rows = [i for i in range(n) if not done[i] and step >= starts[i]]
            if rows:
                toks = [feed[i][0] if feed[i] else gen[i][-1] for i in rows]
                idx, _ = self.step(rows, toks)
                for i, r in zip(rows, idx):
                    if feed[i]:
                        feed[i].pop(0)
                        if feed[i]:
                            continue
                    gen[i].append(int(r))
                    if len(gen[i]) >= max_new or (eos is not None and int(r) == eos):
                        done[i] = True
            step += 1
        return [np.asarray(g, dtype=np.uint32) for g in gen]

