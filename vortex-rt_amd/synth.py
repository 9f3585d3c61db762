"""Synthetic Gemma-3-shape Q8_0 models and inputs.

The reference ships no RNG (its tests use sin/cos fixtures), so the workloads define
one: SplitMix64 -> float64 Box-Muller -> float32, seeded per tensor from (model seed,
FNV-1a of the tensor name). The GGUF file written here is the shared artefact: the
oracle, this package's loader and the reference's own loader all read the same bytes.

Q8_0 quantisation follows the reference's quantiser of record bit for bit
(src/q8_test_main.cpp:18-41 f32_to_f16, :93-124 block loop): fp32 scale = amax/127,
a non-IEEE fp16 encode (ties half-up; a mantissa carry is OR-ed into the exponent
field and lost on odd exponents), q = clamp(nearbyint(v / scale), -127, 127).
Variant "b" is src/ffn_test_main.cpp:112-215 (divide by the dequantised scale,
amax == 0 -> scale 1).
"""
from __future__ import annotations

import numpy as np

from gguf import (GGML_F32, GGML_Q8_0, GgufFile, GgufWriter, T_ARR, T_BOOL, T_F32, T_I32, T_STR, T_U32)

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_seed(seed: int, name: str) -> int:
    return (fnv1a64(name) ^ ((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF


def splitmix64(seed: int, start: int, n: int) -> np.ndarray:
    """Outputs start .. start+n-1 of SplitMix64 seeded with `seed`."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + _GOLDEN * (np.arange(start + 1, start + n + 1, dtype=np.uint64))
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal_f32(seed: int, n: int, std: float = 1.0, mean: float = 0.0, chunk: int = 1 << 20,
               start: int = 0) -> np.ndarray:
    """Values start .. start+n-1 (start even) of the float32 N(mean, std^2) stream of `seed`:
    pairs of SplitMix64 words -> Box-Muller in float64."""
    assert start % 2 == 0
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2
    for p0 in range(0, pairs, chunk):
        m = min(chunk, pairs - p0)
        z = splitmix64(seed, start + 2 * p0, 2 * m).reshape(m, 2)
        u1 = ((z[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u2 = (z[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * np.pi * u2
        v = np.empty(2 * m, dtype=np.float64)
        v[0::2] = r * np.cos(t)
        v[1::2] = r * np.sin(t)
        v = v * std + mean
        lo, hi = 2 * p0, min(n, 2 * (p0 + m))
        out[lo:hi] = v[: hi - lo].astype(np.float32)
    return out


def uniform_ids(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n token ids uniform in [lo, hi) (multiply-shift on the top 32 bits)."""
    z = splitmix64(seed, 0, n) >> np.uint64(32)
    return (np.uint64(lo) + ((z * np.uint64(hi - lo)) >> np.uint64(32))).astype(np.uint32)


# ---------------------------------------------------------------------------------------
# Quantiser of record (numpy restatement, bit-exact)
# ---------------------------------------------------------------------------------------

def f32_to_f16_ref(f: np.ndarray) -> np.ndarray:
    """src/q8_test_main.cpp:18-41 vectorised."""
    x = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (x >> 16) & 0x8000
    mant = x & 0x7FFFFF
    exp = ((x >> 23) & 0xFF) - 127 + 15
    normal = sign | (np.clip(exp, 0, 31) << 10) | ((mant + 0x1000) >> 13)
    shift = np.clip(1 - exp, 0, 63)
    sub = sign + ((((mant | 0x800000) >> shift) + 0x1000) >> 13)
    out = np.where(exp >= 31, sign | 0x7C00, normal)
    out = np.where(exp <= 0, np.where(exp < -10, sign, sub), out)
    return out.astype(np.uint16)


def f16_to_f32_ref(h: np.ndarray) -> np.ndarray:
    """Exact IEEE half -> float (src/gguf.cpp:203-235)."""
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_q8_0(w: np.ndarray, variant: str = "a") -> np.ndarray:
    """Quantise a float32 array (size % 32 == 0) into Q8_0 bytes [nblocks * 34]."""
    v = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, 32)
    nb = v.shape[0]
    amax = np.zeros(nb, dtype=np.float32)
    for k in range(32):  # std::max(abs_max, fabs(v)) in element order
        a = np.abs(v[:, k])
        amax = np.where(amax < a, a, amax)
    if variant == "a":
        scale = (amax / np.float32(127.0)).astype(np.float32)
    else:
        scale = np.where(amax == 0, np.float32(1.0), amax / np.float32(127.0)).astype(np.float32)
    half = f32_to_f16_ref(scale)
    div = scale if variant == "a" else f16_to_f32_ref(half)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = (v / div[:, None]).astype(np.float32)
    n = np.rint(r)
    # static_cast<int> of NaN or |n| >= 2^31 is INT_MIN on x86-64, which the clamp maps to -127
    with np.errstate(invalid="ignore"):
        out_of_range = ~(np.abs(n) < np.float32(2147483648.0))
    q = np.where(out_of_range, -127, np.clip(np.where(out_of_range, 0, n), -127, 127))
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 0:2] = half.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)
    scale = f16_to_f32_ref(b[:, 0:2].copy().view(np.uint16).reshape(-1))
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (scale[:, None] * q).astype(np.float32).reshape(-1)


def q8_matrix_chunks(seed: int, name: str, rows: int, cols: int, std: float = 0.02, variant: str = "a",
                     chunk_values: int = 1 << 21):
    """Yields the Q8_0 bytes of a [rows x cols] N(0, std^2) matrix, quantised along cols, in
    row-aligned chunks (same bytes as q8_matrix)."""
    ts = tensor_seed(seed, name)
    step = max(cols, (chunk_values // cols) * cols)
    step += step % 2 * cols  # keep chunk starts even in the value stream
    total = rows * cols
    for v0 in range(0, total, step):
        n = min(step, total - v0)
        yield quantize_q8_0(normal_f32(ts, n, std, start=v0), variant)


def q8_matrix(seed: int, name: str, rows: int, cols: int, std: float = 0.02, variant: str = "a") -> np.ndarray:
    """Q8_0 bytes of a [rows x cols] N(0, std^2) matrix quantised along cols."""
    return np.concatenate(list(q8_matrix_chunks(seed, name, rows, cols, std, variant)))


# ---------------------------------------------------------------------------------------
# Gemma 3 shapes
# ---------------------------------------------------------------------------------------

GEMMA3_270M = dict(n_layers=18, d_model=640, n_heads=4, head_dim=256, ffn=2048, vocab=262144,
                   context=32768, window=512, eps=1e-6, rope_global=1.0e6)


def write_gemma3_gguf(path, seed: int = 0, n_layers: int = 18, d_model: int = 640, n_heads: int = 4,
                      head_dim: int = 256, ffn: int = 2048, vocab: int = 262144, context: int = 32768,
                      window: int = 512, eps: float = 1e-6, rope_global: float = 1.0e6,
                      weight_std: float = 0.02, norm_std: float = 0.1, with_window: bool = True,
                      embd_std: float | None = None, eos: int = 1):
    """A random-init Gemma-3-architecture GGUF carrying every key the reference executor
    requires (src/gemma3.cpp:174-257, :289-313) and the tensor set of :456-505.
    Norm weights are stored as 1 + N(0, norm_std^2): Gemma GGUFs fold the (1 + w)
    convention into the stored value (src/gemma3.cpp:991-996). embd_std (default
    weight_std) sets the tied embedding / LM head alone, so a model whose block
    projections are all zero (weight_std=0) still has a non-trivial embedding. eos sets
    tokenizer.ggml.eos_token_id (the weights do not depend on it)."""
    w = GgufWriter(alignment=32)
    w.add("general.architecture", T_STR, "gemma3")
    w.add("general.alignment", T_U32, 32)
    w.add("gemma3.context_length", T_U32, context)
    w.add("gemma3.embedding_length", T_U32, d_model)
    w.add("gemma3.block_count", T_U32, n_layers)
    w.add("gemma3.feed_forward_length", T_U32, ffn)
    w.add("gemma3.attention.head_count", T_U32, n_heads)
    w.add("gemma3.attention.head_count_kv", T_U32, 1)
    w.add("gemma3.attention.key_length", T_U32, head_dim)
    w.add("gemma3.attention.value_length", T_U32, head_dim)
    w.add("gemma3.attention.layer_norm_rms_epsilon", T_F32, eps)
    if with_window:
        w.add("gemma3.attention.sliding_window", T_U32, window)
    w.add("gemma3.rope.freq_base", T_F32, rope_global)
    pieces = ["<pad>", "<eos>", "<bos>", "<unk>"]
    types = [3, 3, 3, 2]
    pieces += [f"<0x{b:02X}>" for b in range(256)]
    types += [6] * 256
    pieces += [f"▁t{i}" for i in range(len(pieces), vocab)]
    types += [1] * (vocab - len(types))
    pieces, types = pieces[:vocab], types[:vocab]
    w.add("tokenizer.ggml.model", T_STR, "llama")
    w.add("tokenizer.ggml.tokens", T_ARR, (T_STR, pieces))
    w.add("tokenizer.ggml.scores", T_ARR, (T_F32, np.linspace(0, -1, vocab, dtype=np.float32)))
    w.add("tokenizer.ggml.token_type", T_ARR, (T_I32, np.asarray(types, dtype=np.int32)))
    w.add("tokenizer.ggml.bos_token_id", T_U32, 2)
    w.add("tokenizer.ggml.eos_token_id", T_U32, eos)
    w.add("tokenizer.ggml.unknown_token_id", T_U32, 3)

    def q8(name, rows, cols, std=weight_std):
        w.add_tensor(name, [cols, rows], GGML_Q8_0, rows * cols // 32 * 34,
                     lambda: q8_matrix_chunks(seed, name, rows, cols, std))

    def f32norm(name, n):
        w.add_tensor(name, [n], GGML_F32, 4 * n,
                     lambda: normal_f32(tensor_seed(seed, name), n, norm_std, 1.0))

    q8("token_embd.weight", vocab, d_model, weight_std if embd_std is None else embd_std)
    f32norm("output_norm.weight", d_model)
    qw = n_heads * head_dim
    for l in range(n_layers):
        p = f"blk.{l}."
        f32norm(p + "attn_norm.weight", d_model)
        f32norm(p + "attn_q_norm.weight", head_dim)
        f32norm(p + "attn_k_norm.weight", head_dim)
        f32norm(p + "post_attention_norm.weight", d_model)
        f32norm(p + "ffn_norm.weight", d_model)
        f32norm(p + "post_ffw_norm.weight", d_model)
        q8(p + "attn_q.weight", qw, d_model)
        q8(p + "attn_k.weight", head_dim, d_model)
        q8(p + "attn_v.weight", head_dim, d_model)
        q8(p + "attn_output.weight", d_model, qw)
        q8(p + "ffn_gate.weight", ffn, d_model)
        q8(p + "ffn_up.weight", ffn, d_model)
        q8(p + "ffn_down.weight", d_model, ffn)
    w.write(path)
    return path


def edit_gguf(src: str, dst: str, q8_scale_exp: dict | None = None, q8_zero=(), f32: dict | None = None) -> str:
    """Writes a copy of the GGUF file `src` to `dst` with some tensor payloads changed in place
    (header, metadata and layout untouched):
      q8_scale_exp {name: k}  every Q8_0 block scale of the tensor times 2**k, by moving the
                              fp16 exponent (exact; every nonzero scale must stay a normal half);
      q8_zero [name, ...]     every block scale of the tensor set to +0 (the matrix becomes zero);
      f32 {name: array}       the F32 tensor's values replaced."""
    q8_scale_exp = q8_scale_exp or {}
    f32 = f32 or {}
    f = GgufFile.open(src)
    try:
        buf = bytearray(f._mm[:])
        for name, k in q8_scale_exp.items():
            t = f.tensors[name]
            assert t.type == GGML_Q8_0, name
            start = f.data_offset + t.offset
            blk = np.frombuffer(buf, dtype=np.uint8, count=t.nbytes(), offset=start).reshape(-1, 34).copy()
            h = blk[:, 0].astype(np.uint16) | (blk[:, 1].astype(np.uint16) << 8)
            e = (h >> 10) & 0x1F
            nz = (h & 0x7FFF) != 0
            assert np.all(~nz | ((e >= 1) & (e <= 30))), f"{name}: scale not a normal half"
            ne = e.astype(np.int32) + k
            assert np.all(~nz | ((ne >= 1) & (ne <= 30))), f"{name}: scaled exponent out of range"
            h2 = np.where(nz, (h & 0x83FF) | (ne.astype(np.uint16) << 10), h).astype(np.uint16)
            blk[:, 0] = (h2 & 0xFF).astype(np.uint8)
            blk[:, 1] = (h2 >> 8).astype(np.uint8)
            buf[start:start + blk.size] = blk.tobytes()
        for name in q8_zero:
            t = f.tensors[name]
            assert t.type == GGML_Q8_0, name
            start = f.data_offset + t.offset
            blk = np.frombuffer(buf, dtype=np.uint8, count=t.nbytes(), offset=start).reshape(-1, 34).copy()
            blk[:, 0:2] = 0
            buf[start:start + blk.size] = blk.tobytes()
        for name, arr in f32.items():
            t = f.tensors[name]
            assert t.type == GGML_F32, name
            a = np.ascontiguousarray(arr, dtype=np.float32)
            assert a.nbytes == t.nbytes(), name
            start = f.data_offset + t.offset
            buf[start:start + a.nbytes] = a.tobytes()
    finally:
        f.close()
    with open(dst, "wb") as fp:
        fp.write(buf)
    return dst


def write_tokenizer_gguf(path, pieces, scores, types, bos=2, eos=1, unk=3, add_space_prefix=None):
    """A metadata-only GGUF carrying a tokenizer vocabulary (tokenizer.ggml.* keys of
    src/gemma3.cpp:289-454), for the tokenizer tests; add_space_prefix None leaves the key out."""
    w = GgufWriter(alignment=32)
    w.add("general.architecture", T_STR, "gemma3")
    w.add("tokenizer.ggml.model", T_STR, "llama")
    w.add("tokenizer.ggml.tokens", T_ARR, (T_STR, list(pieces)))
    w.add("tokenizer.ggml.scores", T_ARR, (T_F32, np.asarray(scores, dtype=np.float32)))
    w.add("tokenizer.ggml.token_type", T_ARR, (T_I32, np.asarray(types, dtype=np.int32)))
    w.add("tokenizer.ggml.bos_token_id", T_U32, bos)
    w.add("tokenizer.ggml.eos_token_id", T_U32, eos)
    w.add("tokenizer.ggml.unknown_token_id", T_U32, unk)
    if add_space_prefix is not None:
        w.add("tokenizer.ggml.add_space_prefix", T_BOOL, bool(add_space_prefix))
    w.write(path)


TINY = dict(n_layers=6, d_model=128, n_heads=2, head_dim=64, ffn=256, vocab=1000, context=256, window=8)
