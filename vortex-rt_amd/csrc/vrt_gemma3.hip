// vrt_gemma3.hip -- device-resident Gemma 3 decode step (src/gemma3.cpp:1462-1882) for gfx950.
//
// One decode step is six kinds of kernel, five per decoder block plus the LM head:
//   k_qkv     residual h = RMSNorm(f_prev, post_ffw) + h_mid (or the scaled embedding row),
//             x = RMSNorm(h, attn_norm), then the Wq|Wk|Wv rows            (:1511-1541)
//   k_attn    QK-norm, RoPE, KV append, attention over a split history     (:1557-1696)
//   k_o       attention output projection                                  (:1698-1701)
//   k_gateup  h_mid = RMSNorm(o, post_attn) + h, x = RMSNorm(h_mid, ffn_norm),
//             gate/up rows interleaved, gelu_tanh(gate) * up epilogue      (:1703-1801)
//   k_down    down projection                                              (:1783-1801)
//   k_lm      final residual + output norm, tied Q8_0 LM head fused with greedy argmax
//             (:1866-1872, :1138-1185)
// Norms are recomputed redundantly by every workgroup of the consuming kernel (inputs are
// <= 2048 floats), so the only grid-wide syncs are the kernel boundaries. Each matvec kernel
// issues its own prologue loads, then its weight loads, and only then waits on the
// prologue, so the norm arithmetic overlaps the weight fetch.
//
// Step state (position, token stream, LM-head/feeding switches, EOS stop, non-finite flag)
// lives in device memory, so one captured graph replays every step unchanged and greedy
// generation never returns to the host between tokens.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "vrt_g3_errors.hpp"
#include "vrt_g3_internal.hpp"
#include "vrt_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {

constexpr uint32_t kPrefillMax = 2048;   // positions of one batched prefill segment

constexpr int kThreads = 256;
constexpr int kMaxE = 8;  // vector elements per thread in prologues: d, H*hd, F <= 2048

// ---- workgroup reductions ---------------------------------------------------------------

__device__ __forceinline__ double wg_sum_f64(double v, double* red) {
    v = wave_sum_f64(v);
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0u) red[w] = v;
    __syncthreads();
    double t = 0.0;
    for (uint32_t k = 0; k < (blockDim.x >> 6); ++k) t += red[k];
    __syncthreads();
    return t;
}

// 1.0f / std::sqrt(float(sum_sq / n) + eps), src/gemma3.cpp:967-983.
__device__ __forceinline__ float rms_scale_from(double ss, uint32_t n, float eps) {
#pragma clang fp contract(off)
    const double mean = ss / static_cast<double>(n);
    return 1.0f / sqrtf(static_cast<float>(mean) + eps);
}

template <typename T>
__device__ __forceinline__ void load_vec(const T* src, uint32_t n, T (&r)[kMaxE]) {
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
        r[k] = i < n ? src[i] : T(0);
    }
}

__device__ __forceinline__ double sum_sq(const float (&r)[kMaxE], uint32_t n) {
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < kMaxE; ++k)
        if (threadIdx.x + static_cast<uint32_t>(k) * kThreads < n) acc += static_cast<double>(r[k]) * static_cast<double>(r[k]);
    return acc;
}

// ---- shared-memory layout of the matvec kernels --------------------------------------------

struct MvSmem {
    float* xs;
    LimbLds L;
    float* extra;   // kernel-specific (gate/up staging)
};

__device__ __forceinline__ MvSmem mv_smem(uint32_t K) {
    extern __shared__ __align__(16) unsigned char smem[];
    MvSmem m;
    m.xs = reinterpret_cast<float*>(smem);
    int8_t* lb = reinterpret_cast<int8_t*>(m.xs + K);
    m.L = LimbLds{lb, lb + K, lb + 2 * K, reinterpret_cast<float*>(lb + 3 * K)};
    m.extra = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(m.L.s) + ((K / 32u) * 4u + 15u) / 16u * 16u);
    return m;
}

static size_t mv_smem_bytes(uint32_t K, uint32_t extra_floats) {
    return static_cast<size_t>(K) * 4 + static_cast<size_t>(K) * 3 + ((K / 32u) * 4u + 15u) / 16u * 16u +
           static_cast<size_t>(extra_floats) * 4 + 16;
}

__device__ __forceinline__ void flag_nonfinite(const float (&h)[kMaxE], uint32_t n, G3State* st, uint32_t block,
                                               double* red) {
    double bad = 0.0;
#pragma unroll
    for (int k = 0; k < kMaxE; ++k)
        if (threadIdx.x + static_cast<uint32_t>(k) * kThreads < n && !__builtin_isfinite(h[k])) bad = 1.0;
    bad = wg_sum_f64(bad, red);
    if (bad != 0.0 && threadIdx.x == 0) atomicMin(&st->nonfinite, g3_code_nonfinite(block));
}

// =========================================================================================
// k_qkv
// =========================================================================================

// Rows [r_begin, r_end) of the virtual rows [Wq | Wk | Wv]: the whole range with projection fusion
// (one launch, src/gemma3.cpp:1529-1541 run_q8_triplet), one matrix per launch without it.
template <int S, int NB, int U>
__global__ void __launch_bounds__(kThreads) k_qkv(G3Params P, LayerParams Lc, const float* prev_post_ffw, uint32_t layer,
                                                  uint32_t r_begin, uint32_t r_end) {
#pragma clang fp contract(off)
    __shared__ double red[8];
    if (P.st->stop) return;
    const uint32_t s = P.st->step;
    const uint32_t d = P.d;
    const uint32_t nblk = d >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    MvSmem m = mv_smem(d);

    // prologue inputs first
    float ra[kMaxE], rb[kMaxE], rw[kMaxE], rw2[kMaxE];
    if (layer == 0) {
        const uint8_t* row = P.tok_embd + static_cast<uint64_t>(P.tokens[s]) * row_bytes;
#pragma unroll
        for (int k = 0; k < kMaxE; ++k) {
            const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
            ra[k] = 0.0f;
            if (i < d) {
                const uint8_t* b = row + (i >> 5) * 34u;
                const float sc = half_bits_to_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
                ra[k] = sc * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31u)]));
            }
            rb[k] = rw[k] = 0.0f;
        }
    } else {
        load_vec(P.f, d, ra);
        load_vec(P.hmid, d, rb);
        load_vec(prev_post_ffw, d, rw);
    }
    load_vec(Lc.attn_norm, d, rw2);

    // weight prefetch: virtual rows [Wq | Wk | Wv], packed output like run_staged_triplet
    const uint32_t qw = P.H * P.hd;
    const uint32_t total = qw + 2u * P.hd;
    const uint8_t *wq = Lc.wq, *wk = Lc.wk, *wv = Lc.wv;
    const uint32_t hd = P.hd;
    auto rowp = [=](uint32_t v) -> const uint8_t* {
        const uint8_t* b = v < qw ? wq + static_cast<uint64_t>(v) * row_bytes
                                  : (v < qw + hd ? wk + static_cast<uint64_t>(v - qw) * row_bytes
                                                 : wv + static_cast<uint64_t>(v - qw - hd) * row_bytes);
        return b;
    };
    constexpr uint32_t per_wg = (64u / S) * 4u * U;
    const uint32_t v0 = r_begin + blockIdx.x * per_wg;
    const uint32_t v1 = min(min(total, r_end), v0 + per_wg);
    RowBatch<S, NB, U> batch;
    batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, threadIdx.x >> 6, blockDim.x >> 6, batch);

    // residual stream entering this block
    float h[kMaxE];
    if (layer == 0) {
#pragma unroll
        for (int k = 0; k < kMaxE; ++k) h[k] = ra[k] * P.emb_scale;                 // :1131-1134
    } else {
        const float sc = rms_scale_from(wg_sum_f64(sum_sq(ra, d), red), d, P.eps);
#pragma unroll
        for (int k = 0; k < kMaxE; ++k) h[k] = ra[k] * (sc * rw[k]) + rb[k];       // :1849-1855
        if (blockIdx.x == 0) flag_nonfinite(h, d, P.st, layer - 1u, red);           // :1857-1863
    }
    const float sc2 = rms_scale_from(wg_sum_f64(sum_sq(h, d), red), d, P.eps);
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
        if (i < d) {
            m.xs[i] = h[k] * sc2 * rw2[k];                                           // :991-996
            if (blockIdx.x == 0) P.hres[i] = h[k];
        }
    }
    __syncthreads();
    build_limbs(m.xs, d, m.L, blockDim.x >> 6);
    XLimb xl[NB];
    lane_limbs<S, NB>(m.L, nblk, xl);
    float* out = P.qkv;
    batch_consume<S, NB, U>(batch, nblk, xl, [&](uint32_t v, float val) { out[v] = val; });
}

// =========================================================================================
// k_attn: QK-norm + RoPE + KV append + attention over one history chunk per workgroup (split
// softmax: max, sum and weighted V per chunk); k_attn_merge combines the chunks.
// =========================================================================================

__global__ void __launch_bounds__(kThreads) k_attn(G3Params P, LayerParams Lc) {
#pragma clang fp contract(off)
    __shared__ double red[8];
    if (P.st->stop) return;
    const uint32_t pos = P.st->step;
    const uint32_t H = P.H, hd = P.hd, half = hd >> 1;
    extern __shared__ __align__(16) unsigned char smem[];
    float* sq = reinterpret_cast<float*>(smem);      // [H][hd]
    float* sk = sq + H * hd;                          // [hd]
    float* sv = sk + hd;                              // [hd]
    float* sc = sv + hd;                              // [H][chunk_max]

    // history window (src/gemma3.cpp:1590-1600): local layers keep the last `slots` positions
    const uint32_t n_hist = min(pos + 1u, Lc.slots);
    const uint32_t t_first = pos + 1u - n_hist;
    const uint32_t G = gridDim.x;
    const uint32_t C = (n_hist + G - 1u) / G;
    const uint32_t c0 = t_first + blockIdx.x * C;
    const uint32_t c1 = min(pos + 1u, c0 + C);

    // q, k raw -> LDS, then per-head RMSNorm (src/gemma3.cpp:1045-1104) and RoPE (:1371-1424)
    const float* qkv = P.qkv;
    for (uint32_t i = threadIdx.x; i < (H + 2u) * hd; i += blockDim.x) sq[i] = qkv[i];
    __syncthreads();
    const float* cs = (Lc.global ? P.cos_g : P.cos_l) + static_cast<uint64_t>(pos) * half;
    const float* sn = (Lc.global ? P.sin_g : P.sin_l) + static_cast<uint64_t>(pos) * half;
    for (uint32_t h = 0; h <= H; ++h) {          // heads 0..H-1 are q, head H is k
        float* v = sq + h * hd;
        const float* w = h < H ? Lc.q_norm : Lc.k_norm;
        double acc = 0.0;
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) acc += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        const float scl = rms_scale_from(wg_sum_f64(acc, red), hd, P.eps);
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) v[i] *= scl * w[i];
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
            const float a = v[i], b = v[half + i];
            v[i] = a * cs[i] - b * sn[i];
            v[half + i] = b * cs[i] + a * sn[i];
        }
        __syncthreads();
    }
    // 16-bit KV: the current position's key and value as the cache will hold them
    const uint32_t fmt = P.kv16;
    if (fmt) {
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
            sk[i] = kv16_float(kv16_bits(sk[i], fmt), fmt);
            sv[i] = kv16_float(kv16_bits(sv[i], fmt), fmt);
        }
        __syncthreads();
    }
    // KV append (slot of this position); the current position is read from LDS below
    const uint32_t slot_cur = pos % Lc.slots;
    uint16_t* kh = reinterpret_cast<uint16_t*>(Lc.kc);
    uint16_t* vh = reinterpret_cast<uint16_t*>(Lc.vc);
    if (blockIdx.x == 0)
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
            const uint64_t o = static_cast<uint64_t>(slot_cur) * hd + i;
            if (fmt) {
                kh[o] = kv16_bits(sk[i], fmt);
                vh[o] = kv16_bits(sv[i], fmt);
            } else {
                Lc.kc[o] = sk[i];
                Lc.vc[o] = sv[i];
            }
        }

    const uint32_t stride_part = 2u * H + H * hd;
    float* mypart = P.part + static_cast<uint64_t>(blockIdx.x) * stride_part;
    if (c0 < c1) {
        // scores: wave w takes positions c0 + w, c0 + w + 4, ...; lane l covers dims l, l+64, ...
        const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
        for (uint32_t t = c0 + wave; t < c1; t += blockDim.x >> 6) {
            const uint64_t row = static_cast<uint64_t>(t % Lc.slots) * hd;
            float kr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t i = lane + 64u * j;
                kr[j] = i >= hd ? 0.0f : (t == pos ? sk[i] : (fmt ? kv16_float(kh[row + i], fmt) : Lc.kc[row + i]));
            }
            for (uint32_t h = 0; h < H; ++h) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (lane + 64u * j < hd) p += sq[h * hd + lane + 64u * j] * kr[j];
                p = wave_sum(p);
                if (lane == 0) sc[h * Lc.chunk_max + (t - c0)] = p * P.attn_scale;
            }
        }
        __syncthreads();
        // chunk softmax statistics, one wave per head
        const uint32_t n = c1 - c0;
        for (uint32_t h = threadIdx.x >> 6; h < H; h += blockDim.x >> 6) {
            float mx = -INFINITY;
            for (uint32_t t = lane; t < n; t += 64) mx = fmaxf(mx, sc[h * Lc.chunk_max + t]);
            mx = wave_max(mx);
            double l = 0.0;
            for (uint32_t t = lane; t < n; t += 64) {
                const float e = expf(sc[h * Lc.chunk_max + t] - mx);
                sc[h * Lc.chunk_max + t] = e;
                l += e;
            }
            l = wave_sum_f64(l);
            if (lane == 0) { mypart[h] = mx; mypart[H + h] = static_cast<float>(l); }
        }
        __syncthreads();
        // weighted V: thread i owns dims i, i+256, ...
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (uint32_t t = c0; t < c1; ++t) {
                const uint64_t vo = static_cast<uint64_t>(t % Lc.slots) * hd + i;
                const float vv = (t == pos) ? sv[i] : (fmt ? kv16_float(vh[vo], fmt) : Lc.vc[vo]);
#pragma unroll
                for (uint32_t h = 0; h < 8u; ++h)
                    if (h < H) acc[h] += sc[h * Lc.chunk_max + (t - c0)] * vv;
            }
#pragma unroll
            for (uint32_t h = 0; h < 8u; ++h)
                if (h < H) mypart[2u * H + h * hd + i] = acc[h];
        }
    }
}

// k_attn_merge: combines k_attn's chunk partials of the step (a launch of its own, so the
// partials are visible without a device-wide fence), one workgroup per head:
// att[h][i] = sum_c e^(m_c - M) acc_c[i] / sum_c e^(m_c - M) l_c, the sums in double in chunk
// order. The chunk maxima, sums and weights go through LDS once; each thread then owns dims.
constexpr uint32_t kAttnMaxChunks = 64;   // k_attn workgroups per block, at most
__global__ void __launch_bounds__(kThreads) k_attn_merge(G3Params P, LayerParams Lc) {
#pragma clang fp contract(off)
    __shared__ float s_m[kAttnMaxChunks];
    __shared__ float s_l[kAttnMaxChunks];
    __shared__ double s_w[kAttnMaxChunks];
    __shared__ double s_den;
    if (P.st->stop) return;
    const uint32_t pos = P.st->step;
    const uint32_t H = P.H, hd = P.hd, h = blockIdx.x;
    const uint32_t n_hist = min(pos + 1u, Lc.slots);
    const uint32_t C = (n_hist + Lc.attn_grid - 1u) / Lc.attn_grid;
    const uint32_t n_act = (n_hist + C - 1u) / C;
    const uint32_t stride_part = 2u * H + H * hd;
    for (uint32_t c = threadIdx.x; c < n_act; c += blockDim.x) {
        s_m[c] = P.part[c * stride_part + h];
        s_l[c] = P.part[c * stride_part + H + h];
    }
    __syncthreads();
    float M = -INFINITY;
    for (uint32_t c = 0; c < n_act; ++c) M = fmaxf(M, s_m[c]);
    for (uint32_t c = threadIdx.x; c < n_act; c += blockDim.x) s_w[c] = static_cast<double>(expf(s_m[c] - M));
    __syncthreads();
    if (threadIdx.x == 0) {
        double den = 0.0;
        for (uint32_t c = 0; c < n_act; ++c) den += s_w[c] * static_cast<double>(s_l[c]);
        s_den = den;
        if (!(den > 0.0) || !__builtin_isfinite(den)) atomicMin(&P.st->nonfinite, g3_code_softmax(Lc.index));
    }
    __syncthreads();
    const double den = s_den;
    for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
        const float* src = P.part + 2u * H + h * hd + i;
        double num = 0.0;
#pragma unroll 8
        for (uint32_t c = 0; c < n_act; ++c) num += s_w[c] * static_cast<double>(src[c * stride_part]);
        P.att[h * hd + i] = static_cast<float>(num / den);
    }
}

// =========================================================================================
// k_o: attention output projection
// =========================================================================================

template <int S, int NB, int U>
__global__ void __launch_bounds__(kThreads) k_o(G3Params P, LayerParams Lc) {
    if (P.st->stop) return;
    const uint32_t K = P.H * P.hd;
    const uint32_t nblk = K >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    MvSmem m = mv_smem(K);
    float ra[kMaxE];
    load_vec(P.att, K, ra);
    const uint8_t* wo = Lc.wo;
    auto rowp = [=](uint32_t v) { return wo + static_cast<uint64_t>(v) * row_bytes; };
    constexpr uint32_t per_wg = (64u / S) * 4u * U;
    const uint32_t v0 = blockIdx.x * per_wg;
    const uint32_t v1 = min(P.d, v0 + per_wg);
    RowBatch<S, NB, U> batch;
    batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, threadIdx.x >> 6, blockDim.x >> 6, batch);
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
        if (i < K) m.xs[i] = ra[k];
    }
    __syncthreads();
    build_limbs(m.xs, K, m.L, blockDim.x >> 6);
    XLimb xl[NB];
    lane_limbs<S, NB>(m.L, nblk, xl);
    float* out = P.o;
    batch_consume<S, NB, U>(batch, nblk, xl, [&](uint32_t v, float val) { out[v] = val; });
}

// =========================================================================================
// k_gateup: post-attention residual, FFN norm, gate/up rows, GELU-tanh * up
// =========================================================================================

__device__ __forceinline__ float gelu_tanh_g3(float x) {
#pragma clang fp contract(off)
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float cubic = x * x * x;
    return 0.5f * x * (1.0f + tanhf(kSqrt2OverPi * (x + kCubic * cubic)));
}

// mode 0 (projection fusion): gate/up row pairs with gelu_tanh(gate) * up in the epilogue, as
// run_q8_pair + gelu_mul. mode 1 / 2: the rows of gate / up alone into P.gu[0, F) / P.gu[F, 2F)
// (the unfused sequence, src/gemma3.cpp:1820-1847: separate matvecs, then k_gelu_mul).
template <int S, int NB, int U>
__global__ void __launch_bounds__(kThreads) k_gateup(G3Params P, LayerParams Lc, uint32_t mode) {
#pragma clang fp contract(off)
    __shared__ double red[8];
    if (P.st->stop) return;
    const uint32_t d = P.d;
    const uint32_t nblk = d >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    MvSmem m = mv_smem(d);
    float ra[kMaxE], rb[kMaxE], rw[kMaxE], rw2[kMaxE];
    load_vec(P.o, d, ra);
    load_vec(P.hres, d, rb);
    load_vec(Lc.post_attn, d, rw);
    load_vec(Lc.ffn_norm, d, rw2);
    // mode 0: virtual row v is row v>>1 of gate (v even) or up (v odd); else row v of one matrix
    // (offsets from wg, so that no pointer is selected per row)
    const uint8_t* wg = Lc.wg;
    const int64_t up_off = Lc.wu - Lc.wg;
    const uint32_t pair = mode == 0u ? 1u : 0u, fixed_up = mode == 2u ? 1u : 0u;
    auto rowp = [=](uint32_t v) {
        const uint32_t is_up = pair ? (v & 1u) : fixed_up;
        return wg + (is_up ? up_off : 0) + static_cast<int64_t>(static_cast<uint64_t>(v >> pair) * row_bytes);
    };
    constexpr uint32_t per_wg = (64u / S) * 4u * U;   // even: gate/up pairs stay together
    const uint32_t v0 = blockIdx.x * per_wg;
    const uint32_t v1 = min(mode == 0u ? 2u * P.F : P.F, v0 + per_wg);
    RowBatch<S, NB, U> batch;
    batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, threadIdx.x >> 6, blockDim.x >> 6, batch);

    const float sc = rms_scale_from(wg_sum_f64(sum_sq(ra, d), red), d, P.eps);
    float h[kMaxE];
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) h[k] = ra[k] * (sc * rw[k]) + rb[k];          // :1703-1711
    const float sc2 = rms_scale_from(wg_sum_f64(sum_sq(h, d), red), d, P.eps);
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
        if (i < d) {
            m.xs[i] = h[k] * sc2 * rw2[k];                                           // :1713-1718
            if (blockIdx.x == 0) P.hmid[i] = h[k];
        }
    }
    __syncthreads();
    build_limbs(m.xs, d, m.L, blockDim.x >> 6);
    XLimb xl[NB];
    lane_limbs<S, NB>(m.L, nblk, xl);
    if (mode != 0u) {
        float* raw = P.gu + (mode - 1u) * P.F;
        batch_consume<S, NB, U>(batch, nblk, xl, [&](uint32_t v, float val) { raw[v] = val; });
        return;
    }
    float* gu = m.extra;
    batch_consume<S, NB, U>(batch, nblk, xl, [&](uint32_t v, float val) { gu[v - v0] = val; });
    __syncthreads();
    const uint32_t r0 = v0 >> 1, r1 = v1 >> 1;
    for (uint32_t r = r0 + threadIdx.x; r < r1; r += blockDim.x) {
        const uint32_t j = (r - r0) * 2u;
        P.g[r] = gelu_tanh_g3(gu[j]) * gu[j + 1u];                                   // gelu_mul.comp:23-31
    }
}

// The GELU product of the unfused sequence: g = gelu_tanh(gate) * up over P.gu.
__global__ void __launch_bounds__(kThreads) k_gelu_mul(G3Params P) {
#pragma clang fp contract(off)
    if (P.st->stop) return;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < P.F; i += gridDim.x * blockDim.x)
        P.g[i] = gelu_tanh_g3(P.gu[i]) * P.gu[P.F + i];                              // gelu_mul.comp:23-31
}

// =========================================================================================
// k_down
// =========================================================================================

template <int S, int NB, int U>
__global__ void __launch_bounds__(kThreads) k_down(G3Params P, LayerParams Lc) {
    if (P.st->stop) return;
    const uint32_t K = P.F;
    const uint32_t nblk = K >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    MvSmem m = mv_smem(K);
    float ra[kMaxE];
    load_vec(P.g, K, ra);
    const uint8_t* wd = Lc.wd;
    auto rowp = [=](uint32_t v) { return wd + static_cast<uint64_t>(v) * row_bytes; };
    constexpr uint32_t per_wg = (64u / S) * 4u * U;
    const uint32_t v0 = blockIdx.x * per_wg;
    const uint32_t v1 = min(P.d, v0 + per_wg);
    RowBatch<S, NB, U> batch;
    batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, threadIdx.x >> 6, blockDim.x >> 6, batch);
#pragma unroll
    for (int k = 0; k < kMaxE; ++k) {
        const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
        if (i < K) m.xs[i] = ra[k];
    }
    __syncthreads();
    build_limbs(m.xs, K, m.L, blockDim.x >> 6);
    XLimb xl[NB];
    lane_limbs<S, NB>(m.L, nblk, xl);
    float* out = P.f;
    batch_consume<S, NB, U>(batch, nblk, xl, [&](uint32_t v, float val) { out[v] = val; });
}

// =========================================================================================
// k_lm: final residual + output norm, tied LM head fused with greedy argmax (per-workgroup
// partials; k_lm_final reduces them). mode 0: a decode step; mode 1: timing (no state change).
// =========================================================================================

template <int S, int NB, int U>
__global__ void __launch_bounds__(kThreads) k_lm(G3Params P, const float* last_post_ffw, const float* out_norm,
                                                 uint32_t rows_per_wg, uint32_t mode) {
#pragma clang fp contract(off)
    __shared__ double red[8];
    __shared__ float bvs[4];
    __shared__ uint32_t bis[4];
    if (P.st->stop && mode == 0) return;
    const uint32_t s = P.st->step;
    const bool run_lm = mode != 0 || s >= P.st->lm_from;
    const bool want_logits = mode == 0 && P.st->want_logits != 0u;
    const uint32_t d = P.d;
    const uint32_t nblk = d >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    MvSmem m = mv_smem(d);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;

    if (run_lm || blockIdx.x == 0) {
        float ra[kMaxE], rb[kMaxE], rw[kMaxE], rw2[kMaxE];
        load_vec(P.f, d, ra);
        load_vec(P.hmid, d, rb);
        load_vec(last_post_ffw, d, rw);
        load_vec(out_norm, d, rw2);
        const uint8_t* we = P.tok_embd;
        auto rowp = [=](uint32_t v) { return we + static_cast<uint64_t>(v) * row_bytes; };
        const uint32_t v0 = blockIdx.x * rows_per_wg;
        const uint32_t v1 = min(P.V, v0 + rows_per_wg);
        const uint32_t nw = blockDim.x >> 6;
        RowBatch<S, NB, U> batch;
        if (run_lm) batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, threadIdx.x >> 6, blockDim.x >> 6, batch);

        const float sc = rms_scale_from(wg_sum_f64(sum_sq(ra, d), red), d, P.eps);
        float h[kMaxE];
#pragma unroll
        for (int k = 0; k < kMaxE; ++k) h[k] = ra[k] * (sc * rw[k]) + rb[k];      // :1849-1855
        if (blockIdx.x == 0 && mode == 0) flag_nonfinite(h, d, P.st, P.L - 1u, red);
        const float sc3 = rms_scale_from(wg_sum_f64(sum_sq(h, d), red), d, P.eps);
#pragma unroll
        for (int k = 0; k < kMaxE; ++k) {
            const uint32_t i = threadIdx.x + static_cast<uint32_t>(k) * kThreads;
            if (i < d) {
                const float hn = h[k] * (sc3 * rw2[k]);                              // :1866-1868
                m.xs[i] = hn;
                if (blockIdx.x == 0 && mode == 0) P.hidden[i] = hn;
            }
        }
        __syncthreads();
        if (run_lm) {
            build_limbs(m.xs, d, m.L, blockDim.x >> 6);
            XLimb xl[NB];
            lane_limbs<S, NB>(m.L, nblk, xl);
            float* logits = P.logits;
            auto sink = [&](uint32_t v, float val) {
                if (want_logits) logits[v] = val;
                if (am_better(val, v, bv, bi)) { bv = val; bi = v; }
            };
            batch_consume<S, NB, U>(batch, nblk, xl, sink);
            constexpr uint32_t RPW = 64u / S;
            const uint32_t ngroups = (v1 > v0) ? (v1 - v0 + RPW - 1u) / RPW : 0u;
            for (uint32_t g0 = (threadIdx.x >> 6) + U * nw; g0 < ngroups; g0 += U * nw) {
                batch_load<S, NB, U>(rowp, nblk, P.arena_end, v0, v1, g0, blockDim.x >> 6, batch);
                batch_consume<S, NB, U>(batch, nblk, xl, sink);
            }
        }
    }
    if (run_lm) {
        wave_argmax(bv, bi);
        if ((threadIdx.x & 63u) == 0u) { bvs[threadIdx.x >> 6] = bv; bis[threadIdx.x >> 6] = bi; }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (uint32_t k = 1; k < (blockDim.x >> 6); ++k)
                if (am_better(bvs[k], bis[k], bvs[0], bis[0])) { bvs[0] = bvs[k]; bis[0] = bis[k]; }
            P.lm_part[blockIdx.x] = {bvs[0], bis[0]};
        }
    }
}

// k_lm_final: one workgroup reduces k_lm's per-workgroup argmax partials (a launch of its own, so
// they are visible without a device-wide fence) and advances the step state: mode 0 records
// the step's result, feeds the greedy token and stops at EOS; mode 1 (timing) records only.
__global__ void __launch_bounds__(kThreads) k_lm_final(G3Params P, uint32_t nparts, uint32_t mode) {
    __shared__ float bvs[4];
    __shared__ uint32_t bis[4];
    if (P.st->stop && mode == 0) return;
    const uint32_t s = P.st->step;
    const bool run_lm = mode != 0 || s >= P.st->lm_from;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if (run_lm) {
        for (uint32_t k = threadIdx.x; k < nparts; k += blockDim.x) {
            const LmPartial pp = P.lm_part[k];
            if (am_better(pp.value, pp.index, bv, bi)) { bv = pp.value; bi = pp.index; }
        }
        wave_argmax(bv, bi);
        if ((threadIdx.x & 63u) == 0u) { bvs[threadIdx.x >> 6] = bv; bis[threadIdx.x >> 6] = bi; }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (run_lm) {
            for (uint32_t k = 1; k < (blockDim.x >> 6); ++k)
                if (am_better(bvs[k], bis[k], bvs[0], bis[0])) { bvs[0] = bvs[k]; bis[0] = bis[k]; }
        }
        if (mode == 0) {
            if (run_lm) {
                P.results[s] = {bis[0], bvs[0]};
                if (s + 1u >= P.st->feed_until) {
                    P.tokens[s + 1u] = bis[0] < P.V ? bis[0] : 0u;
                    if (bis[0] == P.eos) P.st->stop = 1u;
                }
            }
            P.st->step = s + 1u;
        } else {
            P.results[P.ctx_len] = {bis[0], bvs[0]};
        }
    }
}

// ---- dispatch -------------------------------------------------------------------------------

// (lanes per row, blocks per lane) instantiated for every kernel kind, and the extra ones the
// projections take under a row-slot width request (VRT_G3_OPT_Q8_LANES)
#define VRT_SHAPES(X) X(1, 1) X(2, 1) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) X(64, 2)
#define VRT_LANE_SHAPES(X) X(8, 2) X(8, 3) X(8, 4) X(16, 2) X(16, 3) X(16, 4) X(32, 2)

enum KernelKind { KQKV, KO, KGATEUP, KDOWN, KLM };

template <int S, int NB, bool LM>
static LaunchDesc pick(KernelKind kind, uint32_t rows, uint32_t K, uint32_t extra_per_wg) {
    constexpr uint32_t rpw = 64u / S;
    LaunchDesc ld{};
    switch (kind) {
    case KQKV: ld.fn = reinterpret_cast<const void*>(&k_qkv<S, NB, 1>); break;
    case KO: ld.fn = reinterpret_cast<const void*>(&k_o<S, NB, 1>); break;
    case KGATEUP: ld.fn = reinterpret_cast<const void*>(&k_gateup<S, NB, 1>); break;
    case KDOWN: ld.fn = reinterpret_cast<const void*>(&k_down<S, NB, 1>); break;
    case KLM:
        if constexpr (LM) ld.fn = reinterpret_cast<const void*>(&k_lm<S, NB, (S >= 16 ? 4 : 1)>);
        break;
    }
    const uint32_t per_wg = rpw * 4u;
    ld.per_wg = per_wg;
    ld.S = S;
    ld.grid = (rows + per_wg - 1u) / per_wg;
    ld.smem = mv_smem_bytes(K, extra_per_wg ? per_wg : 0u);
    return ld;
}

// Row-slot shape of a projection with K inputs. lanes = 0: the shape sized from K (mv_shape).
// lanes = 8..64: slots of `lanes` lanes, each lane taking ceil(blocks / lanes) blocks of a row;
// where that exceeds the instantiated blocks per lane the slot widens (a 2048-input row over
// 8 lanes runs with 16).
static bool pick_shape(KernelKind kind, uint32_t rows, uint32_t K, LaunchDesc* out, uint32_t lanes = 0) {
    const uint32_t extra = kind == KGATEUP ? 1u : 0u;
    MvShape sh;
    if (lanes == 0u || kind == KLM) {
        if (!mv_shape(K, &sh) || sh.NB > 2) return false;
    } else {
        const uint32_t nblk = (K + 31u) / 32u;
        sh.S = 0;
        for (uint32_t w = lanes; w <= 64u && sh.S == 0; w *= 2u) {
            const uint32_t nb = (nblk + w - 1u) / w;
            if (nb <= (w >= 32u ? 2u : 4u)) { sh.S = static_cast<int>(w); sh.NB = static_cast<int>(nb); }
        }
        if (sh.S == 0) return false;
    }
#define VRT_PICK(s_, nb_) \
    if (sh.S == s_ && sh.NB == nb_) { *out = pick<s_, nb_, true>(kind, rows, K, extra); return true; }
    VRT_SHAPES(VRT_PICK)
#undef VRT_PICK
#define VRT_PICK(s_, nb_) \
    if (kind != KLM && sh.S == s_ && sh.NB == nb_) { *out = pick<s_, nb_, false>(kind, rows, K, extra); return true; }
    VRT_LANE_SHAPES(VRT_PICK)
#undef VRT_PICK
    return false;
}

// The projection kernels' shapes for the executor's row-slot request; drops a captured graph.
static int g3_pick_projections(vrt_g3* g) {
    const uint32_t d = g->cfg.embedding_length, H = g->cfg.head_count, hd = g->cfg.head_dim;
    const uint32_t F = g->cfg.feed_forward_length, lanes = g->q8_lanes;
    LaunchDesc qkv, o, gu, down;
    if (!pick_shape(KQKV, H * hd + 2u * hd, d, &qkv, lanes) || !pick_shape(KO, d, H * hd, &o, lanes) ||
        !pick_shape(KGATEUP, 2u * F, d, &gu, lanes) || !pick_shape(KDOWN, d, F, &down, lanes))
        return set_error(VRT_ERR_INVALID, "no kernel shape for this Gemma 3 configuration");
    for (const LaunchDesc* ld : {&qkv, &o, &gu, &down})
        VRT_HIP_CHECK(hipFuncSetAttribute(ld->fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(ld->smem)));
    g->ld_qkv = qkv;
    g->ld_o = o;
    g->ld_gateup = gu;
    g->ld_down = down;
    if (g->graph) {
        (void)hipGraphExecDestroy(g->graph);
        g->graph = nullptr;
    }
    return VRT_OK;
}

}  // namespace vrt

using namespace vrt;

// =======================================================================================
// Host side
// =======================================================================================

static int g3_alloc(vrt_g3* g, size_t bytes, void** out) {
    void* p = nullptr;
    VRT_HIP_CHECK(hipMalloc(&p, bytes + 256));
    g->allocs.push_back(p);
    // zero-filled on the context's (non-blocking) stream, which every later use is ordered on
    VRT_HIP_CHECK(hipMemsetAsync(p, 0, bytes + 256, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    *out = p;
    return VRT_OK;
}

static int g3_upload(vrt_g3* g, const void* host, size_t bytes, const float** out) {
    void* p = nullptr;
    if (int rc = g3_alloc(g, bytes, &p)) return rc;
    // on the context's stream and waited for: a pageable-memory hipMemcpy may return before its
    // DMA lands, and the null stream does not order the non-blocking context stream
    VRT_HIP_CHECK(hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    *out = static_cast<const float*>(p);
    return VRT_OK;
}

// Enqueues one decode step's kernels on `stream`. With projection fusion a block is q|k|v,
// attention, O, gate/up with the GELU product, down; without it q, k and v, and gate and up, are
// launches of their own and the GELU product a launch after them (src/gemma3.cpp:1529-1541,
// :1783-1847).
static int g3_enqueue_step(vrt_g3* g, hipStream_t stream) {
    const uint32_t L = g->cfg.block_count;
    const uint32_t qw = g->cfg.head_count * g->cfg.head_dim, hd = g->cfg.head_dim, F = g->cfg.feed_forward_length;
    auto grid = [](const LaunchDesc& ld, uint32_t rows) { return dim3((rows + ld.per_wg - 1u) / ld.per_wg); };
    for (uint32_t l = 0; l < L; ++l) {
        LayerParams& Lc = g->layers[l];
        const float* prev_post = l ? g->layers[l - 1].post_ffw : nullptr;
        if (g->fusion) {
            uint32_t r0 = 0, r1 = qw + 2u * hd;
            void* args[] = {&g->P, &Lc, &prev_post, &l, &r0, &r1};
            VRT_HIP_CHECK(hipLaunchKernel(g->ld_qkv.fn, grid(g->ld_qkv, r1), dim3(kThreads), args, g->ld_qkv.smem, stream));
        } else {
            const uint32_t cut[4] = {0u, qw, qw + hd, qw + 2u * hd};
            for (int m = 0; m < 3; ++m) {
                uint32_t r0 = cut[m], r1 = cut[m + 1];
                void* args[] = {&g->P, &Lc, &prev_post, &l, &r0, &r1};
                VRT_HIP_CHECK(hipLaunchKernel(g->ld_qkv.fn, grid(g->ld_qkv, r1 - r0), dim3(kThreads), args, g->ld_qkv.smem,
                                              stream));
            }
        }
        {
            void* args[] = {&g->P, &Lc};
            const size_t smem = (static_cast<size_t>(g->cfg.head_count + 2u) * g->cfg.head_dim +
                                 static_cast<size_t>(g->cfg.head_count) * Lc.chunk_max) * 4u + 64u;
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_attn), dim3(Lc.attn_grid), dim3(kThreads), args,
                                          smem, stream));
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_attn_merge), dim3(g->cfg.head_count),
                                          dim3(kThreads), args, 0, stream));
        }
        {
            void* args[] = {&g->P, &Lc};
            VRT_HIP_CHECK(hipLaunchKernel(g->ld_o.fn, dim3(g->ld_o.grid), dim3(kThreads), args, g->ld_o.smem, stream));
        }
        if (g->fusion) {
            uint32_t mode = 0;
            void* args[] = {&g->P, &Lc, &mode};
            VRT_HIP_CHECK(hipLaunchKernel(g->ld_gateup.fn, grid(g->ld_gateup, 2u * F), dim3(kThreads), args,
                                          g->ld_gateup.smem, stream));
        } else {
            for (uint32_t mode = 1; mode <= 2u; ++mode) {
                void* args[] = {&g->P, &Lc, &mode};
                VRT_HIP_CHECK(hipLaunchKernel(g->ld_gateup.fn, grid(g->ld_gateup, F), dim3(kThreads), args,
                                              g->ld_gateup.smem, stream));
            }
            void* args[] = {&g->P};
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_gelu_mul), dim3((F + kThreads - 1u) / kThreads),
                                          dim3(kThreads), args, 0, stream));
        }
        {
            void* args[] = {&g->P, &Lc};
            VRT_HIP_CHECK(hipLaunchKernel(g->ld_down.fn, dim3(g->ld_down.grid), dim3(kThreads), args, g->ld_down.smem, stream));
        }
    }
    return g3_enqueue_lm(g, stream);
}

// Final residual (P.f normed by the last block's post-FFW norm, plus P.hmid), output norm and
// the LM head + argmax of the step in G3State::step.
int vrt::g3_enqueue_lm(vrt_g3* g, hipStream_t stream) {
    const float* last_post = g->layers[g->cfg.block_count - 1].post_ffw;
    uint32_t mode = 0;
    void* args[] = {&g->P, &last_post, &g->out_norm_dev, &g->lm_rows_per_wg, &mode};
    VRT_HIP_CHECK(hipLaunchKernel(g->ld_lm.fn, dim3(g->ld_lm.grid), dim3(kThreads), args, g->ld_lm.smem, stream));
    uint32_t nparts = g->ld_lm.grid;
    void* fargs[] = {&g->P, &nparts, &mode};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_lm_final), dim3(1), dim3(kThreads), fargs, 0, stream));
    return VRT_OK;
}

static int g3_capture(vrt_g3* g) {
    hipStream_t s = g->ctx->stream;
    VRT_HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    int rc = g3_enqueue_step(g, s);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (rc) { if (graph) (void)hipGraphDestroy(graph); return rc; }
    if (e != hipSuccess) return set_error(VRT_ERR_HIP, "hipStreamEndCapture failed: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&g->graph, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return set_error(VRT_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    return VRT_OK;
}

// Runs n steps from position first. With the persistent kernels: the steps at positions below
// the team kernel's limit run on it (vrt_team.hip), the rest on the all-workgroup kernel
// (vrt_decode.hip); both read and leave the same step state, KV cache and token buffer.
static int g3_run_steps(vrt_g3* g, uint32_t n, uint32_t first) {
    hipStream_t s = g->ctx->stream;
    // the persistent kernels are the fused sequence at their own row-slot widths: a request for
    // the unfused sequence or for a slot width runs the multi-kernel steps
    if ((g->mk || g->tk) && g->use_persistent && g->fusion && g->q8_lanes == 0u) {
        uint32_t done = 0;
        const uint32_t lim = g->use_team ? tk_pos_limit(g) : 0u;
        const uint32_t pch = g->use_team ? tk_chunk_from(g) : 0u;   // team steps from here: chunked variant
        int rc = VRT_OK;
        while (rc == VRT_OK && done < n && first + done < lim) {
            const uint32_t p = first + done;
            const bool ch = p >= pch;
            const uint32_t k = std::min(n - done, (ch ? lim : std::min(lim, pch)) - p);
            rc = tk_run(g, k, ch);
            if (rc == VRT_OK) {
                done += k;
                g->last_coop = kCoopTeam;
            }
        }
        if (rc == VRT_OK && done < n) {
            if (g->mk) {
                rc = mk_run(g, n - done);
                if (rc == VRT_OK) {
                    done = n;
                    g->last_coop = kCoopMk;
                }
            } else {
                rc = kMkRefused;   // no all-workgroup kernel for this shape: the multi-kernel step
            }
        }
        if (rc == VRT_OK) return VRT_OK;
        if (rc != kMkRefused) return rc;
        if (done == 0u) {
            g->use_persistent = false;   // refused by the device: multi-kernel steps from here on
            g->mk_refused = true;
        }
        n -= done;
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (g->use_graph) {
            if (!g->graph) { if (int rc = g3_capture(g)) return rc; }
            VRT_HIP_CHECK(hipGraphLaunch(g->graph, s));
        } else {
            if (int rc = g3_enqueue_step(g, s)) return rc;
        }
    }
    return VRT_OK;
}

// Host control block -> device (first 8 words of G3State).
static int g3_write_ctl(vrt_g3* g, uint32_t step, uint32_t lm_from, uint32_t feed_until, uint32_t want_logits) {
    G3State* c = g->host_ctl;
    std::memset(c, 0, sizeof(G3State));
    c->step = step;
    c->stop = 0;
    c->lm_from = lm_from;
    c->feed_until = feed_until;
    c->want_logits = want_logits;
    c->nonfinite = 0xffffffffu;
    VRT_HIP_CHECK(hipMemcpyAsync(g->P.st, c, 8 * sizeof(uint32_t), hipMemcpyHostToDevice, g->ctx->stream));
    return VRT_OK;
}

static int g3_fail_reset(vrt_g3* g, int code, const char* msg) {
    g->next_pos = 0;
    set_error(code, "%s", msg);
    return code;
}

// Reads the step state back (and the persistent kernel's abort word) and maps device-side
// failures to the reference's messages; a raised abort word is cleared for the next launch.
static int g3_check_state(vrt_g3* g, G3State* out) {
    VRT_HIP_CHECK(hipMemcpyAsync(g->host_ctl, g->P.st, sizeof(G3State), hipMemcpyDeviceToHost, g->ctx->stream));
    uint32_t* abort_word = &g->host_ctl->pad[0];
    uint32_t* abort_word_tk = &g->host_ctl->pad[1];
    if (g->mk) {
        if (int rc = mk_read_abort(g, abort_word)) return rc;
    }
    if (g->tk) {
        if (int rc = tk_read_abort(g, abort_word_tk)) return rc;
    }
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    *out = *g->host_ctl;
    const uint32_t abort_mk = g->mk ? *abort_word : 0u, abort_tk = g->tk ? *abort_word_tk : 0u;
    const G3Failure f = g3_map_failure(out->nonfinite, abort_mk | abort_tk);
    if (abort_mk != 0u) {
        if (int rc = mk_clear_abort(g)) return rc;
    }
    if (abort_tk != 0u) {
        if (int rc = tk_clear_abort(g)) return rc;
    }
    if (f.code != VRT_OK) return g3_fail_reset(g, f.code, f.msg);
    return VRT_OK;
}

extern "C" int vrt_g3_create(vrt_ctx* ctx, const vrt_g3_desc* desc, vrt_g3** out) {
    VRT_REQUIRE(ctx && desc && out, "vrt_g3_create: null argument");
    *out = nullptr;
    const vrt_g3_config& c = desc->config;
    // src/gemma3.cpp:219-257
    VRT_REQUIRE(c.embedding_length && c.block_count && c.feed_forward_length && c.head_count && c.head_count_kv &&
                    c.head_dim && c.value_dim && c.vocab_size,
                "Gemma 3 configuration contains zero dimensions");
    VRT_REQUIRE(c.head_count % c.head_count_kv == 0, "Gemma 3 head_count must be divisible by head_count_kv");
    VRT_REQUIRE(c.head_count_kv == 1 && c.value_dim == c.head_dim,
                "Current Gemma 3 decoder requires one KV head and equal key/value head dimensions");
    VRT_REQUIRE(c.context_length > 0, "Gemma 3 context_length must be non-zero");
    VRT_REQUIRE(c.head_dim % 2u == 0u, "Invalid Gemma 3 RoPE frequency configuration");
    const uint32_t d = c.embedding_length, H = c.head_count, hd = c.head_dim, F = c.feed_forward_length;
    VRT_REQUIRE(d % 32u == 0 && F % 32u == 0 && (H * hd) % 32u == 0, "Gemma 3 widths must be multiples of 32 (Q8_0 blocks)");
    VRT_REQUIRE(d <= 2048u && F <= 2048u && H * hd <= 2048u && hd <= 256u && H <= 8u,
                "Gemma 3 shape outside this library's kernels: embedding/ffn/attention width <= 2048, head_dim <= 256, heads <= 8");
    VRT_REQUIRE(desc->arena && desc->layers && desc->output_norm, "vrt_g3_create: null tensor pointer");
    const auto* arena = static_cast<const uint8_t*>(desc->arena);
    auto q8_fits = [&](uint64_t off, uint64_t rows, uint64_t k) {
        return off % 4u == 0 && off + rows * (k / 32u) * 34u <= desc->arena_bytes;
    };
    VRT_REQUIRE(q8_fits(desc->token_embd, c.vocab_size, d), "Unsupported token_embd.weight layout");
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const vrt_g3_layer& Ly = desc->layers[l];
        VRT_REQUIRE(q8_fits(Ly.attn_q, H * hd, d) && q8_fits(Ly.attn_k, hd, d) && q8_fits(Ly.attn_v, hd, d) &&
                        q8_fits(Ly.attn_output, d, H * hd) && q8_fits(Ly.ffn_gate, F, d) && q8_fits(Ly.ffn_up, F, d) &&
                        q8_fits(Ly.ffn_down, d, F),
                    "Unsupported Q8_0 matrix layout in block %u", l);
        VRT_REQUIRE(Ly.attn_norm && Ly.attn_q_norm && Ly.attn_k_norm && Ly.post_attention_norm && Ly.ffn_norm &&
                        Ly.post_ffw_norm,
                    "Uncached RMSNorm tensor in block %u", l);
    }
    VRT_HIP_CHECK(hipSetDevice(ctx->device));
    auto* g = new (std::nothrow) vrt_g3();
    VRT_REQUIRE(g != nullptr, "out of memory");
    g->ctx = ctx;
    g->cfg = c;
    g->eos = desc->eos_token_id;
    auto fail = [&](int rc) { vrt_g3_destroy(g); return rc; };

    G3Params& P = g->P;
    P.d = d; P.H = H; P.hd = hd; P.F = F; P.V = c.vocab_size; P.L = c.block_count; P.ctx_len = c.context_length;
    P.eos = desc->eos_token_id;
    P.eps = c.rms_epsilon;
    P.emb_scale = std::sqrt(static_cast<float>(d));                         // :259-264
    P.attn_scale = 1.0f / std::sqrt(static_cast<float>(hd));                // :265-269
    P.arena_end = arena + desc->arena_bytes;
    g->arena_bytes = desc->arena_bytes;
    P.tok_embd = arena + desc->token_embd;

    void* p;
    const uint32_t half = hd / 2u;
    if (int rc = g3_alloc(g, sizeof(G3State), &p)) return fail(rc);
    P.st = static_cast<G3State*>(p);
    if (int rc = g3_alloc(g, (static_cast<size_t>(c.context_length) + 2u) * 4u, &p)) return fail(rc);
    P.tokens = static_cast<uint32_t*>(p);
    if (int rc = g3_alloc(g, (static_cast<size_t>(c.context_length) + 2u) * sizeof(vrt_argmax_result), &p)) return fail(rc);
    P.results = static_cast<vrt_argmax_result*>(p);
    float** bufs[] = {&P.hres, &P.hmid, &P.o, &P.f, &P.hidden};
    for (float** b : bufs) { if (int rc = g3_alloc(g, d * 4u, &p)) return fail(rc); *b = static_cast<float*>(p); }
    if (int rc = g3_alloc(g, (H + 2u) * hd * 4u, &p)) return fail(rc);
    P.qkv = static_cast<float*>(p);
    if (int rc = g3_alloc(g, H * hd * 4u, &p)) return fail(rc);
    P.att = static_cast<float*>(p);
    if (int rc = g3_alloc(g, F * 4u, &p)) return fail(rc);
    P.g = static_cast<float*>(p);
    if (int rc = g3_alloc(g, 2u * F * 4u, &p)) return fail(rc);
    P.gu = static_cast<float*>(p);
    if (int rc = g3_alloc(g, static_cast<size_t>(c.vocab_size) * 4u, &p)) return fail(rc);
    P.logits = static_cast<float*>(p);

    // RoPE tables on the host with the reference's float formulas (src/gemma3.cpp:1309-1369)
    {
        std::vector<float> inv_l(half), inv_g(half);
        for (uint32_t i = 0; i < half; ++i) {
            const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(hd);
            inv_l[i] = 1.0f / std::pow(c.local_rope_base, e);
            inv_g[i] = 1.0f / std::pow(c.global_rope_base, e);
        }
        const size_t n = static_cast<size_t>(c.context_length) * half;
        std::vector<float> cl(n), sl(n), cg(n), sg(n);
        for (uint32_t pos = 0; pos < c.context_length; ++pos) {
            const float pf = static_cast<float>(pos);
            for (uint32_t i = 0; i < half; ++i) {
                const float al = pf * inv_l[i], ag = pf * inv_g[i];
                cl[static_cast<size_t>(pos) * half + i] = std::cos(al);
                sl[static_cast<size_t>(pos) * half + i] = std::sin(al);
                cg[static_cast<size_t>(pos) * half + i] = std::cos(ag);
                sg[static_cast<size_t>(pos) * half + i] = std::sin(ag);
            }
        }
        if (int rc = g3_upload(g, cl.data(), n * 4u, &P.cos_l)) return fail(rc);
        if (int rc = g3_upload(g, sl.data(), n * 4u, &P.sin_l)) return fail(rc);
        if (int rc = g3_upload(g, cg.data(), n * 4u, &P.cos_g)) return fail(rc);
        if (int rc = g3_upload(g, sg.data(), n * 4u, &P.sin_g)) return fail(rc);
    }
    if (int rc = g3_upload(g, desc->output_norm, d * 4u, &g->out_norm_dev)) return fail(rc);

    // layers: tensors, norms, KV cache (fp32, as the reference's host deque)
    uint32_t max_attn_grid = 1;
    g->layers.resize(c.block_count);
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const vrt_g3_layer& Ly = desc->layers[l];
        LayerParams& Lp = g->layers[l];
        Lp.wq = arena + Ly.attn_q; Lp.wk = arena + Ly.attn_k; Lp.wv = arena + Ly.attn_v; Lp.wo = arena + Ly.attn_output;
        Lp.wg = arena + Ly.ffn_gate; Lp.wu = arena + Ly.ffn_up; Lp.wd = arena + Ly.ffn_down;
        if (int rc = g3_upload(g, Ly.attn_norm, d * 4u, &Lp.attn_norm)) return fail(rc);
        if (int rc = g3_upload(g, Ly.attn_q_norm, hd * 4u, &Lp.q_norm)) return fail(rc);
        if (int rc = g3_upload(g, Ly.attn_k_norm, hd * 4u, &Lp.k_norm)) return fail(rc);
        if (int rc = g3_upload(g, Ly.post_attention_norm, d * 4u, &Lp.post_attn)) return fail(rc);
        if (int rc = g3_upload(g, Ly.ffn_norm, d * 4u, &Lp.ffn_norm)) return fail(rc);
        if (int rc = g3_upload(g, Ly.post_ffw_norm, d * 4u, &Lp.post_ffw)) return fail(rc);
        Lp.global = ((l + 1u) % 6u) == 0u ? 1u : 0u;                                // :1301-1307
        Lp.index = l;
        Lp.slots = (!Lp.global && c.sliding_window) ? std::min(c.sliding_window, c.context_length) : c.context_length;
        const size_t kv = static_cast<size_t>(Lp.slots) * hd * 4u;
        if (int rc = g3_alloc(g, kv, &p)) return fail(rc);
        Lp.kc = static_cast<float*>(p);
        if (int rc = g3_alloc(g, kv, &p)) return fail(rc);
        Lp.vc = static_cast<float*>(p);
        // attention split: ~64 positions per workgroup, at most 8 groups for a window and 64 for a full history
        const uint32_t cap = Lp.global ? kAttnMaxChunks : 8u;
        Lp.attn_grid = std::max(1u, std::min(cap, (Lp.slots + 63u) / 64u));
        Lp.chunk_max = (Lp.slots + Lp.attn_grid - 1u) / Lp.attn_grid;
        max_attn_grid = std::max(max_attn_grid, Lp.attn_grid);
    }
    if (int rc = g3_alloc(g, static_cast<size_t>(max_attn_grid) * (2u * H + H * hd) * 4u, &p)) return fail(rc);
    P.part = static_cast<float*>(p);

    // kernel shapes
    if (int rc = g3_pick_projections(g)) return fail(rc);
    if (!pick_shape(KLM, c.vocab_size, d, &g->ld_lm))
        return fail(set_error(VRT_ERR_INVALID, "no kernel shape for this Gemma 3 configuration"));
    {
        // LM head: ~4 workgroups per CU, each a contiguous run of rows
        MvShape sh;
        mv_shape(d, &sh);
        const uint32_t rpw = 64u / static_cast<uint32_t>(sh.S);
        const uint32_t unit = rpw * 4u;
        const uint32_t target = std::max(1u, ctx->info.compute_units * 4u);
        uint32_t groups = (c.vocab_size + unit - 1u) / unit;
        uint32_t grid = std::min(groups, target);
        g->lm_rows_per_wg = (groups + grid - 1u) / grid * unit;
        g->ld_lm.grid = (c.vocab_size + g->lm_rows_per_wg - 1u) / g->lm_rows_per_wg;
    }
    if (int rc = g3_alloc(g, static_cast<size_t>(g->ld_lm.grid) * sizeof(LmPartial), &p)) return fail(rc);
    P.lm_part = static_cast<LmPartial*>(p);
    VRT_HIP_CHECK(hipFuncSetAttribute(g->ld_lm.fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(g->ld_lm.smem)));
    {
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&g->host_ctl), sizeof(G3State), hipHostMallocDefault);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void**>(&g->host_res), (static_cast<size_t>(c.context_length) + 2u) *
                                                                        sizeof(vrt_argmax_result), hipHostMallocDefault);
        if (e != hipSuccess) return fail(set_error(VRT_ERR_HIP, "hipHostMalloc failed: %s", hipGetErrorString(e)));
    }
    if (int rc = g3_write_ctl(g, 0, 0xffffffffu, 0xffffffffu, 0)) return fail(rc);
    if (int rc = mk_setup(g)) return fail(rc);
    if (int rc = tk_setup(g)) return fail(rc);
    if (int rc = pf_setup(g, std::min(c.context_length, kPrefillMax))) return fail(rc);
    VRT_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    *out = g;
    return VRT_OK;
}

extern "C" int vrt_g3_destroy(vrt_g3* g) {
    if (!g) return VRT_OK;
    // a batched decoder reads this executor's weights and launches on its context's stream
    if (g->live_batches != 0u)
        return set_error(VRT_ERR_STATE, "vrt_g3_destroy: %u batched decoder(s) still use this executor; destroy them first",
                         g->live_batches);
    (void)hipSetDevice(g->ctx->device);
    (void)hipStreamSynchronize(g->ctx->stream);
    if (g->graph) (void)hipGraphExecDestroy(g->graph);
    mk_destroy(g);
    tk_destroy(g);
    for (void* p : g->allocs) (void)hipFree(p);
    if (g->host_ctl) (void)hipHostFree(g->host_ctl);
    if (g->host_res) (void)hipHostFree(g->host_res);
    delete g;
    return VRT_OK;
}

extern "C" int vrt_g3_reset(vrt_g3* g) {
    VRT_REQUIRE(g, "vrt_g3_reset: null executor");
    g->next_pos = 0;
    if (int rc = g3_write_ctl(g, 0, 0xffffffffu, 0xffffffffu, 0)) return rc;
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

// KV cache entries: 0 fp32, 1 fp16, 2 bf16. The kernels read the format from their parameter
// blocks: the captured graph (which holds G3Params by value) is dropped, the persistent kernels'
// blocks re-uploaded, the cache reset.
static int g3_set_kv_format(vrt_g3* g, uint32_t fmt) {
    if (g->P.kv16 == fmt) return VRT_OK;
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    g->P.kv16 = fmt;
    if (g->graph) {
        (void)hipGraphExecDestroy(g->graph);
        g->graph = nullptr;
    }
    if (int rc = mk_set_kv_format(g, fmt)) return rc;
    if (int rc = tk_set_kv_format(g, fmt)) return rc;
    return vrt_g3_reset(g);
}

extern "C" int vrt_g3_set_option(vrt_g3* g, uint32_t option, uint32_t value) {
    VRT_REQUIRE(g, "vrt_g3_set_option: null executor");
    switch (option) {
    case VRT_G3_OPT_USE_GRAPH: g->use_graph = value != 0; return VRT_OK;
    case VRT_G3_OPT_PERSISTENT: g->use_persistent = value != 0; return VRT_OK;
    case VRT_G3_OPT_QUERY_PERSISTENT:
        if (g->mk_refused) return set_error(VRT_ERR_STATE, "persistent decode kernel refused by the device");
        return g->mk ? VRT_OK : set_error(VRT_ERR_STATE, "persistent decode kernel unavailable");
    case VRT_G3_OPT_TRACE:
        if (!g->mk && !g->tk) return set_error(VRT_ERR_STATE, "persistent decode kernel unavailable");
        if (g->mk) { if (int rc = mk_set_trace(g, value != 0)) return rc; }
        return tk_set_trace(g, value != 0);
    case VRT_G3_OPT_TEAM: g->use_team = value != 0; return VRT_OK;
    case VRT_G3_OPT_QUERY_TEAM:
        return g->tk ? VRT_OK : set_error(VRT_ERR_STATE, "team decode kernel unavailable");
    case VRT_G3_OPT_FUSION: {
        const bool on = value != 0;
        if (g->fusion == on) return VRT_OK;
        VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
        g->fusion = on;
        if (g->graph) {   // the captured sequence changes
            (void)hipGraphExecDestroy(g->graph);
            g->graph = nullptr;
        }
        return VRT_OK;
    }
    case VRT_G3_OPT_Q8_LANES: {
        if (value != 0u && value != 8u && value != 16u && value != 32u && value != 64u)
            return set_error(VRT_ERR_INVALID, "Q8 lane override must be 0, 8, 16, 32, or 64");   // src/gemma3.cpp:163-166
        if (g->q8_lanes == value) return VRT_OK;
        VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
        const uint32_t old = g->q8_lanes;
        g->q8_lanes = value;
        if (int rc = g3_pick_projections(g)) {
            g->q8_lanes = old;
            return rc;
        }
        return VRT_OK;
    }
    case VRT_G3_OPT_KV_F16: return g3_set_kv_format(g, value != 0 ? 1u : (g->P.kv16 == 1u ? 0u : g->P.kv16));
    case VRT_G3_OPT_KV_BF16: return g3_set_kv_format(g, value != 0 ? 2u : (g->P.kv16 == 2u ? 0u : g->P.kv16));
    case VRT_G3_OPT_QUERY_Q8_LANES: return set_error(VRT_ERR_INVALID, "VRT_G3_OPT_QUERY_Q8_LANES is read with vrt_g3_get_option");
    case VRT_G3_OPT_QUERY_TEAM_POSITIONS:
        return set_error(VRT_ERR_INVALID, "VRT_G3_OPT_QUERY_TEAM_POSITIONS is read with vrt_g3_get_option");
    case VRT_G3_OPT_QUERY_TEAM_CHUNKED:
        return set_error(VRT_ERR_INVALID, "VRT_G3_OPT_QUERY_TEAM_CHUNKED is read with vrt_g3_get_option");
    default: return set_error(VRT_ERR_INVALID, "unknown executor option %u", option);
    }
}

extern "C" int vrt_g3_get_option(vrt_g3* g, uint32_t option, uint32_t* value) {
    VRT_REQUIRE(g && value, "vrt_g3_get_option: null argument");
    switch (option) {
    case VRT_G3_OPT_USE_GRAPH: *value = g->use_graph ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_PERSISTENT: *value = g->use_persistent ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_TEAM: *value = g->use_team ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_KV_F16: *value = g->P.kv16 == 1u ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_KV_BF16: *value = g->P.kv16 == 2u ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_FUSION: *value = g->fusion ? 1u : 0u; return VRT_OK;
    case VRT_G3_OPT_Q8_LANES: *value = g->q8_lanes; return VRT_OK;
    case VRT_G3_OPT_QUERY_Q8_LANES:
        // lanes per row of the embedding-width (narrow) projections: the request, widened where a
        // row has more blocks per lane than instantiated, or with 0 the width sized from d_model
        *value = g->ld_qkv.S;
        return VRT_OK;
    case VRT_G3_OPT_QUERY_TEAM_POSITIONS: *value = tk_pos_limit(g); return VRT_OK;
    case VRT_G3_OPT_QUERY_TEAM_CHUNKED: *value = tk_chunk_from(g); return VRT_OK;
    default: return set_error(VRT_ERR_INVALID, "unknown executor option %u", option);
    }
}

extern "C" int vrt_g3_decode(vrt_g3* g, uint32_t token, uint32_t position, uint32_t top_k, vrt_argmax_result* out,
                             float* hidden_out) {
    VRT_REQUIRE(g, "vrt_g3_decode: null executor");
    if (position != g->next_pos) return set_error(VRT_ERR_STATE, "Gemma 3 decode positions must be contiguous");
    if (position >= g->cfg.context_length) return set_error(VRT_ERR_STATE, "Gemma 3 context length exceeded");
    if (token >= g->cfg.vocab_size) return g3_fail_reset(g, VRT_ERR_INVALID, "Token id is outside Gemma 3 vocabulary");
    hipStream_t s = g->ctx->stream;
    VRT_HIP_CHECK(hipMemcpyAsync(g->P.tokens + position, &token, 4, hipMemcpyHostToDevice, s));
    if (int rc = g3_write_ctl(g, position, top_k ? position : 0xffffffffu, 0xffffffffu, top_k > 1 ? 1u : 0u)) return rc;
    if (int rc = g3_run_steps(g, 1, position)) return g3_fail_reset(g, rc, vrt_last_error());
    if (hidden_out)
        VRT_HIP_CHECK(hipMemcpyAsync(hidden_out, g->P.hidden, g->cfg.embedding_length * 4u, hipMemcpyDeviceToHost, s));
    VRT_HIP_CHECK(hipMemcpyAsync(g->host_res, g->P.results + position, sizeof(vrt_argmax_result), hipMemcpyDeviceToHost, s));
    G3State st;
    if (int rc = g3_check_state(g, &st)) return rc;
    if (top_k) {
        const vrt_argmax_result r = g->host_res[0];
        if (r.index >= g->cfg.vocab_size || !std::isfinite(r.value))  // :1171-1176
            return g3_fail_reset(g, VRT_ERR_NUMERIC, "GPU argmax produced invalid result");
        if (out) *out = r;
    }
    g->next_pos = position + 1u;
    return VRT_OK;
}

extern "C" int vrt_g3_prefill(vrt_g3* g, const uint32_t* tokens, uint32_t n, uint32_t top_k, vrt_argmax_result* out,
                              float* hidden_out) {
    VRT_REQUIRE(g && tokens, "vrt_g3_prefill: null argument");
    if (n == 0) return set_error(VRT_ERR_INVALID, "Gemma 3 prompt produced no input tokens");
    if (n > g->cfg.context_length) return set_error(VRT_ERR_STATE, "Gemma 3 context length exceeded");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= g->cfg.vocab_size) return g3_fail_reset(g, VRT_ERR_INVALID, "Token id is outside Gemma 3 vocabulary");
    if (g->pf.max_t == 0u) {   // serial decode steps (src/gemma3.cpp:2099-2111)
        g->next_pos = 0;
        for (uint32_t i = 0; i < n; ++i)
            if (int rc = vrt_g3_decode(g, tokens[i], i, i + 1u == n ? top_k : 0u, out, i + 1u == n ? hidden_out : nullptr))
                return rc;
        return VRT_OK;
    }
    hipStream_t s = g->ctx->stream;
    g->next_pos = 0;
    VRT_HIP_CHECK(hipMemcpyAsync(g->P.tokens, tokens, n * 4u, hipMemcpyHostToDevice, s));
    if (int rc = g3_write_ctl(g, n - 1u, top_k ? n - 1u : 0xffffffffu, 0xffffffffu, top_k > 1 ? 1u : 0u)) return rc;
    // segments of at most max_t positions; each one's attention reads the earlier positions'
    // keys and values from the cache, and the last one runs the LM head
    for (uint32_t p0 = 0; p0 < n; p0 += g->pf.max_t) {
        const uint32_t T = std::min(g->pf.max_t, n - p0);
        if (int rc = pf_run(g, T, p0, p0 + T == n)) return g3_fail_reset(g, rc, vrt_last_error());
    }
    if (hidden_out)
        VRT_HIP_CHECK(hipMemcpyAsync(hidden_out, g->P.hidden, g->cfg.embedding_length * 4u, hipMemcpyDeviceToHost, s));
    VRT_HIP_CHECK(hipMemcpyAsync(g->host_res, g->P.results + (n - 1u), sizeof(vrt_argmax_result), hipMemcpyDeviceToHost, s));
    G3State st;
    if (int rc = g3_check_state(g, &st)) return rc;
    if (top_k) {
        const vrt_argmax_result r = g->host_res[0];
        if (r.index >= g->cfg.vocab_size || !std::isfinite(r.value))  // :1171-1176
            return g3_fail_reset(g, VRT_ERR_NUMERIC, "GPU argmax produced invalid result");
        if (out) *out = r;
    }
    g->next_pos = n;
    return VRT_OK;
}

extern "C" int vrt_g3_logits(vrt_g3* g, float* host, uint32_t n) {
    VRT_REQUIRE(g && host, "vrt_g3_logits: null argument");
    VRT_REQUIRE(n <= g->cfg.vocab_size, "vrt_g3_logits: n exceeds vocab_size");
    VRT_HIP_CHECK(hipMemcpyAsync(host, g->P.logits, static_cast<size_t>(n) * 4u, hipMemcpyDeviceToHost, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

extern "C" int vrt_g3_start(vrt_g3* g, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new) {
    VRT_REQUIRE(g, "vrt_g3_start: null executor");
    g->next_pos = 0;
    g->gen_prompt = 0;
    g->gen_max = 0;
    g->gen_steps = 0;
    if (max_new == 0) return vrt_g3_reset(g);
    VRT_REQUIRE(prompt, "vrt_g3_start: null prompt");
    if (n_prompt == 0) return set_error(VRT_ERR_INVALID, "Gemma 3 prompt produced no input tokens");
    const uint64_t steps = static_cast<uint64_t>(n_prompt) + max_new - 1u;
    if (steps > g->cfg.context_length) return set_error(VRT_ERR_STATE, "Gemma 3 context length exceeded");
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= g->cfg.vocab_size) return set_error(VRT_ERR_INVALID, "Token id is outside Gemma 3 vocabulary");
    hipStream_t s = g->ctx->stream;
    VRT_HIP_CHECK(hipMemcpyAsync(g->P.tokens, prompt, n_prompt * 4u, hipMemcpyHostToDevice, s));
    if (int rc = g3_write_ctl(g, 0, n_prompt - 1u, n_prompt, 0)) return rc;
    VRT_HIP_CHECK(hipStreamSynchronize(s));
    g->gen_prompt = n_prompt;
    g->gen_max = max_new;
    return VRT_OK;
}

extern "C" int vrt_g3_step(vrt_g3* g, uint32_t n) {
    VRT_REQUIRE(g, "vrt_g3_step: null executor");
    VRT_REQUIRE(g->gen_max != 0, "vrt_g3_step: no generation started");
    const uint64_t total = static_cast<uint64_t>(g->gen_prompt) + g->gen_max - 1u;
    VRT_REQUIRE(g->gen_steps + n <= total, "vrt_g3_step: more steps than the generation needs");
    if (int rc = g3_run_steps(g, n, static_cast<uint32_t>(g->gen_steps))) return g3_fail_reset(g, rc, vrt_last_error());
    g->gen_steps += n;
    return VRT_OK;
}

extern "C" int vrt_g3_collect(vrt_g3* g, uint32_t* out_tokens, uint32_t* n_out) {
    VRT_REQUIRE(g && n_out, "vrt_g3_collect: null argument");
    *n_out = 0;
    if (g->gen_max == 0) return VRT_OK;
    VRT_REQUIRE(out_tokens, "vrt_g3_collect: null output");
    const uint64_t total = static_cast<uint64_t>(g->gen_prompt) + g->gen_max - 1u;
    if (g->gen_steps < total)
        if (int rc = vrt_g3_step(g, static_cast<uint32_t>(total - g->gen_steps))) return rc;
    hipStream_t s = g->ctx->stream;
    VRT_HIP_CHECK(hipMemcpyAsync(g->host_res, g->P.results + (g->gen_prompt - 1u), g->gen_max * sizeof(vrt_argmax_result),
                                 hipMemcpyDeviceToHost, s));
    G3State st;
    if (int rc = g3_check_state(g, &st)) return rc;
    uint32_t n = 0;
    for (uint32_t i = 0; i < g->gen_max; ++i) {
        const vrt_argmax_result r = g->host_res[i];
        if (r.index >= g->cfg.vocab_size || !std::isfinite(r.value))                  // :1171-1176
            return g3_fail_reset(g, VRT_ERR_NUMERIC, "GPU argmax produced invalid result");
        out_tokens[n++] = r.index;
        if (r.index == g->eos) break;                                                  // :2134-2141
    }
    *n_out = n;
    g->next_pos = st.step;
    g->gen_max = 0;
    return VRT_OK;
}

extern "C" int vrt_g3_generate(vrt_g3* g, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                               uint32_t* out_tokens, uint32_t* n_out) {
    VRT_REQUIRE(g && n_out, "vrt_g3_generate: null argument");
    *n_out = 0;
    if (int rc = vrt_g3_start(g, prompt, n_prompt, max_new)) return rc;
    if (max_new == 0) return VRT_OK;
    return vrt_g3_collect(g, out_tokens, n_out);
}

extern "C" int vrt_g3_forced(vrt_g3* g, const uint32_t* tokens, uint32_t n, uint32_t first_logit_step,
                             vrt_argmax_result* out) {
    VRT_REQUIRE(g && tokens && out, "vrt_g3_forced: null argument");
    VRT_REQUIRE(n >= 1 && n <= g->cfg.context_length, "vrt_g3_forced: 1..context_length tokens");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= g->cfg.vocab_size) return set_error(VRT_ERR_INVALID, "Token id is outside Gemma 3 vocabulary");
    hipStream_t s = g->ctx->stream;
    g->next_pos = 0;
    VRT_HIP_CHECK(hipMemcpyAsync(g->P.tokens, tokens, n * 4u, hipMemcpyHostToDevice, s));
    if (int rc = g3_write_ctl(g, 0, first_logit_step, 0xffffffffu, 0)) return rc;
    if (int rc = g3_run_steps(g, n, 0u)) return g3_fail_reset(g, rc, vrt_last_error());
    VRT_HIP_CHECK(hipMemcpyAsync(out, g->P.results, n * sizeof(vrt_argmax_result), hipMemcpyDeviceToHost, s));
    G3State st;
    if (int rc = g3_check_state(g, &st)) return rc;
    g->next_pos = n;
    return VRT_OK;
}

extern "C" int vrt_g3_read_exchange(vrt_g3* g, uint32_t which, uint64_t* out, uint64_t cap, uint64_t* n) {
    VRT_REQUIRE(g && out && n, "vrt_g3_read_exchange: null argument");
    return mk_read_exchange(g, which, out, cap, n);
}

extern "C" int vrt_g3_read_trace(vrt_g3* g, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots) {
    VRT_REQUIRE(g && out && nwg && slots, "vrt_g3_read_trace: null argument");
    if (g->last_coop == kCoopTeam && g->tk) return tk_read_trace(g, out, cap, nwg, slots);
    return mk_read_trace(g, out, cap, nwg, slots);
}

extern "C" int vrt_g3_time_lm_head(vrt_g3* g, uint32_t iters, float* mean_us) {
    VRT_REQUIRE(g && mean_us && iters > 0, "vrt_g3_time_lm_head: bad argument");
    hipStream_t s = g->ctx->stream;
    const float* last_post = g->layers[g->cfg.block_count - 1].post_ffw;
    uint32_t mode = 1, nparts = g->ld_lm.grid;
    void* args[] = {&g->P, &last_post, &g->out_norm_dev, &g->lm_rows_per_wg, &mode};
    void* fargs[] = {&g->P, &nparts, &mode};
    hipEvent_t a, b;
    VRT_HIP_CHECK(hipEventCreate(&a));
    VRT_HIP_CHECK(hipEventCreate(&b));
    auto launch = [&]() -> int {
        VRT_HIP_CHECK(hipLaunchKernel(g->ld_lm.fn, dim3(g->ld_lm.grid), dim3(kThreads), args, g->ld_lm.smem, s));
        VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_lm_final), dim3(1), dim3(kThreads), fargs, 0, s));
        return VRT_OK;
    };
    if (int rc = launch()) return rc;   // warm-up
    VRT_HIP_CHECK(hipEventRecord(a, s));
    for (uint32_t i = 0; i < iters; ++i)
        if (int rc = launch()) return rc;
    VRT_HIP_CHECK(hipEventRecord(b, s));
    VRT_HIP_CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    VRT_HIP_CHECK(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *mean_us = ms * 1000.0f / static_cast<float>(iters);
    return VRT_OK;
}
