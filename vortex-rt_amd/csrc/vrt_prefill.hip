// vrt_prefill.hip -- batched prompt prefill of the Gemma 3 executor: every prompt position of
// a block at once. The projections are Q8_0 x activation GEMMs on MFMA, attention is causal
// with the local/global pattern, and the last position runs the fused LM head + argmax of the
// decode step. Afterwards the KV cache holds positions 0..T-1 exactly as T serial decode
// steps would have left it (src/gemma3.cpp:2099-2111), so decoding continues at T.
//
// GEMM numerics. C[m][n] = sum_b s[n][b] * sum_{k in b} A[m][k] * q[n][k] with s the block's
// f16 scale and q its int8 quants (exact in f16). A (fp32 activations) is split as
// A = hi + lo with hi = f16(A) and lo = f16(A - hi), so the two f16 MFMA products carry ~22
// bits of A; every f16 x f16 product is exact in fp32 and the MFMA accumulates in fp32. The
// per-block partial is scaled by s in fp32 and added to the fp32 accumulator.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <initializer_list>
#include <utility>

#include "vrt_g3_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kPfThreads = 256;
constexpr uint32_t kPfTile = 64;     // GEMM tile (rows and columns) of one workgroup
constexpr uint32_t kPfQT = 32;       // attention: queries per workgroup
constexpr uint32_t kPfKT = 32;       // attention: keys per LDS tile

// ---- row kernels ---------------------------------------------------------------------------

__device__ __forceinline__ void pf_split(float x, _Float16* hi, _Float16* lo) {
    const _Float16 h = static_cast<_Float16>(x);
    *hi = h;
    *lo = static_cast<_Float16>(x - static_cast<float>(h));
}

// Workgroup double sum (fixed order: 4 waves, DPP inside each).
__device__ __forceinline__ double pf_sum(double v, double* red) {
    v = wave_red_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// 1.0f / std::sqrt(float(sum_sq / n) + eps) (src/gemma3.cpp:967-983).
__device__ __forceinline__ float pf_rms_scale(double ss, uint32_t n, float eps) {
#pragma clang fp contract(off)
    return 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(n)) + eps);
}

// h[t] = dequantised embedding row of tokens[t] * emb_scale (src/gemma3.cpp:1106-1136).
__global__ void __launch_bounds__(kPfThreads) k_pf_embed(const uint8_t* tok_embd, const uint32_t* tokens, uint32_t d,
                                                         float emb_scale, float* h) {
#pragma clang fp contract(off)
    const uint32_t t = blockIdx.x;
    const uint8_t* row = tok_embd + static_cast<uint64_t>(tokens[t]) * (d / 32u) * 34u;
    for (uint32_t i = threadIdx.x; i < d; i += kPfThreads) {
        const uint8_t* b = row + (i >> 5) * 34u;
        const float sc = half_bits_to_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
        h[static_cast<uint64_t>(t) * d + i] = (sc * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31u)]))) * emb_scale;
    }
}

// One row t per workgroup (n <= 8 * kPfThreads). With f (the previous sublayer's output):
// h = (f * scale(f)) * w_post + h (src/gemma3.cpp:1703-1711, :1849-1855). Then, with w_next:
// the GEMM input (h * scale(h)) * w_next as f16 hi/lo (:991-996). nonfinite: lowest block
// whose residual went non-finite (:1857-1863), reported through st->nonfinite.
__global__ void __launch_bounds__(kPfThreads) k_pf_norm(float* h, const float* f, const float* w_post,
                                                        const float* w_next, uint32_t n, float eps, _Float16* xhi,
                                                        _Float16* xlo, G3State* st, uint32_t block) {
#pragma clang fp contract(off)
    __shared__ double red[4];
    const uint32_t t = blockIdx.x;
    float* hr = h + static_cast<uint64_t>(t) * n;
    float hv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t i = threadIdx.x + k * kPfThreads;
        hv[k] = i < n ? hr[i] : 0.0f;
    }
    if (f) {
        const float* fr = f + static_cast<uint64_t>(t) * n;
        float fv[8];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = threadIdx.x + k * kPfThreads;
            fv[k] = i < n ? fr[i] : 0.0f;
            ss += static_cast<double>(fv[k]) * static_cast<double>(fv[k]);
        }
        const float sc = pf_rms_scale(pf_sum(ss, red), n, eps);
        int bad = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = threadIdx.x + k * kPfThreads;
            if (i < n) {
                hv[k] = (fv[k] * sc) * w_post[i] + hv[k];
                hr[i] = hv[k];
                bad |= !__builtin_isfinite(hv[k]);
            }
        }
        if (bad) atomicMin(&st->nonfinite, block);
    }
    if (!w_next) return;
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += static_cast<double>(hv[k]) * static_cast<double>(hv[k]);
    const float sc = pf_rms_scale(pf_sum(ss, red), n, eps);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t i = threadIdx.x + k * kPfThreads;
        if (i < n) pf_split((hv[k] * sc) * w_next[i], xhi + static_cast<uint64_t>(t) * n + i, xlo + static_cast<uint64_t>(t) * n + i);
    }
}

// g = gelu_tanh(gate) * up for row t (gu = [gate(F) | up(F)] per row), as f16 hi/lo
// (shaders/gelu_mul.comp:23-31).
__global__ void __launch_bounds__(kPfThreads) k_pf_gelu(const float* gu, uint32_t F, _Float16* xhi, _Float16* xlo) {
#pragma clang fp contract(off)
    const uint32_t t = blockIdx.x;
    const float* r = gu + static_cast<uint64_t>(t) * 2u * F;
    for (uint32_t i = threadIdx.x; i < F; i += kPfThreads) {
        const float x = r[i];
        const float cubic = x * x * x;
        const float g = 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * cubic)));
        pf_split(g * r[F + i], xhi + static_cast<uint64_t>(t) * F + i, xlo + static_cast<uint64_t>(t) * F + i);
    }
}

// ---- Q8_0 x activation GEMM on MFMA ----------------------------------------------------------

struct PfGemm {
    const _Float16* ahi;     // [M][K] row-major
    const _Float16* alo;
    const uint8_t* w[3];     // Q8_0 matrices concatenated along N (rows[i] rows each)
    uint32_t rows[3];
    uint32_t nseg;
    uint32_t M, N, K;
    float* c;                // [M][N] row-major
    const uint8_t* w_end;    // one past the arena
};

// Workgroup tile 64 x 64, four waves of 32 x 32 (v_mfma_f32_32x32x16_f16). Lane l of a wave:
// A operand rows m = l % 32, k = 8 * (l / 32) + 0..7 of each 16-wide k step; B operand
// column n = l % 32 (a weight row), same k; accumulator element r at row
// 8 * (r / 4) + 4 * (l / 32) + r % 4, column l % 32 -- so the column's block scale is the
// lane's own. The next block's operands load while the current block's MFMAs run.
__global__ void __launch_bounds__(kPfThreads) k_pf_gemm(PfGemm G) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t kh = lane >> 5, l32 = lane & 31u;
    const uint32_t m = blockIdx.y * kPfTile + (wave >> 1) * 32u + l32;
    const uint32_t n = blockIdx.x * kPfTile + (wave & 1u) * 32u + l32;
    const bool mlive = m < G.M, nlive = n < G.N;
    const uint32_t nblk = G.K >> 5;
    const uint64_t row_bytes = static_cast<uint64_t>(nblk) * 34u;
    // this lane's weight row
    const uint8_t* wrow = G.w[0];
    {
        uint32_t r = nlive ? n : 0u, s = 0;
        while (s + 1u < G.nseg && r >= G.rows[s]) r -= G.rows[s++];
        wrow = G.w[s] + static_cast<uint64_t>(r) * row_bytes;
    }
    const uint64_t arow = static_cast<uint64_t>(mlive ? m : 0u) * G.K + 8u * kh;
    typedef const __attribute__((address_space(1))) half8* gh8;
    const uintptr_t ahi_base = reinterpret_cast<uintptr_t>(G.ahi), alo_base = reinterpret_cast<uintptr_t>(G.alo);
    auto load_a = [&](uint32_t b, half8 (&hi)[2], half8 (&lo)[2]) {
#pragma unroll
        for (uint32_t ks = 0; ks < 2; ++ks) {
            const uint64_t o = (arow + 32u * b + 16u * ks) * 2u;
            hi[ks] = *reinterpret_cast<gh8>(ahi_base + o);
            lo[ks] = *reinterpret_cast<gh8>(alo_base + o);
        }
    };
    auto to_half8 = [&](const Q8Raw& r, uint32_t j0) {
        half8 v;
        const uint32_t d0 = __builtin_amdgcn_alignbyte(r.d[j0 + 1], r.d[j0], r.sh);
        const uint32_t d1 = __builtin_amdgcn_alignbyte(r.d[j0 + 2], r.d[j0 + 1], r.sh);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(d0 >> (8 * j))));
            v[4 + j] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(d1 >> (8 * j))));
        }
        return v;
    };
    float16v acc = {};
    half8 ahi[2], alo[2], nhi[2], nlo[2];
    Q8Raw raw, nraw;
    load_a(0, ahi, alo);
    q8_load(wrow, G.w_end, raw);
    for (uint32_t b = 0; b < nblk; ++b) {
        if (b + 1u < nblk) {
            load_a(b + 1u, nhi, nlo);
            q8_load(wrow + 34u * (b + 1u), G.w_end, nraw);
        }
        const half8 w0 = to_half8(raw, 2u * kh), w1 = to_half8(raw, 4u + 2u * kh);
        float16v p1 = {}, p2 = {};
        p1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[0], w0, p1, 0, 0, 0);
        p2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[0], w0, p2, 0, 0, 0);
        p1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi[1], w1, p1, 0, 0, 0);
        p2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo[1], w1, p2, 0, 0, 0);
        const float s = half_bits_to_float(raw.sbits);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += s * (p1[r] + p2[r]);
        if (b + 1u < nblk) {
            ahi[0] = nhi[0]; ahi[1] = nhi[1]; alo[0] = nlo[0]; alo[1] = nlo[1];
            raw = nraw;
        }
    }
    if (!nlive) return;
    const uint32_t mb = blockIdx.y * kPfTile + (wave >> 1) * 32u;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t row = mb + 8u * (r / 4) + 4u * kh + (r % 4);
        if (row < G.M) G.c[static_cast<uint64_t>(row) * G.N + n] = acc[r];
    }
}

// ---- QK-norm, RoPE, KV cache ------------------------------------------------------------

// Row t of qkv = [q (H heads x hd) | k (hd) | v (hd)]: QK-norm per head (src/gemma3.cpp:
// 1045-1104), NeoX RoPE at position t (:1371-1424), in place; then k and v go to the KV
// cache slot t % slots when position t is still in the window after the prompt (the serial
// loop's eviction leaves exactly those, :1590-1600).
__global__ void __launch_bounds__(kPfThreads) k_pf_qk(float* qkv, uint32_t T, uint32_t H, uint32_t hd, const float* q_norm,
                                                      const float* k_norm, const float* cos_t, const float* sin_t,
                                                      float eps, float* kc, float* vc, uint32_t slots) {
#pragma clang fp contract(off)
    __shared__ double red[4];
    __shared__ float xs[256];
    const uint32_t t = blockIdx.x;
    const uint32_t nqkv = (H + 2u) * hd, half = hd >> 1;
    float* row = qkv + static_cast<uint64_t>(t) * nqkv;
    const uint32_t i = threadIdx.x;
    for (uint32_t hh = 0; hh <= H; ++hh) {   // H query heads, then the key head
        float* x = row + hh * hd;
        const float v = i < hd ? x[i] : 0.0f;
        const float sc = pf_rms_scale(pf_sum(static_cast<double>(v) * static_cast<double>(v), red), hd, eps);
        const float* w = hh < H ? q_norm : k_norm;
        const float y = i < hd ? (v * sc) * w[i] : 0.0f;
        if (i < hd) xs[i] = y;
        __syncthreads();
        if (i < hd) {
            const uint32_t e = i < half ? i : i - half;
            const float c = cos_t[static_cast<uint64_t>(t) * half + e], s = sin_t[static_cast<uint64_t>(t) * half + e];
            const float a = xs[e], b = xs[e + half];
            x[i] = i < half ? a * c - b * s : b * c + a * s;
        }
        __syncthreads();
    }
    if (t + slots >= T && i < hd) {
        const uint64_t slot = static_cast<uint64_t>(t % slots) * hd;
        kc[slot + i] = row[H * hd + i];
        vc[slot + i] = row[(H + 1u) * hd + i];
    }
}

// ---- causal attention -----------------------------------------------------------------------

// One workgroup per (32 queries, head h). Key tiles of 32 in LDS; each thread scores one query
// against 4 keys, then owns hd/8 output dims of its query (online softmax, fp32). Keys j of
// query t: j <= t and t - j < window (window = slots of a local block). Output as f16 hi/lo
// att[t][h * hd + e]. Each tile's K and V rows are fetched into registers (float4 loads, all
// in flight together) while the previous tile is being used, then stored to LDS; LDS rows
// are padded by 4 floats against bank conflicts.
template <uint32_t HD>
__global__ void __launch_bounds__(kPfThreads) k_pf_attn(const float* qkv, uint32_t T, uint32_t H, uint32_t window,
                                                        float scale, _Float16* ahi, _Float16* alo) {
    constexpr uint32_t LD = HD + 4u;
    constexpr uint32_t DPT = HD / 8u;                        // output dims per thread
    constexpr uint32_t NV = kPfKT * HD / 4u / kPfThreads;    // f4 of a K (or V) tile per thread
    static_assert(NV >= 1u && NV * 4u * kPfThreads == kPfKT * HD, "tile shape");
    extern __shared__ float sm[];
    float* Qs = sm;                      // [QT][LD]
    float* Ks = Qs + kPfQT * LD;         // [KT][LD]
    float* Vs = Ks + kPfKT * LD;         // [KT][LD]
    float* Ps = Vs + kPfKT * LD;         // [QT][KT + 1]
    const uint32_t t0 = blockIdx.x * kPfQT, h = blockIdx.y;
    const uint32_t nq = min(kPfQT, T - t0);
    const uint32_t nqkv = (H + 2u) * HD;
    const uint32_t tid = threadIdx.x;
    const f4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t i = 0; i < kPfQT * HD / 4u / kPfThreads; ++i) {
        const uint32_t idx = tid + i * kPfThreads, q = idx / (HD / 4u), e = 4u * (idx % (HD / 4u));
        *reinterpret_cast<f4*>(Qs + q * LD + e) =
            q < nq ? *reinterpret_cast<const f4*>(qkv + static_cast<uint64_t>(t0 + q) * nqkv + h * HD + e) : zero4;
    }
    const uint32_t qi = tid >> 3, kg = tid & 7u;   // query of this thread, its key group / dim group
    const uint32_t t = t0 + qi;
    float acc[DPT];
#pragma unroll
    for (uint32_t j = 0; j < DPT; ++j) acc[j] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const uint32_t k_first = (window != 0u && t0 + 1u > window) ? t0 + 1u - window : 0u;
    const uint32_t k_end = t0 + nq;
    f4 kreg[NV], vreg[NV];
    const uint32_t kb0 = k_first - (k_first % kPfKT);
    // this thread's f4 of each tile: row k = i * (KT / NV) + tid / (HD / 4), column
    // e = 4 * (tid % (HD / 4)); rows past k_end load as zero (clamped address, masked value)
    const uint32_t frow = tid / (HD / 4u), fcol = 4u * (tid % (HD / 4u));
#pragma unroll
    for (uint32_t i = 0; i < NV; ++i) {
        const uint32_t k = i * (kPfKT / NV) + frow;
        const bool live = kb0 + k < k_end;
        const float* row = qkv + static_cast<uint64_t>(live ? kb0 + k : 0u) * nqkv + fcol;
        const f4 kv = *reinterpret_cast<const f4*>(row + H * HD);
        const f4 vv = *reinterpret_cast<const f4*>(row + (H + 1u) * HD);
        kreg[i] = live ? kv : zero4;
        vreg[i] = live ? vv : zero4;
    }
    for (uint32_t kb = kb0; kb < k_end; kb += kPfKT) {
        __syncthreads();   // the previous tile's LDS is no longer read
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t k = i * (kPfKT / NV) + frow;
            *reinterpret_cast<f4*>(Ks + k * LD + fcol) = kreg[i];
            *reinterpret_cast<f4*>(Vs + k * LD + fcol) = vreg[i];
        }
        __syncthreads();
        const uint32_t kn = kb + kPfKT;   // the next tile is in flight while this one is used
#pragma unroll
        for (uint32_t i = 0; i < NV; ++i) {
            const uint32_t k = i * (kPfKT / NV) + frow;
            const bool live = kn + k < k_end;
            const float* row = qkv + static_cast<uint64_t>(live ? kn + k : 0u) * nqkv + fcol;
            const f4 kv = *reinterpret_cast<const f4*>(row + H * HD);
            const f4 vv = *reinterpret_cast<const f4*>(row + (H + 1u) * HD);
            kreg[i] = live ? kv : zero4;
            vreg[i] = live ? vv : zero4;
        }
        // scores of query qi against keys kb + 4 kg .. + 3
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
        for (uint32_t e = 0; e < HD; e += 4u) {
            const f4 qv = *reinterpret_cast<const f4*>(Qs + qi * LD + e);
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const f4 kv = *reinterpret_cast<const f4*>(Ks + (4u * kg + j) * LD + e);
                s[j] = fmaf(qv.x, kv.x, s[j]);
                s[j] = fmaf(qv.y, kv.y, s[j]);
                s[j] = fmaf(qv.z, kv.z, s[j]);
                s[j] = fmaf(qv.w, kv.w, s[j]);
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t k = kb + 4u * kg + j;
            const bool ok = qi < nq && k <= t && (window == 0u || t - k < window);
            s[j] = ok ? s[j] * scale : -INFINITY;
            mx = fmaxf(mx, s[j]);
        }
        // row max / sum over the 8 threads of query qi (adjacent lanes)
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mx = fmaxf(mx, __shfl_xor(mx, 4));
        const float m_new = fmaxf(m_run, mx);
        float ls = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const float p = s[j] == -INFINITY ? 0.0f : expf(s[j] - m_new);
            Ps[qi * (kPfKT + 1u) + 4u * kg + j] = p;
            ls += p;
        }
        ls += __shfl_xor(ls, 1);
        ls += __shfl_xor(ls, 2);
        ls += __shfl_xor(ls, 4);
        const float r = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
        l_run = l_run * r + ls;
        m_run = m_new;
        __syncthreads();
        // acc = acc * r + sum_k p_k v_k over this thread's dims e = 4 kg + 32 j' (+0..3)
#pragma unroll
        for (uint32_t j = 0; j < DPT; ++j) acc[j] *= r;
#pragma unroll 4
        for (uint32_t k = 0; k < kPfKT; ++k) {
            const float p = Ps[qi * (kPfKT + 1u) + k];
#pragma unroll
            for (uint32_t j = 0; j < DPT / 4u; ++j) {
                const f4 vv = *reinterpret_cast<const f4*>(Vs + k * LD + 4u * kg + 32u * j);
                acc[4 * j + 0] = fmaf(p, vv.x, acc[4 * j + 0]);
                acc[4 * j + 1] = fmaf(p, vv.y, acc[4 * j + 1]);
                acc[4 * j + 2] = fmaf(p, vv.z, acc[4 * j + 2]);
                acc[4 * j + 3] = fmaf(p, vv.w, acc[4 * j + 3]);
            }
        }
    }
    if (qi >= nq) return;
    const float inv = 1.0f / l_run;
    const uint64_t o = static_cast<uint64_t>(t) * H * HD + h * HD;
#pragma unroll
    for (uint32_t j = 0; j < DPT / 4u; ++j)
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            const uint32_t e = 4u * kg + 32u * j + c;
            pf_split(acc[4 * j + c] * inv, ahi + o + e, alo + o + e);
        }
}

// ---- host side --------------------------------------------------------------------------

static int pf_gemm(vrt_g3* g, const _Float16* ahi, const _Float16* alo, uint32_t M, uint32_t K,
                   std::initializer_list<std::pair<const uint8_t*, uint32_t>> segs, float* c, hipStream_t s) {
    PfGemm G{};
    G.ahi = ahi;
    G.alo = alo;
    G.nseg = 0;
    G.N = 0;
    for (const auto& sg : segs) {
        G.w[G.nseg] = sg.first;
        G.rows[G.nseg++] = sg.second;
        G.N += sg.second;
    }
    G.M = M;
    G.K = K;
    G.c = c;
    G.w_end = g->P.arena_end;
    if (K % 32u != 0u || G.N % 32u != 0u) return set_error(VRT_ERR_INVALID, "prefill GEMM shape not supported");
    dim3 grid((G.N + kPfTile - 1u) / kPfTile, (M + kPfTile - 1u) / kPfTile);
    void* args[] = {&G};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_gemm), grid, dim3(kPfThreads), args, 0, s));
    return VRT_OK;
}

static const void* pf_attn_fn(uint32_t hd) {
    return hd == 256u ? reinterpret_cast<const void*>(&k_pf_attn<256>)
         : hd == 128u ? reinterpret_cast<const void*>(&k_pf_attn<128>)
                      : reinterpret_cast<const void*>(&k_pf_attn<64>);
}

static size_t pf_attn_smem(uint32_t hd) {
    return ((kPfQT + 2u * kPfKT) * (hd + 4u) + kPfQT * (kPfKT + 1u)) * 4u;
}

int pf_setup(vrt_g3* g, uint32_t max_t) {
    const uint32_t d = g->cfg.embedding_length, H = g->cfg.head_count, hd = g->cfg.head_dim;
    const uint32_t F = g->cfg.feed_forward_length, qw = H * hd, nqkv = qw + 2u * hd;
    const uint32_t kmax = std::max(std::max(d, qw), F);
    PfState& p = g->pf;
    p.max_t = 0;
    if (d > 8u * kPfThreads || hd > 256u || (hd != 64u && hd != 128u && hd != 256u) || d % 32u || qw % 32u ||
        F % 32u || nqkv % 32u)
        return VRT_OK;   // prefill unavailable for this shape: vrt_g3_prefill falls back to decode steps
    auto take = [&](size_t bytes, void** out) -> int {
        VRT_HIP_CHECK(hipMalloc(out, bytes + 256u));
        g->allocs.push_back(*out);
        return VRT_OK;
    };
    void* q;
    if (int rc = take(static_cast<size_t>(max_t) * d * 4u, &q)) return rc;
    p.h = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(max_t) * d * 4u, &q)) return rc;
    p.x = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(max_t) * kmax * 2u, &q)) return rc;
    p.ahi = q;
    if (int rc = take(static_cast<size_t>(max_t) * kmax * 2u, &q)) return rc;
    p.alo = q;
    if (int rc = take(static_cast<size_t>(max_t) * std::max(nqkv, 2u * F) * 4u, &q)) return rc;
    p.big = static_cast<float*>(q);
    VRT_HIP_CHECK(hipFuncSetAttribute(pf_attn_fn(hd), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(pf_attn_smem(hd))));
    p.max_t = max_t;
    return VRT_OK;
}

// T prompt positions 0..T-1 on the context's stream; the last one runs the LM head + argmax
// (results[T-1], logits when want_logits). The caller has reset the step state.
int pf_run(vrt_g3* g, uint32_t T) {
    const PfState& p = g->pf;
    hipStream_t s = g->ctx->stream;
    uint32_t d = g->cfg.embedding_length, H = g->cfg.head_count, hd = g->cfg.head_dim;
    uint32_t F = g->cfg.feed_forward_length;
    const uint32_t qw = H * hd, L = g->cfg.block_count;
    const G3Params& P = g->P;
    _Float16* ahi = static_cast<_Float16*>(p.ahi);
    _Float16* alo = static_cast<_Float16*>(p.alo);
    float* h = p.h;
    float* x = p.x;
    float* big = p.big;
    float eps = P.eps;
    G3State* st = P.st;
    auto launch = [&](const void* fn, dim3 grid, void** args, size_t smem) -> int {
        VRT_HIP_CHECK(hipLaunchKernel(fn, grid, dim3(kPfThreads), args, smem, s));
        return VRT_OK;
    };
    {
        const uint8_t* te = P.tok_embd;
        const uint32_t* tok = P.tokens;
        float es = P.emb_scale;
        void* args[] = {&te, &tok, &d, &es, &h};
        if (int rc = launch(reinterpret_cast<const void*>(&k_pf_embed), dim3(T), args, 0)) return rc;
    }
    for (uint32_t l = 0; l < L; ++l) {
        const LayerParams& Ly = g->layers[l];
        {   // previous block's FFN output into the residual, then the attention norm
            const float* f = l ? x : nullptr;
            const float* wpost = l ? g->layers[l - 1].post_ffw : nullptr;
            const float* wnext = Ly.attn_norm;
            uint32_t blk = l ? l - 1u : 0u;
            void* args[] = {&h, &f, &wpost, &wnext, &d, &eps, &ahi, &alo, &st, &blk};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_norm), dim3(T), args, 0)) return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, d, {{Ly.wq, qw}, {Ly.wk, hd}, {Ly.wv, hd}}, big, s)) return rc;
        {
            const float* qn = Ly.q_norm;
            const float* kn = Ly.k_norm;
            const float* ct = Ly.global ? P.cos_g : P.cos_l;
            const float* sn = Ly.global ? P.sin_g : P.sin_l;
            float* kc = Ly.kc;
            float* vc = Ly.vc;
            uint32_t slots = Ly.slots;
            void* args[] = {&big, &T, &H, &hd, &qn, &kn, &ct, &sn, &eps, &kc, &vc, &slots};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_qk), dim3(T), args, 0)) return rc;
        }
        {
            uint32_t window = Ly.slots >= g->cfg.context_length ? 0u : Ly.slots;
            float scale = P.attn_scale;
            const float* qkv = big;
            void* args[] = {&qkv, &T, &H, &window, &scale, &ahi, &alo};
            const dim3 grid((T + kPfQT - 1u) / kPfQT, H);
            if (int rc = launch(pf_attn_fn(hd), grid, args, pf_attn_smem(hd))) return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, qw, {{Ly.wo, d}}, x, s)) return rc;
        {   // attention output into the residual, then the FFN norm
            const float* f = x;
            const float* wpost = Ly.post_attn;
            const float* wnext = Ly.ffn_norm;
            uint32_t blk = l;
            void* args[] = {&h, &f, &wpost, &wnext, &d, &eps, &ahi, &alo, &st, &blk};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_norm), dim3(T), args, 0)) return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, d, {{Ly.wg, F}, {Ly.wu, F}}, big, s)) return rc;
        {
            const float* gu = big;
            void* args[] = {&gu, &F, &ahi, &alo};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_gelu), dim3(T), args, 0)) return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, F, {{Ly.wd, d}}, x, s)) return rc;
    }
    // last position: its FFN output and residual feed the decode step's final norm + LM head
    VRT_HIP_CHECK(hipMemcpyAsync(P.f, x + static_cast<uint64_t>(T - 1u) * d, d * 4u, hipMemcpyDeviceToDevice, s));
    VRT_HIP_CHECK(hipMemcpyAsync(P.hmid, h + static_cast<uint64_t>(T - 1u) * d, d * 4u, hipMemcpyDeviceToDevice, s));
    return g3_enqueue_lm(g, s);
}

}  // namespace vrt
