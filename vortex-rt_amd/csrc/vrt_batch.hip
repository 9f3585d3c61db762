// vrt_batch.hip -- batched greedy decode of independent Gemma 3 sequences (vrt_g3_batch_*).
//
// The reference decodes one sequence per model (src/gemma3.cpp:1462-1882); its roadmap lists
// continuous batching (README.md:193). Here n sequences, each with its own KV cache and
// position, advance one position per step together. The rows of a step are the n sequences'
// current tokens, so every projection is an n-row GEMM over the shared weights on MFMA (the
// prefill's kernels, vrt_prefill.hip): the weights stream once per step for all n rows, which
// is what makes a batch cheaper per token than n batch-1 steps. Per block:
//   k_pf_norm_w   residual fold of the previous block's FFN output + attention RMSNorm (rows)
//   GEMM          q|k|v of the n rows (K split, partials summed by the consumer)
//   k_bd_attn     per (history chunk, row): QK-norm, RoPE at the row's position, KV append to
//                 the row's sequence, chunk of the attention (max, sum, weighted V per head)
//   k_bd_merge    per (head, row): the chunks combined, as f16 hi/lo GEMM input
//   GEMM          O projection; k_pf_norm_w (post-attention norm + residual + FFN norm)
//   GEMM          gelu_tanh(gate) * up; GEMM down projection
// then the final residual + output norm (k_pf_norm_w), the logits of the n rows against the
// tied embedding table (GEMM) and a greedy argmax per row (k_bd_argmax, k_bd_argmax_final).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "vrt_g3_errors.hpp"
#include "vrt_g3_internal.hpp"
#include "vrt_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {

constexpr uint32_t kBdThreads = 256;
constexpr uint32_t kBdMaxChunks = 64;     // history chunks per row and block, at most
constexpr uint32_t kBdMaxRows = 64;       // sequences per step (one 64-row GEMM tile)
constexpr uint32_t kBdArgParts = 256;     // argmax partials per row
constexpr uint32_t kBdMaxSplits = 4;      // K splits of a projection (the consumers' limit)

// One block's attention over the rows of a step.
struct BdAttn {
    const float* qkv;         // [nsplit][n][(H + 2) hd] split partials of the q|k|v projection
    uint64_t sstride;         // floats from one partial to the next
    uint32_t nsplit;
    const uint32_t* pos;      // [n] position of row b
    const uint32_t* seq;      // [n] sequence of row b
    float* kc;                // [max_seqs][slots][hd] key cache of the block
    float* vc;                //   and value cache
    uint32_t slots, H, hd, G, cmax;   // G chunks per row; cmax positions per chunk at most
    const float* q_norm;
    const float* k_norm;
    const float* cos_t;       // [context][hd / 2] RoPE tables of the block's kind
    const float* sin_t;
    float eps, attn_scale;
    float* part;              // [n][G][2 H + H hd]: m and l per head, then acc per head
    _Float16* ohi;            // [n][H hd] attention output, f16 high part
    _Float16* olo;            //   ... and low part
    G3State* st;
    uint32_t block;
};

// Chunking of a row's history: n_hist positions [t_first, pos], G chunks of C positions, the
// first n_act of them non-empty.
__device__ __forceinline__ void bd_chunks(const BdAttn& A, uint32_t p, uint32_t& t_first, uint32_t& C,
                                          uint32_t& n_act) {
    const uint32_t n_hist = min(p + 1u, A.slots);   // local layers keep the last `slots` (src/gemma3.cpp:1590-1600)
    t_first = p + 1u - n_hist;
    C = (n_hist + A.G - 1u) / A.G;
    n_act = (n_hist + C - 1u) / C;
}

// One workgroup per (chunk c, row b). The row's q (H heads), k and v (the split partials added
// in order) go to LDS; one wave per head applies QK-norm (values *= scale * weights,
// src/gemma3.cpp:1045-1104) and NeoX RoPE at the row's position (:1371-1424). The workgroup
// of the last chunk appends k and v to the row's sequence at slot pos % slots (positions of
// this step are read from LDS, never from the cache). Scores of the chunk's positions (wave w
// takes positions c0 + w + 4 i; a wave reduction per head), then per head the chunk maximum,
// e^(s - m) and their sum (double), then the weighted values (thread per head dimension):
// the chunk's partial {m, l, acc} of the masked softmax of :1602-1696.
__global__ void __launch_bounds__(kBdThreads) k_bd_attn(BdAttn A) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float s_bd[];
    const uint32_t c = blockIdx.x, b = blockIdx.y;
    const uint32_t H = A.H, hd = A.hd, half = hd >> 1, nq = (H + 2u) * hd;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t p = A.pos[b], sq = A.seq[b];
    uint32_t t_first, C, n_act;
    bd_chunks(A, p, t_first, C, n_act);
    if (c >= n_act) return;   // whole workgroup
    const uint32_t c0 = t_first + c * C, c1 = min(p + 1u, c0 + C);
    float* sx = s_bd;        // [H + 2][hd]: q heads, k, v
    float* ssc = s_bd + nq;  // [H][cmax]: scores, then weights
    // q|k|v of row b: every load issued at a clamped index before the first add
    {
        constexpr uint32_t kPer = (8u + 2u) * 256u / kBdThreads;   // H <= 8, hd <= 256
        const float* src = A.qkv + static_cast<uint64_t>(b) * nq;
        float pv[kPer][kBdMaxSplits];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t i = min(tid + kBdThreads * k, nq - 1u);
#pragma unroll
            for (uint32_t z = 0; z < kBdMaxSplits; ++z) pv[k][z] = src[min(z, A.nsplit - 1u) * A.sstride + i];
        }
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            float v = 0.0f;
#pragma unroll
            for (uint32_t z = 0; z < kBdMaxSplits; ++z)
                if (z < A.nsplit) v += pv[k][z];
            if (tid + kBdThreads * k < nq) sx[tid + kBdThreads * k] = v;
        }
    }
    __syncthreads();
    // QK-norm and RoPE, one wave per head (heads 0..H-1 query, H key); lane l: dims l + 64 e
    {
        uint32_t ic[4], ei[4];
        bool live[4];
        float cs[4], sn[4];
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            live[e] = lane + 64u * e < hd;
            ic[e] = min(lane + 64u * e, hd - 1u);
            ei[e] = ic[e] < half ? ic[e] : ic[e] - half;
            cs[e] = A.cos_t[static_cast<uint64_t>(p) * half + ei[e]];
            sn[e] = A.sin_t[static_cast<uint64_t>(p) * half + ei[e]];
        }
        for (uint32_t hh = wave; hh <= H; hh += kBdThreads / 64u) {
            float* x = sx + hh * hd;
            const float* w = hh < H ? A.q_norm : A.k_norm;
            float v[4], wv[4];
            double ss = 0.0;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                wv[e] = w[ic[e]];
                v[e] = live[e] ? x[ic[e]] : 0.0f;
                ss += static_cast<double>(v[e]) * static_cast<double>(v[e]);
            }
            const double tot = wave_red_sum_d(ss);
            const float sc = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(hd)) + A.eps);   // :1087-1093
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e)
                if (live[e]) x[ic[e]] = v[e] * (sc * wv[e]);
            __builtin_amdgcn_wave_barrier();   // a wave's LDS accesses complete in order
            float y[4];
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                const float a = x[ei[e]], bb = x[ei[e] + half];
                y[e] = ic[e] < half ? a * cs[e] - bb * sn[e] : bb * cs[e] + a * sn[e];
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e)
                if (live[e]) x[ic[e]] = y[e];
        }
    }
    __syncthreads();
    const float* sk = sx + H * hd;
    const float* sv = sk + hd;
    const uint64_t cache0 = static_cast<uint64_t>(sq) * A.slots * hd;
    if (c + 1u == n_act)   // KV append of this row's position (:1590-1600)
        for (uint32_t i = tid; i < hd; i += kBdThreads) {
            const uint64_t o = cache0 + static_cast<uint64_t>(p % A.slots) * hd + i;
            A.kc[o] = sk[i];
            A.vc[o] = sv[i];
        }
    // scores of the chunk's positions: wave w takes positions c0 + w + 4 i, eight at a time, their
    // key rows loaded together first (at clamped positions; the current position comes from LDS)
    constexpr uint32_t kG8 = 8u, nw = kBdThreads / 64u;
    for (uint32_t t0 = c0 + wave; t0 < c1; t0 += nw * kG8) {
        float kr[kG8][4];
#pragma unroll
        for (uint32_t u = 0; u < kG8; ++u) {
            const uint64_t row = cache0 + static_cast<uint64_t>(min(t0 + nw * u, c1 - 1u) % A.slots) * hd;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) kr[u][e] = A.kc[row + min(lane + 64u * e, hd - 1u)];
        }
#pragma unroll
        for (uint32_t u = 0; u < kG8; ++u) {
            const uint32_t t = t0 + nw * u;
            if (t >= c1) break;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e)
                if (t == p) kr[u][e] = sk[min(lane + 64u * e, hd - 1u)];
            for (uint32_t h = 0; h < H; ++h) {
                float d = 0.0f;
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e)
                    if (lane + 64u * e < hd) d += sx[h * hd + lane + 64u * e] * kr[u][e];
                d = wave_sum(d);
                if (lane == 0u) ssc[h * A.cmax + (t - c0)] = d * A.attn_scale;
            }
        }
    }
    __syncthreads();
    // chunk statistics per head: m = max, e = exp(s - m), l = sum e (double)
    const uint32_t ncp = c1 - c0;
    float* mypart = A.part + (static_cast<uint64_t>(b) * A.G + c) * (2u * H + H * hd);
    for (uint32_t h = wave; h < H; h += kBdThreads / 64u) {
        float mx = -INFINITY;
        for (uint32_t t = lane; t < ncp; t += 64u) mx = fmaxf(mx, ssc[h * A.cmax + t]);
        mx = wave_max(mx);
        double l = 0.0;
        for (uint32_t t = lane; t < ncp; t += 64u) {
            const float e = expf(ssc[h * A.cmax + t] - mx);
            ssc[h * A.cmax + t] = e;
            l += e;
        }
        l = wave_sum_f64(l);
        if (lane == 0u) {
            mypart[h] = mx;
            mypart[H + h] = static_cast<float>(l);
        }
    }
    __syncthreads();
    // weighted values: thread i owns dims i, i + 256, ...; eight positions' values loaded together
    for (uint32_t i = tid; i < hd; i += kBdThreads) {
        float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t t0 = c0; t0 < c1; t0 += kG8) {
            float vv[kG8];
#pragma unroll
            for (uint32_t u = 0; u < kG8; ++u)
                vv[u] = A.vc[cache0 + static_cast<uint64_t>(min(t0 + u, c1 - 1u) % A.slots) * hd + i];
#pragma unroll
            for (uint32_t u = 0; u < kG8; ++u) {
                const uint32_t t = t0 + u;
                if (t >= c1) break;
                const float x = t == p ? sv[i] : vv[u];
#pragma unroll
                for (uint32_t h = 0; h < 8u; ++h)
                    if (h < H) acc[h] += ssc[h * A.cmax + (t - c0)] * x;
            }
        }
#pragma unroll
        for (uint32_t h = 0; h < 8u; ++h)
            if (h < H) mypart[2u * H + h * hd + i] = acc[h];
    }
}

constexpr uint32_t kBdShort = 32;   // rows whose histories are all this short take k_bd_attn_short

// Histories of at most kBdShort positions: one workgroup per (head h, row b) runs the head's whole
// attention and writes its output, with no chunk partials to merge. The cached key and value rows
// are loaded first, before the q|k|v split partials are added, so the loads overlap. Waves 0 and 1
// apply QK-norm and NeoX RoPE to q_h and k (src/gemma3.cpp:1045-1104, :1371-1424); the head-0
// workgroup appends k and v at slot pos % slots (:1590-1600). The scores (wave w: positions
// t_first + w + 4 u), the maximum, e^(s - m) with their double sum, the weighted values (thread per
// dimension, positions in order) and the division follow k_bd_attn and k_bd_merge for one chunk
// (:1602-1696). The current position's k and v come from LDS, never from the cache.
__global__ void __launch_bounds__(kBdThreads) k_bd_attn_short(BdAttn A) {
#pragma clang fp contract(off)
    __shared__ float sq[256], sk[256], sv[256];
    __shared__ float ssc[kBdShort];
    __shared__ double s_l;
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    const uint32_t H = A.H, hd = A.hd, half = hd >> 1, nq = (H + 2u) * hd;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t p = A.pos[b], sqn = A.seq[b];
    const uint32_t n_full = min(p + 1u, A.slots), t_first = p + 1u - n_full;
    const uint32_t n_hist = min(n_full, kBdShort);   // the host sends no longer history here
    const uint64_t cache0 = static_cast<uint64_t>(sqn) * A.slots * hd;
    const uint32_t di = min(tid, hd - 1u);
    // cached key rows (wave w: positions t_first + w + 4 u; lane: dims lane + 64 e) and value rows
    // (thread: its dimension, every position), at clamped in-bounds positions
    float kr[8][4], vv[kBdShort];
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
        const uint64_t row = cache0 + static_cast<uint64_t>(min(t_first + wave + 4u * u, p) % A.slots) * hd;
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) kr[u][e] = A.kc[row + min(lane + 64u * e, hd - 1u)];
    }
#pragma unroll
    for (uint32_t u = 0; u < kBdShort; ++u)
        vv[u] = A.vc[cache0 + static_cast<uint64_t>(min(t_first + u, p) % A.slots) * hd + di];
    float rc[4], rs[4];   // RoPE table entries of the dims lane + 64 e (waves 0 and 1 use them)
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        const uint32_t ic = min(lane + 64u * e, hd - 1u), ei = ic < half ? ic : ic - half;
        rc[e] = A.cos_t[static_cast<uint64_t>(p) * half + ei];
        rs[e] = A.sin_t[static_cast<uint64_t>(p) * half + ei];
    }
    {   // q of head h, k and v: the split partials added in order
        const float* src = A.qkv + static_cast<uint64_t>(b) * nq;
        float pq[kBdMaxSplits], pk[kBdMaxSplits], pw[kBdMaxSplits];
#pragma unroll
        for (uint32_t z = 0; z < kBdMaxSplits; ++z) {
            const uint64_t o = static_cast<uint64_t>(min(z, A.nsplit - 1u)) * A.sstride;
            pq[z] = src[o + h * hd + di];
            pk[z] = src[o + H * hd + di];
            pw[z] = src[o + (H + 1u) * hd + di];
        }
        float a = 0.0f, c = 0.0f, e = 0.0f;
#pragma unroll
        for (uint32_t z = 0; z < kBdMaxSplits; ++z)
            if (z < A.nsplit) { a += pq[z]; c += pk[z]; e += pw[z]; }
        if (tid < hd) { sq[tid] = a; sk[tid] = c; sv[tid] = e; }
    }
    __syncthreads();
    if (wave < 2u) {   // QK-norm and RoPE of q_h (wave 0) and k (wave 1); lane l: dims l + 64 e
        float* x = wave == 0u ? sq : sk;
        const float* w = wave == 0u ? A.q_norm : A.k_norm;
        uint32_t ic[4], ei[4];
        bool live[4];
        float v[4], wv[4];
        double ss = 0.0;
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            live[e] = lane + 64u * e < hd;
            ic[e] = min(lane + 64u * e, hd - 1u);
            ei[e] = ic[e] < half ? ic[e] : ic[e] - half;
            wv[e] = w[ic[e]];
            v[e] = live[e] ? x[ic[e]] : 0.0f;
            ss += static_cast<double>(v[e]) * static_cast<double>(v[e]);
        }
        const double tot = wave_red_sum_d(ss);
        const float sc = 1.0f / sqrtf(static_cast<float>(tot / static_cast<double>(hd)) + A.eps);   // :1087-1093
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e)
            if (live[e]) x[ic[e]] = v[e] * (sc * wv[e]);
        __builtin_amdgcn_wave_barrier();   // a wave's LDS accesses complete in order
        float y[4];
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const float a = x[ei[e]], bb = x[ei[e] + half];
            y[e] = ic[e] < half ? a * rc[e] - bb * rs[e] : bb * rc[e] + a * rs[e];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e)
            if (live[e]) x[ic[e]] = y[e];
    }
    __syncthreads();
    if (h == 0u && tid < hd) {   // KV append of this row's position
        const uint64_t o = cache0 + static_cast<uint64_t>(p % A.slots) * hd + tid;
        A.kc[o] = sk[tid];
        A.vc[o] = sv[tid];
    }
#pragma unroll
    for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t t = t_first + wave + 4u * u;
        if (t > p) break;
        float d = 0.0f;
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e)
            if (lane + 64u * e < hd) d += sq[lane + 64u * e] * (t == p ? sk[lane + 64u * e] : kr[u][e]);
        d = wave_sum(d);
        if (lane == 0u) ssc[t - t_first] = d * A.attn_scale;
    }
    __syncthreads();
    if (wave == 0u) {   // m = max, e = exp(s - m), l = sum e (double)
        float mx = lane < n_hist ? ssc[lane] : -INFINITY;
        mx = wave_max(mx);
        double l = 0.0;
        if (lane < n_hist) {
            const float e = expf(ssc[lane] - mx);
            ssc[lane] = e;
            l = e;
        }
        l = wave_sum_f64(l);
        if (lane == 0u) s_l = l;
    }
    __syncthreads();
    if (tid < hd) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < kBdShort; ++u)
            if (u < n_hist) acc += ssc[u] * (t_first + u == p ? sv[tid] : vv[u]);
        const double den = static_cast<double>(static_cast<float>(s_l));
        if (tid == 0u && (!(den > 0.0) || !__builtin_isfinite(den))) atomicMin(&A.st->nonfinite, g3_code_softmax(A.block));
        const float v = static_cast<float>(static_cast<double>(acc) / den);
        const uint64_t o = static_cast<uint64_t>(b) * H * hd + h * hd + tid;
        const _Float16 hi = static_cast<_Float16>(v);
        A.ohi[o] = hi;
        A.olo[o] = static_cast<_Float16>(v - static_cast<float>(hi));
    }
}

// One workgroup per (head h, row b): att = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c over the
// row's non-empty chunks (sums in double, chunk order), as f16 hi/lo into the O projection's
// input; a denominator that is not > 0 and finite flags the block (src/gemma3.cpp:1666-1670).
__global__ void __launch_bounds__(kBdThreads) k_bd_merge(BdAttn A) {
#pragma clang fp contract(off)
    __shared__ double s_w[kBdMaxChunks];
    __shared__ double s_den;
    const uint32_t h = blockIdx.x, b = blockIdx.y, H = A.H, hd = A.hd;
    uint32_t t_first, C, n_act;
    bd_chunks(A, A.pos[b], t_first, C, n_act);
    const uint32_t stride = 2u * H + H * hd;
    const float* part = A.part + static_cast<uint64_t>(b) * A.G * stride;
    if (threadIdx.x < 64u) {   // wave 0: the chunk weights and the denominator
        float M = -INFINITY;
        for (uint32_t c = threadIdx.x; c < n_act; c += 64u) M = fmaxf(M, part[c * stride + h]);
        M = wave_max(M);
        for (uint32_t c = threadIdx.x; c < n_act; c += 64u) s_w[c] = static_cast<double>(expf(part[c * stride + h] - M));
        __builtin_amdgcn_wave_barrier();
        if (threadIdx.x == 0u) {
            double den = 0.0;
            for (uint32_t c = 0; c < n_act; ++c) den += s_w[c] * static_cast<double>(part[c * stride + H + h]);
            s_den = den;
            if (!(den > 0.0) || !__builtin_isfinite(den)) atomicMin(&A.st->nonfinite, g3_code_softmax(A.block));
        }
    }
    __syncthreads();
    const double den = s_den;
    for (uint32_t i = threadIdx.x; i < hd; i += kBdThreads) {
        double num = 0.0;
        for (uint32_t c = 0; c < n_act; ++c) num += s_w[c] * static_cast<double>(part[c * stride + 2u * H + h * hd + i]);
        const float v = static_cast<float>(num / den);
        const uint64_t o = static_cast<uint64_t>(b) * H * hd + h * hd + i;
        const _Float16 hi = static_cast<_Float16>(v);
        A.ohi[o] = hi;
        A.olo[o] = static_cast<_Float16>(v - static_cast<float>(hi));
    }
}

// Greedy argmax of each row's logits [n][V] (the tie rule of am_better, shaders/argmax.comp:30-43):
// k_bd_argmax, grid (kBdArgParts, n), leaves one partial per (part, row); k_bd_argmax_final,
// one workgroup per row, reduces them into results[b].
__global__ void __launch_bounds__(kBdThreads) k_bd_argmax(const float* logits, uint32_t V, LmPartial* parts) {
    __shared__ float bvs[kBdThreads / 64u];
    __shared__ uint32_t bis[kBdThreads / 64u];
    const uint32_t b = blockIdx.y;
    const uint32_t per = (V + gridDim.x - 1u) / gridDim.x;
    const uint32_t v0 = blockIdx.x * per, v1 = min(V, v0 + per);
    const float* row = logits + static_cast<uint64_t>(b) * V;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t v = v0 + threadIdx.x; v < v1; v += kBdThreads) {
        const float x = row[v];
        if (am_better(x, v, bv, bi)) {
            bv = x;
            bi = v;
        }
    }
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63u) == 0u) {
        bvs[threadIdx.x >> 6] = bv;
        bis[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t k = 1; k < kBdThreads / 64u; ++k)
            if (am_better(bvs[k], bis[k], bvs[0], bis[0])) {
                bvs[0] = bvs[k];
                bis[0] = bis[k];
            }
        parts[static_cast<uint64_t>(b) * gridDim.x + blockIdx.x] = {bvs[0], bis[0]};
    }
}

__global__ void __launch_bounds__(kBdThreads) k_bd_argmax_final(const LmPartial* parts, uint32_t nparts,
                                                                vrt_argmax_result* results) {
    __shared__ float bvs[kBdThreads / 64u];
    __shared__ uint32_t bis[kBdThreads / 64u];
    const uint32_t b = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t k = threadIdx.x; k < nparts; k += kBdThreads) {
        const LmPartial pp = parts[static_cast<uint64_t>(b) * nparts + k];
        if (am_better(pp.value, pp.index, bv, bi)) {
            bv = pp.value;
            bi = pp.index;
        }
    }
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63u) == 0u) {
        bvs[threadIdx.x >> 6] = bv;
        bis[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0u) {
        for (uint32_t k = 1; k < kBdThreads / 64u; ++k)
            if (am_better(bvs[k], bis[k], bvs[0], bis[0])) {
                bvs[0] = bvs[k];
                bis[0] = bis[k];
            }
        results[b] = {bis[0], bvs[0]};
    }
}

}  // namespace vrt

using namespace vrt;

// Per-block state of a batch: the sequences' caches and the attention split.
struct BdLayer {
    float* kc = nullptr;
    float* vc = nullptr;
    uint32_t slots = 0, G = 1, cmax = 1;
};

struct vrt_g3_batch {
    vrt_g3* g = nullptr;
    uint32_t max_seqs = 0, max_ctx = 0;
    uint32_t last_n = 0;            // rows of the last completed step
    std::vector<uint32_t> pos;      // next position of each sequence (host)
    std::vector<BdLayer> layers;
    std::vector<void*> allocs;
    uint32_t* rows = nullptr;       // device: [3][kBdMaxRows] tokens, positions, sequences
    uint32_t* host_rows = nullptr;  // pinned staging of the same
    vrt_argmax_result* res = nullptr;        // device [kBdMaxRows]
    vrt_argmax_result* host_res = nullptr;   // pinned
    G3State* st = nullptr;          // device: failure word (nonfinite)
    G3State* host_st = nullptr;     // pinned
    float* h = nullptr;             // [rows][d] residual stream
    float* x = nullptr;             // [kBdMaxSplits][rows][d] O / down projection partials
    float* qkv = nullptr;           // [kBdMaxSplits][rows][(H + 2) hd] q|k|v partials
    _Float16* ahi = nullptr;        // [rows][max(d, H hd)] GEMM input, f16 high part
    _Float16* alo = nullptr;
    _Float16* ghi = nullptr;        // [rows][F] gelu(gate) * up, f16 high part
    _Float16* glo = nullptr;
    float* part = nullptr;          // [rows][max G][2 H + H hd] attention chunk partials
    float* logits = nullptr;        // [rows][V]
    LmPartial* amx = nullptr;       // [rows][kBdArgParts]
};

static int bd_alloc(vrt_g3_batch* B, size_t bytes, void** out) {
    void* p = nullptr;
    VRT_HIP_CHECK(hipMalloc(&p, bytes + 256));
    B->allocs.push_back(p);
    // zero-filled on the executor's context stream (non-blocking), which every later use is ordered on
    VRT_HIP_CHECK(hipMemsetAsync(p, 0, bytes + 256, B->g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(B->g->ctx->stream));
    *out = p;
    return VRT_OK;
}

extern "C" int vrt_g3_batch_destroy(vrt_g3_batch* B) {
    if (!B) return VRT_OK;
    (void)hipSetDevice(B->g->ctx->device);
    (void)hipStreamSynchronize(B->g->ctx->stream);
    for (void* p : B->allocs) (void)hipFree(p);
    B->g->live_batches--;
    if (B->host_rows) (void)hipHostFree(B->host_rows);
    if (B->host_res) (void)hipHostFree(B->host_res);
    if (B->host_st) (void)hipHostFree(B->host_st);
    delete B;
    return VRT_OK;
}

extern "C" int vrt_g3_batch_create(vrt_g3* g, uint32_t max_seqs, uint32_t max_ctx, vrt_g3_batch** out) {
    VRT_REQUIRE(g && out, "vrt_g3_batch_create: null argument");
    *out = nullptr;
    VRT_REQUIRE(max_seqs >= 1u && max_seqs <= kBdMaxRows, "vrt_g3_batch_create: max_seqs must be 1..%u", kBdMaxRows);
    VRT_REQUIRE(max_ctx >= 1u && max_ctx <= g->cfg.context_length,
                "vrt_g3_batch_create: max_ctx must be 1..context_length (%u)", g->cfg.context_length);
    const vrt_g3_config& c = g->cfg;
    const uint32_t d = c.embedding_length, H = c.head_count, hd = c.head_dim, F = c.feed_forward_length;
    const uint32_t qw = H * hd, nqkv = qw + 2u * hd;
    VRT_REQUIRE(H <= 8u && hd <= 256u && d <= 2048u, "batched decode: shape outside its kernels");
    VRT_HIP_CHECK(hipSetDevice(g->ctx->device));
    auto* B = new (std::nothrow) vrt_g3_batch();
    VRT_REQUIRE(B != nullptr, "out of memory");
    B->g = g;
    g->live_batches++;   // vrt_g3_batch_destroy (also on the failure paths below) gives it back
    B->max_seqs = max_seqs;
    B->max_ctx = max_ctx;
    B->pos.assign(max_seqs, 0u);
    auto fail = [&](int rc) {
        vrt_g3_batch_destroy(B);
        return rc;
    };
    void* p;
    const size_t R = kBdMaxRows;
    uint32_t gmax = 1;
    B->layers.resize(g->layers.size());
    for (size_t l = 0; l < g->layers.size(); ++l) {
        BdLayer& L = B->layers[l];
        L.slots = g->layers[l].global ? max_ctx : std::min(g->layers[l].slots, max_ctx);
        const size_t kv = static_cast<size_t>(max_seqs) * L.slots * hd * 4u;
        if (int rc = bd_alloc(B, kv, &p)) return fail(rc);
        L.kc = static_cast<float*>(p);
        if (int rc = bd_alloc(B, kv, &p)) return fail(rc);
        L.vc = static_cast<float*>(p);
        // ~8 positions per chunk, at most kBdMaxChunks chunks: short histories still spread over
        // several workgroups per row (8 rather than 64 positions per chunk: 1.47 -> 1.39 ms per
        // step of 64 sequences at positions 8..23)
        L.G = std::max(1u, std::min(kBdMaxChunks, (L.slots + 7u) / 8u));
        L.cmax = (L.slots + L.G - 1u) / L.G;
        gmax = std::max(gmax, L.G);
    }
    if (int rc = bd_alloc(B, 3u * R * 4u, &p)) return fail(rc);
    B->rows = static_cast<uint32_t*>(p);
    if (int rc = bd_alloc(B, R * sizeof(vrt_argmax_result), &p)) return fail(rc);
    B->res = static_cast<vrt_argmax_result*>(p);
    if (int rc = bd_alloc(B, sizeof(G3State), &p)) return fail(rc);
    B->st = static_cast<G3State*>(p);
    if (int rc = bd_alloc(B, R * d * 4u, &p)) return fail(rc);
    B->h = static_cast<float*>(p);
    if (int rc = bd_alloc(B, kBdMaxSplits * R * d * 4u, &p)) return fail(rc);
    B->x = static_cast<float*>(p);
    if (int rc = bd_alloc(B, kBdMaxSplits * R * nqkv * 4u, &p)) return fail(rc);
    B->qkv = static_cast<float*>(p);
    const size_t aw = std::max(d, qw);
    if (int rc = bd_alloc(B, R * aw * 2u, &p)) return fail(rc);
    B->ahi = static_cast<_Float16*>(p);
    if (int rc = bd_alloc(B, R * aw * 2u, &p)) return fail(rc);
    B->alo = static_cast<_Float16*>(p);
    if (int rc = bd_alloc(B, R * F * 2u, &p)) return fail(rc);
    B->ghi = static_cast<_Float16*>(p);
    if (int rc = bd_alloc(B, R * F * 2u, &p)) return fail(rc);
    B->glo = static_cast<_Float16*>(p);
    if (int rc = bd_alloc(B, R * gmax * (2u * H + qw) * 4u, &p)) return fail(rc);
    B->part = static_cast<float*>(p);
    if (int rc = bd_alloc(B, R * c.vocab_size * 4u, &p)) return fail(rc);
    B->logits = static_cast<float*>(p);
    if (int rc = bd_alloc(B, R * kBdArgParts * sizeof(LmPartial), &p)) return fail(rc);
    B->amx = static_cast<LmPartial*>(p);
    {
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&B->host_rows), 3u * R * 4u, hipHostMallocDefault);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void**>(&B->host_res), R * sizeof(vrt_argmax_result), hipHostMallocDefault);
        if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&B->host_st), sizeof(G3State), hipHostMallocDefault);
        if (e != hipSuccess) return fail(set_error(VRT_ERR_HIP, "hipHostMalloc failed: %s", hipGetErrorString(e)));
    }
    size_t lds = 0;
    for (const BdLayer& L : B->layers) lds = std::max(lds, static_cast<size_t>((H + 2u) * hd + H * L.cmax) * 4u);
    if (lds > 64u * 1024u) return fail(set_error(VRT_ERR_INVALID, "batched decode: attention chunk does not fit in LDS"));
    VRT_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_bd_attn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
    *out = B;
    return VRT_OK;
}

extern "C" int vrt_g3_batch_reset(vrt_g3_batch* B, uint32_t seq) {
    VRT_REQUIRE(B, "vrt_g3_batch_reset: null batch");
    if (seq == 0xffffffffu) {
        std::fill(B->pos.begin(), B->pos.end(), 0u);
        return VRT_OK;
    }
    VRT_REQUIRE(seq < B->max_seqs, "vrt_g3_batch_reset: sequence %u out of range", seq);
    B->pos[seq] = 0u;
    return VRT_OK;
}

extern "C" int vrt_g3_batch_position(vrt_g3_batch* B, uint32_t seq, uint32_t* pos) {
    VRT_REQUIRE(B && pos, "vrt_g3_batch_position: null argument");
    VRT_REQUIRE(seq < B->max_seqs, "vrt_g3_batch_position: sequence %u out of range", seq);
    *pos = B->pos[seq];
    return VRT_OK;
}

// Enqueues one step over the n rows already uploaded to B->rows.
static int bd_enqueue(vrt_g3_batch* B, uint32_t n, hipStream_t s) {
    vrt_g3* g = B->g;
    const vrt_g3_config& c = g->cfg;
    const uint32_t d = c.embedding_length, H = c.head_count, hd = c.head_dim, qw = H * hd, nqkv = qw + 2u * hd;
    const uint32_t L = c.block_count;
    const float eps = g->P.eps;
    const uint32_t* tok = B->rows;
    const uint32_t* pos = B->rows + kBdMaxRows;
    const uint32_t* seq = B->rows + 2u * kBdMaxRows;
    if (int rc = pf_embed_rows(g, tok, n, B->h, s)) return rc;
    const uint64_t xs = static_cast<uint64_t>(n) * d;   // one O / down partial
    uint32_t s_down = 1;
    for (uint32_t l = 0; l < L; ++l) {
        const LayerParams& Ly = g->layers[l];
        const BdLayer& BL = B->layers[l];
        // previous block's FFN output into the residual, then the attention norm
        if (int rc = pf_norm(B->h, l ? B->x : nullptr, s_down, xs, l ? g->layers[l - 1].post_ffw : nullptr, Ly.attn_norm,
                             d, eps, B->ahi, B->alo, B->st, l ? l - 1u : 0u, n, s, true))
            return rc;
        uint32_t s_qkv = 1;
        if (int rc = pf_project(g, l, kProjQkv, B->ahi, B->alo, n, B->qkv,
                                std::min(kBdMaxSplits, pf_splits(n, nqkv)), &s_qkv, s))
            return rc;
        BdAttn A{};
        A.qkv = B->qkv;
        A.sstride = static_cast<uint64_t>(n) * nqkv;
        A.nsplit = s_qkv;
        A.pos = pos;
        A.seq = seq;
        A.kc = BL.kc;
        A.vc = BL.vc;
        A.slots = BL.slots;
        A.H = H;
        A.hd = hd;
        A.G = BL.G;
        A.cmax = BL.cmax;
        A.q_norm = Ly.q_norm;
        A.k_norm = Ly.k_norm;
        A.cos_t = Ly.global ? g->P.cos_g : g->P.cos_l;
        A.sin_t = Ly.global ? g->P.sin_g : g->P.sin_l;
        A.eps = eps;
        A.attn_scale = g->P.attn_scale;
        A.part = B->part;
        A.ohi = B->ahi;
        A.olo = B->alo;
        A.st = B->st;
        A.block = l;
        {
            void* args[] = {&A};
            uint32_t nh_max = 0;   // longest history of the step's rows in this block
            for (uint32_t i = 0; i < n; ++i) nh_max = std::max(nh_max, std::min(B->host_rows[kBdMaxRows + i] + 1u, BL.slots));
            if (nh_max <= kBdShort && hd <= 256u) {
                VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_bd_attn_short), dim3(H, n), dim3(kBdThreads),
                                              args, 0, s));
            } else {
                const size_t lds = static_cast<size_t>((H + 2u) * hd + H * BL.cmax) * 4u;
                VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_bd_attn), dim3(BL.G, n), dim3(kBdThreads), args,
                                              lds, s));
                VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_bd_merge), dim3(H, n), dim3(kBdThreads), args,
                                              0, s));
            }
        }
        uint32_t s_o = 1;
        if (int rc = pf_project(g, l, kProjO, B->ahi, B->alo, n, B->x, std::min(kBdMaxSplits, pf_splits(n, d)), &s_o, s))
            return rc;
        if (int rc = pf_norm(B->h, B->x, s_o, xs, Ly.post_attn, Ly.ffn_norm, d, eps, B->ahi, B->alo, B->st, l, n, s, true))
            return rc;
        if (int rc = pf_ffn_glu(g, l, B->ahi, B->alo, n, B->ghi, B->glo, s)) return rc;
        if (int rc = pf_project(g, l, kProjDown, B->ghi, B->glo, n, B->x, std::min(kBdMaxSplits, pf_splits(n, d)),
                                &s_down, s))
            return rc;
    }
    // final residual (:1849-1855) and output norm (rms_norm_inplace, :1866-1868) as the LM input
    if (int rc = pf_norm(B->h, B->x, s_down, xs, g->layers[L - 1u].post_ffw, g->out_norm_dev, d, eps, B->ahi, B->alo, B->st,
                         L - 1u, n, s, false))
        return rc;
    if (int rc = pf_lm_logits(g, B->ahi, B->alo, n, B->logits, s)) return rc;
    {
        const float* lg = B->logits;
        uint32_t V = c.vocab_size;
        LmPartial* parts = B->amx;
        void* a1[] = {&lg, &V, &parts};
        VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_bd_argmax), dim3(kBdArgParts, n), dim3(kBdThreads),
                                      a1, 0, s));
        const LmPartial* cp = B->amx;
        uint32_t np = kBdArgParts;
        vrt_argmax_result* res = B->res;
        void* a2[] = {&cp, &np, &res};
        VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_bd_argmax_final), dim3(n), dim3(kBdThreads), a2,
                                      0, s));
    }
    return VRT_OK;
}

// Every sequence of the failed step restarts at position 0 (the reference resets its cache on
// any decode error, src/gemma3.cpp:1878-1881).
static int bd_fail(vrt_g3_batch* B, const uint32_t* seqs, uint32_t n, int rc, const char* msg) {
    B->last_n = 0;
    for (uint32_t i = 0; i < n; ++i)
        if (seqs[i] < B->max_seqs) B->pos[seqs[i]] = 0u;
    return set_error(rc, "%s", msg);
}

extern "C" int vrt_g3_batch_step(vrt_g3_batch* B, const uint32_t* seqs, const uint32_t* tokens, uint32_t n,
                                 vrt_argmax_result* results) {
    VRT_REQUIRE(B && seqs && tokens && results, "vrt_g3_batch_step: null argument");
    VRT_REQUIRE(n >= 1u && n <= B->max_seqs, "vrt_g3_batch_step: n must be 1..%u", B->max_seqs);
    vrt_g3* g = B->g;
    for (uint32_t i = 0; i < n; ++i) {
        VRT_REQUIRE(seqs[i] < B->max_seqs, "vrt_g3_batch_step: sequence %u out of range", seqs[i]);
        for (uint32_t j = 0; j < i; ++j)
            VRT_REQUIRE(seqs[j] != seqs[i], "vrt_g3_batch_step: sequence %u appears twice", seqs[i]);
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (B->pos[seqs[i]] >= B->max_ctx) return set_error(VRT_ERR_STATE, "Gemma 3 context length exceeded");
        if (tokens[i] >= g->cfg.vocab_size)
            return bd_fail(B, seqs, n, VRT_ERR_INVALID, "Token id is outside Gemma 3 vocabulary");
    }
    hipStream_t s = g->ctx->stream;
    for (uint32_t i = 0; i < n; ++i) {
        B->host_rows[i] = tokens[i];
        B->host_rows[kBdMaxRows + i] = B->pos[seqs[i]];
        B->host_rows[2u * kBdMaxRows + i] = seqs[i];
    }
    B->host_st->nonfinite = 0xffffffffu;
    VRT_HIP_CHECK(hipMemcpyAsync(B->rows, B->host_rows, 3u * kBdMaxRows * 4u, hipMemcpyHostToDevice, s));
    VRT_HIP_CHECK(hipMemcpyAsync(&B->st->nonfinite, &B->host_st->nonfinite, 4u, hipMemcpyHostToDevice, s));
    if (int rc = bd_enqueue(B, n, s)) return bd_fail(B, seqs, n, rc, vrt_last_error());
    VRT_HIP_CHECK(hipMemcpyAsync(B->host_res, B->res, n * sizeof(vrt_argmax_result), hipMemcpyDeviceToHost, s));
    VRT_HIP_CHECK(hipMemcpyAsync(&B->host_st->nonfinite, &B->st->nonfinite, 4u, hipMemcpyDeviceToHost, s));
    VRT_HIP_CHECK(hipStreamSynchronize(s));
    const G3Failure f = g3_map_failure(B->host_st->nonfinite, 0u);
    if (f.code != VRT_OK) return bd_fail(B, seqs, n, f.code, f.msg);
    for (uint32_t i = 0; i < n; ++i) {
        const vrt_argmax_result r = B->host_res[i];
        if (r.index >= g->cfg.vocab_size || !std::isfinite(r.value))   // :1171-1176
            return bd_fail(B, seqs, n, VRT_ERR_NUMERIC, "GPU argmax produced invalid result");
        results[i] = r;
    }
    for (uint32_t i = 0; i < n; ++i) ++B->pos[seqs[i]];
    B->last_n = n;
    return VRT_OK;
}

extern "C" int vrt_g3_batch_logits(vrt_g3_batch* B, uint32_t row, float* host, uint32_t n) {
    VRT_REQUIRE(B && host, "vrt_g3_batch_logits: null argument");
    VRT_REQUIRE(row < B->last_n, "vrt_g3_batch_logits: row %u of a step of %u rows", row, B->last_n);
    VRT_REQUIRE(n <= B->g->cfg.vocab_size, "vrt_g3_batch_logits: n exceeds vocab_size");
    hipStream_t s = B->g->ctx->stream;
    VRT_HIP_CHECK(hipMemcpyAsync(host, B->logits + static_cast<uint64_t>(row) * B->g->cfg.vocab_size,
                                 static_cast<size_t>(n) * 4u, hipMemcpyDeviceToHost, s));
    VRT_HIP_CHECK(hipStreamSynchronize(s));
    return VRT_OK;
}
