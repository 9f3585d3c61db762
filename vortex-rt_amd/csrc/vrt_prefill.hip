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

#include "vrt_g3_errors.hpp"
#include "vrt_g3_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kPfThreads = 256;
constexpr uint32_t kPfMaxSplits = 4;   // K splits of the O and down projections (pf_splits)
constexpr uint64_t kPfExpandBudget = 16ull << 30;   // device bytes for the prefill's expanded weights
constexpr uint32_t kPfTile = 64;     // attention score rows are padded to a multiple of this

// ---- row kernels ---------------------------------------------------------------------------

__device__ __forceinline__ void pf_split(float x, _Float16* hi, _Float16* lo) {
    const _Float16 h = static_cast<_Float16>(x);
    *hi = h;
    *lo = static_cast<_Float16>(x - static_cast<float>(h));
}

// Workgroup double sum (fixed order: 4 waves, DPP inside each) behind one barrier. red[0..4)
// belongs to this call: a second sum in the same kernel takes other slots, so no thread can
// still be reading them when they are written.
__device__ __forceinline__ double pf_sum(double v, double* red) {
    v = wave_red_sum_d(v);
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

// One row t per workgroup (n <= 8 * kPfThreads). With f (the previous sublayer's output, the
// sum of nsplit partial rows f + s * sstride added in order s = 0, 1, ...):
// h = f * (scale(f) * w_post) + h (rms_norm_inplace then add_inplace, src/gemma3.cpp:1036-1042,
// :1703-1711, :1849-1855). Then, with w_next:
// the GEMM input (h * scale(h)) * w_next as f16 hi/lo (:991-996). nonfinite: lowest block
// whose residual went non-finite (:1857-1863), reported through st->nonfinite.
__global__ void __launch_bounds__(kPfThreads) k_pf_norm(float* h, const float* f, uint32_t nsplit, uint64_t sstride,
                                                        const float* w_post, const float* w_next, uint32_t n, float eps,
                                                        _Float16* xhi, _Float16* xlo, G3State* st, uint32_t block) {
#pragma clang fp contract(off)
    __shared__ double red[2][4];   // one set per sum
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
        // every partial is loaded before the first add (nsplit <= kPfMaxSplits), then the
        // partials are added in split order
        float fp[8][kPfMaxSplits];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = threadIdx.x + k * kPfThreads;
#pragma unroll
            for (uint32_t q = 0; q < kPfMaxSplits; ++q) fp[k][q] = i < n && q < nsplit ? fr[q * sstride + i] : 0.0f;
        }
        float fv[8];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            fv[k] = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < kPfMaxSplits; ++q)
                if (q < nsplit) fv[k] += fp[k][q];
            ss += static_cast<double>(fv[k]) * static_cast<double>(fv[k]);
        }
        const float sc = pf_rms_scale(pf_sum(ss, red[0]), n, eps);
        int bad = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t i = threadIdx.x + k * kPfThreads;
            if (i < n) {
                hv[k] = fv[k] * (sc * w_post[i]) + hv[k];
                hr[i] = hv[k];
                bad |= !__builtin_isfinite(hv[k]);
            }
        }
        if (bad) atomicMin(&st->nonfinite, g3_code_nonfinite(block));
    }
    if (!w_next) return;
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += static_cast<double>(hv[k]) * static_cast<double>(hv[k]);
    const float sc = pf_rms_scale(pf_sum(ss, red[1]), n, eps);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t i = threadIdx.x + k * kPfThreads;
        if (i < n) pf_split((hv[k] * sc) * w_next[i], xhi + static_cast<uint64_t>(t) * n + i, xlo + static_cast<uint64_t>(t) * n + i);
    }
}

// out[i] = sum over s < nsplit, in order, of the split partials x[s * n + i] of one row.
__global__ void __launch_bounds__(kPfThreads) k_pf_sum(const float* x, uint32_t nsplit, uint32_t n, float* out) {
#pragma clang fp contract(off)
    for (uint32_t i = threadIdx.x; i < n; i += kPfThreads) {
        float v = 0.0f;
        for (uint32_t q = 0; q < nsplit; ++q) v += x[static_cast<uint64_t>(q) * n + i];
        out[i] = v;
    }
}

// gelu_tanh(gate) * up (shaders/gelu_mul.comp:23-31), every operation rounded to fp32.
__device__ __forceinline__ float pf_gelu_mul(float x, float up) {
#pragma clang fp contract(off)
    const float cubic = x * x * x;
    const float g = 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * cubic)));
    return g * up;
}


// ---- GEMM on MFMA: Q8_0 weights or fp32 rows as B ---------------------------------------------

struct PfGemm {
    const _Float16* ahi;     // A [M][K] (row stride lda), f16 high and low parts
    const _Float16* alo;
    uint32_t lda;
    uint64_t a_bs;           // A offset (elements) per batch index blockIdx.z
    const uint8_t* w[3];     // B as Q8_0 matrices concatenated along N (rows[i] rows each), or
    uint32_t rows[3];
    uint32_t nseg;
    const uint8_t* w_end;    //   one past the arena
    const float* b;          // B as fp32 rows: B[n][k] = b[n * ldb + k] (+ b_bs per batch)
    uint32_t ldb;
    uint64_t b_bs;
    float* c;                // C [M][N] fp32 (row stride ldc), or
    _Float16* chi;           //   C as f16 high and low parts
    _Float16* clo;
    uint32_t ldc;
    uint64_t c_bs;
    uint32_t M, N, K;
    uint32_t window;         // causal modes: keys older than window positions are skipped (0: none)
    uint32_t glu;            // Q8_0 GEMM: w[0] = gate, w[1] = up (N = 2F), output gelu_tanh(gate) * up
    const _Float16* wh;      // expanded weights: the quants of N rows as f16 [N][K] (nullptr: Q8_0 w)
    const float* ws;         //   and their block scales [N][K / 32]
};

// One 32 x 32 tile of C per workgroup (v_mfma_f32_32x32x16_f16); the four waves split the
// K blocks (wave w takes blocks w, w + 4, ...) and their partial tiles are summed through LDS
// in wave order (deterministic). Lane l of a wave: A operand row m = l % 32, k = 8 * (l / 32)
// + 0..7 of each 16-wide k step; B operand column n = l % 32, same k; accumulator element r at
// row 8 * (r / 4) + 4 * (l / 32) + r % 4, column l % 32. Q8 B: per 32-wide block, two f16 MFMA
// chains (A hi, A lo) against the exact quants, scaled by the column's block scale (the lane's
// own) in fp32. fp32 B: split into f16 hi + lo in registers, three products (hi hi, lo hi,
// hi lo) per k step. Each wave's next block loads while its current block's MFMAs run.
constexpr int kGemmB32 = 1;       // B is fp32 rows (otherwise Q8_0)
constexpr int kGemmCausalS = 2;   // S = Q K^T: skip key tiles no query of the row tile sees
constexpr int kGemmCausalO = 4;   // O = P V: the K (key) range ends after the row tile's last query
constexpr int kGemmOut16 = 8;     // C as f16 hi/lo
constexpr uint32_t kPfGT = 32;    // GEMM tile (rows and columns)
constexpr uint32_t kPfDepth = 3;  // K blocks in flight per wave
template <int MODE>
__global__ void __launch_bounds__(kPfThreads) k_pf_gemm(PfGemm G) {
    constexpr bool BF32 = (MODE & kGemmB32) != 0, OUT16 = (MODE & kGemmOut16) != 0;
    __shared__ float red[3][16][64];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t kh = lane >> 5, l32 = lane & 31u;
    const uint32_t m0 = blockIdx.y * kPfGT, n0 = blockIdx.x * kPfGT;
    uint32_t k_lo = 0, k_hi = G.K;
    if constexpr ((MODE & (kGemmCausalS | kGemmCausalO)) != 0) {
        const uint32_t q_last = min(G.M, m0 + kPfGT) - 1u;
        const uint32_t k_old = (G.window != 0u && m0 + 1u > G.window) ? m0 + 1u - G.window : 0u;
        if constexpr ((MODE & kGemmCausalS) != 0) {
            if (n0 > q_last || n0 + kPfGT <= k_old) return;   // uniform over the workgroup
        } else {
            k_lo = (k_old / 32u) * 32u;
            k_hi = min(G.K, ((q_last + 32u) / 32u) * 32u);
        }
    }
    const uint32_t m = m0 + l32, n = n0 + l32;
    const bool mlive = m < G.M, nlive = n < G.N;
    const uint64_t zb = blockIdx.z;
    typedef const __attribute__((address_space(1))) half8* gh8;
    typedef const __attribute__((address_space(1))) f4* gf4;
    const uintptr_t ahi_base = reinterpret_cast<uintptr_t>(G.ahi + zb * G.a_bs);
    const uintptr_t alo_base = reinterpret_cast<uintptr_t>(G.alo + zb * G.a_bs);
    const uint64_t arow = static_cast<uint64_t>(mlive ? m : 0u) * G.lda + 8u * kh;
    auto load_a = [&](uint32_t k0, half8 (&hi)[2], half8 (&lo)[2]) {
#pragma unroll
        for (uint32_t ks = 0; ks < 2; ++ks) {
            const uint64_t o = (arow + k0 + 16u * ks) * 2u;
            hi[ks] = *reinterpret_cast<gh8>(ahi_base + o);
            lo[ks] = *reinterpret_cast<gh8>(alo_base + o);
        }
    };
    float16v acc = {};
    const uint32_t b_lo = k_lo / 32u, b_hi = k_hi / 32u;   // this wave: blocks b_lo + wave + 4i
    if constexpr (!BF32) {
        const uint64_t row_bytes = static_cast<uint64_t>(G.K >> 5) * 34u;
        const uint8_t* wrow = G.w[0];   // the lane's weight row (segments unrolled: no indexed struct)
        {
            uint32_t r = nlive ? n : 0u;
            if (G.nseg > 1u && r >= G.rows[0]) {
                r -= G.rows[0];
                wrow = G.w[1];
                if (G.nseg > 2u && r >= G.rows[1]) {
                    r -= G.rows[1];
                    wrow = G.w[2];
                }
            }
            wrow += static_cast<uint64_t>(r) * row_bytes;
        }
        // quants 16 ks + 8 kh .. + 7 of a block as f16 (constant register indices, selected by kh)
        auto to_half8 = [&](const Q8Raw& r, uint32_t ks) {
            half8 v;
            const uint32_t j = 4u * ks;
            const uint32_t a0 = __builtin_amdgcn_alignbyte(r.d[j + 1], r.d[j], r.sh);
            const uint32_t a1 = __builtin_amdgcn_alignbyte(r.d[j + 2], r.d[j + 1], r.sh);
            const uint32_t a2 = __builtin_amdgcn_alignbyte(r.d[j + 3], r.d[j + 2], r.sh);
            const uint32_t a3 = __builtin_amdgcn_alignbyte(r.d[j + 4], r.d[j + 3], r.sh);
            const uint32_t d0 = kh ? a2 : a0, d1 = kh ? a3 : a1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(d0 >> (8 * i))));
                v[4 + i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(d1 >> (8 * i))));
            }
            return v;
        };
        // a ring of kPfDepth blocks in flight per wave (static register sets)
        half8 ah[kPfDepth][2], al[kPfDepth][2];
        Q8Raw rw[kPfDepth];
        const uint32_t b0 = b_lo + wave;
#pragma unroll
        for (uint32_t i = 0; i < kPfDepth; ++i) {
            const uint32_t bb = b0 + 4u * i;
            if (bb < b_hi) {
                load_a(32u * bb, ah[i], al[i]);
                q8_load(wrow + 34u * bb, G.w_end, rw[i]);
            }
        }
        for (uint32_t base = b0; base < b_hi; base += 4u * kPfDepth) {
#pragma unroll
            for (uint32_t i = 0; i < kPfDepth; ++i) {
                const uint32_t bb = base + 4u * i;
                if (bb < b_hi) {
                    const half8 w0 = to_half8(rw[i], 0u), w1 = to_half8(rw[i], 1u);
                    float16v p1 = {}, p2 = {};
                    p1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], w0, p1, 0, 0, 0);
                    p2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], w0, p2, 0, 0, 0);
                    p1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], w1, p1, 0, 0, 0);
                    p2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], w1, p2, 0, 0, 0);
                    const float sc = half_bits_to_float(rw[i].sbits);
                    const uint32_t nb = bb + 4u * kPfDepth;
                    if (nb < b_hi) {
                        load_a(32u * nb, ah[i], al[i]);
                        q8_load(wrow + 34u * nb, G.w_end, rw[i]);
                    }
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[r] += sc * (p1[r] + p2[r]);
                }
            }
        }
    } else {
        const uintptr_t b_base = reinterpret_cast<uintptr_t>(G.b + zb * G.b_bs) +
                                 (static_cast<uint64_t>(nlive ? n : 0u) * G.ldb + 8u * kh) * 4u;
        auto load_b = [&](uint32_t k0, f4 (&v)[4]) {   // k step 0: v[0], v[1]; k step 1: v[2], v[3]
#pragma unroll
            for (uint32_t ks = 0; ks < 2; ++ks) {
                v[2 * ks] = *reinterpret_cast<gf4>(b_base + (k0 + 16u * ks) * 4u);
                v[2 * ks + 1] = *reinterpret_cast<gf4>(b_base + (k0 + 16u * ks + 4u) * 4u);
            }
        };
        half8 ah[kPfDepth][2], al[kPfDepth][2];
        f4 bv[kPfDepth][4];
        const uint32_t b0 = b_lo + wave;
#pragma unroll
        for (uint32_t i = 0; i < kPfDepth; ++i) {
            const uint32_t bb = b0 + 4u * i;
            if (bb < b_hi) {
                load_a(32u * bb, ah[i], al[i]);
                load_b(32u * bb, bv[i]);
            }
        }
        for (uint32_t base = b0; base < b_hi; base += 4u * kPfDepth) {
#pragma unroll
            for (uint32_t i = 0; i < kPfDepth; ++i) {
                const uint32_t bb = base + 4u * i;
                if (bb < b_hi) {
                    half8 bh[2], bl[2], xh[2], xl[2];
#pragma unroll
                    for (uint32_t ks = 0; ks < 2; ++ks) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float x0 = bv[i][2 * ks][j], x1 = bv[i][2 * ks + 1][j];
                            const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
                            bh[ks][j] = h0;
                            bh[ks][4 + j] = h1;
                            bl[ks][j] = static_cast<_Float16>(x0 - static_cast<float>(h0));
                            bl[ks][4 + j] = static_cast<_Float16>(x1 - static_cast<float>(h1));
                        }
                        xh[ks] = ah[i][ks];
                        xl[ks] = al[i][ks];
                    }
                    const uint32_t nb = bb + 4u * kPfDepth;
                    if (nb < b_hi) {
                        load_a(32u * nb, ah[i], al[i]);
                        load_b(32u * nb, bv[i]);
                    }
#pragma unroll
                    for (uint32_t ks = 0; ks < 2; ++ks) {
                        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[ks], bh[ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl[ks], bh[ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[ks], bl[ks], acc, 0, 0, 0);
                    }
                }
            }
        }
    }
    // sum the four waves' partial tiles in wave order
    if (wave != 0u) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[wave - 1u][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave != 0u || !nlive) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = ((acc[r] + red[0][r][lane]) + red[1][r][lane]) + red[2][r][lane];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t row = m0 + 8u * (r / 4) + 4u * kh + (r % 4);
        if (row < G.M) {
            const uint64_t o = zb * G.c_bs + static_cast<uint64_t>(row) * G.ldc + n;
            if constexpr (OUT16) pf_split(acc[r], G.chi + o, G.clo + o);
            else G.c[o] = acc[r];
        }
    }
}

// ---- Q8_0 weight GEMM, LDS-tiled ------------------------------------------------------------
//
// C[M][N] = A[M][K] (f16 hi/lo) x W^T with W the Q8_0 rows (segments concatenated along N).
// Workgroup tile: 64 rows of A x 64 * WN rows of W; wave w computes rows 32 (w / 2) and the
// WN 32-column MFMA tiles from 32 WN (w % 2). K advances 64 (two Q8_0 blocks) per step through
// two LDS stages: A as f16 hi and lo [64][64], W as its exact int8 quants in f16 [64 WN][64]
// plus the fp32 block scales; one barrier per step hands a stage over. Per Q8_0 block and tile the
// two f16 MFMA chains (A hi, A lo) accumulate the exact products in fp32 and the block's partial
// is scaled by the column's scale into the fp32 accumulator, as in k_pf_gemm. blockIdx.z splits
// K: split z covers K blocks [z nkb / S, (z + 1) nkb / S) and writes C + z * c_bs; the consumer
// adds the S partial tiles in split order.
constexpr uint32_t kQgBM = 64;
constexpr uint32_t kQgBK = 64;
constexpr uint32_t kQgPitch = kQgBK * 2u + 16u;   // LDS row pitch in bytes (f16 rows, padded)

constexpr uint32_t kQgAhead = 4;   // K steps whose loads are in flight ahead of the one computed
constexpr uint32_t kQgChunk = 12;  // K steps per straight-line chunk of the main loop

// Epilogue of the Q8_0 GEMMs: with G.glu the wave holding a 64-column group's up columns hands
// them to the wave holding its gate columns through `xch` (LDS of at least NWN / 2 x 16 x 64
// floats per 32-row band, free once the K loop is done), which writes gelu_tanh(gate) * up as
// f16 hi/lo; otherwise the fp32 tile goes to split z's slice of C. Waves with `active` false
// hold no tile but still pass the barriers.
template <int WN, int NWN>
__device__ __forceinline__ void pf_gemm_epilogue(const PfGemm& G, const float16v (&acc)[WN], uint32_t z, uint32_t m0,
                                                 uint32_t n0, uint32_t wm, uint32_t wn, uint32_t kh, uint32_t l32,
                                                 uint32_t lane, float* xch, bool active = true) {
    if (G.glu) {
        // the wave holding a group's up columns hands them to the wave holding its gate columns
        // (gelu_tanh(gate) * up, shaders/gelu_mul.comp:23-31)
        static_assert(WN == 1, "one 32-column MFMA tile per wave");
        __syncthreads();   // every wave is done reading the LDS stages
        const uint32_t pair = wm * (NWN / 2u) + (wn >> 1);
        if (active && (wn & 1u)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) xch[(pair * 16u + r) * 64u + lane] = acc[0][r];
        }
        __syncthreads();
        if (!active || (wn & 1u)) return;
        const uint32_t F = G.N / 2u;
        const uint32_t col = n0 / 2u + 32u * (wn >> 1) + l32;
        if (col >= F) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + 32u * wm + 8u * (r / 4) + 4u * kh + (r % 4);
            if (row < G.M) {
                const uint64_t o = static_cast<uint64_t>(row) * G.ldc + col;
                pf_split(pf_gelu_mul(acc[0][r], xch[(pair * 16u + r) * 64u + lane]), G.chi + o, G.clo + o);
            }
        }
        return;
    }
    if (!active) return;
    float* c = G.c + static_cast<uint64_t>(z) * G.c_bs;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const uint32_t col = n0 + 32u * (WN * wn + j) + l32;
        if (col >= G.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = m0 + 32u * wm + 8u * (r / 4) + 4u * kh + (r % 4);
            if (row < G.M) c[static_cast<uint64_t>(row) * G.ldc + col] = acc[j][r];
        }
    }
}

template <int WN, int NWN>
__global__ void __launch_bounds__(128 * NWN) k_pf_gemm_q8(PfGemm G) {
    constexpr uint32_t NT = 128u * NWN;          // threads: 2 x NWN waves
    constexpr uint32_t BN = 32u * WN * NWN;      // W rows per tile
    constexpr uint32_t AU = 2u * kQgBM * 8u / NT / 2u;   // A 16-byte units per thread and array
    __shared__ __align__(16) unsigned char s_a[2][2][kQgBM * kQgPitch];   // [stage][hi, lo]
    __shared__ __align__(16) unsigned char s_w[2][BN * kQgPitch];          // [stage] quants
    __shared__ float s_sc[2][BN][2];                                       // [stage][row][block]
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kh = lane >> 5, l32 = lane & 31u;
    const uint32_t m0 = blockIdx.y * kQgBM, n0 = blockIdx.x * BN;
    const uint32_t nkb = G.K >> 5;                                         // Q8_0 blocks along K
    const uint32_t S = gridDim.z, z = blockIdx.z;
    const uint32_t kb_lo = nkb * z / S, kb_hi = nkb * (z + 1u) / S;
    const uint32_t nsteps = (kb_hi - kb_lo + 1u) / 2u;
    const uint64_t row_bytes = static_cast<uint64_t>(nkb) * 34u;

    // One K step in registers: A units u = 2t, 2t + 1 of hi and of lo (row u / 8, k 8 (u % 8)
    // .. + 7 of the step), and the 34-byte W block of thread t < 2 BN (row t / 2, block t % 2).
    struct Stage {
        v4u a[2][AU];  // [hi, lo][unit]
        uint32_t d[8]; // dwords at the block start rounded down to 4 bytes
        uint32_t u0;   // 16 bits at that start + 32, 16 bits at the block start + 32
        uint32_t u1;
        uint32_t sh;   // block start & 3 (0 or 2)
        bool wl;       // W block live
    };
    typedef const __attribute__((address_space(1))) v4u* gv4;
    const uint32_t wr = tid >> 1, wb = tid & 1u;
    static_assert(2u * BN <= NT, "one W block per thread");
    const bool wlive_t = tid < 2u * BN && n0 + wr < G.N;
    const uint8_t* wrow = G.w[0];
    if (G.glu) {   // 64-column groups: 32 gate rows, then the same 32 up rows
        const uint32_t n = wlive_t ? n0 + wr : 0u;
        wrow = ((n & 63u) < 32u ? G.w[0] : G.w[1]) + static_cast<uint64_t>(32u * (n >> 6) + (n & 31u)) * row_bytes;
    } else {
        uint32_t r = wlive_t ? n0 + wr : 0u;
        if (G.nseg > 1u && r >= G.rows[0]) {
            r -= G.rows[0];
            wrow = G.w[1];
            if (G.nseg > 2u && r >= G.rows[1]) {
                r -= G.rows[1];
                wrow = G.w[2];
            }
        }
        wrow += static_cast<uint64_t>(r) * row_bytes;
    }
    // Every load is issued unconditionally at a clamped, in-bounds address (dead data is zeroed
    // when it is stored): with no branch around a load the compiler counts the loads in flight
    // exactly, so the wait for step j's data does not also wait for the later steps of the ring.
    typedef const __attribute__((address_space(1))) uint32_t* gu32;
    typedef const __attribute__((address_space(1))) uint16_t* gu16;
    auto load = [&](uint32_t step, Stage& R) {
        const uint32_t kb = kb_lo + 2u * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, r = u >> 3, c = u & 7u;
            const uint32_t k = 32u * kb + 8u * c;
            const uint32_t rr = min(m0 + r, G.M - 1u), kk = min(k, 32u * kb_hi - 8u);
            const uint64_t o = (static_cast<uint64_t>(rr) * G.lda + kk) * 2u;
            R.a[0][j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(G.ahi) + o);
            R.a[1][j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(G.alo) + o);
        }
        const uint32_t b = kb + wb;
        R.wl = wlive_t && b < kb_hi;
        // the block's 34 bytes: 8 dwords from its start rounded down (2 bytes before it when the
        // start is 2 mod 4), then the 16 bits at that start + 32 and at the block start + 32; no
        // byte past the block is read
        const uintptr_t base = reinterpret_cast<uintptr_t>(wrow) + 34u * min(b, kb_hi - 1u);
        const uintptr_t lb = base & ~uintptr_t(3);
        R.sh = static_cast<uint32_t>(base & 3u);
#pragma unroll
        for (int j = 0; j < 8; ++j) R.d[j] = reinterpret_cast<gu32>(lb)[j];
        R.u0 = *reinterpret_cast<gu16>(lb + 32u);
        R.u1 = *reinterpret_cast<gu16>(base + 32u);
    };
    auto store = [&](const Stage& R, uint32_t st, uint32_t step) {
        const uint32_t kb = kb_lo + 2u * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, r = u >> 3, c = u & 7u;
            const bool live = m0 + r < G.M && 32u * kb + 8u * c < 32u * kb_hi;
#pragma unroll
            for (uint32_t p = 0; p < 2; ++p)
                *reinterpret_cast<v4u*>(&s_a[st][p][r * kQgPitch + c * 16u]) = live ? R.a[p][j] : v4u{0u, 0u, 0u, 0u};
        }
        if (tid >= 2u * BN) return;
        // quants at window offset sh + 2: shift 2 (sh == 0) or whole dwords from d[1] (sh == 2)
        const uint32_t d8 = R.sh ? (R.u0 | (R.u1 << 16)) : R.u0;
        uint32_t q[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t hi = j < 7 ? R.d[j + 1] : d8;
            q[j] = R.wl ? (R.sh ? hi : __builtin_amdgcn_alignbyte(hi, R.d[j], 2u)) : 0u;
        }
        unsigned char* dst = &s_w[st][wr * kQgPitch + wb * 64u];
#pragma unroll
        for (int j = 0; j < 4; ++j) {   // 8 quants (two dwords) -> 8 f16 per 16-byte store
            half8 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(q[2 * j] >> (8 * i))));
                v[4 + i] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(q[2 * j + 1] >> (8 * i))));
            }
            *reinterpret_cast<half8*>(dst + 16u * j) = v;
        }
        s_sc[st][wr][wb] = R.wl ? half_bits_to_float(R.sh ? (R.d[0] >> 16) : (R.d[0] & 0xffffu)) : 0.0f;
    };

    const uint32_t wm = wave / NWN, wn = wave % NWN;
    float16v acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = float16v{};
    auto compute = [&](uint32_t st) {
        const unsigned char* pa_hi = &s_a[st][0][(32u * wm + l32) * kQgPitch + 16u * kh];
        const unsigned char* pa_lo = &s_a[st][1][(32u * wm + l32) * kQgPitch + 16u * kh];
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {   // the step's two Q8_0 blocks
            half8 ah[2], al[2];
#pragma unroll
            for (uint32_t ks = 0; ks < 2; ++ks) {
                ah[ks] = *reinterpret_cast<const half8*>(pa_hi + 64u * b + 32u * ks);
                al[ks] = *reinterpret_cast<const half8*>(pa_lo + 64u * b + 32u * ks);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const uint32_t nl = 32u * (WN * wn + j) + l32;   // the lane's column in the tile
                const unsigned char* pw = &s_w[st][nl * kQgPitch + 64u * b + 16u * kh];
                const half8 w0 = *reinterpret_cast<const half8*>(pw), w1 = *reinterpret_cast<const half8*>(pw + 32u);
                float16v p = {};
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], w0, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0], w0, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], w1, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1], w1, p, 0, 0, 0);
                const float sc = s_sc[st][nl][b];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][r] += sc * p[r];
            }
        }
    };

    // The K loop runs in straight-line chunks of kQgChunk steps with a ring of kQgAhead register
    // stages: step j's loads are issued kQgAhead steps before it is stored to LDS, so they
    // overlap the MFMAs of the steps in between. Every load is issued unconditionally (clamped,
    // in-bounds addresses; steps past the end re-load the last one and are never stored), and
    // no loaded value crosses a chunk boundary: with no branch around a load and no value live
    // across a back edge, the compiler waits for exactly the step it stores.
    static_assert(kQgAhead <= kQgChunk, "ring inside a chunk");
    for (uint32_t i = 0; i < nsteps; i += kQgChunk) {
        Stage R[kQgAhead];
        auto clamp = [&](uint32_t j) { return min(i + j, nsteps - 1u); };
#pragma unroll
        for (uint32_t u = 0; u < kQgAhead; ++u) load(clamp(u), R[u]);
#pragma unroll
        for (uint32_t u = 0; u < kQgChunk; ++u) {
            const uint32_t j = i + u;
            if (j < nsteps) {
                // stage j & 1 was last read by step j - 2, which every wave finished before the
                // barrier of step j - 1
                store(R[u % kQgAhead], j & 1u, j);
                __syncthreads();
            }
            if (u + kQgAhead < kQgChunk) load(clamp(u + kQgAhead), R[u % kQgAhead]);
            if (j < nsteps) compute(j & 1u);
        }
    }
    pf_gemm_epilogue<WN, NWN>(G, acc, z, m0, n0, wm, wn, kh, l32, lane, reinterpret_cast<float*>(&s_a[0][0][0]));
}

// Masked softmax of score row (head z, query t): keys j of [max(0, t + 1 - window), t]
// (window 0: all j <= t), p_j = exp(scale * s_j - max) / sum, the sum in double
// (src/gemma3.cpp:1602-1696); p as f16 hi/lo over the row's first ceil((t + 1) / 64) * 64
// columns, zero outside the range (the O = P V GEMM reads up to there).
__global__ void __launch_bounds__(kPfThreads) k_pf_softmax(const float* S, uint32_t T, uint32_t Tp, float scale,
                                                           uint32_t window, _Float16* phi, _Float16* plo,
                                                           G3State* st, uint32_t block) {
#pragma clang fp contract(off)
    __shared__ double redd[4];
    __shared__ float redf[4];
    const uint32_t t = blockIdx.x, z = blockIdx.y;
    const uint64_t row = (static_cast<uint64_t>(z) * T + t) * Tp;   // rows of Tp columns
    const uint32_t j0 = (window != 0u && t + 1u > window) ? t + 1u - window : 0u;
    const uint32_t jend = min(Tp, ((t + kPfTile) / kPfTile) * kPfTile);
    float mx = -INFINITY;
    for (uint32_t j = j0 + threadIdx.x; j <= t; j += kPfThreads) mx = fmaxf(mx, S[row + j] * scale);
    mx = wave_red_max(mx);
    if ((threadIdx.x & 63u) == 0u) redf[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
    double den = 0.0;
    for (uint32_t j = j0 + threadIdx.x; j <= t; j += kPfThreads) den += static_cast<double>(expf(S[row + j] * scale - mx));
    const double den_all = pf_sum(den, redd);
    if (threadIdx.x == 0u && (!(den_all > 0.0) || !__builtin_isfinite(den_all)))   // :1666-1670
        atomicMin(&st->nonfinite, g3_code_softmax(block));
    const float inv_den = static_cast<float>(1.0 / den_all);
    for (uint32_t j = threadIdx.x; j < jend; j += kPfThreads) {
        const float p = (j >= j0 && j <= t) ? expf(S[row + j] * scale - mx) * inv_den : 0.0f;
        pf_split(p, phi + row + j, plo + row + j);
    }
}

// ---- QK-norm, RoPE, KV cache ------------------------------------------------------------

// Row t of qkv = [q (H heads x hd) | k (hd) | v (hd)]: QK-norm per head (src/gemma3.cpp:
// 1045-1104), NeoX RoPE at position t (:1371-1424), in place (q also as f16 hi/lo rows of
// qhi/qlo); then k and v go to the KV cache slot t % slots when position t is still in the
// window after the prompt (the serial loop's eviction leaves exactly those, :1590-1600), and
// v to column t of vt = V^T [hd][Tp], the B operand of O = P V. One workgroup per column
// t < Tp: those with t >= T write the zero padding columns (their weights in P are zero).
// One wave per head (lane l: dims l + 64 e): the sum of squares is a wave reduction and the
// RoPE partners come through the wave's own LDS row, so the kernel has no barrier.
constexpr uint32_t kPfQkMaxWaves = 8;
__global__ void __launch_bounds__(kPfQkMaxWaves * 64) k_pf_qk(float* qkv, uint32_t T, uint32_t H, uint32_t hd,
                                                            const float* q_norm, const float* k_norm,
                                                            const float* cos_t, const float* sin_t, float eps,
                                                            float* kc, float* vc, uint32_t slots, _Float16* qhi,
                                                            _Float16* qlo, uint32_t Tp, float* vt) {
#pragma clang fp contract(off)
    __shared__ float xs[kPfQkMaxWaves][256];
    const uint32_t t = blockIdx.x;
    if (t >= T) {   // whole workgroup
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) vt[static_cast<uint64_t>(i) * Tp + t] = 0.0f;
        return;
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t nqkv = (H + 2u) * hd, half = hd >> 1;
    float* row = qkv + static_cast<uint64_t>(t) * nqkv;
    float* xw = xs[wave];
    const bool keep = t + slots >= T;
    const uint64_t slot = static_cast<uint64_t>(t % slots) * hd;
    for (uint32_t hh = wave; hh <= H; hh += nw) {   // H query heads, then the key head
        float* x = row + hh * hd;
        const float* w = hh < H ? q_norm : k_norm;
        float v[4];
        double sq = 0.0;
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t i = lane + 64u * e;
            v[e] = i < hd ? x[i] : 0.0f;
            sq += static_cast<double>(v[e]) * static_cast<double>(v[e]);
        }
        const float sc = pf_rms_scale(wave_red_sum_d(sq), hd, eps);
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t i = lane + 64u * e;
            if (i < hd) xw[i] = (v[e] * sc) * w[i];
        }
        // the partners are other lanes' values: a wave's LDS accesses complete in order
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            const uint32_t i = lane + 64u * e;
            if (i < hd) {
                const uint32_t ei = i < half ? i : i - half;
                const float c = cos_t[static_cast<uint64_t>(t) * half + ei], s = sin_t[static_cast<uint64_t>(t) * half + ei];
                const float a = xw[ei], b = xw[ei + half];
                const float y2 = i < half ? a * c - b * s : b * c + a * s;
                x[i] = y2;
                if (hh < H) {   // the query as the attention GEMM's A operand, [T][H * hd]
                    const uint64_t o = static_cast<uint64_t>(t) * H * hd + hh * hd + i;
                    pf_split(y2, qhi + o, qlo + o);
                } else if (keep) {
                    kc[slot + i] = y2;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();   // this head's reads of xw come before the next head's writes
    }
    for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {   // v is not normed
        const float vv = row[(H + 1u) * hd + i];
        if (keep) vc[slot + i] = vv;
        vt[static_cast<uint64_t>(i) * Tp + t] = vv;
    }
}

// ---- expanded weights ------------------------------------------------------------------------

// One-time expansion of a Q8_0 matrix for the prefill GEMMs: row n of the expanded matrix gets
// the quants of source row src(n) as f16 (exact: |q| <= 127) and its block scales as fp32. With
// `glu`, the rows are the gate/up matrices interleaved in groups of 64 (32 gate rows, then the
// same 32 up rows: the column order of the gate/up GEMM's epilogue); otherwise up to three
// matrices are concatenated. One thread per (row, block).
__global__ void __launch_bounds__(kPfThreads) k_pf_expand(const uint8_t* w0, const uint8_t* w1, const uint8_t* w2,
                                                          uint32_t rows0, uint32_t rows1, uint32_t N, uint32_t nkb,
                                                          uint32_t glu, _Float16* wh, float* ws) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kPfThreads + threadIdx.x;
    if (i >= static_cast<uint64_t>(N) * nkb) return;
    const uint32_t n = static_cast<uint32_t>(i / nkb), b = static_cast<uint32_t>(i % nkb);
    const uint8_t* src;
    if (glu) {
        const uint32_t grp = n >> 6, wi = n & 63u;
        src = (wi < 32u ? w0 : w1) + static_cast<uint64_t>(32u * grp + (wi & 31u)) * nkb * 34u;
    } else if (n < rows0) {
        src = w0 + static_cast<uint64_t>(n) * nkb * 34u;
    } else if (n < rows0 + rows1) {
        src = w1 + static_cast<uint64_t>(n - rows0) * nkb * 34u;
    } else {
        src = w2 + static_cast<uint64_t>(n - rows0 - rows1) * nkb * 34u;
    }
    const uint8_t* blk = src + 34u * b;
    ws[i] = half_bits_to_float(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
    _Float16* dst = wh + static_cast<uint64_t>(n) * nkb * 32u + 32u * b;
#pragma unroll
    for (uint32_t k = 0; k < 32u; ++k) dst[k] = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(blk[2 + k])));
}

// The Q8_0 GEMM of k_pf_gemm_q8 on expanded weights (G.wh, G.ws): a K step stages the f16 rows
// of the tile's W block with plain 16-byte copies (no int8 conversion on the K loop's critical
// path) and the two block scales per row. Same tiles, splits, LDS layout, K-loop ring and
// epilogues as k_pf_gemm_q8, with twice the waves: wave group kw (of 2 NWN waves) computes the
// step's Q8_0 block kw for every tile, so a SIMD runs two waves whose MFMA chains and
// scale-and-add work overlap; the kw = 1 partial tiles are added to the kw = 0 ones through
// LDS before the epilogue (sum of the even blocks, then of the odd ones).
template <int WN, int NWN>
__global__ void __launch_bounds__(256 * NWN) k_pf_gemm_h(PfGemm G) {
    constexpr uint32_t NT = 256u * NWN;
    constexpr uint32_t BN = 32u * WN * NWN;
    constexpr uint32_t AU = 2u * kQgBM * 8u / NT;   // A 16-byte units per thread (hi units, then lo)
    constexpr uint32_t WU = BN * 8u / NT;           // W 16-byte units per thread (8 per row)
    static_assert(AU >= 1u && 2u * kQgBM * 8u % NT == 0u, "whole A units per thread");
    static_assert(WU >= 1u && BN * 8u % NT == 0u, "whole W units per thread");
    static_assert(BN <= NT, "one scale pair per thread");
    __shared__ __align__(16) unsigned char s_a[2][2][kQgBM * kQgPitch];
    __shared__ __align__(16) unsigned char s_w[2][BN * kQgPitch];
    __shared__ float s_sc[2][BN][2];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kh = lane >> 5, l32 = lane & 31u;
    const uint32_t m0 = blockIdx.y * kQgBM, n0 = blockIdx.x * BN;
    const uint32_t nkb = G.K >> 5;
    const uint32_t S = gridDim.z, z = blockIdx.z;
    const uint32_t kb_lo = nkb * z / S, kb_hi = nkb * (z + 1u) / S;
    const uint32_t nsteps = (kb_hi - kb_lo + 1u) / 2u;
    typedef const __attribute__((address_space(1))) v4u* gv4;
    struct Stage {
        v4u a[AU];   // unit u = AU tid + j: array u / (8 kQgBM), row (u % (8 kQgBM)) / 8, column u % 8
        v4u w[WU];
        float2 sc;
    };
    // Every load is issued at a clamped, in-bounds address (dead data is zeroed when stored).
    auto load = [&](uint32_t step, Stage& R) {
        const uint32_t kb = kb_lo + 2u * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, ui = u % (8u * kQgBM), r = ui >> 3, c = ui & 7u;
            const uint32_t k = 32u * kb + 8u * c;
            const uint32_t rr = min(m0 + r, G.M - 1u), kk = min(k, 32u * kb_hi - 8u);
            const uint64_t o = (static_cast<uint64_t>(rr) * G.lda + kk) * 2u;
            R.a[j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(u < 8u * kQgBM ? G.ahi : G.alo) + o);
        }
#pragma unroll
        for (uint32_t j = 0; j < WU; ++j) {
            const uint32_t u = WU * tid + j, r = u >> 3, c = u & 7u;
            const uint32_t rr = min(n0 + r, G.N - 1u), kk = min(32u * kb + 8u * c, 32u * kb_hi - 8u);
            R.w[j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(G.wh) + (static_cast<uint64_t>(rr) * G.K + kk) * 2u);
        }
        {   // the step's two block scales of row tid (clamped to the split's last block)
            typedef const __attribute__((address_space(1))) float* gf;
            const uint32_t rr = min(n0 + (tid < BN ? tid : 0u), G.N - 1u), bb = min(kb, kb_hi - 1u);
            const gf row = reinterpret_cast<gf>(reinterpret_cast<uintptr_t>(G.ws + static_cast<uint64_t>(rr) * nkb));
            R.sc = make_float2(row[bb], row[min(bb + 1u, kb_hi - 1u)]);
        }
    };
    auto store = [&](const Stage& R, uint32_t st, uint32_t step) {
        const uint32_t kb = kb_lo + 2u * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, ui = u % (8u * kQgBM), r = ui >> 3, c = ui & 7u;
            const bool live = m0 + r < G.M && 32u * kb + 8u * c < 32u * kb_hi;
            *reinterpret_cast<v4u*>(&s_a[st][u / (8u * kQgBM)][r * kQgPitch + c * 16u]) =
                live ? R.a[j] : v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (uint32_t j = 0; j < WU; ++j) {
            const uint32_t u = WU * tid + j, r = u >> 3, c = u & 7u;
            const bool live = n0 + r < G.N && 32u * kb + 8u * c < 32u * kb_hi;
            *reinterpret_cast<v4u*>(&s_w[st][r * kQgPitch + c * 16u]) = live ? R.w[j] : v4u{0u, 0u, 0u, 0u};
        }
        if (tid < BN) {
            const bool rl = n0 + tid < G.N;
            s_sc[st][tid][0] = rl && kb < kb_hi ? R.sc.x : 0.0f;
            s_sc[st][tid][1] = rl && kb + 1u < kb_hi ? R.sc.y : 0.0f;
        }
    };
    const uint32_t kw = wave / (2u * NWN), wv = wave % (2u * NWN);   // block of the step, tile
    const uint32_t wm = wv / NWN, wn = wv % NWN;
    float16v acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = float16v{};
    auto compute = [&](uint32_t st) {
        const unsigned char* pa_hi = &s_a[st][0][(32u * wm + l32) * kQgPitch + 16u * kh];
        const unsigned char* pa_lo = &s_a[st][1][(32u * wm + l32) * kQgPitch + 16u * kh];
        {
            const uint32_t b = kw;
            half8 ah[2], al[2];
#pragma unroll
            for (uint32_t ks = 0; ks < 2; ++ks) {
                ah[ks] = *reinterpret_cast<const half8*>(pa_hi + 64u * b + 32u * ks);
                al[ks] = *reinterpret_cast<const half8*>(pa_lo + 64u * b + 32u * ks);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const uint32_t nl = 32u * (WN * wn + j) + l32;
                const unsigned char* pw = &s_w[st][nl * kQgPitch + 64u * b + 16u * kh];
                const half8 w0 = *reinterpret_cast<const half8*>(pw), w1 = *reinterpret_cast<const half8*>(pw + 32u);
                float16v p = {};
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], w0, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0], w0, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], w1, p, 0, 0, 0);
                p = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1], w1, p, 0, 0, 0);
                const float sc = s_sc[st][nl][b];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][r] += sc * p[r];
            }
        }
    };
    static_assert(kQgAhead <= kQgChunk, "ring inside a chunk");
    for (uint32_t i = 0; i < nsteps; i += kQgChunk) {
        Stage R[kQgAhead];
        auto clamp = [&](uint32_t j) { return min(i + j, nsteps - 1u); };
#pragma unroll
        for (uint32_t u = 0; u < kQgAhead; ++u) load(clamp(u), R[u]);
#pragma unroll
        for (uint32_t u = 0; u < kQgChunk; ++u) {
            const uint32_t j = i + u;
            if (j < nsteps) {
                store(R[u % kQgAhead], j & 1u, j);
                __syncthreads();
            }
            if (u + kQgAhead < kQgChunk) load(clamp(u + kQgAhead), R[u % kQgAhead]);
            if (j < nsteps) compute(j & 1u);
        }
    }
    {   // odd-block partials into the even-block waves (s_w: 2 NWN WN 16 x 64 floats fit)
        static_assert(2u * NWN * WN * 16u * 64u * 4u <= sizeof(s_w), "reduction area");
        __syncthreads();   // every wave is done reading the LDS stages
        float* red = reinterpret_cast<float*>(&s_w[0][0]);
        if (kw == 1u) {
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[((wv * WN + j) * 16u + r) * 64u + lane] = acc[j][r];
        }
        __syncthreads();
        if (kw == 0u) {
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][r] += red[((wv * WN + j) * 16u + r) * 64u + lane];
        }
    }
    pf_gemm_epilogue<WN, NWN>(G, acc, z, m0, n0, wm, wn, kh, l32, lane, reinterpret_cast<float*>(&s_a[0][0][0]),
                              kw == 0u);
}

// ---- host side --------------------------------------------------------------------------

template <int MODE>
static int pf_launch(const PfGemm& G, uint32_t batch, hipStream_t s) {
    const dim3 grid((G.N + kPfGT - 1u) / kPfGT, (G.M + kPfGT - 1u) / kPfGT, batch);
    PfGemm arg = G;
    void* args[] = {&arg};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_gemm<MODE>), grid, dim3(kPfThreads), args, 0, s));
    return VRT_OK;
}

template <int WN, int NWN>
static int pf_launch_q8(const PfGemm& G, uint32_t splits, hipStream_t s) {
    constexpr uint32_t BN = 32u * WN * NWN;
    const dim3 grid((G.N + BN - 1u) / BN, (G.M + kQgBM - 1u) / kQgBM, splits);
    PfGemm arg = G;
    void* args[] = {&arg};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_gemm_q8<WN, NWN>), grid, dim3(128u * NWN), args,
                                  0, s));
    return VRT_OK;
}

template <int WN, int NWN>
static int pf_launch_h(const PfGemm& G, uint32_t splits, hipStream_t s) {
    constexpr uint32_t BN = 32u * WN * NWN;
    const dim3 grid((G.N + BN - 1u) / BN, (G.M + kQgBM - 1u) / kQgBM, splits);
    PfGemm arg = G;
    void* args[] = {&arg};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_gemm_h<WN, NWN>), grid, dim3(256u * NWN), args,
                                  0, s));
    return VRT_OK;
}

// The Q8_0 GEMM's launch: on the expanded weights when `ex` holds them, else on the arena.
static int pf_launch_w(PfGemm& G, const PfMatrix* ex, uint32_t splits, hipStream_t s) {
    const uint32_t mt = (G.M + kQgBM - 1u) / kQgBM;
    const bool wide = G.N % 128u == 0u && (G.N / 128u) * mt >= 128u;
    if (ex && ex->h) {
        G.wh = static_cast<const _Float16*>(ex->h);
        G.ws = ex->s;
        return wide ? pf_launch_h<1, 4>(G, splits, s) : pf_launch_h<1, 2>(G, splits, s);
    }
    return wide ? pf_launch_q8<1, 4>(G, splits, s) : pf_launch_q8<1, 2>(G, splits, s);
}

// C[M][N] = A[M][K] (f16 hi/lo) x W^T, W = Q8_0 matrices concatenated along N (or their
// expansion `ex`). With splits > 1 the K blocks are split and C holds the partial products
// C + z * M * N, z < splits.
static int pf_gemm(vrt_g3* g, const _Float16* ahi, const _Float16* alo, uint32_t M, uint32_t K,
                   std::initializer_list<std::pair<const uint8_t*, uint32_t>> segs, const PfMatrix* ex, float* c,
                   uint32_t splits, hipStream_t s) {
    PfGemm G{};
    G.ahi = ahi;
    G.alo = alo;
    G.lda = K;
    for (const auto& sg : segs) {
        G.w[G.nseg] = sg.first;
        G.rows[G.nseg++] = sg.second;
        G.N += sg.second;
    }
    G.w_end = g->P.arena_end;
    G.c = c;
    G.ldc = G.N;
    G.M = M;
    G.K = K;
    if (K % 32u != 0u || G.N % 32u != 0u) return set_error(VRT_ERR_INVALID, "prefill GEMM shape not supported");
    G.c_bs = static_cast<uint64_t>(M) * G.N;
    splits = std::max(1u, std::min(splits, (K / 32u) / 2u));
    return pf_launch_w(G, ex, splits, s);
}

// gelu_tanh(A Wg^T) * (A Wu^T) as f16 hi/lo [M][F] (row stride F): the gate/up GEMM with the
// product in its epilogue (src/gemma3.cpp:1720-1801 up to the down projection), one K split.
static int pf_gemm_glu(vrt_g3* g, const _Float16* ahi, const _Float16* alo, uint32_t M, uint32_t K, const uint8_t* wg,
                       const uint8_t* wu, uint32_t F, const PfMatrix* ex, _Float16* ohi, _Float16* olo, hipStream_t s) {
    PfGemm G{};
    G.ahi = ahi;
    G.alo = alo;
    G.lda = K;
    G.w[0] = wg;
    G.w[1] = wu;
    G.rows[0] = G.rows[1] = F;
    G.nseg = 2u;
    G.N = 2u * F;
    G.w_end = g->P.arena_end;
    G.chi = ohi;
    G.clo = olo;
    G.ldc = F;
    G.M = M;
    G.K = K;
    G.glu = 1u;
    if (K % 32u != 0u || F % 32u != 0u) return set_error(VRT_ERR_INVALID, "prefill GEMM shape not supported");
    return pf_launch_w(G, ex, 1u, s);
}

// K splits of the 640-row projections (O and down): enough workgroups to cover the CUs.
static uint32_t pf_splits(uint32_t M, uint32_t N) {
    const uint32_t tiles = ((M + kQgBM - 1u) / kQgBM) * ((N + 63u) / 64u);
    return std::min(kPfMaxSplits, std::max(1u, 256u / std::max(1u, tiles)));
}

static uint32_t pf_pad(uint32_t T) { return (T + kPfTile - 1u) / kPfTile * kPfTile; }

int pf_setup(vrt_g3* g, uint32_t max_t) {
    const uint32_t d = g->cfg.embedding_length, H = g->cfg.head_count, hd = g->cfg.head_dim;
    const uint32_t F = g->cfg.feed_forward_length, qw = H * hd, nqkv = qw + 2u * hd;
    const uint32_t kmax = std::max(std::max(d, qw), F);
    PfState& p = g->pf;
    p.max_t = 0;
    if (d > 8u * kPfThreads || hd > 256u || hd % 32u || d % 32u || qw % 32u || F % 32u || nqkv % 32u) return VRT_OK;
    const uint64_t tp = pf_pad(max_t);
    auto take = [&](size_t bytes, void** out) -> int {
        VRT_HIP_CHECK(hipMalloc(out, bytes + 256u));
        g->allocs.push_back(*out);
        return VRT_OK;
    };
    void* q;
    if (int rc = take(static_cast<size_t>(max_t) * d * 4u, &q)) return rc;
    p.h = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(max_t) * d * 4u * kPfMaxSplits, &q)) return rc;
    p.x = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(max_t) * kmax * 2u, &q)) return rc;
    p.ahi = q;
    if (int rc = take(static_cast<size_t>(max_t) * kmax * 2u, &q)) return rc;
    p.alo = q;
    if (int rc = take(static_cast<size_t>(max_t) * std::max(nqkv, 2u * F) * 4u, &q)) return rc;
    p.big = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(H) * max_t * tp * 4u, &q)) return rc;
    p.s = static_cast<float*>(q);
    if (int rc = take(static_cast<size_t>(H) * max_t * tp * 2u, &q)) return rc;
    p.phi = q;
    if (int rc = take(static_cast<size_t>(H) * max_t * tp * 2u, &q)) return rc;
    p.plo = q;
    if (int rc = take(static_cast<size_t>(hd) * tp * 4u, &q)) return rc;
    p.vt = static_cast<float*>(q);
    // Expanded weights: 2 bytes per quant + 4 per 32 (2.125 bytes per weight, twice the Q8_0
    // matrices' 1.0625), made once here when they fit kPfExpandBudget.
    const uint64_t per_layer = static_cast<uint64_t>(nqkv) * d + static_cast<uint64_t>(d) * qw +
                               2ull * F * d + static_cast<uint64_t>(d) * F;
    const uint64_t total = per_layer * g->layers.size() * 2u + per_layer * g->layers.size() / 8u;
    p.lw.clear();
    if (total <= kPfExpandBudget) {
        p.lw.resize(g->layers.size());
        const hipStream_t s = g->ctx->stream;
        auto expand = [&](const uint8_t* w0, const uint8_t* w1, const uint8_t* w2, uint32_t r0, uint32_t r1, uint32_t N,
                          uint32_t K, uint32_t glu, PfMatrix* m) -> int {
            void* hq;
            void* sq;
            if (int rc = take(static_cast<size_t>(N) * K * 2u, &hq)) return rc;
            if (int rc = take(static_cast<size_t>(N) * (K / 32u) * 4u, &sq)) return rc;
            uint32_t nkb = K / 32u;
            _Float16* wh = static_cast<_Float16*>(hq);
            float* ws = static_cast<float*>(sq);
            void* args[] = {&w0, &w1, &w2, &r0, &r1, &N, &nkb, &glu, &wh, &ws};
            const uint64_t n = static_cast<uint64_t>(N) * nkb;
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_expand),
                                          dim3(static_cast<uint32_t>((n + kPfThreads - 1u) / kPfThreads)),
                                          dim3(kPfThreads), args, 0, s));
            m->h = hq;
            m->s = ws;
            return VRT_OK;
        };
        for (size_t l = 0; l < g->layers.size(); ++l) {
            const LayerParams& Ly = g->layers[l];
            PfLayerW& w = p.lw[l];
            if (int rc = expand(Ly.wq, Ly.wk, Ly.wv, qw, hd, nqkv, d, 0u, &w.qkv)) return rc;
            if (int rc = expand(Ly.wo, Ly.wo, Ly.wo, d, 0u, d, qw, 0u, &w.o)) return rc;
            if (int rc = expand(Ly.wg, Ly.wu, Ly.wu, F, F, 2u * F, d, 1u, &w.gu)) return rc;
            if (int rc = expand(Ly.wd, Ly.wd, Ly.wd, d, 0u, d, F, 0u, &w.down)) return rc;
        }
    }
    p.max_t = max_t;
    return VRT_OK;
}

// Causal local/global attention of one block over qkv rows [T][q | k | v] (q, k normed and
// rotated; q also as f16 hi/lo in qhi/qlo) into att hi/lo [T][H * hd], all on MFMA:
// S_h = Q_h K^T (key tiles no query sees skipped), masked softmax -> P_h, O_h = P_h V.
static int pf_attention(vrt_g3* g, const LayerParams& Ly, uint32_t T, const float* qkv, const _Float16* qhi,
                        const _Float16* qlo, _Float16* att_hi, _Float16* att_lo, hipStream_t s) {
    const PfState& p = g->pf;
    const uint32_t H = g->cfg.head_count, hd = g->cfg.head_dim, qw = H * hd, nqkv = qw + 2u * hd;
    const uint32_t Tp = pf_pad(T);
    const uint32_t window = Ly.slots >= g->cfg.context_length ? 0u : Ly.slots;
    {   // S_h = Q_h K^T: [H][T][Tp]
        PfGemm G{};
        G.ahi = qhi;
        G.alo = qlo;
        G.lda = qw;
        G.a_bs = hd;
        G.b = qkv + qw;
        G.ldb = nqkv;
        G.c = p.s;
        G.ldc = Tp;
        G.c_bs = static_cast<uint64_t>(T) * Tp;
        G.M = T;
        G.N = T;
        G.K = hd;
        G.window = window;
        if (int rc = pf_launch<kGemmB32 | kGemmCausalS>(G, H, s)) return rc;
    }
    {
        const float* S = p.s;
        float scale = g->P.attn_scale;
        uint32_t t = T, tp = Tp, w = window;
        _Float16* phi = static_cast<_Float16*>(p.phi);
        _Float16* plo = static_cast<_Float16*>(p.plo);
        G3State* st = g->P.st;
        uint32_t blk = Ly.index;
        void* args[] = {&S, &t, &tp, &scale, &w, &phi, &plo, &st, &blk};
        VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_softmax), dim3(T, H), dim3(kPfThreads), args, 0, s));
    }
    {   // O_h = P_h V -> att[:, h * hd ..]
        PfGemm G{};
        G.ahi = static_cast<const _Float16*>(p.phi);
        G.alo = static_cast<const _Float16*>(p.plo);
        G.lda = Tp;
        G.a_bs = static_cast<uint64_t>(T) * Tp;
        G.b = p.vt;
        G.ldb = Tp;
        G.chi = att_hi;
        G.clo = att_lo;
        G.ldc = qw;
        G.c_bs = hd;
        G.M = T;
        G.N = hd;
        G.K = Tp;
        G.window = window;
        if (int rc = pf_launch<kGemmB32 | kGemmCausalO | kGemmOut16>(G, H, s)) return rc;
    }
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
    auto launch = [&](const void* fn, dim3 grid, void** args) -> int {
        VRT_HIP_CHECK(hipLaunchKernel(fn, grid, dim3(kPfThreads), args, 0, s));
        return VRT_OK;
    };
    {
        const uint8_t* te = P.tok_embd;
        const uint32_t* tok = P.tokens;
        float es = P.emb_scale;
        void* args[] = {&te, &tok, &d, &es, &h};
        if (int rc = launch(reinterpret_cast<const void*>(&k_pf_embed), dim3(T), args)) return rc;
    }
    const PfLayerW* lw = p.lw.empty() ? nullptr : p.lw.data();
    const uint32_t s_o = pf_splits(T, d);        // split partials of the O and down projections
    uint64_t xs = static_cast<uint64_t>(T) * d;  // one partial [T][d]
    uint32_t s_down = 1;                         // splits of the previous block's down projection
    for (uint32_t l = 0; l < L; ++l) {
        const LayerParams& Ly = g->layers[l];
        {   // previous block's FFN output into the residual, then the attention norm
            const float* f = l ? x : nullptr;
            const float* wpost = l ? g->layers[l - 1].post_ffw : nullptr;
            const float* wnext = Ly.attn_norm;
            uint32_t blk = l ? l - 1u : 0u;
            void* args[] = {&h, &f, &s_down, &xs, &wpost, &wnext, &d, &eps, &ahi, &alo, &st, &blk};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_norm), dim3(T), args)) return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, d, {{Ly.wq, qw}, {Ly.wk, hd}, {Ly.wv, hd}}, lw ? &lw[l].qkv : nullptr, big, 1, s)) return rc;
        {
            const float* qn = Ly.q_norm;
            const float* kn = Ly.k_norm;
            const float* ct = Ly.global ? P.cos_g : P.cos_l;
            const float* sn = Ly.global ? P.sin_g : P.sin_l;
            float* kc = Ly.kc;
            float* vc = Ly.vc;
            uint32_t slots = Ly.slots;
            uint32_t tp = pf_pad(T);
            float* vt = g->pf.vt;
            void* args[] = {&big, &T, &H, &hd, &qn, &kn, &ct, &sn, &eps, &kc, &vc, &slots, &ahi, &alo, &tp, &vt};
            const uint32_t waves = std::min(H + 1u, kPfQkMaxWaves);
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_qk), dim3(tp), dim3(64u * waves), args, 0, s));
        }
        // q (hi/lo in ahi/alo) is consumed by S = Q K^T before O = P V overwrites ahi/alo
        if (int rc = pf_attention(g, Ly, T, big, ahi, alo, ahi, alo, s)) return rc;
        uint32_t so = s_o;
        if (int rc = pf_gemm(g, ahi, alo, T, qw, {{Ly.wo, d}}, lw ? &lw[l].o : nullptr, x, so, s)) return rc;
        so = std::max(1u, std::min(so, (qw / 32u) / 2u));
        {   // attention output into the residual, then the FFN norm
            const float* f = x;
            const float* wpost = Ly.post_attn;
            const float* wnext = Ly.ffn_norm;
            uint32_t blk = Ly.index;
            void* args[] = {&h, &f, &so, &xs, &wpost, &wnext, &d, &eps, &ahi, &alo, &st, &blk};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_norm), dim3(T), args)) return rc;
        }
        // gelu(gate) * up as f16 hi/lo in `big` (the gate/up GEMM still reads ahi/alo). The last
        // block's FFN output feeds only the LM head, so there it runs for the last position alone.
        const bool last = l + 1u == L;
        const uint32_t fr = last ? 1u : T;
        const uint64_t a0 = last ? static_cast<uint64_t>(T - 1u) * d : 0u;
        _Float16* ghi = reinterpret_cast<_Float16*>(big);
        _Float16* glo = ghi + static_cast<uint64_t>(fr) * F;
        if (int rc = pf_gemm_glu(g, ahi + a0, alo + a0, fr, d, Ly.wg, Ly.wu, F, lw ? &lw[l].gu : nullptr, ghi, glo, s))
            return rc;
        s_down = std::max(1u, std::min(last ? pf_splits(1u, d) : s_o, (F / 32u) / 2u));
        if (int rc = pf_gemm(g, ghi, glo, fr, F, {{Ly.wd, d}}, lw ? &lw[l].down : nullptr, x, s_down, s)) return rc;
    }
    {   // last position: its FFN output (the split partials summed in order) and its residual
        // feed the decode step's final norm + LM head
        float* out = P.f;
        uint32_t nsplit = s_down;
        void* args[] = {&x, &nsplit, &d, &out};
        if (int rc = launch(reinterpret_cast<const void*>(&k_pf_sum), dim3(1), args)) return rc;
    }
    VRT_HIP_CHECK(hipMemcpyAsync(P.hmid, h + static_cast<uint64_t>(T - 1u) * d, d * 4u, hipMemcpyDeviceToDevice, s));
    return g3_enqueue_lm(g, s);
}

}  // namespace vrt
