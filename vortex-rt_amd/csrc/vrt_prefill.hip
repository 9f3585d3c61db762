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

// pf_split of four consecutive values (8-byte aligned destinations).
__device__ __forceinline__ void pf_split4(f4 x, _Float16* hi, _Float16* lo) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    half4 h, l;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        h[k] = static_cast<_Float16>(x[k]);
        l[k] = static_cast<_Float16>(x[k] - static_cast<float>(h[k]));
    }
    *reinterpret_cast<half4*>(hi) = h;
    *reinterpret_cast<half4*>(lo) = l;
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

// One wave per row t (four rows per workgroup, `rows` rows in all; n <= 64 NE elements, NE per
// lane; the sums are wave reductions, with no barrier). With f (the previous sublayer's output,
// the sum of nsplit partial rows f + s * sstride added in order s = 0, 1, ...):
// h = f * (scale(f) * w_post) + h (rms_norm_inplace then add_inplace, src/gemma3.cpp:1036-1042,
// :1703-1711, :1849-1855). Then, with w_next:
// the GEMM input (h * scale(h)) * w_next as f16 hi/lo (rms_norm_into, :991-996), or with
// `into` 0 h * (scale(h) * w_next) (rms_norm_inplace, the output norm :1866-1868). nonfinite:
// lowest block whose residual went non-finite (:1857-1863), reported through st->nonfinite.
template <uint32_t NE>
__global__ void __launch_bounds__(kPfThreads) k_pf_norm_w(float* h, const float* f, uint32_t nsplit, uint64_t sstride,
                                                          const float* w_post, const float* w_next, uint32_t n, float eps,
                                                          _Float16* xhi, _Float16* xlo, G3State* st, uint32_t block,
                                                          uint32_t rows, uint32_t into) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * (kPfThreads / 64u) + (threadIdx.x >> 6);
    if (t >= rows) return;   // whole wave
    float* hr = h + static_cast<uint64_t>(t) * n;
    // Every load is issued at a clamped, in-bounds index and masked afterwards, so the loads of
    // a row are in flight together (no branch, hence no wait, between them).
    uint32_t ic[NE];
    bool live[NE];
#pragma unroll
    for (uint32_t k = 0; k < NE; ++k) {
        live[k] = lane + 64u * k < n;
        ic[k] = min(lane + 64u * k, n - 1u);
    }
    float hv[NE], wp[NE], wn[NE];
#pragma unroll
    for (uint32_t k = 0; k < NE; ++k) {
        hv[k] = hr[ic[k]];
        wp[k] = w_post ? w_post[ic[k]] : 0.0f;
        wn[k] = w_next ? w_next[ic[k]] : 0.0f;
    }
    if (f) {
        const float* fr = f + static_cast<uint64_t>(t) * n;
        // every partial is loaded before the first add, then the partials are added in split order
        float fp[NE][kPfMaxSplits];
#pragma unroll
        for (uint32_t q = 0; q < kPfMaxSplits; ++q) {
            const float* fq = fr + min(q, nsplit - 1u) * sstride;
#pragma unroll
            for (uint32_t k = 0; k < NE; ++k) fp[k][q] = fq[ic[k]];
        }
        float fv[NE];
        double ss = 0.0;
#pragma unroll
        for (uint32_t k = 0; k < NE; ++k) {
            fv[k] = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < kPfMaxSplits; ++q)
                if (q < nsplit) fv[k] += fp[k][q];
            if (!live[k]) fv[k] = 0.0f;
            ss += static_cast<double>(fv[k]) * static_cast<double>(fv[k]);
        }
        const float sc = pf_rms_scale(wave_red_sum_d(ss), n, eps);
        int bad = 0;
#pragma unroll
        for (uint32_t k = 0; k < NE; ++k) {
            hv[k] = fv[k] * (sc * wp[k]) + hv[k];
            if (live[k]) {
                hr[ic[k]] = hv[k];
                bad |= !__builtin_isfinite(hv[k]);
            }
        }
        if (bad) atomicMin(&st->nonfinite, g3_code_nonfinite(block));
    }
    if (!w_next) return;
    double ss = 0.0;
#pragma unroll
    for (uint32_t k = 0; k < NE; ++k) {
        const float v = live[k] ? hv[k] : 0.0f;
        ss += static_cast<double>(v) * static_cast<double>(v);
    }
    const float sc = pf_rms_scale(wave_red_sum_d(ss), n, eps);
#pragma unroll
    for (uint32_t k = 0; k < NE; ++k) {
        const float y = into ? (hv[k] * sc) * wn[k] : hv[k] * (sc * wn[k]);
        if (live[k]) pf_split(y, xhi + static_cast<uint64_t>(t) * n + ic[k], xlo + static_cast<uint64_t>(t) * n + ic[k]);
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


// ---- GEMM on MFMA: Q8_0 weights ---------------------------------------------------------------

struct PfGemm {
    const _Float16* ahi;     // A [M][K] (row stride lda), f16 high and low parts
    const _Float16* alo;
    uint32_t lda;
    const uint8_t* w[3];     // W as Q8_0 matrices concatenated along N (rows[i] rows each)
    uint32_t rows[3];
    uint32_t nseg;
    const uint8_t* w_end;    //   one past the arena
    float* c;                // C [M][N] fp32 (row stride ldc; split z at c + z * c_bs), or
    _Float16* chi;           //   C as f16 high and low parts
    _Float16* clo;
    uint32_t ldc;
    uint64_t c_bs;
    uint32_t M, N, K;
    uint32_t glu;            // Q8_0 GEMM: w[0] = gate, w[1] = up (N = 2F), output gelu_tanh(gate) * up
    const _Float16* wh;      // expanded weights: the quants of N rows as f16 [N][K] (nullptr: Q8_0 w)
    const float* ws;         //   and their block scales [N][K / 32]
};

// C[M][N] = A[M][K] (f16 hi/lo) x W^T with W the Q8_0 rows (segments concatenated along N).
// Workgroup tile: 64 rows of A x 64 * WN rows of W; wave w computes rows 32 (w / 2) and the
// WN 32-column MFMA tiles from 32 WN (w % 2). K advances 64 (two Q8_0 blocks) per step through
// two LDS stages: A as f16 hi and lo [64][64], W as its exact int8 quants in f16 [64 WN][64]
// plus the fp32 block scales; one barrier per step hands a stage over. Per Q8_0 block and tile the
// two f16 MFMA chains (A hi, A lo) accumulate the exact products in fp32 and the block's partial
// is scaled by the column's scale into the fp32 accumulator. MFMA operands
// (v_mfma_f32_32x32x16_f16): lane l gives A[m = l % 32][k = 8 (l / 32) + j] and B[k][n = l % 32]
// for j < 8 of each 16-wide k step; result r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4]
// [l % 32]. blockIdx.z splits K: split z covers K blocks [z nkb / S, (z + 1) nkb / S) and writes
// C + z * c_bs; the consumer adds the S partial tiles in split order.
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

// Operand layouts of the attention keys and values (per 32-key tile, so that every MFMA operand
// load of a wave is one contiguous 1 KB): the key rows of a tile are stored in the order pkey
// (bits 2 and 3 of the index swapped, an involution), and for S^T = K Q^T the k step s, lane
// half f and row m of the A operand hold K[32 tile + pkey(m)][16 s + 8 f + j], j < 8; for
// O^T += V^T E^T the d tile dt, k step sk, lane half f and row m hold V[32 tile + 16 sk + 8 f + j]
// [32 dt + m]. With the pkey order, S^T's result r of lane half f is key 16 (r / 8) + 8 f +
// r % 8 of the tile, which is the key of O^T's k slot 8 f + j of k step sk = r / 8, j = r % 8.
__device__ __forceinline__ uint32_t pf_pkey(uint32_t w) {
    return (w & ~12u) | ((w & 4u) << 1) | ((w & 8u) >> 1);
}
__device__ __forceinline__ uint64_t pf_kswz(uint32_t t, uint32_t d, uint32_t hd) {
    const uint32_t tile = t >> 5, m = pf_pkey(t & 31u);
    return ((static_cast<uint64_t>(tile) * (hd / 16u) + (d >> 4)) * 2u + ((d >> 3) & 1u)) * 256u + m * 8u + (d & 7u);
}
__device__ __forceinline__ uint64_t pf_vswz(uint32_t t, uint32_t d, uint32_t hd) {
    const uint32_t tile = t >> 5, w = t & 31u;
    return ((static_cast<uint64_t>(tile) * (hd / 32u) + (d >> 5)) * 2u + (w >> 4)) * 512u + ((w >> 3) & 1u) * 256u +
           (d & 31u) * 8u + (w & 7u);
}

// ---- QK-norm, RoPE, KV cache ------------------------------------------------------------

// Row t of qkv = [q (H heads x hd) | k (hd) | v (hd)]: QK-norm per head (src/gemma3.cpp:
// 1045-1104), NeoX RoPE at position t (:1371-1424), in place (q also as f16 hi/lo rows of
// qhi/qlo); then k and v go to the KV cache slot t % slots when position t is still in the
// window after the prompt (the serial loop's eviction leaves exactly those, :1590-1600); with
// kv16 (1 fp16, 2 bf16) the cache holds 16-bit entries and k and v are rounded to them first
// (the attention below then sees the cached values, as the serial loop does). The attention operands as f16 hi/lo: k and
// v in the pf_kswz / pf_vswz tile layouts. One
// workgroup per position t < Tp: those with t >= T write the zero padding keys and values
// (keys past the prompt are masked, and zero values keep the masked products zero).
// One wave per head (lane l: dims l + 64 e): the sum of squares is a wave reduction and the
// RoPE partners come through the wave's own LDS row, so the kernel has no barrier.
constexpr uint32_t kPfQkMaxWaves = 8;
__global__ void __launch_bounds__(kPfQkMaxWaves * 64) k_pf_qk(float* qkv, uint32_t T, uint32_t H, uint32_t hd,
                                                            const float* q_norm, const float* k_norm,
                                                            const float* cos_t, const float* sin_t, float eps,
                                                            float* kc, float* vc, uint32_t slots, _Float16* qhi,
                                                            _Float16* qlo, _Float16* khi, _Float16* klo, _Float16* vhi,
                                                            _Float16* vlo, uint32_t kv16, uint32_t p0, uint32_t qo) {
#pragma clang fp contract(off)
    __shared__ float xs[kPfQkMaxWaves][256];
    const uint32_t t = blockIdx.x;           // row of the segment; position p0 + t, key coordinate qo + t
    const uint32_t kt = qo + t;
    if (t >= T) {   // whole workgroup
        for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {
            const uint64_t ko = pf_kswz(kt, i, hd), vo = pf_vswz(kt, i, hd);
            khi[ko] = klo[ko] = vhi[vo] = vlo[vo] = static_cast<_Float16>(0.0f);
        }
        return;
    }
    const uint32_t pos = p0 + t;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t nqkv = (H + 2u) * hd, half = hd >> 1;
    float* row = qkv + static_cast<uint64_t>(t) * nqkv;
    float* xw = xs[wave];
    const bool keep = t + slots >= T;   // the last `slots` positions of the segment reach the ring
    const uint64_t slot = static_cast<uint64_t>(pos % slots) * hd;
    // Loads are issued at clamped, in-bounds indices and masked afterwards, so each group of
    // them is in flight together (no branch, hence no wait, between them). v first: it is only
    // stored, after the heads.
    const uint32_t vi = min(threadIdx.x, hd - 1u);
    const float vr = row[(H + 1u) * hd + vi];
    uint32_t ic[4], ei[4];
    bool live[4];
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        live[e] = lane + 64u * e < hd;
        ic[e] = min(lane + 64u * e, hd - 1u);
        ei[e] = ic[e] < half ? ic[e] : ic[e] - half;
    }
    float cs[4], sn[4];
#pragma unroll
    for (uint32_t e = 0; e < 4u; ++e) {
        cs[e] = cos_t[static_cast<uint64_t>(pos) * half + ei[e]];
        sn[e] = sin_t[static_cast<uint64_t>(pos) * half + ei[e]];
    }
    for (uint32_t hh = wave; hh <= H; hh += nw) {   // H query heads, then the key head
        const float* x = row + hh * hd;
        const float* w = hh < H ? q_norm : k_norm;
        float v[4], wv[4];
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            v[e] = x[ic[e]];
            wv[e] = w[ic[e]];
        }
        double sq = 0.0;
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            if (!live[e]) v[e] = 0.0f;
            sq += static_cast<double>(v[e]) * static_cast<double>(v[e]);
        }
        const float sc = pf_rms_scale(wave_red_sum_d(sq), hd, eps);
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e)
            if (live[e]) xw[ic[e]] = v[e] * (sc * wv[e]);   // values *= scale * weights (src/gemma3.cpp:1097-1102)
        // the partners are other lanes' values: a wave's LDS accesses complete in order
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            if (!live[e]) continue;
            const uint32_t i = ic[e];
            const float a = xw[ei[e]], b = xw[ei[e] + half];
            const float y2 = i < half ? a * cs[e] - b * sn[e] : b * cs[e] + a * sn[e];
            if (hh < H) {   // the query, [T][H * hd]
                const uint64_t o = static_cast<uint64_t>(t) * H * hd + hh * hd + i;
                pf_split(y2, qhi + o, qlo + o);
            } else {   // 16-bit KV: the key as the cache holds it, for the cache and the attention
                const float kk = kv16 ? kv16_float(kv16_bits(y2, kv16), kv16) : y2;
                const uint64_t o = pf_kswz(kt, i, hd);
                pf_split(kk, khi + o, klo + o);
                if (keep) {
                    if (kv16) reinterpret_cast<uint16_t*>(kc)[slot + i] = kv16_bits(kk, kv16);
                    else kc[slot + i] = kk;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();   // this head's reads of xw come before the next head's writes
    }
    for (uint32_t i = threadIdx.x; i < hd; i += blockDim.x) {   // v is not normed
        const float vv0 = i == vi ? vr : row[(H + 1u) * hd + i];
        const float vv = kv16 ? kv16_float(kv16_bits(vv0, kv16), kv16) : vv0;
        if (keep) {
            if (kv16) reinterpret_cast<uint16_t*>(vc)[slot + i] = kv16_bits(vv, kv16);
            else vc[slot + i] = vv;
        }
        const uint64_t o = pf_vswz(kt, i, hd);
        pf_split(vv, vhi + o, vlo + o);
    }
}

// A segment's history for the attention: key coordinates j < nh hold positions kb + j, read
// from the block's KV cache (ring slot (kb + j) % slots, fp32 or 16-bit entries as the cache
// holds them) and written in the pf_kswz / pf_vswz layouts as f16 hi/lo, as k_pf_qk writes a
// segment's own rows. One workgroup per key coordinate.
__global__ void __launch_bounds__(kPfThreads) k_pf_kv_hist(const float* kc, const float* vc, uint32_t slots, uint32_t kv16,
                                                          uint32_t kb, uint32_t nh, uint32_t hd, _Float16* khi,
                                                          _Float16* klo, _Float16* vhi, _Float16* vlo) {
    const uint32_t j = blockIdx.x;
    if (j >= nh) return;
    const uint64_t slot = static_cast<uint64_t>((kb + j) % slots) * hd;
    for (uint32_t i = threadIdx.x; i < hd; i += kPfThreads) {
        const float k = kv16 ? kv16_float(reinterpret_cast<const uint16_t*>(kc)[slot + i], kv16) : kc[slot + i];
        const float v = kv16 ? kv16_float(reinterpret_cast<const uint16_t*>(vc)[slot + i], kv16) : vc[slot + i];
        const uint64_t ko = pf_kswz(j, i, hd), vo = pf_vswz(j, i, hd);
        pf_split(k, khi + ko, klo + ko);
        pf_split(v, vhi + vo, vlo + vo);
    }
}

// ---- causal attention ----------------------------------------------------------------------

// One unit per (key chunk c, query tile i, head h): queries q0 = 32 i .. q0 + 31 of head h
// against the keys of chunk c (A.kc keys, a multiple of 32) of the tile's key range [ks, ke)
// in key coordinates (a segment's history first, its rows from A.qo: the tile's first query
// sits at qk0 = A.qo + q0; ke = min(A.qo + T, qk0 + 32); ks = 0, or with a local window the
// window's start for qk0, rounded down to 32). The four waves split the head dimension: wave w owns the k steps s = w mod 4 of
// S^T = K Q^T and the d tiles dt = w mod 4 of O^T. Per 32-key tile, with lane l on query
// q0 + l % 32: each wave's partial S^T (three f16 products of the hi/lo parts) goes through LDS
// and every wave sums the four in wave order (the same scores in every wave), masks (key <= qk,
// inside the window, key < ke) and scales them and runs the online softmax in base 2 (the
// scale times log2 e, v_exp_f32): running max m, e_j = 2^(v_j - m), each tile's sum of e_j in
// fp32 added to a running sum in double, its O^T tiles rescaled when m grows and O^T += V^T E^T
// (V^T and E^T as hi/lo). The next tile's operands load during the current one.
// A tile whose key range is one chunk is finished here (out = O / sum as f16 hi/lo into the
// queries' own columns, which only this unit reads); otherwise the chunk's partial goes to
// opart/mpart/lpart and k_pf_attn_merge combines them in the next launch. Same result as the
// masked softmax of src/gemma3.cpp:1602-1696 over the full row up to the rounding of the
// rescaling; a softmax sum that is not > 0 and finite flags the block.
// MFMA operand layouts (v_mfma_f32_32x32x16_f16): lane l gives A[m = l % 32][k = 8 (l / 32) + j]
// and B[k = 8 (l / 32) + j][n = l % 32], j < 8; result r of lane l is C[8 (r / 4) + 4 (l / 32) +
// r % 4][l % 32].
constexpr uint32_t kPfAttKC = 128;   // keys per attention chunk (a multiple of 32)
struct PfAttn {
    const _Float16* qhi;   // [T][H * hd] queries, normed and rotated (overwritten by the output)
    const _Float16* qlo;
    const _Float16* khi;   // keys in pf_kswz order, by key coordinate (32-key tiles)
    const _Float16* klo;
    const _Float16* vhi;   // values in pf_vswz order
    const _Float16* vlo;
    _Float16* ohi;         // [T][H * hd] output
    _Float16* olo;
    float* opart;          // [H][qtmax][maxc][32][hd] chunk partials, sum_j e_j v_j
    float* mpart;          // [H][qtmax][maxc][32] their maxima (base 2)
    double* lpart;         // [H][qtmax][maxc][32] their sums of e_j
    G3State* st;
    uint32_t T, H, window, qtmax, maxc, block, kc;
    uint32_t qt0;          // first query tile of the launch (blockIdx.y, merge: blockIdx.x, counts from it)
    uint32_t qo;           // key coordinate of query row 0 (keys before it: an earlier segment's history)
    float scale2;          // attention scale times log2(e): the scores in base 2
};

// Key range [ks, ke) of the query tile whose first row sits at key coordinate qk0, with keys
// below kend (the key coordinates of a segment's history come first, then its own rows).
__device__ __forceinline__ void pf_att_range(uint32_t qk0, uint32_t kend, uint32_t window, uint32_t& ks, uint32_t& ke) {
    ke = min(kend, qk0 + 32u);
    ks = window != 0u && qk0 + 1u > window ? (qk0 + 1u - window) & ~31u : 0u;
}

template <uint32_t HD>
__global__ void __launch_bounds__(256) k_pf_attn(PfAttn A) {
#pragma clang fp contract(off)
    constexpr uint32_t KS = HD / 16u;               // k steps of S^T
    constexpr uint32_t DT = HD / 32u;               // d tiles of O^T
    constexpr uint32_t KW = (KS + 3u) / 4u;         // k steps per wave (at most)
    constexpr uint32_t DW = (DT + 3u) / 4u;         // d tiles per wave (at most)
    __shared__ __align__(16) float s_s[2][4][16 * 64];   // partial S^T per wave, double-buffered
    // Workgroup b of the launch runs on XCD b % 8: each XCD takes a contiguous eighth of the
    // (query tile, chunk, head) units, heads innermost, so the units that read one chunk's keys
    // and values (the heads share them) run together on one XCD and its L2 (-1.6% on an
    // 8192-token prefill, unchanged at 512).
    uint32_t c, i, h;
    {
        const uint32_t nx = gridDim.x, ny = gridDim.y, nz = gridDim.z, N = nx * ny * nz;
        uint32_t b = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
        if ((N & 7u) == 0u) b = (b & 7u) * (N >> 3) + (b >> 3);
        h = b % nz;
        const uint32_t r = b / nz;
        c = r % nx;
        i = A.qt0 + r / nx;
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, l32 = lane & 31u, hf = lane >> 5;
    const uint32_t T = A.T, q0 = 32u * i, qw = A.H * HD;
    const uint32_t qk0 = A.qo + q0;   // the tile's first query in key coordinates
    uint32_t ks, ke;
    pf_att_range(qk0, A.qo + T, A.window, ks, ke);
    const uint32_t nch = (ke - ks + A.kc - 1u) / A.kc;
    if (c >= nch) return;   // whole workgroup
    const uint32_t k0 = ks + c * A.kc, k1 = min(ke, k0 + A.kc);
    const uint32_t q = q0 + l32, qk = qk0 + l32;   // this lane's query: row, key coordinate
    // this wave's k steps of the queries (B operand of S^T), rows past T clamped (never written)
    v4u qb[KW][2];
    {
        const uint64_t qo = static_cast<uint64_t>(min(q, T - 1u)) * qw + h * HD + 8u * hf;
#pragma unroll
        for (uint32_t j = 0; j < KW; ++j) {
            const uint32_t k = min(wave + 4u * j, KS - 1u);
            qb[j][0] = *reinterpret_cast<const v4u*>(A.qhi + qo + 16u * k);
            qb[j][1] = *reinterpret_cast<const v4u*>(A.qlo + qo + 16u * k);
        }
    }
    // the operands of one 32-key tile for this wave
    struct Ops {
        v4u k[KW][2];       // [k step][hi, lo]
        v4u v[DW][2][2];    // [d tile][k step][hi, lo]
    };
    auto load = [&](uint32_t kt, Ops& R) {
        const uint64_t tile = kt >> 5;
#pragma unroll
        for (uint32_t j = 0; j < KW; ++j) {
            const uint32_t k = min(wave + 4u * j, KS - 1u);
            const uint64_t o = (tile * KS + k) * 512u + 8u * lane;
            R.k[j][0] = *reinterpret_cast<const v4u*>(A.khi + o);
            R.k[j][1] = *reinterpret_cast<const v4u*>(A.klo + o);
        }
#pragma unroll
        for (uint32_t j = 0; j < DW; ++j) {
            const uint32_t dt = min(wave + 4u * j, DT - 1u);
#pragma unroll
            for (uint32_t sk = 0; sk < 2u; ++sk) {
                const uint64_t o = ((tile * DT + dt) * 2u + sk) * 512u + 8u * lane;
                R.v[j][sk][0] = *reinterpret_cast<const v4u*>(A.vhi + o);
                R.v[j][sk][1] = *reinterpret_cast<const v4u*>(A.vlo + o);
            }
        }
    };
    float m = -INFINITY;   // running maximum of the scaled scores of query q
    double lsum = 0.0;     // this lane's share of sum_j e_j
    float16v o[DW];        // O^T tiles of this wave: d = 32 dt + 8 (r / 4) + 4 hf + r % 4, query q
#pragma unroll
    for (uint32_t j = 0; j < DW; ++j) o[j] = float16v{};
    // one 32-key tile: partial S^T, exchange, online softmax, O^T update (operands in R)
    uint32_t buf = 0;
    auto step = [&](uint32_t kt, const Ops& R) {
        float16v sp = {};
#pragma unroll
        for (uint32_t j = 0; j < KW; ++j) {
            if (wave + 4u * j >= KS) continue;
            const half8 ah = __builtin_bit_cast(half8, R.k[j][0]), al = __builtin_bit_cast(half8, R.k[j][1]);
            const half8 bh = __builtin_bit_cast(half8, qb[j][0]), bl = __builtin_bit_cast(half8, qb[j][1]);
            sp = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, sp, 0, 0, 0);
            sp = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, sp, 0, 0, 0);
            sp = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, sp, 0, 0, 0);
        }
        // the four partials through LDS (buffer buf was last read two tiles ago, before the
        // barrier of the previous tile)
#pragma unroll
        for (uint32_t rq = 0; rq < 4u; ++rq)
            *reinterpret_cast<f4*>(&s_s[buf][wave][(rq * 64u + lane) * 4u]) =
                f4{sp[4 * rq], sp[4 * rq + 1], sp[4 * rq + 2], sp[4 * rq + 3]};
        __syncthreads();
        float v[16];
#pragma unroll
        for (uint32_t rq = 0; rq < 4u; ++rq) {
            f4 t = *reinterpret_cast<const f4*>(&s_s[buf][0][(rq * 64u + lane) * 4u]);
#pragma unroll
            for (uint32_t w = 1; w < 4u; ++w) {
                const f4 u = *reinterpret_cast<const f4*>(&s_s[buf][w][(rq * 64u + lane) * 4u]);
#pragma unroll
                for (int e = 0; e < 4; ++e) t[e] += u[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * rq + e] = t[e];
        }
        buf ^= 1u;
        // scores in base 2 (scale * log2 e folded in): e_j = 2^(v_j - m) = exp(scale s_j - m ln 2)
        float tmax = -INFINITY;
        if (kt + 31u < k1 && kt + 31u <= qk0 && (A.window == 0u || kt + A.window > qk0 + 31u)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {   // every key of the tile visible to every query
                v[r] *= A.scale2;
                tmax = fmaxf(tmax, v[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t key = kt + 16u * (r / 8) + 8u * hf + (r % 8);
                const bool ok = key < k1 && key <= qk && (A.window == 0u || key + A.window > qk);
                v[r] = ok ? v[r] * A.scale2 : -INFINITY;
                tmax = fmaxf(tmax, v[r]);
            }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float mn = fmaxf(m, tmax);
        const float base = mn == -INFINITY ? 0.0f : mn;   // nothing visible yet: every e_j is 0
        const float alpha = __builtin_amdgcn_exp2f(m - base);
        float e[16];
        float es = 0.0f;   // the tile's share in fp32, then into the double sum
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            e[r] = __builtin_amdgcn_exp2f(v[r] - base);
            es += e[r];
        }
        lsum = lsum * static_cast<double>(alpha) + static_cast<double>(es);
        m = mn;
        half8 eh[2], el[2];
#pragma unroll
        for (int sk = 0; sk < 2; ++sk)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = e[8 * sk + j];
                eh[sk][j] = static_cast<_Float16>(x);
                el[sk][j] = static_cast<_Float16>(x - static_cast<float>(eh[sk][j]));
            }
#pragma unroll
        for (uint32_t j = 0; j < DW; ++j) {
            if (wave + 4u * j >= DT) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
#pragma unroll
            for (uint32_t sk = 0; sk < 2u; ++sk) {
                const half8 avh = __builtin_bit_cast(half8, R.v[j][sk][0]);
                const half8 avl = __builtin_bit_cast(half8, R.v[j][sk][1]);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(avh, eh[sk], o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(avl, eh[sk], o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(avh, el[sk], o[j], 0, 0, 0);
            }
        }
    };
    // two operand sets in turn, the next tile's loads in flight during the current tile
    Ops ra, rb;
    load(k0, ra);
    for (uint32_t kt = k0; kt < k1; kt += 64u) {
        if (kt + 32u < k1) load(kt + 32u, rb);
        step(kt, ra);
        if (kt + 32u >= k1) break;
        if (kt + 64u < k1) load(kt + 64u, ra);
        step(kt + 32u, rb);
    }
    lsum += __shfl_xor(lsum, 32);   // both lane halves now hold query q's sum
    const uint64_t unit = (static_cast<uint64_t>(h) * A.qtmax + i) * A.maxc + c;
    if (nch == 1u) {   // the whole key range: normalise and write the output rows
        if (q >= T) return;
        const double den = lsum;
        if (wave == 0u && hf == 0u && (!(den > 0.0) || !__builtin_isfinite(den)))   // :1666-1670
            atomicMin(&A.st->nonfinite, g3_code_softmax(A.block));
        const float inv = static_cast<float>(1.0 / den);
        const uint64_t oo = static_cast<uint64_t>(q) * qw + h * HD;
#pragma unroll
        for (uint32_t j = 0; j < DW; ++j) {
            if (wave + 4u * j >= DT) continue;
#pragma unroll
            for (uint32_t rq = 0; rq < 4u; ++rq) {
                const uint32_t d = 32u * (wave + 4u * j) + 8u * rq + 4u * hf;
                pf_split4(f4{o[j][4 * rq] * inv, o[j][4 * rq + 1] * inv, o[j][4 * rq + 2] * inv, o[j][4 * rq + 3] * inv},
                          A.ohi + oo + d, A.olo + oo + d);
            }
        }
        return;
    }
    float* op = A.opart + unit * 32u * HD + static_cast<uint64_t>(l32) * HD;
#pragma unroll
    for (uint32_t j = 0; j < DW; ++j) {
        if (wave + 4u * j >= DT) continue;
#pragma unroll
        for (uint32_t rq = 0; rq < 4u; ++rq)
            *reinterpret_cast<f4*>(op + 32u * (wave + 4u * j) + 8u * rq + 4u * hf) =
                f4{o[j][4 * rq], o[j][4 * rq + 1], o[j][4 * rq + 2], o[j][4 * rq + 3]};
    }
    if (wave == 0u && hf == 0u) {
        A.mpart[unit * 32u + l32] = m;
        A.lpart[unit * 32u + l32] = lsum;
    }
}

// Column groups of a merge workgroup's head: 4, 2 or 1 (whole float4 runs per thread).
template <uint32_t HD>
constexpr uint32_t pf_merge_groups() {
    return (HD / 32u) % 4u == 0u ? 4u : ((HD / 32u) % 2u == 0u ? 2u : 1u);
}

// Merge of the chunk partials of the query tiles k_pf_attn split (one workgroup per (tile, head,
// column group); tiles of one chunk were finished by k_pf_attn): thread t on row r = t / 8 and
// the eighth t % 8 of the group's columns; in chunk order, with M the running maximum of the
// chunk maxima m_c, den = sum_c exp(m_c - M) sum_c (double), out = sum_c exp(m_c - M) O_c / den
// as f16 hi/lo into the queries' columns.
template <uint32_t HD>
__global__ void __launch_bounds__(256) k_pf_attn_merge(PfAttn A) {
#pragma clang fp contract(off)
    constexpr uint32_t CG = pf_merge_groups<HD>();
    constexpr uint32_t NF = HD / 32u / CG;   // float4 per thread
    const uint32_t i = A.qt0 + blockIdx.x, h = blockIdx.y, T = A.T, q0 = 32u * i;
    uint32_t ks, ke;
    pf_att_range(A.qo + q0, A.qo + T, A.window, ks, ke);
    const uint32_t nch = (ke - ks + A.kc - 1u) / A.kc;
    const uint32_t r = threadIdx.x >> 3, g = blockIdx.z * 8u + (threadIdx.x & 7u);
    if (nch == 1u || q0 + r >= T) return;
    const uint64_t unit0 = (static_cast<uint64_t>(h) * A.qtmax + i) * A.maxc;
    // chunks in groups of kG, every load of a group issued together (indices clamped to the last
    // chunk; the clamped duplicates are not used): one round of loads for up to kG chunks
    constexpr uint32_t kG = 4;
    double den = 0.0;
    f4 acc[NF];
#pragma unroll
    for (uint32_t k = 0; k < NF; ++k) acc[k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float M = -INFINITY;
    for (uint32_t c0 = 0; c0 < nch; c0 += kG) {
        float mv[kG];
        double lv[kG];
        f4 x[kG][NF];
#pragma unroll
        for (uint32_t j = 0; j < kG; ++j) {
            const uint64_t u = unit0 + min(c0 + j, nch - 1u);
            mv[j] = A.mpart[u * 32u + r];
            lv[j] = A.lpart[u * 32u + r];
            const float* src = A.opart + (u * 32u + r) * HD + g * (4u * NF);
#pragma unroll
            for (uint32_t k = 0; k < NF; ++k) x[j][k] = *reinterpret_cast<const f4*>(src + 4u * k);
        }
        __builtin_amdgcn_sched_barrier(0);   // the group's loads stay ahead of their first use
        // running merge: the group's maximum rescales what is accumulated so far
        float Mg = M;
#pragma unroll
        for (uint32_t j = 0; j < kG; ++j)
            if (c0 + j < nch) Mg = fmaxf(Mg, mv[j]);
        const float fo = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mg);
        den *= static_cast<double>(fo);
#pragma unroll
        for (uint32_t k = 0; k < NF; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[k][e] *= fo;
        M = Mg;
#pragma unroll
        for (uint32_t j = 0; j < kG; ++j) {
            if (c0 + j >= nch) break;
            const float f = __builtin_amdgcn_exp2f(mv[j] - M);
            den += lv[j] * static_cast<double>(f);
#pragma unroll
            for (uint32_t k = 0; k < NF; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[k][e] += f * x[j][k][e];
        }
    }
    if (g == 0u && (!(den > 0.0) || !__builtin_isfinite(den)))   // :1666-1670
        atomicMin(&A.st->nonfinite, g3_code_softmax(A.block));
    const float inv = static_cast<float>(1.0 / den);
    const uint64_t oo = static_cast<uint64_t>(q0 + r) * (A.H * HD) + h * HD + g * (4u * NF);
#pragma unroll
    for (uint32_t k = 0; k < NF; ++k)
        pf_split4(f4{acc[k][0] * inv, acc[k][1] * inv, acc[k][2] * inv, acc[k][3] * inv}, A.ohi + oo + 4u * k,
                  A.olo + oo + 4u * k);
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

// The Q8_0 GEMM of k_pf_gemm_q8 on expanded weights (G.wh, G.ws): a K step of SB Q8_0 blocks
// (32 SB wide) stages the f16 rows of the tile's W blocks with plain 16-byte copies (no int8
// conversion on the K loop's critical path) and the SB block scales per row. Same tiles,
// splits and epilogues as k_pf_gemm_q8, with KW times the waves: wave group kw (of 2 NWN
// waves) computes the step's Q8_0 blocks kw, kw + KW, ... for every tile, so a SIMD runs KW
// waves whose LDS reads, MFMA chains and scale-and-add work overlap; before the epilogue the
// partial tiles of groups 1..KW-1 are added, in group order, to those of group 0 through LDS.
// The register ring holds 8 / SB steps in flight (the same bytes for every SB).
template <int WN, int NWN, int SB, int KW>
__global__ void __launch_bounds__(128 * NWN * KW) k_pf_gemm_h(PfGemm G) {
    constexpr uint32_t NT = 128u * NWN * KW;
    constexpr uint32_t BN = 32u * WN * NWN;
    constexpr uint32_t UR = 4u * SB;                   // 16-byte units per staged row
    constexpr uint32_t PITCH = 16u * UR + 16u;         // LDS row pitch in bytes (padded)
    constexpr uint32_t AU = 2u * kQgBM * UR / NT;      // A units per thread (hi units, then lo)
    constexpr uint32_t WU = BN * UR / NT;              // W units per thread
    constexpr uint32_t AHEAD = 8u / SB;                // steps in flight ahead of the one computed
    constexpr uint32_t CHUNK = 24u / SB;               // steps per straight-line chunk
    static_assert((SB == 2 || SB == 4) && (KW == 2 || KW == 4) && SB % KW == 0, "blocks per step, wave groups");
    static_assert(AU >= 1u && 2u * kQgBM * UR % NT == 0u, "whole A units per thread");
    static_assert(WU >= 1u && BN * UR % NT == 0u, "whole W units per thread");
    static_assert(BN <= NT, "one row of scales per thread");
    __shared__ __align__(16) unsigned char s_a[2][2][kQgBM * PITCH];
    __shared__ __align__(16) unsigned char s_w[2][BN * PITCH];
    __shared__ float s_sc[2][BN][SB];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kh = lane >> 5, l32 = lane & 31u;
    const uint32_t m0 = blockIdx.y * kQgBM, n0 = blockIdx.x * BN;
    const uint32_t nkb = G.K >> 5;
    const uint32_t S = gridDim.z, z = blockIdx.z;
    const uint32_t kb_lo = nkb * z / S, kb_hi = nkb * (z + 1u) / S;
    const uint32_t nsteps = (kb_hi - kb_lo + SB - 1u) / SB;
    typedef const __attribute__((address_space(1))) v4u* gv4;
    struct Stage {
        v4u a[AU];   // unit u = AU tid + j: array u / (UR kQgBM), row (u % (UR kQgBM)) / UR, column u % UR
        v4u w[WU];
        float sc[SB];
    };
    // Every load is issued at a clamped, in-bounds address (dead data is zeroed when stored).
    auto load = [&](uint32_t step, Stage& R) {
        const uint32_t kb = kb_lo + SB * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, ui = u % (UR * kQgBM), r = ui / UR, c = ui % UR;
            const uint32_t k = 32u * kb + 8u * c;
            const uint32_t rr = min(m0 + r, G.M - 1u), kk = min(k, 32u * kb_hi - 8u);
            const uint64_t o = (static_cast<uint64_t>(rr) * G.lda + kk) * 2u;
            R.a[j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(u < UR * kQgBM ? G.ahi : G.alo) + o);
        }
#pragma unroll
        for (uint32_t j = 0; j < WU; ++j) {
            const uint32_t u = WU * tid + j, r = u / UR, c = u % UR;
            const uint32_t rr = min(n0 + r, G.N - 1u), kk = min(32u * kb + 8u * c, 32u * kb_hi - 8u);
            R.w[j] = *reinterpret_cast<gv4>(reinterpret_cast<uintptr_t>(G.wh) + (static_cast<uint64_t>(rr) * G.K + kk) * 2u);
        }
        {   // the step's block scales of row tid (clamped to the split's last block)
            typedef const __attribute__((address_space(1))) float* gf;
            const uint32_t rr = min(n0 + (tid < BN ? tid : 0u), G.N - 1u);
            const gf row = reinterpret_cast<gf>(reinterpret_cast<uintptr_t>(G.ws + static_cast<uint64_t>(rr) * nkb));
#pragma unroll
            for (uint32_t q = 0; q < SB; ++q) R.sc[q] = row[min(kb + q, kb_hi - 1u)];
        }
    };
    auto store = [&](const Stage& R, uint32_t st, uint32_t step) {
        const uint32_t kb = kb_lo + SB * step;
#pragma unroll
        for (uint32_t j = 0; j < AU; ++j) {
            const uint32_t u = AU * tid + j, ui = u % (UR * kQgBM), r = ui / UR, c = ui % UR;
            const bool live = m0 + r < G.M && 32u * kb + 8u * c < 32u * kb_hi;
            *reinterpret_cast<v4u*>(&s_a[st][u / (UR * kQgBM)][r * PITCH + c * 16u]) = live ? R.a[j] : v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (uint32_t j = 0; j < WU; ++j) {
            const uint32_t u = WU * tid + j, r = u / UR, c = u % UR;
            const bool live = n0 + r < G.N && 32u * kb + 8u * c < 32u * kb_hi;
            *reinterpret_cast<v4u*>(&s_w[st][r * PITCH + c * 16u]) = live ? R.w[j] : v4u{0u, 0u, 0u, 0u};
        }
        if (tid < BN) {
            const bool rl = n0 + tid < G.N;
#pragma unroll
            for (uint32_t q = 0; q < SB; ++q) s_sc[st][tid][q] = rl && kb + q < kb_hi ? R.sc[q] : 0.0f;
        }
    };
    const uint32_t kw = wave / (2u * NWN), wv = wave % (2u * NWN);   // block group of the step, tile
    const uint32_t wm = wv / NWN, wn = wv % NWN;
    float16v acc[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[j] = float16v{};
    auto compute = [&](uint32_t st) {
        const unsigned char* pa_hi = &s_a[st][0][(32u * wm + l32) * PITCH + 16u * kh];
        const unsigned char* pa_lo = &s_a[st][1][(32u * wm + l32) * PITCH + 16u * kh];
#pragma unroll
        for (uint32_t bq = 0; bq < SB / KW; ++bq) {
            const uint32_t b = kw + KW * bq;
            half8 ah[2], al[2];
#pragma unroll
            for (uint32_t ks = 0; ks < 2; ++ks) {
                ah[ks] = *reinterpret_cast<const half8*>(pa_hi + 64u * b + 32u * ks);
                al[ks] = *reinterpret_cast<const half8*>(pa_lo + 64u * b + 32u * ks);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const uint32_t nl = 32u * (WN * wn + j) + l32;
                const unsigned char* pw = &s_w[st][nl * PITCH + 64u * b + 16u * kh];
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
    static_assert(AHEAD <= CHUNK, "ring inside a chunk");
    for (uint32_t i = 0; i < nsteps; i += CHUNK) {
        Stage R[AHEAD];
        auto clamp = [&](uint32_t j) { return min(i + j, nsteps - 1u); };
#pragma unroll
        for (uint32_t u = 0; u < AHEAD; ++u) load(clamp(u), R[u]);
#pragma unroll
        for (uint32_t u = 0; u < CHUNK; ++u) {
            const uint32_t j = i + u;
            if (j < nsteps) {
                store(R[u % AHEAD], j & 1u, j);
                __syncthreads();
            }
            if (u + AHEAD < CHUNK) load(clamp(u + AHEAD), R[u % AHEAD]);
            if (j < nsteps) compute(j & 1u);
        }
    }
    {   // the other groups' partials into group 0 (s_a: (KW - 1) 2 NWN WN 16 x 64 floats fit)
        constexpr uint32_t RS = 2u * NWN * WN * 16u * 64u;   // floats per group
        static_assert((KW - 1u) * RS * 4u <= sizeof(s_a), "reduction area");
        __syncthreads();   // every wave is done reading the LDS stages
        float* red = reinterpret_cast<float*>(&s_a[0][0][0]);
        if (kw != 0u) {
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[(kw - 1u) * RS + ((wv * WN + j) * 16u + r) * 64u + lane] = acc[j][r];
        }
        __syncthreads();
        if (kw == 0u) {
#pragma unroll
            for (uint32_t q = 1; q < KW; ++q)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[j][r] += red[(q - 1u) * RS + ((wv * WN + j) * 16u + r) * 64u + lane];
        }
    }   // (the GLU epilogue's exchange reuses s_a after a barrier of its own)
    pf_gemm_epilogue<WN, NWN>(G, acc, z, m0, n0, wm, wn, kh, l32, lane, reinterpret_cast<float*>(&s_a[0][0][0]),
                              kw == 0u);
}

// ---- host side --------------------------------------------------------------------------

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

constexpr int kPfStepBlocks = 4;   // Q8_0 blocks per K step of the 64 x 64 tiles
constexpr int kPfWaveGroups = 4;   // their wave groups (the 64 x 128 tiles: 2 blocks, 2 groups)

template <int WN, int NWN, int SB, int KW>
static int pf_launch_h(const PfGemm& G, uint32_t splits, hipStream_t s) {
    constexpr uint32_t BN = 32u * WN * NWN;
    const dim3 grid((G.N + BN - 1u) / BN, (G.M + kQgBM - 1u) / kQgBM, splits);
    PfGemm arg = G;
    void* args[] = {&arg};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_gemm_h<WN, NWN, SB, KW>), grid,
                                  dim3(128u * NWN * KW), args, 0, s));
    return VRT_OK;
}

// The Q8_0 GEMM's launch: on the expanded weights when `ex` holds them, else on the arena.
static int pf_launch_w(PfGemm& G, const PfMatrix* ex, uint32_t splits, hipStream_t s) {
    const uint32_t mt = (G.M + kQgBM - 1u) / kQgBM;
    const bool wide = G.N % 128u == 0u && (G.N / 128u) * mt >= 128u;
    if (ex && ex->h) {
        G.wh = static_cast<const _Float16*>(ex->h);
        G.ws = ex->s;
        // one row tile (the batched decode's rows): 32-column tiles, twice the workgroups (1.256 ->
        // 1.211 ms per step of 64 sequences); the GLU epilogue pairs gate and up inside 64 columns
        if (!G.glu && G.M <= kQgBM) return pf_launch_h<1, 1, kPfStepBlocks, kPfWaveGroups>(G, splits, s);
        return wide ? pf_launch_h<1, 4, 2, 2>(G, splits, s) : pf_launch_h<1, 2, kPfStepBlocks, kPfWaveGroups>(G, splits, s);
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
    // any N: rows past N load clamped, in-bounds rows, are zeroed in LDS and never stored
    if (K % 32u != 0u || G.N == 0u) return set_error(VRT_ERR_INVALID, "prefill GEMM shape not supported");
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
uint32_t pf_splits(uint32_t M, uint32_t N) {
    const uint32_t tiles = ((M + kQgBM - 1u) / kQgBM) * ((N + 63u) / 64u);
    return std::min(kPfMaxSplits, std::max(1u, 256u / std::max(1u, tiles)));
}

// k_pf_norm_w over `rows` rows of n <= 2048 elements (elements per lane: the smallest of 4, 8,
// 12, 16, 24, 32 that covers n).
int pf_norm(float* h, const float* f, uint32_t nsplit, uint64_t sstride, const float* w_post, const float* w_next,
            uint32_t n, float eps, _Float16* xhi, _Float16* xlo, G3State* st, uint32_t block, uint32_t rows, hipStream_t s,
            bool into) {
    uint32_t in = into ? 1u : 0u;
    void* args[] = {&h, &f, &nsplit, &sstride, &w_post, &w_next, &n, &eps, &xhi, &xlo, &st, &block, &rows, &in};
    const uint32_t ne = (n + 63u) / 64u;
    const void* fn = ne <= 4u    ? reinterpret_cast<const void*>(&k_pf_norm_w<4>)
                     : ne <= 8u  ? reinterpret_cast<const void*>(&k_pf_norm_w<8>)
                     : ne <= 12u ? reinterpret_cast<const void*>(&k_pf_norm_w<12>)
                     : ne <= 16u ? reinterpret_cast<const void*>(&k_pf_norm_w<16>)
                     : ne <= 24u ? reinterpret_cast<const void*>(&k_pf_norm_w<24>)
                     : ne <= 32u ? reinterpret_cast<const void*>(&k_pf_norm_w<32>)
                                 : nullptr;
    if (!fn || nsplit > kPfMaxSplits) return set_error(VRT_ERR_INVALID, "prefill norm shape not supported");
    const uint32_t per = kPfThreads / 64u;
    VRT_HIP_CHECK(hipLaunchKernel(fn, dim3((rows + per - 1u) / per), dim3(kPfThreads), args, 0, s));
    return VRT_OK;
}

// Block l's projection `which` over M rows (the building blocks of the batched decode): C =
// A x W^T with K split over `splits` workgroups (clamped to the K blocks; the count used goes to
// *used), partial z at c + z * M * N.
int pf_project(vrt_g3* g, uint32_t l, uint32_t which, const _Float16* ahi, const _Float16* alo, uint32_t M, float* c,
               uint32_t splits, uint32_t* used, hipStream_t s) {
    const LayerParams& Ly = g->layers[l];
    const PfLayerW* lw = g->pf.lw.empty() ? nullptr : &g->pf.lw[l];
    const uint32_t d = g->cfg.embedding_length, hd = g->cfg.head_dim, qw = g->cfg.head_count * hd;
    const uint32_t F = g->cfg.feed_forward_length;
    const uint32_t K = which == kProjQkv ? d : (which == kProjO ? qw : F);
    *used = std::max(1u, std::min(splits, (K / 32u) / 2u));
    switch (which) {
    case kProjQkv: return pf_gemm(g, ahi, alo, M, d, {{Ly.wq, qw}, {Ly.wk, hd}, {Ly.wv, hd}}, lw ? &lw->qkv : nullptr, c, splits, s);
    case kProjO: return pf_gemm(g, ahi, alo, M, qw, {{Ly.wo, d}}, lw ? &lw->o : nullptr, c, splits, s);
    case kProjDown: return pf_gemm(g, ahi, alo, M, F, {{Ly.wd, d}}, lw ? &lw->down : nullptr, c, splits, s);
    default: return set_error(VRT_ERR_INVALID, "unknown projection %u", which);
    }
}

// Block l's gelu_tanh(gate) * up over M rows, as f16 hi/lo [M][F].
int pf_ffn_glu(vrt_g3* g, uint32_t l, const _Float16* ahi, const _Float16* alo, uint32_t M, _Float16* ghi,
               _Float16* glo, hipStream_t s) {
    const LayerParams& Ly = g->layers[l];
    const PfLayerW* lw = g->pf.lw.empty() ? nullptr : &g->pf.lw[l];
    return pf_gemm_glu(g, ahi, alo, M, g->cfg.embedding_length, Ly.wg, Ly.wu, g->cfg.feed_forward_length,
                       lw ? &lw->gu : nullptr, ghi, glo, s);
}

// Embedding rows of `rows` tokens (device array) into h [rows][d].
int pf_embed_rows(vrt_g3* g, const uint32_t* tokens, uint32_t rows, float* h, hipStream_t s) {
    const uint8_t* te = g->P.tok_embd;
    uint32_t d = g->cfg.embedding_length;
    float es = g->P.emb_scale;
    void* args[] = {&te, &tokens, &d, &es, &h};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_embed), dim3(rows), dim3(kPfThreads), args, 0, s));
    return VRT_OK;
}

// Logits of M rows against the tied Q8_0 embedding table: logits [M][vocab] = x W_embd^T, x as
// f16 hi/lo [M][d] (MFMA on the Q8_0 rows of the arena, one K split).
int pf_lm_logits(vrt_g3* g, const _Float16* xhi, const _Float16* xlo, uint32_t M, float* logits, hipStream_t s) {
    return pf_gemm(g, xhi, xlo, M, g->cfg.embedding_length, {{g->P.tok_embd, g->cfg.vocab_size}}, nullptr, logits, 1u, s);
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
    // keys and values of a segment's history and rows (f16 each): prompts longer than max_t run
    // in segments whose keys reach back to position 0 in a global block
    p.tkv = static_cast<uint32_t>(std::max<uint64_t>(tp, pf_pad(g->cfg.context_length)));
    void** kv[] = {&p.khi, &p.klo, &p.vhi, &p.vlo};
    for (void** b : kv)
        if (int rc = take(static_cast<size_t>(hd) * p.tkv * 2u, b)) return rc;
    p.qtmax = (max_t + 31u) / 32u;
    p.maxc = (max_t + 31u + kPfAttKC - 1u) / kPfAttKC;
    const size_t units = static_cast<size_t>(H) * p.qtmax * p.maxc;
    if (int rc = take(units * 32u * hd * 4u, &q)) return rc;
    p.opart = static_cast<float*>(q);
    if (int rc = take(units * 32u * 4u, &q)) return rc;
    p.mpart = static_cast<float*>(q);
    if (int rc = take(units * 32u * 8u, &q)) return rc;
    p.lpart = static_cast<double*>(q);
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

template <uint32_t HD>
static int pf_attn_launch(const PfAttn& A, dim3 grid, hipStream_t s) {
    PfAttn arg = A;
    void* args[] = {&arg};
    VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_attn<HD>), grid, dim3(256), args, 0, s));
    if (grid.x > 1u)   // some tile has several chunks
        VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_attn_merge<HD>),
                                      dim3(grid.y, grid.z, pf_merge_groups<HD>()), dim3(256), args, 0, s));
    return VRT_OK;
}

// Causal local/global attention of one block (k_pf_attn) over the queries in qhi/qlo [T][H hd],
// written back in place as the attention output, for the query tiles from qt0 on.
static int pf_attention(vrt_g3* g, const LayerParams& Ly, uint32_t T, uint32_t qt0, _Float16* qhi, _Float16* qlo,
                        hipStream_t s, uint32_t qo = 0) {
    const PfState& p = g->pf;
    const uint32_t H = g->cfg.head_count, hd = g->cfg.head_dim;
    PfAttn A{};
    A.qhi = A.ohi = qhi;
    A.qlo = A.olo = qlo;
    A.khi = static_cast<const _Float16*>(p.khi);
    A.klo = static_cast<const _Float16*>(p.klo);
    A.vhi = static_cast<const _Float16*>(p.vhi);
    A.vlo = static_cast<const _Float16*>(p.vlo);
    A.opart = p.opart;
    A.mpart = p.mpart;
    A.lpart = p.lpart;
    A.st = g->P.st;
    A.T = T;
    A.H = H;
    A.window = Ly.slots >= g->cfg.context_length ? 0u : Ly.slots;
    A.qtmax = p.qtmax;
    A.maxc = p.maxc;
    A.block = Ly.index;
    A.scale2 = g->P.attn_scale * 1.4426950408889634f;
    const uint32_t qt = (T + 31u) / 32u;
    A.qt0 = qt0;
    A.qo = qo;
    // the longest key range of a query tile (the same ranges as pf_att_range), then a chunk size
    // that keeps it within maxc chunks (a segment's history can reach back to position 0)
    uint32_t span = 32;
    for (uint32_t i = qt0; i < qt; ++i) {
        const uint32_t qk0 = qo + 32u * i, ke = std::min(qo + T, qk0 + 32u);
        const uint32_t ks = A.window != 0u && qk0 + 1u > A.window ? (qk0 + 1u - A.window) & ~31u : 0u;
        span = std::max(span, ke - ks);
    }
    A.kc = std::max(kPfAttKC, (span + 32u * p.maxc - 1u) / (32u * p.maxc) * 32u);
    const uint32_t nch = (span + A.kc - 1u) / A.kc;
    if (qt > p.qtmax || nch > p.maxc || qt0 >= qt || pf_pad(qo + T) > p.tkv)
        return set_error(VRT_ERR_STATE, "prefill attention workspace too small");
    const dim3 grid(nch, qt - qt0, H);
    switch (hd) {
    case 32: return pf_attn_launch<32>(A, grid, s);
    case 64: return pf_attn_launch<64>(A, grid, s);
    case 96: return pf_attn_launch<96>(A, grid, s);
    case 128: return pf_attn_launch<128>(A, grid, s);
    case 160: return pf_attn_launch<160>(A, grid, s);
    case 192: return pf_attn_launch<192>(A, grid, s);
    case 224: return pf_attn_launch<224>(A, grid, s);
    case 256: return pf_attn_launch<256>(A, grid, s);
    default: return set_error(VRT_ERR_INVALID, "prefill head_dim not supported");
    }
}

// Prompt positions p0..p0+T-1 on the context's stream (positions before p0 are already in the
// KV cache). With `final`, the last one runs the LM head + argmax (results[p0+T-1], logits when
// want_logits); otherwise the segment ends after the last block's keys and values. The caller
// has reset the step state before the first segment.
int pf_run(vrt_g3* g, uint32_t T, uint32_t p0, bool final) {
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
    if (T == 0u || T > p.max_t || static_cast<uint64_t>(p0) + T > g->cfg.context_length)
        return set_error(VRT_ERR_STATE, "prefill segment outside the workspace or the context");
    auto launch = [&](const void* fn, dim3 grid, void** args) -> int {
        VRT_HIP_CHECK(hipLaunchKernel(fn, grid, dim3(kPfThreads), args, 0, s));
        return VRT_OK;
    };
    {
        const uint8_t* te = P.tok_embd;
        const uint32_t* tok = P.tokens + p0;
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
            if (int rc = pf_norm(h, f, s_down, xs, wpost, Ly.attn_norm, d, eps, ahi, alo, st, l ? l - 1u : 0u, T, s, true))
                return rc;
        }
        if (int rc = pf_gemm(g, ahi, alo, T, d, {{Ly.wq, qw}, {Ly.wk, hd}, {Ly.wv, hd}}, lw ? &lw[l].qkv : nullptr, big, 1, s)) return rc;
        // key coordinates: the history this segment's queries can see (from kb: position 0 in a
        // global block, the window's start rounded down to 32 in a local one), then its rows
        const uint32_t window = Ly.slots >= g->cfg.context_length ? 0u : Ly.slots;
        const uint32_t kb = window != 0u && p0 + 1u > window ? (p0 + 1u - window) & ~31u : 0u;
        uint32_t qo = p0 - kb;
        if (qo != 0u) {
            const float* kc = Ly.kc;
            const float* vc = Ly.vc;
            uint32_t slots = Ly.slots, kvf = P.kv16, kb_ = kb;
            _Float16* khi = static_cast<_Float16*>(p.khi);
            _Float16* klo = static_cast<_Float16*>(p.klo);
            _Float16* vhi = static_cast<_Float16*>(p.vhi);
            _Float16* vlo = static_cast<_Float16*>(p.vlo);
            void* args[] = {&kc, &vc, &slots, &kvf, &kb_, &qo, &hd, &khi, &klo, &vhi, &vlo};
            if (int rc = launch(reinterpret_cast<const void*>(&k_pf_kv_hist), dim3(qo), args)) return rc;
        }
        {
            const float* qn = Ly.q_norm;
            const float* kn = Ly.k_norm;
            const float* ct = Ly.global ? P.cos_g : P.cos_l;
            const float* sn = Ly.global ? P.sin_g : P.sin_l;
            float* kc = Ly.kc;
            float* vc = Ly.vc;
            uint32_t slots = Ly.slots;
            // rows past the segment zero the keys and values up to the next 64 key coordinates
            const uint32_t tp = pf_pad(qo + T) - qo;
            _Float16* khi = static_cast<_Float16*>(p.khi);
            _Float16* klo = static_cast<_Float16*>(p.klo);
            _Float16* vhi = static_cast<_Float16*>(p.vhi);
            _Float16* vlo = static_cast<_Float16*>(p.vlo);
            uint32_t kvf = P.kv16, p0_ = p0, qo_ = qo;
            void* args[] = {&big, &T, &H, &hd, &qn, &kn, &ct, &sn, &eps, &kc, &vc, &slots, &ahi, &alo, &khi, &klo, &vhi, &vlo,
                            &kvf, &p0_, &qo_};
            const uint32_t waves = std::min(H + 1u, kPfQkMaxWaves);
            VRT_HIP_CHECK(hipLaunchKernel(reinterpret_cast<const void*>(&k_pf_qk), dim3(tp), dim3(64u * waves), args, 0, s));
        }
        // The last block's output feeds only the LM head, so past its q/k/v (every position's
        // keys and values go to the cache) it runs for the last position alone: attention for
        // that position's query tile, then one row.
        const bool last = l + 1u == L;
        if (last && !final) break;   // an earlier segment: the last block's keys and values are all it leaves
        const uint32_t fr = last ? 1u : T;
        const uint64_t a0 = last ? static_cast<uint64_t>(T - 1u) * d : 0u;
        const uint64_t aq = last ? static_cast<uint64_t>(T - 1u) * qw : 0u;
        // the attention output replaces q (hi/lo in ahi/alo)
        if (int rc = pf_attention(g, Ly, T, last ? (T - 1u) / 32u : 0u, ahi, alo, s, qo)) return rc;
        uint32_t so = last ? pf_splits(1u, d) : s_o;
        if (int rc = pf_gemm(g, ahi + aq, alo + aq, fr, qw, {{Ly.wo, d}}, lw ? &lw[l].o : nullptr, x, so, s)) return rc;
        so = std::max(1u, std::min(so, (qw / 32u) / 2u));
        {   // attention output into the residual, then the FFN norm (the O partials of fr rows)
            const uint64_t xo = static_cast<uint64_t>(fr) * d;
            if (int rc = pf_norm(h + a0, x, so, xo, Ly.post_attn, Ly.ffn_norm, d, eps, ahi + a0, alo + a0, st, Ly.index,
                                 fr, s, true))
                return rc;
        }
        // gelu(gate) * up as f16 hi/lo in `big` (the gate/up GEMM still reads ahi/alo).
        _Float16* ghi = reinterpret_cast<_Float16*>(big);
        _Float16* glo = ghi + static_cast<uint64_t>(fr) * F;
        if (int rc = pf_gemm_glu(g, ahi + a0, alo + a0, fr, d, Ly.wg, Ly.wu, F, lw ? &lw[l].gu : nullptr, ghi, glo, s))
            return rc;
        s_down = std::max(1u, std::min(last ? pf_splits(1u, d) : s_o, (F / 32u) / 2u));
        if (int rc = pf_gemm(g, ghi, glo, fr, F, {{Ly.wd, d}}, lw ? &lw[l].down : nullptr, x, s_down, s)) return rc;
    }
    if (!final) return VRT_OK;
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
