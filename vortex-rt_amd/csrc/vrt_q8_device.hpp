// vrt_q8_device.hpp -- gfx950 device primitives for Q8_0 matrix-vector work.
//
// Q8_0 (GGUF type 8): 34-byte blocks {f16 scale little-endian, int8 q[32]} along K, rows
// contiguous. y[r] = sum_b f16(s_rb) * sum_k q_rbk * x[32b + k]   (shaders/q8_matvec*.comp).
//
// Activation limbs. Every 32-element block j of x is rewritten once per launch as
//     x_k ~= s_j * (a_k + b_k / 254 + c_k / 254^2),   s_j = amax_j / 127,  a, b, c int8,
// with |error| <= s_j * 0.5 / 254^2 = amax_j * 6.1e-8 (fp32 resolution). The block dot then
// runs on the integer dot unit: A = sum q*a, B = sum q*b, C = sum q*c via v_dot4_i32_i8
// (exact int32), and y_block = d_w * s_j * (A + B/254 + C/254^2) in fp32. That is 24 dot4 +
// 8 byte-realigns per 34-byte block instead of 32 int->float converts and 32 FMAs, which
// keeps the streaming kernels under the VALU ceiling at full HBM rate.
//
// Lane layout. A wave is split into 64/S row slots of S lanes; slot lane t owns blocks
// t, t+S, ... (NB of them) for the whole launch, so its limbs live in registers. Every
// lane reads its block with nine aligned dword loads (plus the 2-byte scale); neighbouring
// lanes read neighbouring blocks, so a slot streams its row contiguously.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vrt {

constexpr int kWave = 64;

// ---- cross-lane reductions -------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// v(lane) + v(lane ^ 16) on the VALU: v_permlane16_swap exchanges the odd 16-lane rows of one
// copy with the even rows of the other, so the two results hold both rows of each pair.
__device__ __forceinline__ float add_xor16(float v) {
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// v(lane) + v(lane ^ 32) on the VALU, the same way with v_permlane32_swap (wave halves).
__device__ __forceinline__ float add_xor32(float v) {
    const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// Sum over each aligned group of S lanes (S a power of two <= 64). Every lane of a group
// ends with the group total (S <= 32); for S == 64 lanes 0..31 and 32..63 each hold
// half sums, so use wave_sum for a full-wave total.
template <int S>
__device__ __forceinline__ float slot_sum(float v) {
    if constexpr (S >= 2) v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    if constexpr (S >= 4) v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    if constexpr (S >= 8) v += dpp_mov<0x141>(v);   // row_half_mirror
    if constexpr (S >= 16) v += dpp_mov<0x140>(v);  // row_mirror
    if constexpr (S >= 32) v = add_xor16(v);
    return v;
}

// Full-wave sum, wave-uniform result.
__device__ __forceinline__ float wave_sum(float v) {
    v = slot_sum<32>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// Full-wave reductions on the DPP path (no LDS round trips): rows of 16 lanes first, then
// row_bcast15 / row_bcast31 fold the rows into lane 63, which is read back uniformly.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_or_zero(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_red_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    // lanes outside the row mask keep their own value (old = v): max is unchanged
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_d(double v, bool zero_fill) {
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = static_cast<int>(b), hi = static_cast<int>(b >> 32);
    const int olo = zero_fill ? 0 : lo, ohi = zero_fill ? 0 : hi;
    const int rlo = __builtin_amdgcn_update_dpp(olo, lo, CTRL, ROW_MASK, 0xf, false);
    const int rhi = __builtin_amdgcn_update_dpp(ohi, hi, CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, (static_cast<long long>(rhi) << 32) | static_cast<unsigned int>(rlo));
}

// Full-wave double sum (uniform result). The order of the adds is fixed, so every workgroup
// reducing the same values gets the same bits.
__device__ __forceinline__ double wave_red_sum_d(double v) {
    v += dpp_d<0xB1, 0xf>(v, false);
    v += dpp_d<0x4E, 0xf>(v, false);
    v += dpp_d<0x141, 0xf>(v, false);
    v += dpp_d<0x140, 0xf>(v, false);
    v += dpp_d<0x142, 0xa>(v, true);
    v += dpp_d<0x143, 0xc>(v, true);
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), 63);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), 63);
    return __builtin_bit_cast(double, (static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// ---- argmax rule (shaders/argmax.comp:30-43) --------------------------------------------

__device__ __forceinline__ bool am_better(float cv, uint32_t ci, float bv, uint32_t bi) {
    if (__builtin_isnan(cv)) return false;
    return cv > bv || (cv == bv && ci < bi);
}

// Wave-wide argmax under am_better; result valid in every lane.
__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const uint32_t oi = __shfl_xor(i, off);
        if (am_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
}

// ---- f16 -------------------------------------------------------------------------------

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);   // v_cvt_f32_f16, exact
}

// 16-bit KV cache entries, fmt 1 fp16 and 2 bf16: IEEE round to nearest even into the entry
// (v_cvt_f16_f32 / v_cvt_pk_bf16_f32), exact back to fp32.
__device__ __forceinline__ uint16_t kv16_bits(float x, uint32_t fmt) {
    return fmt == 2u ? __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)) : __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
__device__ __forceinline__ float kv16_float(uint16_t b, uint32_t fmt) {
    return fmt == 2u ? __uint_as_float(static_cast<uint32_t>(b) << 16) : static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// ---- Q8_0 block loads ------------------------------------------------------------------

struct Q8Raw {
    uint32_t d[9];   // dwords covering the 32 quants, starting at (block + 2) & ~3
    uint32_t sbits;  // f16 scale bits
    uint32_t sh;     // byte shift of the quants inside d: 0 or 2
};

// blk: start of a 34-byte block (2-byte aligned); end: one past the last readable byte.
// Reads stay inside [blk, blk + 34) except for up to 2 bytes past the block, which are
// read only when they lie before `end`.
// Weights always live in global memory: global (not FLAT) loads.
__device__ __forceinline__ void q8_load(const uint8_t* blk, const uint8_t* end, Q8Raw& r) {
    typedef const __attribute__((address_space(1))) uint32_t* gu32;
    typedef const __attribute__((address_space(1))) uint16_t* gu16;
    const uintptr_t q = reinterpret_cast<uintptr_t>(blk) + 2u;
    const gu32 lb = reinterpret_cast<gu32>(q & ~uintptr_t(3));
    r.sh = static_cast<uint32_t>(q & 3u);
    r.sbits = *(gu16)(blk);
#pragma unroll
    for (int j = 0; j < 8; ++j) r.d[j] = lb[j];
    r.d[8] = 0u;
    if (r.sh) {
        const uintptr_t tail = (q & ~uintptr_t(3)) + 32u;
        r.d[8] = (tail + 4 <= reinterpret_cast<uintptr_t>(end)) ? lb[8] : static_cast<uint32_t>(*reinterpret_cast<gu16>(tail));
    }
}

// ---- activation limbs --------------------------------------------------------------------

struct XLimb {
    int a[8], b[8], c[8];   // 32 int8 each, packed 4 per dword in k order
    float s;                // block scale: amax/127; 0 for an all-zero block; NaN if non-finite
};

// LDS image of the limbs for a K-vector: la/lb/lc int8[K], ls float[K/32].
struct LimbLds {
    int8_t* a;
    int8_t* b;
    int8_t* c;
    float* s;
};

// Limbs of one element against its block's scale (amax m > 0): x / s = a + b/254 + c/254^2.
__device__ __forceinline__ void limb3(float v, float m, int8_t& qa, int8_t& qb, int8_t& qc) {
    const float inv = 127.0f / m;
    const float r = v * inv;
    const float a = rintf(r);
    const float e1 = (r - a) * 254.0f;
    const float b = fminf(fmaxf(rintf(e1), -127.0f), 127.0f);
    const float e2 = (e1 - b) * 254.0f;
    const float c = fminf(fmaxf(rintf(e2), -127.0f), 127.0f);
    qa = static_cast<int8_t>(fminf(fmaxf(a, -127.0f), 127.0f));
    qb = static_cast<int8_t>(b);
    qc = static_cast<int8_t>(c);
}

// Cooperative limb build for xs[0..K) (LDS) by all threads of the block. A block of 32
// elements is one 16-lane row of a wave (two elements per lane), so its amax is a DPP
// reduction within the row and a wave covers four blocks per pass. A non-finite element
// enters the amax as +inf and makes the block scale NaN. `nwaves` is the workgroup's wave
// count. Ends with __syncthreads().
__device__ __forceinline__ void build_limbs(const float* xs, uint32_t K, LimbLds L, uint32_t nwaves) {
    const uint32_t nblk = K >> 5;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t quad = wave; quad * 4u < nblk; quad += nwaves) {
        const uint32_t blk = quad * 4u + (lane >> 4);
        const bool live = blk < nblk;
        const uint32_t k = blk * 32u + 2u * (lane & 15u);
        const float2 v = live ? *reinterpret_cast<const float2*>(xs + k) : make_float2(0.0f, 0.0f);
        auto mag = [](float x) { return __builtin_isfinite(x) ? fabsf(x) : INFINITY; };
        float m = fmaxf(mag(v.x), mag(v.y));
        m = fmaxf(m, dpp_mov<0xB1>(m));    // quad_perm [1,0,3,2]
        m = fmaxf(m, dpp_mov<0x4E>(m));    // quad_perm [2,3,0,1]
        m = fmaxf(m, dpp_mov<0x141>(m));   // row_half_mirror
        m = fmaxf(m, dpp_mov<0x140>(m));   // row_mirror: every lane of the row holds its amax
        int8_t qa0 = 0, qb0 = 0, qc0 = 0, qa1 = 0, qb1 = 0, qc1 = 0;
        float s = 0.0f;
        if (m == INFINITY) {
            s = __builtin_nanf("");
        } else if (m >= 1e-30f) {
            s = m * (1.0f / 127.0f);
            limb3(v.x, m, qa0, qb0, qc0);
            limb3(v.y, m, qa1, qb1, qc1);
        }
        if (live) {
            auto pk = [](int8_t lo, int8_t hi) {
                return static_cast<uint16_t>(static_cast<uint8_t>(lo) | (static_cast<uint16_t>(static_cast<uint8_t>(hi)) << 8));
            };
            *reinterpret_cast<uint16_t*>(L.a + k) = pk(qa0, qa1);
            *reinterpret_cast<uint16_t*>(L.b + k) = pk(qb0, qb1);
            *reinterpret_cast<uint16_t*>(L.c + k) = pk(qc0, qc1);
            if ((lane & 15u) == 0u) L.s[blk] = s;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void load_limb(const LimbLds& L, uint32_t blk, XLimb& x) {
    const int* pa = reinterpret_cast<const int*>(L.a + blk * 32u);
    const int* pb = reinterpret_cast<const int*>(L.b + blk * 32u);
    const int* pc = reinterpret_cast<const int*>(L.c + blk * 32u);
#pragma unroll
    for (int j = 0; j < 8; ++j) { x.a[j] = pa[j]; x.b[j] = pb[j]; x.c[j] = pc[j]; }
    x.s = L.s[blk];
}

// One block's contribution: d_w * s_x * (A + B/254 + C/254^2).
__device__ __forceinline__ float q8_dot(const Q8Raw& r, const XLimb& x) {
    int A = 0, B = 0, Cc = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = static_cast<int>(__builtin_amdgcn_alignbyte(r.d[j + 1], r.d[j], r.sh));
        A = __builtin_amdgcn_sdot4(q, x.a[j], A, false);
        B = __builtin_amdgcn_sdot4(q, x.b[j], B, false);
        Cc = __builtin_amdgcn_sdot4(q, x.c[j], Cc, false);
    }
    const float t = fmaf(static_cast<float>(Cc), 1.0f / 64516.0f,
                         fmaf(static_cast<float>(B), 1.0f / 254.0f, static_cast<float>(A)));
    return half_bits_to_float(r.sbits) * x.s * t;
}

// One block's contribution against fp32 activations x[0..31] (LDS, 16-byte aligned): the 32
// int8 products in four partial sums by k mod 4 (four short FMA chains instead of one of 32),
// added pairwise, then scaled: d_w * ((s0 + s1) + (s2 + s3)).
__device__ __forceinline__ float q8_dot_x(const Q8Raw& r, const float* x) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = static_cast<int>(__builtin_amdgcn_alignbyte(r.d[j + 1], r.d[j], r.sh));
        const float4 xv = *reinterpret_cast<const float4*>(x + 4 * j);
        a0 = fmaf(static_cast<float>((q << 24) >> 24), xv.x, a0);
        a1 = fmaf(static_cast<float>((q << 16) >> 24), xv.y, a1);
        a2 = fmaf(static_cast<float>((q << 8) >> 24), xv.z, a2);
        a3 = fmaf(static_cast<float>(q >> 24), xv.w, a3);
    }
    return half_bits_to_float(r.sbits) * ((a0 + a1) + (a2 + a3));
}

// ---- row streaming ----------------------------------------------------------------------

// A virtual row space over up to kMaxSeg Q8_0 matrices sharing K. Either the segments are
// concatenated (rows of segment 0, then 1, ...) or, with `interleave`, virtual row v is
// row v>>1 of segment v&1 (gate/up pairs).
constexpr int kMaxSeg = 8;

struct RowSpace {
    const uint8_t* base[kMaxSeg];
    uint32_t rows[kMaxSeg];
    uint32_t first[kMaxSeg];   // first virtual row of each segment (concatenated mode)
    uint32_t nseg;
    uint32_t total;
    uint32_t interleave;
};

__device__ __forceinline__ const uint8_t* row_ptr(const RowSpace& rs, uint32_t v, uint64_t row_bytes,
                                                  uint32_t& seg, uint32_t& local) {
    // Unrolled compare-select over the segment table keeps RowSpace in registers.
    const uint8_t* base;
    if (rs.interleave) {
        seg = v & 1u;
        local = v >> 1;
        base = seg ? rs.base[1] : rs.base[0];
    } else {
        seg = 0;
        base = rs.base[0];
        uint32_t first = 0;
#pragma unroll
        for (int i = 1; i < kMaxSeg; ++i) {
            if (static_cast<uint32_t>(i) < rs.nseg && v >= rs.first[i]) {
                seg = static_cast<uint32_t>(i);
                base = rs.base[i];
                first = rs.first[i];
            }
        }
        local = v - first;
    }
    return base + static_cast<uint64_t>(local) * row_bytes;
}

// Streams virtual rows [v_begin, v_end) with the calling wave: row groups of 64/S rows,
// wave w of the block takes groups w, w + nwaves, ... and keeps U groups in flight.
// sink(v, value) is called on the lane that owns row v's total (slot lane 0).
template <int S, int NB, int U, typename Sink>
__device__ __forceinline__ void stream_rows(const RowSpace& rs, uint64_t row_bytes, uint32_t nblk,
                                            const uint8_t* w_end, const XLimb (&xl)[NB],
                                            uint32_t v_begin, uint32_t v_end, Sink&& sink) {
    constexpr uint32_t RPW = 64u / S;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t slot = lane / S;
    const uint32_t sl = lane % S;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t ngroups = (v_end - v_begin + RPW - 1u) / RPW;
    for (uint32_t g0 = wave; g0 < ngroups; g0 += U * nwaves) {
        Q8Raw raw[U][NB];
        uint32_t vrow[U];
        bool live[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t g = g0 + static_cast<uint32_t>(u) * nwaves;
            vrow[u] = v_begin + g * RPW + slot;
            live[u] = g < ngroups && vrow[u] < v_end;
            uint32_t seg, local;
            const uint8_t* rp = live[u] ? row_ptr(rs, vrow[u], row_bytes, seg, local) : nullptr;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const uint32_t b = sl + static_cast<uint32_t>(n) * S;
                if (live[u] && b < nblk) q8_load(rp + 34u * b, w_end, raw[u][n]);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float acc = 0.0f;
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const uint32_t b = sl + static_cast<uint32_t>(n) * S;
                if (live[u] && b < nblk) acc += q8_dot(raw[u][n], xl[n]);
            }
            float tot;
            if constexpr (S == 64) {
                const float h = slot_sum<32>(acc);
                tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 0)) +
                      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 32));
            } else {
                tot = slot_sum<S>(acc);
            }
            if (live[u] && sl == 0u) sink(vrow[u], tot);
        }
    }
}

// ---- batched row streaming (prefetch, then consume) ------------------------------------------

template <int S, int NB, int U>
struct RowBatch {
    Q8Raw raw[U][NB];
    uint32_t vrow[U];
    bool live[U];
};

// rowp(v) returns the first byte of virtual row v. Pass U = 1 passes rows to wave group g0;
// pass u to g0 + u * nwaves (a constant where the workgroup size is one: reading blockDim is
// a load, and its wait would also wait for the weight loads issued before it).
template <int S, int NB, int U, typename RowFn>
__device__ __forceinline__ void batch_load(RowFn&& rowp, uint32_t nblk, const uint8_t* w_end, uint32_t v_begin,
                                           uint32_t v_end, uint32_t g0, uint32_t nwaves, RowBatch<S, NB, U>& rb) {
    constexpr uint32_t RPW = 64u / S;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t slot = lane / S, sl = lane % S;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t g = g0 + static_cast<uint32_t>(u) * nwaves;
        rb.vrow[u] = v_begin + g * RPW + slot;
        rb.live[u] = rb.vrow[u] < v_end;
        const uint8_t* rp = rb.live[u] ? rowp(rb.vrow[u]) : nullptr;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const uint32_t b = sl + static_cast<uint32_t>(n) * S;
            if (rb.live[u] && b < nblk) q8_load(rp + 34u * b, w_end, rb.raw[u][n]);
        }
    }
}

template <int S, int NB, int U, typename Sink>
__device__ __forceinline__ void batch_consume(const RowBatch<S, NB, U>& rb, uint32_t nblk, const XLimb (&xl)[NB],
                                              Sink&& sink) {
    const uint32_t sl = (threadIdx.x & 63u) % S;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const uint32_t b = sl + static_cast<uint32_t>(n) * S;
            if (rb.live[u] && b < nblk) acc += q8_dot(rb.raw[u][n], xl[n]);
        }
        float tot;
        if constexpr (S == 64) {
            const float h = slot_sum<32>(acc);
            tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 0)) +
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 32));
        } else {
            tot = slot_sum<S>(acc);
        }
        if (rb.live[u] && sl == 0u) sink(rb.vrow[u], tot);
    }
}

// As batch_consume, against fp32 activations xs[0..K) in LDS (q8_dot_x per block).
template <int S, int NB, int U, typename Sink>
__device__ __forceinline__ void batch_consume_x(const RowBatch<S, NB, U>& rb, uint32_t nblk, const float* xs,
                                                Sink&& sink) {
    const uint32_t sl = (threadIdx.x & 63u) % S;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const uint32_t b = sl + static_cast<uint32_t>(n) * S;
            if (rb.live[u] && b < nblk) acc += q8_dot_x(rb.raw[u][n], xs + 32u * b);
        }
        float tot;
        if constexpr (S == 64) {
            const float h = slot_sum<32>(acc);
            tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 0)) +
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(h), 32));
        } else {
            tot = slot_sum<S>(acc);
        }
        if (rb.live[u] && sl == 0u) sink(rb.vrow[u], tot);
    }
}

template <int S, int NB>
__device__ __forceinline__ void lane_limbs(const LimbLds& L, uint32_t nblk, XLimb (&xl)[NB]) {
    const uint32_t sl = (threadIdx.x & 63u) % S;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        const uint32_t b = sl + static_cast<uint32_t>(n) * S;
        if (b < nblk) load_limb(L, b, xl[n]);
    }
}


}  // namespace vrt
