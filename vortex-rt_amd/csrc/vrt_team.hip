// vrt_team.hip -- phase-team persistent decode kernel for gfx950: the Gemma 3 token loop of
// src/gemma3.cpp:1462-1882 and :2080-2149 at short attention histories, several steps per launch.
//
// Why teams. A block is four dependent matvec phases with a hand-off between each: q|k|v, then
// attention and the O projection, then the post-attention/FFN norms with gate/up, then down. On
// MI355X a tagged exchange in which every workgroup both publishes and then polls (an all-gather
// over all 256 workgroups) costs ~2.1-2.4 us per round: a wave's vector-memory operations complete
// in issue order, so the poll that follows its own system-scope stores waits for their
// acknowledgement, and the round waits for the slowest of 256 producers. A one-way hand-off from
// one group of workgroups to another that has nothing in flight costs ~1.3 us. So the 256
// workgroups are split into four phase teams of nwg/4, and each team runs one phase type for
// every block:
//
//   team A  h = RMSNorm(d_{l-1}, post_ffw) + hm_{l-1} (or the scaled embedding row),
//           x = RMSNorm(h, attn_norm), rows of [Wq | Wk | Wv]                    (:1511-1541)
//   team B  QK-norm, RoPE, KV append, attention of one query head over the whole history,
//           normalised, times that head's columns of Wo: per-head partials o_h   (:1557-1701)
//   team D  hm = RMSNorm(sum_h o_h, post_attn) + h, x = RMSNorm(hm, ffn_norm), gate/up row
//           pairs, g = gelu_tanh(gate) * up                                        (:1703-1801)
//   team E  rows of Wd -> d                                                        (:1803-1855)
//
// Every hand-off is one-way (A -> B -> D -> E -> A), and a team's next phase of the same type
// comes three phases later: right after publishing block l a team issues the loads of block
// l + 1's weight rows (and team B the key/value rows of block l + 1's history) into registers,
// so the weight fetch overlaps the other teams' phases and a phase's critical path is its poll,
// its norm and its dot products. The residual stream travels with the hand-offs (A publishes h,
// D publishes hm), and every reader of a vector computes the same bits from the same words.
// After the last block every workgroup runs the final norm and an even share of the tied Q8_0
// LM head fused with the greedy argmax (as the all-workgroup persistent kernel does), and the
// next step starts from the argmax partials.
//
// Histories. Each head is computed by tsize/H workgroups, each producing its group of Wo rows
// over that head's columns. While a head's history fits on chip, every one of them attends over
// all of it: the first 64 positions in registers (eight waves of eight), the next hist_lds in
// LDS (direct-to-LDS loads issued with the register loads, one phase ahead; 72 positions of fp32
// entries at head_dim 256, 144 of 16-bit ones). Longer histories split into tsize/H chunks, one
// per workgroup of the head, laid out the same way (passes past the LDS rows load when they
// run); the chunks' partials {acc, max, sum} go through x_p and every workgroup of the head
// merges them in chunk order. Each wave runs an online softmax over its eight positions of every
// 64-position pass.
//
// Buffer reuse without double buffering: every exchange buffer is written once per block, and
// a team rewrites a buffer for block l + 1 only after consuming data that every reader of the
// block-l contents produced after reading them (A(l+1) needs d(l) from every E workgroup, which
// needed g(l) from every D workgroup, which read h(l) and o(l) before publishing, ...). Across
// steps the LM head reads hm and d of the last block and the next step's first phase needs the
// argmax of every workgroup (or, for prompt steps without an LM head, team A folds the last
// block's output before it starts the next step).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <type_traits>
#include <vector>

#include "vrt_g3_errors.hpp"
#include "vrt_g3_internal.hpp"
#include "vrt_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {
namespace tk {

typedef unsigned long long u64;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

#define TK_AS_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ TK_AS_GLOBAL T* gp(T* p) { return (TK_AS_GLOBAL T*)p; }
template <typename T>
__device__ __forceinline__ const TK_AS_GLOBAL T* gp(const T* p) { return (const TK_AS_GLOBAL T*)p; }

constexpr uint32_t kThreads = 512;          // 8 waves: two per SIMD
constexpr uint32_t kWaves = kThreads / 64;
constexpr uint32_t kTeams = 4;              // A, B, D, E
constexpr uint32_t kSpinLimit = 1u << 21;   // polls before a hand-off is declared lost
constexpr int kRsrcFlags = 0x00020000;      // raw buffer resource, 32-bit data format
constexpr int kCoherent = 17;               // buffer access aux bits: sc0 | sc1 (system scope)
constexpr uint32_t kLine = 8;               // tagged words per 64-byte line
constexpr uint32_t kBPos = 8;               // attention positions per wave
constexpr uint32_t kHistMax = kWaves * kBPos;   // longest history (positions) a block can attend to
constexpr uint32_t kMaxHeads = 4;           // query heads (partials summed by team D)
constexpr uint32_t kPartUnits = 4;          // 16-byte polls per thread of a head's chunk accumulators
constexpr uint32_t kMaxTeamChunks = 64;     // history chunks per head (one lane of a wave each)
constexpr uint32_t kLmUnits = 3;            // 16-byte LM-head loads per thread per tile
constexpr uint32_t kLmRing = 4;             // LM-head tile slots in LDS
constexpr uint32_t kLmAhead = kLmRing - 1u; // tiles in flight while one is computed
constexpr uint32_t kLmTileBytes = kLmUnits * kThreads * 16u;
// matrix-core LM head: each of the first kLmWaves waves streams its own 16-row tiles through a
// ring of its own
constexpr uint32_t kLmWaves = 4;
constexpr uint32_t kLmWaveRows = 16;
constexpr uint32_t kLmWaveLoads = 11;       // 1 KB direct-to-LDS loads per wave tile
constexpr uint32_t kLmWaveSlot = kLmWaveLoads * 1024u;
constexpr uint32_t kLmWaveRing = 3;         // slots per wave: two tiles in flight while one is computed
constexpr uint32_t kLdsBytes = 159u * 1024u;
constexpr uint32_t kMaxLayers = 64;
constexpr uint32_t kAnySets = 4;

struct Layer {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw;
    float* kc;
    float* vc;
    uint32_t slots;
    uint32_t global;
};

// Byte offsets of the LDS carve-up (phases run one at a time, so x, the attention scratch and
// the LM-head ring are separate only where a phase uses them together).
struct Lds {
    uint32_t x;      // matvec input: A's x, B's head attention, D's x, E's g; the LM head's x
    uint32_t red;    // residual folds: wave totals [waves][4] and flags [waves]
    uint32_t dn;     // A, D: row partials and norm sums of the deferred-norm projections (DnLds)
    uint32_t scr;    // A, D: each wave's activation limbs of its K blocks
    uint32_t qkv;    // B: q_h after QK-norm and RoPE (shares am: the argmax partials are read before)
    uint32_t kvc;    // B: the current position's k and v after QK-norm and RoPE
    uint32_t kvx;    // B: key rows, then value rows, of history positions 64 .. 64 + hist_lds - 1
    uint32_t part;   // B: per-wave attention partials [waves][hd], then m [waves], l [waves] (shares x)
    uint32_t la, lb, lc, ls;   // LM head activation limbs
    uint32_t am;     // argmax partials [2 * nwg]
    uint32_t any;    // workgroup OR flags
    uint32_t ring;   // LM-head tiles
    uint32_t tr;     // trace stamps
    uint32_t total;
};

struct Params {
    uint32_t d, H, hd, F, V, L, ctx_len, eos;
    float eps, emb_scale, attn_scale;
    uint32_t nwg, tsize;           // workgroups; workgroups per team
    uint32_t lm_tile_rows;
    uint32_t trace_slots;          // stamps per workgroup (0: tracing off)
    uint32_t kv16;                 // KV cache entries: 0 fp32, 1 fp16, 2 bf16
    uint32_t hist_lds;             // history positions past the registers held in LDS (multiple of 8)
    uint32_t poll_sleep;           // back-off between unsuccessful polls (s_sleep units of 64 clocks)
    Lds lds;
    const uint8_t* tok_embd;
    const uint8_t* arena_end;
    const float* out_norm;
    const float *cos_l, *sin_l, *cos_g, *sin_g;
    u64 *x_h, *x_qkv, *x_o, *x_hm, *x_g, *x_d, *x_am;   // x_o: [H][d] per-head partials
    u64* x_p;                      // [H][tsize / H][hd + 8] attention chunk partials {acc, M, l} (chunked histories)
    uint32_t* abort_flag;
    G3State* st;
    uint32_t* tokens;
    vrt_argmax_result* results;
    float* logits;
    float* hidden;
    uint64_t* trace;               // [nwg][trace_slots] s_memrealtime ticks of the first step
};

__constant__ Params g_tk;
__constant__ Layer g_tk_layers[kMaxLayers];

__shared__ __align__(16) unsigned char g_tk_lds[kLdsBytes];

template <typename T>
__device__ __forceinline__ T* lds(uint32_t off) { return reinterpret_cast<T*>(g_tk_lds + off); }

// Team and member of workgroup w: workgroup w runs on XCD w % 8, so each team is the 64
// workgroups of two XCDs (correctness does not depend on the placement: every exchange is
// system-coherent).
__device__ __forceinline__ uint32_t team_of(uint32_t w) { return (w & 7u) >> 1; }
__device__ __forceinline__ uint32_t member_of(uint32_t w) { return (w >> 3) * 2u + (w & 1u); }

// tags of block l's buffers in the step whose base is tagb; the argmax partials of that step
// take tagb + nph (the next step's base, which no buffer of that step uses)
constexpr uint32_t kTagsPerBlock = 7;
enum : uint32_t { kTH = 1, kTQkv = 2, kTO = 3, kTHm = 4, kTG = 5, kTD = 6, kTP = 7 };
__device__ __forceinline__ uint32_t tagof(uint32_t tagb, uint32_t l, uint32_t k) { return tagb + kTagsPerBlock * l + k; }

// ---- tagged exchange ---------------------------------------------------------------------

__device__ __forceinline__ void st_word(u64* p, float v, uint32_t tag) {
    __hip_atomic_store(gp(p), static_cast<u64>(__float_as_uint(v)) | (static_cast<u64>(tag) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_bits(u64* p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(gp(p), static_cast<u64>(bits) | (static_cast<u64>(tag) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool aborted() {
    return __hip_atomic_load(gp(g_tk.abort_flag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void raise_abort() {
    __hip_atomic_store(gp(g_tk.abort_flag), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_min(uint32_t v) {
    __hip_atomic_fetch_min(gp(&g_tk.st->nonfinite), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), kRsrcFlags);
}

// Polls N 16-byte units (two tagged words each) of up to two buffers until both tags of every
// live unit equal its tag; unit k reads buffer which[k] at byte off[k]. out[2k], out[2k+1] get
// the values. Returns 1 if the wait was abandoned (spin limit, or another workgroup's abort).
// Backs off between two unsuccessful polls: s_sleep of g_tk.poll_sleep (x 64 clocks).
__device__ __forceinline__ void poll_backoff() {
    switch (g_tk.poll_sleep) {
    case 0: break;
    case 1: __builtin_amdgcn_s_sleep(1); break;
    case 2: __builtin_amdgcn_s_sleep(2); break;
    case 4: __builtin_amdgcn_s_sleep(4); break;
    case 8: __builtin_amdgcn_s_sleep(8); break;
    default: __builtin_amdgcn_s_sleep(16); break;
    }
}

template <int N>
__device__ __forceinline__ int poll_units(__amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1, const int (&off)[N],
                                          const bool (&which)[N], const bool (&live)[N], const uint32_t (&tag)[N],
                                          float (&out)[2 * N]) {
    v4u v[N];
#pragma unroll
    for (int k = 0; k < N; ++k)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(which[k] ? r1 : r0, live[k] ? off[k] : 0x7ffffff0, 0, kCoherent);
    int fail = 0;
    uint32_t spins = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < N; ++k) ready &= !live[k] || (v[k].y == tag[k] && v[k].w == tag[k]);
        if (ready) break;
        if ((++spins & 63u) == 0u && (spins > kSpinLimit || aborted())) {
            fail = 1;
            raise_abort();
            break;
        }
        poll_backoff();
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < N; ++k)
            v[k] = __builtin_amdgcn_raw_buffer_load_b128(which[k] ? r1 : r0, live[k] ? off[k] : 0x7ffffff0, 0, kCoherent);
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        out[2 * k] = __uint_as_float(v[k].x);
        out[2 * k + 1] = __uint_as_float(v[k].z);
    }
    return fail;
}

// Workgroup OR of `pred` behind one barrier (flag set `id`).
__device__ __forceinline__ bool blk_any(int pred, uint32_t id) {
    uint32_t* f = lds<uint32_t>(g_tk.lds.any) + id * kWaves;
    const bool wa = __builtin_amdgcn_ballot_w64(pred != 0) != 0u;
    if ((threadIdx.x & 63u) == 0u) f[threadIdx.x >> 6] = wa ? 1u : 0u;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (uint32_t k = 0; k < kWaves; ++k) r |= f[k];
    return r != 0u;
}

// Gathers the tagged words src[0..n) (n even) into LDS dst with every thread (MAXP 16-byte
// pairs each), then a barrier; false in every thread if abandoned.
template <int MAXP>
__device__ __forceinline__ bool gather(const u64* src, uint32_t n, uint32_t tag, float* dst, uint32_t any_id) {
    const __amdgpu_buffer_rsrc_t r = rsrc(src, n * 8u);
    int off[MAXP];
    bool live[MAXP], which[MAXP];
    uint32_t tg[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        const uint32_t j = threadIdx.x + static_cast<uint32_t>(p) * kThreads;
        live[p] = 2u * j < n;
        off[p] = static_cast<int>(j * 16u);
        which[p] = false;
        tg[p] = tag;
    }
    float v[2 * MAXP];
    const int fail = poll_units<MAXP>(r, r, off, which, live, tg, v);
#pragma unroll
    for (int p = 0; p < MAXP; ++p)
        if (live[p]) reinterpret_cast<float2*>(dst)[threadIdx.x + p * kThreads] = make_float2(v[2 * p], v[2 * p + 1]);
    return !blk_any(fail, any_id);
}

__device__ __forceinline__ void split_range(uint32_t total, uint32_t parts, uint32_t idx, uint32_t& a, uint32_t& b) {
    a = static_cast<uint32_t>(static_cast<uint64_t>(total) * idx / parts);
    b = static_cast<uint32_t>(static_cast<uint64_t>(total) * (idx + 1u) / parts);
}
// As split_range in whole 64-byte lines of tagged words: no two producers write one line.
__device__ __forceinline__ void split_lines(uint32_t total, uint32_t parts, uint32_t idx, uint32_t& a, uint32_t& b) {
    split_range((total + kLine - 1u) / kLine, parts, idx, a, b);
    a = min(total, a * kLine);
    b = min(total, b * kLine);
}

// 1.0f / std::sqrt(float(sum_sq / n) + eps) (src/gemma3.cpp:967-983).
__device__ __forceinline__ float rms_scale(double ss, uint32_t n, float eps) {
#pragma clang fp contract(off)
    return 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(n)) + eps);
}

__device__ __forceinline__ float gelu(float x) {
#pragma clang fp contract(off)
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float cubic = x * x * x;
    return 0.5f * x * (1.0f + tanhf(kSqrt2OverPi * (x + kCubic * cubic)));
}

// gelu_tanh with tanh(u) = 1 - 2 / (exp(2u) + 1) on the hardware exponential and reciprocal:
// within ~1e-6 relative of the reference's tanhf form (shaders/gelu_mul.comp:23-31).
__device__ __forceinline__ float gelu_fast(float x) {
#pragma clang fp contract(off)
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float u = kSqrt2OverPi * (x + kCubic * (x * x * x));
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * u) + 1.0f);
    return 0.5f * x * (1.0f + t);
}

// Limbs of one element given 127 / amax of its block (limb3 of vrt_q8_device.hpp with the
// reciprocal computed once per block on v_rcp_f32 instead of a division per element: the limbs
// then represent v to within ~1.2e-7 relative plus the 6.1e-8 amax residual).
__device__ __forceinline__ void limb3_r(float v, float inv, int8_t& qa, int8_t& qb, int8_t& qc) {
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

template <int N>
__device__ __forceinline__ double tree_sum(double (&v)[N]) {
#pragma unroll
    for (int s = 1; s < N; s *= 2)
#pragma unroll
        for (int i = 0; i + s < N; i += 2 * s) v[i] += v[i + s];
    return v[0];
}

// Sums v[0..7] over the wave and transposes: lane l ends with the total of v[l & 7] (three
// exchanges inside each group of 8 lanes, then across the groups; partners add the same
// operands, so every lane of a position holds the same bits).
__device__ __forceinline__ float wave_sum8_t(const float (&v)[8]) {
    const uint32_t lane = __lane_id();
    const bool b2 = (lane & 4u) != 0u, b1 = (lane & 2u) != 0u, b0 = (lane & 1u) != 0u;
    float a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = (b2 ? v[i + 4] : v[i]) + dpp_mov<0x141>(b2 ? v[i] : v[i + 4]);   // row_half_mirror
#pragma unroll
    for (int i = 0; i < 2; ++i) b[i] = (b1 ? a[i + 2] : a[i]) + dpp_mov<0x4E>(b1 ? a[i] : a[i + 2]);    // quad_perm [2,3,0,1]
    float c = (b0 ? b[1] : b[0]) + dpp_mov<0xB1>(b0 ? b[0] : b[1]);                                    // quad_perm [1,0,3,2]
    c += dpp_mov<0x128>(c);   // row_ror:8
    c = add_xor16(c);
    return add_xor32(c);
}

// ---- trace -------------------------------------------------------------------------------------

// Stamp k of the traced step: k < L this workgroup's phase of block k had its inputs, L + k it had
// published; 2L step start (token known), 2L + 1 the LM head's final norm done, 2L + 2 LM head done.
__device__ __forceinline__ void stamp(bool tr, uint32_t k) {
    if (tr && threadIdx.x == 0u) lds<uint64_t>(g_tk.lds.tr)[k] = __builtin_amdgcn_s_memrealtime();
}
// Sub-phase mark k (< kSubMarks) of block 1 of the traced step, after the 2L + 3 phase stamps.
constexpr uint32_t kSubMarks = 8;
__device__ __forceinline__ void submark(bool on, uint32_t k) { stamp(on, 2u * g_tk.L + 3u + k); }

// ---- the residual fold ----------------------------------------------------------------------

// Norm weights of one fold for this lane's element pair (prefetched with the phase's weights).
struct FoldW {
    float2 post, next;
};
// The pair of a d-vector that lane l of wave w owns in a fold: p = 64 w + l (waves w < EP2).
__device__ __forceinline__ uint32_t fold_pair() { return threadIdx.x; }
__device__ __forceinline__ FoldW fold_weights(const float* w_post, const float* w_next) {
    const uint32_t p = fold_pair(), pp = p < (g_tk.d >> 1) ? p : 0u;
    FoldW f;
    f.post = w_post ? make_float2(gp(w_post)[2u * pp], gp(w_post)[2u * pp + 1u]) : make_float2(0.0f, 0.0f);
    f.next = make_float2(gp(w_next)[2u * pp], gp(w_next)[2u * pp + 1u]);
    return f;
}

// rms(v) = 1 / sqrt(sum v^2 / d + eps) from a float sum of squares: v_rsq_f32 (1 ulp) of the
// mean square. The reference accumulates the squares in double and divides with
// 1.0f / std::sqrt (src/gemma3.cpp:967-983); the float sum of these pairwise reductions is within
// ~1e-6 relative of it, far inside the parity tolerances.
__device__ __forceinline__ float rms_fast(float ss, float inv_n, float eps) {
#pragma clang fp contract(off)
    return __builtin_amdgcn_rsqf(ss * inv_n + eps);
}

// Sums of four values over the wave, the four DPP chains interleaved (uniform results).
__device__ __forceinline__ void wave_sum4(float& a, float& b, float& c, float& e) {
    float v[4] = {a, b, c, e};
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_mov<0xB1>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_mov<0x4E>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_mov<0x141>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_mov<0x140>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_or_zero<0x142, 0xa>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += dpp_or_zero<0x143, 0xc>(v[i]);
    a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), 63));
    b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[1]), 63));
    c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[2]), 63));
    e = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[3]), 63));
}

// The fold of a sublayer output into the residual stream and the norm of the result, spread over
// the workgroup: thread t (waves w < EP2) owns the element pair p = t of the d-vector and polls its
// pair of h (HS; else the scaled embedding row emb, src/gemma3.cpp:1106-1136) and of the ny
// partials of y:
//   if NY: y = sum_{q < ny} partial q in order q; h' = y * (rms(y) * w_post) + h  (:1703-1711, :1849-1855)
//   x = (h' * rms(h')) * w_next (INTO: rms_norm_into, :991-996) or h' * (rms(h') * w_next) (rms_norm_inplace)
// One reduction round serves both norms: with a = y * w_post, sum h'^2 = rms(y)^2 sum a^2 +
// 2 rms(y) sum a h + sum h^2, so each wave reduces sum y^2, sum a^2, sum a h and sum h^2 together
// and the wave totals are added in wave order through LDS (the same bits in every workgroup).
// x goes to LDS x_lds and, when Lx.a, as activation limbs (build_limbs' layout: a 32-element block
// is one 16-lane row of a wave); x_glob and the pairs of h' in [e0, e1) (to hout, tag thout) go
// out from the owning threads. A non-finite h' raises code nf_code when nf_raise (:1857-1863).
// Ends with a barrier; returns 1 in every thread if a wait was abandoned.
template <int EP2, bool HS, int NY, bool INTO>
__device__ __forceinline__ int fold_dist(const u64* hsrc, uint32_t th, const uint8_t* emb, const u64* ysrc, uint32_t ny,
                                         uint32_t ty, const FoldW& fw, float* x_lds, LimbLds Lx, float* x_glob,
                                         u64* hout, uint32_t e0, uint32_t e1, uint32_t thout, bool nf_raise,
                                         uint32_t nf_code, bool mk = false) {
#pragma clang fp contract(off)
    static_assert(EP2 <= static_cast<int>(kWaves), "one pair per thread");
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, d = g_tk.d, npair = d >> 1;
    const uint32_t p = fold_pair();
    const bool own = wave < static_cast<uint32_t>(EP2);   // wave-uniform
    const bool live = p < npair;
    float* red = lds<float>(g_tk.lds.red);                 // [kWaves][4] wave totals
    int* flg = reinterpret_cast<int*>(red + 4u * kWaves);  // [kWaves] abandoned waits
    float2 h = make_float2(0.0f, 0.0f), y = make_float2(0.0f, 0.0f);
    int fail = 0;
    if (own) {
        if constexpr (!HS) {
            if (live) {
                const TK_AS_GLOBAL uint8_t* b = gp(emb) + ((2u * p) >> 5) * 34u;
                const float sc = half_bits_to_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
                const uint32_t i = (2u * p) & 31u;
                h.x = (sc * static_cast<float>(static_cast<int8_t>(b[2 + i]))) * g_tk.emb_scale;
                h.y = (sc * static_cast<float>(static_cast<int8_t>(b[3 + i]))) * g_tk.emb_scale;
            }
        }
        if constexpr (HS || NY > 0) {
            constexpr int NU = (HS ? 1 : 0) + NY;
            int off[NU];
            bool which[NU], lv[NU];
            uint32_t tg[NU];
            if constexpr (HS) {
                off[0] = static_cast<int>(p * 16u);
                which[0] = false;
                lv[0] = live;
                tg[0] = th;
            }
#pragma unroll
            for (int q = 0; q < NY; ++q) {
                const int j = (HS ? 1 : 0) + q;
                off[j] = static_cast<int>((static_cast<uint32_t>(q) * d + 2u * p) * 8u);
                which[j] = true;
                lv[j] = live && static_cast<uint32_t>(q) < ny;
                tg[j] = ty;
            }
            float v[2 * NU];
            fail = poll_units<NU>(rsrc(hsrc, HS ? d * 8u : 0u), rsrc(ysrc, NY ? NY * d * 8u : 0u), off, which, lv, tg, v);
            if constexpr (HS) h = live ? make_float2(v[0], v[1]) : make_float2(0.0f, 0.0f);
            constexpr int y0 = HS ? 1 : 0;
#pragma unroll
            for (int q = 0; q < NY; ++q)
                if (lv[y0 + q]) {
                    if (q == 0) y = make_float2(v[2 * y0], v[2 * y0 + 1]);
                    else {
                        y.x += v[2 * (y0 + q)];
                        y.y += v[2 * (y0 + q) + 1];
                    }
                }
        }
    }
    submark(mk, 0);
    const float2 a = make_float2(y.x * fw.post.x, y.y * fw.post.y);
    if (own) {
        float syy = y.x * y.x + y.y * y.y, saa = a.x * a.x + a.y * a.y, sah = a.x * h.x + a.y * h.y,
              shh = h.x * h.x + h.y * h.y;
        wave_sum4(syy, saa, sah, shh);
        const bool wf = __builtin_amdgcn_ballot_w64(fail != 0) != 0u;
        if (lane == 0u) {
            *reinterpret_cast<float4*>(red + 4u * wave) = make_float4(syy, saa, sah, shh);
            flg[wave] = wf ? 1 : 0;
        }
    }
    __syncthreads();
    float syy = 0.0f, saa = 0.0f, sah = 0.0f, shh = 0.0f;
    int any = 0;
#pragma unroll
    for (int k = 0; k < EP2; ++k) {
        const float4 t = *reinterpret_cast<const float4*>(red + 4u * k);
        syy += t.x;
        saa += t.y;
        sah += t.z;
        shh += t.w;
        any |= flg[k];
    }
    if (any) return 1;
    submark(mk, 1);
    const float inv_d = 1.0f / static_cast<float>(d);
    float sc2;
    if constexpr (NY > 0) {
        const float sc = rms_fast(syy, inv_d, g_tk.eps);
        h.x = y.x * (sc * fw.post.x) + h.x;
        h.y = y.y * (sc * fw.post.y) + h.y;
        sc2 = rms_fast(sc * sc * saa + 2.0f * sc * sah + shh, inv_d, g_tk.eps);
    } else {
        sc2 = rms_fast(shh, inv_d, g_tk.eps);
    }
    if (own) {
        if (nf_raise) {
            const int nf = live && (!__builtin_isfinite(h.x) || !__builtin_isfinite(h.y));
            if (__builtin_amdgcn_ballot_w64(nf != 0) != 0u && lane == 0u) flag_min(nf_code);
        }
        float2 x;
        if constexpr (INTO) {
            x.x = h.x * sc2 * fw.next.x;
            x.y = h.y * sc2 * fw.next.y;
        } else {
            x.x = h.x * (sc2 * fw.next.x);
            x.y = h.y * (sc2 * fw.next.y);
        }
        if (!live) x = make_float2(0.0f, 0.0f);
        if (live) {
            reinterpret_cast<float2*>(x_lds)[p] = x;
            if (x_glob) {
                gp(x_glob)[2u * p] = x.x;
                gp(x_glob)[2u * p + 1u] = x.y;
            }
            if (hout && 2u * p >= e0 && 2u * p < e1) {
                st_word(hout + 2u * p, h.x, thout);
                st_word(hout + 2u * p + 1u, h.y, thout);
            }
        }
        if (Lx.a) {   // limbs of this wave's four blocks (build_limbs' arithmetic)
            auto mag = [](float v) { return __builtin_isfinite(v) ? fabsf(v) : INFINITY; };
            float mm = fmaxf(mag(x.x), mag(x.y));
            mm = fmaxf(mm, dpp_mov<0xB1>(mm));
            mm = fmaxf(mm, dpp_mov<0x4E>(mm));
            mm = fmaxf(mm, dpp_mov<0x141>(mm));
            mm = fmaxf(mm, dpp_mov<0x140>(mm));
            int8_t qa0 = 0, qb0 = 0, qc0 = 0, qa1 = 0, qb1 = 0, qc1 = 0;
            float sb = 0.0f;
            if (mm == INFINITY) {
                sb = __builtin_nanf("");
            } else if (mm >= 1e-30f) {
                sb = mm * (1.0f / 127.0f);
                const float inv = 127.0f * __builtin_amdgcn_rcpf(mm);
                limb3_r(x.x, inv, qa0, qb0, qc0);
                limb3_r(x.y, inv, qa1, qb1, qc1);
            }
            if (live) {
                auto pk = [](int8_t lo, int8_t hi) {
                    return static_cast<uint16_t>(static_cast<uint8_t>(lo) | (static_cast<uint16_t>(static_cast<uint8_t>(hi)) << 8));
                };
                const uint32_t k = 2u * p;
                *reinterpret_cast<uint16_t*>(Lx.a + k) = pk(qa0, qa1);
                *reinterpret_cast<uint16_t*>(Lx.b + k) = pk(qb0, qb1);
                *reinterpret_cast<uint16_t*>(Lx.c + k) = pk(qc0, qc1);
                if ((lane & 15u) == 0u) Lx.s[k >> 5] = sb;
            }
        }
    }
    submark(mk, 3);
    __syncthreads();
    submark(mk, 4);
    return 0;
}

// ---- LM head --------------------------------------------------------------------------------

// One 34-byte block at byte `off` (even) of an LDS tile with a 16-byte aligned base.
__device__ __forceinline__ void q8_load_lds(const uint8_t* tile, uint32_t off, Q8Raw& r) {
    const uint32_t sh = (off + 2u) & 3u;
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(tile + (off + 2u - sh));
    r.sh = sh;
    r.sbits = *reinterpret_cast<const uint16_t*>(tile + off);
#pragma unroll
    for (int j = 0; j < 9; ++j) r.d[j] = lb[j];
}

// Rows [r0, r1) of the LM head as the 16-byte units of their aligned span into an LDS tile with
// direct global->LDS loads (unit j at tile byte 16 j); returns the offset of row r0 in the span.
// Thread t moves units t + kThreads k (k < kLmUnits); units past the span re-load its last unit
// (the host requires 16 readable bytes after the table). Non-temporal: streamed once per step.
__device__ __forceinline__ uint32_t lm_tile_issue(uint32_t r0, uint32_t r1, uint64_t row_bytes, uint8_t* tile) {
    const uintptr_t s = reinterpret_cast<uintptr_t>(g_tk.tok_embd) + static_cast<uint64_t>(r0) * row_bytes;
    const uintptr_t a0 = s & ~uintptr_t(15);
    const uint32_t pre = static_cast<uint32_t>(s - a0);
    const uint64_t nbytes = pre + static_cast<uint64_t>(r1 - r0) * row_bytes;
    const uint32_t n16 = static_cast<uint32_t>((nbytes + 15u) / 16u);
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (uint32_t k = 0; k < kLmUnits; ++k) {
        const uint32_t j = threadIdx.x + k * kThreads;
        const uintptr_t p = a0 + static_cast<uintptr_t>(j < n16 ? j : n16 - 1u) * 16u;
        __builtin_amdgcn_global_load_lds((const TK_AS_GLOBAL void*)p,
                                         (__attribute__((address_space(3))) void*)(tile + 16u * (k * kThreads + 64u * wave)),
                                         16, 0, 2 /* nt */);
    }
    return pre;
}

// Waits until this wave's tile loads issued before its last `later` tiles are complete.
__device__ __forceinline__ void lm_wait_tiles(uint32_t later) {
    static_assert(kLmUnits * (kLmAhead - 1u) <= 15u && kLmAhead <= 4u, "vmcnt immediate");
    // s_waitcnt: vmcnt in bits 3:0, expcnt (7) and lgkmcnt (15) left unconstrained
    if (later >= 3u) __builtin_amdgcn_s_waitcnt(0x0F70 | (3u * kLmUnits));
    else if (later == 2u) __builtin_amdgcn_s_waitcnt(0x0F70 | (2u * kLmUnits));
    else if (later == 1u) __builtin_amdgcn_s_waitcnt(0x0F70 | kLmUnits);
    else __builtin_amdgcn_s_waitcnt(0x0F70);
}

enum : uint32_t { kAnyFold = 0, kAnyGather = 1, kAnyArgmax = 2, kAnyB = 3 };

// The final residual fold and output norm (src/gemma3.cpp:1849-1868) into LDS x; workgroup 0
// writes the hidden state and the block's non-finite flag. Ends with a barrier; false if abandoned.
template <int EP2>
__device__ __forceinline__ bool final_fold(uint32_t tagb, const FoldW& fw) {
    const uint32_t L = g_tk.L, w = blockIdx.x;
    const LimbLds Lm{lds<int8_t>(g_tk.lds.la), lds<int8_t>(g_tk.lds.lb), lds<int8_t>(g_tk.lds.lc), lds<float>(g_tk.lds.ls)};
    const int fail = fold_dist<EP2, true, 1, false>(g_tk.x_hm, tagof(tagb, L - 1u, kTHm), nullptr, g_tk.x_d, 1u,
                                                    tagof(tagb, L - 1u, kTD), fw, lds<float>(g_tk.lds.x), Lm,
                                                    w == 0u ? g_tk.hidden : nullptr, nullptr, 0u, 0u, 0u, w == 0u,
                                                    g3_code_nonfinite(L - 1u));
    return !fail;
}

typedef int v4i __attribute__((ext_vector_type(4)));

// The tied LM head on the matrix cores (v_mfma_i32_16x16x32_i8) for rows of NB Q8_0 blocks. Each of
// waves 0 .. kLmWaves - 1 streams its own tiles of 16 rows (rows (w + i nwg) * 64 + 16 wave ..) into
// a ring of its own with direct-to-LDS loads, so the loop has no workgroup barrier: a wave waits
// only for its own loads (the other waves only join the argmax). For block j the A operand holds
// the activation limbs block-diagonally: row m = 4 q + t of A is limb t (t < 3) of x's block j when
// q = j % 4, and zero otherwise; the B operand is the 32 quants of row n (lane n + 16 g: quants
// 8 g .. 8 g + 7), so one product covers the tile's 16 rows. After
// the blocks of group G (4G .. 4G + 3), C[4 q + t][n] is the limb-t dot product of block 4G + q
// with row n, held by lane n + 16 q, which combines the three limb products as q8_dot does and
// scales them by the block scales; the four lanes of a row then add their groups' sums.
template <int NB, int EP2>
__device__ __forceinline__ bool lm_waves(uint32_t tagb, uint32_t want_logits, bool tr, const FoldW& fw, float& bv,
                                         uint32_t& bi) {
#pragma clang fp contract(off)
    constexpr uint32_t NG = (NB + 3) / 4;
    constexpr uint32_t kRound = kLmWaves * kLmWaveRows;   // rows per workgroup round
    const uint32_t w = blockIdx.x, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15u, grp = lane >> 4;
    const uint32_t nwg = g_tk.nwg, V = g_tk.V;
    const uint32_t rb = static_cast<uint32_t>(NB) * 34u;
    const uint64_t first = static_cast<uint64_t>(w) * kRound + wave * kLmWaveRows;
    const uint64_t stride = static_cast<uint64_t>(kRound) * nwg;
    const uint32_t nt = wave < kLmWaves && first < V ? static_cast<uint32_t>((V - first + stride - 1u) / stride) : 0u;
    auto row0 = [&](uint32_t i) { return static_cast<uint32_t>(first + static_cast<uint64_t>(i) * stride); };
    uint8_t* ring = lds<uint8_t>(g_tk.lds.ring) + wave * (kLmWaveRing * kLmWaveSlot);
    auto slot = [&](uint32_t i) { return ring + (i % kLmWaveRing) * kLmWaveSlot; };
    // rows [r0, r1) as the 16-byte units of their aligned span, unit u at slot byte 16 u; units past
    // the span re-load its last unit (16 readable bytes follow the table). Non-temporal.
    auto issue = [&](uint32_t i) {
        const uint32_t r0 = row0(i), r1 = min(V, r0 + kLmWaveRows);
        const uintptr_t s0 = reinterpret_cast<uintptr_t>(g_tk.tok_embd) + static_cast<uint64_t>(r0) * rb;
        const uintptr_t a0 = s0 & ~uintptr_t(15);
        const uint32_t n16 = static_cast<uint32_t>(((s0 - a0) + static_cast<uint64_t>(r1 - r0) * rb + 15u) / 16u);
        uint8_t* dst = slot(i);
#pragma unroll
        for (uint32_t k = 0; k < kLmWaveLoads; ++k) {
            const uint32_t u = lane + 64u * k;
            __builtin_amdgcn_global_load_lds((const TK_AS_GLOBAL void*)(a0 + static_cast<uintptr_t>(u < n16 ? u : n16 - 1u) * 16u),
                                             (__attribute__((address_space(3))) void*)(dst + 1024u * k), 16, 0, 2 /* nt */);
        }
    };
#pragma unroll
    for (uint32_t i = 0; i + 1u < kLmWaveRing; ++i)
        if (i < nt) issue(i);
    if (!final_fold<EP2>(tagb, fw)) return false;
    stamp(tr, 2u * g_tk.L + 1u);
    long aop[NB];
    {
        const uint32_t q = n >> 2, limb = n & 3u;
        const int8_t* src = lds<int8_t>(limb == 0u ? g_tk.lds.la : (limb == 1u ? g_tk.lds.lb : g_tk.lds.lc));
#pragma unroll
        for (uint32_t j = 0; j < static_cast<uint32_t>(NB); ++j)
            aop[j] = (q == (j & 3u) && limb < 3u) ? *reinterpret_cast<const long*>(src + 32u * j + 8u * grp) : 0;
    }
    float sx[NG];   // activation scale of this lane's block in each group
    {
        const float* ls = lds<float>(g_tk.lds.ls);
#pragma unroll
        for (uint32_t G = 0; G < NG; ++G) sx[G] = 4u * G + grp < static_cast<uint32_t>(NB) ? ls[4u * G + grp] : 0.0f;
    }
    const float inv254 = 1.0f / 254.0f, inv64516 = 1.0f / 64516.0f;
    for (uint32_t i = 0; i < nt; ++i) {
        // this wave's loads of tile i are complete: at most those of tile i + 1 are outstanding
        static_assert(kLmWaveLoads <= 15u && kLmWaveRing == 3u, "vmcnt immediate");
        if (i + 1u < nt) __builtin_amdgcn_s_waitcnt(0x0F70 | kLmWaveLoads);
        else __builtin_amdgcn_s_waitcnt(0x0F70);
        // slot (i + 2) % 3 held tile i - 1, whose reads this wave has consumed
        if (i + 2u < nt) issue(i + 2u);
        const uint32_t r0 = row0(i);
        const uint8_t* tile = slot(i);
        const uint32_t pre = static_cast<uint32_t>((reinterpret_cast<uintptr_t>(g_tk.tok_embd) + static_cast<uint64_t>(r0) * rb) & 15u);
        const uint32_t rbase = pre + (n % kLmWaveRows) * rb;
        v4i acc[NG];
#pragma unroll
        for (uint32_t G = 0; G < NG; ++G) acc[G] = v4i{0, 0, 0, 0};
#pragma unroll
        for (uint32_t j = 0; j < static_cast<uint32_t>(NB); ++j) {
            const uint32_t addr = rbase + 34u * j + 2u + 8u * grp;
            const uint32_t* q = reinterpret_cast<const uint32_t*>(tile + (addr & ~3u));
            const uint32_t sh = addr & 3u, d0 = q[0], d1 = q[1], d2 = q[2];
            const long bop = static_cast<long>(__builtin_amdgcn_alignbyte(d1, d0, sh)) |
                             (static_cast<long>(__builtin_amdgcn_alignbyte(d2, d1, sh)) << 32);
            acc[j / 4u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[j], bop, acc[j / 4u], 0, 0, 0);
        }
        float part = 0.0f;
#pragma unroll
        for (uint32_t G = 0; G < NG; ++G) {
            const uint32_t j = 4u * G + grp;
            if (j < static_cast<uint32_t>(NB)) {
                const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t*>(tile + rbase + 34u * j));
                const float t = fmaf(static_cast<float>(acc[G][2]), inv64516,
                                     fmaf(static_cast<float>(acc[G][1]), inv254, static_cast<float>(acc[G][0])));
                part += dw * sx[G] * t;
            }
        }
        const float tot = add_xor32(add_xor16(part));
        const uint32_t v = r0 + lane;
        if (lane < kLmWaveRows && v < V) {
            if (want_logits) gp(g_tk.logits)[v] = tot;
            if (am_better(tot, v, bv, bi)) { bv = tot; bi = v; }
        }
    }
    return true;
}

// Final norm, tied Q8_0 LM head over this workgroup's tiles, local greedy argmax published with
// tag tLM (src/gemma3.cpp:1138-1185, shaders/argmax.comp:30-43).
template <int SD, int EP2, int LMB>
__device__ __attribute__((noinline)) bool phase_lm(uint32_t tagb, uint32_t tLM, uint32_t want_logits, bool tr) {
#pragma clang fp contract(off)
    tagb = __builtin_amdgcn_readfirstlane(tagb);
    tLM = __builtin_amdgcn_readfirstlane(tLM);
    want_logits = __builtin_amdgcn_readfirstlane(want_logits);
    __shared__ float s_v[kWaves];
    __shared__ uint32_t s_i[kWaves];
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t d = g_tk.d, nblk_d = d >> 5;
    const uint64_t rb_d = static_cast<uint64_t>(nblk_d) * 34u;
    const uint32_t TR = g_tk.lm_tile_rows, nwg = g_tk.nwg;
    const uint32_t tiles = (g_tk.V + TR - 1u) / TR;
    const uint32_t ntiles = w < tiles ? (tiles - w + nwg - 1u) / nwg : 0u;
    auto tile_row = [&](uint32_t ti) { return (w + ti * nwg) * TR; };
    const FoldW fw = fold_weights(g_tk_layers[g_tk.L - 1u].post_ffw, g_tk.out_norm);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    if constexpr (LMB > 0) {
        if (!lm_waves<LMB, EP2>(tagb, want_logits, tr, fw, bv, bi)) return false;
    } else {
        uint8_t* ring = lds<uint8_t>(g_tk.lds.ring);
        auto issue = [&](uint32_t ti) {
            const uint32_t r0 = tile_row(ti);
            return lm_tile_issue(r0, min(g_tk.V, r0 + TR), rb_d, ring + (ti % kLmRing) * kLmTileBytes);
        };
#pragma unroll
        for (uint32_t i = 0; i < kLmAhead; ++i)
            if (i < ntiles) (void)issue(i);
        if (!final_fold<EP2>(tagb, fw)) return false;
        stamp(tr, 2u * g_tk.L + 1u);
        const LimbLds Lm{lds<int8_t>(g_tk.lds.la), lds<int8_t>(g_tk.lds.lb), lds<int8_t>(g_tk.lds.lc), lds<float>(g_tk.lds.ls)};
        // row slots of LS lanes, LNB blocks per lane (20-block rows: 16-lane slots, four lanes with two)
        constexpr int LS = SD >= 32 ? SD / 2 : SD;
        constexpr int LNB = SD / LS;
        XLimb xl[LNB];
        lane_limbs<LS, LNB>(Lm, nblk_d, xl);
        constexpr uint32_t RPW = 64u / LS;
        const uint32_t slot = lane / LS, sl = lane % LS;
        for (uint32_t ti = 0; ti < ntiles; ++ti) {
            const uint32_t t0 = tile_row(ti), t1 = min(g_tk.V, t0 + TR);
            const uint8_t* tile = ring + (ti % kLmRing) * kLmTileBytes;
            const uint32_t pre_cur = static_cast<uint32_t>(
                (reinterpret_cast<uintptr_t>(g_tk.tok_embd) + static_cast<uint64_t>(t0) * rb_d) & 15u);
            lm_wait_tiles(min(kLmAhead - 1u, ntiles - 1u - ti));
            __syncthreads();   // tile ti is in LDS for every wave; every wave is done with tile ti - 1
            if (ti + kLmAhead < ntiles) (void)issue(ti + kLmAhead);
            const uint32_t nrows = t1 - t0;
            for (uint32_t rg = wave * RPW; rg < nrows; rg += kWaves * RPW) {
                const uint32_t r = rg + slot;
                const bool live = r < nrows;
                float acc = 0.0f;
    #pragma unroll
                for (int b = 0; b < LNB; ++b) {
                    const uint32_t blk = sl + static_cast<uint32_t>(b) * LS;
                    if (live && blk < nblk_d) {
                        Q8Raw raw;
                        q8_load_lds(tile, pre_cur + r * static_cast<uint32_t>(rb_d) + 34u * blk, raw);
                        acc += q8_dot(raw, xl[b]);
                    }
                }
                float tot;
                if constexpr (LS == 64) {
                    const float hsum = slot_sum<32>(acc);
                    tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hsum), 0)) +
                          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hsum), 32));
                } else {
                    tot = slot_sum<LS>(acc);
                }
                if (live && sl == 0u) {
                    const uint32_t v = t0 + r;
                    if (want_logits) gp(g_tk.logits)[v] = tot;
                    if (am_better(tot, v, bv, bi)) { bv = tot; bi = v; }
                }
            }
        }
    }
    wave_argmax(bv, bi);
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    // published by the last wave: the next step's argmax poll runs on waves 0-3, whose queues
    // then hold no store to wait for
    if (tid == kThreads - 64u) {
        for (uint32_t k = 0; k < kWaves; ++k)
            if (k && am_better(s_v[k], s_i[k], s_v[0], s_i[0])) { s_v[0] = s_v[k]; s_i[0] = s_i[k]; }
        st_word(g_tk.x_am + kLine * w, s_v[0], tLM);   // one 64-byte line per workgroup
        st_bits(g_tk.x_am + kLine * w + 1u, s_i[0], tLM);
    }
    stamp(tr, 2u * g_tk.L + 2u);
    return true;
}

struct Arg {
    uint32_t idx;
    float val;
    bool ok;
};

// Reduces the argmax partials tagged `tag` (every workgroup gets the same result).
__device__ __attribute__((always_inline)) Arg reduce_argmax(uint32_t tag) {
    tag = __builtin_amdgcn_readfirstlane(tag);
    __shared__ float s_v[kWaves];
    __shared__ uint32_t s_i[kWaves];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, nwg = g_tk.nwg;
    float* buf = lds<float>(g_tk.lds.am);
    int fail = 0;
    {
        int off[1];
        bool live[1], which[1];
        uint32_t tg[1];
        live[0] = tid < nwg;
        off[0] = static_cast<int>(tid * kLine * 8u);
        which[0] = false;
        tg[0] = tag;
        float v[2];
        if (tid < nwg) {
            const __amdgpu_buffer_rsrc_t r = rsrc(g_tk.x_am, kLine * nwg * 8u);
            fail = poll_units<1>(r, r, off, which, live, tg, v);
            buf[2u * tid] = v[0];
            buf[2u * tid + 1u] = v[1];
        }
    }
    const bool good = !blk_any(fail, kAnyArgmax);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t k = tid; k < nwg; k += kThreads) {
        const float v = buf[2u * k];
        const uint32_t i = __float_as_uint(buf[2u * k + 1u]);
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wave_argmax(bv, bi);
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    bv = s_v[0];
    bi = s_i[0];
    for (uint32_t k = 1; k < kWaves; ++k)
        if (am_better(s_v[k], s_i[k], bv, bi)) { bv = s_v[k]; bi = s_i[k]; }
    __syncthreads();
    return Arg{bi, bv, good};
}

// ---- step bookkeeping shared by the teams --------------------------------------------------------

struct StepCtl {
    uint32_t step0, stop, lm_from, feed_until, want_logits;
};

__device__ __forceinline__ StepCtl read_ctl() {
    StepCtl c;
    c.step0 = gp(g_tk.st)->step;
    c.stop = gp(g_tk.st)->stop;
    c.lm_from = gp(g_tk.st)->lm_from;
    c.feed_until = gp(g_tk.st)->feed_until;
    c.want_logits = gp(g_tk.st)->want_logits;
    return c;
}

// The token of step s: the host's, or the previous step's greedy result (argmax partials tagged
// prev_tag != 0). Workgroup 0 records the result; EOS stops the generation (src/gemma3.cpp:2134-2141).
// Returns false when the step must not run (stop set) or a wait was abandoned (ok cleared).
__device__ __forceinline__ bool step_token(uint32_t s, uint32_t prev_tag, StepCtl& c, bool& ok, uint32_t& token) {
    const uint32_t w = blockIdx.x, tid = threadIdx.x;
    if (prev_tag == 0u) {
        token = gp(g_tk.tokens)[s];
        return true;
    }
    const Arg a = reduce_argmax(prev_tag);
    ok = a.ok;
    if (!ok) return false;
    if (w == 0 && tid == 0) {
        TK_AS_GLOBAL vrt_argmax_result* r = gp(g_tk.results) + (s - 1u);
        r->index = a.idx;
        r->value = a.val;
    }
    if (s >= c.feed_until) {
        token = a.idx < g_tk.V ? a.idx : 0u;
        if (w == 0 && tid == 0) gp(g_tk.tokens)[s] = token;
        if (a.idx == g_tk.eos) {
            c.stop = 1u;
            return false;
        }
    } else {
        token = gp(g_tk.tokens)[s];
    }
    return true;
}

__device__ __forceinline__ void trace_begin(bool tr) {
    if (tr && threadIdx.x == 0u) {
        uint64_t* img = lds<uint64_t>(g_tk.lds.tr);
        for (uint32_t k = 0; k < g_tk.trace_slots; ++k) img[k] = 0u;
    }
}
__device__ __forceinline__ void trace_end(bool tr) {
    if (tr && threadIdx.x == 0u) {
        const uint64_t* img = lds<uint64_t>(g_tk.lds.tr);
        for (uint32_t k = 0; k < g_tk.trace_slots; ++k) gp(g_tk.trace)[blockIdx.x * g_tk.trace_slots + k] = img[k];
    }
}

// ---- weight rows in registers ---------------------------------------------------------------------

// A team's weight rows for its next phase are loaded into registers right after it publishes
// (three phases ahead of their use). At the start of the phase, before its poll, each block is
// realigned to eight dwords of quants and its f16 scale converted to fp32, so the dot products on
// the critical path are the integer dot4s on the activation limbs and the block scaling only.
__device__ __forceinline__ void q8_prep(Q8Raw& r) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r.d[j] = __builtin_amdgcn_alignbyte(r.d[j + 1], r.d[j], r.sh);
    r.sbits = __float_as_uint(half_bits_to_float(r.sbits));
    r.sh = 0;
}

// q8_dot on a prepared block: d_w * s_x * (A + B/254 + C/254^2).
__device__ __forceinline__ float q8_dot_p(const Q8Raw& r, const XLimb& x) {
    int A = 0, B = 0, Cc = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        A = __builtin_amdgcn_sdot4(static_cast<int>(r.d[j]), x.a[j], A, false);
        B = __builtin_amdgcn_sdot4(static_cast<int>(r.d[j]), x.b[j], B, false);
        Cc = __builtin_amdgcn_sdot4(static_cast<int>(r.d[j]), x.c[j], Cc, false);
    }
    const float t = fmaf(static_cast<float>(Cc), 1.0f / 64516.0f, fmaf(static_cast<float>(B), 1.0f / 254.0f, static_cast<float>(A)));
    return __uint_as_float(r.sbits) * x.s * t;
}

template <int S, int NB, int U>
__device__ __forceinline__ void batch_prep(RowBatch<S, NB, U>& rb) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int n = 0; n < NB; ++n) q8_prep(rb.raw[u][n]);
}

// batch_consume on prepared blocks.
template <int S, int NB, int U, typename Sink>
__device__ __forceinline__ void batch_consume_p(const RowBatch<S, NB, U>& rb, uint32_t nblk, const XLimb (&xl)[NB],
                                                Sink&& sink) {
    const uint32_t sl = (threadIdx.x & 63u) % S;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const uint32_t b = sl + static_cast<uint32_t>(n) * S;
            if (rb.live[u] && b < nblk) acc += q8_dot_p(rb.raw[u][n], xl[n]);
        }
        float tot;
        if constexpr (S == 64) {
            const float hs = slot_sum<32>(acc);
            tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), 0)) +
                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs), 32));
        } else {
            tot = slot_sum<S>(acc);
        }
        if (rb.live[u] && sl == 0u) sink(rb.vrow[u], tot);
    }
}

// Rows [v0, v1) (at most 64) with one row per lane, the waves splitting the K blocks: wave w
// takes blocks split_range(nblk, kWaves, w), at most KB of them. Each lane's partial over its
// wave's blocks goes to LDS, and the waves' partials are added in wave order.
template <int KB>
struct RowK {
    Q8Raw raw[KB];
};

template <int KB, typename RowFn>
__device__ __forceinline__ void rowk_load(RowFn&& rowp, uint32_t nblk, const uint8_t* end, uint32_t v0, uint32_t v1,
                                          RowK<KB>& rb) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t b0, b1;
    split_range(nblk, kWaves, wave, b0, b1);
    const uint32_t v = v0 + lane;
    const uint8_t* rp = v < v1 ? rowp(v) : nullptr;
#pragma unroll
    for (int j = 0; j < KB; ++j)
        if (v < v1 && b0 + static_cast<uint32_t>(j) < b1) q8_load(rp + 34u * (b0 + static_cast<uint32_t>(j)), end, rb.raw[j]);
}

template <int KB>
__device__ __forceinline__ void rowk_prep(RowK<KB>& rb) {
#pragma unroll
    for (int j = 0; j < KB; ++j) q8_prep(rb.raw[j]);
}

// This lane's partial over its wave's blocks, the activation limbs read from LDS (every lane of
// the wave reads the same block: broadcast).
template <int KB>
__device__ __forceinline__ float rowk_dot(const RowK<KB>& rb, const LimbLds& L, uint32_t nblk) {
    const uint32_t wave = threadIdx.x >> 6;
    uint32_t b0, b1;
    split_range(nblk, kWaves, wave, b0, b1);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < KB; ++j) {
        const uint32_t b = b0 + static_cast<uint32_t>(j);
        if (b < b1) {
            XLimb x;
            load_limb(L, b, x);
            acc += q8_dot_p(rb.raw[j], x);
        }
    }
    return acc;
}

// Limbs of the 32-element block whose element j sits in lane 2 j of the calling wave (odd lanes
// hold 0), in build_limbs' layout and arithmetic (with limb3_r): afterwards lane 8 k (k < 8) holds
// dword k of the int8 limbs a, b and c, and every lane the block scale (amax / 127; 0 for an
// all-zero block; NaN if an element is not finite).
__device__ __forceinline__ void block_limbs_even(float v, uint32_t& wa, uint32_t& wb, uint32_t& wc, float& scale) {
    const uint32_t lane = threadIdx.x & 63u;
    const float mg = __builtin_isfinite(v) ? fabsf(v) : INFINITY;
    const float mm = wave_red_max(mg);
    int8_t qa = 0, qb = 0, qc = 0;
    scale = 0.0f;
    if (mm == INFINITY) {
        scale = __builtin_nanf("");
    } else if (mm >= 1e-30f) {
        scale = mm * (1.0f / 127.0f);
        limb3_r(v, 127.0f * __builtin_amdgcn_rcpf(mm), qa, qb, qc);
    }
    const uint32_t sh = 8u * ((lane >> 1) & 3u);
    const bool ev = (lane & 1u) == 0u;
    wa = ev ? static_cast<uint32_t>(static_cast<uint8_t>(qa)) << sh : 0u;
    wb = ev ? static_cast<uint32_t>(static_cast<uint8_t>(qb)) << sh : 0u;
    wc = ev ? static_cast<uint32_t>(static_cast<uint8_t>(qc)) << sh : 0u;
    // lane 4q gathers lane 4q + 2's byte (quad_perm [2,3,0,1]), then lane 8k lane 8k + 4's (xor 4)
    wa |= static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(wa), 0x4E, 0xf, 0xf, false));
    wb |= static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(wb), 0x4E, 0xf, 0xf, false));
    wc |= static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(wc), 0x4E, 0xf, 0xf, false));
    wa |= static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(wa), 0x101F));
    wb |= static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(wb), 0x101F));
    wc |= static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(wc), 0x101F));
}

// Gathers the tagged words src[0..n) of a vector published as limbs (32 words per 32-element
// block) into LDS as their payload words, block b's word j at dst[33 b + j]: the odd stride puts
// the blocks that the 64 lanes of a wave read at once in 64 different banks. Every thread polls
// MAXP 16-byte pairs; ends with a barrier; false in every thread if abandoned.
template <int MAXP>
__device__ __forceinline__ bool gather_img(const u64* src, uint32_t n, uint32_t tag, uint32_t* dst, uint32_t any_id) {
    const __amdgpu_buffer_rsrc_t r = rsrc(src, n * 8u);
    int off[MAXP];
    bool live[MAXP], which[MAXP];
    uint32_t tg[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        const uint32_t j = threadIdx.x + static_cast<uint32_t>(p) * kThreads;
        live[p] = 2u * j < n;
        off[p] = static_cast<int>(j * 16u);
        which[p] = false;
        tg[p] = tag;
    }
    float v[2 * MAXP];
    const int fail = poll_units<MAXP>(r, r, off, which, live, tg, v);
#pragma unroll
    for (int p = 0; p < MAXP; ++p)
        if (live[p]) {
            const uint32_t i = 2u * (threadIdx.x + p * kThreads), o = 33u * (i >> 5) + (i & 31u);
            dst[o] = __float_as_uint(v[2 * p]);
            dst[o + 1u] = __float_as_uint(v[2 * p + 1]);
        }
    return !blk_any(fail, any_id);
}

// The limbs of block b of a vector published as 32 tagged words per block (a, b, c: 8 dwords each,
// then the scale) from its gather_img image.
__device__ __forceinline__ void load_limb_img(const uint32_t* img, uint32_t b, XLimb& x) {
    const uint32_t* p = img + 33u * b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        x.a[j] = static_cast<int>(p[j]);
        x.b[j] = static_cast<int>(p[8 + j]);
        x.c[j] = static_cast<int>(p[16 + j]);
    }
    x.s = __uint_as_float(p[24]);
}

// ---- projections with the norms applied after the dot products --------------------------------

// A projection of a normed residual fold, x = (h' * rms(h')) * w_next with h' = y * (rms(y) * w_post)
// + h (src/gemma3.cpp:1703-1718, :991-996), is linear in x, so each output row is
//     rms(h') * (rms(y) * W (y . w_post . w_next) + W (h . w_next))
// and the dot products need no global norm: W (h . w_next) runs as soon as h arrives (it is
// published phases before y), W (y . w_post . w_next) as soon as y arrives, and the two norms come
// from one reduction round afterwards (sum h'^2 = rms(y)^2 sum a^2 + 2 rms(y) sum a h + sum h^2,
// a = y . w_post). Layout: one output row per lane (at most 64 rows), the waves splitting the K
// blocks (wave w: blocks split_range(nblk, kWaves, w), at most KB); lane l of wave w owns the element
// pair 16 b0 + l of the wave's blocks, so a 32-element block is one 16-lane row of the wave. Each
// wave turns its elements into activation limbs in a scratch of its own in LDS (block j of the wave at
// scr + 112 j: a, b, c, then the scale) and every lane dots its row's blocks against them.

constexpr uint32_t kLimbBlkBytes = 112;   // one block's limbs in a wave scratch: 3 x 32 + scale, padded

// The pair of the d-vector that this lane owns in a deferred-norm projection (live: pair exists).
__device__ __forceinline__ uint32_t dn_pair(uint32_t nblk, bool& live, uint32_t& nb) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t b0, b1;
    split_range(nblk, kWaves, wave, b0, b1);
    nb = b1 - b0;
    live = lane < 16u * nb;
    return 16u * b0 + (live ? lane : 0u);
}

// Limbs of the wave's blocks from v (this lane's two elements; 0 where !live) into scr, then this
// lane's partial dot over the wave's blocks (row_live: the lane has a row).
template <int KB>
__device__ __forceinline__ float wave_limbs_dot(float2 v, bool live, uint32_t nb, uint8_t* scr, const RowK<KB>& rb,
                                                bool row_live, uint32_t jb = 0u, uint32_t je = ~0u) {
    const uint32_t lane = threadIdx.x & 63u;
    auto mag = [](float x) { return __builtin_isfinite(x) ? fabsf(x) : INFINITY; };
    float mm = fmaxf(mag(v.x), mag(v.y));
    mm = fmaxf(mm, dpp_mov<0xB1>(mm));
    mm = fmaxf(mm, dpp_mov<0x4E>(mm));
    mm = fmaxf(mm, dpp_mov<0x141>(mm));
    mm = fmaxf(mm, dpp_mov<0x140>(mm));   // every lane of a 16-lane row: its block's amax
    int8_t qa0 = 0, qb0 = 0, qc0 = 0, qa1 = 0, qb1 = 0, qc1 = 0;
    float sb = 0.0f;
    if (mm == INFINITY) {
        sb = __builtin_nanf("");
    } else if (mm >= 1e-30f) {
        sb = mm * (1.0f / 127.0f);
        const float inv = 127.0f * __builtin_amdgcn_rcpf(mm);
        limb3_r(v.x, inv, qa0, qb0, qc0);
        limb3_r(v.y, inv, qa1, qb1, qc1);
    }
    if (live) {
        auto pk = [](int8_t lo, int8_t hi) {
            return static_cast<uint16_t>(static_cast<uint8_t>(lo) | (static_cast<uint16_t>(static_cast<uint8_t>(hi)) << 8));
        };
        uint8_t* bp = scr + (lane >> 4) * kLimbBlkBytes + 2u * (lane & 15u);
        *reinterpret_cast<uint16_t*>(bp) = pk(qa0, qa1);
        *reinterpret_cast<uint16_t*>(bp + 32) = pk(qb0, qb1);
        *reinterpret_cast<uint16_t*>(bp + 64) = pk(qc0, qc1);
        if ((lane & 15u) == 0u) *reinterpret_cast<float*>(scr + (lane >> 4) * kLimbBlkBytes + 96u) = sb;
    }
    // the wave's own LDS writes precede its reads (in order within a wave)
    // this lane's blocks: jb + jj < min(je, nb), its weights in rb.raw[jj]
    float acc = 0.0f;
    const uint32_t jn = min(je, nb);
#pragma unroll
    for (int jj = 0; jj < KB; ++jj)
        if (jb + static_cast<uint32_t>(jj) < jn) {
            const uint32_t j = jb + static_cast<uint32_t>(jj);
            const uint32_t* q = reinterpret_cast<const uint32_t*>(scr + j * kLimbBlkBytes);
            XLimb x;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x.a[i] = static_cast<int>(q[i]);
                x.b[i] = static_cast<int>(q[8 + i]);
                x.c[i] = static_cast<int>(q[16 + i]);
            }
            x.s = __uint_as_float(q[24]);
            if (row_live) acc += q8_dot_p(rb.raw[jj], x);
        }
    return acc;
}

// Team A's split of a wave's K blocks over the two halves of the wave: lane l takes row l % 32
// and, of the wave's nb blocks, [0, ceil(nb / 2)) for l < 32 or [ceil(nb / 2), nb) for l >= 32.
__device__ __forceinline__ void half_blocks(uint32_t nb, uint32_t& jb, uint32_t& je) {
    const uint32_t h = (nb + 1u) >> 1;
    const bool hi = (threadIdx.x & 63u) >= 32u;
    jb = hi ? h : 0u;
    je = hi ? nb : h;
}

// Rows [v0, v1) (at most 32) with row v0 + l % 32 on lane l, each half of the wave loading its
// share of the wave's blocks (half_blocks), at most KB2 each.
template <int KB2, typename RowFn>
__device__ __forceinline__ void rowk_load_half(RowFn&& rowp, uint32_t nblk, const uint8_t* end, uint32_t v0, uint32_t v1,
                                               RowK<KB2>& rb) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t b0, b1, jb, je;
    split_range(nblk, kWaves, wave, b0, b1);
    half_blocks(b1 - b0, jb, je);
    const uint32_t v = v0 + (lane & 31u);
    const uint8_t* rp = v < v1 ? rowp(v) : nullptr;
#pragma unroll
    for (int jj = 0; jj < KB2; ++jj)
        if (v < v1 && jb + static_cast<uint32_t>(jj) < je) q8_load(rp + 34u * (b0 + jb + static_cast<uint32_t>(jj)), end, rb.raw[jj]);
}

// Polls this lane's pair of the ny (<= NY) tagged d-vectors src[q d ..] and sums them in order q.
template <int NY>
__device__ __forceinline__ int poll_pair_sum(const u64* src, uint32_t ny, uint32_t tag, uint32_t pb, bool live,
                                             float2& out) {
    const uint32_t d = g_tk.d;
    int off[NY];
    bool which[NY], lv[NY];
    uint32_t tg[NY];
#pragma unroll
    for (int q = 0; q < NY; ++q) {
        off[q] = static_cast<int>((static_cast<uint32_t>(q) * d + 2u * pb) * 8u);
        which[q] = false;
        lv[q] = live && static_cast<uint32_t>(q) < ny;
        tg[q] = tag;
    }
    float v[2 * NY];
    const __amdgpu_buffer_rsrc_t r = rsrc(src, NY * d * 8u);
    const int fail = poll_units<NY>(r, r, off, which, lv, tg, v);
    out = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int q = 0; q < NY; ++q)
        if (lv[q]) {
            out.x = q == 0 ? v[2 * q] : out.x + v[2 * q];
            out.y = q == 0 ? v[2 * q + 1] : out.y + v[2 * q + 1];
        }
    return fail;
}

// Per-wave totals of a deferred-norm projection in LDS (dn region): [kWaves][64] row partials of
// W (h . w_next), the same for W (y . w_post . w_next), [kWaves][4] sums and [kWaves] flags.
struct DnLds {
    float* p0;
    float* p1;
    float* sums;
    int* flg;
};
__device__ __forceinline__ DnLds dn_lds() {
    float* b = lds<float>(g_tk.lds.dn);
    return DnLds{b, b + kWaves * 64u, b + 2u * kWaves * 64u, reinterpret_cast<int*>(b + 2u * kWaves * 64u + 4u * kWaves)};
}

// The norm scalars from the wave totals (wave order; every thread the same bits).
__device__ __forceinline__ void dn_scalars(const DnLds& t, bool has_y, float& sc1, float& sc2, int& anyflag) {
    float syy = 0.0f, saa = 0.0f, sah = 0.0f, shh = 0.0f;
    int fl = 0;
#pragma unroll
    for (uint32_t k = 0; k < kWaves; ++k) {
        const float4 v = *reinterpret_cast<const float4*>(t.sums + 4u * k);
        syy += v.x;
        saa += v.y;
        sah += v.z;
        shh += v.w;
        fl |= t.flg[k];
    }
    anyflag = fl;
    const float inv_d = 1.0f / static_cast<float>(g_tk.d);
    sc1 = has_y ? rms_fast(syy, inv_d, g_tk.eps) : 0.0f;
    sc2 = rms_fast(has_y ? sc1 * sc1 * saa + 2.0f * sc1 * sah + shh : shh, inv_d, g_tk.eps);
}

// ---- shapes -------------------------------------------------------------------------------------

// Row-slot width S, blocks per lane NB and passes U of each team's matvec, and EP2 = the residual
// pairs per lane of the fold (d / 128 rounded up).
template <int SA_, int UA_, int SB_, int SD_, int KBD_, int SE_, int NBE_, int UE_, int EP2_, int LMB_ = 0>
struct Cfg {
    static constexpr int LMB = LMB_;             // LM head on the matrix cores for rows of LMB blocks (0: row slots)
    static constexpr int SA = SA_, UA = UA_;     // q|k|v rows: K = d
    static constexpr int SB = SB_;               // Wo rows over one head: K = head_dim
    static constexpr int SD = SD_;               // LM head row slots: K = d
    static constexpr int KBD = KBD_;             // gate/up: one row per lane, K blocks per wave
    static constexpr int SE = SE_, NBE = NBE_, UE = UE_;   // down rows: K = F
    static constexpr int EP2 = EP2_;
};

// ---- team A: q|k|v ---------------------------------------------------------------------------------

template <class C>
__device__ __attribute__((always_inline)) void team_a(uint32_t nsteps, uint32_t tag0) {
#pragma clang fp contract(off)
    nsteps = __builtin_amdgcn_readfirstlane(nsteps);
    tag0 = __builtin_amdgcn_readfirstlane(tag0);
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t m = member_of(w), ts = g_tk.tsize;
    const uint32_t d = g_tk.d, hd = g_tk.hd, qw = g_tk.H * hd, nqkv = qw + 2u * hd, L = g_tk.L;
    const uint32_t nblk_d = d >> 5;
    const uint64_t rb_d = static_cast<uint64_t>(nblk_d) * 34u;
    const uint32_t nph = kTagsPerBlock * L + 1u;
    uint32_t v0, v1, e0, e1;
    split_lines(nqkv, ts, m, v0, v1);   // at most 64 rows: one per lane
    split_lines(d, ts, m, e0, e1);
    const bool row_live = (lane & 31u) < v1 - v0;   // two lanes per row (half_blocks)
    const DnLds t = dn_lds();
    uint8_t* scr = lds<uint8_t>(g_tk.lds.scr) + wave * C::KBD * kLimbBlkBytes;
    bool plive;
    uint32_t pnb;
    const uint32_t pb = dn_pair(nblk_d, plive, pnb);
    uint32_t jb, je;
    half_blocks(pnb, jb, je);
    constexpr int KB2 = (C::KBD + 1) / 2;
    RowK<KB2> rb;
    float2 wp = make_float2(0.0f, 0.0f), wn = make_float2(0.0f, 0.0f);
    auto load = [&](uint32_t l) {
        const Layer& Ly = g_tk_layers[l];
        const uint8_t *wq = Ly.wq, *wk = Ly.wk, *wv = Ly.wv;
        auto rowp = [=](uint32_t v) -> const uint8_t* {
            return v < qw ? wq + static_cast<uint64_t>(v) * rb_d
                          : (v < qw + hd ? wk + static_cast<uint64_t>(v - qw) * rb_d
                                         : wv + static_cast<uint64_t>(v - qw - hd) * rb_d);
        };
        rowk_load_half<KB2>(rowp, nblk_d, g_tk.arena_end, v0, v1, rb);
        wn = make_float2(gp(Ly.attn_norm)[2u * pb], gp(Ly.attn_norm)[2u * pb + 1u]);
        if (l > 0u) {
            const float* wpost = g_tk_layers[l - 1u].post_ffw;
            wp = make_float2(gp(wpost)[2u * pb], gp(wpost)[2u * pb + 1u]);
        }
    };
    load(0);
    StepCtl c = read_ctl();
    uint32_t prev_tag = 0;
    uint32_t s = c.step0;
    bool ok = true;
    for (uint32_t si = 0; si < nsteps && ok; ++si, ++s) {
        if (c.stop || s >= g_tk.ctx_len) break;
        const bool tr = g_tk.trace_slots != 0u && si == 0u;
        const uint32_t tagb = tag0 + si * nph;
        uint32_t token;
        if (!step_token(s, prev_tag, c, ok, token)) break;
        prev_tag = 0u;
        trace_begin(tr);
        stamp(tr, 2u * L);
        for (uint32_t l = 0; l < L && ok; ++l) {
            const bool mk = tr && l == 1u;
            rowk_prep<KB2>(rb);
            // stage 1: h, the block's input residual (the scaled embedding row, or hm of block l - 1)
            float2 h = make_float2(0.0f, 0.0f);
            int fail = 0;
            if (l == 0u) {
                if (plive) {
                    const TK_AS_GLOBAL uint8_t* bq = gp(g_tk.tok_embd) + static_cast<uint64_t>(token) * rb_d + ((2u * pb) >> 5) * 34u;
                    const float sc = half_bits_to_float(static_cast<uint32_t>(bq[0]) | (static_cast<uint32_t>(bq[1]) << 8));
                    const uint32_t i = (2u * pb) & 31u;
                    h.x = (sc * static_cast<float>(static_cast<int8_t>(bq[2 + i]))) * g_tk.emb_scale;   // :1106-1136
                    h.y = (sc * static_cast<float>(static_cast<int8_t>(bq[3 + i]))) * g_tk.emb_scale;
                }
            } else {
                fail |= poll_pair_sum<1>(g_tk.x_hm, 1u, tagof(tagb, l - 1u, kTHm), pb, plive, h);
            }
            const float p0 = add_xor32(
                wave_limbs_dot<KB2>(make_float2(h.x * wn.x, h.y * wn.y), plive, pnb, scr, rb, row_live, jb, je));
            submark(mk, 0);
            // stage 2: y = d of block l - 1
            float2 a = make_float2(0.0f, 0.0f);
            float p1 = 0.0f, syy = 0.0f, saa = 0.0f, sah = 0.0f, shh = h.x * h.x + h.y * h.y;
            if (l > 0u) {
                float2 y;
                fail |= poll_pair_sum<1>(g_tk.x_d, 1u, tagof(tagb, l - 1u, kTD), pb, plive, y);
                submark(mk, 1);
                a = make_float2(y.x * wp.x, y.y * wp.y);
                p1 = add_xor32(
                    wave_limbs_dot<KB2>(make_float2(a.x * wn.x, a.y * wn.y), plive, pnb, scr, rb, row_live, jb, je));
                syy = y.x * y.x + y.y * y.y;
                saa = a.x * a.x + a.y * a.y;
                sah = a.x * h.x + a.y * h.y;
            }
            wave_sum4(syy, saa, sah, shh);
            t.p0[wave * 64u + lane] = p0;
            t.p1[wave * 64u + lane] = p1;
            const bool wf = __builtin_amdgcn_ballot_w64(fail != 0) != 0u;
            if (lane == 0u) {
                *reinterpret_cast<float4*>(t.sums + 4u * wave) = make_float4(syy, saa, sah, shh);
                t.flg[wave] = wf ? 1 : 0;
            }
            submark(mk, 2);
            __syncthreads();
            float sc1, sc2;
            int anyf;
            dn_scalars(t, l > 0u, sc1, sc2, anyf);
            if (anyf) { ok = false; break; }
            stamp(tr, l);
            // h' = y * (rms(y) * w_post) + h, published for team D; a non-finite h' fails block l - 1 (:1857-1863)
            const float2 hn = make_float2(a.x * sc1 + h.x, a.y * sc1 + h.y);
            if (l > 0u && m == 0u) {
                const bool nf = plive && (!__builtin_isfinite(hn.x) || !__builtin_isfinite(hn.y));
                if (__builtin_amdgcn_ballot_w64(nf) != 0u && lane == 0u) flag_min(g3_code_nonfinite(l - 1u));
            }
            if (plive && 2u * pb >= e0 && 2u * pb < e1) {
                st_word(g_tk.x_h + 2u * pb, hn.x, tagof(tagb, l, kTH));
                st_word(g_tk.x_h + 2u * pb + 1u, hn.y, tagof(tagb, l, kTH));
            }
            if (wave == 0u && lane < v1 - v0) {   // row v0 + lane: rms(h') * (rms(y) * P1 + P0), partials in wave order
                float q0[kWaves], q1[kWaves];
#pragma unroll
                for (uint32_t k = 0; k < kWaves; ++k) {
                    q0[k] = t.p0[k * 64u + lane];
                    q1[k] = t.p1[k * 64u + lane];
                }
                float P0 = q0[0], P1 = q1[0];
#pragma unroll
                for (uint32_t k = 1; k < kWaves; ++k) {
                    P0 += q0[k];
                    P1 += q1[k];
                }
                st_word(g_tk.x_qkv + v0 + lane, sc2 * (sc1 * P1 + P0), tagof(tagb, l, kTQkv));
            }
            stamp(tr, L + l);
            __syncthreads();   // the wave totals are rewritten by the next block
            if (l + 1u < L) load(l + 1u);
        }
        if (!ok) break;
        if (s >= c.lm_from) {
            ok = phase_lm<C::SD, C::EP2, C::LMB>(tagb, tagb + nph, c.want_logits, tr);
            prev_tag = tagb + nph;
        } else {
            // a prompt step: no LM head, but the next step may only start once the last block's
            // output is complete (its buffers are rewritten), and the hidden state is reported
            ok = final_fold<C::EP2>(tagb, fold_weights(g_tk_layers[L - 1u].post_ffw, g_tk.out_norm));
        }
        load(0);
        trace_end(tr);
    }
    // end of the launch: workgroup 0 records the last step's result and the step state
    if (w == 0) {
        if (ok && prev_tag != 0u && !c.stop) {
            const Arg a = reduce_argmax(prev_tag);
            ok = a.ok;
            if (ok && tid == 0) {
                TK_AS_GLOBAL vrt_argmax_result* r = gp(g_tk.results) + (s - 1u);
                r->index = a.idx;
                r->value = a.val;
                if (s >= c.feed_until) {
                    gp(g_tk.tokens)[s] = a.idx < g_tk.V ? a.idx : 0u;
                    if (a.idx == g_tk.eos) c.stop = 1u;
                }
            }
        }
        if (tid == 0) {
            gp(g_tk.st)->step = s;
            gp(g_tk.st)->stop = c.stop;
            if (!ok) flag_min(kG3HandoffLost);
        }
    }
}

// ---- team B: attention and the O projection ---------------------------------------------------

// Workgroup m takes query head h = m % H and row group m / H of Wo (over head h's columns). Wave
// j holds positions t_first + 8 j + i (i < 8) of the history; the key and value rows of cached
// positions are loaded into registers one phase ahead, the current position's come from the q|k|v
// hand-off (after QK-norm, RoPE and, for an fp16 cache, rounding). Wave 0 polls q_h, wave 1 k and
// v; they normalise (src/gemma3.cpp:1045-1104), rotate (:1371-1424) and share them through LDS,
// and member 0 appends k and v to the cache (:1590-1600). Each wave then runs a softmax over its
// eight positions (scores reduced and transposed together: lane l holds position l & 7's), the
// waves' partials are merged in wave order, att = acc / l (:1602-1696), and the workgroup's Wo
// rows over head h's blocks are published as x_o[h][row].
template <class C, typename KE, bool CH>
__device__ __attribute__((always_inline)) void team_b(uint32_t nsteps, uint32_t tag0) {
#pragma clang fp contract(off)
    nsteps = __builtin_amdgcn_readfirstlane(nsteps);
    tag0 = __builtin_amdgcn_readfirstlane(tag0);
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t m = member_of(w), ts = g_tk.tsize;
    const uint32_t d = g_tk.d, H = g_tk.H, hd = g_tk.hd, qw = H * hd, nqkv = qw + 2u * hd, L = g_tk.L;
    const uint32_t half = hd >> 1, nbh = hd >> 5;
    const uint64_t rb_a = static_cast<uint64_t>(qw >> 5) * 34u;
    const uint32_t nph = kTagsPerBlock * L + 1u;
    // head h and row group grp of member m. With an even team half per head count, the H heads
    // of one group sit on one XCD (member parity = XCD parity): a history chunk's key and value
    // rows, read by the H workgroups of its group, then come from one L2.
    const uint32_t ngrp = ts / H;
    const bool pair = (ts / 2u) % H == 0u;
    const uint32_t h = pair ? (m >> 1) % H : m % H;
    const uint32_t grp = pair ? ((m >> 1) / H) * 2u + (m & 1u) : m / H;
    uint32_t o0, o1;
    split_lines(d, ngrp, grp, o0, o1);
    const uint32_t dl = lane * 4u;                 // this lane's 4 head dims
    const bool dlive = dl < hd;
    const bool lo = dl < half;
    const uint32_t e0 = lo ? dl : dl - half;       // RoPE index of dim dl
    const int partner = static_cast<int>(lo ? lane + (half >> 2) : lane - (half >> 2));
    float* q_s = lds<float>(g_tk.lds.qkv);         // [hd] q_h
    float* kv_s = lds<float>(g_tk.lds.kvc);        // [2][hd] the current position's k, v
    float* part = lds<float>(g_tk.lds.part);       // [kWaves][hd], then m [kWaves], l [kWaves]
    const LimbLds Lx{lds<int8_t>(g_tk.lds.la), lds<int8_t>(g_tk.lds.lb), lds<int8_t>(g_tk.lds.lc), lds<float>(g_tk.lds.ls)};
    constexpr bool KVH = sizeof(KE) == 2;   // 16-bit entries: KE is _Float16 or __bf16
    constexpr uint32_t esz = KVH ? 2u : 4u;
    typedef KE half4_t __attribute__((ext_vector_type(4)));
    using KvReg = typename std::conditional<KVH, v2u, v4u>::type;
    auto kv_el = [](const KvReg& v, uint32_t e) -> float {
        if constexpr (KVH) return static_cast<float>(__builtin_bit_cast(half4_t, v)[e]);
        else return __uint_as_float(v[e]);
    };
    // The history of a block is positions [0, hist) by age (index i is position t_first + i,
    // ring slot (t_first + i) % slots; the current one is hist - 1). A workgroup attends over
    // its share [hb, he): the whole history while it fits on chip (64 + hist_lds positions),
    // else chunk grp of ngrp equal chunks, whose partials the head's ngrp workgroups exchange
    // and merge (x_p). Share positions hb + 64 .. hb + 64 + hist_lds - 1 sit in LDS: key row of
    // position hb + 64 + j at kvx + j * rowb, value rows after the hist_lds key rows. Pass p >= 1
    // of wave j covers share positions 64 p + 8 j + i (i < 8); the wave loads exactly those rows
    // (direct-to-LDS, 1 KB = ppi rows per load, 16 bytes per lane) and is their only reader, so
    // no barrier orders the loads: a wave waits for its own. Passes past the LDS rows load into
    // registers when they run.
    const uint32_t hist_lds = g_tk.hist_lds;
    const uint32_t rowb = hd * esz, ppi = 1024u / rowb, lpp = 64u / ppi;
    uint8_t* kvk = lds<uint8_t>(g_tk.lds.kvx);
    uint8_t* kvv = kvk + hist_lds * rowb;
    struct Geo {
        uint32_t hist, t_first, hb, he;
        bool chunked;
    };
    auto geo = [&](const Layer& Ly, uint32_t pos) {
        Geo G;
        G.hist = min(pos + 1u, Ly.slots);
        G.t_first = pos + 1u - G.hist;
        G.chunked = CH && G.hist > kHistMax + hist_lds;
        const uint32_t cs = G.chunked ? (G.hist + ngrp - 1u) / ngrp : G.hist;
        G.hb = G.chunked ? min(G.hist, grp * cs) : 0u;
        G.he = min(G.hist, G.hb + cs);
        return G;
    };
    RowBatch<C::SB, 1, 1> orb;
    KvReg kr[kBPos], vr[kBPos];
    // this wave's eight rows of share positions b0 .. b0 + 7 from the cache (cached positions
    // below he only: the others, and the current position, load zeros)
    auto load_rows = [&](const Layer& Ly, const Geo& G, uint32_t b0) {
        const uint32_t kv_bytes = Ly.slots * hd * esz;
        const __amdgpu_buffer_rsrc_t rk = rsrc(Ly.kc, kv_bytes), rv = rsrc(Ly.vc, kv_bytes);
        const uint32_t lane_off = dlive ? dl * esz : 0x7ffffff0u;
#pragma unroll
        for (uint32_t i = 0; i < kBPos; ++i) {
            const uint32_t idx = b0 + i;
            const int o = static_cast<int>(idx < G.he && idx + 1u < G.hist ? ((G.t_first + idx) % Ly.slots) * hd * esz + lane_off
                                                                            : 0x7ffffff0u);
            if constexpr (KVH) {
                kr[i] = __builtin_amdgcn_raw_buffer_load_b64(rk, o, 0, kCoherent);
                vr[i] = __builtin_amdgcn_raw_buffer_load_b64(rv, o, 0, kCoherent);
            } else {
                kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, kCoherent);
                vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, kCoherent);
            }
        }
    };
    // Wo rows of block l (head h's blocks) and this wave's cached key/value rows at position pos
    auto load = [&](uint32_t l, uint32_t pos) {
        const Layer& Ly = g_tk_layers[l];
        const uint8_t* wo = Ly.wo + static_cast<uint64_t>(h) * nbh * 34u;
        auto rowp = [=](uint32_t v) { return wo + static_cast<uint64_t>(v) * rb_a; };
        batch_load<C::SB, 1, 1>(rowp, nbh, g_tk.arena_end, o0, o1, wave, kWaves, orb);
        const Geo G = geo(Ly, pos);
        load_rows(Ly, G, G.hb + kBPos * wave);
        // the cached share positions hb + 64 .. past the registers (up to hist_lds of them); lanes
        // past the last one repeat it into slots that are masked or hold the current position
        const uint32_t ncached = min(min(G.he, G.hist - 1u), G.hb + kHistMax + hist_lds);
        const uint32_t t_first = G.t_first;
        for (uint32_t i0 = G.hb + kHistMax + kBPos * wave; i0 < ncached; i0 += kHistMax) {
            for (uint32_t i = 0; i < kBPos && i0 + i < ncached; i += ppi) {
                const uint32_t idx = min(i0 + i + lane / lpp, ncached - 1u);
                const uint64_t go = static_cast<uint64_t>((t_first + idx) % Ly.slots) * rowb + (lane % lpp) * 16u;
                const uint32_t so = (i0 + i - G.hb - kHistMax) * rowb;
                __builtin_amdgcn_global_load_lds((const TK_AS_GLOBAL void*)(reinterpret_cast<const uint8_t*>(Ly.kc) + go),
                                                 (__attribute__((address_space(3))) void*)(kvk + so), 16, 0, kCoherent);
                __builtin_amdgcn_global_load_lds((const TK_AS_GLOBAL void*)(reinterpret_cast<const uint8_t*>(Ly.vc) + go),
                                                 (__attribute__((address_space(3))) void*)(kvv + so), 16, 0, kCoherent);
            }
        }
    };
    StepCtl c = read_ctl();
    load(0, c.step0);
    uint32_t prev_tag = 0;
    uint32_t s = c.step0;
    bool ok = true;
    for (uint32_t si = 0; si < nsteps && ok; ++si, ++s) {
        if (c.stop || s >= g_tk.ctx_len) break;
        const bool tr = g_tk.trace_slots != 0u && si == 0u;
        const uint32_t tagb = tag0 + si * nph;
        uint32_t token;
        if (!step_token(s, prev_tag, c, ok, token)) break;
        prev_tag = 0u;
        trace_begin(tr);
        stamp(tr, 2u * L);
        const uint32_t pos = s;
        for (uint32_t l = 0; l < L && ok; ++l) {
            const Layer& Ly = g_tk_layers[l];
            const Geo G = geo(Ly, pos);
            const uint32_t hist = G.hist, he = G.he;
            const uint32_t tA = tagof(tagb, l, kTQkv);
            batch_prep<C::SB, 1, 1>(orb);
            int fail = 0;
            if (wave < 2u) {
                // wave 0: q_h; wave 1: k and v. Norm weights and RoPE factors first.
                const bool isq = wave == 0u;
                const float* ct = (Ly.global ? g_tk.cos_g : g_tk.cos_l) + static_cast<uint64_t>(pos) * half;
                const float* stb = (Ly.global ? g_tk.sin_g : g_tk.sin_l) + static_cast<uint64_t>(pos) * half;
                float wn[4], cs[4], sn[4];
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) {
                    wn[e] = dlive ? gp(isq ? Ly.q_norm : Ly.k_norm)[dl + e] : 0.0f;
                    cs[e] = dlive ? gp(ct)[e0 + e] : 0.0f;
                    sn[e] = dlive ? gp(stb)[e0 + e] : 0.0f;
                }
                int off[4];
                bool which[4], live[4];
                uint32_t tg[4];
                const uint32_t a0 = isq ? h * hd + dl : qw + dl, a1 = qw + hd + dl;
                off[0] = static_cast<int>(a0 * 8u);
                off[1] = static_cast<int>(a0 * 8u + 16u);
                off[2] = static_cast<int>(a1 * 8u);
                off[3] = static_cast<int>(a1 * 8u + 16u);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    which[k] = false;
                    live[k] = dlive && (k < 2 || !isq);
                    tg[k] = tA;
                }
                float v8[8];
                const __amdgpu_buffer_rsrc_t rq = rsrc(g_tk.x_qkv, nqkv * 8u);
                fail = poll_units<4>(rq, rq, off, which, live, tg, v8);
                float xv[4], vv[4];
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) {
                    xv[e] = dlive ? v8[e] : 0.0f;
                    vv[e] = dlive ? v8[4 + e] : 0.0f;
                }
                // QK-norm: values *= scale * weights (src/gemma3.cpp:1097-1102)
                float sq = (xv[0] * xv[0] + xv[1] * xv[1]) + (xv[2] * xv[2] + xv[3] * xv[3]), z0 = 0.0f, z1 = 0.0f, z2 = 0.0f;
                wave_sum4(sq, z0, z1, z2);
                const float sc = rms_fast(sq, 1.0f / static_cast<float>(hd), g_tk.eps);
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) xv[e] = xv[e] * (sc * wn[e]);
                // RoPE, NeoX halves: (a, b) = (x[e], x[e + half]) -> (a c - b s, b c + a s)
                float xo[4];
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) xo[e] = __shfl(xv[e], partner);
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) xv[e] = lo ? xv[e] * cs[e] - xo[e] * sn[e] : xv[e] * cs[e] + xo[e] * sn[e];
                if constexpr (KVH) {   // the current key and value as the cache holds them
                    if (!isq) {
#pragma unroll
                        for (uint32_t e = 0; e < 4u; ++e) {
                            xv[e] = static_cast<float>(static_cast<KE>(xv[e]));
                            vv[e] = static_cast<float>(static_cast<KE>(vv[e]));
                        }
                    }
                }
                if (dlive) {
                    *reinterpret_cast<float4*>((isq ? q_s : kv_s) + dl) = make_float4(xv[0], xv[1], xv[2], xv[3]);
                    if (!isq) *reinterpret_cast<float4*>(kv_s + hd + dl) = make_float4(vv[0], vv[1], vv[2], vv[3]);
                }
                if (!isq && m == 0u && dlive && !fail) {   // KV append of the current position
                    const uint32_t kv_bytes = Ly.slots * hd * esz;
                    const __amdgpu_buffer_rsrc_t rk = rsrc(Ly.kc, kv_bytes), rv = rsrc(Ly.vc, kv_bytes);
                    const int so = static_cast<int>(((pos % Ly.slots) * hd + dl) * esz);
                    if constexpr (KVH) {
                        auto pack = [](float a, float b) {
                            return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(a))) |
                                   (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(b))) << 16);
                        };
                        __builtin_amdgcn_raw_buffer_store_b64(v2u{pack(xv[0], xv[1]), pack(xv[2], xv[3])}, rk, so, 0, kCoherent);
                        __builtin_amdgcn_raw_buffer_store_b64(v2u{pack(vv[0], vv[1]), pack(vv[2], vv[3])}, rv, so, 0, kCoherent);
                    } else {
                        __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(xv[0]), __float_as_uint(xv[1]),
                                                                   __float_as_uint(xv[2]), __float_as_uint(xv[3])},
                                                               rk, so, 0, kCoherent);
                        __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(vv[0]), __float_as_uint(vv[1]),
                                                                   __float_as_uint(vv[2]), __float_as_uint(vv[3])},
                                                               rv, so, 0, kCoherent);
                    }
                }
            }
            if (blk_any(fail, kAnyB)) { ok = false; break; }
            stamp(tr, l);
            // this wave's share positions: hb + 8 wave + i from the registers, then hb + 64 p +
            // 8 wave + i (p >= 1) from LDS or, past the LDS rows, loaded now; the current one,
            // hist - 1, from kv_s
            const uint32_t ci = hist - 1u;
            const bool has = kBPos * wave < he - G.hb;
            if (has) {
                const float4 q4 = dlive ? *reinterpret_cast<const float4*>(q_s + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                const float q[4] = {q4.x, q4.y, q4.z, q4.w};
                KvReg kc, vc;   // the current position's key and value as the cache holds them
                {
                    const float4 k4 = dlive ? *reinterpret_cast<const float4*>(kv_s + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    const float4 v4 = dlive ? *reinterpret_cast<const float4*>(kv_s + hd + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if constexpr (KVH) {
                        auto pack = [](float a, float b) {
                            return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(a))) |
                                   (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(b))) << 16);
                        };
                        kc = v2u{pack(k4.x, k4.y), pack(k4.z, k4.w)};
                        vc = v2u{pack(v4.x, v4.y), pack(v4.z, v4.w)};
                    } else {
                        kc = v4u{__float_as_uint(k4.x), __float_as_uint(k4.y), __float_as_uint(k4.z), __float_as_uint(k4.w)};
                        vc = v4u{__float_as_uint(v4.x), __float_as_uint(v4.y), __float_as_uint(v4.z), __float_as_uint(v4.w)};
                    }
                }
                // the current position replaces its register row (ci in this wave's first group)
                if (ci >= G.hb + kBPos * wave && ci < G.hb + kBPos * wave + kBPos) {
                    const uint32_t cs = ci - G.hb - kBPos * wave;
#pragma unroll
                    for (uint32_t i = 0; i < kBPos; ++i)
                        if (i == cs) { kr[i] = kc; vr[i] = vc; }
                }
                // online softmax of the wave's positions, one pass of eight at a time: running
                // maximum wm, sum wl and accumulator wacc over this lane's four dims (the first pass
                // leaves exactly that pass's softmax terms: alpha = 0 against wl = wacc = 0)
                float wm = -INFINITY, wl = 0.0f, wacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                const uint32_t pl = lane & 7u;
                auto pass = [&](const KvReg (&kk)[kBPos], const KvReg (&vv)[kBPos], uint32_t b0) {
                    float sp[kBPos];
#pragma unroll
                    for (uint32_t i = 0; i < kBPos; ++i) {
                        float p = q[0] * kv_el(kk[i], 0);
#pragma unroll
                        for (uint32_t e = 1; e < 4u; ++e) p = fmaf(q[e], kv_el(kk[i], e), p);
                        sp[i] = p;
                    }
                    const float st = wave_sum8_t(sp);
                    const float sl = b0 + pl < he ? st * g_tk.attn_scale : -INFINITY;
                    float mx = fmaxf(sl, dpp_mov<0xB1>(sl));
                    mx = fmaxf(mx, dpp_mov<0x4E>(mx));
                    mx = fmaxf(mx, dpp_mov<0x141>(mx));
                    mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));   // >= one finite score
                    const float mn = fmaxf(wm, mx);
                    const float alpha = __expf(wm - mn);
                    const float pe = sl == -INFINITY ? 0.0f : __expf(sl - mn);
                    float pw[kBPos], ls = 0.0f;
#pragma unroll
                    for (uint32_t i = 0; i < kBPos; ++i) {
                        pw[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), i));
                        ls += pw[i];
                    }
#pragma unroll
                    for (uint32_t e = 0; e < 4u; ++e) {
                        float a = 0.0f;
#pragma unroll
                        for (uint32_t i = 0; i < kBPos; ++i) a = fmaf(pw[i], kv_el(vv[i], e), a);
                        wacc[e] = wacc[e] * alpha + a;
                    }
                    wl = wl * alpha + ls;
                    wm = mn;
                };
                pass(kr, vr, G.hb + kBPos * wave);
                if (he - G.hb > kHistMax) {
                    __builtin_amdgcn_s_waitcnt(0x0F70);   // this wave's direct-to-LDS rows
                    const uint32_t lo_b = dlive ? dl * esz : 0u;
                    // the LDS rows (or the rows loaded now) replace the register rows (consumed
                    // above; the next block's are loaded after this block)
                    for (uint32_t b0 = G.hb + kHistMax + kBPos * wave; b0 < he; b0 += kHistMax) {
                        const uint32_t j0 = b0 - G.hb - kHistMax;   // LDS row of the group's first position
                        if (j0 < hist_lds) {
#pragma unroll
                            for (uint32_t i = 0; i < kBPos; ++i) {
                                const uint32_t so = (j0 + i) * rowb + lo_b;
                                const KvReg kl = *reinterpret_cast<const KvReg*>(kvk + so);
                                const KvReg vl = *reinterpret_cast<const KvReg*>(kvv + so);
                                // rows past the share hold stale bytes: their scores are masked
                                // (each position's score sums its own products only), and zero
                                // values keep their weight-0 terms finite, as the registers'
                                // out-of-range loads do
                                kr[i] = b0 + i == ci ? kc : kl;
                                vr[i] = b0 + i == ci ? vc : (b0 + i < he ? vl : KvReg{});
                            }
                        } else if constexpr (CH) {
                            load_rows(Ly, G, b0);
#pragma unroll
                            for (uint32_t i = 0; i < kBPos; ++i)
                                if (b0 + i == ci) { kr[i] = kc; vr[i] = vc; }
                        }
                        pass(kr, vr, b0);
                    }
                }
                if (dlive) *reinterpret_cast<float4*>(part + wave * hd + dl) = make_float4(wacc[0], wacc[1], wacc[2], wacc[3]);
                if (lane == 0u) {
                    part[kWaves * hd + wave] = wm;
                    part[kWaves * hd + kWaves + wave] = wl;
                }
            }
            submark(tr && l == 1u, 5);
            __syncthreads();
            submark(tr && l == 1u, 6);
            // merge the waves in order: sum_j e^(m_j - M) acc_j and sum_j e^(m_j - M) l_j over the
            // waves that hold positions (none for an empty chunk: M = -inf, sums 0)
            const uint32_t nw = (he - G.hb + kBPos - 1u) / kBPos;
            float M = -INFINITY, num = 0.0f, den = 0.0f;
            if (tid < hd) {   // whole waves (head_dim is a multiple of 64)
                float mj[kWaves], lj[kWaves], aj[kWaves];
#pragma unroll
                for (uint32_t j = 0; j < kWaves; ++j) {
                    const bool on = j < nw;
                    mj[j] = on ? part[kWaves * hd + j] : -INFINITY;
                    lj[j] = on ? part[kWaves * hd + kWaves + j] : 0.0f;
                    aj[j] = on ? part[j * hd + tid] : 0.0f;
                }
                M = mj[0];
#pragma unroll
                for (uint32_t j = 1; j < kWaves; ++j) M = fmaxf(M, mj[j]);
#pragma unroll
                for (uint32_t j = 0; j < kWaves; ++j) {
                    const float f = j < nw ? __expf(mj[j] - M) : 0.0f;
                    num += f * aj[j];
                    den += f * lj[j];
                }
            }
            if (CH && G.chunked) {
                // the head's chunks: publish this one's {acc, M, l} (x_p[h][grp]), gather all
                // ngrp, merge them in chunk order (the same bits in every workgroup of the head)
                const uint32_t pst = hd + 8u;   // words per chunk partial (M, l at hd, hd + 1)
                u64* xp = g_tk.x_p + static_cast<uint64_t>(h) * ngrp * pst;
                const uint32_t tP = tagof(tagb, l, kTP);
                if (tid < hd) {
                    st_word(xp + grp * pst + tid, num, tP);
                    if (tid == 0u) {
                        st_word(xp + grp * pst + hd, M, tP);
                        st_word(xp + grp * pst + hd + 1u, den, tP);
                    }
                }
                submark(tr && l == 1u, 3);
                float* cp = lds<float>(g_tk.lds.kvx);   // [ngrp][hd] acc, then [ngrp][2] M, l
                const uint32_t upc = hd / 2u, nun = ngrp * upc;   // 16-byte units of the accumulators
                const __amdgpu_buffer_rsrc_t rp = rsrc(xp, ngrp * pst * 8u);
                int pfail;
                {
                    int off[kPartUnits + 1u];
                    bool which[kPartUnits + 1u], live[kPartUnits + 1u];
                    uint32_t tg[kPartUnits + 1u];
#pragma unroll
                    for (uint32_t k = 0; k < kPartUnits; ++k) {
                        const uint32_t u = tid + kThreads * k, c = u / upc, j = u % upc;
                        live[k] = u < nun;
                        which[k] = false;
                        tg[k] = tP;
                        off[k] = static_cast<int>((c * pst + 2u * j) * 8u);
                    }
                    live[kPartUnits] = tid < ngrp;   // and chunk tid's M and l
                    which[kPartUnits] = false;
                    tg[kPartUnits] = tP;
                    off[kPartUnits] = static_cast<int>((tid * pst + hd) * 8u);
                    float pv[2u * (kPartUnits + 1u)];
                    pfail = poll_units<kPartUnits + 1u>(rp, rp, off, which, live, tg, pv);
#pragma unroll
                    for (uint32_t k = 0; k < kPartUnits; ++k) {
                        const uint32_t u = tid + kThreads * k, c = u / upc, j = u % upc;
                        if (live[k]) *reinterpret_cast<float2*>(cp + c * hd + 2u * j) = make_float2(pv[2 * k], pv[2 * k + 1]);
                    }
                    if (live[kPartUnits])
                        *reinterpret_cast<float2*>(cp + ngrp * hd + 2u * tid) =
                            make_float2(pv[2 * kPartUnits], pv[2 * kPartUnits + 1]);
                }
                if (blk_any(pfail, kAnyB)) { ok = false; break; }
                submark(tr && l == 1u, 4);
                if (tid < hd) {
                    // chunk weights: lane c holds chunk c's max, weight e^(M_c - M) and l_c
                    const bool cl = lane < ngrp;
                    const float2 ml = cl ? *reinterpret_cast<const float2*>(cp + ngrp * hd + 2u * lane) : make_float2(-INFINITY, 0.0f);
                    const float Mx = wave_max(ml.x);
                    const float f = ml.x == -INFINITY ? 0.0f : __expf(ml.x - Mx);
                    const float fl = f * ml.y;
                    // sums in chunk order, four accumulator rows loaded together
                    num = 0.0f;
                    den = 0.0f;
                    auto fc = [&](float v, uint32_t c) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), c)); };
                    uint32_t c = 0;
                    for (; c + 4u <= ngrp; c += 4u) {
                        const float a0 = cp[c * hd + tid], a1 = cp[(c + 1u) * hd + tid];
                        const float a2 = cp[(c + 2u) * hd + tid], a3 = cp[(c + 3u) * hd + tid];
                        num += fc(f, c) * a0;
                        num += fc(f, c + 1u) * a1;
                        num += fc(f, c + 2u) * a2;
                        num += fc(f, c + 3u) * a3;
                        den += fc(fl, c);
                        den += fc(fl, c + 1u);
                        den += fc(fl, c + 2u);
                        den += fc(fl, c + 3u);
                    }
                    for (; c < ngrp; ++c) {
                        num += fc(f, c) * cp[c * hd + tid];
                        den += fc(fl, c);
                    }
                }
            }
            if (tid < hd) {
                const float att = num * __builtin_amdgcn_rcpf(den);
                if (tid == 0u && grp == 0u && (!(den > 0.0f) || !__builtin_isfinite(den))) flag_min(g3_code_softmax(l));   // :1666-1670
                // activation limbs of the head's 32-element blocks (each one half of a wave)
                const float mg = __builtin_isfinite(att) ? fabsf(att) : INFINITY;
                float mm = fmaxf(mg, dpp_mov<0xB1>(mg));
                mm = fmaxf(mm, dpp_mov<0x4E>(mm));
                mm = fmaxf(mm, dpp_mov<0x141>(mm));
                mm = fmaxf(mm, dpp_mov<0x140>(mm));
                const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mm), 0));
                const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mm), 16));
                const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mm), 32));
                const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mm), 48));
                mm = lane < 32u ? fmaxf(r0, r1) : fmaxf(r2, r3);
                int8_t qa = 0, qb = 0, qc = 0;
                float sb = 0.0f;
                if (mm == INFINITY) {
                    sb = __builtin_nanf("");
                } else if (mm >= 1e-30f) {
                    sb = mm * (1.0f / 127.0f);
                    limb3_r(att, 127.0f * __builtin_amdgcn_rcpf(mm), qa, qb, qc);
                }
                Lx.a[tid] = qa;
                Lx.b[tid] = qb;
                Lx.c[tid] = qc;
                if ((lane & 31u) == 0u) Lx.s[tid >> 5] = sb;
            }
            __syncthreads();
            submark(tr && l == 1u, 7);
            u64* out = g_tk.x_o + static_cast<uint64_t>(h) * d;
            const uint32_t to = tagof(tagb, l, kTO);
            XLimb xl[1];
            lane_limbs<C::SB, 1>(Lx, nbh, xl);
            batch_consume_p<C::SB, 1, 1>(orb, nbh, xl, [&](uint32_t v, float val) { st_word(out + v, val, to); });
            stamp(tr, L + l);
            if (l + 1u < L) load(l + 1u, pos);
            __syncthreads();   // LDS scratch is rewritten by the next block
        }
        if (!ok) break;
        if (s >= c.lm_from) {
            ok = phase_lm<C::SD, C::EP2, C::LMB>(tagb, tagb + nph, c.want_logits, tr);
            prev_tag = tagb + nph;
        }
        load(0, s + 1u);
        trace_end(tr);
    }
}

// ---- team D: post-attention and FFN norms, gate/up, GELU product ------------------------------

template <class C>
__device__ __attribute__((always_inline)) void team_d(uint32_t nsteps, uint32_t tag0) {
#pragma clang fp contract(off)
    nsteps = __builtin_amdgcn_readfirstlane(nsteps);
    tag0 = __builtin_amdgcn_readfirstlane(tag0);
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t m = member_of(w), ts = g_tk.tsize;
    const uint32_t d = g_tk.d, F = g_tk.F, L = g_tk.L, H = g_tk.H;
    const uint32_t nblk_d = d >> 5;
    const uint64_t rb_d = static_cast<uint64_t>(nblk_d) * 34u;
    const uint32_t nph = kTagsPerBlock * L + 1u;
    // this workgroup's 32-element blocks of g (at most one): pairs [p0, p1), rows [2 p0, 2 p1)
    uint32_t gb0, gb1, e0, e1;
    split_range(F >> 5, ts, m, gb0, gb1);
    split_lines(d, ts, m, e0, e1);
    const uint32_t p0 = 32u * gb0, p1 = 32u * gb1, v0 = 2u * p0, v1 = 2u * p1;
    const bool row_live = lane < v1 - v0;
    const DnLds t = dn_lds();
    uint8_t* scr = lds<uint8_t>(g_tk.lds.scr) + wave * C::KBD * kLimbBlkBytes;
    bool plive;
    uint32_t pnb;
    const uint32_t pb = dn_pair(nblk_d, plive, pnb);
    RowK<C::KBD> rb;
    float2 wp = make_float2(0.0f, 0.0f), wn = make_float2(0.0f, 0.0f);
    auto load = [&](uint32_t l) {
        const Layer& Ly = g_tk_layers[l];
        const uint8_t *wg = Ly.wg, *wu = Ly.wu;
        auto rowp = [=](uint32_t v) { return ((v & 1u) ? wu : wg) + static_cast<uint64_t>(v >> 1) * rb_d; };
        rowk_load<C::KBD>(rowp, nblk_d, g_tk.arena_end, v0, v1, rb);
        wp = make_float2(gp(Ly.post_attn)[2u * pb], gp(Ly.post_attn)[2u * pb + 1u]);
        wn = make_float2(gp(Ly.ffn_norm)[2u * pb], gp(Ly.ffn_norm)[2u * pb + 1u]);
    };
    load(0);
    StepCtl c = read_ctl();
    uint32_t prev_tag = 0;
    uint32_t s = c.step0;
    bool ok = true;
    for (uint32_t si = 0; si < nsteps && ok; ++si, ++s) {
        if (c.stop || s >= g_tk.ctx_len) break;
        const bool tr = g_tk.trace_slots != 0u && si == 0u;
        const uint32_t tagb = tag0 + si * nph;
        uint32_t token;
        if (!step_token(s, prev_tag, c, ok, token)) break;
        prev_tag = 0u;
        trace_begin(tr);
        stamp(tr, 2u * L);
        for (uint32_t l = 0; l < L && ok; ++l) {
            const bool mk = tr && l == 1u;
            rowk_prep<C::KBD>(rb);
            // stage 1: h of block l (team A)
            float2 h;
            int fail = poll_pair_sum<1>(g_tk.x_h, 1u, tagof(tagb, l, kTH), pb, plive, h);
            const float q0p = wave_limbs_dot<C::KBD>(make_float2(h.x * wn.x, h.y * wn.y), plive, pnb, scr, rb, row_live);
            submark(mk, 0);
            // stage 2: y = the attention output, the per-head O partials added in head order (team B)
            float2 y;
            fail |= poll_pair_sum<kMaxHeads>(g_tk.x_o, H, tagof(tagb, l, kTO), pb, plive, y);
            submark(mk, 1);
            const float2 a = make_float2(y.x * wp.x, y.y * wp.y);
            const float q1p = wave_limbs_dot<C::KBD>(make_float2(a.x * wn.x, a.y * wn.y), plive, pnb, scr, rb, row_live);
            float syy = y.x * y.x + y.y * y.y, saa = a.x * a.x + a.y * a.y, sah = a.x * h.x + a.y * h.y,
                  shh = h.x * h.x + h.y * h.y;
            wave_sum4(syy, saa, sah, shh);
            t.p0[wave * 64u + lane] = q0p;
            t.p1[wave * 64u + lane] = q1p;
            const bool wf = __builtin_amdgcn_ballot_w64(fail != 0) != 0u;
            if (lane == 0u) {
                *reinterpret_cast<float4*>(t.sums + 4u * wave) = make_float4(syy, saa, sah, shh);
                t.flg[wave] = wf ? 1 : 0;
            }
            submark(mk, 2);
            __syncthreads();
            float sc1, sc2;
            int anyf;
            dn_scalars(t, true, sc1, sc2, anyf);
            if (anyf) { ok = false; break; }
            stamp(tr, l);
            // hm = y * (rms(y) * post_attn) + h, published for team A of block l + 1 and the LM head
            if (plive && 2u * pb >= e0 && 2u * pb < e1) {
                st_word(g_tk.x_hm + 2u * pb, a.x * sc1 + h.x, tagof(tagb, l, kTHm));
                st_word(g_tk.x_hm + 2u * pb + 1u, a.y * sc1 + h.y, tagof(tagb, l, kTHm));
            }
            if (wave == 0u && v0 < v1) {
                // row v0 + lane: rms(hm) * (rms(y) * P1 + P0); gate rows are even, up rows odd
                float r0[kWaves], r1[kWaves];
#pragma unroll
                for (uint32_t k = 0; k < kWaves; ++k) {
                    r0[k] = t.p0[k * 64u + lane];
                    r1[k] = t.p1[k * 64u + lane];
                }
                float P0 = r0[0], P1 = r1[0];
#pragma unroll
                for (uint32_t k = 1; k < kWaves; ++k) {
                    P0 += r0[k];
                    P1 += r1[k];
                }
                const float val = sc2 * (sc1 * P1 + P0);
                const float up = dpp_mov<0xB1>(val);   // even lanes: the odd neighbour's up row
                // even lane 2 j: g of pair p0 + j (shaders/gelu_mul.comp:23-31)
                const float gv = (lane & 1u) ? 0.0f : gelu_fast(val) * up;
                uint32_t wa, wb, wc;
                float sc;
                block_limbs_even(gv, wa, wb, wc, sc);
                const uint32_t tg = tagof(tagb, l, kTG);
                if ((lane & 7u) == 0u) {
                    const uint32_t k = lane >> 3;
                    u64* out = g_tk.x_g + p0;
                    st_bits(out + k, wa, tg);
                    st_bits(out + 8u + k, wb, tg);
                    st_bits(out + 16u + k, wc, tg);
                    st_bits(out + 24u + k, k == 0u ? __float_as_uint(sc) : 0u, tg);
                }
            }
            (void)row_live;
            stamp(tr, L + l);
            __syncthreads();   // the wave totals are rewritten by the next block
            if (l + 1u < L) load(l + 1u);
        }
        if (!ok) break;
        if (s >= c.lm_from) {
            ok = phase_lm<C::SD, C::EP2, C::LMB>(tagb, tagb + nph, c.want_logits, tr);
            prev_tag = tagb + nph;
        }
        load(0);
        trace_end(tr);
    }
}

// ---- team E: down projection -------------------------------------------------------------------

template <class C>
__device__ __attribute__((always_inline)) void team_e(uint32_t nsteps, uint32_t tag0) {
#pragma clang fp contract(off)
    nsteps = __builtin_amdgcn_readfirstlane(nsteps);
    tag0 = __builtin_amdgcn_readfirstlane(tag0);
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t m = member_of(w), ts = g_tk.tsize;
    const uint32_t d = g_tk.d, F = g_tk.F, L = g_tk.L;
    const uint32_t nblk_f = F >> 5;
    const uint64_t rb_f = static_cast<uint64_t>(nblk_f) * 34u;
    const uint32_t nph = kTagsPerBlock * L + 1u;
    uint32_t r0, r1;
    split_lines(d, ts, m, r0, r1);
    float* x = lds<float>(g_tk.lds.x);
    RowBatch<C::SE, C::NBE, C::UE> rb;
    auto load = [&](uint32_t l) {
        const uint8_t* wd = g_tk_layers[l].wd;
        auto rowp = [=](uint32_t v) { return wd + static_cast<uint64_t>(v) * rb_f; };
        batch_load<C::SE, C::NBE, C::UE>(rowp, nblk_f, g_tk.arena_end, r0, r1, wave, kWaves, rb);
    };
    load(0);
    StepCtl c = read_ctl();
    uint32_t prev_tag = 0;
    uint32_t s = c.step0;
    bool ok = true;
    for (uint32_t si = 0; si < nsteps && ok; ++si, ++s) {
        if (c.stop || s >= g_tk.ctx_len) break;
        const bool tr = g_tk.trace_slots != 0u && si == 0u;
        const uint32_t tagb = tag0 + si * nph;
        uint32_t token;
        if (!step_token(s, prev_tag, c, ok, token)) break;
        prev_tag = 0u;
        trace_begin(tr);
        stamp(tr, 2u * L);
        for (uint32_t l = 0; l < L && ok; ++l) {
            batch_prep<C::SE, C::NBE, C::UE>(rb);
            constexpr int GP = 2;   // F <= 2048: two 16-byte pairs per thread
            // g as activation limbs: 32 tagged words per 32-element block (team D)
            if (!gather_img<GP>(g_tk.x_g, F, tagof(tagb, l, kTG), reinterpret_cast<uint32_t*>(x), kAnyGather)) {
                ok = false;
                break;
            }
            stamp(tr, l);
            u64* out = g_tk.x_d;
            const uint32_t td = tagof(tagb, l, kTD);
            XLimb xl[C::NBE];
            {
                const uint32_t sl = lane % C::SE;
#pragma unroll
                for (int n = 0; n < C::NBE; ++n) {
                    const uint32_t b = sl + static_cast<uint32_t>(n) * C::SE;
                    if (b < nblk_f) load_limb_img(reinterpret_cast<const uint32_t*>(x), b, xl[n]);
                }
            }
            batch_consume_p<C::SE, C::NBE, C::UE>(rb, nblk_f, xl, [&](uint32_t v, float val) { st_word(out + v, val, td); });
            stamp(tr, L + l);
            if (l + 1u < L) load(l + 1u);
            __syncthreads();
        }
        if (!ok) break;
        if (s >= c.lm_from) {
            ok = phase_lm<C::SD, C::EP2, C::LMB>(tagb, tagb + nph, c.want_logits, tr);
            prev_tag = tagb + nph;
        }
        load(0);
        trace_end(tr);
    }
}

// CH: the variant for steps whose histories may exceed what a workgroup holds on chip (team B
// then splits them into chunks per head); the other variant leaves that code out, for registers.
template <class C, typename KE, bool CH>
__global__ void __launch_bounds__(kThreads, 1) k_team(uint32_t nsteps, uint32_t tag0) {
    switch (team_of(blockIdx.x)) {
    case 0: team_a<C>(nsteps, tag0); break;
    case 1: team_b<C, KE, CH>(nsteps, tag0); break;
    case 2: team_d<C>(nsteps, tag0); break;
    default: team_e<C>(nsteps, tag0); break;
    }
}

}  // namespace tk

// =============================================================================================
// Host side
// =============================================================================================

struct TkFns {
    const void* f32 = nullptr;     // histories held on chip, per KV entry type
    const void* f16 = nullptr;
    const void* bf16 = nullptr;
    const void* f32c = nullptr;    // and with chunked histories
    const void* f16c = nullptr;
    const void* bf16c = nullptr;
    uint32_t lm_blocks = 0;   // blocks per row of the matrix-core LM head (0: row-slot LM head)
};

struct TkState {
    tk::Params P{};
    std::vector<tk::Layer> layers;
    uint64_t version = 1;
    TkFns fns{};
    uint32_t grid = 0;
    uint32_t trace_slots = 0;
    uint32_t pos_limit = 0;        // steps at positions below this run here
    uint32_t hist_lds[2] = {0, 0}; // LDS history rows past the registers: fp32, 16-bit entries
    bool chunked = false;          // longer histories run as chunks per head (any position)
    bool registered = false;
    std::vector<void*> allocs;
};

template <class C>
static TkFns tk_fn() {
    return TkFns{reinterpret_cast<const void*>(&tk::k_team<C, float, false>),
                 reinterpret_cast<const void*>(&tk::k_team<C, _Float16, false>),
                 reinterpret_cast<const void*>(&tk::k_team<C, __bf16, false>),
                 reinterpret_cast<const void*>(&tk::k_team<C, float, true>),
                 reinterpret_cast<const void*>(&tk::k_team<C, _Float16, true>),
                 reinterpret_cast<const void*>(&tk::k_team<C, __bf16, true>),
                 static_cast<uint32_t>(C::LMB)};
}

// Instantiated shapes: (d, heads x head_dim, FFN) -> row slots, passes and residual pairs.
static TkFns tk_pick(uint32_t d, uint32_t H, uint32_t hd, uint32_t F) {
    using namespace tk;
    // Gemma-3-270M: d 640 (20 blocks: 32-lane slots), Wo over one 256-wide head (8 blocks), FFN 2048
    if (d == 640 && H == 4 && hd == 256 && F == 2048) return tk_fn<Cfg<32, 2, 8, 32, 3, 64, 1, 2, 5, 20>>();
    // test shape: d 128 (4 blocks), 2 x 64 heads (2 blocks), FFN 256 (8 blocks)
    if (d == 128 && H == 2 && hd == 64 && F == 256) return tk_fn<Cfg<4, 1, 2, 4, 1, 8, 1, 1, 1>>();
    return TkFns{};
}

static int tk_alloc(TkState* tk, hipStream_t stream, size_t bytes, void** out) {
    void* p = nullptr;
    VRT_HIP_CHECK(hipMalloc(&p, bytes + 256));
    tk->allocs.push_back(p);
    VRT_HIP_CHECK(hipMemsetAsync(p, 0, bytes + 256, stream));   // on the context's stream, as every later use
    VRT_HIP_CHECK(hipStreamSynchronize(stream));
    *out = p;
    return VRT_OK;
}

void tk_destroy(vrt_g3* g) {
    if (!g || !g->tk) return;
    (void)hipStreamSynchronize(g->ctx->stream);
    {
        CoopSlot& ds = coop_slot(g->ctx->device);
        std::lock_guard<std::mutex> lock(ds.mu);
        if (ds.owner[kCoopTeam] == g->tk) ds.owner[kCoopTeam] = nullptr;
        if (g->tk->registered && --ds.users == 0u) {
            if (ds.last) (void)hipEventDestroy(ds.last);
            ds.last = nullptr;
            ds.last_stream = nullptr;
            ds.version[kCoopMk] = 0;
            ds.version[kCoopTeam] = 0;
            ds.owner[kCoopMk] = nullptr;
        }
    }
    for (void* p : g->tk->allocs) (void)hipFree(p);
    delete g->tk;
    g->tk = nullptr;
}

uint32_t tk_pos_limit(const vrt_g3* g) { return g->tk ? g->tk->pos_limit : 0u; }

uint32_t tk_chunk_from(const vrt_g3* g) {
    if (!g->tk) return 0u;
    return g->tk->chunked ? tk::kHistMax + g->tk->P.hist_lds : g->tk->pos_limit;
}

int tk_setup(vrt_g3* g) {
    using namespace tk;
    const vrt_g3_config& c = g->cfg;
    const uint32_t d = c.embedding_length, H = c.head_count, hd = c.head_dim, F = c.feed_forward_length;
    const uint32_t qw = H * hd, nqkv = qw + 2u * hd;
    if (!g->use_persistent) return VRT_OK;
    const TkFns fns = tk_pick(d, H, hd, F);
    if (!fns.f32) return VRT_OK;
    // three blocks at least: a key/value row appended in block l is visible to the next step's
    // reads of it because the appender's later waits precede publications that those reads
    // depend on through blocks l + 1 .. l + 2
    if (c.block_count < 3u || c.block_count > kMaxLayers || H > kMaxHeads || hd % 64u != 0u || hd > 256u) return VRT_OK;
    if ((d / 32u) % 2u != 0u || (qw / 32u) % 2u != 0u || (F / 32u) % 2u != 0u) return VRT_OK;
    if (static_cast<uint64_t>(g->P.tok_embd - (g->P.arena_end - g->arena_bytes)) +
            static_cast<uint64_t>(c.vocab_size) * (d / 32u) * 34u + 16u > g->arena_bytes)
        return VRT_OK;
    int coop = 0;
    VRT_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, g->ctx->device));
    if (!coop) return VRT_OK;
    const uint32_t nwg = g->ctx->info.compute_units;
    if (nwg % 8u != 0u || nwg < 32u || nwg > 512u) return VRT_OK;
    const uint32_t ts = nwg / kTeams;
    if (ts % H != 0u || 3u * hd > 2u * kThreads || F > 2u * 2u * kThreads) return VRT_OK;

    // every member's rows fit one batch of its team's matvec
    auto max_lines = [&](uint32_t total, uint32_t parts) { return ((total + kLine - 1u) / kLine + parts - 1u) / parts * kLine; };
    MvShape sd, sb, sf;
    if (!mv_shape(d, &sd) || !mv_shape(hd, &sb) || !mv_shape(F, &sf)) return VRT_OK;
    // capacity (rows) of one batch: waves x rows per wave x passes, read back from the template
    // (teams A and D: one row per lane, at most kbd K blocks of d per wave; team D: at most one
    // 32-element block of g per workgroup)
    struct Caps { uint32_t a, b, kbd, e; };
    Caps caps{};
    if (d == 640) caps = Caps{32u, kWaves * 8u, 3u, kWaves * 1u * 2u};
    else caps = Caps{32u, kWaves * 32u, 1u, kWaves * 8u * 1u};
    if (max_lines(nqkv, ts) > caps.a || max_lines(d, ts / H) > caps.b || F / 32u > ts ||
        (d / 32u + kWaves - 1u) / kWaves > caps.kbd || max_lines(d, ts) > caps.e)
        return VRT_OK;

    auto* tk = new (std::nothrow) TkState();
    VRT_REQUIRE(tk != nullptr, "out of memory");
    g->tk = tk;
    Params& P = tk->P;
    P.d = d; P.H = H; P.hd = hd; P.F = F; P.V = c.vocab_size; P.L = c.block_count; P.ctx_len = c.context_length;
    P.eos = g->P.eos;
    P.eps = g->P.eps; P.emb_scale = g->P.emb_scale; P.attn_scale = g->P.attn_scale;
    P.nwg = nwg;
    P.tsize = ts;
    const uint64_t rb = static_cast<uint64_t>(d / 32u) * 34u;
    {   // whole passes of the LM-head loop per tile
        const uint32_t ls = sd.S >= 32 ? sd.S / 2u : sd.S, rpp = kWaves * (64u / ls);
        uint64_t tr = (kLmTileBytes - 24u) / rb;
        if (tr >= rpp) tr = tr / rpp * rpp;
        P.lm_tile_rows = static_cast<uint32_t>(std::min<uint64_t>((c.vocab_size + nwg - 1u) / nwg, tr));
    }
    if (P.lm_tile_rows == 0u) { tk_destroy(g); return VRT_OK; }
    P.kv16 = g->P.kv16;
    P.poll_sleep = 1u;   // measured at positions 8..27: 0 and 1 fastest, 2 +1%, 8 +5%, 16 +10%

    // LDS layout
    const uint32_t kmax = std::max(std::max(d, qw), F);
    uint32_t off = 0;
    auto take = [&](uint32_t bytes) { const uint32_t o = off; off += (bytes + 15u) & ~15u; return o; };
    // x also holds team B's per-wave partials and am team B's q_h during the blocks
    P.lds.x = take(std::max(std::max(kmax, 33u * (F / 32u)), kWaves * hd + 2u * kWaves) * 4u);
    P.lds.part = P.lds.x;
    P.lds.red = take(4u * kWaves * 4u + kWaves * 4u);
    P.lds.la = take(d);
    P.lds.lb = take(d);
    P.lds.lc = take(d);
    P.lds.ls = take(d / 32u * 4u);
    P.lds.am = take(std::max(2u * nwg, hd) * 4u);
    P.lds.qkv = P.lds.am;
    P.lds.any = take(kAnySets * kWaves * 4u);
    tk->trace_slots = 2u * c.block_count + 3u + kSubMarks;
    P.lds.tr = take(tk->trace_slots * 8u);
    // the block phases' scratch (teams A and D: dn, scr; team B: the current k and v, then the
    // history rows past the registers) and the LM-head ring overlay each other: the LM head
    // follows the blocks, and a workgroup runs one team
    const uint32_t blk0 = off;
    P.lds.dn = take((2u * kWaves * 64u + 4u * kWaves + kWaves) * 4u);
    P.lds.scr = take(kWaves * 3u * kLimbBlkBytes);
    const uint32_t end_ad = off;
    off = blk0;
    P.lds.kvc = take(2u * hd * 4u);
    P.lds.kvx = off;
    // LDS history rows (key and value) for fp32 and fp16 entries: whole 1 KB loads of rows, in
    // multiples of 8 positions (one wave's share of a pass)
    for (uint32_t f = 0; f < 2u; ++f) {
        const uint32_t rowb = hd * (f ? 2u : 4u);
        tk->hist_lds[f] = 1024u % rowb == 0u && P.lds.kvx < kLdsBytes ? (kLdsBytes - P.lds.kvx) / (2u * rowb) / 8u * 8u : 0u;
    }
    off = std::max(end_ad, P.lds.kvx);
    if (fns.lm_blocks != 0u) {   // per-wave rings of 16-row tiles (waves 0 .. kLmWaves - 1)
        if (fns.lm_blocks != d / 32u || kLmWaveRows * rb + 16u > kLmWaveSlot) { tk_destroy(g); return VRT_OK; }
        off = std::max(off, blk0 + kLmWaves * kLmWaveRing * kLmWaveSlot);
    } else {
        off = std::max(off, blk0 + kLmRing * kLmTileBytes);
    }
    P.lds.ring = blk0;
    P.lds.total = off;
    if (off > kLdsBytes) { tk_destroy(g); return VRT_OK; }

    void* p;
    hipStream_t st = g->ctx->stream;
    if (int rc = tk_alloc(tk, st, d * 8u, &p)) return rc;
    P.x_h = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, nqkv * 8u, &p)) return rc;
    P.x_qkv = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, static_cast<size_t>(kMaxHeads) * d * 8u, &p)) return rc;
    P.x_o = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, d * 8u, &p)) return rc;
    P.x_hm = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, F * 8u, &p)) return rc;
    P.x_g = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, d * 8u, &p)) return rc;
    P.x_d = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, kLine * nwg * 8u, &p)) return rc;
    P.x_am = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, static_cast<size_t>(ts) * (hd + 8u) * 8u, &p)) return rc;
    P.x_p = static_cast<u64*>(p);
    if (int rc = tk_alloc(tk, st, 64, &p)) return rc;
    P.abort_flag = static_cast<uint32_t*>(p);
    if (int rc = tk_alloc(tk, st, static_cast<size_t>(nwg) * tk->trace_slots * 8u, &p)) return rc;
    P.trace = static_cast<uint64_t*>(p);
    P.trace_slots = 0u;
    std::vector<Layer> hl(c.block_count);
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const LayerParams& s = g->layers[l];
        hl[l] = Layer{s.wq, s.wk, s.wv, s.wo, s.wg, s.wu, s.wd, s.attn_norm, s.q_norm, s.k_norm, s.post_attn,
                      s.ffn_norm, s.post_ffw, s.kc, s.vc, s.slots, s.global};
    }
    tk->layers = hl;
    P.tok_embd = g->P.tok_embd;
    P.arena_end = g->P.arena_end;
    P.out_norm = g->out_norm_dev;
    P.cos_l = g->P.cos_l; P.sin_l = g->P.sin_l; P.cos_g = g->P.cos_g; P.sin_g = g->P.sin_g;
    P.st = g->P.st;
    P.tokens = g->P.tokens;
    P.results = g->P.results;
    P.logits = g->P.logits;
    P.hidden = g->P.hidden;
    for (const void* fn : {fns.f32, fns.f16, fns.bf16, fns.f32c, fns.f16c, fns.bf16c}) {
        int per_cu = 0;
        VRT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, 0));
        if (per_cu < 1) { tk_destroy(g); return VRT_OK; }
    }
    tk->fns = fns;
    tk->grid = nwg;
    P.hist_lds = tk->hist_lds[P.kv16 ? 1 : 0];
    // longer histories split into ts / H chunks per head when a workgroup can gather a head's
    // chunk partials (kPartUnits accumulator polls per thread, one more for M and l) and hold
    // them in the LDS history rows
    const uint32_t ngrp = ts / H;
    tk->chunked = ngrp * (hd / 2u) <= kPartUnits * kThreads && ngrp <= kMaxTeamChunks &&
                  P.lds.kvx + ngrp * (hd + 2u) * 4u <= kLdsBytes;
    tk->pos_limit = tk->chunked ? c.context_length : std::min(c.context_length, kHistMax + P.hist_lds);
    g->tk_tag = 1u;
    {
        CoopSlot& ds = coop_slot(g->ctx->device);
        std::lock_guard<std::mutex> lock(ds.mu);
        ++ds.users;
        tk->registered = true;
    }
    return VRT_OK;
}

int tk_set_trace(vrt_g3* g, bool on) {
    if (!g->tk) return VRT_OK;
    g->tk->P.trace_slots = on ? g->tk->trace_slots : 0u;
    ++g->tk->version;
    return VRT_OK;
}

int tk_set_kv_format(vrt_g3* g, uint32_t fmt) {
    if (!g->tk) return VRT_OK;
    g->tk->P.kv16 = fmt;
    g->tk->P.hist_lds = g->tk->hist_lds[fmt != 0u ? 1 : 0];
    g->tk->pos_limit = g->tk->chunked ? g->cfg.context_length
                                      : std::min(g->cfg.context_length, tk::kHistMax + g->tk->P.hist_lds);
    ++g->tk->version;
    return VRT_OK;
}

int tk_read_trace(vrt_g3* g, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots) {
    VRT_REQUIRE(g->tk, "team decode kernel unavailable");
    const uint64_t n = static_cast<uint64_t>(g->tk->grid) * g->tk->trace_slots;
    *nwg = g->tk->grid;
    *slots = g->tk->trace_slots;
    VRT_REQUIRE(cap >= n, "trace buffer too small: %llu entries needed", static_cast<unsigned long long>(n));
    VRT_HIP_CHECK(hipMemcpyAsync(out, g->tk->P.trace, n * 8u, hipMemcpyDeviceToHost, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

int tk_read_abort(vrt_g3* g, uint32_t* dst) {
    VRT_HIP_CHECK(hipMemcpyAsync(dst, g->tk->P.abort_flag, 4, hipMemcpyDeviceToHost, g->ctx->stream));
    return VRT_OK;
}

int tk_clear_abort(vrt_g3* g) {
    if (!g->tk) return VRT_OK;
    VRT_HIP_CHECK(hipMemsetAsync(g->tk->P.abort_flag, 0, 4, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

int tk_run(vrt_g3* g, uint32_t nsteps, bool chunked) {
    TkState* tk = g->tk;
    if (nsteps == 0) return VRT_OK;
    const uint32_t nph = tk::kTagsPerBlock * g->cfg.block_count + 1u;
    if (static_cast<uint64_t>(g->tk_tag) + static_cast<uint64_t>(nsteps + 1u) * nph >= 0xfff00000ull) {
        // tags only grow; on wrap clear every exchange buffer and start again
        VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
        const tk::Params& P = tk->P;
        const uint32_t nqkv = P.H * P.hd + 2u * P.hd;
        for (auto pr : {std::make_pair(static_cast<void*>(P.x_h), P.d), std::make_pair(static_cast<void*>(P.x_qkv), nqkv),
                        std::make_pair(static_cast<void*>(P.x_o), tk::kMaxHeads * P.d),
                        std::make_pair(static_cast<void*>(P.x_hm), P.d), std::make_pair(static_cast<void*>(P.x_g), P.F),
                        std::make_pair(static_cast<void*>(P.x_d), P.d),
                        std::make_pair(static_cast<void*>(P.x_am), tk::kLine * tk->grid),
                        std::make_pair(static_cast<void*>(P.x_p), P.tsize * (P.hd + 8u))})
            VRT_HIP_CHECK(hipMemsetAsync(pr.first, 0, static_cast<size_t>(pr.second) * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
        g->tk_tag = 1u;
    }
    uint32_t tag0 = g->tk_tag;
    hipStream_t stream = g->ctx->stream;
    CoopSlot& ds = coop_slot(g->ctx->device);
    std::lock_guard<std::mutex> lock(ds.mu);
    if (ds.last && ds.last_stream != stream) VRT_HIP_CHECK(hipStreamWaitEvent(stream, ds.last, 0));
    if (ds.owner[kCoopTeam] != tk || ds.version[kCoopTeam] != tk->version) {
        VRT_HIP_CHECK(hipMemcpyToSymbolAsync(HIP_SYMBOL(tk::g_tk), &tk->P, sizeof(tk::Params), 0, hipMemcpyHostToDevice, stream));
        VRT_HIP_CHECK(hipMemcpyToSymbolAsync(HIP_SYMBOL(tk::g_tk_layers), tk->layers.data(),
                                             tk->layers.size() * sizeof(tk::Layer), 0, hipMemcpyHostToDevice, stream));
        ds.owner[kCoopTeam] = tk;
        ds.version[kCoopTeam] = tk->version;
    }
    void* args[] = {&nsteps, &tag0};
    const TkFns& F = tk->fns;
    const void* fn = tk->P.kv16 == 2u ? (chunked ? F.bf16c : F.bf16)
                                      : (tk->P.kv16 ? (chunked ? F.f16c : F.f16) : (chunked ? F.f32c : F.f32));
    const hipError_t le = hipLaunchCooperativeKernel(fn, dim3(tk->grid),
                                                     dim3(tk::kThreads), args, 0, stream);
    if (le == hipErrorIllegalState || le == hipErrorCooperativeLaunchTooLarge) {
        (void)hipGetLastError();
        return kMkRefused;
    }
    if (le != hipSuccess)
        return set_error(VRT_ERR_HIP, "hipLaunchCooperativeKernel (team decode) failed: %s", hipGetErrorString(le));
    if (!ds.last) VRT_HIP_CHECK(hipEventCreateWithFlags(&ds.last, hipEventDisableTiming));
    VRT_HIP_CHECK(hipEventRecord(ds.last, stream));
    ds.last_stream = stream;
    g->tk_tag += nsteps * nph;
    return VRT_OK;
}

}  // namespace vrt
