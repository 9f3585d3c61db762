// vrt_decode.hip -- persistent Gemma 3 decode kernel for gfx950 (the token loop of
// src/gemma3.cpp:1462-1882 and :2080-2149, several steps per launch).
//
// Why one kernel. A batch-1 step of the Gemma-3-270M shape is ~91 dependent phases (five per
// block plus the LM head) over small matrices (0.17-2.8 MB each). Separate kernels pay ~1.6 us
// of dispatch per phase even inside a hipGraph, and a grid barrier built on device-scope
// atomics costs 5-11 us at 256 workgroups on this part. Here every workgroup (one per CU,
// launched cooperatively so all are resident) runs the whole step and the phases hand their
// outputs to each other through "tagged" 8-byte words: {fp32 value, u32 tag} written with one
// device-coherent store and read with device-coherent loads until the tag matches. A phase's
// consumer therefore waits for exactly the data it needs, with no separate flag or barrier,
// and issues its weight loads before it starts waiting, so the HBM fetch overlaps the
// hand-off latency.
//
// Phases of block l (rows are split over workgroups; "all" = every workgroup):
//   A  all   h = RMSNorm(f_{l-1}, post_ffw) + h (or the scaled embedding row), x = RMSNorm(h,
//            attn_norm), rows of [Wq | Wk | Wv]                                   (:1511-1541)
//   B  nch   QK-norm, RoPE, KV append, attention over one chunk of the history: per head the
//            chunk max m, sum l and the unnormalised sum acc                      (:1557-1696)
//   C  nc    merge the chunks (att = sum_c e^(m_c-M) acc_c / sum_c e^(m_c-M) l_c), Wo rows
//   D  all   h = RMSNorm(o, post_attn) + h, x = RMSNorm(h, ffn_norm), gate/up row pairs,
//            g = gelu_tanh(gate) * up                                             (:1703-1801)
//   E  ne    Wd rows -> f
// Short histories (min(pos + 1, slots) <= kMkFuseHist) replace B and C with one phase on the
// first nbc workgroups: workgroup w takes query head w % H and a group of output rows, runs head
// h's attention over the whole history (the same values in every group of the head: the history
// is short, and the hand-off B -> C it saves costs more), normalises it and computes its rows of
// the O projection over head h's columns only; D adds the H per-head partials of each row in
// head order. Every workgroup then produces in A and D.
// Inside an attention workgroup the roles are split by wave, because a wave's vector-memory
// operations complete in issue order: waves 0-3 load the history's keys and values and take
// positions, waves 4 and 5 poll q and k|v and hand them over through LDS, waves 6-7 hold the
// fused phase's Wo rows. A poll thus never waits behind the key/value loads.
// After the last block every workgroup folds f into h; when the step runs the LM head all of
// them stream an even share of the tied Q8_0 table (staged through LDS with 16-byte loads),
// keep a local greedy argmax and publish it; the next step (or workgroup 0 at the end of the
// launch) reduces the partials with the argmax rule of shaders/argmax.comp:30-43.
//
// Every workgroup keeps its own copy of the residual stream h in LDS. All copies are computed
// by the same code from the same exchanged inputs, so they are bitwise identical and h itself
// is never exchanged.
//
// Buffer reuse is safe without double buffering: a producer can only rewrite an exchange
// buffer after it has consumed data that every reader of the previous contents produced after
// reading them (each step ends with all workgroups reading f of the last block).
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

typedef unsigned long long u64;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// Address spaces. Pointers that reach device code through the parameter block are generic,
// so every access would become a FLAT instruction (slower, and it makes the compiler wait on
// both the vector-memory and the LDS counters); these casts restore global / constant
// (scalar-load) addressing.
#define VRT_AS_GLOBAL __attribute__((address_space(1)))
#define VRT_AS_CONST __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ VRT_AS_GLOBAL T* gp(T* p) { return (VRT_AS_GLOBAL T*)p; }
template <typename T>
__device__ __forceinline__ const VRT_AS_GLOBAL T* gp(const T* p) { return (const VRT_AS_GLOBAL T*)p; }
template <typename T>
__device__ __forceinline__ const VRT_AS_CONST T* cp(const T* p) { return (const VRT_AS_CONST T*)p; }

constexpr uint32_t kMkThreads = 512;         // 8 waves: two per SIMD
constexpr uint32_t kMkWaves = kMkThreads / 64;
constexpr uint32_t kVec = 4;                 // vector elements per thread (vectors <= 2048)
constexpr uint32_t kSpinLimit = 1u << 21;    // polls before a hand-off is declared lost
constexpr int kPollSleep = 4;                // s_sleep between unsuccessful polls (64 clocks each)
constexpr uint32_t kMaxChunks = 16;          // attention chunks per block
constexpr uint32_t kMaxBUnits = 64;          // attention workgroups (chunks x query heads) per block
constexpr uint32_t kLmUnits = 3;             // 16-byte LM-head loads per thread per tile
constexpr uint32_t kLmRing = 4;              // LM-head tile slots in LDS
constexpr uint32_t kLmAhead = kLmRing - 1u;  // tiles in flight while one is computed
constexpr uint32_t kLmTileBytes = kLmUnits * 512u * 16u;
constexpr uint32_t kPartRound = 24 * kMkThreads;   // attention partials gathered per wait (many chunks)
constexpr uint32_t kPartRoundS = 12 * kMkThreads;  // the same when they all fit in one smaller round
constexpr int kRsrcFlags = 0x00020000;       // raw buffer resource, 32-bit data format
// Cache policy of exchange and KV-cache accesses: system scope (sc0 sc1), coherent across the
// XCDs' L2s. (A tagged exchange among 256 workgroups takes ~2.6 us per round on MI355X with
// either system- or device-scope stores and loads.)
constexpr int kCoherent = 17;                // buffer-load aux bits: sc0 | sc1
constexpr uint32_t kMarks = 40;              // sub-phase trace marks (the last two: shader clock)
constexpr uint32_t kMkFuseHeads = 4;         // query heads of the fused attention + O phase, at most
// Histories up to this length use it: measured on the 270M shape, a step with every block fused
// takes 339 us at histories 9-28 and 365 us at 41-60 (375 and 387 us unfused), but 409 us at
// 101-164 (397 us unfused), where the redundant per-group attention costs more than the hand-off.
constexpr uint32_t kMkFuseHist = 64;

struct MkLayer {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw;
    float* kc;
    float* vc;
    uint32_t slots;
    uint32_t global;
};

// Byte offsets of the dynamic LDS carve-up. `u` is phase-local scratch shared by the
// attention partial sums (B), the gathered chunk partials (C) and the LM-head tile.
struct MkLds {
    uint32_t h, xs, xa, xd, red, any, la, lb, lc, ls, sc, mw, gu, u, tr, total;
};

constexpr uint32_t kMkLdsBytes = 144u * 1024u;   // static LDS of the persistent kernel

struct MkParams {
    uint32_t d, H, hd, F, V, L, ctx_len, eos;
    float eps, emb_scale, attn_scale;
    uint32_t nwg, nc, ne;          // workgroups: all, phase C, phase E
    uint32_t chunk_min;            // attention: positions per chunk before splitting further
    uint32_t max_chunks;           // attention: chunks per block (H * max_chunks <= kMaxBUnits)
    uint32_t lm_rows;              // LM-head rows per workgroup
    uint32_t lm_tile_rows;         // rows per LDS tile
    uint32_t trace_slots;          // phase timestamps per workgroup (0: tracing off)
    uint32_t kv16;               // KV cache entries: 0 fp32, 1 fp16, 2 bf16
    uint32_t fuse_hist;            // histories up to this length run the fused attention + O phase (0: never)
    uint32_t nbc;                  // workgroups of the fused phase (whole groups of H)
    uint32_t sh_o, sh_f;           // x_o / x_f layout: 2^sh rows per 64-byte line (2: one producer's
                                   // four rows per line, the other half unused; 3: dense)
    MkLds lds;
    const uint8_t* tok_embd;
    const uint8_t* arena_end;
    const float* out_norm;
    const float *cos_l, *sin_l, *cos_g, *sin_g;
    u64 *x_qkv, *x_part, *x_o, *x_g, *x_f, *x_am;
    u64* x_o4;                     // fused phase: the O projection's per-head partials [H][d]
    uint32_t* abort_flag;
    G3State* st;
    uint32_t* tokens;
    vrt_argmax_result* results;
    float* logits;
    float* hidden;
    uint64_t* trace;               // [nwg][trace_slots] s_memrealtime ticks of the first step
};

constexpr uint32_t kMkMaxLayers = 64;

// The parameter block of the launch in flight, in constant memory: every access is a scalar
// load through the scalar cache (no pointer chase through global memory on the critical path).
// One block per device: persistent launches of different executors are serialised by the host.
__constant__ MkParams g_mk;
__constant__ MkLayer g_mk_layers[kMkMaxLayers];

__shared__ __align__(16) unsigned char g_mk_lds[kMkLdsBytes];

// Workgroup OR of `pred` behind one plain barrier: each wave's ballot goes to its word of flag
// set `id` in LDS, every thread reads the set after the barrier. (HIP's __syncthreads_or is a
// generic reduction that reads the dispatch packet and takes three barriers.) A set is rewritten
// only by the next use of the same call site, after other barriers, so no reader sees it change.
constexpr uint32_t kAnySets = 8;
__device__ __forceinline__ bool blk_any(int pred, uint32_t id) {
    uint32_t* f = reinterpret_cast<uint32_t*>(g_mk_lds + g_mk.lds.any) + id * kMkWaves;
    const bool wa = __builtin_amdgcn_ballot_w64(pred != 0) != 0u;
    if ((threadIdx.x & 63u) == 0u) f[threadIdx.x >> 6] = wa ? 1u : 0u;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (uint32_t k = 0; k < kMkWaves; ++k) r |= f[k];
    return r != 0u;
}
// call sites of blk_any (flag sets)
constexpr uint32_t kAnyGather0 = 0, kAnyGather1 = 1, kAnyGatherE = 2, kAnyArgmax = 3, kAnyB = 4;

// ---- tagged exchange -----------------------------------------------------------------------

__device__ __forceinline__ void ll_st(u64* p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(gp(p), static_cast<u64>(bits) | (static_cast<u64>(tag) << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void ll_stf(u64* p, float v, uint32_t tag) { ll_st(p, __float_as_uint(v), tag); }
// 16 bytes at byte `off` of a buffer, device-coherent (bypasses a possibly stale local L2).
__device__ __forceinline__ v4u co_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, kCoherent);
}
__device__ __forceinline__ bool mk_aborted() {
    return __hip_atomic_load(gp(g_mk.abort_flag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void mk_abort() {
    __hip_atomic_store(gp(g_mk.abort_flag), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mk_flag_min(uint32_t v) {
    __hip_atomic_fetch_min(gp(&g_mk.st->nonfinite), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 1.0f / std::sqrt(float(sum_sq / n) + eps) (src/gemma3.cpp:967-983).
__device__ __forceinline__ float mk_rms_scale(double ss, uint32_t n, float eps) {
#pragma clang fp contract(off)
    return 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(n)) + eps);
}

__device__ __forceinline__ float mk_gelu(float x) {
#pragma clang fp contract(off)
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float cubic = x * x * x;
    return 0.5f * x * (1.0f + tanhf(kSqrt2OverPi * (x + kCubic * cubic)));
}

// ---- LDS views -----------------------------------------------------------------------------

struct MkSmem {
    float* h;       // residual stream
    float* xs;      // matvec input of phases C and E
    float* xa;      // normed input of phase A and of the LM head
    float* xd;      // normed input of phase D
    LimbLds L;      // LM-head activation limbs
    float* sc;      // argmax partials (2 nwg words)
    float* mw;      // phase B/C per-head scalars
    float* gu;      // phase D gate/up values of this workgroup
    float* u;       // phase-local scratch
};

__device__ __forceinline__ MkSmem mk_smem() {
    unsigned char* smem = g_mk_lds;
    MkSmem m;
    m.h = reinterpret_cast<float*>(smem + g_mk.lds.h);
    m.xs = reinterpret_cast<float*>(smem + g_mk.lds.xs);
    m.xa = reinterpret_cast<float*>(smem + g_mk.lds.xa);
    m.xd = reinterpret_cast<float*>(smem + g_mk.lds.xd);
    m.L = LimbLds{reinterpret_cast<int8_t*>(smem + g_mk.lds.la), reinterpret_cast<int8_t*>(smem + g_mk.lds.lb),
                  reinterpret_cast<int8_t*>(smem + g_mk.lds.lc), reinterpret_cast<float*>(smem + g_mk.lds.ls)};
    m.sc = reinterpret_cast<float*>(smem + g_mk.lds.sc);
    m.mw = reinterpret_cast<float*>(smem + g_mk.lds.mw);
    m.gu = reinterpret_cast<float*>(smem + g_mk.lds.gu);
    m.u = reinterpret_cast<float*>(smem + g_mk.lds.u);
    return m;
}

__device__ __forceinline__ void split_range(uint32_t total, uint32_t parts, uint32_t idx, uint32_t& a, uint32_t& b) {
    a = static_cast<uint32_t>(static_cast<uint64_t>(total) * idx / parts);
    b = static_cast<uint32_t>(static_cast<uint64_t>(total) * (idx + 1u) / parts);
}

// As split_range, in granules of kLine words: a producer's range of tagged exchange words
// starts on a 64-byte line and no two producers write the same line. (Producers on different
// XCDs writing one line cost ~0.5 us per exchange on MI355X.)
constexpr uint32_t kLine = 8;   // tagged words per 64-byte line
__device__ __forceinline__ void split_lines(uint32_t total, uint32_t parts, uint32_t idx, uint32_t& a, uint32_t& b) {
    split_range((total + kLine - 1u) / kLine, parts, idx, a, b);
    a = min(total, a * kLine);
    b = min(total, b * kLine);
}

// Word of row v in an exchange buffer that holds 2^sh rows per 64-byte line (sh <= 3): with
// sh = 2 each producer of four rows owns a line of its own, the line's other half unused.
__device__ __forceinline__ uint32_t line_word(uint32_t v, uint32_t sh) {
    return ((v >> sh) << 3) | (v & ((1u << sh) - 1u));
}

// Attention split of a history of `hist` positions: number of chunks and chunk length.
// Chunk c runs on workgroup nwg - 1 - c; every other workgroup produces rows in phases A and
// D. So every workgroup either produces in A/D or publishes an attention chunk, which is what
// makes rewriting an exchange buffer safe once its successors' data has arrived.
__device__ __forceinline__ void attn_split(uint32_t hist, uint32_t max_chunks, uint32_t chunk_min, uint32_t& nch,
                                           uint32_t& clen) {
    // histories of 256 positions and more take chunks of at least twice chunk_min: phase C
    // gathers every chunk's partials in every one of its workgroups (at 512 positions, 8 chunks
    // of 64 measured 428 us per step at position 8192 against 444 with 16 of 32)
    if (hist >= 256u) chunk_min *= 2u;
    nch = min(max_chunks, (hist + chunk_min - 1u) / chunk_min);
    clen = (hist + nch - 1u) / nch;
}

// Attention workgroups of a block at a position: one per (chunk, query head).
__device__ __forceinline__ bool mk_fused(uint32_t slots, uint32_t pos) { return min(pos + 1u, slots) <= g_mk.fuse_hist; }
__device__ __forceinline__ uint32_t n_bunits(uint32_t slots, uint32_t pos) {
    if (mk_fused(slots, pos)) return 0u;   // the fused phase's workgroups also produce in A and D
    uint32_t nch, clen;
    attn_split(min(pos + 1u, slots), g_mk.max_chunks, g_mk.chunk_min, nch, clen);
    return nch * g_mk.H;
}

// ---- LM head tiles ---------------------------------------------------------------------------

// One 34-byte block at byte `off` (even) of an LDS tile whose base is 16-byte aligned; up to
// 4 bytes past the block are read.
__device__ __forceinline__ void q8_load_lds(const uint8_t* tile, uint32_t off, Q8Raw& r) {
    const uint32_t sh = (off + 2u) & 3u;
    const uint32_t* lb = reinterpret_cast<const uint32_t*>(tile + (off + 2u - sh));
    r.sh = sh;
    r.sbits = *reinterpret_cast<const uint16_t*>(tile + off);
#pragma unroll
    for (int j = 0; j < 9; ++j) r.d[j] = lb[j];
}

// Copies rows [r0, r1) of the LM head, as the 16-byte units of their 16-byte aligned span, into
// an LDS tile with direct global->LDS loads (unit j of the span at tile byte 16 j; pre = the
// offset of row r0 in the span). Thread t moves units t + kMkThreads k, k < kLmUnits: each
// wave's instruction writes 64 consecutive units. Branch-free: units past the span re-load its
// last unit (the host only enables this kernel when the table is followed by at least 16
// readable bytes of the arena). Non-temporal: the table is streamed once per step.
__device__ __forceinline__ uint32_t lm_tile_issue(uint32_t r0, uint32_t r1, uint64_t row_bytes, uint8_t* tile) {
    const uintptr_t s = reinterpret_cast<uintptr_t>(g_mk.tok_embd) + static_cast<uint64_t>(r0) * row_bytes;
    const uintptr_t a0 = s & ~uintptr_t(15);
    const uint32_t pre = static_cast<uint32_t>(s - a0);
    const uint64_t nbytes = pre + static_cast<uint64_t>(r1 - r0) * row_bytes;
    const uint32_t n16 = static_cast<uint32_t>((nbytes + 15u) / 16u);
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (uint32_t k = 0; k < kLmUnits; ++k) {
        const uint32_t j = threadIdx.x + k * kMkThreads;
        const uintptr_t p = a0 + static_cast<uintptr_t>(j < n16 ? j : n16 - 1u) * 16u;
        __builtin_amdgcn_global_load_lds((const VRT_AS_GLOBAL void*)p,
                                         (__attribute__((address_space(3))) void*)(tile + 16u * (k * kMkThreads + 64u * wave)),
                                         16, 0, 2 /* nt */);
    }
    return pre;
}

// Waits until this wave's LM-head tile loads issued before the last `later` tiles are complete
// (vector-memory operations complete in issue order; a later store only makes the wait longer).
__device__ __forceinline__ void lm_wait_tiles(uint32_t later) {
    static_assert(kLmUnits * (kLmAhead - 1u) <= 15u, "vmcnt immediate");
    // s_waitcnt: vmcnt in bits 3:0, expcnt (7) and lgkmcnt (15) left unconstrained
    if (later >= 2u) __builtin_amdgcn_s_waitcnt(0x0F70 | (2u * kLmUnits));
    else if (later == 1u) __builtin_amdgcn_s_waitcnt(0x0F70 | kLmUnits);
    else __builtin_amdgcn_s_waitcnt(0x0F70);
}

// =============================================================================================
// Phases (each its own function, so every phase gets the whole register budget)
// =============================================================================================

#define MK_LOCALS                                                                                            \
    const MkSmem m = mk_smem();                                                                             \
    const uint32_t w = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;                    \
    const uint32_t d = g_mk.d, H = g_mk.H, hd = g_mk.hd, F = g_mk.F, L = g_mk.L;                                           \
    const uint32_t qw = H * hd, nqkv = qw + 2u * hd, half = hd >> 1, part_stride = qw + kLine * H;             \
    const uint32_t nblk_d = d >> 5, nblk_a = qw >> 5, nblk_f = F >> 5;                                      \
    const uint64_t rb_d = static_cast<uint64_t>(nblk_d) * 34u, rb_a = static_cast<uint64_t>(nblk_a) * 34u,  \
                   rb_f = static_cast<uint64_t>(nblk_f) * 34u;                                              \
    (void)w; (void)tid; (void)lane; (void)wave; (void)d; (void)H; (void)hd; (void)F; (void)L; (void)qw;     \
    (void)nqkv; (void)half; (void)part_stride; (void)nblk_d; (void)nblk_a; (void)nblk_f; (void)rb_d;         \
    (void)rb_a; (void)rb_f

// Sub-phase mark k (< kMarks) of the traced block, in the last kMarks trace slots.
// Trace timestamps go to a per-workgroup LDS image (an LDS store does not hold up the wave's
// later vector-memory waits, as a global store would) that is copied out at the end of the step.
__device__ __forceinline__ void mk_stamp(uint32_t slot, uint64_t t) {
    reinterpret_cast<uint64_t*>(g_mk_lds + g_mk.lds.tr)[slot] = t;
}
#define MK_MARK(k)                                                                                        \
    do {                                                                                                  \
        if (tr && tid == 0u) mk_stamp(g_mk.trace_slots - kMarks + (k), __builtin_amdgcn_s_memrealtime());  \
    } while (0)

// Scalar (uniform) copies of a phase's arguments: function arguments arrive in vector
// registers, which would turn every parameter-block access into a vector load.
#define MK_UNIFORM(x) x = __builtin_amdgcn_readfirstlane(x)

#define MK_TAGS(l)                                                                                   \
    const uint32_t tA = tagb + 5u * (l) + 1u, tB = tA + 1u, tC = tA + 2u, tD = tA + 3u, tE = tA + 4u; \
    (void)tA; (void)tB; (void)tC; (void)tD; (void)tE

// Attention unit of workgroup w: units run on the last workgroups, away from the O-projection
// and down-projection workgroups (the first ones).
__device__ __forceinline__ uint32_t bunit_of(uint32_t w, uint32_t nwg) { return nwg - 1u - w; }

// Full-wave sums of N independent values (uniform results), the N DPP chains interleaved step
// by step so that each chain's hazard wait is filled by the others.
template <int N>
__device__ __forceinline__ void wave_red_sum_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_mov<0xB1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_mov<0x4E>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_mov<0x141>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_mov<0x140>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_or_zero<0x142, 0xa>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_or_zero<0x143, 0xc>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), 63));
}

// Sums v[0..7] over the wave and transposes: lane l ends with the total of v[l & 7]. Three
// exchanges inside each group of 8 lanes (lanes l and 7 - l, then l ^ 2, then l ^ 1) each
// halve the values a lane carries; lanes l ^ 8, l ^ 16 and l ^ 32 then hold the same
// position. Partners add the same two operands, so every lane of a position gets the same bits.
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

// Polls 16-byte units (two tagged words each) at byte offsets off[k] of r until both tags of
// every unit equal `tag` (or !live); out[2k], out[2k+1] get the two values of unit k. Returns
// 0, or 1 if the wait was abandoned (abort raised); the caller turns the per-thread result
// into a workgroup decision at its next barrier. The polls are system-coherent buffer loads
// (a load past the buffer's range returns 0 and is never used), backing off between rounds.
template <int MAXK>
__device__ __forceinline__ int ll_poll2(__amdgpu_buffer_rsrc_t r, const int (&off)[MAXK], const bool (&live)[MAXK],
                                        uint32_t tag, float (&out)[2 * MAXK]) {
    v4u v[MAXK];
#pragma unroll
    for (int k = 0; k < MAXK; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, off[k], 0, kCoherent);
    int fail = 0;
    uint32_t spins = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < MAXK; ++k) ready &= (v[k].y == tag && v[k].w == tag) || !live[k];
        if (ready) break;
        if ((++spins & 63u) == 0u && (spins > kSpinLimit || mk_aborted())) {
            fail = 1;
            mk_abort();
            break;
        }
        __builtin_amdgcn_s_sleep(kPollSleep);   // back off: fewer polls in flight while the data is far off
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < MAXK; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, off[k], 0, kCoherent);
    }
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        out[2 * k] = __uint_as_float(v[k].x);
        out[2 * k + 1] = __uint_as_float(v[k].z);
    }
    return fail;
}

// Gathers the tagged words src[0..n) (n even) into LDS dst[0..n), then a barrier (flag set
// any_id); false (in every thread) if abandoned. Thread t polls the 16-byte pairs
// t + kMkThreads p, p < MAXP: half the requests of word-sized polls.
template <int MAXP>
__device__ __forceinline__ bool ll_gather2(const u64* src, uint32_t n, uint32_t tag, float* dst, uint32_t any_id) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<u64*>(src), 0, static_cast<int>(n * 8u), kRsrcFlags);
    int off[MAXP];
    bool live[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        const uint32_t j = threadIdx.x + static_cast<uint32_t>(p) * kMkThreads;
        live[p] = 2u * j < n;
        off[p] = live[p] ? static_cast<int>(j * 16u) : 0x7ffffff0;   // past the buffer: no access
    }
    float v[2 * MAXP];
    const int fail = ll_poll2<MAXP>(r, off, live, tag, v);
#pragma unroll
    for (int p = 0; p < MAXP; ++p)
        if (live[p]) reinterpret_cast<float2*>(dst)[threadIdx.x + p * kMkThreads] = make_float2(v[2 * p], v[2 * p + 1]);
    return !blk_any(fail, any_id);
}

// 1.0f / std::sqrt(float(sum_sq / n) + eps) for n a power of two: sum_sq * (1/n) is the exact
// quotient, one multiply instead of the double-precision division sequence.
__device__ __forceinline__ float mk_rms_scale_pow2(double ss, uint32_t n, float eps) {
#pragma clang fp contract(off)
    return 1.0f / sqrtf(static_cast<float>(ss * (1.0 / static_cast<double>(n))) + eps);
}

// Pairwise sum of N doubles (a short dependency chain).
template <int N>
__device__ __forceinline__ double tree_sum(double (&v)[N]) {
#pragma unroll
    for (int s = 1; s < N; s *= 2)
#pragma unroll
        for (int i = 0; i + s < N; i += 2 * s) v[i] += v[i + s];
    return v[0];
}

// The eight wave totals of a workgroup reduction, summed in wave order (every thread gets the
// same bits).
__device__ __forceinline__ double sum_waves(const double* r) {
    return ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
}
static_assert(kMkWaves == 8, "sum_waves adds eight wave totals");

// Residual update and RMSNorm of the d-vector residual stream h, which every workgroup keeps in
// LDS, spread over all eight waves: thread t owns the element pairs j = t + 512 k (k < P). It
// gathers its pairs of y (two tagged words per 16-byte unit) and reads its pairs of h and of the
// norm weights (global loads issued before the gather waits); each sum of squares is a per-thread
// double sum, a DPP wave reduction and the eight wave totals through LDS behind one barrier:
//   h = y * (rms(y) * w_post) + h   if ysrc != nullptr        (src/gemma3.cpp:1703-1711, :1849-1855)
//   x = (h * rms(h)) * w_next        (INTO: rms_norm_into, :991-996, :1713-1718)
//   x = h * (rms(h) * w_next)        (!INTO: rms_norm_inplace, the output norm :1866-1868)
// with rms(v) = 1.0f / sqrtf(float(sum double(v)^2 / d) + eps) (:967-983). Each thread rewrites
// only its own pairs of h; x goes to x_lds and, if given, to x_glob. `bad` is set when h has a
// non-finite element (:1857-1863). Ends with a barrier; returns 1 if the gather was abandoned
// (the same decision in every thread).
template <int EP, bool INTO, int NP = 1>
__device__ __forceinline__ int mk_resid(const u64* ysrc, uint32_t tag, const float* w_post, const float* w_next,
                                        float* hl, float* x_lds, float* x_glob, uint32_t d, float eps, int& bad,
                                        bool tr = false, uint32_t mk0 = 31u, uint32_t nparts = 1u,
                                        uint32_t ysh = 3u) {
#pragma clang fp contract(off)
    constexpr int P = (EP * 64 + static_cast<int>(kMkThreads) - 1) / static_cast<int>(kMkThreads);
    auto mark = [&](uint32_t k) {
        if (tr && threadIdx.x == 0u)
            mk_stamp(g_mk.trace_slots - kMarks + k, __builtin_amdgcn_s_memrealtime());
    };
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t npair = d >> 1u;
    double* red = reinterpret_cast<double*>(g_mk_lds + g_mk.lds.red);   // [2][waves] totals
    int* flg = reinterpret_cast<int*>(red + 2u * kMkWaves);               // [2][waves] flags
    uint32_t j[P];
    bool live[P];
    float2 wp[P], wn[P], h[P], y[P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        j[k] = tid + kMkThreads * static_cast<uint32_t>(k);
        live[k] = j[k] < npair;
        const uint32_t jj = live[k] ? j[k] : 0u;
        wn[k] = make_float2(gp(w_next)[2u * jj], gp(w_next)[2u * jj + 1u]);
        wp[k] = make_float2(0.0f, 0.0f);
        if (ysrc) wp[k] = make_float2(gp(w_post)[2u * jj], gp(w_post)[2u * jj + 1u]);
        h[k] = live[k] ? reinterpret_cast<const float2*>(hl)[jj] : make_float2(0.0f, 0.0f);
        y[k] = make_float2(0.0f, 0.0f);
    }
    if (ysrc) {
        // y is the sum of nparts <= NP partial vectors ysrc[q * d ..], added in order q = 0, 1, ...
        // (NP == 1: element v at word line_word(v, ysh); a pair never straddles a line)
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<u64*>(ysrc), 0, static_cast<int>(NP * (d << (3u - ysh)) * 8u), kRsrcFlags);
        int off[P * NP];
        bool lv[P * NP];
#pragma unroll
        for (int k = 0; k < P; ++k)
#pragma unroll
            for (int q = 0; q < NP; ++q) {
                lv[k * NP + q] = live[k] && static_cast<uint32_t>(q) < nparts;
                off[k * NP + q] = lv[k * NP + q] ? static_cast<int>((q * d + line_word(2u * j[k], ysh)) * 8u)
                                                 : 0x7ffffff0;   // past: no access
            }
        float yv[2 * P * NP];
        const int fail = ll_poll2<P * NP>(r, off, lv, tag, yv);
#pragma unroll
        for (int k = 0; k < P; ++k) {
            y[k] = lv[k * NP] ? make_float2(yv[2 * k * NP], yv[2 * k * NP + 1]) : make_float2(0.0f, 0.0f);
#pragma unroll
            for (int q = 1; q < NP; ++q)
                if (lv[k * NP + q]) {
                    y[k].x += yv[2 * (k * NP + q)];
                    y[k].y += yv[2 * (k * NP + q) + 1];
                }
        }
        mark(mk0);
        double sq[2 * P];
#pragma unroll
        for (int k = 0; k < P; ++k) {
            sq[2 * k] = static_cast<double>(y[k].x) * static_cast<double>(y[k].x);
            sq[2 * k + 1] = static_cast<double>(y[k].y) * static_cast<double>(y[k].y);
        }
        const double s = wave_red_sum_d(tree_sum(sq));
        const bool wf = __builtin_amdgcn_ballot_w64(fail != 0) != 0u;
        if (lane == 0u) {
            red[wave] = s;
            flg[wave] = wf ? 1 : 0;
        }
        __syncthreads();
        int any = 0;
#pragma unroll
        for (uint32_t k = 0; k < kMkWaves; ++k) any |= flg[k];
        if (any) return 1;
        mark(mk0 + 1u);
        const float sc = mk_rms_scale(sum_waves(red), d, eps);
#pragma unroll
        for (int k = 0; k < P; ++k) {
            h[k].x = y[k].x * (sc * wp[k].x) + h[k].x;
            h[k].y = y[k].y * (sc * wp[k].y) + h[k].y;
        }
    }
    int nf = 0;
    double sq2[2 * P];
#pragma unroll
    for (int k = 0; k < P; ++k) {
        nf |= !__builtin_isfinite(h[k].x) || !__builtin_isfinite(h[k].y);
        sq2[2 * k] = static_cast<double>(h[k].x) * static_cast<double>(h[k].x);
        sq2[2 * k + 1] = static_cast<double>(h[k].y) * static_cast<double>(h[k].y);
    }
    const double s2 = wave_red_sum_d(tree_sum(sq2));
    const bool wnf = __builtin_amdgcn_ballot_w64(nf != 0) != 0u;
    if (lane == 0u) {
        red[kMkWaves + wave] = s2;
        flg[kMkWaves + wave] = wnf ? 1 : 0;
    }
    __syncthreads();
    int anynf = 0;
#pragma unroll
    for (uint32_t k = 0; k < kMkWaves; ++k) anynf |= flg[kMkWaves + k];
    bad = anynf;
    const float sc2 = mk_rms_scale(sum_waves(red + kMkWaves), d, eps);
    mark(mk0 + 2u);
#pragma unroll
    for (int k = 0; k < P; ++k)
        if (live[k]) {
            float2 x;
            if constexpr (INTO) {
                x.x = h[k].x * sc2 * wn[k].x;
                x.y = h[k].y * sc2 * wn[k].y;
            } else {
                x.x = h[k].x * (sc2 * wn[k].x);
                x.y = h[k].y * (sc2 * wn[k].y);
            }
            reinterpret_cast<float2*>(hl)[j[k]] = h[k];
            reinterpret_cast<float2*>(x_lds)[j[k]] = x;
            if (x_glob) {
                gp(x_glob)[2u * j[k]] = x.x;
                gp(x_glob)[2u * j[k] + 1u] = x.y;
            }
        }
    __syncthreads();   // h and x are complete for every wave
    return 0;
}

// Phase A: fold f of block l-1 into h, RMSNorm(attn_norm), rows of [Wq | Wk | Wv].
template <int SD, int EP>
__device__ __attribute__((noinline)) bool mk_phase_a(uint32_t l, uint32_t pos, uint32_t tagb, bool tr) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(l);
    MK_UNIFORM(tagb);
    MK_UNIFORM(pos);
    MK_TAGS(l);
    const MkLayer& Ly = g_mk_layers[l];
    MK_MARK(0);
    // producers: every workgroup that is not an attention chunk of this block at this position
    uint32_t v0 = 0, v1 = 0;
    const uint32_t nprod = g_mk.nwg - n_bunits(Ly.slots, pos);
    if (w < nprod) split_lines(nqkv, nprod, w, v0, v1);
    const uint8_t *wq = Ly.wq, *wk = Ly.wk, *wv = Ly.wv;
    auto rowp = [=](uint32_t v) -> const uint8_t* {
        return v < qw ? wq + static_cast<uint64_t>(v) * rb_d
                      : (v < qw + hd ? wk + static_cast<uint64_t>(v - qw) * rb_d
                                     : wv + static_cast<uint64_t>(v - qw - hd) * rb_d);
    };
    RowBatch<SD, 1, 1> rb;
    batch_load<SD, 1, 1>(rowp, nblk_d, g_mk.arena_end, v0, v1, wave, kMkWaves, rb);
    MK_MARK(1);
    int bad = 0;
    if (mk_resid<EP, true>(l > 0 ? g_mk.x_f : nullptr, tagb + 5u * (l - 1u) + 5u,
                           l > 0 ? g_mk_layers[l - 1u].post_ffw : nullptr, Ly.attn_norm, m.h, m.xa, nullptr, d,
                           g_mk.eps, bad, tr, 31u, 1u, g_mk.sh_f))
        return false;
    if (bad && w == 0 && tid == 0 && l > 0) mk_flag_min(g3_code_nonfinite(l - 1u));   // :1857-1863
    MK_MARK(3);
    u64* out = g_mk.x_qkv;
    batch_consume_x<SD, 1, 1>(rb, nblk_d, m.xa, [&](uint32_t v, float val) { ll_stf(out + v, val, tA); });
    MK_MARK(5);
    return true;
}

constexpr uint32_t kBMaxWaves = 8;                 // waves of an attention unit that take positions (at most)
constexpr uint32_t kBPos = 8;                      // positions per wave per group
constexpr uint32_t kBLongChunk = 128;              // chunks at least this long use all kBMaxWaves waves

// Phase B: one workgroup per (chunk c, query head h); waves 0..3 work (all eight for chunks of
// kBLongChunk positions or more), the others wait at the closing barrier. Lane i of a wave owns
// head dims 4i..4i+3. Every working wave gathers its lanes' q_h, k and v itself, applies
// QK-norm (src/gemma3.cpp:1045-1104) and RoPE (:1371-1424; the partner dims e +- head_dim/2
// come from another lane of the same wave), and runs an online softmax over its cached
// positions t = c0 + wave + n i of the chunk (n working waves; :1602-1696), in groups of 8 n
// positions whose K/V rows are loaded one group ahead (a short chunk is one group, loaded
// before the wait for q, k, v). A group's 8 scores per wave are reduced and transposed together, so that lane l
// holds the score of its position l & 7: the max, the exponentials and the masks are one
// lane-parallel operation per group. The current position is taken from registers by the
// wave whose turn it is. No barrier until the n partials {m, l, acc} are merged through
// LDS. Wave 0 of head 0 of
// the chunk holding the current position appends k and v to the cache (:1590-1600).
// Publishes the unnormalised partial {acc[hd] of head h, m, l} of (c, h).
// Inlined into the kernel: as a call it would save and restore callee-saved registers through
// scratch.
template <typename KE, bool fused>
__device__ __attribute__((always_inline)) bool mk_phase_b(uint32_t l, uint32_t pos, uint32_t tagb, bool tr) {
#pragma clang fp contract(off)
    constexpr bool KVH = sizeof(KE) == 2;   // 16-bit entries: KE is _Float16 or __bf16
    MK_LOCALS;
    MK_UNIFORM(l);
    MK_UNIFORM(tagb);
    MK_UNIFORM(pos);
    MK_TAGS(l);
    const MkLayer& Ly = g_mk_layers[l];
    const uint32_t hist = min(pos + 1u, Ly.slots);
    const uint32_t t_first = pos + 1u - hist;
    uint32_t nch, clen;
    attn_split(hist, g_mk.max_chunks, g_mk.chunk_min, nch, clen);
    if constexpr (fused) {   // one chunk: the whole (short) history
        nch = 1u;
        clen = hist;
    }
    const uint32_t u = fused ? w % H : bunit_of(w, g_mk.nwg);   // caller guarantees u < H * nch (fused: w < nbc)
    const uint32_t c = u / H, h = u % H;
    const uint32_t c0 = t_first + c * clen;
    const uint32_t c1 = min(pos + 1u, c0 + clen);
    const uint32_t uw = __builtin_amdgcn_readfirstlane(wave);   // scalar: positions and branches on SALU
    // waves taking positions: four (one per SIMD) for short chunks, all eight for long ones
    const uint32_t nbw = clen >= kBLongChunk ? kBMaxWaves : 4u, grp = nbw * kBPos;
    const bool worker = uw < nbw;
    // With four workers, wave 4 polls q and wave 5 polls k and v; they normalise and rotate them
    // and hand them to the workers through LDS, so the workers' key/value loads and the polls
    // wait in different waves' memory queues (a wave's vector-memory operations complete in
    // issue order), and the q and k norms run side by side. With eight workers each one polls
    // and prepares all three for itself.
    const bool shared_q = nbw < kBMaxWaves;
    const bool doq = shared_q ? uw == nbw : worker;        // polls and prepares q
    const bool dok = shared_q ? uw == nbw + 1u : worker;   // polls and prepares k and v
    const bool poller = doq || dok;
    // fused: this workgroup's O-projection rows over head h's columns, loaded before any wait, by
    // the waves past the poller when they can hold them all (8 rows each)
    const uint32_t nbh = hd >> 5;
    RowBatch<8, 1, 1> orb;
    if constexpr (fused) {
        uint32_t v0, v1;
        split_range(d, g_mk.nbc / H, w / H, v0, v1);
        const uint32_t ow0 = shared_q && v1 - v0 <= (kBMaxWaves - nbw - 2u) * 8u ? nbw + 2u : 0u;
        const uint8_t* wo = Ly.wo + static_cast<uint64_t>(h) * nbh * 34u;
        auto rowp = [=](uint32_t v) { return wo + static_cast<uint64_t>(v) * rb_a; };
        orb.live[0] = false;
        if (uw >= ow0) batch_load<8, 1, 1>(rowp, nbh, g_mk.arena_end, v0, v1, uw - ow0, kMkWaves, orb);
    }
    MK_MARK(6);
    const uint32_t dl = lane * 4u;                 // this lane's 4 head dims
    const bool dlive = dl < hd;
    const bool lo = dl < half;                     // first half of the RoPE pairs
    const uint32_t e0 = lo ? dl : dl - half;       // RoPE index of dim dl
    const int partner = static_cast<int>(lo ? lane + (half >> 2) : lane - (half >> 2));
    float* ra = m.u;                               // [kBMaxWaves][hd] partial sums
    float* rml = m.mw;                             // [kBMaxWaves] m, then [kBMaxWaves] l
    float* qsh = m.u + kBMaxWaves * hd;            // [3][hd] q, k, v handed from the poller to the workers
    int fail = 0;
    // K/V cache of this block (device-coherent accesses)
    constexpr uint32_t esz = KVH ? 2u : 4u;   // 16-bit entries: 8 bytes per lane and position
    const uint32_t kv_bytes = Ly.slots * hd * esz;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(Ly.kc, 0, kv_bytes, kRsrcFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(Ly.vc, 0, kv_bytes, kRsrcFlags);
    // cached positions [c0, cend); the current position itself comes from registers
    const uint32_t cend = c1 == pos + 1u ? pos : c1;
    // Byte offset of this lane's dims of position t, past the buffer (a load that returns
    // zeros) for dead lanes and for positions that are not valid. The positions of a chunk
    // are consecutive and fewer than `slots`, so their ring index wraps at most once.
    const uint32_t r0 = c0 % Ly.slots, row_bytes = hd * esz;
    const uint32_t lane_off = dlive ? dl * esz : 0x7ffffff0u;
    auto kv_off = [&](uint32_t t, bool valid) {
        uint32_t sl = r0 + (t - c0);
        sl = sl >= Ly.slots ? sl - Ly.slots : sl;
        return static_cast<int>((valid ? sl * row_bytes : 0x7ffffff0u) + lane_off);
    };
    // this lane's four dims of a cached position, as loaded (fp32 bits, or four fp16 halves
    // that are converted where they are used, so the prefetch of the next group does not wait)
    typedef KE half4_t __attribute__((ext_vector_type(4)));
    using KvReg = typename std::conditional<KVH, v2u, v4u>::type;
    auto kv_ld = [&](__amdgpu_buffer_rsrc_t r, int off) -> KvReg {
        if constexpr (KVH) return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCoherent);
        else return co_ld4(r, static_cast<uint32_t>(off));
    };
    auto kv_el = [](const KvReg& x, uint32_t e) -> float {
        if constexpr (KVH) return static_cast<float>(__builtin_bit_cast(half4_t, x)[e]);
        else return __uint_as_float(x[e]);
    };
    // how many of this wave's positions g0 + uw + nbw i fall below g1 (wave-uniform)
    auto nvalid = [&](uint32_t g0, uint32_t g1) { return g1 > g0 + uw ? (g1 - g0 - uw + nbw - 1u) / nbw : 0u; };
    // positions past a wave's share of a group load zeros: no branch per load, and the
    // masked positions' value rows are zeros (not stale cache entries) under weight 0
    KvReg kr[kBPos], vr[kBPos];
    if (worker) {   // this wave's K/V rows of the first group
        const uint32_t nv = nvalid(c0, min(cend, c0 + grp));
#pragma unroll
        for (uint32_t i = 0; i < kBPos; ++i) {
            const int o = kv_off(c0 + uw + nbw * i, i < nv);
            kr[i] = kv_ld(rk, o);
            vr[i] = kv_ld(rv, o);
        }
    }
    // KV append (the current position's k and v, post-norm and post-RoPE): by the poller of
    // head 0 (fused: of workgroup 0) of the chunk that holds the current position, and with
    // eight workers by wave 0 after its loop, so that no wait of the loop covers the stores.
    // Positions < pos are read from the cache by the next step only; this wave's next
    // vector-memory wait in a later phase completes the stores, and every such phase precedes
    // a publication that the next step's attention depends on (vector memory operations
    // complete in issue order), so no wait is needed here.
    const bool appender = (fused ? w == 0u : h == 0u) && c1 == pos + 1u && (shared_q ? dok : uw == 0u);
    auto append = [&](const float (&k)[4], const float (&v)[4]) {
        const uint32_t so = ((pos % Ly.slots) * hd + dl) * esz;
        if constexpr (KVH) {   // k and v are already 16-bit values: the conversion is exact
            auto pack = [](float a, float b) {
                return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(a))) |
                       (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<KE>(b))) << 16);
            };
            __builtin_amdgcn_raw_buffer_store_b64(v2u{pack(k[0], k[1]), pack(k[2], k[3])}, rk, static_cast<int>(so), 0,
                                                  kCoherent);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{pack(v[0], v[1]), pack(v[2], v[3])}, rv, static_cast<int>(so), 0,
                                                  kCoherent);
        } else {
            __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(k[0]), __float_as_uint(k[1]),
                                                       __float_as_uint(k[2]), __float_as_uint(k[3])},
                                                   rk, static_cast<int>(so), 0, kCoherent);
            __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                       __float_as_uint(v[2]), __float_as_uint(v[3])},
                                                   rv, static_cast<int>(so), 0, kCoherent);
        }
    };
    float q[4], k[4], v[4];
    if (poller) {
        // norm weights and RoPE factors of this lane's dims
        float wq[4], wk[4], cs[4], sn[4];
        {
            const VRT_AS_GLOBAL float* ct = gp(Ly.global ? g_mk.cos_g : g_mk.cos_l) + static_cast<uint64_t>(pos) * half;
            const VRT_AS_GLOBAL float* st = gp(Ly.global ? g_mk.sin_g : g_mk.sin_l) + static_cast<uint64_t>(pos) * half;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                wq[e] = dlive && doq ? gp(Ly.q_norm)[dl + e] : 0.0f;
                wk[e] = dlive && dok ? gp(Ly.k_norm)[dl + e] : 0.0f;
                cs[e] = dlive ? ct[e0 + e] : 0.0f;
                sn[e] = dlive ? st[e0 + e] : 0.0f;
            }
        }
        // q_h, k, v of this lane's dims
        float qkv[12];
        {
            const __amdgpu_buffer_rsrc_t rq =
                __builtin_amdgcn_make_buffer_rsrc(g_mk.x_qkv, 0, static_cast<int>(nqkv * 8u), kRsrcFlags);
            const int oq = static_cast<int>((h * hd + dl) * 8u), ok = static_cast<int>((qw + dl) * 8u),
                      ov = static_cast<int>((qw + hd + dl) * 8u);
            const int off[6] = {oq, oq + 16, ok, ok + 16, ov, ov + 16};
            const bool lq = dlive && doq, lk = dlive && dok;
            const bool live6[6] = {lq, lq, lk, lk, lk, lk};
            fail = ll_poll2<6>(rq, off, live6, tA, qkv);
        }
        if (tr && lane == 0u && uw == (shared_q ? nbw : 0u))
            mk_stamp(g_mk.trace_slots - kMarks + 7u, __builtin_amdgcn_s_memrealtime());
#pragma unroll
        for (uint32_t e = 0; e < 4u; ++e) {
            q[e] = dlive ? qkv[e] : 0.0f;
            k[e] = dlive ? qkv[4 + e] : 0.0f;
            v[e] = dlive ? qkv[8 + e] : 0.0f;
        }
        // QK-norm: sums of squares of q_h and of k over the wave
        auto qk_norm_rope = [&](float (&x)[4], const float (&wx)[4]) {
            double sq = 0.0;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) sq += static_cast<double>(x[e]) * static_cast<double>(x[e]);
            const float sc = mk_rms_scale_pow2(wave_red_sum_d(sq), hd, g_mk.eps);
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) x[e] = x[e] * (sc * wx[e]);   // values *= scale * weights (src/gemma3.cpp:1097-1102)
            // RoPE (NeoX halves): (a, b) = (x[e], x[e + half]) -> (a c - b s, b c + a s)
            float xo[4];
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) xo[e] = __shfl(x[e], partner);
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) x[e] = lo ? x[e] * cs[e] - xo[e] * sn[e] : x[e] * cs[e] + xo[e] * sn[e];
        };
        if (doq) qk_norm_rope(q, wq);
        if (dok) qk_norm_rope(k, wk);
        if constexpr (KVH) {   // the current position's key and value as the cache will hold them
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) {
                k[e] = static_cast<float>(static_cast<KE>(k[e]));
                v[e] = static_cast<float>(static_cast<KE>(v[e]));
            }
        }
        if (shared_q && dlive) {
            if (doq) *reinterpret_cast<float4*>(qsh + dl) = make_float4(q[0], q[1], q[2], q[3]);
            if (dok) {
                *reinterpret_cast<float4*>(qsh + hd + dl) = make_float4(k[0], k[1], k[2], k[3]);
                *reinterpret_cast<float4*>(qsh + 2u * hd + dl) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
        if (shared_q && appender && dlive && !fail) append(k, v);
    }
    if (shared_q) {   // the pollers' q, k, v reach the workers
        __syncthreads();
        if (worker) {
            const float4 q4 = dlive ? *reinterpret_cast<const float4*>(qsh + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 k4 = dlive ? *reinterpret_cast<const float4*>(qsh + hd + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 v4 =
                dlive ? *reinterpret_cast<const float4*>(qsh + 2u * hd + dl) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            q[0] = q4.x; q[1] = q4.y; q[2] = q4.z; q[3] = q4.w;
            k[0] = k4.x; k[1] = k4.y; k[2] = k4.z; k[3] = k4.w;
            v[0] = v4.x; v[1] = v4.y; v[2] = v4.z; v[3] = v4.w;
        }
    }
    MK_MARK(8);
    if (worker) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float m_run = -INFINITY, l_run = 0.0f;
        const float attn_scale = g_mk.attn_scale;
        static_assert(kBPos == 8u, "one position per lane of each group of 8 lanes");
        const uint32_t pl = lane & 7u;   // the position of this wave's group that this lane scores
        for (uint32_t g0 = c0; g0 < cend; g0 += grp) {
            const uint32_t nv = nvalid(g0, min(cend, g0 + grp));
            float part[kBPos];
#pragma unroll
            for (uint32_t i = 0; i < kBPos; ++i) {
                float p = q[0] * kv_el(kr[i], 0);
#pragma unroll
                for (uint32_t e = 1; e < 4u; ++e) p = fmaf(q[e], kv_el(kr[i], e), p);
                part[i] = p;
            }
            // lane l: the score of position g0 + uw + nbw (l & 7). The reduction runs in every
            // lane (its exchanges read all of them); the mask comes after.
            const float st = wave_sum8_t(part);
            const float sl = pl < nv ? st * attn_scale : -INFINITY;
            // the next group's keys load while this group's softmax and values run
            const uint32_t n0 = g0 + grp;
            const uint32_t nn = n0 < cend ? nvalid(n0, min(cend, n0 + grp)) : 0u;
            int no[kBPos];
            if (nn != 0u) {
#pragma unroll
                for (uint32_t i = 0; i < kBPos; ++i) {
                    no[i] = kv_off(n0 + uw + nbw * i, i < nn);
                    kr[i] = kv_ld(rk, no[i]);
                }
            }
            if (nv != 0u) {   // this wave has a position in the group
                float mx = fmaxf(sl, dpp_mov<0xB1>(sl));
                mx = fmaxf(mx, dpp_mov<0x4E>(mx));
                mx = fmaxf(mx, dpp_mov<0x141>(mx));
                mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mx)));
                const float m_new = fmaxf(m_run, mx);
                if (m_new != -INFINITY) {
                    // softmax weights through the hardware exp2 (__expf): arguments are <= 0 after
                    // the max subtraction, the weights' relative error stays near 1e-6
                    const float r = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
                    const float pe = sl == -INFINITY ? 0.0f : __expf(sl - m_new);
                    float pw[kBPos];
                    float ls = 0.0f;
#pragma unroll
                    for (uint32_t i = 0; i < kBPos; ++i) {
                        pw[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), i));
                        ls += pw[i];
                    }
#pragma unroll
                    for (uint32_t e = 0; e < 4u; ++e) {
                        float a = acc[e] * r;
#pragma unroll
                        for (uint32_t i = 0; i < kBPos; ++i) a = fmaf(pw[i], kv_el(vr[i], e), a);
                        acc[e] = a;
                    }
                    l_run = l_run * r + ls;
                    m_run = m_new;
                }
            }
            if (nn != 0u) {
#pragma unroll
                for (uint32_t i = 0; i < kBPos; ++i) vr[i] = kv_ld(rv, no[i]);
            }
        }
        // the current position, from registers, by the wave whose turn it is
        if (c1 == pos + 1u && uw == (pos - c0) % nbw) {
            float sp[1] = {0.0f};
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e) sp[0] += q[e] * k[e];
            wave_red_sum_n<1>(sp);
            const float sc = sp[0] * attn_scale;
            const float m_new = fmaxf(m_run, sc);
            if (m_new != -INFINITY) {
                const float r = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
                const float pw = sc == -INFINITY ? 0.0f : __expf(sc - m_new);
#pragma unroll
                for (uint32_t e = 0; e < 4u; ++e) acc[e] = acc[e] * r + pw * v[e];
                l_run = l_run * r + pw;
                m_run = m_new;
            }
        }
        if (!shared_q && appender && dlive && !fail) append(k, v);
        if (dlive) *reinterpret_cast<float4*>(ra + uw * hd + dl) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        if (lane == 0) {
            rml[uw] = m_run;
            rml[kBMaxWaves + uw] = l_run;
        }
    }
    MK_MARK(9);
    if (blk_any(fail, kAnyB)) return false;
    // merge the waves: acc = sum_w e^(m_w - M) acc_w, l = sum_w e^(m_w - M) l_w (fixed order)
    u64* part = g_mk.x_part + static_cast<uint64_t>(c) * part_stride;
    if (tid < hd) {
        // wave weights f_k = e^(m_k - M): lane k computes f_k, then every lane takes them by readlane
        const float mk = lane < nbw ? rml[lane] : -INFINITY;
        float M = fmaxf(mk, dpp_mov<0xB1>(mk));
        M = fmaxf(M, dpp_mov<0x4E>(M));
        M = fmaxf(M, dpp_mov<0x141>(M));   // lanes 0..7: the max over the waves
        static_assert(kBMaxWaves <= 8u, "DPP max over one half row (lanes past nbw hold -inf)");
        const float fk = lane < nbw && mk != -INFINITY ? __expf(mk - M) : 0.0f;
        const float lk = lane < nbw ? rml[kBMaxWaves + lane] : 0.0f;
        float f[kBMaxWaves];
#pragma unroll
        for (uint32_t k = 0; k < kBMaxWaves; ++k) f[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fk), k));
        float sacc = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kBMaxWaves; ++k)
            if (k < nbw) sacc += f[k] * ra[k * hd + tid];   // the other waves' slots are stale
        float L = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < kBMaxWaves; ++k)
            if (k < nbw) L += f[k] * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lk), k));
        if constexpr (fused) {
            // att = acc / l: phase C's merge for one chunk (its weight e^(m - m) is 1); the
            // softmax check of :1666-1670 by the first group of each head
            m.xs[tid] = sacc / L;
            if (tid == 0u && w < H && (!(L > 0.0f) || !__builtin_isfinite(L))) mk_flag_min(g3_code_softmax(l));
        } else {
            ll_stf(part + h * hd + tid, sacc, tB);
            if (tid < kLine) {   // this unit's line: m, l, then padding (every word is tagged)
                const float Mu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(M), 0));
                ll_stf(part + qw + kLine * h + tid, tid == 0u ? Mu : (tid == 1u ? L : 0.0f), tB);
            }
        }
    }
    MK_MARK(10);
    if constexpr (fused) {   // head h's share of the O projection rows: x_o4[h][row]
        __syncthreads();
        u64* out = g_mk.x_o4 + static_cast<uint64_t>(h) * d;
        batch_consume_x<8, 1, 1>(orb, nbh, m.xs, [&](uint32_t v, float val) { ll_stf(out + v, val, tC); });
        MK_MARK(14);
    }
    return true;
}

// Whether this workgroup runs an attention unit of block l at position pos.
__device__ __forceinline__ bool mk_in_b(uint32_t l, uint32_t pos) {
    return bunit_of(blockIdx.x, g_mk.nwg) < n_bunits(g_mk_layers[l].slots, pos);
}

// Phase C: merge the chunks (att = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c), Wo rows.
// Inlined into the kernel: its gather keeps many loads in flight, and as a call it would save
// and restore callee-saved registers through scratch in every block.
template <int SA>
__device__ __attribute__((always_inline)) bool mk_phase_c(uint32_t l, uint32_t pos, uint32_t tagb, bool tr) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(l);
    MK_UNIFORM(tagb);
    MK_UNIFORM(pos);
    MK_TAGS(l);
    const MkLayer& Ly = g_mk_layers[l];
    const uint32_t hist = min(pos + 1u, Ly.slots);
    uint32_t nch, clen;
    attn_split(hist, g_mk.max_chunks, g_mk.chunk_min, nch, clen);
    const uint32_t nc = g_mk.nc;
    if (w >= nc) return true;
    MK_MARK(11);
    uint32_t v0, v1;
    split_range(d, nc, w, v0, v1);
    const uint8_t* wo = Ly.wo;
    auto rowp = [=](uint32_t v) { return wo + static_cast<uint64_t>(v) * rb_a; };
    RowBatch<SA, 1, 1> rb;
    batch_load<SA, 1, 1>(rowp, nblk_a, g_mk.arena_end, v0, v1, wave, kMkWaves, rb);
    float* parts = m.u;
    const uint32_t ntot = nch * part_stride;
    if (ntot <= kPartRoundS) {   // few chunks: one round with fewer polls per thread
        if (!ll_gather2<kPartRoundS / kMkThreads / 2>(g_mk.x_part, ntot, tB, parts, kAnyGather0)) return false;
    } else {
        for (uint32_t o = 0; o < ntot; o += kPartRound)
            if (!ll_gather2<kPartRound / kMkThreads / 2>(g_mk.x_part + o, min(kPartRound, ntot - o), tB, parts + o,
                                                         (o / kPartRound) & 1u ? kAnyGather1 : kAnyGather0))
                return false;
    }
    MK_MARK(12);
    // Chunk weights: wave h < H takes head h, lane c chunk c (M, e_c = exp(m_c - M) and
    // den = sum_c double(e_c) * double(l_c) by DPP over the 16 lanes of row 0).
    float* wts = m.mw;   // [8][kMaxChunks] weights, then den [8]
    static_assert(kMaxChunks <= 16u, "one DPP row of chunks");
    if (wave < H) {
        const uint32_t h = wave;
        const bool on = lane < nch;
        const uint32_t base = (on ? lane : 0u) * part_stride;
        const float mq = on ? parts[base + qw + kLine * h] : -INFINITY;
        const float lq = parts[base + qw + kLine * h + 1u];
        float M = fmaxf(mq, dpp_mov<0xB1>(mq));
        M = fmaxf(M, dpp_mov<0x4E>(M));
        M = fmaxf(M, dpp_mov<0x141>(M));
        M = fmaxf(M, dpp_mov<0x140>(M));
        const float e = on ? __expf(mq - M) : 0.0f;
        double den = on ? static_cast<double>(e) * static_cast<double>(lq) : 0.0;
        den += dpp_d<0xB1, 0xf>(den, false);
        den += dpp_d<0x4E, 0xf>(den, false);
        den += dpp_d<0x141, 0xf>(den, false);
        den += dpp_d<0x140, 0xf>(den, false);
        if (on) wts[h * kMaxChunks + lane] = e;
        if (lane == 0u) {
            wts[8u * kMaxChunks + h] = static_cast<float>(den);
            if (!(den > 0.0) || !__builtin_isfinite(den)) mk_flag_min(g3_code_softmax(l));   // :1666-1670
        }
    }
    __syncthreads();
    // att[idx] = sum_c e_c acc_c[idx] / den, the chunks in order, four loads in flight
    for (uint32_t idx = tid; idx < qw; idx += kMkThreads) {
        const uint32_t h = idx / hd;
        const float* wh = wts + h * kMaxChunks;
        float num = 0.0f;
        uint32_t q = 0;
        for (; q + 4u <= nch; q += 4u) {
            float wv[4], av[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                wv[k] = wh[q + k];
                av[k] = parts[(q + k) * part_stride + idx];
            }
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) num += wv[k] * av[k];
        }
        for (; q < nch; ++q) num += wh[q] * parts[q * part_stride + idx];
        m.xs[idx] = num / wts[8u * kMaxChunks + h];
    }
    __syncthreads();
    MK_MARK(13);
    u64* out = g_mk.x_o;
    const uint32_t sh = g_mk.sh_o;
    batch_consume_x<SA, 1, 1>(rb, nblk_a, m.xs, [&](uint32_t v, float val) { ll_stf(out + line_word(v, sh), val, tC); });
    MK_MARK(14);
    return true;
}

// Phase D: h = RMSNorm(o, post_attn) + h, x = RMSNorm(h, ffn_norm), gate/up row pairs,
// g = gelu_tanh(gate) * up (src/gemma3.cpp:1703-1801, shaders/gelu_mul.comp:23-31).
template <int SD, int EP, bool fused>
__device__ __attribute__((noinline)) bool mk_phase_d(uint32_t l, uint32_t pos, uint32_t tagb, bool tr) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(l);
    MK_UNIFORM(tagb);
    MK_UNIFORM(pos);
    MK_TAGS(l);
    const MkLayer& Ly = g_mk_layers[l];
    MK_MARK(15);
    uint32_t p0 = 0, p1 = 0;
    const uint32_t nprod = g_mk.nwg - n_bunits(Ly.slots, pos);
    if (w < nprod) split_lines(F, nprod, w, p0, p1);
    const uint32_t v0 = 2u * p0, v1 = 2u * p1;
    const uint8_t *wg = Ly.wg, *wu = Ly.wu;
    auto rowp = [=](uint32_t v) { return ((v & 1u) ? wu : wg) + static_cast<uint64_t>(v >> 1) * rb_d; };
    RowBatch<SD, 1, 2> rb;
    batch_load<SD, 1, 2>(rowp, nblk_d, g_mk.arena_end, v0, v1, wave, kMkWaves, rb);
    // The fused phase's four partial vectors make this the block's heaviest poll (every
    // workgroup reads 4 d tagged words per round). Waiting for this wave's weight rows first
    // starts it when the partials are nearly complete, which measured faster.
    if constexpr (fused) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    int none = 0;
    if constexpr (fused) {   // the fused phase's per-head partials, added in head order
        if (mk_resid<EP, true, kMkFuseHeads>(g_mk.x_o4, tC, Ly.post_attn, Ly.ffn_norm, m.h, m.xd, nullptr, d, g_mk.eps,
                                             none, tr, 27u, H))
            return false;
    } else if (mk_resid<EP, true>(g_mk.x_o, tC, Ly.post_attn, Ly.ffn_norm, m.h, m.xd, nullptr, d, g_mk.eps, none, tr,
                                  27u, 1u, g_mk.sh_o)) {
        return false;
    }
    MK_MARK(17);
    float* gu = m.gu;
    batch_consume_x<SD, 1, 2>(rb, nblk_d, m.xd, [&](uint32_t v, float val) { gu[v - v0] = val; });
    __syncthreads();
    MK_MARK(18);
    u64* out = g_mk.x_g;
    for (uint32_t r = p0 + tid; r < p1; r += kMkThreads) {
        const uint32_t j = (r - p0) * 2u;
        ll_stf(out + r, mk_gelu(gu[j]) * gu[j + 1u], tD);
    }
    MK_MARK(19);
    return true;
}

// Phase E: down-projection rows -> f.
template <int SF>
__device__ __attribute__((noinline)) bool mk_phase_e(uint32_t l, uint32_t tagb, bool tr) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(l);
    MK_UNIFORM(tagb);
    MK_TAGS(l);
    const MkLayer& Ly = g_mk_layers[l];
    if (w >= g_mk.ne) return true;
    MK_MARK(20);
    uint32_t v0, v1;
    split_range(d, g_mk.ne, w, v0, v1);
    const uint8_t* wd = Ly.wd;
    auto rowp = [=](uint32_t v) { return wd + static_cast<uint64_t>(v) * rb_f; };
    RowBatch<SF, 1, 1> rb;
    batch_load<SF, 1, 1>(rowp, nblk_f, g_mk.arena_end, v0, v1, wave, kMkWaves, rb);
    if (!ll_gather2<kVec / 2>(g_mk.x_g, F, tD, m.xs, kAnyGatherE)) return false;
    MK_MARK(21);
    u64* out = g_mk.x_f;
    const uint32_t sh = g_mk.sh_f;
    batch_consume_x<SF, 1, 1>(rb, nblk_f, m.xs, [&](uint32_t v, float val) { ll_stf(out + line_word(v, sh), val, tE); });
    MK_MARK(22);
    return true;
}

// End of the step: fold the last block's f into h, output norm (src/gemma3.cpp:1866-1868);
// the normed hidden state goes to xs (LM head input) and, from workgroup 0, to g_mk.hidden.
// Final residual (the last block's FFN output, post-FFW norm) and output norm into m.xs
// (src/gemma3.cpp:1849-1868); workgroup 0 also writes the hidden state.
template <int EP>
__device__ __forceinline__ bool mk_fold(uint32_t tagb) {
    MK_LOCALS;
    MK_UNIFORM(tagb);
    int bad = 0;
    if (mk_resid<EP, false>(g_mk.x_f, tagb + 5u * (L - 1u) + 5u, g_mk_layers[L - 1u].post_ffw, g_mk.out_norm, m.h, m.xa,
                            w == 0 ? g_mk.hidden : nullptr, d, g_mk.eps, bad, false, 31u, 1u, g_mk.sh_f))
        return false;
    if (bad && w == 0 && tid == 0) mk_flag_min(g3_code_nonfinite(L - 1u));
    return true;
}

template <int EP>
__device__ __attribute__((noinline)) bool mk_phase_fold(uint32_t tagb) {
    MK_UNIFORM(tagb);
    return mk_fold<EP>(tagb);
}

// Tied Q8_0 LM head over this workgroup's rows, local greedy argmax published with tag tLM.
template <int SD, int EP>
__device__ __attribute__((noinline)) bool mk_phase_lm(uint32_t tagb, uint32_t tLM, uint32_t want_logits, bool tr) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(tagb);
    MK_UNIFORM(tLM);
    MK_UNIFORM(want_logits);
    __shared__ float s_v[kMkWaves];
    __shared__ uint32_t s_i[kMkWaves];
    // Tiles of TR rows are dealt round-robin: tile ti of this workgroup is tile w + ti * nwg of the
    // table, so the workgroups stream one contiguous window of the table at a time.
    const uint32_t TR = g_mk.lm_tile_rows, nwg = g_mk.nwg;
    const uint32_t tiles = (g_mk.V + TR - 1u) / TR;
    const uint32_t ntiles = w < tiles ? (tiles - w + nwg - 1u) / nwg : 0u;
    auto tile_row = [&](uint32_t ti) { return (w + ti * nwg) * TR; };
    // the first kLmAhead tiles are in flight before the final residual is gathered
    uint8_t* ring = reinterpret_cast<uint8_t*>(m.u);
    auto issue = [&](uint32_t ti) {
        const uint32_t r0 = tile_row(ti);
        return lm_tile_issue(r0, min(g_mk.V, r0 + TR), rb_d, ring + (ti % kLmRing) * kLmTileBytes);
    };
#pragma unroll
    for (uint32_t i = 0; i < kLmAhead; ++i)
        if (i < ntiles) (void)issue(i);
    if (!mk_fold<EP>(tagb)) return false;
    MK_MARK(23);
    build_limbs(m.xa, d, m.L, kMkWaves);
    // row slots of LS lanes, LNB blocks per lane: 20-block rows fill 16-lane slots with four
    // lanes holding two blocks, four rows per wave
    constexpr int LS = SD >= 32 ? SD / 2 : SD;
    constexpr int LNB = SD / LS;
    XLimb xl[LNB];
    lane_limbs<LS, LNB>(m.L, nblk_d, xl);
    MK_MARK(24);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    constexpr uint32_t RPW = 64u / LS;
    const uint32_t slot = lane / LS, sl = lane % LS;
    for (uint32_t ti = 0; ti < ntiles; ++ti) {
        const uint32_t t0 = tile_row(ti), t1 = min(g_mk.V, t0 + TR);
        const uint8_t* tile = ring + (ti % kLmRing) * kLmTileBytes;
        const uint32_t pre_cur = static_cast<uint32_t>(
            (reinterpret_cast<uintptr_t>(g_mk.tok_embd) + static_cast<uint64_t>(t0) * rb_d) & 15u);
        lm_wait_tiles(min(kLmAhead - 1u, ntiles - 1u - ti));
        // every wave's share of tile ti is in LDS, and every wave is done with tile ti - 1,
        // whose slot now takes tile ti + kLmAhead
        __syncthreads();
        if (ti + kLmAhead < ntiles) (void)issue(ti + kLmAhead);
        const uint32_t nrows = t1 - t0;
        for (uint32_t rg = wave * RPW; rg < nrows; rg += kMkWaves * RPW) {   // wave-uniform trip count
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
                if (want_logits) gp(g_mk.logits)[v] = tot;
                if (am_better(tot, v, bv, bi)) { bv = tot; bi = v; }
            }
        }
        if (ti == 0u) MK_MARK(25);
    }
    MK_MARK(26);
    wave_argmax(bv, bi);
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (uint32_t k = 1; k < kMkWaves; ++k)
            if (am_better(s_v[k], s_i[k], s_v[0], s_i[0])) { s_v[0] = s_v[k]; s_i[0] = s_i[k]; }
        ll_stf(g_mk.x_am + kLine * w, s_v[0], tLM);   // one 64-byte line per workgroup
        ll_st(g_mk.x_am + kLine * w + 1u, s_i[0], tLM);
    }
    __syncthreads();
    return true;
}

// Reduces the argmax partials tagged `tag` (every workgroup that calls it gets the same result).
struct MkArg {
    uint32_t idx;
    float val;
    bool ok;
};

// Returned by value (in registers): reference out-parameters would go through scratch.
__device__ __attribute__((noinline)) MkArg mk_reduce_argmax(uint32_t tag) {
    MK_LOCALS;
    MK_UNIFORM(tag);
    __shared__ float s_v[kMkWaves];
    __shared__ uint32_t s_i[kMkWaves];
    float* buf = m.sc;   // 2 * nwg floats
    bool good;
    {   // value and index of workgroup k: the 16-byte pair at words kLine k, kLine k + 1
        static_assert(kMkThreads >= 512u, "one pair per thread for up to 512 workgroups");
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            g_mk.x_am, 0, static_cast<int>(kLine * g_mk.nwg * 8u), kRsrcFlags);
        int off[1];
        bool live[1];
        live[0] = tid < g_mk.nwg;
        off[0] = live[0] ? static_cast<int>(tid * kLine * 8u) : 0x7ffffff0;   // past the buffer: no access
        float v[2];
        const int fail = ll_poll2<1>(r, off, live, tag, v);
        if (live[0]) {
            buf[2u * tid] = v[0];
            buf[2u * tid + 1u] = v[1];
        }
        good = !blk_any(fail, kAnyArgmax);
    }
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t k = tid; k < g_mk.nwg; k += kMkThreads) {
        const float v = buf[2u * k];
        const uint32_t i = __float_as_uint(buf[2u * k + 1u]);
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wave_argmax(bv, bi);
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    bv = s_v[0];
    bi = s_i[0];
    for (uint32_t k = 1; k < kMkWaves; ++k)
        if (am_better(s_v[k], s_i[k], bv, bi)) { bv = s_v[k]; bi = s_i[k]; }
    __syncthreads();
    return MkArg{bi, bv, good};
}

// The step embedding: dequantised row * sqrt(d) (src/gemma3.cpp:1106-1136), written to h by
// wave 0 in its pair layout.
__device__ __attribute__((noinline)) void mk_embed(uint32_t token) {
#pragma clang fp contract(off)
    MK_LOCALS;
    MK_UNIFORM(token);
    if (__builtin_amdgcn_readfirstlane(wave) == 0u) {   // wave 0 writes h
        const VRT_AS_GLOBAL uint8_t* row = gp(g_mk.tok_embd) + static_cast<uint64_t>(token) * rb_d;
        for (uint32_t j = lane; 2u * j < d; j += 64u) {
            const uint32_t i = 2u * j;
            const VRT_AS_GLOBAL uint8_t* b = row + (i >> 5) * 34u;
            const float sc = half_bits_to_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
            float2 v;
            v.x = (sc * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31u)]))) * g_mk.emb_scale;
            v.y = (sc * static_cast<float>(static_cast<int8_t>(b[3 + (i & 31u)]))) * g_mk.emb_scale;
            reinterpret_cast<float2*>(m.h)[j] = v;
        }
    }
    __syncthreads();   // the next residual fold reads h before its first barrier
}

template <int SD, int SA, int SF, int EP, typename KE>
__global__ void __launch_bounds__(kMkThreads, 1)
k_decode(uint32_t nsteps, uint32_t tag0) {
    const uint32_t w = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t L = g_mk.L;
    const uint32_t nph = 5u * L + 1u;   // tags per step

    // step state (written by the host or the previous launch before this one started)
    const uint32_t step0 = gp(g_mk.st)->step;
    uint32_t stop = gp(g_mk.st)->stop;
    const uint32_t lm_from = gp(g_mk.st)->lm_from;
    const uint32_t feed_until = gp(g_mk.st)->feed_until;
    const uint32_t want_logits = gp(g_mk.st)->want_logits;

    uint32_t prev_lm_tag = 0;     // tag of the previous step's argmax partials (0: none)
    uint32_t s = step0;
    bool ok = true;
#define MK_TRACE(k)                                                                                    \
    do {                                                                                               \
        if (g_mk.trace_slots != 0u && si == 0u && tid == 0u) mk_stamp((k), __builtin_amdgcn_s_memrealtime()); \
    } while (0)

    for (uint32_t si = 0; si < nsteps && ok; ++si, ++s) {
        if (stop || s >= g_mk.ctx_len) break;
        const uint32_t tagb = tag0 + si * nph;

        // ---- token of this step ----
        uint32_t token;
        if (prev_lm_tag != 0u) {
            const MkArg a = mk_reduce_argmax(prev_lm_tag);
            ok = a.ok;
            if (!ok) break;
            const uint32_t idx = a.idx;
            const float val = a.val;
            if (w == 0 && tid == 0) { VRT_AS_GLOBAL vrt_argmax_result* r = gp(g_mk.results) + (s - 1u); r->index = idx; r->value = val; }
            if (s >= feed_until) {
                token = idx < g_mk.V ? idx : 0u;
                if (w == 0 && tid == 0) gp(g_mk.tokens)[s] = token;
                if (idx == g_mk.eos) {   // generation ends after EOS (src/gemma3.cpp:2134-2141)
                    stop = 1u;
                    break;
                }
            } else {
                token = gp(g_mk.tokens)[s];
            }
        } else {
            token = gp(g_mk.tokens)[s];
        }
        prev_lm_tag = 0u;
        if (g_mk.trace_slots != 0u && si == 0u && tid == 0u) {   // phases a workgroup skips keep older values
            uint64_t* img = reinterpret_cast<uint64_t*>(g_mk_lds + g_mk.lds.tr);
            for (uint32_t k = 0; k < g_mk.trace_slots; ++k) img[k] = gp(g_mk.trace)[w * g_mk.trace_slots + k];
        }
        MK_TRACE(0u);
        if (g_mk.trace_slots != 0u && si == 0u && tid == 0u)   // shader-clock ticks: clock = d(memtime) / d(realtime)
            mk_stamp(g_mk.trace_slots - 2u, __builtin_amdgcn_s_memtime());
        mk_embed(token);

        for (uint32_t l = 0; l < L && ok; ++l) {
            const bool tr = g_mk.trace_slots != 0u && si == 0u && l == 1u;   // sub-phase marks of block 1
            ok = mk_phase_a<SD, EP>(l, s, tagb, tr);
            MK_TRACE(5u * l + 1u);
            // B, C and E run on a subset of the workgroups; the others skip the call (and its
            // register save/restore through scratch) entirely. Short histories run B fused
            // with the O projection on the first nbc workgroups, and no C.
            const bool fz = mk_fused(g_mk_layers[l].slots, s);
            if (fz) ok = ok && (w >= g_mk.nbc || mk_phase_b<KE, true>(l, s, tagb, tr));
            else ok = ok && (!mk_in_b(l, s) || mk_phase_b<KE, false>(l, s, tagb, tr));
            MK_TRACE(5u * l + 2u);
            ok = ok && (fz || w >= g_mk.nc || mk_phase_c<SA>(l, s, tagb, tr));
            MK_TRACE(5u * l + 3u);
            ok = ok && (fz ? mk_phase_d<SD, EP, true>(l, s, tagb, tr) : mk_phase_d<SD, EP, false>(l, s, tagb, tr));
            MK_TRACE(5u * l + 4u);
            ok = ok && (w >= g_mk.ne || mk_phase_e<SF>(l, tagb, tr));
            MK_TRACE(5u * l + 5u);
        }
        if (s >= lm_from) {   // final norm, LM head + local argmax (src/gemma3.cpp:1138-1185)
            MK_TRACE(5u * L + 1u);
            ok = ok && mk_phase_lm<SD, EP>(tagb, tagb + nph, want_logits, g_mk.trace_slots != 0u && si == 0u);
            if (!ok) break;
            prev_lm_tag = tagb + nph;
        } else {
            ok = ok && mk_phase_fold<EP>(tagb);
            if (!ok) break;
            MK_TRACE(5u * L + 1u);
        }
        MK_TRACE(5u * L + 2u);
        if (g_mk.trace_slots != 0u && si == 0u && tid == 0u) {
            mk_stamp(g_mk.trace_slots - 1u, __builtin_amdgcn_s_memtime());
            // the traced step is over: its stamps go to the trace buffer
            const uint64_t* img = reinterpret_cast<const uint64_t*>(g_mk_lds + g_mk.lds.tr);
            for (uint32_t k = 0; k < g_mk.trace_slots; ++k) gp(g_mk.trace)[w * g_mk.trace_slots + k] = img[k];
        }
    }
#undef MK_TRACE

    // ---- end of launch: workgroup 0 records the last step's result and the step state ----
    if (w == 0) {
        if (ok && prev_lm_tag != 0u) {
            const MkArg a = mk_reduce_argmax(prev_lm_tag);
            ok = a.ok;
            const uint32_t idx = a.idx;
            const float val = a.val;
            if (ok && tid == 0) {
                { VRT_AS_GLOBAL vrt_argmax_result* r = gp(g_mk.results) + (s - 1u); r->index = idx; r->value = val; }
                if (s >= feed_until) {
                    gp(g_mk.tokens)[s] = idx < g_mk.V ? idx : 0u;
                    if (idx == g_mk.eos) stop = 1u;
                }
            }
        }
        if (tid == 0) {
            gp(g_mk.st)->step = s;
            gp(g_mk.st)->stop = stop;
            if (!ok) mk_flag_min(kG3HandoffLost);
        }
    }
}

// =============================================================================================
// Host side
// =============================================================================================

struct MkFns {
    const void* f32 = nullptr;
    const void* f16 = nullptr;
    const void* bf16 = nullptr;
};

struct MkState {
    MkParams P{};
    std::vector<MkLayer> layers;   // host image of g_mk_layers
    uint64_t version = 1;          // bumped whenever P changes
    MkFns fns{};                   // k_decode for fp32, fp16 and bf16 KV entries
    size_t lds_bytes = 0;
    uint32_t grid = 0;
    uint32_t trace_slots = 0;      // slots per workgroup when tracing is enabled
    bool registered = false;       // counted in its device slot's users
    std::vector<void*> allocs;
};

// One slot per device (vrt_g3_internal.hpp): heap-allocated and never freed. The slots hold no
// HIP resource once their last executor is gone, and executors released late in process exit
// may still lock them.
CoopSlot& coop_slot(int device) {
    static CoopSlot* s = new CoopSlot[kMaxCoopDevices];
    return s[device % kMaxCoopDevices];
}

template <int SD, int SA, int SF, int EP>
static MkFns mk_fn() {
    return MkFns{reinterpret_cast<const void*>(&k_decode<SD, SA, SF, EP, float>),
                 reinterpret_cast<const void*>(&k_decode<SD, SA, SF, EP, _Float16>),
                 reinterpret_cast<const void*>(&k_decode<SD, SA, SF, EP, __bf16>)};
}

// Row-slot widths of the three matvec input lengths (d, H * head_dim, FFN) and the residual
// pairs per lane, ep = ceil(d / 128); the smallest instantiated EP >= ep is taken.
static MkFns mk_pick(int sd, int sa, int sf, int ep) {
#define VRT_MK(a, b, c, e) if (sd == a && sa == b && sf == c && ep <= e) return mk_fn<a, b, c, e>();
    VRT_MK(32, 32, 64, 5)   // Gemma-3-270M: d 640, 4 x 256 heads, FFN 2048
    VRT_MK(32, 32, 64, 8)
    VRT_MK(4, 4, 8, 1)      // d 128, 2 x 64 heads, FFN 256 (test shape)
    VRT_MK(32, 64, 64, 5)
    VRT_MK(32, 64, 64, 8)
    VRT_MK(16, 16, 32, 4)
    VRT_MK(8, 8, 16, 2)
#undef VRT_MK
    return MkFns{};
}

static int mk_alloc(MkState* mk, hipStream_t stream, size_t bytes, void** out) {
    void* p = nullptr;
    VRT_HIP_CHECK(hipMalloc(&p, bytes + 256));
    mk->allocs.push_back(p);
    // zero-filled on the context's (non-blocking) stream, which every later use is ordered on
    VRT_HIP_CHECK(hipMemsetAsync(p, 0, bytes + 256, stream));
    VRT_HIP_CHECK(hipStreamSynchronize(stream));
    *out = p;
    return VRT_OK;
}

void mk_destroy(vrt_g3* g) {
    if (!g || !g->mk) return;
    (void)hipStreamSynchronize(g->ctx->stream);   // no launch may still use the buffers freed below
    {
        CoopSlot& ds = coop_slot(g->ctx->device);
        std::lock_guard<std::mutex> lock(ds.mu);
        if (ds.owner[kCoopMk] == g->mk) ds.owner[kCoopMk] = nullptr;
        if (g->mk->registered && --ds.users == 0u) {
            // the last executor on the device: its stream is drained by the caller
            if (ds.last) (void)hipEventDestroy(ds.last);
            ds.last = nullptr;
            ds.last_stream = nullptr;
            ds.version[kCoopMk] = 0;
            ds.version[kCoopTeam] = 0;
            ds.owner[kCoopTeam] = nullptr;
        }
    }
    for (void* p : g->mk->allocs) (void)hipFree(p);
    delete g->mk;
    g->mk = nullptr;
}

int mk_setup(vrt_g3* g) {
    const vrt_g3_config& c = g->cfg;
    const uint32_t d = c.embedding_length, H = c.head_count, hd = c.head_dim, F = c.feed_forward_length;
    const uint32_t qw = H * hd;
    if (!g->use_persistent) return VRT_OK;
    if (hd % 64u != 0u || hd > 256u || H > 8u || d > 2048u || F > 2048u || qw > 2048u) return VRT_OK;
    if (c.block_count > kMkMaxLayers) return VRT_OK;
    // branch-free block loads need even block counts (no block reads past its matrix), and the
    // LM-head tile loads need 16 readable bytes after the table
    if ((d / 32u) % 2u != 0u || (qw / 32u) % 2u != 0u || (F / 32u) % 2u != 0u) return VRT_OK;
    if (static_cast<uint64_t>(g->P.tok_embd - (g->P.arena_end - g->arena_bytes)) +
            static_cast<uint64_t>(c.vocab_size) * (d / 32u) * 34u + 16u > g->arena_bytes)
        return VRT_OK;
    MvShape sd, sa, sf;
    if (!mv_shape(d, &sd) || !mv_shape(qw, &sa) || !mv_shape(F, &sf) || sd.NB != 1 || sa.NB != 1 || sf.NB != 1) return VRT_OK;
    const MkFns fns = mk_pick(sd.S, sa.S, sf.S, static_cast<int>((d + 127u) / 128u));
    if (!fns.f32) return VRT_OK;
    int coop = 0;
    VRT_HIP_CHECK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, g->ctx->device));
    if (!coop) return VRT_OK;

    auto* mk = new (std::nothrow) MkState();
    VRT_REQUIRE(mk != nullptr, "out of memory");
    g->mk = mk;
    MkParams& P = mk->P;
    const uint32_t nwg = g->ctx->info.compute_units;
    const uint32_t cap_d = kMkWaves * (64u / static_cast<uint32_t>(sd.S));
    const uint32_t cap_a = kMkWaves * (64u / static_cast<uint32_t>(sa.S));
    const uint32_t cap_f = kMkWaves * (64u / static_cast<uint32_t>(sf.S));
    const uint32_t nqkv = qw + 2u * hd;
    // every workgroup must cover its share of the all-workgroup phases in one batch
    const uint32_t max_chunks = std::min(kMaxChunks, kMaxBUnits / H);
    const uint32_t nprod = nwg - H * max_chunks;
    // most rows of one producer under the line-granular split
    auto max_rows = [&](uint32_t total, uint32_t gr) { return ((total + gr - 1u) / gr + nprod - 1u) / nprod * gr; };
    if (nwg < 2u * H * max_chunks || nwg > 512u || 3u * hd > 2u * kMkThreads || max_rows(nqkv, kLine) > cap_d ||
        max_rows(F, kLine) > cap_d || nqkv > kVec * kMkThreads) {
        mk_destroy(g);
        return VRT_OK;
    }
    P.d = d; P.H = H; P.hd = hd; P.F = F; P.V = c.vocab_size; P.L = c.block_count; P.ctx_len = c.context_length;
    P.eos = g->P.eos;
    P.eps = g->P.eps; P.emb_scale = g->P.emb_scale; P.attn_scale = g->P.attn_scale;
    P.nwg = nwg;
    // C and E: four output rows (half a 64-byte line) per workgroup: more workgroups, shorter
    // matvecs (C's workgroups stay clear of the attention units at the end)
    P.nc = std::min(nwg - H * max_chunks, (d + std::min(cap_a, kLine / 2u) - 1u) / std::min(cap_a, kLine / 2u));
    P.ne = std::min(nwg, (d + std::min(cap_f, kLine / 2u) - 1u) / std::min(cap_f, kLine / 2u));
    if ((d + P.nc - 1u) / P.nc > cap_a || (d + P.ne - 1u) / P.ne > cap_f) { mk_destroy(g); return VRT_OK; }
    // producers of exactly four rows each get a line of their own (producers on different
    // XCDs that share a line slow the exchange)
    P.sh_o = d == 4u * P.nc ? 2u : 3u;
    P.sh_f = d == 4u * P.ne ? 2u : 3u;
    {   // fused attention + O phase: nc / H row groups per head, one 64-row pass of 8-lane slots
        const uint32_t ng = P.nc / H;
        const bool ok = H <= kMkFuseHeads && ng >= 1u && (d + ng - 1u) / ng <= kMkWaves * 8u && hd / 32u <= 8u;
        P.fuse_hist = ok ? kMkFuseHist : 0u;
        P.nbc = ok ? ng * H : 0u;
    }
    P.chunk_min = 32u;
    P.max_chunks = max_chunks;
    P.lm_rows = (c.vocab_size + nwg - 1u) / nwg;
    const uint64_t rb = static_cast<uint64_t>(d / 32u) * 34u;
    {   // whole passes of the LM-head loop per tile (row slots of sd/2 lanes for 32- and 64-lane shapes)
        const uint32_t ls = sd.S >= 32 ? sd.S / 2u : sd.S, rpp = kMkWaves * (64u / ls);
        // margin: the span's alignment offset (< 16 bytes) and the 4 bytes a block read may
        // take past the last row
        uint64_t tr = (kLmTileBytes - 24u) / rb;
        if (tr >= rpp) tr = tr / rpp * rpp;
        P.lm_tile_rows = static_cast<uint32_t>(std::min<uint64_t>(P.lm_rows, tr));
    }
    if (P.lm_tile_rows == 0u) { mk_destroy(g); return VRT_OK; }
    uint32_t slots_max = 1;
    for (const auto& Ly : g->layers) slots_max = std::max(slots_max, Ly.slots);
    (void)slots_max;

    // LDS layout
    const uint32_t kmax = std::max(std::max(d, qw), F);
    uint32_t off = 0;
    auto take = [&](uint32_t bytes) { const uint32_t o = off; off += (bytes + 15u) & ~15u; return o; };
    P.lds.h = take(d * 4u);
    P.lds.xs = take(kmax * 4u);
    P.lds.xa = take(d * 4u);
    P.lds.xd = take(d * 4u);
    P.lds.red = take(2u * kMkWaves * (8u + 4u));   // residual norms: wave totals and flags, two rounds
    P.lds.any = take(kAnySets * kMkWaves * 4u);
    P.lds.la = take(d);
    P.lds.lb = take(d);
    P.lds.lc = take(d);
    P.lds.ls = take(d / 32u * 4u);
    P.lds.sc = take(2u * nwg * 4u);
    P.lds.mw = take((8u * kMaxChunks + 16u) * 4u);
    P.lds.gu = take(2u * ((F + nprod - 1u) / nprod + 1u) * 4u);
    P.lds.u = take(std::max(std::max(kMkWaves * qw, kMaxChunks * (qw + kLine * H)) * 4u, kLmRing * kLmTileBytes));
    P.lds.tr = take((5u * c.block_count + 3u + kMarks) * 8u);   // trace stamps of the traced step
    P.lds.total = off;
    mk->lds_bytes = off;
    if (off > kMkLdsBytes) { mk_destroy(g); return VRT_OK; }

    // exchange buffers
    void* p;
    if (int rc = mk_alloc(mk, g->ctx->stream, nqkv * 8u, &p)) return rc;
    P.x_qkv = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, static_cast<size_t>(kMaxChunks) * (qw + kLine * H) * 8u, &p)) return rc;
    P.x_part = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, 2u * d * 8u, &p)) return rc;   // room for the line-per-producer layout
    P.x_o = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, static_cast<size_t>(kMkFuseHeads) * d * 8u, &p)) return rc;
    P.x_o4 = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, F * 8u, &p)) return rc;
    P.x_g = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, 2u * d * 8u, &p)) return rc;
    P.x_f = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, kLine * nwg * 8u, &p)) return rc;
    P.x_am = static_cast<u64*>(p);
    if (int rc = mk_alloc(mk, g->ctx->stream, 64, &p)) return rc;
    P.abort_flag = static_cast<uint32_t*>(p);
    mk->trace_slots = 5u * c.block_count + 3u + kMarks;
    if (int rc = mk_alloc(mk, g->ctx->stream, static_cast<size_t>(nwg) * mk->trace_slots * 8u, &p)) return rc;
    P.trace = static_cast<uint64_t*>(p);
    P.trace_slots = 0u;
    std::vector<MkLayer> hl(c.block_count);
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const LayerParams& s = g->layers[l];
        hl[l] = MkLayer{s.wq, s.wk, s.wv, s.wo, s.wg, s.wu, s.wd, s.attn_norm, s.q_norm, s.k_norm, s.post_attn,
                        s.ffn_norm, s.post_ffw, s.kc, s.vc, s.slots, s.global};
    }
    mk->layers = hl;
    P.tok_embd = g->P.tok_embd;
    P.arena_end = g->P.arena_end;
    P.out_norm = g->out_norm_dev;
    P.cos_l = g->P.cos_l; P.sin_l = g->P.sin_l; P.cos_g = g->P.cos_g; P.sin_g = g->P.sin_g;
    P.st = g->P.st;
    P.tokens = g->P.tokens;
    P.results = g->P.results;
    P.logits = g->P.logits;
    P.hidden = g->P.hidden;

    for (const void* fn : {fns.f32, fns.f16, fns.bf16}) {   // every KV element type must fit a CU
        int per_cu = 0;
        VRT_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kMkThreads, 0));
        if (per_cu < 1) { mk_destroy(g); return VRT_OK; }
    }
    mk->fns = fns;
    mk->grid = nwg;
    g->mk_tag = 1u;
    {
        CoopSlot& ds = coop_slot(g->ctx->device);
        std::lock_guard<std::mutex> lock(ds.mu);
        ++ds.users;
        mk->registered = true;
    }
    return VRT_OK;
}

int mk_set_trace(vrt_g3* g, bool on) {
    VRT_REQUIRE(g->mk, "persistent decode kernel unavailable");
    g->mk->P.trace_slots = on ? g->mk->trace_slots : 0u;
    ++g->mk->version;
    return VRT_OK;
}

int mk_set_kv_format(vrt_g3* g, uint32_t fmt) {
    if (!g->mk) return VRT_OK;
    g->mk->P.kv16 = fmt;
    ++g->mk->version;
    return VRT_OK;
}

int mk_read_trace(vrt_g3* g, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots) {
    VRT_REQUIRE(g->mk, "persistent decode kernel unavailable");
    const uint64_t n = static_cast<uint64_t>(g->mk->grid) * g->mk->trace_slots;
    *nwg = g->mk->grid;
    *slots = g->mk->trace_slots;
    VRT_REQUIRE(cap >= n, "trace buffer too small: %llu entries needed", static_cast<unsigned long long>(n));
    VRT_HIP_CHECK(hipMemcpyAsync(out, g->mk->P.trace, n * 8u, hipMemcpyDeviceToHost, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

int mk_read_exchange(vrt_g3* g, uint32_t which, uint64_t* out, uint64_t cap, uint64_t* n) {
    VRT_REQUIRE(g->mk, "persistent decode kernel unavailable");
    const MkParams& P = g->mk->P;
    const uint32_t qw = P.H * P.hd;
    const u64* src = nullptr;
    uint64_t cnt = 0;
    uint32_t sh = 3u;   // rows per line of the device layout (x_o, x_f): the copy is compacted
    switch (which) {
    case 0: src = P.x_qkv; cnt = qw + 2u * P.hd; break;
    case 1: src = P.x_part; cnt = static_cast<uint64_t>(kMaxChunks) * (qw + kLine * P.H); break;
    case 2: src = P.x_o; cnt = P.d; sh = P.sh_o; break;
    case 3: src = P.x_g; cnt = P.F; break;
    case 4: src = P.x_f; cnt = P.d; sh = P.sh_f; break;
    case 5: src = P.x_am; cnt = kLine * P.nwg; break;
    default: return set_error(VRT_ERR_INVALID, "unknown exchange buffer %u", which);
    }
    *n = cnt;
    VRT_REQUIRE(cap >= cnt, "exchange buffer needs %llu words", static_cast<unsigned long long>(cnt));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    const uint64_t raw_words = cnt << (3u - sh);
    std::vector<uint64_t> raw(raw_words);
    VRT_HIP_CHECK(hipMemcpyAsync(raw.data(), src, raw_words * 8u, hipMemcpyDeviceToHost, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    for (uint64_t v = 0; v < cnt; ++v) out[v] = raw[((v >> sh) << 3) | (v & ((1u << sh) - 1u))];
    return VRT_OK;
}

int mk_read_abort(vrt_g3* g, uint32_t* dst) {
    VRT_HIP_CHECK(hipMemcpyAsync(dst, g->mk->P.abort_flag, 4, hipMemcpyDeviceToHost, g->ctx->stream));
    return VRT_OK;
}

int mk_clear_abort(vrt_g3* g) {
    if (!g->mk) return VRT_OK;
    VRT_HIP_CHECK(hipMemsetAsync(g->mk->P.abort_flag, 0, 4, g->ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
    return VRT_OK;
}

int mk_run(vrt_g3* g, uint32_t nsteps) {
    MkState* mk = g->mk;
    if (nsteps == 0) return VRT_OK;
    const uint32_t nph = 5u * g->cfg.block_count + 1u;
    // tags only grow; on wrap clear every exchange buffer and start again
    if (static_cast<uint64_t>(g->mk_tag) + static_cast<uint64_t>(nsteps + 1u) * nph >= 0xfff00000ull) {
        VRT_HIP_CHECK(hipStreamSynchronize(g->ctx->stream));
        const uint32_t d = g->cfg.embedding_length, F = g->cfg.feed_forward_length;
        const uint32_t qw = g->cfg.head_count * g->cfg.head_dim;
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_qkv, 0, (qw + 2u * g->cfg.head_dim) * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_part, 0, static_cast<size_t>(kMaxChunks) * (qw + kLine * g->cfg.head_count) * 8u,
                                     g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_o, 0, 2u * d * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_o4, 0, static_cast<size_t>(kMkFuseHeads) * d * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_g, 0, F * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_f, 0, 2u * d * 8u, g->ctx->stream));
        VRT_HIP_CHECK(hipMemsetAsync(mk->P.x_am, 0, kLine * mk->grid * 8u, g->ctx->stream));
        g->mk_tag = 1u;
    }
    uint32_t tag0 = g->mk_tag;
    hipStream_t stream = g->ctx->stream;
    CoopSlot& ds = coop_slot(g->ctx->device);
    std::lock_guard<std::mutex> lock(ds.mu);
    // the parameter block is one per device: order this launch after any other executor's
    if (ds.last && ds.last_stream != stream) VRT_HIP_CHECK(hipStreamWaitEvent(stream, ds.last, 0));
    if (ds.owner[kCoopMk] != mk || ds.version[kCoopMk] != mk->version) {
        VRT_HIP_CHECK(hipMemcpyToSymbolAsync(HIP_SYMBOL(g_mk), &mk->P, sizeof(MkParams), 0, hipMemcpyHostToDevice, stream));
        VRT_HIP_CHECK(hipMemcpyToSymbolAsync(HIP_SYMBOL(g_mk_layers), mk->layers.data(), mk->layers.size() * sizeof(MkLayer), 0,
                                             hipMemcpyHostToDevice, stream));
        ds.owner[kCoopMk] = mk;
        ds.version[kCoopMk] = mk->version;
    }
    void* args[] = {&nsteps, &tag0};
    const hipError_t le = hipLaunchCooperativeKernel(mk->P.kv16 == 2u ? mk->fns.bf16 : (mk->P.kv16 ? mk->fns.f16 : mk->fns.f32), dim3(mk->grid),
                                                     dim3(kMkThreads), args, 0, stream);
    if (le == hipErrorIllegalState || le == hipErrorCooperativeLaunchTooLarge) {
        // The device refuses the cooperative launch (on this stack: while another live process
        // has made one on the same GPU). Nothing ran; the caller takes the multi-kernel path.
        (void)hipGetLastError();
        return kMkRefused;
    }
    if (le != hipSuccess)
        return set_error(VRT_ERR_HIP, "hipLaunchCooperativeKernel (persistent decode) failed: %s", hipGetErrorString(le));
    if (!ds.last) VRT_HIP_CHECK(hipEventCreateWithFlags(&ds.last, hipEventDisableTiming));
    VRT_HIP_CHECK(hipEventRecord(ds.last, stream));
    ds.last_stream = stream;
    g->mk_tag += nsteps * nph;
    return VRT_OK;
}

}  // namespace vrt
