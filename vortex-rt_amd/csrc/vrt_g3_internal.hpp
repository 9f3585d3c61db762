// vrt_g3_internal.hpp -- Gemma 3 executor state shared by the multi-kernel step
// (vrt_gemma3.hip) and the persistent decode kernel (vrt_decode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <vector>

#include "vrt_hip.h"
#include "vrt_internal.hpp"

namespace vrt {

struct G3State {
    uint32_t step;         // position of the next step (== steps since reset)
    uint32_t stop;         // EOS generated: later steps do nothing
    uint32_t lm_from;      // steps >= lm_from run the LM head
    uint32_t feed_until;   // tokens[s+1] comes from the host when s+1 < feed_until
    uint32_t want_logits;  // LM head also writes the logits
    uint32_t nonfinite;    // first failure (vrt_g3_errors.hpp codes; ~0u: none)
    uint32_t pad[2];
};

struct LmPartial {
    float value;
    uint32_t index;
};

struct G3Params {
    uint32_t d, H, hd, F, V, L, ctx_len, eos;
    float eps, emb_scale, attn_scale;
    uint32_t kv16;        // KV cache entries: 0 fp32, 1 fp16, 2 bf16 (VRT_G3_OPT_KV_F16 / _KV_BF16)
    const uint8_t* arena_end;
    const uint8_t* tok_embd;
    G3State* st;
    uint32_t* tokens;
    vrt_argmax_result* results;
    float* hres;
    float* hmid;
    float* qkv;
    float* att;
    float* part;
    float* o;
    float* g;
    float* gu;            // [2F] raw gate and up rows of the unfused sequence (VRT_G3_OPT_FUSION 0)
    float* f;
    float* hidden;
    float* logits;
    LmPartial* lm_part;
    const float* cos_l;
    const float* sin_l;
    const float* cos_g;
    const float* sin_g;
};

struct LayerParams {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw;
    float* kc;            // [slots][hd] fp32, or 16-bit entries in the first half of the buffer (kv16 != 0)
    float* vc;
    uint32_t slots;       // KV slots: window for local layers, context_length otherwise
    uint32_t global;
    uint32_t attn_grid;   // workgroups of k_attn
    uint32_t chunk_max;   // max positions per attention workgroup
    uint32_t index;       // block number
};

struct LaunchDesc {
    const void* fn;
    uint32_t grid;
    size_t smem;
    uint32_t per_wg;   // rows per workgroup
    uint32_t S;        // row-slot width (lanes per row)
};

struct MkState;   // persistent decode kernel: exchange buffers and launch shape (vrt_decode.hip)
struct TkState;   // phase-team decode kernel (vrt_team.hip)

// Cooperative launches on one device. Each persistent kernel keeps its parameter block in
// constant memory, one per device: `owner` and `version` say which executor's block was last
// uploaded for each kernel, and `last` is the event after the device's last cooperative launch,
// on `last_stream`, so a launch from another executor's stream is ordered after it. The event
// lives while at least one executor with a persistent kernel exists on the device (`users`).
enum CoopKernel : int { kCoopMk = 0, kCoopTeam = 1, kCoopKinds = 2 };
struct CoopSlot {
    std::mutex mu;
    const void* owner[kCoopKinds] = {nullptr, nullptr};
    uint64_t version[kCoopKinds] = {0, 0};
    uint32_t users = 0;
    hipEvent_t last = nullptr;
    hipStream_t last_stream = nullptr;
};
constexpr int kMaxCoopDevices = 64;
CoopSlot& coop_slot(int device);   // vrt_decode.hip

// A block's weight matrices expanded once for the prefill GEMMs: the quants as f16 [N][K] and
// the block scales as fp32 [N][K / 32]. qkv: the q, k, v rows concatenated; gu: the gate and up
// rows interleaved in groups of 64 (32 gate rows, then the same 32 up rows).
struct PfMatrix {
    const void* h = nullptr;
    const float* s = nullptr;
};
struct PfLayerW {
    PfMatrix qkv, o, gu, down;
};

// Batched prefill workspace (vrt_prefill.hip); max_t == 0: prefill unavailable for the shape.
struct PfState {
    uint32_t max_t = 0;     // prompt positions per call
    float* h = nullptr;     // [max_t][d] residual stream
    float* x = nullptr;     // [max_t][d] sublayer outputs (O projection, down projection)
    void* ahi = nullptr;    // [max_t][max(d, H*hd, F)] GEMM input, f16 high part
    void* alo = nullptr;    //   ... and low part
    float* big = nullptr;   // [max_t][max(H*hd + 2*hd, 2F)] q|k|v rows, then gate|up rows
    void* khi = nullptr;    // attention keys (tkv x hd), f16 high part: a segment's history, then its rows
    void* klo = nullptr;    //   ... and low part
    void* vhi = nullptr;    // attention values (Tp x hd), f16 high part
    void* vlo = nullptr;    //   ... and low part
    uint32_t tkv = 0;       // key coordinates of khi..vlo: max(max_t, context_length), padded
    uint32_t qtmax = 0;     // 32-query tiles of max_t
    uint32_t maxc = 0;      // key chunks per query tile, at most
    float* opart = nullptr;     // [H][qtmax][maxc][32][hd] attention unit partials
    float* mpart = nullptr;     // [H][qtmax][maxc][32] their maxima
    double* lpart = nullptr;    // [H][qtmax][maxc][32] their exp sums
    std::vector<PfLayerW> lw;   // expanded weights per block (empty: the GEMMs read the Q8_0 arena)
};

}  // namespace vrt

struct vrt_g3 {
    vrt_ctx* ctx = nullptr;
    vrt_g3_config cfg{};
    uint32_t eos = 1;
    uint64_t arena_bytes = 0;
    vrt::G3Params P{};
    std::vector<vrt::LayerParams> layers;
    vrt::LaunchDesc ld_qkv{}, ld_o{}, ld_gateup{}, ld_down{}, ld_lm{};
    uint32_t lm_rows_per_wg = 0;
    const float* out_norm_dev = nullptr;
    std::vector<void*> allocs;   // device allocations owned by the executor
    vrt::G3State* host_ctl = nullptr; // pinned control block
    vrt_argmax_result* host_res = nullptr;
    uint32_t next_pos = 0;
    bool use_graph = true;
    bool fusion = true;          // projection fusion (VRT_G3_OPT_FUSION)
    uint32_t q8_lanes = 0;       // row-slot width request of the projections, 0 = auto (VRT_G3_OPT_Q8_LANES)
    bool use_persistent = true;  // one cooperative launch per batch of steps (vrt_decode.hip)
    bool mk_refused = false;     // the device refused a cooperative launch: multi-kernel steps
    vrt::MkState* mk = nullptr;
    uint32_t mk_tag = 1;         // first exchange tag of the next persistent launch
    bool use_team = true;        // positions below the team kernel's history limit run on it (vrt_team.hip)
    vrt::TkState* tk = nullptr;
    uint32_t tk_tag = 1;         // first exchange tag of the next team-kernel launch
    int last_coop = 0;           // kernel of the last persistent launch (vrt::CoopKernel)
    hipGraphExec_t graph = nullptr;
    vrt::PfState pf;             // batched prefill (vrt_prefill.hip)
    uint32_t gen_prompt = 0;     // generation in flight (vrt_g3_start .. vrt_g3_collect)
    uint32_t gen_max = 0;
    uint64_t gen_steps = 0;
    uint32_t live_batches = 0;   // vrt_g3_batch objects over this executor's weights and stream
};

namespace vrt {
// Persistent decode kernel (vrt_decode.hip). mk_setup returns VRT_OK and leaves g->mk null
// when the configuration or device does not support it (the multi-kernel step is used).
int mk_setup(vrt_g3* g);
// Enqueues nsteps steps as one cooperative launch; kMkRefused when the device refuses the
// cooperative launch (nothing enqueued: the caller runs the steps on the multi-kernel path).
constexpr int kMkRefused = 1000;
int mk_run(vrt_g3* g, uint32_t nsteps);
void mk_destroy(vrt_g3* g);
int mk_clear_abort(vrt_g3* g);
// Enqueues a copy of the abort word into host memory at *dst (stream-ordered, no sync).
int mk_read_abort(vrt_g3* g, uint32_t* dst);
int mk_read_exchange(vrt_g3* g, uint32_t which, uint64_t* out, uint64_t cap, uint64_t* n);
int mk_set_trace(vrt_g3* g, bool on);
int mk_set_kv_format(vrt_g3* g, uint32_t fmt);
// Batched prefill (vrt_prefill.hip): workspace for up to max_t positions, and one prefill of T
// positions from position 0 whose last position runs g3_enqueue_lm.
int pf_setup(vrt_g3* g, uint32_t max_t);
// The blocks over the segment of T prompt positions from p0 (earlier positions already in the
// KV cache); the final segment also runs the LM head of its last position.
int pf_run(vrt_g3* g, uint32_t T, uint32_t p0 = 0, bool final = true);
// Row-batch building blocks shared by the prefill and the batched decode (vrt_prefill.hip):
// block l's projections over M rows as (split-K) GEMMs, its gate/up product, the residual
// norms over rows, embedding rows, and the logits of M rows against the tied embedding table.
enum PfProj : uint32_t { kProjQkv = 0, kProjO = 1, kProjDown = 2 };
int pf_project(vrt_g3* g, uint32_t l, uint32_t which, const _Float16* ahi, const _Float16* alo, uint32_t M, float* c,
               uint32_t splits, uint32_t* used, hipStream_t s);
int pf_ffn_glu(vrt_g3* g, uint32_t l, const _Float16* ahi, const _Float16* alo, uint32_t M, _Float16* ghi,
               _Float16* glo, hipStream_t s);
int pf_norm(float* h, const float* f, uint32_t nsplit, uint64_t sstride, const float* w_post, const float* w_next,
            uint32_t n, float eps, _Float16* xhi, _Float16* xlo, G3State* st, uint32_t block, uint32_t rows, hipStream_t s,
            bool into);
int pf_embed_rows(vrt_g3* g, const uint32_t* tokens, uint32_t rows, float* h, hipStream_t s);
int pf_lm_logits(vrt_g3* g, const _Float16* xhi, const _Float16* xlo, uint32_t M, float* logits, hipStream_t s);
uint32_t pf_splits(uint32_t M, uint32_t N);
// Final residual + output norm + LM head + argmax of the current step (vrt_gemma3.hip).
int g3_enqueue_lm(vrt_g3* g, hipStream_t s);
int mk_read_trace(vrt_g3* g, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots);
// Phase-team decode kernel (vrt_team.hip): like mk_setup / mk_run, for the steps whose
// attention histories stay within tk_hist_limit(g) positions (positions < the limit).
int tk_setup(vrt_g3* g);
uint32_t tk_pos_limit(const vrt_g3* g);
uint32_t tk_chunk_from(const vrt_g3* g);
// chunked: the variant for steps at positions from tk_chunk_from(g) on (histories longer than a
// workgroup holds on chip); the other one for earlier steps.
int tk_run(vrt_g3* g, uint32_t nsteps, bool chunked);
void tk_destroy(vrt_g3* g);
int tk_read_abort(vrt_g3* g, uint32_t* dst);
int tk_clear_abort(vrt_g3* g);
int tk_set_trace(vrt_g3* g, bool on);
int tk_set_kv_format(vrt_g3* g, uint32_t fmt);
int tk_read_trace(vrt_g3* g, uint64_t* out, uint64_t cap, uint32_t* nwg, uint32_t* slots);
}  // namespace vrt
