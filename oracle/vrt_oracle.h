/*
 * vrt_oracle.h -- CPU restatement of Vortex-RT's Gemma 3 Q8_0 token-loop arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle: only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it. The
 * product (libvrt_hip.so, libvortexrt.so) never links or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Floating-point order follows the reference operation for operation; the file
 * is compiled with -ffp-contract=off so no multiply-add is fused behind the
 * reference's back.
 *
 * Parity pins (what checks each function independently of its own formula):
 *   or_f32_to_f16        numpy float16 (IEEE RNE) on every non-tie, non-carry input;
 *                        closed-form tie (half-up) and carry-loss cases; golden bytes.
 *   or_f16_to_f32        exhaustive over all 65536 halves against numpy float16.
 *   or_f32_to_bf16_rne   nearest of the two neighbouring bf16 values chosen in float64
 *                        (ties to the even one), on random and constructed tie/carry/
 *                        subnormal/inf/NaN inputs; or_bf16_to_f32 exhaustive against the
 *                        16-bit shift into a float32.
 *   or_q8_quantize_*     numpy float32 rint/division; |q|<=127 and the amax element
 *                        quantises to +-127; golden bytes.
 *   or_q8_matvec_lanes   exact float64 dot (products are exact in float64) within the
 *                        reference test's 2e-3 abs bound and a 1e-5 relative bound.
 *   or_gelu_tanh         closed form via numpy float64 tanh within 5e-5 (the
 *                        reference gelu test's bound), gelu(0)=0, odd-symmetry identity.
 *   or_argmax            numpy argmax (first max) on NaN-free data; tie/NaN/-inf cases.
 *   or_rms_norm_*        all-ones input closed form; numpy float64 restatement.
 *   or_rope_*            position 0 is the identity; per-pair norm preserved; numpy.
 *   or_attention         single position returns v; equal keys give the mean of v;
 *                        numpy float64 softmax.
 *   or_g3_*              zero-projection model closed form (hidden = normed scaled
 *                        embedding); window eviction; composition of the pinned parts;
 *                        block-wiring invariants (scale absorption, window-1 flow, RoPE base
 *                        reach, branch norms) with compiled mutants that must fail them.
 *   attention sub-path   through or_g3_set_taps, per block and step: the query and newest key
 *   of or_g3_decode      against float64 per-head RMSNorm then NeoX RoPE at the block's base,
 *                        the newest value equal to the v projection (no norm on v), q.k at the
 *                        current position unchanged by RoPE (one table for q and k), the cache
 *                        rows in time order with window eviction, and the output against a
 *                        float64 softmax(q K^T / sqrt(head_dim)) V.
 * Functions none of these reach are marked "parity unpinned" at their definition.
 */
#ifndef VRT_ORACLE_H
#define VRT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 codec (quantiser of record) ---- */
uint16_t or_f32_to_f16(float f);                 /* src/q8_test_main.cpp:18-41 */
float or_f16_to_f32(uint16_t h);                 /* src/gguf.cpp:203-235 */
/* IEEE 754 binary16 conversion with round to nearest, ties to even (subnormals, overflow to
 * infinity, quiet NaN): the rounding of the fp16 KV cache option, which the reference lists as
 * a roadmap item (README.md:190-192) without an implementation. Bulk form for the pins. */
uint16_t or_f32_to_f16_rne(float f);
void or_f32_to_f16_rne_n(const float* x, uint64_t n, uint16_t* out);
/* IEEE round to nearest even to bfloat16 (NaN -> quiet NaN), and its exact inverse: the bf16
 * KV cache format. */
uint16_t or_f32_to_bf16_rne(float f);
void or_f32_to_bf16_rne_n(const float* x, uint64_t n, uint16_t* out);
float or_bf16_to_f32(uint16_t h);

/* ---- Q8_0 quantisers: 34-byte blocks {f16 scale LE, int8 q[32]} along k ---- */
/* Variant A, src/q8_test_main.cpp:93-124: q = nearbyint(v / (amax/127)), fp32 scale. */
void or_q8_quantize_a(const float* w, uint64_t rows, uint32_t k, uint8_t* out);
/* Variant B, src/ffn_test_main.cpp:112-215: q = nearbyint(v / f16(scale)), amax==0 -> 1. */
void or_q8_quantize_b(const float* w, uint64_t rows, uint32_t k, uint8_t* out);
/* Row dequant, src/gguf.cpp:620-635. */
void or_q8_dequant(const uint8_t* blocks, uint64_t n_blocks, float* out);

/* ---- Q8_0 matvec ---- */
/* Lane-faithful fp32 order of shaders/q8_matvec_u8{,_32,_16,_8}.comp: lane l sums blocks
 * l, l+lanes, ...; then an LDS tree over lanes. lanes in {8,16,32,64}. */
void or_q8_matvec_lanes(const uint8_t* w, const float* x, float* y,
                        uint32_t k, uint64_t rows, uint32_t lanes);
/* Exact float64 accumulation (every product is exact in float64). */
void or_q8_matvec_f64(const uint8_t* w, const float* x, double* y, uint32_t k, uint64_t rows);

/* ---- elementwise / reductions ---- */
float or_gelu_tanh(float x);                     /* src/gemma3.cpp:1440-1452, shaders/gelu_mul.comp:23-31 */
void or_gelu_mul(float* gate, const float* up, uint32_t n);   /* shaders/gelu_mul.comp:17-31 */
/* shaders/argmax.comp:30-100: NaN never wins, larger wins, equal -> lower index.
 * Returns index 0xffffffff / value -inf when no element qualifies. */
void or_argmax(const float* v, uint64_t n, uint32_t* index, float* value);

/* src/gemma3.cpp:948-998: out[i] = in[i] * scale * w[i] (left to right). */
void or_rms_norm_into(const float* in, const float* w, float* out, uint32_t n, float eps);
/* src/gemma3.cpp:1000-1043: v[i] *= scale * w[i]. */
void or_rms_norm_inplace(float* v, const float* w, uint32_t n, float eps);
/* src/gemma3.cpp:1045-1104: per-head rms_norm_inplace with a shared [head_dim] weight. */
void or_rms_norm_heads(float* v, const float* w, uint32_t heads, uint32_t head_dim, float eps);

void or_rope_inv_freq(uint32_t head_dim, float theta, float* out);              /* :1309-1341 */
void or_rope_table(const float* inv, uint32_t half, uint32_t pos, float* c, float* s); /* :1343-1369 */
void or_apply_rope(float* v, uint32_t heads, uint32_t head_dim, const float* c, const float* s); /* :1371-1424 */

/* src/gemma3.cpp:1609-1696 for one layer: q [heads*head_dim], keys/values [history][head_dim]
 * in time order (oldest first), out [heads*head_dim]. Returns 0, or -1 if the softmax
 * denominator is not finite and positive. */
int or_attention(const float* q, const float* keys, const float* values, uint32_t history,
                 uint32_t heads, uint32_t head_dim, float scale, float* out);

/* ---- whole-model executor over a GGUF file ---- */
typedef struct or_g3 or_g3;
typedef struct or_g3_info {
    uint32_t context_length, embedding_length, block_count, feed_forward_length;
    uint32_t head_count, head_count_kv, head_dim, value_dim, vocab_size, sliding_window;
    float rms_epsilon, global_rope_base, local_rope_base;
    uint32_t eos_id, bos_id;
} or_g3_info;

/* Opens a GGUF v2/v3 file (src/gguf.cpp:312-403) and builds the executor state
 * (src/gemma3.cpp:72-654). lanes selects the matvec order (8 = Lavapipe's). Returns NULL
 * on error with a message in err. */
or_g3* or_g3_open(const char* path, uint32_t lanes, char* err, size_t errlen);
void or_g3_close(or_g3* m);
void or_g3_get_info(const or_g3* m, or_g3_info* info);
void or_g3_reset(or_g3* m);                      /* src/gemma3.cpp:1454-1460 */
/* One decode_token step (src/gemma3.cpp:1462-1882). want_logits=0 skips the LM head.
 * hidden_out (embedding_length) and logits_out (vocab) may be NULL. Returns 0 or a
 * negative code with the reference's message in the per-model error buffer. */
int or_g3_decode(or_g3* m, uint32_t token, uint32_t pos, int want_logits,
                 float* hidden_out, float* logits_out, uint32_t* argmax_index, float* argmax_value);
/* generate_greedy_tokens (src/gemma3.cpp:2080-2149). */
int or_g3_generate(or_g3* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                   uint32_t* out_tokens, uint32_t* n_out);
const char* or_g3_error(const or_g3* m);
/* fp16 KV cache: keys and values are rounded with or_f32_to_f16_rne when they enter the cache
 * (every position's attention, the current one's included, reads the cache). Resets the cache. */
void or_g3_set_kv_f16(or_g3* m, int on);
/* KV cache entries: 0 fp32, 1 fp16 (as or_g3_set_kv_f16), 2 bf16 (or_f32_to_bf16_rne as they
 * enter the cache). Resets the cache. */
void or_g3_set_kv_format(or_g3* m, int fmt);

/* Intermediate values of the attention sub-path, for the parity tests that pin it
 * (src/gemma3.cpp:1511-1696 computes them inside decode_token and exposes none). While taps
 * are set, every decode step writes, for each block l (arrays indexed [l][...]):
 *   xn       [d]          the attention-norm output the q/k/v projections read
 *   q_proj   [H*hd]       the q projection as the matvec left it (before QK-norm)
 *   k_proj   [hd], v_proj [hd]   the k and v projections
 *   q_att    [H*hd]       the query the attention reads (after QK-norm and RoPE)
 *   keys, values [hist_cap][hd]  the cache rows the attention reads, oldest first
 *   history  (u32)        how many rows that is (rows past hist_cap are not written)
 *   att      [H*hd]       the attention output the O projection reads
 * Any pointer may be NULL. Passing NULL clears the taps. */
typedef struct or_g3_taps {
    float* xn;
    float* q_proj;
    float* k_proj;
    float* v_proj;
    float* q_att;
    float* keys;
    float* values;
    uint32_t* history;
    float* att;
    uint32_t hist_cap;
} or_g3_taps;
void or_g3_set_taps(or_g3* m, const or_g3_taps* taps);
/* Threads used by the OpenMP loops (matvec rows). */
int or_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
