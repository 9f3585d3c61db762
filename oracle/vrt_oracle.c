/*
 * vrt_oracle.c -- CPU restatement of Vortex-RT's Gemma 3 Q8_0 token loop.
 *
 * TEST INFRASTRUCTURE ONLY (see vrt_oracle.h): the oracle, never the product.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 * Citations are to the reference tree (yannickfan67-ai/Vortex-RT v0.2.0).
 */
#include "vrt_oracle.h"

#include <float.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* src/q8_test_main.cpp:18-41. Not IEEE: ties round half-up ((m + 0x1000) >> 13), and a
 * mantissa carry is OR-ed (not added) into the exponent field, so it is lost whenever the
 * biased fp16 exponent is odd. Inputs with exponent >= 31 (incl. NaN) become +-inf. */
uint16_t or_f32_to_f16(float f) {
    const uint32_t x = bits_of(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mantissa = x & 0x7fffffu;
    const int exponent = (int)((x >> 23) & 0xffu) - 127 + 15;
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        mantissa = (mantissa | 0x800000u) >> (1 - exponent);
        return (uint16_t)(sign + ((mantissa + 0x1000u) >> 13));
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | ((mantissa + 0x1000u) >> 13));
}

/* src/gguf.cpp:203-235 (identical to src/q8_test_main.cpp:43-74): exact half -> float. */
uint16_t or_f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u)); /* NaN, inf */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds past 65504 */
    const uint32_t e = ax >> 23;
    if (e < 113u) {   /* below 2^-14: a multiple of 2^-24 (subnormal half) or zero */
        const uint32_t shift = 126u - e;   /* value = m 2^(e - 150) = (m >> shift) 2^-24 + rest */
        if (shift > 24u) return (uint16_t)sign;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((e - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;   /* a carry moves into the exponent */
    return (uint16_t)(sign | h);
}

void or_f32_to_f16_rne_n(const float* x, uint64_t n, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_f32_to_f16_rne(x[i]);
}

/* bf16 (the upper half of an fp32) by round to nearest even of the lower 16 bits; NaN stays a
 * quiet NaN of the same sign; a carry out of the mantissa moves into the exponent (finite
 * values at the top round to infinity). The bf16 KV cache format: the reference's README lists
 * an fp16/bf16 cache as a roadmap item (README.md:190-192) with no arithmetic to follow, so this
 * is IEEE RNE to bfloat16. */
uint16_t or_f32_to_bf16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    const uint32_t rem = x & 0xffffu, hi = x >> 16;
    return (uint16_t)(hi + (rem > 0x8000u || (rem == 0x8000u && (hi & 1u))));
}

void or_f32_to_bf16_rne_n(const float* x, uint64_t n, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16_rne(x[i]);
}

float or_bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 31u;
    uint32_t mantissa = h & 1023u;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            int e = -14;
            while ((mantissa & 0x400u) == 0) { mantissa <<= 1; --e; }
            mantissa &= 0x3ffu;
            bits = sign | ((uint32_t)(e + 127) << 23) | (mantissa << 13);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent - 15u + 127u) << 23) | (mantissa << 13);
    }
    return float_of(bits);
}

/* static_cast<int>(std::nearbyint(r)) then std::clamp(-127, 127). A NaN quotient (0/0 in
 * variant A when a block is all zero) converts to INT_MIN on x86-64 (cvttss2si), which the
 * clamp maps to -127; that x86 result is restated here explicitly. */
static int8_t quant_round(float r) {
    if (isnan(r)) return -127;
    const float n = nearbyintf(r);
    int q;
    if (n >= 2147483648.0f || n < -2147483648.0f) q = INT32_MIN; /* cvttss2si overflow */
    else q = (int)n;
    if (q < -127) q = -127;
    if (q > 127) q = 127;
    return (int8_t)q;
}

static void quantize_block(const float* v, uint8_t* out, int variant) {
    float amax = 0.0f;
    for (int k = 0; k < 32; ++k) {
        const float a = fabsf(v[k]);
        amax = (amax < a) ? a : amax; /* std::max(abs_max, fabs): (a < b) ? b : a */
    }
    float scale;
    if (variant == 0) scale = amax / 127.0f;                       /* q8_test_main.cpp:106 */
    else scale = amax == 0.0f ? 1.0f : amax / 127.0f;              /* ffn_test_main.cpp:169-172 */
    const uint16_t half = or_f32_to_f16(scale);
    const float divisor = variant == 0 ? scale : or_f16_to_f32(half); /* :116 vs :190 */
    out[0] = (uint8_t)(half & 0xffu);
    out[1] = (uint8_t)(half >> 8);
    for (int k = 0; k < 32; ++k) out[2 + k] = (uint8_t)quant_round(v[k] / divisor);
}

void or_q8_quantize_a(const float* w, uint64_t rows, uint32_t k, uint8_t* out) {
    const uint64_t blocks = (uint64_t)rows * (k / 32u);
    #pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (int64_t)blocks; ++b) quantize_block(w + 32u * b, out + 34u * b, 0);
}

void or_q8_quantize_b(const float* w, uint64_t rows, uint32_t k, uint8_t* out) {
    const uint64_t blocks = (uint64_t)rows * (k / 32u);
    #pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < (int64_t)blocks; ++b) quantize_block(w + 32u * b, out + 34u * b, 1);
}

/* src/gguf.cpp:620-635: value = scale * float(int8 q). */
void or_q8_dequant(const uint8_t* blocks, uint64_t n_blocks, float* out) {
    for (uint64_t b = 0; b < n_blocks; ++b) {
        const uint8_t* p = blocks + 34u * b;
        const float scale = or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
        for (int k = 0; k < 32; ++k) out[32u * b + k] = scale * (float)(int8_t)p[2 + k];
    }
}

/* shaders/q8_matvec_u8_8.comp:47-101 (and the 16/32/64-lane variants): per-lane fp32
 * running sum "sum += scale * float(q) * x" over blocks lane, lane+L, ...; LDS tree. */
static float matvec_row_lanes(const uint8_t* row, const float* x, uint32_t blocks, uint32_t lanes) {
    float partial[64];
    for (uint32_t lane = 0; lane < lanes; ++lane) {
        float sum = 0.0f;
        for (uint32_t block = lane; block < blocks; block += lanes) {
            const uint8_t* p = row + 34u * block;
            const float scale = or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
            const float* xb = x + 32u * block;
            for (uint32_t k = 0; k < 32u; ++k) sum += scale * (float)(int8_t)p[2 + k] * xb[k];
        }
        partial[lane] = sum;
    }
    for (uint32_t stride = lanes / 2u; stride > 0u; stride >>= 1u)
        for (uint32_t lane = 0; lane < stride; ++lane) partial[lane] += partial[lane + stride];
    return partial[0];
}

void or_q8_matvec_lanes(const uint8_t* w, const float* x, float* y, uint32_t k, uint64_t rows, uint32_t lanes) {
    const uint32_t blocks = k / 32u;
    if (lanes != 8 && lanes != 16 && lanes != 32 && lanes != 64) lanes = 64;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
        y[r] = matvec_row_lanes(w + (uint64_t)r * blocks * 34u, x, blocks, lanes);
}

/* Exact in float64: f16 scale (11 bits) x int8 (8 bits) x fp32 (24 bits) = 43 bits. The
 * order of this sum is the only rounding; src/ffn_test_main.cpp:217-250 uses the same. */
void or_q8_matvec_f64(const uint8_t* w, const float* x, double* y, uint32_t k, uint64_t rows) {
    const uint32_t blocks = k / 32u;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        const uint8_t* row = w + (uint64_t)r * blocks * 34u;
        double sum = 0.0;
        for (uint32_t b = 0; b < blocks; ++b) {
            const uint8_t* p = row + 34u * b;
            const double scale = (double)or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
            for (uint32_t j = 0; j < 32u; ++j)
                sum += scale * (double)(int8_t)p[2 + j] * (double)x[32u * b + j];
        }
        y[r] = sum;
    }
}

/* src/gemma3.cpp:1440-1452 == shaders/gelu_mul.comp:23-31. */
float or_gelu_tanh(float x) {
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float cubic = x * x * x;
    return 0.5f * x * (1.0f + tanhf(kSqrt2OverPi * (x + kCubic * cubic)));
}

void or_gelu_mul(float* gate, const float* up, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) gate[i] = or_gelu_tanh(gate[i]) * up[i];
}

/* shaders/argmax.comp:30-43. */
static int argmax_better(float cv, uint32_t ci, float bv, uint32_t bi) {
    if (isnan(cv)) return 0;
    return cv > bv || (cv == bv && ci < bi);
}

/* shaders/argmax.comp:45-100: 256 strided lanes then an LDS tree. The rule is a total order
 * on (value desc, index asc) over non-NaN entries, so the result is the same for any
 * reduction shape; the lane structure is restated anyway. */
void or_argmax(const float* v, uint64_t n, uint32_t* index, float* value) {
    float bv[256];
    uint32_t bi[256];
    for (uint32_t lane = 0; lane < 256u; ++lane) {
        float best_v = -INFINITY;
        uint32_t best_i = 0xffffffffu;
        for (uint64_t i = lane; i < n; i += 256u)
            if (argmax_better(v[i], (uint32_t)i, best_v, best_i)) { best_v = v[i]; best_i = (uint32_t)i; }
        bv[lane] = best_v;
        bi[lane] = best_i;
    }
    for (uint32_t stride = 128u; stride > 0u; stride >>= 1u)
        for (uint32_t lane = 0; lane < stride; ++lane)
            if (argmax_better(bv[lane + stride], bi[lane + stride], bv[lane], bi[lane])) {
                bv[lane] = bv[lane + stride];
                bi[lane] = bi[lane + stride];
            }
    *index = bi[0];
    *value = bv[0];
}

/* scale = 1.0f / std::sqrt(float(sum_sq_double / n) + eps); src/gemma3.cpp:967-983. */
static float rms_scale(const float* v, uint32_t n, float eps) {
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)v[i] * (double)v[i];
    const double mean = ss / (double)n;
    return 1.0f / sqrtf((float)mean + eps);
}

void or_rms_norm_into(const float* in, const float* w, float* out, uint32_t n, float eps) {
    const float scale = rms_scale(in, n, eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = in[i] * scale * w[i];   /* :991-996 */
}

void or_rms_norm_inplace(float* v, const float* w, uint32_t n, float eps) {
    const float scale = rms_scale(v, n, eps);
    for (uint32_t i = 0; i < n; ++i) v[i] *= scale * w[i];            /* :1036-1042 */
}

void or_rms_norm_heads(float* v, const float* w, uint32_t heads, uint32_t head_dim, float eps) {
    for (uint32_t h = 0; h < heads; ++h) or_rms_norm_inplace(v + (size_t)h * head_dim, w, head_dim, eps);
}

/* src/gemma3.cpp:1309-1341: inv[i] = 1 / powf(theta, (2i)/head_dim). */
void or_rope_inv_freq(uint32_t head_dim, float theta, float* out) {
    const uint32_t half = head_dim / 2u;
    for (uint32_t i = 0; i < half; ++i) {
        const float exponent = (2.0f * (float)i) / (float)head_dim;
        out[i] = 1.0f / powf(theta, exponent);
    }
}

/* src/gemma3.cpp:1343-1369: angle = float(pos) * inv[i]; cosf / sinf. */
void or_rope_table(const float* inv, uint32_t half, uint32_t pos, float* c, float* s) {
    const float pf = (float)pos;
    for (uint32_t i = 0; i < half; ++i) {
        const float angle = pf * inv[i];
        c[i] = cosf(angle);
        s[i] = sinf(angle);
    }
}

/* src/gemma3.cpp:1371-1424: NeoX half split (x[i], x[i+half]). */
void or_apply_rope(float* v, uint32_t heads, uint32_t head_dim, const float* c, const float* s) {
    const uint32_t half = head_dim / 2u;
    for (uint32_t h = 0; h < heads; ++h) {
        float* base = v + (size_t)h * head_dim;
        for (uint32_t i = 0; i < half; ++i) {
            const float a = base[i];
            const float b = base[half + i];
            base[i] = a * c[i] - b * s[i];
            base[half + i] = b * c[i] + a * s[i];
        }
    }
}

/* src/gemma3.cpp:1609-1696. */
int or_attention(const float* q, const float* keys, const float* values, uint32_t history,
                 uint32_t heads, uint32_t head_dim, float scale, float* out) {
    float* scores = (float*)malloc(sizeof(float) * (history ? history : 1));
    float* probs = (float*)malloc(sizeof(float) * (history ? history : 1));
    if (!scores || !probs) { free(scores); free(probs); return -2; }
    memset(out, 0, sizeof(float) * heads * head_dim);
    /* Long histories split the independent work over threads without changing any result: each
     * score is its own dot product, and each output dimension keeps the time-ordered sum. */
    const int par = history >= 256;
    for (uint32_t h = 0; h < heads; ++h) {
        const float* qh = q + (size_t)h * head_dim;
#pragma omp parallel for schedule(static) if (par)
        for (uint32_t t = 0; t < history; ++t) {
            const float* kt = keys + (size_t)t * head_dim;
            double dot = 0.0;
            for (uint32_t d = 0; d < head_dim; ++d) dot += (double)qh[d] * (double)kt[d];
            scores[t] = (float)dot * scale;
        }
        float max_score = -INFINITY;
        for (uint32_t t = 0; t < history; ++t)
            max_score = max_score < scores[t] ? scores[t] : max_score; /* std::max(a, b) */
        double den = 0.0;
        for (uint32_t t = 0; t < history; ++t) {
            const float e = expf(scores[t] - max_score);
            scores[t] = e;
            den += e;
        }
        if (!(den > 0.0) || !isfinite(den)) { free(scores); free(probs); return -1; }
        for (uint32_t t = 0; t < history; ++t) probs[t] = (float)((double)scores[t] / den);
        float* oh = out + (size_t)h * head_dim;
#pragma omp parallel for schedule(static) if (par)
        for (uint32_t d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (uint32_t t = 0; t < history; ++t) acc += probs[t] * values[(size_t)t * head_dim + d];
            oh[d] = acc;
        }
    }
    free(scores);
    free(probs);
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* Minimal GGUF v2/v3 reader (src/gguf.cpp:312-403): what the executor needs.            */
/* ------------------------------------------------------------------------------------ */

typedef struct { const uint8_t* p; uint64_t n, pos; int bad; } rd_t;

static uint64_t rd_u(rd_t* r, int bytes) {
    if (r->bad || r->pos + (uint64_t)bytes > r->n) { r->bad = 1; return 0; }
    uint64_t v = 0;
    memcpy(&v, r->p + r->pos, (size_t)bytes);
    r->pos += (uint64_t)bytes;
    return v;
}

typedef struct {
    char key[96];
    int kind; /* 0 none, 1 unsigned, 2 signed, 3 float, 4 string, 5 array, 6 bool */
    uint64_t u;
    int64_t i;
    double f;
    uint64_t array_len;
    char str[64];
} meta_t;

static void rd_skip_value(rd_t* r, uint32_t type, int depth, meta_t* out);

static void rd_value(rd_t* r, uint32_t type, int depth, meta_t* out) {
    rd_skip_value(r, type, depth, out);
}

static void rd_skip_value(rd_t* r, uint32_t type, int depth, meta_t* out) {
    if (depth > 8) { r->bad = 1; return; }
    switch (type) {
    case 0: { uint64_t v = rd_u(r, 1); if (out) { out->kind = 1; out->u = v; } } break;
    case 1: { int8_t v = (int8_t)rd_u(r, 1); if (out) { out->kind = 2; out->i = v; } } break;
    case 2: { uint64_t v = rd_u(r, 2); if (out) { out->kind = 1; out->u = v; } } break;
    case 3: { int16_t v = (int16_t)rd_u(r, 2); if (out) { out->kind = 2; out->i = v; } } break;
    case 4: { uint64_t v = rd_u(r, 4); if (out) { out->kind = 1; out->u = v; } } break;
    case 5: { int32_t v = (int32_t)rd_u(r, 4); if (out) { out->kind = 2; out->i = v; } } break;
    case 6: { uint32_t b = (uint32_t)rd_u(r, 4); float f = float_of(b); if (out) { out->kind = 3; out->f = f; } } break;
    case 7: { uint64_t v = rd_u(r, 1); if (v > 1) r->bad = 1; if (out) { out->kind = 6; out->u = v; } } break;
    case 8: {
        uint64_t len = rd_u(r, 8);
        if (len > (1ull << 30) || r->pos + len > r->n) { r->bad = 1; return; }
        if (out) {
            out->kind = 4;
            size_t c = len < sizeof(out->str) - 1 ? (size_t)len : sizeof(out->str) - 1;
            memcpy(out->str, r->p + r->pos, c);
            out->str[c] = 0;
        }
        r->pos += len;
    } break;
    case 9: {
        uint32_t et = (uint32_t)rd_u(r, 4);
        uint64_t count = rd_u(r, 8);
        if (et > 12 || count > (1ull << 28)) { r->bad = 1; return; }
        if (out) { out->kind = 5; out->array_len = count; }
        for (uint64_t i = 0; i < count && !r->bad; ++i) rd_skip_value(r, et, depth + 1, NULL);
    } break;
    case 10: { uint64_t v = rd_u(r, 8); if (out) { out->kind = 1; out->u = v; } } break;
    case 11: { int64_t v = (int64_t)rd_u(r, 8); if (out) { out->kind = 2; out->i = v; } } break;
    case 12: { uint64_t b = rd_u(r, 8); double d; memcpy(&d, &b, 8); if (out) { out->kind = 3; out->f = d; } } break;
    default: r->bad = 1;
    }
}

typedef struct { char name[96]; uint32_t n_dims; uint64_t dims[8]; uint32_t type; uint64_t offset; } tinfo_t;

/* ------------------------------------------------------------------------------------ */
/* Executor (src/gemma3.cpp).                                                           */
/* ------------------------------------------------------------------------------------ */

typedef struct {
    uint64_t q, k, v, o, gate, up, down;             /* byte offsets into the data section */
    const float *attn_norm, *q_norm, *k_norm, *post_attn_norm, *ffn_norm, *post_ffw_norm;
    float *keys, *vals;                              /* ring or linear store */
    uint32_t cap, start, count;
    int global;
} or_layer_t;

struct or_g3 {
    or_g3_info info;
    uint8_t* file;
    uint64_t file_size;
    const uint8_t* data;
    uint64_t data_bytes;
    uint64_t token_embd;
    const float* output_norm;
    or_layer_t* layers;
    float emb_scale, attn_scale;
    float *inv_local, *inv_global;
    uint32_t next_pos;
    uint32_t lanes;
    int kv_fmt;   /* KV cache entries: 0 fp32, 1 fp16, 2 bf16 */
    int tapping;
    or_g3_taps taps;
    char err[256];
};

static void set_err(char* buf, size_t n, const char* fmt, ...) {
    if (!buf || !n) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, n, fmt, ap);
    va_end(ap);
}

static uint64_t tensor_bytes(const tinfo_t* t) {
    uint64_t elems = 1;
    for (uint32_t d = 0; d < t->n_dims; ++d) elems *= t->dims[d];
    switch (t->type) {
    case 0: return elems * 4;
    case 1: return elems * 2;
    case 8: return elems / 32 * 34;
    default: return 0;
    }
}

or_g3* or_g3_open(const char* path, uint32_t lanes, char* err, size_t errlen) {
    FILE* fp = fopen(path, "rb");
    if (!fp) { set_err(err, errlen, "Failed to open GGUF file: %s", path); return NULL; }
    fseek(fp, 0, SEEK_END);
    long sz = ftell(fp);
    fseek(fp, 0, SEEK_SET);
    or_g3* m = (or_g3*)calloc(1, sizeof(or_g3));
    m->file = (uint8_t*)malloc((size_t)sz + 64);
    m->file_size = (uint64_t)sz;
    if (fread(m->file, 1, (size_t)sz, fp) != (size_t)sz) { fclose(fp); set_err(err, errlen, "short read"); or_g3_close(m); return NULL; }
    fclose(fp);
    m->lanes = lanes ? lanes : 8;

    rd_t r = { m->file, m->file_size, 0, 0 };
    if (rd_u(&r, 4) != 0x46554747u) { set_err(err, errlen, "Invalid GGUF magic"); or_g3_close(m); return NULL; }
    uint32_t version = (uint32_t)rd_u(&r, 4);
    if (version < 2 || version > 3) { set_err(err, errlen, "Unsupported GGUF version: %u", version); or_g3_close(m); return NULL; }
    uint64_t n_tensors = rd_u(&r, 8), n_meta = rd_u(&r, 8);
    if (n_tensors > 1000000 || n_meta > 1000000) { set_err(err, errlen, "GGUF header counts exceed safety limits"); or_g3_close(m); return NULL; }

    meta_t* metas = (meta_t*)calloc(n_meta ? n_meta : 1, sizeof(meta_t));
    for (uint64_t i = 0; i < n_meta && !r.bad; ++i) {
        uint64_t klen = rd_u(&r, 8);
        if (klen > (1ull << 30) || r.pos + klen > r.n) { r.bad = 1; break; }
        size_t c = klen < sizeof(metas[i].key) - 1 ? (size_t)klen : sizeof(metas[i].key) - 1;
        memcpy(metas[i].key, r.p + r.pos, c);
        r.pos += klen;
        uint32_t type = (uint32_t)rd_u(&r, 4);
        if (type > 12) { r.bad = 1; break; }
        rd_value(&r, type, 0, &metas[i]);
    }
    #define FIND(keystr) ({ const meta_t* _f = NULL; for (uint64_t _i = 0; _i < n_meta; ++_i) if (!strcmp(metas[_i].key, keystr)) { _f = &metas[_i]; break; } _f; })
    uint64_t alignment = 32;
    const meta_t* al = FIND("general.alignment");
    if (al) alignment = al->kind == 1 ? al->u : (uint64_t)al->i;

    tinfo_t* tis = (tinfo_t*)calloc(n_tensors ? n_tensors : 1, sizeof(tinfo_t));
    for (uint64_t i = 0; i < n_tensors && !r.bad; ++i) {
        uint64_t nlen = rd_u(&r, 8);
        if (nlen > (1ull << 30) || r.pos + nlen > r.n) { r.bad = 1; break; }
        size_t c = nlen < sizeof(tis[i].name) - 1 ? (size_t)nlen : sizeof(tis[i].name) - 1;
        memcpy(tis[i].name, r.p + r.pos, c);
        r.pos += nlen;
        tis[i].n_dims = (uint32_t)rd_u(&r, 4);
        if (tis[i].n_dims == 0 || tis[i].n_dims > 8) { r.bad = 1; break; }
        for (uint32_t d = 0; d < tis[i].n_dims; ++d) tis[i].dims[d] = rd_u(&r, 8);
        tis[i].type = (uint32_t)rd_u(&r, 4);
        tis[i].offset = rd_u(&r, 8);
    }
    if (r.bad) { set_err(err, errlen, "Unexpected end of GGUF file"); free(metas); free(tis); or_g3_close(m); return NULL; }
    uint64_t data_offset = (r.pos + alignment - 1) / alignment * alignment;
    m->data = m->file + data_offset;
    m->data_bytes = m->file_size - data_offset;
    #define TFIND(namestr) ({ const tinfo_t* _t = NULL; for (uint64_t _i = 0; _i < n_tensors; ++_i) if (!strcmp(tis[_i].name, namestr)) { _t = &tis[_i]; break; } _t; })

    const meta_t* arch = FIND("general.architecture");
    if (!arch || arch->kind != 4 || strcmp(arch->str, "gemma3")) { set_err(err, errlen, "Gemma3Model requires general.architecture=gemma3"); goto fail; }
    {
        const char* u32keys[] = { "gemma3.context_length", "gemma3.embedding_length", "gemma3.block_count",
            "gemma3.feed_forward_length", "gemma3.attention.head_count", "gemma3.attention.head_count_kv",
            "gemma3.attention.key_length", "gemma3.attention.value_length" };
        uint32_t* dst[] = { &m->info.context_length, &m->info.embedding_length, &m->info.block_count,
            &m->info.feed_forward_length, &m->info.head_count, &m->info.head_count_kv, &m->info.head_dim, &m->info.value_dim };
        for (int i = 0; i < 8; ++i) {
            const meta_t* v = FIND(u32keys[i]);
            if (!v || (v->kind != 1 && !(v->kind == 2 && v->i >= 0))) { set_err(err, errlen, "Missing/invalid Gemma 3 metadata: %s", u32keys[i]); goto fail; }
            *dst[i] = (uint32_t)(v->kind == 1 ? v->u : (uint64_t)v->i);
        }
        const meta_t* eps = FIND("gemma3.attention.layer_norm_rms_epsilon");
        if (!eps || eps->kind != 3) { set_err(err, errlen, "Missing Gemma 3 metadata: gemma3.attention.layer_norm_rms_epsilon"); goto fail; }
        m->info.rms_epsilon = (float)eps->f;
        const meta_t* sw = FIND("gemma3.attention.sliding_window");
        m->info.sliding_window = (sw && (sw->kind == 1 || (sw->kind == 2 && sw->i >= 0))) ? (uint32_t)(sw->kind == 1 ? sw->u : (uint64_t)sw->i) : 0;
        m->info.global_rope_base = 1.0e6f;
        m->info.local_rope_base = 1.0e4f;
        const meta_t* rb = FIND("gemma3.rope.freq_base");
        if (rb && rb->kind == 3 && isfinite(rb->f) && rb->f > 0.0) m->info.global_rope_base = (float)rb->f;
        const meta_t* eos = FIND("tokenizer.ggml.eos_token_id");
        m->info.eos_id = eos ? (uint32_t)(eos->kind == 1 ? eos->u : (uint64_t)eos->i) : 1u;
        const meta_t* bos = FIND("tokenizer.ggml.bos_token_id");
        m->info.bos_id = bos ? (uint32_t)(bos->kind == 1 ? bos->u : (uint64_t)bos->i) : 2u;
    }
    {
        const tinfo_t* emb = TFIND("token_embd.weight");
        if (!emb) { set_err(err, errlen, "Missing Gemma 3 tensor: token_embd.weight"); goto fail; }
        if (emb->type != 8 || emb->n_dims != 2 || emb->dims[0] != m->info.embedding_length) { set_err(err, errlen, "Unsupported token_embd.weight layout"); goto fail; }
        m->info.vocab_size = (uint32_t)emb->dims[1];
        m->token_embd = emb->offset;
        if (m->info.head_count_kv != 1 || m->info.value_dim != m->info.head_dim) { set_err(err, errlen, "Current Gemma 3 decoder requires one KV head and equal key/value head dimensions"); goto fail; }
        if (m->info.head_dim > 512u) { set_err(err, errlen, "oracle: head_dim above 512 is not supported"); goto fail; }
        const tinfo_t* on = TFIND("output_norm.weight");
        if (!on || on->type != 0) { set_err(err, errlen, "Missing Gemma 3 tensor: output_norm.weight"); goto fail; }
        m->output_norm = (const float*)(m->data + on->offset);
    }
    m->emb_scale = sqrtf((float)m->info.embedding_length);
    m->attn_scale = 1.0f / sqrtf((float)m->info.head_dim);
    m->inv_local = (float*)malloc(sizeof(float) * m->info.head_dim / 2);
    m->inv_global = (float*)malloc(sizeof(float) * m->info.head_dim / 2);
    or_rope_inv_freq(m->info.head_dim, m->info.local_rope_base, m->inv_local);
    or_rope_inv_freq(m->info.head_dim, m->info.global_rope_base, m->inv_global);
    m->layers = (or_layer_t*)calloc(m->info.block_count, sizeof(or_layer_t));
    for (uint32_t l = 0; l < m->info.block_count; ++l) {
        or_layer_t* L = &m->layers[l];
        char name[96];
        const char* q8names[7] = { "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down" };
        uint64_t* q8dst[7] = { &L->q, &L->k, &L->v, &L->o, &L->gate, &L->up, &L->down };
        for (int i = 0; i < 7; ++i) {
            snprintf(name, sizeof name, "blk.%u.%s.weight", l, q8names[i]);
            const tinfo_t* t = TFIND(name);
            if (!t || t->type != 8) { set_err(err, errlen, "Missing Gemma 3 tensor: %s", name); goto fail; }
            *q8dst[i] = t->offset;
        }
        const char* fnames[6] = { "attn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm" };
        const float** fdst[6] = { &L->attn_norm, &L->q_norm, &L->k_norm, &L->post_attn_norm, &L->ffn_norm, &L->post_ffw_norm };
        for (int i = 0; i < 6; ++i) {
            snprintf(name, sizeof name, "blk.%u.%s.weight", l, fnames[i]);
            const tinfo_t* t = TFIND(name);
            if (!t || t->type != 0) { set_err(err, errlen, "Missing Gemma 3 tensor: %s", name); goto fail; }
            *fdst[i] = (const float*)(m->data + t->offset);
        }
        L->global = ((l + 1u) % 6u) == 0u;                       /* src/gemma3.cpp:1301-1307 */
        L->cap = (!L->global && m->info.sliding_window) ? m->info.sliding_window : 0;
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        if (tis[i].offset % alignment) { set_err(err, errlen, "GGUF tensor offset is not aligned: %s", tis[i].name); goto fail; }
        if (tis[i].offset + tensor_bytes(&tis[i]) > m->data_bytes) { set_err(err, errlen, "GGUF tensor payload lies beyond end of file: %s", tis[i].name); goto fail; }
    }
    free(metas);
    free(tis);
    return m;
fail:
    free(metas);
    free(tis);
    or_g3_close(m);
    return NULL;
}

void or_g3_close(or_g3* m) {
    if (!m) return;
    if (m->layers)
        for (uint32_t l = 0; l < m->info.block_count; ++l) { free(m->layers[l].keys); free(m->layers[l].vals); }
    free(m->layers);
    free(m->inv_local);
    free(m->inv_global);
    free(m->file);
    free(m);
}

void or_g3_get_info(const or_g3* m, or_g3_info* info) { *info = m->info; }
const char* or_g3_error(const or_g3* m) { return m->err; }

void or_g3_reset(or_g3* m) {
    for (uint32_t l = 0; l < m->info.block_count; ++l) { m->layers[l].start = 0; m->layers[l].count = 0; }
    m->next_pos = 0;
}

void or_g3_set_kv_format(or_g3* m, int fmt) {
    m->kv_fmt = fmt == 1 || fmt == 2 ? fmt : 0;
    or_g3_reset(m);
}

void or_g3_set_kv_f16(or_g3* m, int on) { or_g3_set_kv_format(m, on ? 1 : 0); }

void or_g3_set_taps(or_g3* m, const or_g3_taps* taps) {
    m->tapping = taps != NULL;
    if (taps) m->taps = *taps;
    else memset(&m->taps, 0, sizeof m->taps);
}

/* Copies n floats into tap array a at row l (row length n), when that tap is set. */
static void tap_row(float* a, uint32_t l, const float* src, uint32_t n) {
    if (a) memcpy(a + (size_t)l * n, src, sizeof(float) * n);
}

/* push_back then pop_front while size > window (src/gemma3.cpp:1590-1600). */
static int kv_push(or_layer_t* L, const float* k_in, const float* v_in, uint32_t hd, int kv_fmt) {
    float kr[512], vr[512];   /* hd <= 512 (checked at open) */
    const float* k = k_in;
    const float* v = v_in;
    if (kv_fmt == 1) {   /* the fp16 cache holds the rounded values */
        for (uint32_t i = 0; i < hd; ++i) {
            kr[i] = or_f16_to_f32(or_f32_to_f16_rne(k_in[i]));
            vr[i] = or_f16_to_f32(or_f32_to_f16_rne(v_in[i]));
        }
        k = kr;
        v = vr;
    } else if (kv_fmt == 2) {   /* and the bf16 cache its rounded values */
        for (uint32_t i = 0; i < hd; ++i) {
            kr[i] = or_bf16_to_f32(or_f32_to_bf16_rne(k_in[i]));
            vr[i] = or_bf16_to_f32(or_f32_to_bf16_rne(v_in[i]));
        }
        k = kr;
        v = vr;
    }
    if (L->cap) {
        if (!L->keys) {
            L->keys = (float*)malloc(sizeof(float) * (size_t)L->cap * hd);
            L->vals = (float*)malloc(sizeof(float) * (size_t)L->cap * hd);
        }
        uint32_t slot;
        if (L->count < L->cap) { slot = (L->start + L->count) % L->cap; L->count++; }
        else { slot = L->start; L->start = (L->start + 1) % L->cap; }
        memcpy(L->keys + (size_t)slot * hd, k, sizeof(float) * hd);
        memcpy(L->vals + (size_t)slot * hd, v, sizeof(float) * hd);
        return 0;
    }
    static const uint32_t kChunk = 1024;
    if (L->count % kChunk == 0) {
        size_t n = (size_t)(L->count + kChunk) * hd;
        float* nk = (float*)realloc(L->keys, sizeof(float) * n);
        float* nv = (float*)realloc(L->vals, sizeof(float) * n);
        if (!nk || !nv) return -1;
        L->keys = nk;
        L->vals = nv;
    }
    memcpy(L->keys + (size_t)L->count * hd, k, sizeof(float) * hd);
    memcpy(L->vals + (size_t)L->count * hd, v, sizeof(float) * hd);
    L->count++;
    return 0;
}

static int decode_impl(or_g3* m, uint32_t token, uint32_t pos, int want_logits,
                       float* hidden_out, float* logits_out, uint32_t* am_i, float* am_v) {
    const or_g3_info* c = &m->info;
    if (pos != m->next_pos) { set_err(m->err, sizeof m->err, "Gemma 3 decode positions must be contiguous"); return -1; }
    if (pos >= c->context_length) { set_err(m->err, sizeof m->err, "Gemma 3 context length exceeded"); return -1; }
    if (token >= c->vocab_size) { set_err(m->err, sizeof m->err, "Token id is outside Gemma 3 vocabulary"); return -2; }
    const uint32_t d = c->embedding_length, hd = c->head_dim, H = c->head_count, F = c->feed_forward_length;
    const uint32_t half = hd / 2u, lanes = m->lanes;
    const float eps = c->rms_epsilon;
    int rc = 0;
    float* hidden = (float*)malloc(sizeof(float) * d);
    float* xn = (float*)malloc(sizeof(float) * d);
    float* qkv = (float*)malloc(sizeof(float) * (H + 2) * hd);
    float* att = (float*)malloc(sizeof(float) * H * hd);
    float* o = (float*)malloc(sizeof(float) * d);
    float* gate = (float*)malloc(sizeof(float) * F);
    float* up = (float*)malloc(sizeof(float) * F);
    float* f = (float*)malloc(sizeof(float) * d);
    float *lc = (float*)malloc(sizeof(float) * half), *ls = (float*)malloc(sizeof(float) * half);
    float *gc = (float*)malloc(sizeof(float) * half), *gs = (float*)malloc(sizeof(float) * half);
    float *kbuf = NULL, *vbuf = NULL;

    /* token_embedding: read_q8_0_row * embedding_scale (src/gemma3.cpp:1106-1136). */
    or_q8_dequant(m->data + m->token_embd + (uint64_t)token * (d / 32u) * 34u, d / 32u, hidden);
    for (uint32_t i = 0; i < d; ++i) hidden[i] *= m->emb_scale;
    or_rope_table(m->inv_local, half, pos, lc, ls);
    or_rope_table(m->inv_global, half, pos, gc, gs);

    for (uint32_t l = 0; l < c->block_count; ++l) {
        or_layer_t* L = &m->layers[l];
        or_rms_norm_into(hidden, L->attn_norm, xn, d, eps);
        float* q = qkv;
        float* k = qkv + (size_t)H * hd;
        float* v = k + hd;
        or_q8_matvec_lanes(m->data + L->q, xn, q, d, (uint64_t)H * hd, lanes);
        or_q8_matvec_lanes(m->data + L->k, xn, k, d, hd, lanes);
        or_q8_matvec_lanes(m->data + L->v, xn, v, d, hd, lanes);
        if (m->tapping) {
            tap_row(m->taps.xn, l, xn, d);
            tap_row(m->taps.q_proj, l, q, H * hd);
            tap_row(m->taps.k_proj, l, k, hd);
            tap_row(m->taps.v_proj, l, v, hd);
        }
        or_rms_norm_heads(q, L->q_norm, H, hd, eps);
        or_rms_norm_heads(k, L->k_norm, 1, hd, eps);
        or_apply_rope(q, H, hd, L->global ? gc : lc, L->global ? gs : ls);
        or_apply_rope(k, 1, hd, L->global ? gc : lc, L->global ? gs : ls);
        if (kv_push(L, k, v, hd, m->kv_fmt)) { set_err(m->err, sizeof m->err, "out of memory"); rc = -3; goto done; }
        const uint32_t hist = L->count;
        const float *K = L->keys, *V = L->vals;
        if (L->cap && L->start) { /* gather the ring in time order */
            if (!kbuf) { kbuf = (float*)malloc(sizeof(float) * (size_t)L->cap * hd); vbuf = (float*)malloc(sizeof(float) * (size_t)L->cap * hd); }
            for (uint32_t t = 0; t < hist; ++t) {
                uint32_t slot = (L->start + t) % L->cap;
                memcpy(kbuf + (size_t)t * hd, L->keys + (size_t)slot * hd, sizeof(float) * hd);
                memcpy(vbuf + (size_t)t * hd, L->vals + (size_t)slot * hd, sizeof(float) * hd);
            }
            K = kbuf;
            V = vbuf;
        }
        if (m->tapping) {
            tap_row(m->taps.q_att, l, q, H * hd);
            const uint32_t cap = m->taps.hist_cap, rows = hist < cap ? hist : cap;
            if (m->taps.keys) memcpy(m->taps.keys + (size_t)l * cap * hd, K, sizeof(float) * rows * hd);
            if (m->taps.values) memcpy(m->taps.values + (size_t)l * cap * hd, V, sizeof(float) * rows * hd);
            if (m->taps.history) m->taps.history[l] = hist;
        }
        if (or_attention(q, K, V, hist, H, hd, m->attn_scale, att)) { set_err(m->err, sizeof m->err, "Gemma 3 attention softmax failed"); rc = -4; goto done; }
        if (m->tapping) tap_row(m->taps.att, l, att, H * hd);
        or_q8_matvec_lanes(m->data + L->o, att, o, H * hd, d, lanes);
        or_rms_norm_inplace(o, L->post_attn_norm, d, eps);
        for (uint32_t i = 0; i < d; ++i) o[i] += hidden[i];              /* add_inplace(o, hidden) */
        memcpy(hidden, o, sizeof(float) * d);
        or_rms_norm_into(hidden, L->ffn_norm, xn, d, eps);
        /* run_staged_ffn: gate/up, gelu_mul, down, all on the narrow pipeline (:1722-1801). */
        or_q8_matvec_lanes(m->data + L->gate, xn, gate, d, F, lanes);
        or_q8_matvec_lanes(m->data + L->up, xn, up, d, F, lanes);
        or_gelu_mul(gate, up, F);
        or_q8_matvec_lanes(m->data + L->down, gate, f, F, d, lanes);
        or_rms_norm_inplace(f, L->post_ffw_norm, d, eps);
        for (uint32_t i = 0; i < d; ++i) f[i] += hidden[i];
        memcpy(hidden, f, sizeof(float) * d);
        for (uint32_t i = 0; i < d; ++i)
            if (!isfinite(hidden[i])) { set_err(m->err, sizeof m->err, "Non-finite value after Gemma 3 block %u", l); rc = -5; goto done; }
    }
    or_rms_norm_inplace(hidden, m->output_norm, d, eps);
    if (want_logits) {
        float* logits = logits_out ? logits_out : (float*)malloc(sizeof(float) * c->vocab_size);
        or_q8_matvec_lanes(m->data + m->token_embd, hidden, logits, d, c->vocab_size, lanes);
        uint32_t ai;
        float av;
        or_argmax(logits, c->vocab_size, &ai, &av);
        if (!logits_out) free(logits);
        if (ai >= c->vocab_size || !isfinite(av)) { set_err(m->err, sizeof m->err, "GPU argmax produced invalid result"); rc = -6; goto done; }
        if (am_i) *am_i = ai;
        if (am_v) *am_v = av;
    }
    if (hidden_out) memcpy(hidden_out, hidden, sizeof(float) * d);
    m->next_pos++;
done:
    free(hidden); free(xn); free(qkv); free(att); free(o); free(gate); free(up); free(f);
    free(lc); free(ls); free(gc); free(gs); free(kbuf); free(vbuf);
    return rc;
}

int or_g3_decode(or_g3* m, uint32_t token, uint32_t pos, int want_logits,
                 float* hidden_out, float* logits_out, uint32_t* argmax_index, float* argmax_value) {
    int rc = decode_impl(m, token, pos, want_logits, hidden_out, logits_out, argmax_index, argmax_value);
    /* reset_cache on any exception inside the step's try block (src/gemma3.cpp:1476-1881);
     * the position checks before it (:1467-1474, rc -1) leave the cache alone */
    if (rc && rc != -1) {
        for (uint32_t l = 0; l < m->info.block_count; ++l) { m->layers[l].start = 0; m->layers[l].count = 0; }
        m->next_pos = 0;
    }
    return rc;
}

/* src/gemma3.cpp:2080-2149. */
int or_g3_generate(or_g3* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                   uint32_t* out_tokens, uint32_t* n_out) {
    or_g3_reset(m);
    *n_out = 0;
    if (max_new == 0) return 0;
    if (n_prompt == 0) { set_err(m->err, sizeof m->err, "Gemma 3 prompt produced no input tokens"); return -1; }
    uint32_t pos = 0, am = 0;
    float av;
    for (uint32_t i = 0; i < n_prompt; ++i) {
        int last = i + 1 == n_prompt;
        int rc = or_g3_decode(m, prompt[i], pos++, last, NULL, NULL, &am, &av);
        if (rc) return rc;
    }
    uint32_t cur = 0;
    for (uint32_t i = 0; i < max_new; ++i) {
        if (i) {
            int rc = or_g3_decode(m, cur, pos++, 1, NULL, NULL, &am, &av);
            if (rc) return rc;
        }
        cur = am;
        out_tokens[(*n_out)++] = cur;
        if (cur == m->info.eos_id) break;
    }
    return 0;
}
