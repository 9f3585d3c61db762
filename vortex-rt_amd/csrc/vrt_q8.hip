// vrt_q8.hip -- context/memory runtime and the standalone Q8_0 kernels of the C ABI.
//
// Replaces the reference's Vulkan runtime (src/vulkan_context.cpp, src/buffer.cpp) and
// the pipelines of src/q8_matvec.cpp / src/argmax.cpp with HIP on one in-order stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>

#include "vrt_internal.hpp"
#include "vrt_q8_device.hpp"

namespace vrt {

static thread_local std::string t_error;

// Workspace of vrt_q8_ffn_noalloc: [h | up] of up to kFfnNoAllocMax FFN rows, one copy per GPU
// (128 KiB, held until the process ends). Host code never uses this name as an address: the
// device address comes from hipGetSymbolAddress at context creation (vrt_ctx::ffn_scratch).
constexpr uint32_t kFfnNoAllocMax = 16384;
static __device__ __align__(256) float scratch[2 * kFfnNoAllocMax];

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_error = buf;
    return code;
}

void clear_error() { t_error.clear(); }

bool mv_shape(uint32_t K, MvShape* out) {
    const uint32_t nblk = K / 32u;
    if (nblk == 0) return false;
    if (nblk <= 64) {
        int S = 1;
        while (static_cast<uint32_t>(S) < nblk) S <<= 1;
        *out = {S, 1};
        return true;
    }
    const uint32_t nb = (nblk + 63u) / 64u;
    if (nb <= 2) *out = {64, 2};
    else if (nb <= 4) *out = {64, 4};
    else if (nb <= 8) *out = {64, 8};
    else return false;
    return true;
}

// ---------------------------------------------------------------------------------------
// Generic matvec: y[v] = row_v(W) . x over a virtual row space.
// ---------------------------------------------------------------------------------------

template <int S, int NB, int U>
__global__ void __launch_bounds__(256) k_matvec(RowSpace rs, uint64_t row_bytes, uint32_t K, const uint8_t* w_end,
                                                const float* __restrict__ x, float* __restrict__ y,
                                                uint32_t rows_per_wg) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = reinterpret_cast<float*>(smem);
    LimbLds L{reinterpret_cast<int8_t*>(xs + K), reinterpret_cast<int8_t*>(xs + K) + K,
              reinterpret_cast<int8_t*>(xs + K) + 2 * K, reinterpret_cast<float*>(reinterpret_cast<int8_t*>(xs + K) + 3 * K)};
    for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    build_limbs(xs, K, L, blockDim.x >> 6);
    const uint32_t nblk = K >> 5;
    const uint32_t sl = (threadIdx.x & 63u) % S;
    XLimb xl[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        const uint32_t b = sl + static_cast<uint32_t>(n) * S;
        if (b < nblk) load_limb(L, b, xl[n]);
    }
    const uint32_t v0 = blockIdx.x * rows_per_wg;
    const uint32_t v1 = min(rs.total, v0 + rows_per_wg);
    if (v0 >= v1) return;
    stream_rows<S, NB, U>(rs, row_bytes, nblk, w_end, xl, v0, v1, [&](uint32_t v, float val) { y[v] = val; });
}

static size_t matvec_smem(uint32_t K) {
    // xs fp32[K] + limbs int8[3K] + scales fp32[K/32], 16-byte rounded
    return (static_cast<size_t>(K) * 4 + static_cast<size_t>(K) * 3 + (K / 32u) * 4 + 15) & ~size_t(15);
}

template <int S, int NB, int U>
static int launch_mv_t(hipStream_t stream, const RowSpace& rs, uint64_t row_bytes, uint32_t K, const uint8_t* w_end,
                       const float* x, float* y) {
    constexpr uint32_t rpw = 64u / S;
    const uint32_t unit = rpw * 4u;  // rows per block pass (4 waves)
    uint32_t groups = (rs.total + unit - 1u) / unit;
    uint32_t grid = std::min<uint32_t>(groups, 2048u);
    uint32_t per = (groups + grid - 1u) / grid * unit;
    grid = (rs.total + per - 1u) / per;
    const size_t smem = matvec_smem(K);
    hipLaunchKernelGGL((k_matvec<S, NB, U>), dim3(grid), dim3(256), smem, stream, rs, row_bytes, K, w_end, x, y, per);
    VRT_HIP_CHECK(hipGetLastError());
    return VRT_OK;
}

int launch_matvec(hipStream_t stream, const uint8_t* const* bases, const uint32_t* rows, uint32_t nseg,
                  int interleave, uint32_t K, const uint8_t* w_end, const float* x, float* y) {
    MvShape sh;
    VRT_REQUIRE(mv_shape(K, &sh), "Q8MatVecPipeline input_dim %u is outside the supported range (32..16384)", K);
    VRT_REQUIRE(nseg >= 1 && nseg <= static_cast<uint32_t>(kMaxSeg), "Q8 matvec segment count must be 1..%d", kMaxSeg);
    RowSpace rs{};
    uint64_t total = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        rs.base[i] = bases[i];
        rs.rows[i] = rows[i];
        rs.first[i] = static_cast<uint32_t>(total);
        total += rows[i];
    }
    VRT_REQUIRE(total <= 0x7fffffffu, "Q8 matvec output dimension too large");
    rs.nseg = nseg;
    rs.total = static_cast<uint32_t>(total);
    rs.interleave = interleave ? 1u : 0u;
    const uint64_t row_bytes = static_cast<uint64_t>(K / 32u) * 34u;
    switch (sh.S * 16 + sh.NB) {
    case 1 * 16 + 1: return launch_mv_t<1, 1, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 2 * 16 + 1: return launch_mv_t<2, 1, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 4 * 16 + 1: return launch_mv_t<4, 1, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 8 * 16 + 1: return launch_mv_t<8, 1, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 16 * 16 + 1: return launch_mv_t<16, 1, 4>(stream, rs, row_bytes, K, w_end, x, y);
    case 32 * 16 + 1: return launch_mv_t<32, 1, 4>(stream, rs, row_bytes, K, w_end, x, y);
    case 64 * 16 + 1: return launch_mv_t<64, 1, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 64 * 16 + 2: return launch_mv_t<64, 2, 2>(stream, rs, row_bytes, K, w_end, x, y);
    case 64 * 16 + 4: return launch_mv_t<64, 4, 1>(stream, rs, row_bytes, K, w_end, x, y);
    case 64 * 16 + 8: return launch_mv_t<64, 8, 1>(stream, rs, row_bytes, K, w_end, x, y);
    default: return set_error(VRT_ERR_INVALID, "unsupported Q8 matvec shape");
    }
}

// ---------------------------------------------------------------------------------------
// Elementwise, argmax, quantiser, dequantiser.
// ---------------------------------------------------------------------------------------

// src/gemma3.cpp:1440-1452 == shaders/gelu_mul.comp:23-31, evaluated in the reference's
// operation order (no contraction).
__device__ __forceinline__ float gelu_tanh_dev(float x) {
#pragma clang fp contract(off)
    const float kSqrt2OverPi = 0.7978845608028654f;
    const float kCubic = 0.044715f;
    const float cubic = x * x * x;
    return 0.5f * x * (1.0f + tanhf(kSqrt2OverPi * (x + kCubic * cubic)));
}

__global__ void __launch_bounds__(256) k_gelu_mul(float* __restrict__ gate, const float* __restrict__ up, uint32_t n) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = gelu_tanh_dev(gate[i]) * up[i];
}

// Gate/up half of the fused FFN (src/q8_matvec.cpp:1360-2004 with shaders/gelu_mul.comp as its
// epilogue): pair i is gate row i and up row i, computed by two neighbouring row slots of one
// wave (S <= 32, so a wave holds whole pairs); the even slot then writes h[i] = gelu_tanh(gate)
// * up (and up[i] for the workspace image). Pairs [pairs_per_wg * blockIdx.x, ...) per workgroup.
template <int S, int NB, int U>
__global__ void __launch_bounds__(256) k_ffn_gateup(const uint8_t* gate_w, const uint8_t* up_w, uint64_t row_bytes,
                                                    uint32_t K, const uint8_t* w_end, const float* __restrict__ x,
                                                    float* __restrict__ h, float* __restrict__ up_out, uint32_t F,
                                                    uint32_t pairs_per_wg) {
#pragma clang fp contract(off)
    static_assert(S <= 32, "a wave must hold whole gate/up pairs");
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = reinterpret_cast<float*>(smem);
    LimbLds L{reinterpret_cast<int8_t*>(xs + K), reinterpret_cast<int8_t*>(xs + K) + K,
              reinterpret_cast<int8_t*>(xs + K) + 2 * K, reinterpret_cast<float*>(reinterpret_cast<int8_t*>(xs + K) + 3 * K)};
    for (uint32_t i = threadIdx.x; i < K; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    build_limbs(xs, K, L, blockDim.x >> 6);
    const uint32_t nblk = K >> 5;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const uint32_t slot = lane / S, sl = lane % S;
    XLimb xl[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        const uint32_t b = sl + static_cast<uint32_t>(n) * S;
        if (b < nblk) load_limb(L, b, xl[n]);
    }
    constexpr uint32_t RPW = 64u / S;   // virtual rows per wave pass: RPW / 2 pairs
    const uint32_t v_begin = 2u * blockIdx.x * pairs_per_wg;
    const uint32_t v_end = min(2u * F, v_begin + 2u * pairs_per_wg);
    if (v_begin >= v_end) return;
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
            const uint8_t* rp = ((vrow[u] & 1u) ? up_w : gate_w) + static_cast<uint64_t>(vrow[u] >> 1) * row_bytes;
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
            const float tot = slot_sum<S>(acc);
            // the up total of this pair, from the odd slot next to it (every lane takes part)
            const float upv = __shfl(tot, static_cast<int>(min(lane + static_cast<uint32_t>(S), 63u)));
            if (live[u] && sl == 0u && (slot & 1u) == 0u) {
                const uint32_t i = vrow[u] >> 1;
                h[i] = gelu_tanh_dev(tot) * upv;
                up_out[i] = upv;
            }
        }
    }
}

struct AmPartial {
    float value;
    uint32_t index;
};

// Per-block strided scan and block reduction into parts[blockIdx.x]; k_argmax_final, a launch
// of its own (so the partials are visible without a device-wide fence), reduces the partials.
__global__ void __launch_bounds__(256) k_argmax(const float* __restrict__ x, uint32_t n, AmPartial* parts) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float v = x[i];
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    wave_argmax(bv, bi);
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0u) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < (blockDim.x >> 6); ++k)
            if (am_better(sv[k], si[k], sv[0], si[0])) { sv[0] = sv[k]; si[0] = si[k]; }
        parts[blockIdx.x] = {sv[0], si[0]};
    }
}

__global__ void __launch_bounds__(256) k_argmax_final(const AmPartial* parts, uint32_t nparts, vrt_argmax_result* out) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t k = threadIdx.x; k < nparts; k += blockDim.x) {
        const AmPartial p = parts[k];
        if (am_better(p.value, p.index, bv, bi)) { bv = p.value; bi = p.index; }
    }
    wave_argmax(bv, bi);
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0u) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < (blockDim.x >> 6); ++k)
            if (am_better(sv[k], si[k], sv[0], si[0])) { sv[0] = sv[k]; si[0] = si[k]; }
        out->index = si[0];
        out->value = sv[0];
    }
}

// src/q8_test_main.cpp:18-41 restated on integers (identical bits on any IEEE target).
__device__ __forceinline__ uint32_t f32_to_f16_ref(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mantissa = x & 0x7fffffu;
    const int exponent = static_cast<int>((x >> 23) & 0xffu) - 127 + 15;
    if (exponent <= 0) {
        if (exponent < -10) return sign;
        mantissa = (mantissa | 0x800000u) >> (1 - exponent);
        return (sign + ((mantissa + 0x1000u) >> 13)) & 0xffffu;
    }
    if (exponent >= 31) return sign | 0x7c00u;
    return sign | (static_cast<uint32_t>(exponent) << 10) | ((mantissa + 0x1000u) >> 13);
}

// One half-wave per 32-value block, one lane per value.
__global__ void __launch_bounds__(256) k_quantize(const float* __restrict__ x, uint64_t nblocks, uint32_t variant,
                                                  uint8_t* __restrict__ out) {
    const uint64_t blk = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 5;
    const uint32_t k = threadIdx.x & 31u;
    const bool live = blk < nblocks;
    const float v = live ? x[blk * 32u + k] : 0.0f;
    // abs_max starts at 0 and std::max(abs_max, fabs(v)) never takes a NaN: fmaxf(0, .)
    float amax = fmaxf(0.0f, fabsf(v));
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (!live) return;
    float scale = amax / 127.0f;
    if (variant == 1u && amax == 0.0f) scale = 1.0f;
    const uint32_t half = f32_to_f16_ref(scale);
    const float div = variant == 1u ? half_bits_to_float(half) : scale;
    const float r = rintf(v / div);
    // static_cast<int> of NaN or |r| >= 2^31 is INT_MIN on x86-64; clamp -> -127
    const int q = !(fabsf(r) < 2147483648.0f) ? -127 : max(-127, min(127, static_cast<int>(r)));
    uint8_t* o = out + blk * 34u;
    o[2 + k] = static_cast<uint8_t>(static_cast<int8_t>(q));
    if (k == 0) { o[0] = static_cast<uint8_t>(half & 0xffu); o[1] = static_cast<uint8_t>(half >> 8); }
}

__global__ void __launch_bounds__(256) k_dequantize(const uint8_t* __restrict__ blocks, uint64_t nblocks,
                                                    float* __restrict__ out) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= nblocks * 32u) return;
    const uint8_t* b = blocks + (i >> 5) * 34u;
    const float s = half_bits_to_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8));
    out[i] = s * static_cast<float>(static_cast<int8_t>(b[2 + (i & 31u)]));
}

// The gate/up launch of the fused FFN into the workspace image ws = [h | up]: gelu_tanh(gate) *
// up into ws[0..F), up into ws[F..2F). K of more than 32 blocks (64-lane row slots) runs the
// gate/up matvec and the GELU as two kernels.
static int launch_ffn_gateup(hipStream_t stream, const uint8_t* gate_w, const uint8_t* up_w, uint32_t K, uint32_t F,
                             const uint8_t* w_end, const float* x, float* ws) {
    float* h = ws;
    float* up_out = ws + F;
    MvShape sh;
    VRT_REQUIRE(mv_shape(K, &sh), "Q8 fused FFN input_dim %u is outside the supported range (32..16384)", K);
    const uint64_t row_bytes = static_cast<uint64_t>(K / 32u) * 34u;
    auto go = [&](auto kern, uint32_t S) -> int {
        const uint32_t pairs_per_pass = 4u * (64u / S) / 2u;   // 4 waves per workgroup
        uint32_t groups = (F + pairs_per_pass - 1u) / pairs_per_pass;
        uint32_t grid = std::min<uint32_t>(groups, 2048u);
        const uint32_t per = (groups + grid - 1u) / grid * pairs_per_pass;
        grid = (F + per - 1u) / per;
        hipLaunchKernelGGL(kern, dim3(grid), dim3(256), matvec_smem(K), stream, gate_w, up_w, row_bytes, K, w_end, x, h,
                           up_out, F, per);
        VRT_HIP_CHECK(hipGetLastError());
        return VRT_OK;
    };
    switch (sh.S) {
    case 1: return go(k_ffn_gateup<1, 1, 2>, 1);
    case 2: return go(k_ffn_gateup<2, 1, 2>, 2);
    case 4: return go(k_ffn_gateup<4, 1, 2>, 4);
    case 8: return go(k_ffn_gateup<8, 1, 2>, 8);
    case 16: return go(k_ffn_gateup<16, 1, 4>, 16);
    case 32: return go(k_ffn_gateup<32, 1, 4>, 32);
    default: {
        const uint8_t* gu[2] = {gate_w, up_w};
        const uint32_t gu_rows[2] = {F, F};
        if (int rc = launch_matvec(stream, gu, gu_rows, 2, 0, K, w_end, x, ws)) return rc;
        hipLaunchKernelGGL(k_gelu_mul, dim3((F + 255u) / 256u), dim3(256), 0, stream, h, up_out, F);
        VRT_HIP_CHECK(hipGetLastError());
        return VRT_OK;
    }
    }
}

}  // namespace vrt

using namespace vrt;

// =======================================================================================
// C ABI
// =======================================================================================

extern "C" const char* vrt_last_error(void) { return t_error.c_str(); }

static bool icontains(const std::string& hay, const std::string& needle) {
    std::string h(hay), n(needle);
    for (auto& c : h) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    for (auto& c : n) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    return h.find(n) != std::string::npos;
}

extern "C" int vrt_ctx_create(const char* selector, vrt_ctx** out) {
    VRT_REQUIRE(out != nullptr, "vrt_ctx_create: null output");
    *out = nullptr;
    int count = 0;
    VRT_HIP_CHECK(hipGetDeviceCount(&count));
    VRT_REQUIRE(count > 0, "No HIP devices found");
    std::string sel = selector ? selector : "";
    if (sel.empty()) {
        const char* env = std::getenv("VORTEXRT_DEVICE");  // src/vulkan_context.cpp:119-123
        if (env) sel = env;
    }
    int dev = 0;
    if (!sel.empty()) {
        bool numeric = std::all_of(sel.begin(), sel.end(), [](char c) { return std::isdigit(static_cast<unsigned char>(c)); });
        if (numeric) {
            dev = std::atoi(sel.c_str());
            VRT_REQUIRE(dev >= 0 && dev < count, "Device index out of range: %s", sel.c_str());
        } else {
            dev = -1;
            for (int i = 0; i < count && dev < 0; ++i) {
                hipDeviceProp_t p;
                VRT_HIP_CHECK(hipGetDeviceProperties(&p, i));
                if (icontains(p.name, sel) || icontains(p.gcnArchName, sel)) dev = i;
            }
            VRT_REQUIRE(dev >= 0, "No device matches selector: %s", sel.c_str());
        }
    }
    VRT_HIP_CHECK(hipSetDevice(dev));
    hipDeviceProp_t p;
    VRT_HIP_CHECK(hipGetDeviceProperties(&p, dev));
    auto* c = new (std::nothrow) vrt_ctx();
    VRT_REQUIRE(c != nullptr, "out of memory");
    c->device = dev;
    std::snprintf(c->info.name, sizeof c->info.name, "%s", p.name);
    std::snprintf(c->info.arch, sizeof c->info.arch, "%s", p.gcnArchName);
    c->info.device_index = static_cast<uint32_t>(dev);
    c->info.vendor_id = 0x1002u;
    c->info.device_id = static_cast<uint32_t>(p.pciDeviceID);
    c->info.subgroup_size = static_cast<uint32_t>(p.warpSize);
    c->info.compute_units = static_cast<uint32_t>(p.multiProcessorCount);
    c->info.fp16 = c->info.int8 = c->info.storage8 = c->info.storage16 = 1u;
    c->info.device_local_bytes = p.totalGlobalMem;
    c->info.l2_bytes = static_cast<uint64_t>(p.l2CacheSize);
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) {
        c->scratch_bytes = 1u << 16;
        e = hipMalloc(&c->scratch, c->scratch_bytes);
        if (e == hipSuccess) e = hipMemsetAsync(c->scratch, 0, c->scratch_bytes, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    }
    if (e == hipSuccess) {   // this device's copy of the no-allocation FFN workspace (dev is current)
        void* sp = nullptr;
        e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        c->ffn_scratch = static_cast<float*>(sp);
        if (e == hipSuccess && !sp) e = hipErrorInvalidSymbol;
    }
    if (e != hipSuccess) {
        if (c->scratch) (void)hipFree(c->scratch);
        if (c->stream) (void)hipStreamDestroy(c->stream);
        delete c;
        return set_error(VRT_ERR_HIP, "context setup failed: %s", hipGetErrorString(e));
    }
    *out = c;
    return VRT_OK;
}

extern "C" int vrt_ctx_destroy(vrt_ctx* ctx) {
    if (!ctx) return VRT_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return VRT_OK;
}

extern "C" int vrt_ctx_info(const vrt_ctx* ctx, vrt_device_info* out) {
    VRT_REQUIRE(ctx && out, "vrt_ctx_info: null argument");
    *out = ctx->info;
    return VRT_OK;
}

extern "C" int vrt_alloc(vrt_ctx* ctx, uint64_t bytes, uint32_t kind, void** out) {
    VRT_REQUIRE(ctx && out, "vrt_alloc: null argument");
    VRT_REQUIRE(kind == VRT_MEM_DEVICE || kind == VRT_MEM_HOST, "vrt_alloc: unknown memory kind %u", kind);
    *out = nullptr;
    const uint64_t padded = ((bytes + 255u) & ~uint64_t(255)) + 256u;
    VRT_HIP_CHECK(hipSetDevice(ctx->device));
    void* p = nullptr;
    if (kind == VRT_MEM_DEVICE) {
        VRT_HIP_CHECK(hipMalloc(&p, padded));
        // The zero-fill goes on the context's stream, which every later copy and kernel of the
        // context uses: that stream is non-blocking, so a fill on the null stream would not be
        // ordered before them.
        hipError_t e = hipMemsetAsync(p, 0, padded, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) { (void)hipFree(p); return set_error(VRT_ERR_HIP, "hipMemsetAsync failed: %s", hipGetErrorString(e)); }
    } else {
        VRT_HIP_CHECK(hipHostMalloc(&p, padded, hipHostMallocDefault));
        std::memset(p, 0, padded);
    }
    *out = p;
    return VRT_OK;
}

extern "C" int vrt_free(vrt_ctx* ctx, void* ptr) {
    VRT_REQUIRE(ctx, "vrt_free: null context");
    if (!ptr) return VRT_OK;
    // work still queued on the context's stream may read or write the buffer
    VRT_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    hipPointerAttribute_t attr{};
    VRT_HIP_CHECK(hipPointerGetAttributes(&attr, ptr));
    if (attr.type == hipMemoryTypeHost) {
        VRT_HIP_CHECK(hipHostFree(ptr));
    } else {
        VRT_HIP_CHECK(hipFree(ptr));
    }
    return VRT_OK;
}

extern "C" int vrt_memcpy(vrt_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
    VRT_REQUIRE(ctx, "vrt_memcpy: null context");
    if (bytes == 0) return VRT_OK;
    VRT_REQUIRE(dst && src, "vrt_memcpy: null pointer");
    VRT_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    return VRT_OK;
}

extern "C" int vrt_memset(vrt_ctx* ctx, void* dst, int value, uint64_t bytes) {
    VRT_REQUIRE(ctx && dst, "vrt_memset: null argument");
    VRT_HIP_CHECK(hipMemsetAsync(dst, value, bytes, ctx->stream));
    VRT_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    return VRT_OK;
}

extern "C" int vrt_sync(vrt_ctx* ctx) {
    VRT_REQUIRE(ctx, "vrt_sync: null context");
    VRT_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    return VRT_OK;
}

extern "C" int vrt_stream(vrt_ctx* ctx, void** stream) {
    VRT_REQUIRE(ctx && stream, "vrt_stream: null argument");
    *stream = ctx->stream;
    return VRT_OK;
}

extern "C" int vrt_event_create(vrt_ctx* ctx, void** ev) {
    VRT_REQUIRE(ctx && ev, "vrt_event_create: null argument");
    hipEvent_t e;
    VRT_HIP_CHECK(hipEventCreate(&e));
    *ev = e;
    return VRT_OK;
}

extern "C" int vrt_event_record(vrt_ctx* ctx, void* ev) {
    VRT_REQUIRE(ctx && ev, "vrt_event_record: null argument");
    VRT_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev), ctx->stream));
    return VRT_OK;
}

extern "C" int vrt_event_elapsed_ms(void* a, void* b, float* ms) {
    VRT_REQUIRE(a && b && ms, "vrt_event_elapsed_ms: null argument");
    VRT_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(b)));
    VRT_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)));
    return VRT_OK;
}

extern "C" int vrt_event_destroy(void* ev) {
    if (ev) VRT_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return VRT_OK;
}

// Validation shared by the matvec entry points (src/q8_matvec.cpp:801-860).
static int check_matrix(uint64_t weights_bytes, uint32_t off, uint32_t input_dim, uint32_t output_dim, const char* who) {
    VRT_REQUIRE(input_dim != 0 && output_dim != 0, "%s dimensions must be non-zero", who);
    VRT_REQUIRE(input_dim % 32u == 0u, "%s input_dim must be divisible by 32", who);
    VRT_REQUIRE((off & 3u) == 0u, "%s weight byte offset must be 4-byte aligned", who);
    const uint64_t need = static_cast<uint64_t>(off) + static_cast<uint64_t>(output_dim) * (input_dim / 32u) * 34u;
    VRT_REQUIRE(need <= weights_bytes, "%s weight buffer is too small", who);
    return VRT_OK;
}

extern "C" int vrt_q8_matvec(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t off,
                             const float* x, float* y, uint32_t input_dim, uint32_t output_dim) {
    VRT_REQUIRE(ctx && weights && x && y, "Q8MatVecPipeline::run: null argument");
    if (int rc = check_matrix(weights_bytes, off, input_dim, output_dim, "Q8MatVecPipeline")) return rc;
    const auto* w = static_cast<const uint8_t*>(weights);
    const uint8_t* base = w + off;
    return launch_matvec(ctx->stream, &base, &output_dim, 1, 0, input_dim, w + weights_bytes, x, y);
}

extern "C" int vrt_q8_matvec_multi(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t n,
                                   const uint32_t* offs, const uint32_t* dims, uint32_t input_dim,
                                   const float* x, float* y) {
    VRT_REQUIRE(ctx && weights && offs && dims && x && y, "Q8 multi matvec: null argument");
    VRT_REQUIRE(n >= 1 && n <= static_cast<uint32_t>(kMaxSeg), "Q8 multi matvec: 1..%d matrices", kMaxSeg);
    VRT_REQUIRE(input_dim != 0 && input_dim % 32u == 0u, "Q8MatVecPipeline triplet input_dim must be non-zero and divisible by 32");
    const auto* w = static_cast<const uint8_t*>(weights);
    const uint8_t* bases[kMaxSeg];
    for (uint32_t i = 0; i < n; ++i) {
        VRT_REQUIRE(dims[i] != 0, "Q8 triplet output dimensions must be non-zero");
        VRT_REQUIRE((offs[i] & 3u) == 0u, "Q8 triplet weight offsets must be 4-byte aligned");
        VRT_REQUIRE(static_cast<uint64_t>(offs[i]) + static_cast<uint64_t>(dims[i]) * (input_dim / 32u) * 34u <= weights_bytes,
                    "Q8 triplet weight buffer is too small");
        bases[i] = w + offs[i];
    }
    return launch_matvec(ctx->stream, bases, dims, n, 0, input_dim, w + weights_bytes, x, y);
}

extern "C" int vrt_q8_ffn(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t gate_off,
                          uint32_t up_off, uint32_t down_off, uint32_t input_dim, uint32_t ffn_dim, uint32_t output_dim,
                          const float* x, float* ws, uint64_t ws_bytes, float* y) {
    VRT_REQUIRE(ctx && weights && x && ws && y, "Q8MatVecPipeline::run_staged_ffn received null buffer");
    VRT_REQUIRE(input_dim && ffn_dim && output_dim && input_dim % 32u == 0 && ffn_dim % 32u == 0,
                "Q8 fused FFN dimensions must be non-zero and Q8 aligned");
    VRT_REQUIRE(((gate_off | up_off | down_off) & 3u) == 0u, "Q8 fused FFN weight offsets must be 4-byte aligned");
    const uint64_t gate_end = gate_off + static_cast<uint64_t>(ffn_dim) * (input_dim / 32u) * 34u;
    const uint64_t up_end = up_off + static_cast<uint64_t>(ffn_dim) * (input_dim / 32u) * 34u;
    const uint64_t down_end = down_off + static_cast<uint64_t>(output_dim) * (ffn_dim / 32u) * 34u;
    VRT_REQUIRE(gate_end <= weights_bytes && up_end <= weights_bytes && down_end <= weights_bytes,
                "Q8 fused FFN weight buffer is too small");
    VRT_REQUIRE(ws_bytes >= 2ull * ffn_dim * sizeof(float), "Q8 fused FFN activation/staging buffer is too small");
    const auto* w = static_cast<const uint8_t*>(weights);
    if (int rc = launch_ffn_gateup(ctx->stream, w + gate_off, w + up_off, input_dim, ffn_dim, w + weights_bytes, x, ws))
        return rc;
    const uint8_t* dn = w + down_off;
    return launch_matvec(ctx->stream, &dn, &output_dim, 1, 0, ffn_dim, w + weights_bytes, ws, y);
}

extern "C" int vrt_q8_ffn_noalloc(vrt_ctx* ctx, const void* weights, uint64_t weights_bytes, uint32_t gate_off,
                                  uint32_t up_off, uint32_t down_off, uint32_t input_dim, uint32_t ffn_dim,
                                  uint32_t output_dim, const float* x, float* y) {
    VRT_REQUIRE(ctx && ctx->ffn_scratch, "vrt_q8_ffn_noalloc: null context");
    VRT_REQUIRE(ffn_dim <= kFfnNoAllocMax, "vrt_q8_ffn_noalloc: ffn_dim %u exceeds the static workspace (%u rows)",
                ffn_dim, kFfnNoAllocMax);
    // the same kernels as vrt_q8_ffn, on this device's static [h | up] workspace
    return vrt_q8_ffn(ctx, weights, weights_bytes, gate_off, up_off, down_off, input_dim, ffn_dim, output_dim, x,
                      ctx->ffn_scratch, 2ull * kFfnNoAllocMax * sizeof(float), y);
}

extern "C" int vrt_gelu_mul(vrt_ctx* ctx, float* gate, const float* up, uint32_t n) {
    VRT_REQUIRE(ctx && gate && up, "vrt_gelu_mul: null argument");
    if (n == 0) return VRT_OK;
    hipLaunchKernelGGL(k_gelu_mul, dim3((n + 255u) / 256u), dim3(256), 0, ctx->stream, gate, up, n);
    VRT_HIP_CHECK(hipGetLastError());
    return VRT_OK;
}

extern "C" int vrt_argmax(vrt_ctx* ctx, const float* x, uint32_t n, vrt_argmax_result* out) {
    VRT_REQUIRE(ctx && x && out, "ArgmaxPipeline: null argument");
    VRT_REQUIRE(n != 0, "ArgmaxPipeline requires non-zero input");  // src/argmax.cpp:507-511
    const uint32_t grid = std::min<uint32_t>((n + 2047u) / 2048u, 1024u);
    auto* parts = reinterpret_cast<AmPartial*>(static_cast<char*>(ctx->scratch) + 256);
    hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, ctx->stream, x, n, parts);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, ctx->stream, parts, grid, out);
    VRT_HIP_CHECK(hipGetLastError());
    return VRT_OK;
}

extern "C" int vrt_q8_quantize(vrt_ctx* ctx, const float* x, uint64_t n, uint32_t variant, void* out) {
    VRT_REQUIRE(ctx && x && out, "vrt_q8_quantize: null argument");
    VRT_REQUIRE(n % 32u == 0u, "test matrix input must be divisible by 32");
    VRT_REQUIRE(variant <= 1u, "vrt_q8_quantize: variant must be 0 or 1");
    if (n == 0) return VRT_OK;
    const uint64_t nb = n / 32u;
    const uint64_t threads = nb * 32u;
    VRT_REQUIRE((threads + 255u) / 256u <= 0x7fffffffu, "vrt_q8_quantize: input too large");
    hipLaunchKernelGGL(k_quantize, dim3(static_cast<uint32_t>((threads + 255u) / 256u)), dim3(256), 0, ctx->stream, x, nb,
                       variant, static_cast<uint8_t*>(out));
    VRT_HIP_CHECK(hipGetLastError());
    return VRT_OK;
}

extern "C" int vrt_q8_dequantize(vrt_ctx* ctx, const void* blocks, uint64_t nblocks, float* out) {
    VRT_REQUIRE(ctx && blocks && out, "vrt_q8_dequantize: null argument");
    if (nblocks == 0) return VRT_OK;
    const uint64_t n = nblocks * 32u;
    VRT_REQUIRE((n + 255u) / 256u <= 0x7fffffffu, "vrt_q8_dequantize: input too large");
    hipLaunchKernelGGL(k_dequantize, dim3(static_cast<uint32_t>((n + 255u) / 256u)), dim3(256), 0, ctx->stream,
                       static_cast<const uint8_t*>(blocks), nblocks, out);
    VRT_HIP_CHECK(hipGetLastError());
    return VRT_OK;
}
