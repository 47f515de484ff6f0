// qmag_synth.hip -- synthetic bench/test inputs (not part of the reference):
// a counter-based N(mean, std) generator and the build's fp32 -> Q4_K / Q6_K
// quantisers.  The quantisers use only exact reductions and IEEE elementwise
// ops with fusion disabled, so given the same fp32 input they reproduce the
// CPU oracle's quantiser byte for byte.
#include "qmag_internal.h"

namespace qmag {

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// N(0,1) pair for pair index p of stream `seed` (Box-Muller on two 24-bit
// uniforms; u1 in (0,1]).
__device__ __forceinline__ float2 normal2(uint64_t seed, uint64_t p)
{
    const uint64_t h = mix64(seed + (p + 1) * 0x9E3779B97F4A7C15ull);
    const float u1 = (float)((uint32_t)(h >> 40) + 1u) * (1.0f / 16777216.0f);
    const float u2 = (float)((uint32_t)(h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    float s, c;
    sincospif(2.0f * u2, &s, &c);
    return make_float2(r * c, r * s);
}

__global__ __launch_bounds__(256) void synth_normal_kernel(uint64_t seed, size_t n, float mean,
                                                           float std, float *__restrict__ out)
{
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * p >= n) return;
    const float2 z = normal2(seed, p);
    out[2 * p] = mean + std * z.x;
    if (2 * p + 1 < n) out[2 * p + 1] = mean + std * z.y;
}

__device__ __forceinline__ float clampf_(float v, float lo, float hi)
{
    return v < lo ? lo : (v > hi ? hi : v);
}

__device__ __forceinline__ uint32_t f2h_bits(float f)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// One wave quantises one 256-float block; lane l holds elements 4l..4l+3.
// Mirrors orc_quantize_q4k step by step.
__device__ void quant_q4k_wave(float4 v, uint8_t *blk)
{
#pragma clang fp contract(off)
    const int L = lane_id();
    const float e[4] = {v.x, v.y, v.z, v.w};
    float lo = 0.0f, hi = e[0];
    for (int i = 0; i < 4; i++) {
        lo = e[i] < lo ? e[i] : lo;
        hi = e[i] > hi ? e[i] : hi;
    }
    lo = group_min<8>(lo);       // sub-block j = L/8 spans 8 lanes
    hi = group_max<8>(hi);
    const float scale = (hi - lo) / 15.0f;
    const float minv = -lo;
    float maxs = group_max<64>(scale);
    float maxm = group_max<64>(minv);
    maxs = maxs > 0.0f ? maxs : 0.0f;
    maxm = maxm > 0.0f ? maxm : 0.0f;
    const uint32_t dh = f2h_bits(maxs / 63.0f), mh = f2h_bits(maxm / 63.0f);
    const float dq = h2f(dh), mq = h2f(mh);
    const uint32_t sc = dq > 0.0f ? (uint32_t)clampf_(roundf(scale / dq), 0.0f, 63.0f) : 0u;
    const uint32_t mm = mq > 0.0f ? (uint32_t)clampf_(roundf(minv / mq), 0.0f, 63.0f) : 0u;
    const float ds = dq * (float)sc;
    const float dm = mq * (float)mm;
    uint32_t packed = 0;
    for (int i = 0; i < 4; i++) {
        uint32_t q = 0;
        if (ds > 0.0f) {
            const float t = e[i] + dm;
            q = (uint32_t)clampf_(roundf(t / ds), 0.0f, 15.0f);
        }
        packed |= q << (8 * i);
    }
    // lanes with (L % 16) < 8 hold the low nibbles of qs[32g + 4(L%16) ..];
    // lane L + 8 holds the high nibbles of the same bytes
    const uint32_t hip_ = (uint32_t)__shfl_down((int)packed, 8);
    if ((L & 15) < 8) {
        const uint32_t word = packed | (hip_ << 4);
        const int g = L >> 4;
        *(uint32_t *)(blk + 16 + 32 * g + 4 * (L & 15)) = word;
    }
    uint32_t s[8], m[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        s[j] = (uint32_t)__builtin_amdgcn_readlane((int)sc, 8 * j);
        m[j] = (uint32_t)__builtin_amdgcn_readlane((int)mm, 8 * j);
    }
    if (L == 0) {
        uint32_t w[4] = {dh | (mh << 16), 0, 0, 0};
        for (int j = 0; j < 4; j++) {
            w[1] |= ((s[j] & 63) | ((s[j + 4] >> 4) << 6)) << (8 * j);
            w[2] |= ((m[j] & 63) | ((m[j + 4] >> 4) << 6)) << (8 * j);
            w[3] |= ((s[j + 4] & 15) | ((m[j + 4] & 15) << 4)) << (8 * j);
        }
        *(uint4 *)blk = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Mirrors orc_quantize_q6k.  Lane l: elements 4l..4l+3 = half n = l/32,
// quarter Q = (l%32)/8, lanes-in-quarter 4(l%8)..+3.
__device__ void quant_q6k_wave(float4 v, uint8_t *blk)
{
#pragma clang fp contract(off)
    const int L = lane_id();
    const float e[4] = {v.x, v.y, v.z, v.w};
    float a = 0.0f;
    for (int i = 0; i < 4; i++) {
        const float t = fabsf(e[i]);
        a = t > a ? t : a;
    }
    a = group_max<4>(a);                 // 16-element group = 4 lanes
    const float sf = a / 31.0f;
    float maxs = group_max<64>(sf);
    maxs = maxs > 0.0f ? maxs : 0.0f;
    const uint32_t dh = f2h_bits(maxs / 127.0f);
    const float dq = h2f(dh);
    const int sc = dq > 0.0f ? (int)clampf_(roundf(sf / dq), -128.0f, 127.0f) : 0;
    const float ds = dq * (float)sc;
    uint32_t u[4];
    for (int i = 0; i < 4; i++) {
        int q = 0;
        if (ds > 0.0f) q = (int)clampf_(roundf(e[i] / ds), -32.0f, 31.0f);
        u[i] = (uint32_t)(q + 32);
    }
    uint32_t lo4 = 0, hi2 = 0;
    for (int i = 0; i < 4; i++) {
        lo4 |= (u[i] & 15) << (8 * i);
        hi2 |= ((u[i] >> 4) & 3) << (8 * i);
    }
    const int n = L >> 5, Q = (L & 31) >> 3, l = 4 * (L & 7);
    const uint32_t lo4_up = (uint32_t)__shfl_down((int)lo4, 16);  // quarter Q+2
    const uint32_t h1 = (uint32_t)__shfl_down((int)hi2, 8);
    const uint32_t h2 = (uint32_t)__shfl_down((int)hi2, 16);
    const uint32_t h3 = (uint32_t)__shfl_down((int)hi2, 24);
    if (Q < 2) {
        const uint32_t word = lo4 | (lo4_up << 4);
        __builtin_memcpy(blk + 64 * n + 32 * Q + l, &word, 4);
    }
    if (Q == 0) {
        const uint32_t word = hi2 | (h1 << 2) | (h2 << 4) | (h3 << 6);
        __builtin_memcpy(blk + 128 + 32 * n + l, &word, 4);
    }
    if ((L & 3) == 0) blk[192 + (L >> 2)] = (uint8_t)(int8_t)sc;
    if (L == 0) {
        const uint16_t d16 = (uint16_t)dh;
        __builtin_memcpy(blk + 208, &d16, 2);
    }
}

template <int WT>
__global__ __launch_bounds__(256) void quantize_kernel(const float *__restrict__ x, size_t nblocks,
                                                       uint8_t *__restrict__ out)
{
    const size_t b = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (b >= nblocks) return;
    const float4 v = ((const float4 *)(x + b * QK_K))[lane_id()];
    if constexpr (WT == QMAG_TYPE_Q4_K)
        quant_q4k_wave(v, out + b * Q4K_BYTES);
    else
        quant_q6k_wave(v, out + b * Q6K_BYTES);
}

template <int WT>
__global__ __launch_bounds__(256) void synth_weights_kernel(uint64_t seed, size_t nblocks, float std,
                                                            uint8_t *__restrict__ out)
{
    const size_t b = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (b >= nblocks) return;
    const size_t p = (b * QK_K + 4 * (size_t)lane_id()) / 2;
    const float2 z0 = normal2(seed, p), z1 = normal2(seed, p + 1);
    const float4 v = make_float4(std * z0.x, std * z0.y, std * z1.x, std * z1.y);
    if constexpr (WT == QMAG_TYPE_Q4_K)
        quant_q4k_wave(v, out + b * Q4K_BYTES);
    else
        quant_q6k_wave(v, out + b * Q6K_BYTES);
}

}  // namespace qmag

using namespace qmag;

extern "C" int qmag_synth_normal(uint64_t seed, size_t n, float mean, float std, float *out)
{
    int st = require_ready();
    if (st) return st;
    if (!out) return fail(QMAG_ERR_ARG, "synth_normal: null");
    if (n == 0) return QMAG_OK;
    const size_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(synth_normal_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                       ctx().stream, seed, n, mean, std, out);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

extern "C" int qmag_synth_weights(uint64_t seed, size_t n, float std, int wtype, void *out)
{
    int st = require_ready();
    if (st) return st;
    if (!out || n % QK_K) return fail(QMAG_ERR_ARG, "synth_weights: n=%zu", n);
    const size_t nb = n / QK_K;
    const unsigned wgs = (unsigned)((nb + 3) / 4);
    if (wtype == QMAG_TYPE_Q4_K)
        hipLaunchKernelGGL(synth_weights_kernel<QMAG_TYPE_Q4_K>, dim3(wgs), dim3(256), 0,
                           ctx().stream, seed, nb, std, (uint8_t *)out);
    else if (wtype == QMAG_TYPE_Q6_K)
        hipLaunchKernelGGL(synth_weights_kernel<QMAG_TYPE_Q6_K>, dim3(wgs), dim3(256), 0,
                           ctx().stream, seed, nb, std, (uint8_t *)out);
    else
        return fail(QMAG_ERR_ARG, "synth_weights: wtype %d", wtype);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

extern "C" int qmag_quantize_dev(const float *x, size_t n, int wtype, void *out)
{
    int st = require_ready();
    if (st) return st;
    if (!x || !out || n % QK_K) return fail(QMAG_ERR_ARG, "quantize: n=%zu", n);
    const size_t nb = n / QK_K;
    const unsigned wgs = (unsigned)((nb + 3) / 4);
    if (wtype == QMAG_TYPE_Q4_K)
        hipLaunchKernelGGL(quantize_kernel<QMAG_TYPE_Q4_K>, dim3(wgs), dim3(256), 0, ctx().stream,
                           x, nb, (uint8_t *)out);
    else if (wtype == QMAG_TYPE_Q6_K)
        hipLaunchKernelGGL(quantize_kernel<QMAG_TYPE_Q6_K>, dim3(wgs), dim3(256), 0, ctx().stream,
                           x, nb, (uint8_t *)out);
    else
        return fail(QMAG_ERR_ARG, "quantize: wtype %d", wtype);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}
