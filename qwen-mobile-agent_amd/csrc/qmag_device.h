// qmag_device.h -- device-side building blocks for gfx950 (wave64, CDNA4).
//
// GGUF super-block layouts (src/qma.h:77-90), fp16 decode, DPP/permlane
// wave reductions, and the per-lane dot "tasks" the matvec and MoE kernels
// are built from.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define QK_K 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210

namespace qmag {

// ---------------------------------------------------------------- fp16 ----
__device__ __forceinline__ float h2f(uint32_t h16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// ------------------------------------------------------------ reductions --
// All-reduce over aligned groups of W lanes (W = 4, 8, 16, 32, 64) using DPP
// quad permutes, row mirrors and the gfx950 permlane swaps; no LDS traffic.
// Every pattern used reads a valid lane of the same row, so the move can be
// folded into the consuming add/max (one v_add_f32_dpp per step).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <- 15-i within 16

template <int W>
__device__ __forceinline__ float group_sum(float v)
{
    if constexpr (W >= 2) v += dpp_f<DPP_XOR1>(v);
    if constexpr (W >= 4) v += dpp_f<DPP_XOR2>(v);
    if constexpr (W >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp_f<DPP_MIRROR>(v);
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

template <int W>
__device__ __forceinline__ int group_sum_i(int v)
{
    if constexpr (W >= 2) v += dpp_i<DPP_XOR1>(v);
    if constexpr (W >= 4) v += dpp_i<DPP_XOR2>(v);
    if constexpr (W >= 8) v += dpp_i<DPP_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp_i<DPP_MIRROR>(v);
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        v = (int)(p[0] + p[1]);
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        v = (int)(p[0] + p[1]);
    }
    return v;
}

template <int W>
__device__ __forceinline__ float group_max(float v)
{
    if constexpr (W >= 2) v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    if constexpr (W >= 4) v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    return v;
}

template <int W>
__device__ __forceinline__ float group_min(float v)
{
    if constexpr (W >= 2) v = fminf(v, dpp_f<DPP_XOR1>(v));
    if constexpr (W >= 4) v = fminf(v, dpp_f<DPP_XOR2>(v));
    if constexpr (W >= 8) v = fminf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if constexpr (W >= 16) v = fminf(v, dpp_f<DPP_MIRROR>(v));
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fminf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fminf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    return v;
}

template <int W>
__device__ __forceinline__ int group_max_i(int v)
{
    if constexpr (W >= 2) v = max(v, dpp_i<DPP_XOR1>(v));
    if constexpr (W >= 4) v = max(v, dpp_i<DPP_XOR2>(v));
    if constexpr (W >= 8) v = max(v, dpp_i<DPP_HALF_MIRROR>(v));
    if constexpr (W >= 16) v = max(v, dpp_i<DPP_MIRROR>(v));
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        v = max((int)p[0], (int)p[1]);
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        v = max((int)p[0], (int)p[1]);
    }
    return v;
}

template <int W>
__device__ __forceinline__ int group_min_i(int v)
{
    if constexpr (W >= 2) v = min(v, dpp_i<DPP_XOR1>(v));
    if constexpr (W >= 4) v = min(v, dpp_i<DPP_XOR2>(v));
    if constexpr (W >= 8) v = min(v, dpp_i<DPP_HALF_MIRROR>(v));
    if constexpr (W >= 16) v = min(v, dpp_i<DPP_MIRROR>(v));
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        v = min((int)p[0], (int)p[1]);
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        v = min((int)p[0], (int)p[1]);
    }
    return v;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// --------------------------------------------------------------- loads ----
// Byte-addressed loads of weights and activations in HBM.  Q6_K
// super-blocks are 210 B, so odd blocks sit at 2-byte alignment; gfx9 global
// memory runs in unaligned mode and these compile to single
// global_load_dword{,x2,x4}.  The pointers are cast to the global address
// space explicitly: a pointer read from memory (a layer table) would
// otherwise stay generic, and a flat load also counts against lgkmcnt, so
// every later wait for an LDS read would wait for the weight load as well.
typedef uint32_t g_u32x4 __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t g_u32x2 __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t g_u32 __attribute__((aligned(1)));
typedef uint16_t g_u16 __attribute__((aligned(1)));
#define QMAG_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ uint4 ld16(const uint8_t *p)
{
    const g_u32x4 v = *(const QMAG_GLOBAL g_u32x4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p)
{
    const g_u32x2 v = *(const QMAG_GLOBAL g_u32x2 *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p)
{
    return *(const QMAG_GLOBAL g_u32 *)p;
}
__device__ __forceinline__ uint32_t ld2(const uint8_t *p)
{
    return *(const QMAG_GLOBAL g_u16 *)p;
}
// naturally aligned scalar / float4 of an array in HBM, through a global pointer
template <typename T>
__device__ __forceinline__ T ldg(const T *p)
{
    return *(const QMAG_GLOBAL T *)p;
}
typedef float g_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ldg4(const float *p)
{
    const g_f32x4 v = *(const QMAG_GLOBAL g_f32x4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// -------------------------------------------------------------- Q8_K -----
// One wave quantises one 256-float block (src/q8k.c:34-85).  Lane l holds
// elements 4l..4l+3.  Outputs: the 4 int8 packed in a word, the block scale
// d, and in every lane the 16-element group sum of its group (lanes 4k..4k+3
// share group k).  amax is an exact max; d = amax/127 and 1/d are IEEE
// divisions; q = clamp(round-half-away(x * inv), +-127).
struct Q8Lane {
    uint32_t packed;
    float d;
    int gsum;
};

__device__ __forceinline__ int q8_round(float v)
{
    int q = (int)__builtin_roundf(v);
    q = q > 127 ? 127 : q;
    q = q < -127 ? -127 : q;
    return q;
}

// |x| as an integer whose order is the order of the values: every NaN lies
// above +Inf, so an integer maximum of these is the block's amax as
// vmaxq_f32 finds it in q8k.c:46-52 (NaN as soon as one value is NaN, which
// then gives d = 1, as amax > 0 is false); fmaxf would skip the NaN
__device__ __forceinline__ int abs_bits(float v) { return (int)(__float_as_uint(v) & 0x7fffffffu); }

__device__ __forceinline__ Q8Lane q8k_quant_lane(float4 v)
{
    const int a = max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w)));
    const float amax = __int_as_float(group_max_i<64>(a));
    Q8Lane r;
    r.d = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / r.d;
    const int q0 = q8_round(v.x * inv), q1 = q8_round(v.y * inv);
    const int q2 = q8_round(v.z * inv), q3 = q8_round(v.w * inv);
    r.packed = (uint32_t)(q0 & 255) | ((uint32_t)(q1 & 255) << 8) | ((uint32_t)(q2 & 255) << 16) |
               ((uint32_t)(q3 & 255) << 24);
    r.gsum = group_sum_i<4>(q0 + q1 + q2 + q3);
    return r;
}

// The same quantisation with a 256-block spread over 32 lanes, 8 values per
// lane (a = values 8L..8L+3, b = 8L+4..8L+7): each half of a wave quantises
// its own block, with the same results as q8k_quant_lane.  gsum is the sum of
// the 16-value group of the lane pair (2j, 2j+1).
struct Q8Lane2 {
    uint32_t packed[2];
    float d;
    int gsum;
};

__device__ __forceinline__ uint32_t q8_pack4(float4 v, float inv, int &sum)
{
    const int q0 = q8_round(v.x * inv), q1 = q8_round(v.y * inv);
    const int q2 = q8_round(v.z * inv), q3 = q8_round(v.w * inv);
    sum += q0 + q1 + q2 + q3;
    return (uint32_t)(q0 & 255) | ((uint32_t)(q1 & 255) << 8) | ((uint32_t)(q2 & 255) << 16) |
           ((uint32_t)(q3 & 255) << 24);
}

__device__ __forceinline__ Q8Lane2 q8k_quant_half(float4 a, float4 b)
{
    int m = max(max(abs_bits(a.x), abs_bits(a.y)), max(abs_bits(a.z), abs_bits(a.w)));
    m = max(m, max(max(abs_bits(b.x), abs_bits(b.y)), max(abs_bits(b.z), abs_bits(b.w))));
    const float amax = __int_as_float(group_max_i<32>(m));
    Q8Lane2 r;
    r.d = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / r.d;
    int s = 0;
    r.packed[0] = q8_pack4(a, inv, s);
    r.packed[1] = q8_pack4(b, inv, s);
    r.gsum = group_sum_i<2>(s);
    return r;
}

// -------------------------------------------------------------- Q4_K -----
// Task = (super-block ib, 64-lane group g): bytes qs[32g..32g+31] give the
// low nibbles of sub-block 2g and the high nibbles of sub-block 2g+1.
// Plo/Phi are the exact 32-lane int32 sums of src/q8k.c:117-120.
struct Q4Act {      // activation operand of one Q4_K task
    uint32_t x[16]; // xq[256ib+64g .. +63]
    float xd;       // xd[ib]
    float sx0, sx1; // xsum pairs of sub-blocks 2g, 2g+1 as floats
};

__device__ __forceinline__ void q4_load_act(Q4Act &a, const int8_t *xq, const float *xd,
                                            const int16_t *xsum, int ib, int g)
{
    const uint4 *p = (const uint4 *)(xq + ib * QK_K + 64 * g);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint4 w = p[k];
        a.x[4 * k + 0] = w.x;
        a.x[4 * k + 1] = w.y;
        a.x[4 * k + 2] = w.z;
        a.x[4 * k + 3] = w.w;
    }
    a.xd = xd[ib];
    const uint2 s = *(const uint2 *)(xsum + ib * 16 + 4 * g);
    const int s0 = (int16_t)(s.x & 0xffff), s1 = (int16_t)(s.x >> 16);
    const int s2 = (int16_t)(s.y & 0xffff), s3 = (int16_t)(s.y >> 16);
    a.sx0 = (float)(s0 + s1);
    a.sx1 = (float)(s2 + s3);
}

// 6-bit (scale, min) of sub-block j (src/q8k.c:22-30) from the 12 scale
// bytes held as words y = bytes 0-3, z = 4-7, w = 8-11.
__device__ __forceinline__ void q4_scale_min(int j, uint32_t y, uint32_t z, uint32_t w,
                                             uint32_t &sc, uint32_t &m)
{
    const int sh = 8 * (j & 3);
    const uint32_t by = (y >> sh) & 255, bz = (z >> sh) & 255, bw = (w >> sh) & 255;
    if (j < 4) {
        sc = by & 63;
        m = bz & 63;
    } else {
        sc = (bw & 15) | ((by >> 6) << 4);
        m = (bw >> 4) | ((bz >> 6) << 4);
    }
}

struct Q4Int {
    int plo, phi;
};

__device__ __forceinline__ Q4Int q4_int_dot(uint4 q0, uint4 q1, const Q4Act &a)
{
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    int lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        lo = sdot4(qw[k] & 0x0F0F0F0Fu, a.x[k], lo);
        hi = sdot4((qw[k] >> 4) & 0x0F0F0F0Fu, a.x[8 + k], hi);
    }
    return {lo, hi};
}

// fp32 contribution of one task: (d*s1*xd)*Plo + (d*s2*xd)*Phi
//                                 - (dmin*m1*sx0 + dmin*m2*sx1)*xd
__device__ __forceinline__ float q4_task(uint4 hdr, uint4 q0, uint4 q1, const Q4Act &a, int g)
{
    const float d = h2f(hdr.x & 0xffff), dmin = h2f(hdr.x >> 16);
    uint32_t s1, m1, s2, m2;
    q4_scale_min(2 * g, hdr.y, hdr.z, hdr.w, s1, m1);
    q4_scale_min(2 * g + 1, hdr.y, hdr.z, hdr.w, s2, m2);
    const Q4Int p = q4_int_dot(q0, q1, a);
    const float d1 = d * (float)s1, d2 = d * (float)s2;
    const float mm1 = dmin * (float)m1, mm2 = dmin * (float)m2;
    const float acc = (float)p.plo * (d1 * a.xd) + (float)p.phi * (d2 * a.xd);
    const float bias = (mm1 * a.sx0 + mm2 * a.sx1) * a.xd;
    return acc - bias;
}

// -------------------------------------------------------------- Q6_K -----
// Task = (super-block ib, half n, lane-half l16): 16 lanes l = 16*l16+t of
// half n across its four 32-lane quarters (src/quants.c:57-73,
// src/q8k.c:225-257).  The four tasks of a block sit in one lane quad and
// their int32 partials add to the exact per-block sum of q8k.c:259.
struct Q6Act {
    uint32_t x[16]; // quarter Q words 4Q..4Q+3: xq[256ib+128n+32Q+16l16 .. +15]
};

__device__ __forceinline__ void q6_load_act(Q6Act &a, const int8_t *xq, int ib, int n, int l16)
{
#pragma unroll
    for (int Q = 0; Q < 4; Q++) {
        const uint4 w = *(const uint4 *)(xq + ib * QK_K + 128 * n + 32 * Q + 16 * l16);
        a.x[4 * Q + 0] = w.x;
        a.x[4 * Q + 1] = w.y;
        a.x[4 * Q + 2] = w.z;
        a.x[4 * Q + 3] = w.w;
    }
}

struct Q6Raw {      // the bytes of one Q6_K task
    uint4 ql_lo, ql_hi, qh;
    uint2 sc;       // scales[8n .. 8n+7]
    uint32_t d;     // fp16 bits
};

__device__ __forceinline__ void q6_load_raw(Q6Raw &r, const uint8_t *blk, int n, int l16)
{
    r.ql_lo = ld16(blk + 64 * n + 16 * l16);
    r.ql_hi = ld16(blk + 64 * n + 32 + 16 * l16);
    r.qh = ld16(blk + 128 + 32 * n + 16 * l16);
    r.sc = ld8(blk + 192 + 8 * n);
    r.d = ld2(blk + 208);
}

// bytes (q6 - 32) for q6 in 0..63, per byte without cross-byte borrow
__device__ __forceinline__ uint32_t q6_center(uint32_t q)
{
    return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

__device__ __forceinline__ int q6_int_dot(const Q6Raw &r, const Q6Act &a, int l16)
{
    const uint32_t L[4] = {r.ql_lo.x, r.ql_lo.y, r.ql_lo.z, r.ql_lo.w};
    const uint32_t H[4] = {r.ql_hi.x, r.ql_hi.y, r.ql_hi.z, r.ql_hi.w};
    const uint32_t B[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    int s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t w0 = (L[k] & 0x0F0F0F0Fu) | ((B[k] & 0x03030303u) << 4);
        const uint32_t w1 = (H[k] & 0x0F0F0F0Fu) | (((B[k] >> 2) & 0x03030303u) << 4);
        const uint32_t w2 = ((L[k] >> 4) & 0x0F0F0F0Fu) | (((B[k] >> 4) & 0x03030303u) << 4);
        const uint32_t w3 = ((H[k] >> 4) & 0x0F0F0F0Fu) | (((B[k] >> 6) & 0x03030303u) << 4);
        s[0] = sdot4(q6_center(w0), a.x[0 + k], s[0]);
        s[1] = sdot4(q6_center(w1), a.x[4 + k], s[1]);
        s[2] = sdot4(q6_center(w2), a.x[8 + k], s[2]);
        s[3] = sdot4(q6_center(w3), a.x[12 + k], s[3]);
    }
    // scale of quarter Q is scales[8n + l16 + 2Q] = byte (l16 + 2Q) of r.sc
    const uint64_t sc8 = ((uint64_t)r.sc.y << 32) | r.sc.x;
    int tot = 0;
#pragma unroll
    for (int Q = 0; Q < 4; Q++) {
        const int scq = (int)(int8_t)((sc8 >> (8 * (l16 + 2 * Q))) & 255);
        tot += s[Q] * scq;
    }
    return tot;
}

// ------------------------------------------------ fp32 dequant-dot ----
// One 64-value task of an fp32 dot deq(row) . x (quants.c:80-133): Q4_K task
// t covers the nibble group t & 3 of super-block t >> 2 (its 16-byte header
// and 32 bytes of nibbles), Q6_K task t a quarter of super-block t >> 2.  xs
// is the fp32 operand (in LDS).  The tasks of a row summed in any order give
// the row's dot to fp32 rounding.
template <int WT>
__device__ __forceinline__ float f32_task(const uint8_t *row, int t, const float *xs)
{
    const int ib = t >> 2, q = t & 3;
    if constexpr (WT == QMAG_TYPE_Q4_K) {
        const uint8_t *b = row + (size_t)ib * Q4K_BYTES;
        const uint4 hdr = ld16(b), q0 = ld16(b + 16 + 32 * q), q1 = ld16(b + 32 + 32 * q);
        const float d = h2f(hdr.x & 0xffff), dmin = h2f(hdr.x >> 16);
        uint32_t s1, m1, s2, m2;
        q4_scale_min(2 * q, hdr.y, hdr.z, hdr.w, s1, m1);
        q4_scale_min(2 * q + 1, hdr.y, hdr.z, hdr.w, s2, m2);
        const float d1 = d * (float)s1, dm1 = dmin * (float)m1;
        const float d2 = d * (float)s2, dm2 = dmin * (float)m2;
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const float4 *xv = (const float4 *)(xs + ib * QK_K + 64 * q);
        float lo = 0.0f, hi = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 a = xv[k], c = xv[8 + k];
            const uint32_t w = qw[k];
            lo += (d1 * (float)(w & 15) - dm1) * a.x + (d1 * (float)((w >> 8) & 15) - dm1) * a.y +
                  (d1 * (float)((w >> 16) & 15) - dm1) * a.z + (d1 * (float)((w >> 24) & 15) - dm1) * a.w;
            hi += (d2 * (float)((w >> 4) & 15) - dm2) * c.x + (d2 * (float)((w >> 12) & 15) - dm2) * c.y +
                  (d2 * (float)((w >> 20) & 15) - dm2) * c.z + (d2 * (float)((w >> 28) & 15) - dm2) * c.w;
        }
        return lo + hi;
    } else {
        const uint8_t *b = row + (size_t)ib * Q6K_BYTES;
        const int n = q >> 1, l16 = q & 1;
        Q6Raw r;
        q6_load_raw(r, b, n, l16);
        const float d = h2f(r.d);
        const uint64_t sc8 = ((uint64_t)r.sc.y << 32) | r.sc.x;
        const uint32_t L[4] = {r.ql_lo.x, r.ql_lo.y, r.ql_lo.z, r.ql_lo.w};
        const uint32_t H[4] = {r.ql_hi.x, r.ql_hi.y, r.ql_hi.z, r.ql_hi.w};
        const uint32_t B[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        float acc = 0.0f;
#pragma unroll
        for (int Q = 0; Q < 4; Q++) {
            const float ds = d * (float)(int)(int8_t)((sc8 >> (8 * (l16 + 2 * Q))) & 255);
            const float4 *xv = (const float4 *)(xs + ib * QK_K + 128 * n + 32 * Q + 16 * l16);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t src = (Q & 1) ? H[k] : L[k];
                const uint32_t lo = (Q >= 2 ? src >> 4 : src) & 0x0F0F0F0Fu;
                const uint32_t qv = lo | (((B[k] >> (2 * Q)) & 0x03030303u) << 4);
                const float4 a = xv[k];
                acc += ds * (float)((int)(qv & 255) - 32) * a.x + ds * (float)((int)((qv >> 8) & 255) - 32) * a.y +
                       ds * (float)((int)((qv >> 16) & 255) - 32) * a.z + ds * (float)((int)(qv >> 24) - 32) * a.w;
            }
        }
        return acc;
    }
}

// ---------------------------------------------------------- routing ----
// The reference's softmax (nn.c:517-527) turns every probability into NaN
// when one logit is NaN or +Inf (its term is NaN), or when every logit is
// strictly below its -1e30 starting maximum (every term underflows to 0, and
// so does the sum; a logit of exactly -1e30 leaves the maximum there and
// makes a term expf(0) = 1, so routing stays ordinary).  Then no `p > -1e30`
// test of the top-K scan holds and every pick is expert 0 with value -1e30
// (nn.c:529-533), renormalised to -1e30 / (K * -1e30) summed in pick order.
// The E <= 256 logits sit 4 per lane of one wave, expert lane + 64j.
__device__ __forceinline__ bool route_degenerate(const float (&l)[4], int E)
{
    bool bad = false;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (lane_id() + 64 * j < E) {
            bad = bad || !(l[j] < INFINITY);            // NaN or +Inf
            mx = fmaxf(mx, l[j]);
        }
    }
    return __ballot(bad) != 0 || group_max<64>(mx) < -1e30f;
}
__device__ __forceinline__ float route_degenerate_weight(int K)
{
    float ws = 0.0f;
    for (int k = 0; k < K; k++) ws += -1e30f;
    return -1e30f / ws;
}

}  // namespace qmag
