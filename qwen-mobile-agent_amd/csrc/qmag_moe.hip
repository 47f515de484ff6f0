// qmag_moe.hip -- MoE FFN layer (src/nn.c:509-707, q8k branch) as a launch
// sequence over HBM-resident experts:
//
//   router_kernel   logits[t][e] = Wr[e] . x[t] (+ synthetic bias)   nn.c:514-524
//   topk_kernel     softmax, top-n_used (strict >, lowest index wins),
//                   renormalised weights; Q8_K(x[t]); shared-expert gate
//                   sigmoid(wsh . deq(Q8_K(x)))                       nn.c:525-536, 452-454, 598-602
//   gateup_kernel   per (slot, row): g,u = two Q4_K rows . Q8_K(x), h = silu(g)*u
//                   slot < n_used: routed expert sel[slot]; slot n_used: shared
//                                                                     nn.c:423-432, 458-464
//   q8k_quant       Q8_K(h) per slot                                  nn.c:434, 465
//   down_kernel     out[r] = sum_k w_k * down_k[r] . Q8_K(h_k) + gs * down_sh[r] . Q8_K(h_sh)
//                   in the reference's combine order (k = 0..n_used-1, then shared),
//                   optionally plus a residual                         nn.c:435-437, 468-472, 614-629
#include <limits.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "qmag_internal.h"

namespace qmag {

// --------------------------------------------------------------- router --
__global__ __launch_bounds__(256) void router_kernel(const float *__restrict__ Wr,
                                                     const float *__restrict__ bias,
                                                     const float *__restrict__ x, int N, int E,
                                                     int T, float *__restrict__ logits)
{
    const int wid = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    if (wid >= E * T) return;
    const int t = wid / E, e = wid % E;
    const int lane = lane_id();
    const float *w = Wr + (size_t)e * N;
    const float *xp = x + (size_t)t * N;
    float s = 0.0f;
    for (int i = 4 * lane; i < N; i += 256) {
        const float4 a = *(const float4 *)(w + i);
        const float4 b = *(const float4 *)(xp + i);
        s += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
    s = group_sum<64>(s);
    if (lane == 0) logits[(size_t)t * E + e] = bias ? s + bias[e] : s;
}

// ----------------------------------------------------------------- top-k --
// (p, e) ordering of the selection: larger p first, the lower expert index
// among equal p (the reference's strict-> scan from e = 0)
__device__ __forceinline__ bool tk_before(float pa, int ea, float pb, int eb)
{
    return pa > pb || (pa == pb && ea < eb);
}

__device__ __forceinline__ void tk_cswap(float (&p)[4], int (&id)[4], int a, int b)
{
    if (tk_before(p[b], id[b], p[a], id[a])) {
        const float tp = p[a];
        const int ti = id[a];
        p[a] = p[b];
        id[a] = id[b];
        p[b] = tp;
        id[b] = ti;
    }
}

// One workgroup per token.  Every load is issued first (each wave's x
// blocks with the matching shared-gate weights, and the logits in wave 0),
// so the workgroup waits for one round trip.  Each wave quantises its
// blocks and adds its share of the shared gate from registers; wave 0 then
// runs the softmax and the top-K: each lane sorts its four (p, e) once, and
// a pick is one wave max over the lane heads, a ballot for the lanes holding
// it (more than one only on an exact tie, then the lowest index among them)
// and a shift of the winning lane's list.
__global__ __launch_bounds__(256) void topk_kernel(float *__restrict__ logits, int npart, size_t pstride,
                                                   const float *__restrict__ lbias,
                                                   const float *__restrict__ x,
                                                   const float *__restrict__ wsh, int N, int E,
                                                   int K, int *__restrict__ sel,
                                                   float *__restrict__ wout,
                                                   float *__restrict__ gs_out,
                                                   int8_t *__restrict__ xq, float *__restrict__ xd,
                                                   int16_t *__restrict__ xs, float *__restrict__ xmb)
{
    constexpr int MB = 4;                     // 256-blocks per wave (n_embd <= 4096)
    __shared__ float s_red[4];
    const int t = blockIdx.x;
    const int lane = lane_id(), wv = threadIdx.x >> 6;
    const int NB = N / QK_K;

    float4 xv[MB], gw[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int b = min(wv + 4 * i, NB - 1);   // unconditional; blocks past NB unused
        xv[i] = ((const float4 *)(x + (size_t)t * N + b * QK_K))[lane];
        gw[i] = ((const float4 *)(wsh + b * QK_K))[lane];
    }
    // logits[t][e] = the npart chunk partials summed in order, then the bias
    float l[4];
    if (wv == 0) {
        const float *lg = logits + (size_t)t * E;
#pragma unroll
        for (int j = 0; j < 4; j++) l[j] = lg[min(lane + 64 * j, E - 1)];
        // every partial requested before the first add (npart <= 16)
        float pv[15][4];
#pragma unroll
        for (int p = 1; p < 16; p++)
#pragma unroll
            for (int j = 0; j < 4; j++) pv[p - 1][j] = p < npart ? lg[p * pstride + min(lane + 64 * j, E - 1)] : 0.0f;
#pragma unroll
        for (int p = 1; p < 16; p++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (p < npart) l[j] += pv[p - 1][j];
        if (lbias)
#pragma unroll
            for (int j = 0; j < 4; j++) l[j] = l[j] + lbias[min(lane + 64 * j, E - 1)];
        // the final logits replace chunk 0's partial (read only here), so
        // the buffer reads as logits[T][E] afterwards
        if (npart > 1 || lbias)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (lane + 64 * j < E) logits[(size_t)t * E + lane + 64 * j] = l[j];
    }

    // Q8_K of x[t] (one wave per 256-block) and the shared gate's
    // sum_i wsh[i] * xq[i] * xd[i/256] over the wave's blocks
    float g = 0.0f;
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const int b = wv + 4 * i;
        if (b < NB) {
            const Q8Lane r = q8k_quant_lane(xv[i]);
            ((uint32_t *)(xq + (size_t)t * N + b * QK_K))[lane] = r.packed;
            if (lane == 0) xd[(size_t)t * NB + b] = r.d;
            if ((lane & 3) == 0) xs[(size_t)t * (N / 16) + b * 16 + (lane >> 2)] = (int16_t)r.gsum;
            // the grouped prefill's Q4_K min-term operand: d * (sum of the
            // 32 values of each sub-block), lanes 8j .. 8j+7 holding sub-block j
            const int s32 = r.gsum + __shfl_xor(r.gsum, 4);
            if (xmb && (lane & 7) == 0) xmb[(size_t)t * (N / 32) + b * 8 + (lane >> 3)] = r.d * (float)s32;
            const int8_t *q8 = (const int8_t *)&r.packed;
            g += gw[i].x * (float)q8[0] * r.d + gw[i].y * (float)q8[1] * r.d + gw[i].z * (float)q8[2] * r.d +
                 gw[i].w * (float)q8[3] * r.d;
        }
    }
    g = group_sum<64>(g);
    if (lane == 0) s_red[wv] = g;

    if (wv == 0 && route_degenerate(l, E)) {      // the reference's NaN softmax: expert 0, K times
        if (lane < K) {
            sel[(size_t)t * K + lane] = 0;
            wout[(size_t)t * K + lane] = route_degenerate_weight(K);
        }
    } else if (wv == 0) {
        // softmax over E <= 256 logits, 4 per lane
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (lane + 64 * j >= E) l[j] = -INFINITY;
            mx = fmaxf(mx, l[j]);
        }
        mx = group_max<64>(mx);
        float p[4];
        int id[4];
        float se = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            p[j] = e < E ? expf(l[j] - mx) : 0.0f;
            se += p[j];
        }
        se = group_sum<64>(se);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            id[j] = e;
            p[j] = e < E ? p[j] / se : -1.0f;  // p >= 0 for every expert
        }
        tk_cswap(p, id, 0, 1);
        tk_cswap(p, id, 2, 3);
        tk_cswap(p, id, 0, 2);
        tk_cswap(p, id, 1, 3);
        tk_cswap(p, id, 1, 2);
        float wk = 0.0f;
        int sk = 0;
        for (int k = 0; k < K; k++) {
            const float m = group_max<64>(p[0]);
            const unsigned long long bal = __ballot(p[0] == m);
            // a NaN maximum equals nothing: fall back to lane 0's head, in range
            int win = bal ? __builtin_ctzll(bal) : 0;
            if (bal & (bal - 1)) {                // exact tie: the lowest index wins (one wave min)
                const int best = group_min_i<64>(p[0] == m ? id[0] : INT_MAX);
                win = __builtin_ctzll(__ballot(p[0] == m && id[0] == best));
            }
            const int e = __builtin_amdgcn_readlane(id[0], win);
            if (lane == k) {
                sk = e;
                wk = m;
            }
            if (lane == win) {
                p[0] = p[1];
                p[1] = p[2];
                p[2] = p[3];
                p[3] = -2.0f;
                id[0] = id[1];
                id[1] = id[2];
                id[2] = id[3];
            }
        }
        // w_k = p_k / sum_sel p, the sum in pick order
        float ws = 0.0f;
        for (int k = 0; k < K; k++) ws += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wk), k));
        if (lane < K) {
            sel[(size_t)t * K + lane] = sk;
            wout[(size_t)t * K + lane] = wk / ws;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float s = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
        gs_out[t] = 1.0f / (1.0f + expf(-s));
    }
}

// Routed experts addressed through per-slot record pointers (records of
// the HBM expert cache: gate slab, up slab, down slab back to back) instead
// of the layer's expert-major slabs; rec[0] == nullptr selects the slabs.
struct ExpertRecs {
    const uint8_t *rec[8];
    unsigned long long gu;                  // bytes of one gate (= up) slab
};

// --------------------------------------------------------------- gate/up --
// A wave holds R = 32/LPR row pairs: lanes [0,32) the gate rows, lanes
// [32,64) the matching up rows.  After the per-row reduction the two halves
// swap values with permlane32 so the gate lane sees its up value.
template <int NBE>
__global__ __launch_bounds__(256) void gateup_kernel(const uint8_t *__restrict__ gate_exps,
                                                     const uint8_t *__restrict__ up_exps,
                                                     const uint8_t *__restrict__ gate_sh,
                                                     const uint8_t *__restrict__ up_sh, const ExpertRecs recs,
                                                     const int *__restrict__ sel, int K, int F,
                                                     const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xd,
                                                     const int16_t *__restrict__ xs,
                                                     float *__restrict__ h)
{
    constexpr int TPR = 4 * NBE;
    constexpr int LPR = TPR < 32 ? TPR : 32;
    constexpr int TPL = TPR / LPR;
    constexpr int R = 32 / LPR;              // row pairs per wave step
    constexpr int U = 2;
    constexpr size_t RB = (size_t)NBE * Q4K_BYTES;

    const int lane = lane_id();
    const int half = lane >> 5, l32 = lane & 31;
    const int sub = l32 % LPR, rr = l32 / LPR, q = sub & 3;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int steps_per_slot = (F + R * U - 1) / (R * U);
    const int slot = wave / steps_per_slot;
    if (slot > K) return;
    const int base = (wave % steps_per_slot) * R * U;

    const uint8_t *mat;
    if (slot < K && recs.rec[0]) {
        mat = recs.rec[slot] + (half ? recs.gu : 0);
    } else if (slot < K) {
        const size_t slab = (size_t)F * RB;
        mat = (half ? up_exps : gate_exps) + (size_t)sel[slot] * slab;
    } else {
        mat = half ? up_sh : gate_sh;
    }

    Q4Act act[TPL];
#pragma unroll
    for (int j = 0; j < TPL; j++) q4_load_act(act[j], xq, xd, xs, (sub + LPR * j) >> 2, q);

    uint4 hdr[U][TPL], q0[U][TPL], q1[U][TPL];
#pragma unroll
    for (int u = 0; u < U; u++) {
        int row = base + u * R + rr;
        row = row < F ? row : F - 1;
#pragma unroll
        for (int j = 0; j < TPL; j++) {
            const uint8_t *blk = mat + (size_t)row * RB + (size_t)((sub + LPR * j) >> 2) * Q4K_BYTES;
            hdr[u][j] = ld16(blk);
            q0[u][j] = ld16(blk + 16 + 32 * q);
            q1[u][j] = ld16(blk + 32 + 32 * q);
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < TPL; j++) v += q4_task(hdr[u][j], q0[u][j], q1[u][j], act[j], q);
        v = group_sum<LPR>(v);
        // swap(A=v, B=v) exchanges A's upper half with B's lower half, so
        // the new B holds the upper-half (up-row) values in lanes < 32
        auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        const float other = __uint_as_float(p[1]);
        const int row = base + u * R + rr;
        if (half == 0 && sub == 0 && row < F) {
            const float g = v, up = other;
            h[(size_t)slot * F + row] = (g / (1.0f + expf(-g))) * up;
        }
    }
}

// ------------------------------------------------------------------ down --
template <int WT>
struct DownTask;

template <>
struct DownTask<QMAG_TYPE_Q4_K> {
    static constexpr int BLOCK = Q4K_BYTES;
    __device__ static float dot(const uint8_t *blk, const int8_t *hq, const float *hd,
                                const int16_t *hs, int ib, int q)
    {
        Q4Act a;
        q4_load_act(a, hq, hd, hs, ib, q);
        const uint4 hdr = ld16(blk), q0 = ld16(blk + 16 + 32 * q), q1 = ld16(blk + 32 + 32 * q);
        return q4_task(hdr, q0, q1, a, q);
    }
};

template <>
struct DownTask<QMAG_TYPE_Q6_K> {
    static constexpr int BLOCK = Q6K_BYTES;
    __device__ static float dot(const uint8_t *blk, const int8_t *hq, const float *hd,
                                const int16_t *, int ib, int q)
    {
        Q6Act a;
        q6_load_act(a, hq, ib, q >> 1, q & 1);
        Q6Raw r;
        q6_load_raw(r, blk, q >> 1, q & 1);
        const int isum = group_sum_i<4>(q6_int_dot(r, a, q & 1));
        return q == 0 ? h2f(r.d) * hd[ib] * (float)isum : 0.0f;
    }
};

template <int NBF, int TD, int TDS>
__global__ __launch_bounds__(256) void down_kernel(const uint8_t *__restrict__ down_exps,
                                                   const uint8_t *__restrict__ down_sh, const ExpertRecs recs,
                                                   const int *__restrict__ sel,
                                                   const float *__restrict__ w,
                                                   const float *__restrict__ gs, int K, int N,
                                                   const int8_t *__restrict__ hq,
                                                   const float *__restrict__ hd,
                                                   const int16_t *__restrict__ hs,
                                                   const float *resid, float *out)
{
    constexpr int TPR = 4 * NBF;             // tasks per (row, slot) dot
    constexpr int LPR = TPR;                 // NBF in {1, 2, 4}
    constexpr int RPW = 64 / LPR;
    constexpr int F = NBF * QK_K;
    const int lane = lane_id();
    const int sub = lane % LPR, rw = lane / LPR, q = sub & 3, ib = sub >> 2;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int row = wave * RPW + rw;
    if (wave * RPW >= N) return;               // wave-uniform
    const int rowc = row < N ? row : N - 1;

    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const size_t slab = (size_t)N * NBF * DownTask<TD>::BLOCK;
        const uint8_t *mat = recs.rec[0] ? recs.rec[k] + 2 * recs.gu : down_exps + (size_t)sel[k] * slab;
        const uint8_t *blk = mat + ((size_t)rowc * NBF + ib) * DownTask<TD>::BLOCK;
        const float d = group_sum<LPR>(DownTask<TD>::dot(blk, hq + (size_t)k * F, hd + (size_t)k * NBF,
                                                         hs + (size_t)k * (F / 16), ib, q));
        acc = __fadd_rn(acc, __fmul_rn(w[k], d));
    }
    {
        const uint8_t *blk = down_sh + ((size_t)rowc * NBF + ib) * DownTask<TDS>::BLOCK;
        const float d = group_sum<LPR>(DownTask<TDS>::dot(blk, hq + (size_t)K * F, hd + (size_t)K * NBF,
                                                          hs + (size_t)K * (F / 16), ib, q));
        acc = __fadd_rn(acc, __fmul_rn(gs[0], d));
    }
    if (sub == 0 && row < N) out[row] = resid ? __fadd_rn(acc, resid[row]) : acc;
}

// ------------------------------------------------------------------ host --
// -------------------------------------------- fp32 twins (QMA_NOQ8K) --
// moe_expert_one and moe_shared (nn.c:393-407, 475-492), which the reference
// takes when QMA_NOQ8K is set or q8k is unavailable (nn.c:585): no
// activation quantisation, every dot dequantise-then-dot in fp32 (f32_task).
// Routing is the q8k branch's (router_kernel, topk_kernel).
constexpr int F32_MAX_N = 4096, F32_MAX_SF = 9 * 1024;   // n_embd; (n_used + 1) * n_ff

// h[t][s][i] = silu(gate_i . x[t]) * (up_i . x[t]) for slot s (s < K: expert
// sel[t][s]; s = K: the shared expert).  Grid (row blocks, K + 1, T); LPR
// lanes per row.  Workgroup (0, K, t) also writes the fp32 shared gate
// sigmoid(wsh . x[t]) (nn.c:477-479) to gs[t].
template <int LPR>
__global__ __launch_bounds__(256) void moe_f32_gateup_kernel(const uint8_t *__restrict__ gate_exps,
                                                             const uint8_t *__restrict__ up_exps,
                                                             const uint8_t *__restrict__ gate_shexp,
                                                             const uint8_t *__restrict__ up_shexp,
                                                             const float *__restrict__ wsh,
                                                             const int *__restrict__ sel, int K, int N, int F,
                                                             const float *__restrict__ x, float *__restrict__ h,
                                                             float *__restrict__ gs)
{
    __shared__ __align__(16) float s_x[F32_MAX_N];
    const int t = (int)blockIdx.z, s = (int)blockIdx.y, S = K + 1;
    for (int i = (int)threadIdx.x; i < N / 4; i += (int)blockDim.x)
        ((float4 *)s_x)[i] = ldg4(x + (size_t)t * N + 4 * i);
    __syncthreads();
    const int nb = N / QK_K, ntask = 4 * nb;
    const size_t rb = (size_t)nb * Q4K_BYTES, slab = (size_t)F * rb;
    const uint8_t *ge = s < K ? gate_exps + (size_t)sel[(size_t)t * K + s] * slab : gate_shexp;
    const uint8_t *ue = s < K ? up_exps + (size_t)sel[(size_t)t * K + s] * slab : up_shexp;
    const int lane = lane_id(), wave = (int)(threadIdx.x >> 6), sub = lane % LPR;
    const int row = ((int)blockIdx.x * 4 + wave) * (64 / LPR) + lane / LPR;
    float g = 0.0f, u = 0.0f;
    if (row < F)
        for (int tk = sub; tk < ntask; tk += LPR) {
            g += f32_task<QMAG_TYPE_Q4_K>(ge + (size_t)row * rb, tk, s_x);
            u += f32_task<QMAG_TYPE_Q4_K>(ue + (size_t)row * rb, tk, s_x);
        }
    g = group_sum<LPR>(g);
    u = group_sum<LPR>(u);
    if (sub == 0 && row < F) h[((size_t)t * S + s) * F + row] = (g / (1.0f + expf(-g))) * u;
    if (blockIdx.x == 0 && s == K && wave == 0) {
        float v = 0.0f;
        for (int i = lane; i < N; i += 64) v += wsh[i] * s_x[i];
        v = group_sum<64>(v);
        if (lane == 0) gs[t] = 1.0f / (1.0f + expf(-v));
    }
}

// out[t][r] = sum_k w_k * (down_k[r] . h_k) + gs * (down_sh[r] . h_sh), the
// partials summed in the reference's order (slots 0..K-1, then the shared
// expert; nn.c:614-629), products and sums separately rounded.  Grid (row
// blocks, T); the token's K + 1 h vectors in LDS.
template <int LPR, int TD, int TDS>
__global__ __launch_bounds__(256) void moe_f32_down_kernel(const uint8_t *__restrict__ down_exps,
                                                           const uint8_t *__restrict__ down_shexp,
                                                           const int *__restrict__ sel, const float *__restrict__ w,
                                                           const float *__restrict__ gs, int K, int N, int F,
                                                           const float *__restrict__ h, float *__restrict__ out)
{
    __shared__ __align__(16) float s_h[F32_MAX_SF];
    const int t = (int)blockIdx.y, S = K + 1;
    for (int i = (int)threadIdx.x; i < S * F / 4; i += (int)blockDim.x)
        ((float4 *)s_h)[i] = ldg4(h + (size_t)t * S * F + 4 * i);
    __syncthreads();
    const int nb = F / QK_K, ntask = 4 * nb;
    const size_t rb = (size_t)nb * (TD == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES), slab = (size_t)N * rb;
    const size_t rbs = (size_t)nb * (TDS == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES);
    const int lane = lane_id(), wave = (int)(threadIdx.x >> 6), sub = lane % LPR;
    const int row = ((int)blockIdx.x * 4 + wave) * (64 / LPR) + lane / LPR;
    const bool live = row < N;
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const uint8_t *dr = down_exps + (size_t)sel[(size_t)t * K + k] * slab + (size_t)(live ? row : 0) * rb;
        float y = 0.0f;
        if (live)
            for (int tk = sub; tk < ntask; tk += LPR) y += f32_task<TD>(dr, tk, s_h + k * F);
        y = group_sum<LPR>(y);
        acc = __fadd_rn(acc, __fmul_rn(w[(size_t)t * K + k], y));
    }
    float y = 0.0f;
    if (live)
        for (int tk = sub; tk < ntask; tk += LPR) y += f32_task<TDS>(down_shexp + (size_t)row * rbs, tk, s_h + K * F);
    y = group_sum<LPR>(y);
    acc = __fadd_rn(acc, __fmul_rn(gs[t], y));
    if (sub == 0 && live) out[(size_t)t * N + row] = acc;
}

template <int TD, int TDS>
static void launch_f32_down(const qmag_moe_layer *L, const int *sel, const float *w, const float *gs,
                            const float *h, float *out, int T, hipStream_t s)
{
    const int N = L->n_embd, F = L->n_ff, K = L->n_used;
    const int ntask = 4 * (F / QK_K);
    const uint8_t *de = (const uint8_t *)L->down_exps, *ds = (const uint8_t *)L->down_shexp;
    switch (ntask) {
    case 4: hipLaunchKernelGGL((moe_f32_down_kernel<4, TD, TDS>), dim3((N + 63) / 64, T), dim3(256), 0, s, de, ds,
                               sel, w, gs, K, N, F, h, out); break;
    case 8: hipLaunchKernelGGL((moe_f32_down_kernel<8, TD, TDS>), dim3((N + 31) / 32, T), dim3(256), 0, s, de, ds,
                               sel, w, gs, K, N, F, h, out); break;
    default: hipLaunchKernelGGL((moe_f32_down_kernel<16, TD, TDS>), dim3((N + 15) / 16, T), dim3(256), 0, s, de,
                                ds, sel, w, gs, K, N, F, h, out); break;
    }
}

static bool pow2_in(int v, int lo, int hi) { return v >= lo && v <= hi && (v & (v - 1)) == 0; }

// batches of at least this many tokens take the grouped expert GEMM
// (qmag_prefill.hip) when QMAG_OPT_GROUPED is on; smaller ones the
// per-token launch sequence below
constexpr int GROUPED_MIN_T = 8;

int moe_check_layer(const qmag_moe_layer *L, bool need_exps)
{
    if (!L) return fail(QMAG_ERR_ARG, "moe: null layer");
    if (L->n_embd % QK_K || !pow2_in(L->n_embd / QK_K, 1, 16))
        return fail(QMAG_ERR_ARG, "moe: n_embd=%d unsupported (256..4096, power of two)", L->n_embd);
    if (L->n_ff % QK_K || !pow2_in(L->n_ff / QK_K, 1, 4))
        return fail(QMAG_ERR_ARG, "moe: n_ff=%d unsupported (256, 512, 1024)", L->n_ff);
    if (L->n_expert < 1 || L->n_expert > 256) return fail(QMAG_ERR_ARG, "moe: n_expert=%d", L->n_expert);
    if (L->n_used < 1 || L->n_used > 8 || L->n_used > L->n_expert)
        return fail(QMAG_ERR_ARG, "moe: n_used=%d", L->n_used);
    for (int t : {L->t_down_exps, L->t_down_shexp})
        if (t != QMAG_TYPE_Q4_K && t != QMAG_TYPE_Q6_K) return fail(QMAG_ERR_ARG, "moe: down type %d", t);
    if (!L->gate_inp || (need_exps && (!L->gate_exps || !L->up_exps || !L->down_exps)) || !L->gate_inp_shexp ||
        !L->gate_shexp || !L->up_shexp || !L->down_shexp)
        return fail(QMAG_ERR_ARG, "moe: null tensor pointer");
    return QMAG_OK;
}

struct MoeWs {
    float *logits, *w, *gs, *h, *hd;
    int *sel;
    int8_t *xq, *hq;
    float *xd, *xmb;
    int16_t *xs, *hs;
};

static int moe_ws(const qmag_moe_layer *L, int T, MoeWs &ws)
{
    const int N = L->n_embd, F = L->n_ff, E = L->n_expert, K = L->n_used, S = K + 1;
    int st;
#define WS(field, type, slot, count)                                              \
    ws.field = (type *)workspace(slot, sizeof(type) * (size_t)(count), &st);      \
    if (st) return st;
    WS(logits, float, WS_LOGITS, (size_t)T * E * (N / QK_K));   // the grouped router's chunk partials
    WS(sel, int, WS_SEL, (size_t)T * K);
    WS(w, float, WS_W, (size_t)T * K);
    WS(gs, float, WS_GS, T);
    WS(xq, int8_t, WS_XQ, (size_t)T * N);
    WS(xd, float, WS_XD, (size_t)T * (N / QK_K));
    WS(xs, int16_t, WS_XS, (size_t)T * (N / 16));
    WS(xmb, float, WS_XMB, (size_t)T * (N / 32));
    WS(h, float, WS_H, (size_t)T * S * F);
    WS(hq, int8_t, WS_HQ, (size_t)T * S * F);
    WS(hd, float, WS_HD, (size_t)T * S * (F / QK_K));
    WS(hs, int16_t, WS_HS, (size_t)T * S * (F / 16));
#undef WS
    return QMAG_OK;
}

static MoeWs g_last;
static int g_last_K = 0;

template <int NBE>
static void launch_gateup(const qmag_moe_layer *L, const MoeWs &ws, int t, const ExpertRecs &recs, hipStream_t s)
{
    constexpr int TPR = 4 * NBE;
    constexpr int LPR = TPR < 32 ? TPR : 32;
    constexpr int R = 32 / LPR;
    const int N = L->n_embd, F = L->n_ff, K = L->n_used, S = K + 1;
    const int steps = (F + R * 2 - 1) / (R * 2);
    const int waves = steps * S;
    hipLaunchKernelGGL(gateup_kernel<NBE>, dim3((waves + 3) / 4), dim3(256), 0, s,
                       (const uint8_t *)L->gate_exps, (const uint8_t *)L->up_exps,
                       (const uint8_t *)L->gate_shexp, (const uint8_t *)L->up_shexp, recs,
                       ws.sel + (size_t)t * K, K, F, ws.xq + (size_t)t * N, ws.xd + (size_t)t * (N / QK_K),
                       ws.xs + (size_t)t * (N / 16), ws.h + (size_t)t * S * F);
}

template <int NBF, int TD, int TDS>
static void launch_down3(const qmag_moe_layer *L, const MoeWs &ws, int t, const ExpertRecs &recs,
                         const float *resid, float *out, hipStream_t s)
{
    const int N = L->n_embd, F = L->n_ff, K = L->n_used, S = K + 1;
    constexpr int RPW = 64 / (4 * NBF);
    const int waves = (N + RPW - 1) / RPW;
    // one wave per workgroup: the grid is only N/RPW waves, spread it over CUs
    hipLaunchKernelGGL((down_kernel<NBF, TD, TDS>), dim3(waves), dim3(64), 0, s,
                       (const uint8_t *)L->down_exps, (const uint8_t *)L->down_shexp, recs,
                       ws.sel + (size_t)t * K, ws.w + (size_t)t * K, ws.gs + t, K, N,
                       ws.hq + (size_t)t * S * F, ws.hd + (size_t)t * S * (F / QK_K),
                       ws.hs + (size_t)t * S * (F / 16), resid ? resid + (size_t)t * N : nullptr,
                       out + (size_t)t * N);
}

template <int NBF>
static void launch_down2(const qmag_moe_layer *L, const MoeWs &ws, int t, const ExpertRecs &recs,
                         const float *resid, float *out, hipStream_t s)
{
    const bool r6 = L->t_down_exps == QMAG_TYPE_Q6_K, s6 = L->t_down_shexp == QMAG_TYPE_Q6_K;
    if (r6 && s6) launch_down3<NBF, QMAG_TYPE_Q6_K, QMAG_TYPE_Q6_K>(L, ws, t, recs, resid, out, s);
    else if (r6) launch_down3<NBF, QMAG_TYPE_Q6_K, QMAG_TYPE_Q4_K>(L, ws, t, recs, resid, out, s);
    else if (s6) launch_down3<NBF, QMAG_TYPE_Q4_K, QMAG_TYPE_Q6_K>(L, ws, t, recs, resid, out, s);
    else launch_down3<NBF, QMAG_TYPE_Q4_K, QMAG_TYPE_Q4_K>(L, ws, t, recs, resid, out, s);
}

// the per-token expert stages of the launch sequence: gate/up, Q8_K(h),
// down + combine
static int token_experts(const qmag_moe_layer *L, const MoeWs &ws, int t, const ExpertRecs &recs,
                         const float *resid, float *out, hipStream_t s)
{
    const int N = L->n_embd, F = L->n_ff, K = L->n_used, S = K + 1;
    prof_begin(PROF_GATEUP, s);
    switch (N / QK_K) {
    case 1: launch_gateup<1>(L, ws, t, recs, s); break;
    case 2: launch_gateup<2>(L, ws, t, recs, s); break;
    case 4: launch_gateup<4>(L, ws, t, recs, s); break;
    case 8: launch_gateup<8>(L, ws, t, recs, s); break;
    default: launch_gateup<16>(L, ws, t, recs, s); break;
    }
    prof_end(PROF_GATEUP, s);
    prof_begin(PROF_HQUANT, s);
    int st = launch_q8k_quant(ws.h + (size_t)t * S * F, S * (F / QK_K), ws.hq + (size_t)t * S * F,
                              ws.hd + (size_t)t * S * (F / QK_K), ws.hs + (size_t)t * S * (F / 16), s);
    prof_end(PROF_HQUANT, s);
    if (st) return st;
    prof_begin(PROF_DOWN, s);
    switch (F / QK_K) {
    case 1: launch_down2<1>(L, ws, t, recs, resid, out, s); break;
    case 2: launch_down2<2>(L, ws, t, recs, resid, out, s); break;
    default: launch_down2<4>(L, ws, t, recs, resid, out, s); break;
    }
    prof_end(PROF_DOWN, s);
    return QMAG_OK;
}

// router and top-k (with Q8_K(x) and the shared gate) for T tokens
static int route_tokens(const qmag_moe_layer *L, const float *x, int T, bool grouped, const MoeWs &ws,
                        hipStream_t s)
{
    const int N = L->n_embd, E = L->n_expert, K = L->n_used;
    prof_begin(PROF_ROUTER, s);
    if (grouped) {
        int st = launch_router_mfma(L, x, T, ws.logits, s);
        if (st) return st;
    } else {
        hipLaunchKernelGGL(router_kernel, dim3((E * T + 3) / 4), dim3(256), 0, s, L->gate_inp,
                           L->router_bias, x, N, E, T, ws.logits);
    }
    prof_end(PROF_ROUTER, s);
    prof_begin(PROF_TOPK, s);
    // the grouped router leaves one partial per 256-wide k chunk and no bias
    hipLaunchKernelGGL(topk_kernel, dim3(T), dim3(256), 0, s, ws.logits, grouped ? N / 256 : 1, (size_t)T * E,
                       grouped ? L->router_bias : nullptr, x, L->gate_inp_shexp, N, E, K, ws.sel, ws.w, ws.gs,
                       ws.xq, ws.xd, ws.xs, grouped ? ws.xmb : nullptr);
    prof_end(PROF_TOPK, s);
    return QMAG_OK;
}

int moe_ffn(const qmag_moe_layer *L, const float *x, float *out, int T, const float *resid,
            hipStream_t s)
{
    int st = moe_check_layer(L);
    if (st) return st;
    if (T <= 0 || !x || !out) return fail(QMAG_ERR_ARG, "moe: T=%d x=%p out=%p", T, x, out);
    MoeWs ws;
    st = moe_ws(L, T, ws);
    if (st) return st;
    const int K = L->n_used;
    const bool grouped = T >= GROUPED_MIN_T && option(QMAG_OPT_GROUPED);
    st = route_tokens(L, x, T, grouped, ws, s);
    if (st) return st;
    if (grouped) {
        st = moe_grouped(L, T, ws.sel, ws.w, ws.gs, ws.xq, ws.xd, ws.xmb, ws.h, ws.hq, ws.hd, ws.hs, resid, out,
                         s);
        if (st) return st;
        g_last = ws;
        g_last_K = K;
        return QMAG_OK;
    }
    const ExpertRecs slabs = {};
    for (int t = 0; t < T; t++) {
        st = token_experts(L, ws, t, slabs, resid, out, s);
        if (st) return st;
    }
    QMAG_HIP(hipGetLastError());
    g_last = ws;
    g_last_K = K;
    return QMAG_OK;
}

}  // namespace qmag

using namespace qmag;

static bool g_last_fused = false;

extern "C" int qmag_moe_ffn_dev(const qmag_moe_layer *L, const float *x, float *out, int T)
{
    int st = require_ready();
    if (st) return st;
    st = moe_check_layer(L);
    if (st) return st;
    if (T == 1 && option(QMAG_OPT_FUSED) && fused_eligible(L, 1)) {
        if (!x || !out) return fail(QMAG_ERR_ARG, "moe: null x/out");
        g_last_fused = true;
        return fused_call(L, 1, (float *)x, out, 1, ctx().stream);
    }
    g_last_fused = false;
    return moe_ffn(L, x, out, T, nullptr, ctx().stream);
}

// The moe_ffn seam on host buffers: x staged through pinned memory and
// copied to the device on the library stream, the layer queued behind it,
// out copied back the same way together with the persistent decode kernel's
// abort word, then one synchronisation.  Pinned staging is allocated (never
// registered) and grown as needed; one call at a time.
static std::mutex g_host_mu;
static uint8_t *g_host_pin = nullptr;
static size_t g_host_pin_cap = 0;

extern "C" int qmag_moe_ffn_host(const qmag_moe_layer *L, const float *x, float *out, int T)
{
    int st = require_ready();
    if (st) return st;
    st = moe_check_layer(L);
    if (st) return st;
    if (!x || !out || T <= 0) return fail(QMAG_ERR_ARG, "moe_host: x=%p out=%p T=%d", x, out, T);
    const size_t bytes = sizeof(float) * (size_t)T * L->n_embd, half = (bytes + 255) & ~(size_t)255;
    std::lock_guard<std::mutex> guard(g_host_mu);
    hipStream_t s = ctx().stream;
    if (2 * half + 256 > g_host_pin_cap) {
        if (g_host_pin) {
            // a call that failed after queueing its copies returned without
            // waiting for them: none may still read the buffer being freed
            QMAG_HIP(hipStreamSynchronize(s));
            QMAG_HIP(hipHostFree(g_host_pin));
        }
        g_host_pin = nullptr;
        g_host_pin_cap = 0;
        QMAG_HIP(hipHostMalloc((void **)&g_host_pin, 2 * half + 256, hipHostMallocDefault));
        g_host_pin_cap = 2 * half + 256;
    }
    uint8_t *dev = (uint8_t *)workspace(WS_HOSTIO, 2 * half, &st);
    if (!dev) return st;
    float *pin_x = (float *)g_host_pin, *pin_out = (float *)(g_host_pin + half);
    int *pin_word = (int *)(g_host_pin + 2 * half);
    float *d_x = (float *)dev, *d_out = (float *)(dev + half);
    memcpy(pin_x, x, bytes);
    QMAG_HIP(hipMemcpyAsync(d_x, pin_x, bytes, hipMemcpyHostToDevice, s));
    st = qmag_moe_ffn_dev(L, d_x, d_out, T);
    if (st) return st;
    QMAG_HIP(hipMemcpyAsync(pin_out, d_out, bytes, hipMemcpyDeviceToHost, s));
    const bool pending = fused_pending();
    if (pending) {
        st = fused_abort_copy(pin_word, s);
        if (st) return st;
    }
    QMAG_HIP(hipStreamSynchronize(s));
    if (pending) {
        // a persistent launch whose wait expired: the affected calls (this one
        // among them) are re-run, then out is copied again
        const long r0 = fused_recoveries();
        st = fused_status_word(*pin_word);
        if (st) return st;
        if (fused_recoveries() != r0) {
            QMAG_HIP(hipMemcpyAsync(pin_out, d_out, bytes, hipMemcpyDeviceToHost, s));
            QMAG_HIP(hipStreamSynchronize(s));
        }
    }
    memcpy(out, pin_out, bytes);
    return QMAG_OK;
}

extern "C" int qmag_moe_stack_dev(const qmag_moe_layer *layers, int n_layer, float *x, int n_tok)
{
    int st = require_ready();
    if (st) return st;
    if (!layers || n_layer <= 0 || n_tok <= 0 || !x) return fail(QMAG_ERR_ARG, "moe_stack: bad args");
    for (int l = 0; l < n_layer; l++) {
        st = moe_check_layer(&layers[l]);
        if (st) return st;
        if (layers[l].n_embd != layers[0].n_embd) return fail(QMAG_ERR_ARG, "moe_stack: n_embd differs");
    }
    const int N = layers[0].n_embd;
    if (option(QMAG_OPT_FUSED) && fused_eligible(layers, n_layer)) {
        g_last_fused = true;
        return fused_call(layers, n_layer, x, nullptr, n_tok, ctx().stream);
    }
    if (option(QMAG_OPT_FUSED)) {
        st = fused_stack_runs(layers, n_layer, x, n_tok, ctx().stream);
        if (st != 1) {
            // the stage buffers hold the last layer's, from whichever path ran it
            g_last_fused = fused_eligible(&layers[n_layer - 1], 1);
            return st;
        }
    }
    g_last_fused = false;
    for (int t = 0; t < n_tok; t++) {
        float *xt = x + (size_t)t * N;
        for (int l = 0; l < n_layer; l++) {
            st = moe_ffn(&layers[l], xt, xt, 1, xt, ctx().stream);
            if (st) return st;
        }
    }
    return QMAG_OK;
}

namespace qmag {
void moe_note_sequence_ran() { g_last_fused = false; }
}  // namespace qmag

// moe_ffn with the expert cache on (nn.c:553-571, 677-694): route all T
// tokens, hint the distinct selected experts in (token, slot) order, then per
// token hold its n_used records, run the expert stages on them and release.
extern "C" int qmag_moe_ffn_paged_dev(const qmag_moe_layer *L, qmag_ecache *c, int il, qmag_fetch_fn fetch,
                                      void *user, const float *x, float *out, int T)
{
    int st = require_ready();
    if (st) return st;
    st = moe_check_layer(L, false);
    if (st) return st;
    if (!c || !x || !out || T <= 0 || il < 0) return fail(QMAG_ERR_ARG, "moe_paged: bad arguments");
    qmag_ecache_counters cc;
    st = qmag_ecache_stats(c, &cc);
    if (st) return st;
    const int N = L->n_embd, F = L->n_ff, K = L->n_used;
    const size_t gu = (size_t)F * (N / QK_K) * Q4K_BYTES;
    const size_t dn = (size_t)N * (F / QK_K) * (L->t_down_exps == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES);
    if (cc.n_slots < 4 || cc.rec_bytes < 2 * gu + dn)
        return fail(QMAG_ERR_ARG, "moe_paged: cache records of %zu bytes (%d slots) cannot hold a %zu-byte expert",
                    cc.rec_bytes, cc.n_slots, 2 * gu + dn);
    hipStream_t s = ctx().stream;
    MoeWs ws;
    st = moe_ws(L, T, ws);
    if (st) return st;
    g_last_fused = false;
    st = route_tokens(L, x, T, false, ws, s);
    if (st) return st;
    std::vector<int> sel((size_t)T * K);
    QMAG_HIP(hipMemcpyAsync(sel.data(), ws.sel, sizeof(int) * sel.size(), hipMemcpyDeviceToHost, s));
    QMAG_HIP(hipStreamSynchronize(s));
    std::vector<int> ids;
    std::vector<char> seen((size_t)L->n_expert, 0);
    for (int e : sel)
        if (!seen[(size_t)e]) {
            seen[(size_t)e] = 1;
            ids.push_back(e);
        }
    qmag_ecache_hint(c, il, ids.data(), (int)ids.size());
    for (int t = 0; t < T; t++) {
        ExpertRecs recs = {};
        recs.gu = gu;
        for (int k = 0; k < K; k++) {
            recs.rec[k] = qmag_ecache_hold(c, il, sel[(size_t)t * K + k], fetch, user);
            if (!recs.rec[k]) {
                qmag_ecache_release(c);
                return fail(QMAG_ERR_ARG, "moe_paged: layer %d expert %d could not be read", il,
                            sel[(size_t)t * K + k]);
            }
        }
        st = token_experts(L, ws, t, recs, nullptr, out, s);
        qmag_ecache_release(c);      // after the launches: later copies wait for them
        if (st) return st;
    }
    QMAG_HIP(hipGetLastError());
    g_last = ws;
    g_last_K = K;
    return QMAG_OK;
}

// the QMA_NOQ8K layer (nn.c:585): the q8k branch's routing, then the fp32
// expert stages; the stage buffers hold its logits, selection, weights,
// fp32 shared gate and fp32 h
extern "C" int qmag_moe_ffn_f32_dev(const qmag_moe_layer *L, const float *x, float *out, int T)
{
    int st = require_ready();
    if (st) return st;
    st = moe_check_layer(L);
    if (st) return st;
    if (T <= 0 || T > 65535 || !x || !out) return fail(QMAG_ERR_ARG, "moe_f32: T=%d x=%p out=%p", T, x, out);
    const int N = L->n_embd, F = L->n_ff, K = L->n_used, S = K + 1;
    if (N > F32_MAX_N || S * F > F32_MAX_SF) return fail(QMAG_ERR_ARG, "moe_f32: n_embd=%d n_ff=%d", N, F);
    hipStream_t s = ctx().stream;
    MoeWs ws;
    st = moe_ws(L, T, ws);
    if (st) return st;
    g_last_fused = false;
    st = route_tokens(L, x, T, false, ws, s);
    if (st) return st;
    const int ntask = 4 * (N / QK_K);
    const dim3 gu_grid((unsigned)((F + 15) / 16), (unsigned)S, (unsigned)T);
    const uint8_t *ge = (const uint8_t *)L->gate_exps, *ue = (const uint8_t *)L->up_exps;
    const uint8_t *gsh = (const uint8_t *)L->gate_shexp, *ush = (const uint8_t *)L->up_shexp;
    prof_begin(PROF_GATEUP, s);
    if (ntask >= 32) {
        hipLaunchKernelGGL(moe_f32_gateup_kernel<32>, dim3((F + 7) / 8, S, T), dim3(256), 0, s, ge, ue, gsh, ush,
                           L->gate_inp_shexp, ws.sel, K, N, F, x, ws.h, ws.gs);
    } else {
        hipLaunchKernelGGL(moe_f32_gateup_kernel<16>, gu_grid, dim3(256), 0, s, ge, ue, gsh, ush, L->gate_inp_shexp,
                           ws.sel, K, N, F, x, ws.h, ws.gs);
    }
    prof_end(PROF_GATEUP, s);
    prof_begin(PROF_DOWN, s);
    const bool r6 = L->t_down_exps == QMAG_TYPE_Q6_K, s6 = L->t_down_shexp == QMAG_TYPE_Q6_K;
    if (r6 && s6) launch_f32_down<QMAG_TYPE_Q6_K, QMAG_TYPE_Q6_K>(L, ws.sel, ws.w, ws.gs, ws.h, out, T, s);
    else if (r6) launch_f32_down<QMAG_TYPE_Q6_K, QMAG_TYPE_Q4_K>(L, ws.sel, ws.w, ws.gs, ws.h, out, T, s);
    else if (s6) launch_f32_down<QMAG_TYPE_Q4_K, QMAG_TYPE_Q6_K>(L, ws.sel, ws.w, ws.gs, ws.h, out, T, s);
    else launch_f32_down<QMAG_TYPE_Q4_K, QMAG_TYPE_Q4_K>(L, ws.sel, ws.w, ws.gs, ws.h, out, T, s);
    prof_end(PROF_DOWN, s);
    QMAG_HIP(hipGetLastError());
    g_last = ws;
    g_last_K = K;
    return QMAG_OK;
}

extern "C" int qmag_moe_last_stage(const float **logits, const int **sel, const float **w,
                                   const float **gs, const float **h)
{
    if (g_last_fused) return fused_last_stage(logits, sel, w, gs, h);
    if (!g_last.logits) return fail(QMAG_ERR_ARG, "no MoE call yet");
    if (logits) *logits = g_last.logits;
    if (sel) *sel = g_last.sel;
    if (w) *w = g_last.w;
    if (gs) *gs = g_last.gs;
    if (h) *h = g_last.h;
    return QMAG_OK;
}
