// qmag_matvec.hip -- Q8_K activation quantisation and the Q4_K / Q6_K x Q8_K
// matvec (src/q8k.c:34-262 driven as in mm_worker, src/nn.c:276-289).
//
// Decode matvecs are HBM-bound: each row's bytes are read once.  A row is
// split into "tasks" (Q4_K: one 64-lane group of a super-block = 32 B of
// nibbles + the 16 B header; Q6_K: a quarter of a super-block = 3x16 B +
// scales + d).  LPR lanes cooperate on a row (LPR = tasks per row, <= 64) so
// a wave covers 64/LPR rows per step; each lane keeps its task's activation
// slice in registers across rows and issues its weight loads for U row
// steps before consuming any of them.  Row sums use DPP/permlane reductions.
//
// Also here: Q6_K rows repacked into aligned planes (QMAG_TYPE_Q6_K_R, same
// bytes and results, for large matrices such as the LM head), and one launch
// for several matrices over the same x (the projections of one activation
// vector), bit-identical to separate calls.
#include "qmag_internal.h"

// Launch shape of the tiled matvec: wave steps of rows in flight per wave,
// waves per CU the grid is capped at, threads per workgroup.
#ifndef QMAG_MV_U
#define QMAG_MV_U 2
#endif
#ifndef QMAG_MV_CAP
#define QMAG_MV_CAP 64
#endif
#ifndef QMAG_MV_WG
#define QMAG_MV_WG 256
#endif

namespace qmag {

__global__ __launch_bounds__(256) void q8k_quant_kernel(const float *__restrict__ x, int nblocks,
                                                        int8_t *__restrict__ xq,
                                                        float *__restrict__ xd,
                                                        int16_t *__restrict__ xsum)
{
    const int blk = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    if (blk >= nblocks) return;           // wave-uniform
    const int lane = lane_id();
    const float4 v = ((const float4 *)(x + (size_t)blk * QK_K))[lane];
    const Q8Lane r = q8k_quant_lane(v);
    ((uint32_t *)(xq + (size_t)blk * QK_K))[lane] = r.packed;
    if (lane == 0) xd[blk] = r.d;
    if ((lane & 3) == 0) xsum[(size_t)blk * 16 + (lane >> 2)] = (int16_t)r.gsum;
}

int launch_q8k_quant(const float *x, int nblocks, int8_t *xq, float *xd, int16_t *xsum,
                     hipStream_t s)
{
    if (nblocks <= 0) return QMAG_OK;
    if (!x || !xq || !xd || !xsum) return fail(QMAG_ERR_ARG, "q8k_quant: null pointer");
    const int wgs = (nblocks + 3) / 4;
    prof_begin(PROF_Q8K, s);
    hipLaunchKernelGGL(q8k_quant_kernel, dim3(wgs), dim3(256), 0, s, x, nblocks, xq, xd, xsum);
    prof_end(PROF_Q8K, s);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// ------------------------------------------------------------------------
template <int WT>
struct RowTask;

template <>
struct RowTask<QMAG_TYPE_Q4_K> {
    struct Raw {
        uint4 hdr, q0, q1;
    };
    using Act = Q4Act;
    static constexpr int BLOCK = Q4K_BYTES;
    // task q of super-block ib of the row at rowp (nb super-blocks)
    __device__ static void load_raw(Raw &r, const uint8_t *rowp, int ib, int q, int)
    {
        const uint8_t *blk = rowp + (size_t)ib * BLOCK;
        r.hdr = ld16(blk);
        r.q0 = ld16(blk + 16 + 32 * q);
        r.q1 = ld16(blk + 32 + 32 * q);
    }
    __device__ static void load_act(Act &a, const int8_t *xq, const float *xd, const int16_t *xs,
                                    int ib, int q)
    {
        q4_load_act(a, xq, xd, xs, ib, q);
    }
    // float contribution of this lane's task
    // the task's value is rounded before any caller sums it (the empty asm
    // keeps the compiler from fusing its last product into that sum, which
    // it would do differently in different kernels)
    __device__ static float dot(const Raw &r, const Act &a, int q)
    {
        float p = q4_task(r.hdr, r.q0, r.q1, a, q);
        __asm__ volatile("" : "+v"(p));
        return p;
    }
};

template <>
struct RowTask<QMAG_TYPE_Q6_K> {
    using Raw = Q6Raw;
    struct Act {
        Q6Act a;
        float xd;
    };
    static constexpr int BLOCK = Q6K_BYTES;
    __device__ static void load_raw(Raw &r, const uint8_t *rowp, int ib, int q, int)
    {
        q6_load_raw(r, rowp + (size_t)ib * BLOCK, q >> 1, q & 1);
    }
    __device__ static void load_act(Act &a, const int8_t *xq, const float *xd, const int16_t *,
                                    int ib, int q)
    {
        q6_load_act(a.a, xq, ib, q >> 1, q & 1);
        a.xd = xd[ib];
    }
    // the quad's int32 block sum is formed exactly, then d*xd*isum once
    __device__ static float dot(const Raw &r, const Act &a, int q)
    {
        const int part = q6_int_dot(r, a.a, q & 1);
        const int isum = group_sum_i<4>(part);
        float p = h2f(r.d) * a.xd * (float)isum;
        __asm__ volatile("" : "+v"(p));             // rounded here, as for Q4_K
        return q == 0 ? p : 0.0f;
    }
};

// Q6_K rows repacked for the matvec (QMAG_TYPE_Q6_K_R; a layout of this
// library, not of the GGUF): a row of nb super-blocks, nb a multiple of 8 so
// every row starts on 16 bytes, is stored as planes -- each block's four
// 16-byte low ql task pieces (ql[0,16), [16,32), [64,80), [80,96)), then
// every block's four high ones ([32,48), [48,64), [96,112), [112,128)), then
// the qh bytes, the scales and the d values of every block, nb * 210 bytes
// as before.  A task's loads are then aligned and the row's lanes read 512
// contiguous bytes per ql or qh load; the bytes a task holds, and so its dot,
// are those of the block layout.
template <>
struct RowTask<QMAG_TYPE_Q6_K_R> : RowTask<QMAG_TYPE_Q6_K> {
    __device__ static void load_raw(Raw &r, const uint8_t *rowp, int ib, int q, int nb)
    {
        r.ql_lo = ld16(rowp + 64 * ib + 16 * q);
        r.ql_hi = ld16(rowp + 64 * (nb + ib) + 16 * q);
        r.qh = ld16(rowp + 64 * (2 * nb + ib) + 16 * q);
        r.sc = ld8(rowp + 192 * nb + 16 * ib + 8 * (q >> 1));
        r.d = ld2(rowp + 208 * nb + 2 * ib);
    }
};

// Block layout -> repacked rows: one thread per super-block.
__global__ __launch_bounds__(256) void repack_q6k_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                         int nb, long nblocks)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblocks) return;
    const long row = i / nb;
    const int ib = (int)(i % nb);
    const uint8_t *b = src + i * Q6K_BYTES;
    uint8_t *rp = dst + row * nb * Q6K_BYTES;
    for (int q = 0; q < 4; q++)
        for (int j = 0; j < 16; j++) {
            rp[64 * ib + 16 * q + j] = b[64 * (q >> 1) + 16 * (q & 1) + j];
            rp[64 * (nb + ib) + 16 * q + j] = b[64 * (q >> 1) + 32 + 16 * (q & 1) + j];
        }
    for (int j = 0; j < 64; j++) rp[64 * (2 * nb + ib) + j] = b[128 + j];
    for (int j = 0; j < 16; j++) rp[192 * nb + 16 * ib + j] = b[192 + j];
    rp[208 * nb + 2 * ib] = b[208];
    rp[208 * nb + 2 * ib + 1] = b[209];
}

// The same transform in place: one workgroup per row reads the whole row
// into LDS before any byte of it is written back (rows are independent), so
// no second copy of the matrix is needed.  Destination byte o of the row
// takes the block-layout byte the out-of-place kernel puts there.
__device__ __forceinline__ int repack_src(int o, int nb)
{
    if (o < 128 * nb) {                           // the low, then the high ql planes
        const int hi = o >= 64 * nb, r = hi ? o - 64 * nb : o;
        const int ib = r / 64, q = (r % 64) / 16, j = r % 16;
        return ib * Q6K_BYTES + 64 * (q >> 1) + 32 * hi + 16 * (q & 1) + j;
    }
    if (o < 192 * nb) return ((o - 128 * nb) / 64) * Q6K_BYTES + 128 + (o - 128 * nb) % 64;   // qh
    if (o < 208 * nb) return ((o - 192 * nb) / 16) * Q6K_BYTES + 192 + (o - 192 * nb) % 16;   // scales
    return ((o - 208 * nb) / 2) * Q6K_BYTES + 208 + (o - 208 * nb) % 2;                       // d
}
__global__ __launch_bounds__(256) void repack_q6k_inplace_kernel(uint8_t *__restrict__ W, int nb)
{
    extern __shared__ uint8_t s_row[];
    const int rb = nb * Q6K_BYTES;
    uint8_t *rp = W + (size_t)blockIdx.x * rb;
    for (int i = (int)threadIdx.x; i < rb; i += 256) s_row[i] = rp[i];
    __syncthreads();
    for (int o = (int)threadIdx.x; o < rb; o += 256) rp[o] = s_row[repack_src(o, nb)];
}

constexpr int REPACK_INPLACE_MAX_ROW = 65536;     // bytes of a row staged in LDS

int launch_repack_q6k(const void *src, void *dst, int n_in, int n_out, hipStream_t s)
{
    if (n_in <= 0 || n_in % (8 * QK_K) || n_out <= 0)
        return fail(QMAG_ERR_ARG, "repack_q6k: n_in=%d (a multiple of 2048) n_out=%d", n_in, n_out);
    if (!src || !dst || ((uintptr_t)dst & 15))
        return fail(QMAG_ERR_ARG, "repack_q6k: null or unaligned pointer (dst needs 16-byte alignment)");
    const size_t bytes = (size_t)n_out * (n_in / QK_K) * Q6K_BYTES;
    const uintptr_t a = (uintptr_t)src, b = (uintptr_t)dst;
    if (a == b) {
        const int nb = n_in / QK_K, rb = nb * Q6K_BYTES;
        if (rb > REPACK_INPLACE_MAX_ROW)
            return fail(QMAG_ERR_ARG, "repack_q6k: in place needs rows of at most %d bytes (n_in=%d)",
                        REPACK_INPLACE_MAX_ROW, n_in);
        hipLaunchKernelGGL(repack_q6k_inplace_kernel, dim3((unsigned)n_out), dim3(256), (size_t)rb, s,
                           (uint8_t *)dst, nb);
        QMAG_HIP(hipGetLastError());
        return QMAG_OK;
    }
    if (a < b + bytes && b < a + bytes)
        return fail(QMAG_ERR_ARG, "repack_q6k: src and dst overlap without being the same buffer");
    const long nblocks = (long)n_out * (n_in / QK_K);
    hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t *)src, (uint8_t *)dst, n_in / QK_K, nblocks);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// Q8_K of one activation vector of NB blocks into a workgroup's LDS: each
// half-wave quantises one 256-block (8 values per lane, q8k_quant_half, the
// same bits as q8k_quant_kernel), so a wave covers two blocks at once.
template <int NB>
__device__ __forceinline__ void q8k_x_to_lds(const float *__restrict__ xf, int8_t *s_xq, float *s_xd,
                                             int16_t *s_xs)
{
    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6), hl = lane >> 5, L = lane & 31;
    for (int b0 = 2 * wv; b0 < NB; b0 += 2 * (QMAG_MV_WG / 64)) {
        const int b = b0 + hl;
        const int bb = b < NB ? b : NB - 1;    // the half past the last block (NB = 1) stores nothing
        const Q8Lane2 r = q8k_quant_half(ldg4(xf + bb * QK_K + 8 * L), ldg4(xf + bb * QK_K + 8 * L + 4));
        if (b < NB) {
            ((uint2 *)(s_xq + b * QK_K))[L] = make_uint2(r.packed[0], r.packed[1]);
            if (L == 0) s_xd[b] = r.d;
            if ((L & 1) == 0) s_xs[b * 16 + (L >> 1)] = (int16_t)r.gsum;
        }
    }
}

// ONE_TOKEN: T = 1, the activation operand is loaded once per lane.  XF
// (with ONE_TOKEN): the kernel takes x itself and every workgroup computes
// its Q8_K into LDS with the same per-block routine as q8k_quant_kernel
// (bit-identical), after its first weight rows are requested -- one launch
// per matvec instead of two.
template <int WT, int NB, bool ONE_TOKEN, bool XF = false>
__global__ __launch_bounds__(QMAG_MV_WG) void matvec_kernel(const uint8_t *__restrict__ W,
                                                     const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xd,
                                                     const int16_t *__restrict__ xsum,
                                                     float *__restrict__ out, int n_out, int T,
                                                     const float *__restrict__ xf = nullptr)
{
    using RT = RowTask<WT>;
    constexpr int TPR = 4 * NB;                 // tasks per row
    constexpr int LPR = TPR < 64 ? TPR : 64;    // lanes per row
    constexpr int TPL = TPR / LPR;              // tasks per lane
    constexpr int RPW = 64 / LPR;               // rows per wave step
    constexpr int U = QMAG_MV_U;                // wave steps in flight
    constexpr size_t RB = (size_t)NB * RT::BLOCK;
    constexpr int N_IN = NB * QK_K;

    const int lane = lane_id();
    const int sub = lane % LPR, rw = lane / LPR;
    const int q = sub & 3;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nwave = (int)((gridDim.x * blockDim.x) >> 6);

    typename RT::Raw raw[U][TPL];
    auto load_rows = [&](int base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = base + u * RPW + rw;
#pragma unroll
            for (int j = 0; j < TPL; j++) {
                if (row < n_out)
                    RT::load_raw(raw[u][j], W + (size_t)row * RB, (sub + LPR * j) >> 2, q, NB);
                else
                    raw[u][j] = typename RT::Raw{};
            }
        }
    };
    const int base0 = wave * RPW * U;
    typename RT::Act act[TPL];
    if constexpr (XF) {
        __shared__ __align__(16) int8_t s_xq[N_IN];
        __shared__ float s_xd[NB];
        __shared__ __align__(16) int16_t s_xs[N_IN / 16];
        load_rows(base0);                       // the weights are in flight during the quantisation
        q8k_x_to_lds<NB>(xf, s_xq, s_xd, s_xs);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TPL; j++) RT::load_act(act[j], s_xq, s_xd, s_xs, (sub + LPR * j) >> 2, q);
    } else if constexpr (ONE_TOKEN) {
#pragma unroll
        for (int j = 0; j < TPL; j++) RT::load_act(act[j], xq, xd, xsum, (sub + LPR * j) >> 2, q);
    }

    for (int base = base0; base < n_out; base += nwave * RPW * U) {
        if (!XF || base != base0) load_rows(base);
        for (int t = 0; t < T; t++) {
            if constexpr (!ONE_TOKEN) {
#pragma unroll
                for (int j = 0; j < TPL; j++)
                    RT::load_act(act[j], xq + (size_t)t * N_IN, xd + (size_t)t * NB,
                                 xsum + (size_t)t * (N_IN / 16), (sub + LPR * j) >> 2, q);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                float v = 0.0f;
#pragma unroll
                for (int j = 0; j < TPL; j++) v = __fadd_rn(v, RT::dot(raw[u][j], act[j], q));   // no contraction
                v = group_sum<LPR>(v);
                const int row = base + u * RPW + rw;
                if (sub == 0 && row < n_out) out[(size_t)t * n_out + row] = v;
            }
        }
    }
}

template <int WT, int NB>
static int launch_mv_nb(const int8_t *xq, const float *xd, const int16_t *xsum, const void *W,
                        int n_out, int T, float *out, hipStream_t s, const float *xf)
{
    constexpr int TPR = 4 * NB;
    constexpr int LPR = TPR < 64 ? TPR : 64;
    constexpr int RPW = 64 / LPR;
    constexpr int WPG = QMAG_MV_WG / 64;        // waves per workgroup
    const long groups = ((long)n_out + RPW * QMAG_MV_U - 1) / (RPW * QMAG_MV_U);
    const long cap = (long)(ctx().n_cu > 0 ? ctx().n_cu : 256) * QMAG_MV_CAP;    // waves
    const long waves = groups < cap ? groups : cap;
    const int wgs = (int)((waves + WPG - 1) / WPG);
    prof_begin(PROF_MATVEC, s);
    if (xf)
        hipLaunchKernelGGL((matvec_kernel<WT, NB, true, true>), dim3(wgs), dim3(QMAG_MV_WG), 0, s,
                           (const uint8_t *)W, xq, xd, xsum, out, n_out, 1, xf);
    else if (T == 1)
        hipLaunchKernelGGL((matvec_kernel<WT, NB, true>), dim3(wgs), dim3(QMAG_MV_WG), 0, s,
                           (const uint8_t *)W, xq, xd, xsum, out, n_out, T, nullptr);
    else
        hipLaunchKernelGGL((matvec_kernel<WT, NB, false>), dim3(wgs), dim3(QMAG_MV_WG), 0, s,
                           (const uint8_t *)W, xq, xd, xsum, out, n_out, T, nullptr);
    prof_end(PROF_MATVEC, s);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// Several matrices over the same x at T = 1 (the projections the engine
// computes from one activation vector, nn.c:2111-2113, 2162-2170) in one
// launch: waves are dealt to the matrices in order (matrix m takes waves
// wave0[m] .. wave0[m+1]-1, one wave step of rows each, no grid stride), each
// wave requests its rows with its matrix's row task, then every workgroup
// computes Q8_K(x) into LDS exactly as the one-token kernel does, and each
// wave finishes its rows with that kernel's dot and reduction: every output
// is bit-identical to a separate qmag_matmul_dev call.
template <int NB>
__global__ __launch_bounds__(QMAG_MV_WG) void matvec_group_kernel(MvGroup g, const float *__restrict__ xf)
{
    using R4 = RowTask<QMAG_TYPE_Q4_K>;
    using R6 = RowTask<QMAG_TYPE_Q6_K>;
    using R6R = RowTask<QMAG_TYPE_Q6_K_R>;
    constexpr int TPR = 4 * NB;
    constexpr int LPR = TPR < 64 ? TPR : 64;
    constexpr int TPL = TPR / LPR;
    constexpr int RPW = 64 / LPR;
    constexpr int U = QMAG_MV_U;
    constexpr int N_IN = NB * QK_K;
    __shared__ __align__(16) int8_t s_xq[N_IN];
    __shared__ float s_xd[NB];
    __shared__ __align__(16) int16_t s_xs[N_IN / 16];

    const int lane = lane_id();
    const int sub = lane % LPR, rw = lane / LPR;
    const int q = sub & 3;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    int m = 0;
    while (m + 1 < g.n && wave >= g.wave0[m + 1]) m++;          // wave-uniform
    const bool live = wave < g.wave0[g.n];
    const int wt = g.wtype[m], n_out = g.n_out[m];
    const uint8_t *W = g.W[m];
    const int base = (wave - g.wave0[m]) * RPW * U;
    constexpr size_t RB4 = (size_t)NB * Q4K_BYTES, RB6 = (size_t)NB * Q6K_BYTES;

    typename R4::Raw r4[U][TPL];
    typename R6::Raw r6[U][TPL];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int row = base + u * RPW + rw;
#pragma unroll
        for (int j = 0; j < TPL; j++) {
            r4[u][j] = typename R4::Raw{};
            r6[u][j] = typename R6::Raw{};
            const int ib = (sub + LPR * j) >> 2;
            if (live && row < n_out) {
                if (wt == QMAG_TYPE_Q4_K) R4::load_raw(r4[u][j], W + (size_t)row * RB4, ib, q, NB);
                else if (wt == QMAG_TYPE_Q6_K) R6::load_raw(r6[u][j], W + (size_t)row * RB6, ib, q, NB);
                else R6R::load_raw(r6[u][j], W + (size_t)row * RB6, ib, q, NB);
            }
        }
    }
    q8k_x_to_lds<NB>(xf, s_xq, s_xd, s_xs);
    __syncthreads();
    if (!live) return;
    float *out = g.out[m];
    if (wt == QMAG_TYPE_Q4_K) {
        typename R4::Act act[TPL];
#pragma unroll
        for (int j = 0; j < TPL; j++) R4::load_act(act[j], s_xq, s_xd, s_xs, (sub + LPR * j) >> 2, q);
#pragma unroll
        for (int u = 0; u < U; u++) {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < TPL; j++) v = __fadd_rn(v, R4::dot(r4[u][j], act[j], q));
            v = group_sum<LPR>(v);
            const int row = base + u * RPW + rw;
            if (sub == 0 && row < n_out) out[row] = v;
        }
    } else {
        typename R6::Act act[TPL];
#pragma unroll
        for (int j = 0; j < TPL; j++) R6::load_act(act[j], s_xq, s_xd, s_xs, (sub + LPR * j) >> 2, q);
#pragma unroll
        for (int u = 0; u < U; u++) {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < TPL; j++) v = __fadd_rn(v, R6::dot(r6[u][j], act[j], q));
            v = group_sum<LPR>(v);
            const int row = base + u * RPW + rw;
            if (sub == 0 && row < n_out) out[row] = v;
        }
    }
}

int launch_matvec_group(const float *x, int n_in, int n_mat, const void *const *W, const int *n_out,
                        const int *wtype, float *const *out, hipStream_t s)
{
    if (n_mat < 1 || n_mat > QMAG_MV_GROUP_MAX) return fail(QMAG_ERR_ARG, "matmul_group: n_mat=%d (1..%d)", n_mat, QMAG_MV_GROUP_MAX);
    if (!x || !W || !n_out || !wtype || !out) return fail(QMAG_ERR_ARG, "matmul_group: null pointer");
    const int nb = n_in / QK_K;
    if (n_in <= 0 || n_in % QK_K || !(nb == 1 || nb == 2 || nb == 4 || nb == 8 || nb == 16 || nb == 32))
        return fail(QMAG_ERR_ARG, "matmul_group: n_in=%d (a power of two from 256 to 8192)", n_in);
    const int lpr = 4 * nb < 64 ? 4 * nb : 64, rows_per_wave = 64 / lpr * QMAG_MV_U;
    MvGroup g{};
    g.n = n_mat;
    long waves = 0;
    for (int i = 0; i < n_mat; i++) {
        const int t = wtype[i];
        if (t != QMAG_TYPE_Q4_K && t != QMAG_TYPE_Q6_K && t != QMAG_TYPE_Q6_K_R)
            return fail(QMAG_ERR_ARG, "matmul_group: matrix %d: unsupported wtype %d", i, t);
        if (!W[i] || !out[i] || n_out[i] <= 0) return fail(QMAG_ERR_ARG, "matmul_group: matrix %d: null or empty", i);
        if (t == QMAG_TYPE_Q6_K_R && (n_in % (8 * QK_K) || ((uintptr_t)W[i] & 15)))
            return fail(QMAG_ERR_ARG, "matmul_group: matrix %d: repacked Q6_K needs n_in %% 2048 == 0 and 16-byte aligned rows", i);
        g.W[i] = (const uint8_t *)W[i];
        g.out[i] = out[i];
        g.n_out[i] = n_out[i];
        g.wtype[i] = t;
        g.wave0[i] = (int)waves;
        waves += (n_out[i] + rows_per_wave - 1) / rows_per_wave;
        if (waves > QMAG_MV_GROUP_MAX_WAVES)
            return fail(QMAG_ERR_ARG, "matmul_group: %ld row steps exceed %d (call the matrices separately)", waves,
                        QMAG_MV_GROUP_MAX_WAVES);
    }
    g.wave0[n_mat] = (int)waves;
    const int wgs = (int)((waves + QMAG_MV_WG / 64 - 1) / (QMAG_MV_WG / 64));
    prof_begin(PROF_MATVEC, s);
    switch (nb) {
    case 1: hipLaunchKernelGGL(matvec_group_kernel<1>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    case 2: hipLaunchKernelGGL(matvec_group_kernel<2>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    case 4: hipLaunchKernelGGL(matvec_group_kernel<4>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    case 8: hipLaunchKernelGGL(matvec_group_kernel<8>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    case 16: hipLaunchKernelGGL(matvec_group_kernel<16>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    default: hipLaunchKernelGGL(matvec_group_kernel<32>, dim3(wgs), dim3(QMAG_MV_WG), 0, s, g, x); break;
    }
    prof_end(PROF_MATVEC, s);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// Any row length (nb super-blocks, not only the powers of two the tiled
// kernel is instantiated for): one wave per row, lane l taking tasks
// l, l + 64, ... of the row (4 per super-block, so the 4 tasks of a Q6_K
// block stay in one lane quad for its exact integer block sum).
template <int WT>
__global__ __launch_bounds__(256) void matvec_any_kernel(const uint8_t *__restrict__ W,
                                                         const int8_t *__restrict__ xq,
                                                         const float *__restrict__ xd,
                                                         const int16_t *__restrict__ xsum,
                                                         float *__restrict__ out, int nb, int n_out, int T)
{
    using RT = RowTask<WT>;
    const int lane = lane_id(), q = lane & 3;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nwave = (int)((gridDim.x * blockDim.x) >> 6);
    const size_t rb = (size_t)nb * RT::BLOCK;
    const int ntask = 4 * nb, n_in = nb * QK_K;
    for (int row = wave; row < n_out; row += nwave) {
        for (int t = 0; t < T; t++) {
            float v = 0.0f;
            for (int tk = lane; tk < ntask; tk += 64) {
                typename RT::Raw r;
                typename RT::Act a;
                RT::load_raw(r, W + (size_t)row * rb, tk >> 2, q, nb);
                RT::load_act(a, xq + (size_t)t * n_in, xd + (size_t)t * nb, xsum + (size_t)t * (n_in / 16),
                             tk >> 2, q);
                v += RT::dot(r, a, q);
            }
            v = group_sum<64>(v);
            if (lane == 0) out[(size_t)t * n_out + row] = v;
        }
    }
}

template <int WT>
static int launch_mv_any(const int8_t *xq, const float *xd, const int16_t *xsum, const void *W, int nb,
                         int n_out, int T, float *out, hipStream_t s)
{
    const long cap = (long)(ctx().n_cu > 0 ? ctx().n_cu : 256) * 32;    // waves
    const long waves = n_out < cap ? n_out : cap;
    const int wgs = (int)((waves + 3) / 4);
    prof_begin(PROF_MATVEC, s);
    hipLaunchKernelGGL(matvec_any_kernel<WT>, dim3(wgs), dim3(256), 0, s, (const uint8_t *)W, xq, xd, xsum, out,
                       nb, n_out, T);
    prof_end(PROF_MATVEC, s);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// the tiled kernel is instantiated for these row lengths (super-blocks)
static bool tiled_nb(int nb) { return nb == 1 || nb == 2 || nb == 4 || nb == 8 || nb == 16 || nb == 32; }

template <int WT>
static int launch_mv_t(const int8_t *xq, const float *xd, const int16_t *xsum, const void *W,
                       int n_in, int n_out, int T, float *out, hipStream_t s, const float *xf)
{
    if (!tiled_nb(n_in / QK_K)) {
        if (xf) return fail(QMAG_ERR_ARG, "matvec: internal: fused Q8_K path needs a tiled row length");
        return launch_mv_any<WT>(xq, xd, xsum, W, n_in / QK_K, n_out, T, out, s);
    }
    switch (n_in / QK_K) {
    case 1: return launch_mv_nb<WT, 1>(xq, xd, xsum, W, n_out, T, out, s, xf);
    case 2: return launch_mv_nb<WT, 2>(xq, xd, xsum, W, n_out, T, out, s, xf);
    case 4: return launch_mv_nb<WT, 4>(xq, xd, xsum, W, n_out, T, out, s, xf);
    case 8: return launch_mv_nb<WT, 8>(xq, xd, xsum, W, n_out, T, out, s, xf);
    case 16: return launch_mv_nb<WT, 16>(xq, xd, xsum, W, n_out, T, out, s, xf);
    case 32: return launch_mv_nb<WT, 32>(xq, xd, xsum, W, n_out, T, out, s, xf);
    default: return fail(QMAG_ERR_ARG, "matvec: internal: n_in=%d has no tiled instance", n_in);
    }
}

int launch_matvec(const int8_t *xq, const float *xd, const int16_t *xsum, const void *W, int n_in,
                  int n_out, int T, int wtype, float *out, hipStream_t s)
{
    if (n_in <= 0 || n_in % QK_K || n_out <= 0 || T <= 0)
        return fail(QMAG_ERR_ARG, "matvec: n_in=%d n_out=%d T=%d", n_in, n_out, T);
    if (!xq || !xd || !W || !out || (wtype == QMAG_TYPE_Q4_K && !xsum))
        return fail(QMAG_ERR_ARG, "matvec: null pointer");
    if (wtype == QMAG_TYPE_Q4_K) return launch_mv_t<QMAG_TYPE_Q4_K>(xq, xd, xsum, W, n_in, n_out, T, out, s, nullptr);
    if (wtype == QMAG_TYPE_Q6_K) return launch_mv_t<QMAG_TYPE_Q6_K>(xq, xd, xsum, W, n_in, n_out, T, out, s, nullptr);
    if (wtype == QMAG_TYPE_Q6_K_R) {
        if (n_in % (8 * QK_K) || ((uintptr_t)W & 15))
            return fail(QMAG_ERR_ARG, "matvec: repacked Q6_K needs n_in %% 2048 == 0 and 16-byte aligned rows");
        return launch_mv_t<QMAG_TYPE_Q6_K_R>(xq, xd, xsum, W, n_in, n_out, T, out, s, nullptr);
    }
    return fail(QMAG_ERR_ARG, "matvec: unsupported wtype %d", wtype);
}

bool matvec_x_supported(int n_in) { return n_in > 0 && n_in % QK_K == 0 && tiled_nb(n_in / QK_K); }

int launch_matvec_x(const float *x, const void *W, int n_in, int n_out, int wtype, float *out, hipStream_t s)
{
    if (n_in <= 0 || n_in % QK_K || n_out <= 0) return fail(QMAG_ERR_ARG, "matvec: n_in=%d n_out=%d", n_in, n_out);
    if (!matvec_x_supported(n_in)) return fail(QMAG_ERR_ARG, "matvec: internal: n_in=%d has no fused Q8_K form", n_in);
    if (!x || !W || !out) return fail(QMAG_ERR_ARG, "matvec: null pointer");
    if (wtype == QMAG_TYPE_Q4_K)
        return launch_mv_t<QMAG_TYPE_Q4_K>(nullptr, nullptr, nullptr, W, n_in, n_out, 1, out, s, x);
    if (wtype == QMAG_TYPE_Q6_K)
        return launch_mv_t<QMAG_TYPE_Q6_K>(nullptr, nullptr, nullptr, W, n_in, n_out, 1, out, s, x);
    if (wtype == QMAG_TYPE_Q6_K_R) {
        if (n_in % (8 * QK_K) || ((uintptr_t)W & 15))
            return fail(QMAG_ERR_ARG, "matvec: repacked Q6_K needs n_in %% 2048 == 0 and 16-byte aligned rows");
        return launch_mv_t<QMAG_TYPE_Q6_K_R>(nullptr, nullptr, nullptr, W, n_in, n_out, 1, out, s, x);
    }
    return fail(QMAG_ERR_ARG, "matvec: unsupported wtype %d", wtype);
}

}  // namespace qmag
