// qmag_prefill.hip -- the MoE FFN layer for a batch of tokens (prefill,
// src/nn.c:509-649 with T > 1) as a grouped expert GEMM on int8 MFMA.
//
//   router_tile_kernel   per 256-wide k chunk, part[kc][T][E] = x . Wr^T, fp32
//                        MFMA; topk_kernel sums the chunks and adds the bias
//   topk_kernel          (qmag_moe.hip) softmax/top-k, Q8_K(x), shared gate
//   group_kernel         (token, slot) pairs bucketed by expert; the shared
//                        expert is bucket E with one pair per token
//   gateup_rows_kernel   h = silu(x.G) * (x.U) per pair: chunks of up to 64
//                        pairs of one expert x 32 rows of h, the weight rows
//                        resident in registers (16-byte pieces per lane); the
//                        6-bit sub-block scales folded into the weight operand
//                        (sc = 8 sh + sl), two v_mfma_i32_16x16x64_i8 chains
//                        per 16 pairs x 16 rows (8 gate, 8 up) x 64 k, the min
//                        term on the fp32 MFMA
//   q8k_quant_kernel     Q8_K(h) per pair
//   down_rows_kernel     y[pair] = Q8_K(h) . D^T per chunk x 64 rows: Q6_K
//                        one 16-value group per MFMA result (the activations
//                        of the other three lane quarters zero), or Q4_K per
//                        sub-block
//   combine_kernel       out[t] = sum_k w_k y[t,k] + gs y[t,shared] in the
//                        reference order (nn.c:614-629), plus an optional
//                        residual
//
// Integer parity: each MFMA result is an exact int32 sum -- of one
// sub-block or group (the down path), or of a super-block with the
// sub-block scales folded in (gate/up: sum_j sc_j P_j = sum(q sl) + 8
// sum(q sh), every operand byte <= 105) -- the integer sums of src/q8k.c;
// where the scale products are formed after the MFMA they are accumulated
// exactly in int32 per super-block (with 24-bit multiplies, exact here:
// |MFMA result| <= 32*15*128 < 2^17 for a Q4_K sub-block, 16*32*128 for a
// Q6_K group, and the scales are 6- or 8-bit; v_mad_i32_i24 runs at the full
// VALU rate where a 32-bit multiply takes four passes); only the
// fp32 epilogue (scale * xd * integer sum) is associated differently from
// the reference's per-sub-block fp32 terms, well inside 1e-4 of max|y|.
//
// Every expert's weights are read once per 64-pair chunk (the shared
// expert's by every chunk of 64 tokens); the pair buffers (h: T*S*F fp32,
// y: T*S*N fp32) stay in HBM between kernels.
#include "qmag_internal.h"

namespace qmag {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int PB = 16;            // pairs per MFMA tile (the 16-wide M side)

// --------------------------------------------------------------- router --
// grid: (T / 64) x (E / 64) x (N / 256), 512 threads; a workgroup = 64 tokens
// x 64 experts x one 256-wide k chunk kc.  The 64 x rows and 64 router rows
// of the chunk are staged in LDS by DMA (one 1 KB row per instruction,
// rows padded by 16 bytes so the 16 rows one read touches start 4 banks
// apart), and wave w computes tokens 16 (w & 3) .. +16 against experts
// 32 (w >> 2) .. +32 as two 16 x 16 tiles.  Each tile's product over the
// chunk is 64 v_mfma_f32_16x16x4f32 into four accumulators (lane quarter q
// takes k = 16 u + 4 q .. +4 of step u, accumulator u % 4), summed as
// (a0 + a1) + (a2 + a3) and stored as the chunk's partial
// part[kc][token][expert]; topk_kernel adds the chunks in order and then
// the bias.  Each x and router row is read by 4 (not 16) workgroups, from
// LDS instead of registers, so one workgroup per CU suffices.  Rows past T or
// E are clamped to the last one: they only reach outputs that are not
// stored.
constexpr int RT_ROWS = 64;                    // tokens (experts) per workgroup
constexpr int RT_STRIDE = 256 + 4;             // padded LDS row, floats
__global__ __launch_bounds__(512) void router_tile_kernel(const float *__restrict__ Wr,
                                                          const float *__restrict__ x, int N, int E, int T,
                                                          float *__restrict__ part)
{
    __shared__ __align__(16) float s_x[RT_ROWS * RT_STRIDE], s_w[RT_ROWS * RT_STRIDE];
    const int tb = (int)blockIdx.x, eb = (int)blockIdx.y, kc = (int)blockIdx.z;
    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6), lr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int i = 0; i < RT_ROWS / 8; i++) {
        const int r = wv + 8 * i;
        const int tok = min(tb * RT_ROWS + r, T - 1), e = min(eb * RT_ROWS + r, E - 1);
        __builtin_amdgcn_global_load_lds((const QMAG_GLOBAL void *)(x + (size_t)tok * N + kc * 256 + lane * 4),
                                         (__attribute__((address_space(3))) void *)(s_x + r * RT_STRIDE), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const QMAG_GLOBAL void *)(Wr + (size_t)e * N + kc * 256 + lane * 4),
                                         (__attribute__((address_space(3))) void *)(s_w + r * RT_STRIDE), 16, 0, 0);
    }
    __syncthreads();
    const int t0 = 16 * (wv & 3), e0 = 32 * (wv >> 2);
    const float *xa = s_x + (t0 + lr) * RT_STRIDE + 4 * q;
    const float *wa = s_w + (e0 + lr) * RT_STRIDE + 4 * q;
    v4f acc[2][4];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[j][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 16; u++) {
        const float4 a = *(const float4 *)(xa + 16 * u);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float4 b = *(const float4 *)(wa + 16 * RT_STRIDE * j + 16 * u);
            v4f &c = acc[j][u & 3];
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
        }
    }
    // lane holds tile rows 4q + i (tokens) x column lr (expert)
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const v4f sum = (acc[j][0] + acc[j][1]) + (acc[j][2] + acc[j][3]);
        const int eo = eb * RT_ROWS + e0 + 16 * j + lr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int to = tb * RT_ROWS + t0 + 4 * q + i;
            if (to < T && eo < E) part[((size_t)kc * T + to) * E + eo] = sum[i];
        }
    }
}

// ---------------------------------------------------------------- group --
// grp layout: cnt[E+1], off[E+2]; chunk[c] = {bucket
// (-1 past the last chunk), pairs, offset of its first pair in perm, 0}, one
// int4 per MC-pair chunk, so a workgroup learns all it needs from one load;
// perm[T*S] (pair ids = t*S + slot, bucketed by expert).  Positions
// inside a bucket come from LDS atomics; every pair's result is computed
// independently of its neighbours, so the order does not change any output.
//
// Chunk order (the dispatch order of the chunked GEMMs): every full chunk
// first, then the partial ones by decreasing size, so the longest
// workgroups start first and the grid ends on the shortest ones.
constexpr int MC = 64;            // pairs per chunk of the chunked GEMMs (4 MFMA tiles)
// the GEMM workgroups' 4 waves read 16 of a chunk's pair ids each, and the
// group kernel's chunk scans run within one wave: a chunk is 4 x 16 pairs
static_assert(MC == 4 * 16 && MC <= 64, "chunk size is tied to the 4-wave id loads");

__global__ __launch_bounds__(1024) void group_kernel(const int *__restrict__ sel, int T, int K, int E,
                                                     int *__restrict__ grp,
                                                     int4 *__restrict__ chunk, int max_chunks,
                                                     int *__restrict__ perm)
{
    __shared__ int s_cnt[257], s_off[258], s_fill[257], s_inc[257], s_finc[257];
    __shared__ int s_bin[MC], s_binf[MC];     // partial chunks by MC - size
    __shared__ int s_nch, s_wtot[2][5];
    const int tid = (int)threadIdx.x, S = K + 1;
    for (int e = tid; e <= E; e += 1024) {
        s_cnt[e] = 0;
        s_fill[e] = 0;
    }
    if (tid < MC) {
        s_bin[tid] = 0;
        s_binf[tid] = 0;
    }
    __syncthreads();
    // ids come from the top-k (always < E); clamp anyway, this indexes LDS
    auto expert = [&](int p) { return min(max(sel[p], 0), E - 1); };
    for (int p = tid; p < T * K; p += 1024) atomicAdd(&s_cnt[expert(p)], 1);
    if (tid == 0) s_cnt[E] = T;      // shared expert: every token
    __syncthreads();
    // inclusive prefix sums of the pair counts and the full-chunk counts over
    // the E + 1 <= 257 buckets: a scan inside each of waves 0-4, then the
    // totals of the waves before; the partial chunks are counted per size
    {
        const int lane = tid & 63, wv = tid >> 6;
        const int c = tid <= E ? s_cnt[tid] : 0;
        if (c % MC) atomicAdd(&s_bin[MC - c % MC], 1);
        int ci = c, fi = c / MC;
        if (wv < 5) {                          // wave-uniform
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int o = __shfl_up(ci, d), of = __shfl_up(fi, d);
                if (lane >= d) {
                    ci += o;
                    fi += of;
                }
            }
            if (lane == 63) {
                s_wtot[0][wv] = ci;
                s_wtot[1][wv] = fi;
            }
        }
        __syncthreads();
        if (tid <= E) {
            for (int w = 0; w < wv; w++) {
                ci += s_wtot[0][w];
                fi += s_wtot[1][w];
            }
            s_inc[tid] = ci;
            s_finc[tid] = fi;
        }
        __syncthreads();
    }
    // exclusive prefix of the size bins (one wave; bin i holds chunks of
    // MC - i pairs, so increasing i is decreasing size)
    if (tid < MC) {
        const int v = s_bin[tid];
        int incl = v;
#pragma unroll
        for (int d = 1; d < MC; d <<= 1) {
            const int o = __shfl_up(incl, d, MC);
            if (tid >= d) incl += o;
        }
        s_bin[tid] = incl - v;
        if (tid == MC - 1) s_nch = s_finc[E] + incl;
    }
    __syncthreads();
    if (tid <= E) {
        int *cnt = grp, *off = grp + (E + 1);
        const int c = s_cnt[tid];
        s_off[tid] = s_inc[tid] - c;
        cnt[tid] = c;
        off[tid] = s_inc[tid] - c;
        const int nf = c / MC, f0 = s_finc[tid] - nf, o = s_inc[tid] - c;
        for (int i = 0; i < nf; i++) chunk[f0 + i] = make_int4(tid, MC, o + i * MC, 0);
        if (c % MC) {
            const int bin = MC - c % MC;
            chunk[s_finc[E] + s_bin[bin] + atomicAdd(&s_binf[bin], 1)] = make_int4(tid, c % MC, o + nf * MC, 0);
        }
        if (tid == E) off[E + 1] = s_inc[E];
    }
    __syncthreads();
    for (int p = tid; p < T * K; p += 1024) {
        const int e = expert(p);
        perm[s_off[e] + atomicAdd(&s_fill[e], 1)] = (p / K) * S + (p % K);
    }
    for (int t = tid; t < T; t += 1024) perm[s_off[E] + t] = t * S + K;
    for (int i = s_nch + tid; i < max_chunks; i += 1024) chunk[i] = make_int4(-1, 0, 0, 0);
}

// LDS row stride of the staged activations: 16 bytes of padding move each
// row 4 banks on, so the 16 rows one MFMA operand read touches (8 bytes
// each, 4 lane groups 8 bytes apart) fall on 64 distinct banks
template <int NB>
constexpr int arow() { return NB * QK_K + 16; }

__device__ __forceinline__ long pack_nib(uint2 v, int hi)
{
    const unsigned long long w = ((unsigned long long)v.y << 32) | v.x;
    return (long)((hi ? w >> 4 : w) & 0x0F0F0F0F0F0F0F0Full);
}

// ------------------------------------------------------- Q4_K x Q8_K tile --
// One wave: 16 weight rows (row lane%16, consecutive super-blocks) against
// the 16 staged activation rows; adds the fp32 results of pairs
// 4*(lane/16)+i for row lane%16 into r[i].  The lane's weight bytes of CH
// super-blocks are loaded into registers first (q4w_load, issued before the
// activations are staged), then consumed (q4w_mma).  Activation staging in
// LDS: aq[16][arow] int8, ad[NB][16] scales, as[NB*8][16] sub-block sums.
template <int CH>
struct Q4W {
    uint4 hdr[CH];
    uint2 qs[CH][4];
};

template <int CH>
__device__ __forceinline__ void q4w_load(Q4W<CH> &w, const uint8_t *wrow, int c0)
{
    const int q = lane_id() >> 4;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint8_t *blk = wrow + (size_t)(c0 + c) * Q4K_BYTES;
        w.hdr[c] = ld16(blk);
#pragma unroll
        for (int g = 0; g < 4; g++) w.qs[c][g] = ld8(blk + 16 + 32 * g + 8 * q);
    }
}

template <int CH>
__device__ __forceinline__ void q4w_opaque(Q4W<CH> &w)
{
#pragma unroll
    for (int c = 0; c < CH; c++) {
        asm volatile("" : "+v"(w.hdr[c].x), "+v"(w.hdr[c].y), "+v"(w.hdr[c].z), "+v"(w.hdr[c].w));
#pragma unroll
        for (int g = 0; g < 4; g++) asm volatile("" : "+v"(w.qs[c][g].x), "+v"(w.qs[c][g].y));
    }
}

template <int NB, int CH>
__device__ __forceinline__ void q4w_mma(const Q4W<CH> &w, int c0, const int8_t *aq, const float *ad,
                                        float (&r)[4])
{
    const int lane = lane_id(), lr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ib = c0 + c;
        // the 8 six-bit scales and mins of the block (src/q8k.c:22-30),
        // packed one per byte: sub-blocks 0-3 and 4-7
        const uint32_t y = w.hdr[c].y, z = w.hdr[c].z, x = w.hdr[c].w;
        const uint32_t sc_lo = y & 0x3F3F3F3Fu, m_lo = z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (x & 0x0F0F0F0Fu) | (((y >> 6) & 0x03030303u) << 4);
        const uint32_t m_hi = ((x >> 4) & 0x0F0F0F0Fu) | (((z >> 6) & 0x03030303u) << 4);
        int accs[4] = {0, 0, 0, 0};
        // min term: sum over the block of m(sub-block of k) * xq[k] -- an
        // MFMA against the mins broadcast over each sub-block, accumulated in
        // the matrix core across the block (exact: int32).  The K=64 form
        // takes two sub-blocks: bytes 0-7 of a lane's operands are its k of
        // sub-block 2t, bytes 8-15 its k of sub-block 2t+1, the same
        // assignment for both operands, so the sum runs over exactly those k.
        v4i accm = {0, 0, 0, 0};
        // per half block: four sub-block MFMAs back to back (independent),
        // the two min MFMAs, then the scale multiply-adds on their results,
        // so the matrix core stays busy while the VALU waits for the first
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
            long a[4];
            v4i p[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = 4 * hb + jj;
                a[jj] = *(const long *)(aq + lr * arow<NB>() + ib * QK_K + 32 * j + 8 * q);
                p[jj] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[jj], pack_nib(w.qs[c][j >> 1], j & 1),
                                                              v4i{0, 0, 0, 0}, 0, 0, 0);
            }
            // mins of sub-blocks 4hb .. 4hb+3 are bytes 0-3 of m_lo / m_hi;
            // each pair broadcast to all four bytes by one byte permute
            const uint32_t mw = hb ? m_hi : m_lo;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t m0 = __builtin_amdgcn_perm(0u, mw, 0x01010101u * (2 * t));
                const uint32_t m1 = __builtin_amdgcn_perm(0u, mw, 0x01010101u * (2 * t + 1));
                const v4i av = {(int)(uint32_t)a[2 * t], (int)(uint32_t)((unsigned long)a[2 * t] >> 32),
                                (int)(uint32_t)a[2 * t + 1], (int)(uint32_t)((unsigned long)a[2 * t + 1] >> 32)};
                accm = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, v4i{(int)m0, (int)m0, (int)m1, (int)m1}, accm, 0, 0,
                                                             0);
            }
            const uint32_t sw = hb ? sc_hi : sc_lo;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int sc = (int)((sw >> (8 * jj)) & 63);
                accs[0] = __mul24(sc, p[jj][0]) + accs[0];
                accs[1] = __mul24(sc, p[jj][1]) + accs[1];
                accs[2] = __mul24(sc, p[jj][2]) + accs[2];
                accs[3] = __mul24(sc, p[jj][3]) + accs[3];
            }
        }
        const float d = h2f(w.hdr[c].x & 0xffff), dmin = h2f(w.hdr[c].x >> 16);
        const float4 xd = *(const float4 *)(ad + ib * 16 + 4 * q);
        r[0] += (d * xd.x) * (float)accs[0] - (dmin * xd.x) * (float)accm[0];
        r[1] += (d * xd.y) * (float)accs[1] - (dmin * xd.y) * (float)accm[1];
        r[2] += (d * xd.z) * (float)accs[2] - (dmin * xd.z) * (float)accm[2];
        r[3] += (d * xd.w) * (float)accs[3] - (dmin * xd.w) * (float)accm[3];
    }
}

// The gate/up product for one or two M tiles (NT) sharing the weight rows,
// with the 6-bit sub-block scale folded into the weight operand instead of
// applied to each result: sc = 8*sh + sl with sl, sh in 0..7, so q*sl and
// q*sh (q <= 15) are int8 values <= 105, and
//     sum_j sc_j P_j = sum_k a_k (q_k sl_j) + 8 sum_k a_k (q_k sh_j)
// is two K = 64 MFMA chains over the block, exact in int32.  The scaled
// operands are built once per block (a packed 16-bit multiply per 4 bytes:
// no byte overflows into the next) and serve every tile; there are no
// per-result multiply-adds.  The min term dmin * sum_j m_j * xd * bsum_j
// takes a precomputed operand, amb[(c*2 + h)*64 + 16*k + p] = xd_c(pair p) *
// (sum of sub-block 4h + k of pair p's Q8_K block c): one fp32 MFMA pair per
// block (k = sub-block), accumulated apart from the integer sums.
//
// The weight bytes are loaded 16 per lane: lane (row lr, quarter q) holds
// the block header and nibble bytes [16q, 16q+16) and [64+16q, 64+16q+16)
// of the block's 128, so one load instruction reads 64 contiguous bytes of
// each of its 16 rows (8-byte pieces, 32 bytes per row per instruction, cap
// the HBM reads of this pattern at about 3.9 TB/s on this part; 16-byte
// pieces reach about 5.8).  The MFMA k-assignment follows the bytes: nibble
// byte j holds k = 64 (j / 32) + j % 32 (low nibble, sub-block 2 (j / 32))
// and k + 32 (high nibble, sub-block 2 (j / 32) + 1), so for step
// s = 2 half + hi a lane's 16 operand bytes are k = 128 half + 32 hi +
// 64 (q >> 1) + 16 (q & 1) + [0, 16), all of sub-block 4 half + 2 (q >> 1) +
// hi.  Its scale bytes are per lane, and the activation operand is one
// 16-byte LDS read at the same k.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t mul_bytes(uint32_t q4, uint32_t m16)
{
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q4) * __builtin_bit_cast(u16x2, m16));
}

template <int CH>
struct Q4V {
    uint4 hdr[CH], qa[CH], qb[CH];
};

template <int CH>
__device__ __forceinline__ void q4v_load(Q4V<CH> &w, const uint8_t *wrow, int c0)
{
    const int q = lane_id() >> 4;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint8_t *blk = wrow + (size_t)(c0 + c) * Q4K_BYTES;
        w.hdr[c] = ld16(blk);
        w.qa[c] = ld16(blk + 16 + 16 * q);
        w.qb[c] = ld16(blk + 80 + 16 * q);
    }
}

template <int CH>
__device__ __forceinline__ void q4v_opaque(Q4V<CH> &w)
{
#pragma unroll
    for (int c = 0; c < CH; c++) {
        asm volatile("" : "+v"(w.hdr[c].x), "+v"(w.hdr[c].y), "+v"(w.hdr[c].z), "+v"(w.hdr[c].w));
        asm volatile("" : "+v"(w.qa[c].x), "+v"(w.qa[c].y), "+v"(w.qa[c].z), "+v"(w.qa[c].w));
        asm volatile("" : "+v"(w.qb[c].x), "+v"(w.qb[c].y), "+v"(w.qb[c].z), "+v"(w.qb[c].w));
    }
}

template <int NB, int CH, int NT>
__device__ __forceinline__ void q4v_mma_sp(const Q4V<CH> &w, const int8_t *aqA, const float *adA, const float *ambA,
                                           float (&rA)[4], const int8_t *aqB, const float *adB, const float *ambB,
                                           float (&rB)[4])
{
    const int lane = lane_id(), lr = lane & 15, q = lane >> 4;
    // byte selectors broadcasting sub-block scale byte 2 (q >> 1) (+1) to
    // both 16-bit halves
    const uint32_t b0 = 2u * (uint32_t)(q >> 1);
    const uint32_t sel0 = (b0 * 0x00010001u) | 0x0C000C00u, sel1 = sel0 + 0x00010001u;
    const int koff = 64 * (q >> 1) + 16 * (q & 1);
    v4f rmA = {0.0f, 0.0f, 0.0f, 0.0f}, rmB = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const uint32_t y = w.hdr[c].y, z = w.hdr[c].z, x = w.hdr[c].w;
        const uint32_t sc_lo = y & 0x3F3F3F3Fu, m_lo = z & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (x & 0x0F0F0F0Fu) | (((y >> 6) & 0x03030303u) << 4);
        const uint32_t m_hi = ((x >> 4) & 0x0F0F0F0Fu) | (((z >> 6) & 0x03030303u) << 4);
        const float d = h2f(w.hdr[c].x & 0xffff), ndmin = -h2f(w.hdr[c].x >> 16);
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float bm = ndmin * (float)(((hh ? m_hi : m_lo) >> (8 * q)) & 63);
            rmA = __builtin_amdgcn_mfma_f32_16x16x4f32(ambA[(c * 2 + hh) * 64 + lane], bm, rmA, 0, 0, 0);
            if constexpr (NT == 2)
                rmB = __builtin_amdgcn_mfma_f32_16x16x4f32(ambB[(c * 2 + hh) * 64 + lane], bm, rmB, 0, 0, 0);
        }
        const uint32_t sl[2] = {sc_lo & 0x07070707u, sc_hi & 0x07070707u};
        const uint32_t sh[2] = {(sc_lo >> 3) & 0x07070707u, (sc_hi >> 3) & 0x07070707u};
        v4i a1A = {0, 0, 0, 0}, a2A = a1A, a1B = a1A, a2B = a1A;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int half = s >> 1, hi = s & 1;
            const uint4 src = half ? w.qb[c] : w.qa[c];
            const uint32_t n0 = hi ? (src.x >> 4) & 0x0F0F0F0Fu : src.x & 0x0F0F0F0Fu;
            const uint32_t n1 = hi ? (src.y >> 4) & 0x0F0F0F0Fu : src.y & 0x0F0F0F0Fu;
            const uint32_t n2 = hi ? (src.z >> 4) & 0x0F0F0F0Fu : src.z & 0x0F0F0F0Fu;
            const uint32_t n3 = hi ? (src.w >> 4) & 0x0F0F0F0Fu : src.w & 0x0F0F0F0Fu;
            const uint32_t ml = __builtin_amdgcn_perm(0u, sl[half], hi ? sel1 : sel0);
            const uint32_t mh = __builtin_amdgcn_perm(0u, sh[half], hi ? sel1 : sel0);
            const v4i B1 = {(int)mul_bytes(n0, ml), (int)mul_bytes(n1, ml), (int)mul_bytes(n2, ml),
                            (int)mul_bytes(n3, ml)};
            const v4i B2 = {(int)mul_bytes(n0, mh), (int)mul_bytes(n1, mh), (int)mul_bytes(n2, mh),
                            (int)mul_bytes(n3, mh)};
            const int ko = c * QK_K + 128 * half + 32 * hi + koff;
            {
                const v4i av = *(const v4i *)(aqA + lr * arow<NB>() + ko);
                a1A = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, B1, a1A, 0, 0, 0);
                a2A = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, B2, a2A, 0, 0, 0);
            }
            if constexpr (NT == 2) {
                const v4i av = *(const v4i *)(aqB + lr * arow<NB>() + ko);
                a1B = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, B1, a1B, 0, 0, 0);
                a2B = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, B2, a2B, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        {
            const float4 xd = *(const float4 *)(adA + c * 16 + 4 * q);
            rA[0] += (d * xd.x) * (float)(a1A[0] + 8 * a2A[0]);
            rA[1] += (d * xd.y) * (float)(a1A[1] + 8 * a2A[1]);
            rA[2] += (d * xd.z) * (float)(a1A[2] + 8 * a2A[2]);
            rA[3] += (d * xd.w) * (float)(a1A[3] + 8 * a2A[3]);
        }
        if constexpr (NT == 2) {
            const float4 xd = *(const float4 *)(adB + c * 16 + 4 * q);
            rB[0] += (d * xd.x) * (float)(a1B[0] + 8 * a2B[0]);
            rB[1] += (d * xd.y) * (float)(a1B[1] + 8 * a2B[1]);
            rB[2] += (d * xd.z) * (float)(a1B[2] + 8 * a2B[2]);
            rB[3] += (d * xd.w) * (float)(a1B[3] + 8 * a2B[3]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        rA[i] += rmA[i];
        if constexpr (NT == 2) rB[i] += rmB[i];
    }
}

// ------------------------------------------------------- Q6_K x Q8_K tile --
// Same contract for Q6_K rows (scales per 16 values, so each MFMA result
// must hold one 16-value group).  A lane (row lr, quarter q) loads 16-byte
// pieces: ql bytes [16q, 16q+16) of each half n (64 bytes per half), the qh
// bytes [16 (q & 1), +16) of each half, the 16 scales and d -- 64 contiguous
// bytes of each row per ql load instruction.  Per half, ql byte l' = 16q + i
// holds element 32 Q + l (l = l' % 32 = 16 (q & 1) + i) with Q = q >> 1 in
// its low nibble and Q = (q >> 1) + 2 in its high nibble, whose top two bits
// are bits 2Q, 2Q+1 of qh byte l (src/quants.c:56-69): so each lane holds
// four whole groups per block, g = 2n + hi, of scale 8n + 2Q + (q & 1).
// One v_mfma_i32_16x16x64_i8 per (group slot g, lane quarter t): every lane
// supplies its slot-g group as the weight operand, and only lanes q = t
// supply activations (the others read a zero row), so the result is the dot
// of quarter t's group alone, which its scale then multiplies.
template <int NB>
struct Q6V {
    uint4 ql[NB][2], qh[NB][2];                // [block][half]
    uint4 sc16[NB];
    uint32_t dbits[NB];
};

template <int NB>
__device__ __forceinline__ void q6v_load(Q6V<NB> &w, const uint8_t *wrow)
{
    const int q = lane_id() >> 4;
#pragma unroll
    for (int ib = 0; ib < NB; ib++) {
        const uint8_t *blk = wrow + (size_t)ib * Q6K_BYTES;
#pragma unroll
        for (int n = 0; n < 2; n++) {
            w.ql[ib][n] = ld16(blk + 64 * n + 16 * q);
            w.qh[ib][n] = ld16(blk + 128 + 32 * n + 16 * (q & 1));
        }
        w.sc16[ib] = ld16(blk + 192);
        w.dbits[ib] = ld2(blk + 208);
    }
}

// the four groups of each block as centred int8 operands
template <int NB>
struct Q6VB {
    v4i b[NB][4];
    uint4 sc16[NB];
    uint32_t dbits[NB];
};

template <int NB>
__device__ __forceinline__ void q6v_unpack(Q6VB<NB> &u, const Q6V<NB> &w)
{
    const int q = lane_id() >> 4;
    const uint32_t sh0 = 2u * (uint32_t)(q >> 1);  // 2Q of the low-nibble group
#pragma unroll
    for (int ib = 0; ib < NB; ib++) {
        u.sc16[ib] = w.sc16[ib];
        u.dbits[ib] = w.dbits[ib];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int n = g >> 1, hi = g & 1;
            const uint32_t L[4] = {w.ql[ib][n].x, w.ql[ib][n].y, w.ql[ib][n].z, w.ql[ib][n].w};
            const uint32_t H[4] = {w.qh[ib][n].x, w.qh[ib][n].y, w.qh[ib][n].z, w.qh[ib][n].w};
            const uint32_t sh = sh0 + 4u * hi;
            int v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo4 = hi ? (L[k] >> 4) & 0x0F0F0F0Fu : L[k] & 0x0F0F0F0Fu;
                v[k] = (int)q6_center(lo4 | (((H[k] >> sh) & 0x03030303u) << 4));
            }
            u.b[ib][g] = v4i{v[0], v[1], v[2], v[3]};
        }
    }
}

template <int NB>
__device__ __forceinline__ void q6v_opaque(Q6VB<NB> &u)
{
#pragma unroll
    for (int ib = 0; ib < NB; ib++)
#pragma unroll
        for (int g = 0; g < 4; g++) asm volatile("" : "+v"(u.b[ib][g]));
}

// abase[t] = this lane's activation row (pair lr) when q == t, else a zero
// row of the same length
template <int NB>
__device__ __forceinline__ void q6v_mma(const Q6VB<NB> &u, const int8_t *const (&abase)[4], const float *ad,
                                        float (&r)[4])
{
    const int q = lane_id() >> 4;
#pragma unroll
    for (int ib = 0; ib < NB; ib++) {
        int acc[4] = {0, 0, 0, 0};
        const uint32_t scw[4] = {u.sc16[ib].x, u.sc16[ib].y, u.sc16[ib].z, u.sc16[ib].w};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int n = g >> 1, hi = g & 1;
            // four MFMAs back to back, then their scale multiply-adds
            v4i p[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int Q = (t >> 1) + 2 * hi;
                const v4i a = *(const v4i *)(abase[t] + ib * QK_K + 128 * n + 32 * Q + 16 * (t & 1));
                p[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, u.b[ib][g], v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int si = 8 * n + 2 * ((t >> 1) + 2 * hi) + (t & 1);
                const int sc = (int)(int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 255);
                acc[0] = __mul24(sc, p[t][0]) + acc[0];
                acc[1] = __mul24(sc, p[t][1]) + acc[1];
                acc[2] = __mul24(sc, p[t][2]) + acc[2];
                acc[3] = __mul24(sc, p[t][3]) + acc[3];
            }
        }
        const float d = h2f(u.dbits[ib]);
        const float4 xd = *(const float4 *)(ad + ib * 16 + 4 * q);
        r[0] += d * xd.x * (float)acc[0];
        r[1] += d * xd.y * (float)acc[1];
        r[2] += d * xd.z * (float)acc[2];
        r[3] += d * xd.w * (float)acc[3];
    }
}

// --------------------------------------------- gate / up, rows resident --
// grid: (max MC-pair chunks) x (F / GR_ROWS); a workgroup = one chunk of up
// to 64 pairs of one bucket x 32 rows of h.  Wave w holds 8 of them: the gate
// rows in lanes 0-7 of its 16-row tile and the same rows of up in lanes
// 8-15, so silu(g) * u pairs lanes lr and lr + 8 of one result.  A wave
// loads its 16 rows whole (KH super-blocks = 1152 contiguous bytes per row
// for n_embd 2048) into registers at once -- HBM sees each row read as one
// burst -- and keeps
// them while the chunk's pairs stream past in M tiles of 16: the tile's
// Q8_K(x) rows go global -> LDS by DMA (no registers), double buffered, the
// next tile's DMA in flight during the current tile's MFMAs.  n_embd 4096
// runs as four passes of 4 super-blocks.
constexpr int GR_ROWS = 32;

// stage the Q8_K rows (super-blocks [kb0, kb0 + KH)) and scales of the M
// tile's 16 tokens tok[0..15] into aq[16][arow<KH>()] / ad[KH][16].  The
// DMAs are unconditional (an absent pair carries token 0, whose staged row
// feeds only results that are never stored), so no branch separates them
// and each wave's token reads batch into one LDS round trip.
template <int KH>
__device__ __forceinline__ void stage_dma(const int *tok, int nbe, int kb0, const int8_t *xq, const float *xd,
                                          const float *xmb, int8_t *aq, float *ad, float *amb)
{
    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6);
    const size_t xrow = (size_t)nbe * QK_K;
    if constexpr (KH >= 4) {
        constexpr int PER = KH / 4;            // 1 KB pieces per staged row
#pragma unroll
        for (int i = wv; i < PB * PER; i += 4) {
            const int p = i / PER, piece = i % PER;
            __builtin_amdgcn_global_load_lds(
                (const QMAG_GLOBAL void *)(xq + (size_t)tok[p] * xrow + (size_t)kb0 * QK_K + piece * 1024 + lane * 16),
                (__attribute__((address_space(3))) void *)(aq + p * arow<KH>() + piece * 1024), 16, 0, 0);
        }
    } else {
        constexpr int PER = KH;                // 256 B pieces, one dword per lane
#pragma unroll
        for (int i = wv; i < PB * PER; i += 4) {
            const int p = i / PER, piece = i % PER;
            __builtin_amdgcn_global_load_lds(
                (const QMAG_GLOBAL void *)(xq + (size_t)tok[p] * xrow + (size_t)kb0 * QK_K + piece * 256 + lane * 4),
                (__attribute__((address_space(3))) void *)(aq + p * arow<KH>() + piece * 256), 4, 0, 0);
        }
    }
    // scales, ad[c][p]: thread t -> block c = t / 16, pair p = t % 16; the
    // lanes past the KH * 16 scales stay masked (their DMA slot would lie
    // beyond ad)
    if (wv * 64 < PB * KH) {
        const int t = wv * 64 + lane, c = t / PB, p = t % PB;
        if (t < PB * KH)
            __builtin_amdgcn_global_load_lds((const QMAG_GLOBAL void *)(xd + (size_t)tok[p] * nbe + kb0 + c),
                                             (__attribute__((address_space(3))) void *)(ad + wv * 64), 4, 0, 0);
    }
    // min-term operands, amb[(c*2 + h)*64 + 16*k + p] = xmb of pair p,
    // block c, sub-block 4h + k: one 256-byte DMA per (block, half), each
    // lane gathering its pair's value
#pragma unroll
    for (int i = wv; i < 2 * KH; i += 4) {
        const int c = i >> 1, hh = i & 1;
        __builtin_amdgcn_global_load_lds(
            (const QMAG_GLOBAL void *)(xmb + (size_t)tok[lane & 15] * (nbe * 8) + (kb0 + c) * 8 + 4 * hh + (lane >> 4)),
            (__attribute__((address_space(3))) void *)(amb + i * 64), 4, 0, 0);
    }
}

template <int NBE>
__global__ __launch_bounds__(256, 2) void gateup_rows_kernel(
    const uint8_t *__restrict__ gate_exps, const uint8_t *__restrict__ up_exps,
    const uint8_t *__restrict__ gate_sh, const uint8_t *__restrict__ up_sh, int E, int S, int F,
    const int4 *__restrict__ chunk, const int *__restrict__ perm,
    const int8_t *__restrict__ xq, const float *__restrict__ xd, const float *__restrict__ xmb,
    float *__restrict__ h)
{
    constexpr int KH = NBE <= 8 ? NBE : 4;     // super-blocks held per pass (n_embd 4096: 4 passes of 4)
    constexpr int NPASS = NBE / KH;
    // the two buffers are separate LDS objects: the compiler then knows
    // that reading one need not wait for the DMA into the other
    __shared__ __align__(16) int8_t s_aq0[PB * arow<KH>()], s_aq1[PB * arow<KH>()];
    __shared__ __align__(16) float s_ad0[KH * PB], s_ad1[KH * PB];
    __shared__ __align__(16) float s_mb0[KH * 128], s_mb1[KH * 128];
    __shared__ int s_pair[MC], s_tok[MC];
    const int rchunks = F / GR_ROWS;
    const int u = (int)blockIdx.x / rchunks, rc = (int)blockIdx.x % rchunks;
    const int4 ck = chunk[u];
    if (ck.x < 0) return;
    const int e = ck.x, npair = ck.y, mtn = (npair + PB - 1) / PB;
    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6);
    const int lr = lane & 15, q = lane >> 4;
    // wave w holds rows row0 .. row0 + 7 of h: lanes lr < 8 the gate rows,
    // lanes 8-15 the same rows of up
    const int row0 = rc * GR_ROWS + 8 * wv;
    constexpr size_t rowb = (size_t)NBE * Q4K_BYTES;
    const uint8_t *wrow = (lr < 8 ? (e < E ? gate_exps + (size_t)e * F * rowb : gate_sh)
                                  : (e < E ? up_exps + (size_t)e * F * rowb : up_sh)) +
                          (size_t)(row0 + (lr & 7)) * rowb;
    // the weight rows go out first; the pair ids follow as scalar loads
    // (their own counter), so waiting for them leaves the weights in flight
    Q4V<KH> w;
    q4v_load(w, wrow, 0);
    {
        const int wvu = __builtin_amdgcn_readfirstlane(wv);
        const int base = ck.z + 16 * wvu, last = ck.z + npair - 1;
        int v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = perm[min(base + k, last)];
        int mine = -1;
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (lane == k && 16 * wvu + k < npair) mine = v[k];
        if (lane < 16) {
            s_pair[16 * wvu + lane] = mine;
            s_tok[16 * wvu + lane] = mine >= 0 ? mine / S : 0;
        }
    }
    __syncthreads();

    float r[MC / PB][4];
#pragma unroll
    for (int m = 0; m < MC / PB; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) r[m][i] = 0.0f;
#pragma unroll
    for (int ps = 0; ps < NPASS; ps++) {
        if (ps > 0) q4v_load(w, wrow, ps * KH);
        // tiles in pairs, both buffers staged at once: a pair shares the
        // scaled weight operands
        stage_dma<KH>(s_tok, NBE, ps * KH, xq, xd, xmb, s_aq0, s_ad0, s_mb0);
        if (mtn > 1) stage_dma<KH>(s_tok + PB, NBE, ps * KH, xq, xd, xmb, s_aq1, s_ad1, s_mb1);
#pragma unroll
        for (int mp = 0; mp < MC / PB / 2; mp++) {
            if (2 * mp < mtn) {                // workgroup-uniform
                __syncthreads();               // the pair's DMA has landed (every wave's)
                q4v_opaque(w);
                if (2 * mp + 1 < mtn)
                    q4v_mma_sp<KH, KH, 2>(w, s_aq0, s_ad0, s_mb0, r[2 * mp], s_aq1, s_ad1, s_mb1, r[2 * mp + 1]);
                else
                    q4v_mma_sp<KH, KH, 1>(w, s_aq0, s_ad0, s_mb0, r[2 * mp], s_aq1, s_ad1, s_mb1, r[2 * mp + 1]);
                if (2 * mp + 2 < mtn) {
                    __syncthreads();           // both buffers read: stage the next pair
                    stage_dma<KH>(s_tok + PB * (2 * mp + 2), NBE, ps * KH, xq, xd, xmb, s_aq0, s_ad0, s_mb0);
                    if (2 * mp + 3 < mtn)
                        stage_dma<KH>(s_tok + PB * (2 * mp + 3), NBE, ps * KH, xq, xd, xmb, s_aq1, s_ad1, s_mb1);
                }
            }
        }
        if (ps + 1 < NPASS) __syncthreads();   // the buffers are free for the next pass
    }
    // h = silu(g) * u: gate lane lr and up lane lr + 8 of one result (row_ror:8)
#pragma unroll
    for (int m = 0; m < MC / PB; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float g = r[m][i], uu = dpp_f<0x128>(r[m][i]);
            const int pr = s_pair[PB * m + 4 * q + i];
            if (lr < 8 && m < mtn && pr >= 0) h[(size_t)pr * F + row0 + lr] = (g / (1.0f + expf(-g))) * uu;
        }
}

// ----------------------------------------------------------------- down --
// grid: (max MC-pair chunks) x (N / 64); a workgroup = one chunk of up to 64
// pairs of one bucket x 64 rows, 16 per wave.  Each wave loads its rows
// whole (NBF super-blocks, 420 contiguous bytes per Q6_K row for n_ff 512)
// into registers, the chunk's Q8_K(h) rows are staged in LDS at once by
// DMA, and y[pair][row] = row . Q8_K(h[pair]) runs M tile by M tile.
constexpr int DN_ROWS = 64;

// stage rows[0 .. 16*mtn) of Q8_K(h) (NB super-blocks each) into
// aq[p][arow<NB>()] and their scales into ad[p / 16][block][p % 16]: 16-byte
// loads into registers (Staged::load), written to LDS once they arrive
// (Staged::store); per-dword DMAs into LDS, four times the instructions,
// made the staging of a 64-pair chunk cost about 4 us more than that of a
// 16-pair one.  Every pair slot has a valid row (absent pairs repeat the
// chunk's first).
template <int NB>
struct Staged {
    static constexpr int PPR = NB * QK_K / 16;     // 16-byte pieces per row
    static constexpr int IT = MC * PPR / 256;      // pieces per thread, full chunk
    uint4 v[IT];
    float sv;

    __device__ __forceinline__ void load(const int *rows, int mtn, const int8_t *hq, const float *hd)
    {
        const int t = (int)threadIdx.x, n = PB * mtn * PPR;
#pragma unroll
        for (int k = 0; k < IT; k++) {
            const int i = t + 256 * k, p = i / PPR, pc = i % PPR;
            if (k * 256 < n) v[k] = ld16((const uint8_t *)hq + (size_t)rows[p] * (NB * QK_K) + pc * 16);
        }
        sv = 0.0f;
        if (t < PB * mtn * NB) {
            const int mt = t / (NB * PB), ib = (t / PB) % NB, p = PB * mt + t % PB;
            sv = ldg(hd + (size_t)rows[p] * NB + ib);
        }
    }
    __device__ __forceinline__ void store(int mtn, int8_t *aq, float *ad) const
    {
        const int t = (int)threadIdx.x, n = PB * mtn * PPR;
#pragma unroll
        for (int k = 0; k < IT; k++) {
            const int i = t + 256 * k, p = i / PPR, pc = i % PPR;
            if (k * 256 < n) *(uint4 *)(aq + p * arow<NB>() + pc * 16) = v[k];
        }
        if (t < PB * mtn * NB) ad[t] = sv;
    }
};

#ifndef QMAG_DN_WPC
#define QMAG_DN_WPC 2
#endif
template <int NBF>
__global__ __launch_bounds__(256, QMAG_DN_WPC) void down_rows_kernel(
    const uint8_t *__restrict__ down_exps, int t_down, const uint8_t *__restrict__ down_sh, int t_down_sh,
    int E, int N, const int4 *__restrict__ chunk, const int *__restrict__ perm, const int8_t *__restrict__ hq,
    const float *__restrict__ hd, float *__restrict__ y)
{
    __shared__ __align__(16) int8_t s_aq[MC * arow<NBF>()];
    __shared__ __align__(16) int8_t s_zero[arow<NBF>()];     // the Q6_K MFMAs' inactive activation lanes
    __shared__ __align__(16) float s_ad[MC * NBF];
    __shared__ int s_pair[MC], s_row[MC];
    const int rblocks = N / DN_ROWS;
    const int u = (int)blockIdx.x / rblocks, rb = (int)blockIdx.x % rblocks;
    const int4 ck = chunk[u];
    if (ck.x < 0) return;
    const int e = ck.x, npair = ck.y, mtn = (npair + PB - 1) / PB;
    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6), lr = lane & 15, q = lane >> 4;
    const int row = rb * DN_ROWS + wv * 16 + lr;
    const int td = e < E ? t_down : t_down_sh;
    const size_t rowb = (size_t)NBF * (td == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES);
    const uint8_t *D = (e < E ? down_exps + (size_t)e * N * rowb : down_sh) + row * rowb;
    float r[MC / PB][4];
#pragma unroll
    for (int m = 0; m < MC / PB; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) r[m][i] = 0.0f;
    // the pair ids go out first, one vector load per pair (rows of absent
    // pairs repeat the first pair's), then the wave's 16 weight rows, then,
    // once the ids are in LDS, the chunk's Q8_K(h) rows: each wait leaves
    // the later requests in flight (the load counter drains in issue order).
    // Requesting the ids after the rows made them wait behind the rows
    // (67.0 against 64.9 us per layer).
    const int idx = 16 * wv + lane;
    int mine = -1, first = 0;
    auto ids_load = [&]() __attribute__((always_inline)) {
        if (lane < 16 && idx < npair) mine = perm[ck.z + idx];
        first = perm[ck.z];
        asm volatile("" ::: "memory");
    };
    auto ids_store = [&]() __attribute__((always_inline)) {
        if (lane < 16) {
            s_pair[idx] = mine;
            s_row[idx] = mine >= 0 ? mine : first;
        }
        for (int i = (int)threadIdx.x; i < arow<NBF>() / 16; i += 256) ((uint4 *)s_zero)[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
    };
    Staged<NBF> stg;
    if (td == QMAG_TYPE_Q6_K) {
        Q6VB<NBF> ub;
        {
            Q6V<NBF> w;
            ids_load();
            q6v_load(w, D);
            ids_store();
            stg.load(s_row, mtn, hq, hd);
            stg.store(mtn, s_aq, s_ad);
            q6v_unpack(ub, w);
        }
        __syncthreads();                       // every wave's staged rows are in LDS
        const int8_t *arow_m = s_aq + lr * arow<NBF>();
#pragma unroll
        for (int m = 0; m < MC / PB; m++)
            if (m < mtn) {
                q6v_opaque(ub);
                const int8_t *const abase[4] = {q == 0 ? arow_m : s_zero, q == 1 ? arow_m : s_zero,
                                                q == 2 ? arow_m : s_zero, q == 3 ? arow_m : s_zero};
                q6v_mma<NBF>(ub, abase, s_ad + m * NBF * PB, r[m]);
                arow_m += PB * arow<NBF>();
            }
    } else {
        Q4W<NBF> w;
        ids_load();
        q4w_load(w, D, 0);
        ids_store();
        stg.load(s_row, mtn, hq, hd);
        stg.store(mtn, s_aq, s_ad);
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MC / PB; m++)
            if (m < mtn) {
                q4w_opaque(w);
                q4w_mma<NBF, NBF>(w, 0, s_aq + PB * m * arow<NBF>(), s_ad + m * NBF * PB, r[m]);
            }
    }
#pragma unroll
    for (int m = 0; m < MC / PB; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pr = s_pair[PB * m + 4 * q + i];
            if (m < mtn && pr >= 0) y[(size_t)pr * N + row] = r[m][i];
        }
}

// -------------------------------------------------------------- combine --
// One thread per 4 consecutive outputs of one token: the 9 slot rows (and the
// residual) are requested as float4 before any is used; each element is
// summed in the reference's order with unfused multiply and add.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y, const float *__restrict__ w,
                                                      const float *__restrict__ gs, int T, int K, int N,
                                                      const float *__restrict__ resid, float *__restrict__ out)
{
    const size_t i = 4 * ((size_t)blockIdx.x * 256 + threadIdx.x);   // N % 4 == 0
    if (i >= (size_t)T * N) return;
    const int t = (int)(i / N), r = (int)(i % N), S = K + 1;
    float4 v[9];                                                       // K <= 8
#pragma unroll
    for (int k = 0; k < 9; k++) v[k] = *(const float4 *)(y + ((size_t)t * S + min(k, K)) * N + r);
    const float4 rs = resid ? *(const float4 *)(resid + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (k < K) {
            const float wk = w[t * K + k];
            acc.x = __fadd_rn(acc.x, __fmul_rn(wk, v[k].x));
            acc.y = __fadd_rn(acc.y, __fmul_rn(wk, v[k].y));
            acc.z = __fadd_rn(acc.z, __fmul_rn(wk, v[k].z));
            acc.w = __fadd_rn(acc.w, __fmul_rn(wk, v[k].w));
        }
    }
    const float g = gs[t];
    const float4 sh = v[8];                    // row min(8, K) = K: the shared slot
    acc.x = __fadd_rn(acc.x, __fmul_rn(g, sh.x));
    acc.y = __fadd_rn(acc.y, __fmul_rn(g, sh.y));
    acc.z = __fadd_rn(acc.z, __fmul_rn(g, sh.z));
    acc.w = __fadd_rn(acc.w, __fmul_rn(g, sh.w));
    if (resid) {
        acc.x = __fadd_rn(acc.x, rs.x);
        acc.y = __fadd_rn(acc.y, rs.y);
        acc.z = __fadd_rn(acc.z, rs.z);
        acc.w = __fadd_rn(acc.w, rs.w);
    }
    *(float4 *)(out + i) = acc;
}

// ------------------------------------------------------------------ host --
int launch_router_mfma(const qmag_moe_layer *L, const float *x, int T, float *part, hipStream_t s)
{
    const int N = L->n_embd, E = L->n_expert;
    if (N % 256) return fail(QMAG_ERR_ARG, "router: n_embd=%d", N);
    hipLaunchKernelGGL(router_tile_kernel, dim3((T + RT_ROWS - 1) / RT_ROWS, (E + RT_ROWS - 1) / RT_ROWS, N / 256),
                       dim3(512), 0, s, L->gate_inp, x, N, E, T, part);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

template <int NBE>
static void launch_gu(const qmag_moe_layer *L, int S, int max_chunks, const int4 *chunk,
                      const int *perm, const int8_t *xq, const float *xd, const float *xmb, float *h, hipStream_t s)
{
    hipLaunchKernelGGL(gateup_rows_kernel<NBE>, dim3(max_chunks * (L->n_ff / GR_ROWS)), dim3(256), 0, s,
                       (const uint8_t *)L->gate_exps, (const uint8_t *)L->up_exps, (const uint8_t *)L->gate_shexp,
                       (const uint8_t *)L->up_shexp, L->n_expert, S, L->n_ff, chunk, perm, xq, xd, xmb, h);
}

template <int NBF>
static void launch_dn(const qmag_moe_layer *L, int max_chunks, const int4 *chunk, const int *perm, const int8_t *hq,
                      const float *hd, float *y, hipStream_t s)
{
    hipLaunchKernelGGL(down_rows_kernel<NBF>, dim3(max_chunks * (L->n_embd / DN_ROWS)), dim3(256), 0, s,
                       (const uint8_t *)L->down_exps, L->t_down_exps, (const uint8_t *)L->down_shexp,
                       L->t_down_shexp, L->n_expert, L->n_embd, chunk, perm, hq, hd, y);
}

int moe_grouped(const qmag_moe_layer *L, int T, const int *sel, const float *w, const float *gs,
                const int8_t *xq, const float *xd, const float *xmb, float *h, int8_t *hq, float *hd,
                int16_t *hs, const float *resid, float *out, hipStream_t s)
{
    const int N = L->n_embd, F = L->n_ff, E = L->n_expert, K = L->n_used, S = K + 1;
    int st;
    // upper bound of the MC-pair chunks: sum ceil(n_e / MC) <= T*K/MC + E,
    // plus the shared bucket
    const int max_chunks = (T * K + MC - 1) / MC + E + (T + MC - 1) / MC;
    // int4 chunk descriptors first (16-byte aligned), then the int tables
    int4 *chunk = (int4 *)workspace(WS_GRP, sizeof(int4) * (size_t)max_chunks +
                                                sizeof(int) * ((size_t)2 * (E + 2) + (size_t)T * S),
                                    &st);
    if (st) return st;
    int *grp = (int *)(chunk + max_chunks), *perm = grp + 2 * (E + 2);
    float *y = (float *)workspace(WS_Y, sizeof(float) * (size_t)T * S * N, &st);
    if (st) return st;

    prof_begin(PROF_GROUP, s);
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, sel, T, K, E, grp, chunk, max_chunks, perm);
    prof_end(PROF_GROUP, s);
    prof_begin(PROF_GATEUP, s);
    switch (N / QK_K) {
    case 1: launch_gu<1>(L, S, max_chunks, chunk, perm, xq, xd, xmb, h, s); break;
    case 2: launch_gu<2>(L, S, max_chunks, chunk, perm, xq, xd, xmb, h, s); break;
    case 4: launch_gu<4>(L, S, max_chunks, chunk, perm, xq, xd, xmb, h, s); break;
    case 8: launch_gu<8>(L, S, max_chunks, chunk, perm, xq, xd, xmb, h, s); break;
    default: launch_gu<16>(L, S, max_chunks, chunk, perm, xq, xd, xmb, h, s); break;
    }
    prof_end(PROF_GATEUP, s);
    prof_begin(PROF_HQUANT, s);
    st = launch_q8k_quant(h, T * S * (F / QK_K), hq, hd, hs, s);
    prof_end(PROF_HQUANT, s);
    if (st) return st;
    prof_begin(PROF_DOWN, s);
    switch (F / QK_K) {
    case 1: launch_dn<1>(L, max_chunks, chunk, perm, hq, hd, y, s); break;
    case 2: launch_dn<2>(L, max_chunks, chunk, perm, hq, hd, y, s); break;
    default: launch_dn<4>(L, max_chunks, chunk, perm, hq, hd, y, s); break;
    }
    prof_end(PROF_DOWN, s);
    prof_begin(PROF_COMBINE, s);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)(((size_t)T * N / 4 + 255) / 256)), dim3(256), 0, s, y, w, gs,
                       T, K, N, resid, out);
    prof_end(PROF_COMBINE, s);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

}  // namespace qmag
