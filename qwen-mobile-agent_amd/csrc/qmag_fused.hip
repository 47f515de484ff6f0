// qmag_fused.hip -- one persistent, cooperatively launched kernel that runs
// the whole qwen35moe MoE FFN decode (batch 1) for a run of layers
// (src/nn.c:509-707 per layer, residual add of nn.c:2252 between layers).
//
// Shapes are the engine's compile-time ones (src/qma.h:28, 57-60): hidden
// 2048, expert ff 512, up to 256 experts, top-k <= 8, plus the shared
// expert.  512 workgroups x 4 waves = 2048 waves, two workgroups per CU;
// wave w owns down row w of every layer.
//
// Data flow of one layer, five hand-offs between workgroups:
//   1  x_l rows             down waves of layer l-1  -> the router workgroups
//   2  router logits        router waves              -> the collector (wave 0 of wg 0)
//   3  selection record     collector: top-k ids, renormalised weights and the
//                           shared-expert gate; with it Q8_K(x_l)  -> every workgroup
//   4  h = silu(g)*u        gate/up waves             -> 18 quantiser waves
//   5  Q8_K(h) blocks       quantiser waves           -> every workgroup
// No counters or cross-workgroup barriers exist.  Every published value is
// one 64-bit word {32 data bits, 32-bit tag}, written with a single-copy-
// atomic device-scope store; the tag is epoch*256 + layer + 1 (the epoch
// counts launches).  A consumer reads words with device-scope atomic loads
// and accepts a word only when it carries the current tag, so data is its own
// ready flag and no read-modify-write or cache maintenance is needed.  Bulk
// data is read once its sentinel words are valid (every word is still
// validated), so waiting workgroups poll a handful of words, not the bulk.
// Values all 512 workgroups read are written in 8 replicas 64 KB apart.
//
// Weight bytes move as early as they are known: the router row (straight
// into LDS) at layer start, and right after the selection record the gate/up
// row pairs and down-row slices of the routed and shared experts, all issued
// before any is consumed, so the down bytes stream while gate/up computes.
// Every poll is bounded: an exhausted waiter raises an abort flag that all
// pollers check, so the grid always drains; qmag_sync() reports it.
#include <string.h>

#include "qmag_internal.h"

namespace qmag {
namespace fused {

constexpr int N = 2048, F = 512;
constexpr int NBE = N / QK_K, NBF = F / QK_K;     // 8, 2
constexpr int SMAX = 9;                           // 8 routed + shared
constexpr int WGS = 512, WAVES = WGS * 4;
constexpr int MAX_RP = (SMAX * F + WAVES - 1) / WAVES;   // gate/up row pairs per wave: 3
constexpr long SPIN_LIMIT = 1L << 22;

// Q8_K(x): 512 packed xq words, 8 block scales, 128 group sums
constexpr int XQ_WORDS = N / 4 + NBE + N / 16;    // 648
constexpr int XQ_D = N / 4, XQ_S = N / 4 + NBE;
// selection record: 8 expert ids, 8 weights, the shared-expert gate
constexpr int SEL_WORDS = 17;
// Q8_K(h): per 256-value block 64 packed words, the scale (the block's
// sentinel), 16 group sums; block k is quantised by wave 1 of workgroup
// QWG0 + k*QWG_STEP (odd step: spread over the 8 XCDs, which take
// workgroups round-robin)
constexpr int HQ_BLK = 64 + 1 + 16;
constexpr int HQ_PER_THREAD = (SMAX * NBF * HQ_BLK + 255) / 256;   // 6
constexpr int QWG0 = 3, QWG_STEP = 29;
static_assert(QWG0 + QWG_STEP * (SMAX * NBF - 1) < WGS, "quantiser workgroups out of range");

// The selection record, polled by every workgroup, is written in REP
// replicas 4 KB apart (workgroup b polls replica b % REP).  The bulk values
// every workgroup reads (Q8_K(x), Q8_K(h)) get one buffer per layer slot, so
// a cache line read in one layer is not looked up again until the slot comes
// round on the next token.
constexpr int REP = 8, REP_WORDS = 512;
constexpr int MAXL = 64;                          // layer slots (layer l uses l % MAXL)
constexpr int XQ_PAD = 656, HQ_PAD = 1472;        // words, multiples of 16 (128 B)
struct Tagged {
    unsigned long long sel[REP][REP_WORDS];
    unsigned long long xq[MAXL][XQ_PAD];
    unsigned long long hq[MAXL][HQ_PAD];
    unsigned long long x[N];             // x_l, l >= 1 (read by the router workgroups)
    unsigned long long logits[256];      // read by the collector
    unsigned long long h[SMAX * F];      // read by the quantiser waves
};
static_assert(XQ_PAD >= XQ_WORDS && HQ_PAD >= SMAX * NBF * HQ_BLK, "slot sizes");

__device__ __forceinline__ unsigned long long ld64(const unsigned long long *p)
{
    return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(unsigned long long *p, uint32_t v, uint32_t seq)
{
    __hip_atomic_store(p, ((unsigned long long)seq << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// p points into replica 0; the word is written in every replica
__device__ __forceinline__ void st64r(unsigned long long *p, uint32_t v, uint32_t seq)
{
#pragma nounroll
    for (int r = 0; r < REP; r++) st64(p + r * REP_WORDS, v, seq);
}
// wait until all of this wave's outstanding memory operations completed
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ int ld_flag(const int *p)
{
    return __hip_atomic_load(const_cast<int *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave reads CNT tagged words per lane, p[idx(k)] (idx < 0: no word),
// until every word carries `seq`; the low halves land in val[].  All loads of
// a round are issued together, and a retry reloads only the stale words.
template <int CNT, typename Idx>
__device__ bool poll(const unsigned long long *p, Idx idx, uint32_t seq, uint32_t (&val)[CNT],
                     int *abort_flag)
{
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < CNT; k++)
        if (idx(k) >= 0) pending |= 1u << k;
    for (long it = 0; it < SPIN_LIMIT; it++) {
#pragma unroll
        for (int k = 0; k < CNT; k++) {
            if (pending & (1u << k)) {
                const unsigned long long w = ld64(p + idx(k));
                if ((uint32_t)(w >> 32) == seq) {
                    val[k] = (uint32_t)w;
                    pending &= ~(1u << k);
                }
            }
        }
        if (__all(pending == 0)) return true;
        if ((it & 31) == 31 && ld_flag(abort_flag) != 0) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// Bulk read after the sentinels were seen: one pass of ordinary (L2-cached)
// loads, so the 64 workgroups of an XCD share one fetch from memory; words
// with a stale tag (a stale cache line) are then polled device-coherently.
template <int CNT, typename Idx>
__device__ bool read_bulk(const unsigned long long *p, Idx idx, uint32_t seq, uint32_t (&val)[CNT],
                          int *abort_flag)
{
    bool fresh = true;
#pragma unroll
    for (int k = 0; k < CNT; k++) {
        if (idx(k) >= 0) {
            const unsigned long long w = p[idx(k)];
            val[k] = (uint32_t)w;
            fresh = fresh && (uint32_t)(w >> 32) == seq;
        }
    }
    if (__all(fresh)) return true;
    return poll<CNT>(p, idx, seq, val, abort_flag);
}

// workgroup-wide AND of one flag per wave (slot: a distinct LDS row per call site)
__device__ __forceinline__ bool wg_all(bool ok, int (*s_vote)[4], int slot)
{
    if (lane_id() == 0) s_vote[slot][threadIdx.x >> 6] = ok ? 1 : 0;
    __syncthreads();
    return (s_vote[slot][0] & s_vote[slot][1] & s_vote[slot][2] & s_vote[slot][3]) != 0;
}

// ---- down-projection task (row r of one expert, 8 tasks per 512-wide row)
template <int TD>
struct DRaw;
template <>
struct DRaw<QMAG_TYPE_Q6_K> {
    Q6Raw r;
};
template <>
struct DRaw<QMAG_TYPE_Q4_K> {
    uint4 hdr, q0, q1;
};

template <int TD>
__device__ __forceinline__ void d_zero(DRaw<TD> &d)
{
    d = DRaw<TD>{};
}

template <int TD>
__device__ __forceinline__ void d_load(DRaw<TD> &d, const uint8_t *slab, int row, int q)
{
    if constexpr (TD == QMAG_TYPE_Q6_K) {
        const uint8_t *blk = slab + ((size_t)row * NBF + (q >> 2)) * Q6K_BYTES;
        q6_load_raw(d.r, blk, (q >> 1) & 1, q & 1);
    } else {
        const uint8_t *blk = slab + ((size_t)row * NBF + (q >> 2)) * Q4K_BYTES;
        d.hdr = ld16(blk);
        d.q0 = ld16(blk + 16 + 32 * (q & 3));
        d.q1 = ld16(blk + 32 + 32 * (q & 3));
    }
}

// fp32 contribution of task q against one slot's Q8_K(h) held in LDS
template <int TD>
__device__ __forceinline__ float d_dot(const DRaw<TD> &d, const uint32_t *hq, const float *hd,
                                       const int16_t *hs, int q)
{
    const int ib = q >> 2, sub = q & 3;
    if constexpr (TD == QMAG_TYPE_Q6_K) {
        const int n = sub >> 1, l16 = sub & 1;
        Q6Act a;
#pragma unroll
        for (int Q = 0; Q < 4; Q++) {
            const uint4 w = *(const uint4 *)(hq + (ib * QK_K + 128 * n + 32 * Q + 16 * l16) / 4);
            a.x[4 * Q + 0] = w.x;
            a.x[4 * Q + 1] = w.y;
            a.x[4 * Q + 2] = w.z;
            a.x[4 * Q + 3] = w.w;
        }
        const int isum = group_sum_i<4>(q6_int_dot(d.r, a, l16));
        return sub == 0 ? h2f(d.r.d) * hd[ib] * (float)isum : 0.0f;
    } else {
        Q4Act a;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 w = *(const uint4 *)(hq + (ib * QK_K + 64 * sub) / 4 + 4 * k);
            a.x[4 * k + 0] = w.x;
            a.x[4 * k + 1] = w.y;
            a.x[4 * k + 2] = w.z;
            a.x[4 * k + 3] = w.w;
        }
        a.xd = hd[ib];
        const int16_t *s = hs + ib * 16 + 4 * sub;
        a.sx0 = (float)(s[0] + s[1]);
        a.sx1 = (float)(s[2] + s[3]);
        return q4_task(d.hdr, d.q0, d.q1, a, sub);
    }
}

// softmax over E <= 256 logits (4 per lane of one wave), top-K with strict
// > and the lowest index winning ties (nn.c:525-536).  Lane k < K receives
// pick k: its expert id and its weight renormalised over the K picks (the
// sum taken in pick order, as the reference does).
__device__ void route_topk(const float (&lg)[4], int E, int K, int &my_sel, float &my_w)
{
    const int lane = lane_id();
    float p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) mx = fmaxf(mx, lg[j]);
    mx = group_max<64>(mx);
    float se = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        p[j] = lane + 64 * j < E ? expf(lg[j] - mx) : 0.0f;
        se += p[j];
    }
    se = group_sum<64>(se);
#pragma unroll
    for (int j = 0; j < 4; j++) p[j] = lane + 64 * j < E ? p[j] / se : -1.0f;
    for (int k = 0; k < K; k++) {
        const float m = group_max<64>(fmaxf(fmaxf(p[0], p[1]), fmaxf(p[2], p[3])));
        int cand = 1 << 30;
#pragma unroll
        for (int j = 3; j >= 0; j--)
            if (p[j] == m) cand = lane + 64 * j;
        int s = group_min_i<64>(cand);
        s = s < E ? s : 0;          // NaN logits match nothing: keep the index in range
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (lane + 64 * j == s) p[j] = -1.0f;
        if (lane == k) {
            my_sel = s;
            my_w = m;
        }
    }
    float ws = 0.0f;
    for (int k = 0; k < K; k++) ws += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_w), k));
    my_w = my_w / ws;
}

template <int TD>
__global__ __launch_bounds__(256, 2) void moe_decode_kernel(const qmag_moe_layer *__restrict__ layers,
                                                            int n_layer, float *x, float *out,
                                                            Tagged *tg, float *g_logits, float *g_h,
                                                            int *g_sel, float *g_w, float *g_gs,
                                                            int *abort_flag, unsigned epoch,
                                                            unsigned long long *trace)
{
    __shared__ uint4 s_xq[N / 16];
    __shared__ float s_xd[NBE];
    __shared__ int16_t s_xs[N / 16];
    __shared__ uint4 s_hq[SMAX * F / 16];
    __shared__ float s_hd[SMAX * NBF];
    __shared__ int16_t s_hs[SMAX * F / 16];
    __shared__ int s_sel[8];
    __shared__ float s_w[8];
    __shared__ float s_gs;
    __shared__ float s_red[4];
    __shared__ int s_vote[4][4];
    __shared__ float4 s_x[N / 4];
    __shared__ float4 s_wr[4][N / 4];             // router rows of the 4 waves
    __shared__ float4 s_wsh[N / 4];               // shared-expert gate vector (collector)

    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6);
    const int gw = (int)blockIdx.x * 4 + wv;          // global wave = down row
    const int nw = (int)gridDim.x * 4;
    const int half = lane >> 5, l32 = lane & 31;
    const int gib = l32 >> 2, gg = l32 & 3;            // gate/up task: block, 64-lane group
    const int ds = lane >> 3, dq = lane & 7;           // down task: slot, task
    constexpr size_t GU_ROW = (size_t)NBE * Q4K_BYTES;                 // 1152
    constexpr size_t GU_SLAB = (size_t)F * GU_ROW;                     // 589,824
    constexpr size_t DN_SLAB = (size_t)N * NBF * (TD == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES);
    const unsigned long long *my_sel = tg->sel[blockIdx.x % REP];
    const int qk = ((int)blockIdx.x - QWG0) / QWG_STEP;
    const bool quantiser = wv == 1 && (int)blockIdx.x >= QWG0 && ((int)blockIdx.x - QWG0) % QWG_STEP == 0;

    float xrow = x[gw];            // x_0 of this wave's row (residual input)

    for (int l = 0; l < n_layer; l++) {
        const qmag_moe_layer &L = layers[l];
        const int E = L.n_expert, K = L.n_used, S = K + 1;
        const uint32_t seq = epoch * 256u + (uint32_t)l + 1u;
        const bool router_wg = (int)blockIdx.x * 4 < max(E, NBE);       // workgroup-uniform

        // optional phase timestamps (100 MHz real-time counter), thread 0 only
#define TR(i)                                                                              \
    if (trace && threadIdx.x == 0)                                                         \
        trace[((size_t)blockIdx.x * n_layer + l) * 8 + (i)] = __builtin_amdgcn_s_memrealtime();
        TR(0);

        // ---- 1. router workgroups: router rows into LDS, gather x_l, logits;
        // workgroup 0 also Q8_K(x_l) and, in its wave 0, the collector role
        bool ok = true;
        if (router_wg) {
            if (gw < E) {
                const float4 *row = (const float4 *)(L.gate_inp + (size_t)gw * N);
#pragma unroll
                for (int j = 0; j < 8; j++)
                    __builtin_amdgcn_global_load_lds((const void *)(row + lane + 64 * j),
                                                     (__attribute__((address_space(3))) void *)&s_wr[wv][64 * j],
                                                     16, 0, 0);
            }
            if (blockIdx.x == 0) {
#pragma unroll
                for (int j = 0; j < 2; j++)
                    __builtin_amdgcn_global_load_lds((const void *)((const float4 *)L.gate_inp_shexp + threadIdx.x + 256 * j),
                                                     (__attribute__((address_space(3))) void *)&s_wsh[wv * 64 + 256 * j],
                                                     16, 0, 0);
            }
            if (l == 0) {
#pragma unroll
                for (int k = 0; k < 2; k++)
                    s_x[threadIdx.x + 256 * k] = ((const float4 *)x)[threadIdx.x + 256 * k];
            } else {
                uint32_t v[8];
                ok = poll<8>(tg->x, [&](int k) { return 4 * ((int)threadIdx.x + 256 * (k >> 2)) + (k & 3); },
                             seq, v, abort_flag);
#pragma unroll
                for (int k = 0; k < 2; k++)
                    s_x[threadIdx.x + 256 * k] =
                        make_float4(__uint_as_float(v[4 * k]), __uint_as_float(v[4 * k + 1]),
                                    __uint_as_float(v[4 * k + 2]), __uint_as_float(v[4 * k + 3]));
            }
            drain();                 // router rows and gate vector have landed in LDS
            ok = wg_all(ok, s_vote, 2);
            if (ok && gw < E) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 a = s_x[lane + 64 * j], w = s_wr[wv][lane + 64 * j];
                    s += w.x * a.x + w.y * a.y + w.z * a.z + w.w * a.w;
                }
                s = group_sum<64>(s);
                if (lane == 0)
                    st64(tg->logits + gw, __float_as_uint(L.router_bias ? s + L.router_bias[gw] : s), seq);
            }
            if (ok && blockIdx.x == 0) {
                // Q8_K(x_l): wave wv quantises blocks wv and wv+4, publishes them
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int b = wv + 4 * i;
                    const Q8Lane q = q8k_quant_lane(s_x[b * 64 + lane]);
                    ((uint32_t *)s_xq)[b * 64 + lane] = q.packed;
                    if (lane == 0) s_xd[b] = q.d;
                    if ((lane & 3) == 0) s_xs[b * 16 + (lane >> 2)] = (int16_t)q.gsum;
                    unsigned long long *o = tg->xq[l % MAXL];
                    st64(o + b * 64 + lane, q.packed, seq);
                    if (lane == 0) st64(o + XQ_D + b, __float_as_uint(q.d), seq);
                    if ((lane & 3) == 0) st64(o + XQ_S + b * 16 + (lane >> 2), (uint32_t)q.gsum, seq);
                }
                __syncthreads();
                // shared-expert gate input sum_i wsh[i] * xq[i] * xd[i/256] (nn.c:452-454)
                {
                    const int8_t *xq8 = (const int8_t *)s_xq;
                    float g = 0.0f;
                    for (int i = (int)threadIdx.x; i < N; i += 256)
                        g += ((const float *)s_wsh)[i] * (float)xq8[i] * s_xd[i / QK_K];
                    g = group_sum<64>(g);
                    if (lane == 0) s_red[wv] = g;
                }
                __syncthreads();
                if (wv == 0) {
                    // collector: all logits -> top-K -> selection record
                    uint32_t v[4];
                    ok = poll<4>(tg->logits, [&](int j) { return lane + 64 * j < E ? lane + 64 * j : -1; },
                                 seq, v, abort_flag);
                    float lg[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        lg[j] = lane + 64 * j < E ? __uint_as_float(v[j]) : -INFINITY;
                        if (lane + 64 * j < E) g_logits[lane + 64 * j] = lg[j];
                    }
                    int my_sel = 0;
                    float my_w = 0.0f;
                    route_topk(lg, E, K, my_sel, my_w);
                    const float gs = 1.0f / (1.0f + expf(-((s_red[0] + s_red[1]) + (s_red[2] + s_red[3]))));
                    // lanes 8..15 take the weights of lanes 0..7
                    const float w_hi = __shfl(my_w, lane - 8);
                    if (ok && lane < SEL_WORDS) {
                        const uint32_t word = lane < 8 ? (uint32_t)my_sel
                                            : lane < 16 ? __float_as_uint(w_hi) : __float_as_uint(gs);
                        st64r(tg->sel[0] + lane, word, seq);
                        if (lane < K) {
                            g_sel[lane] = my_sel;
                            g_w[lane] = my_w;
                        }
                        if (lane == 16) g_gs[0] = gs;
                    }
                }
            }
        }
        TR(1);

        // ---- 2. every workgroup: selection record (17 words, wave 0), then
        // Q8_K(x_l) (648 words, all threads, read once the record is valid)
        if (wv == 0) {
            uint32_t v[1];
            ok = poll<1>(my_sel, [&](int) { return lane < SEL_WORDS && (lane < K || (lane >= 8 && lane < 8 + K) || lane == 16) ? lane : -1; },
                         seq, v, abort_flag) && ok;
            if (lane < K) s_sel[lane] = (int)v[0];
            else if (lane >= 8 && lane < 8 + K) s_w[lane - 8] = __uint_as_float(v[0]);
            else if (lane == 16) s_gs = __uint_as_float(v[0]);
        }
        if (!wg_all(ok, s_vote, 0)) return;
        TR(2);

        // ---- 3. this wave's gate/up and down bytes (routed slots and the
        // shared slot), all issued before any is consumed
        uint4 gh[MAX_RP], g0[MAX_RP], g1[MAX_RP];
#pragma unroll
        for (int j = 0; j < MAX_RP; j++) {
            gh[j] = g0[j] = g1[j] = make_uint4(0, 0, 0, 0);
            const int rp = gw + j * nw;
            const int slot = rp / F;
            if (rp < S * F) {
                const uint8_t *m = slot < K ? (const uint8_t *)(half ? L.up_exps : L.gate_exps) +
                                                  (size_t)s_sel[slot] * GU_SLAB
                                            : (const uint8_t *)(half ? L.up_shexp : L.gate_shexp);
                const uint8_t *blk = m + (size_t)(rp % F) * GU_ROW + (size_t)gib * Q4K_BYTES;
                gh[j] = ld16(blk);
                g0[j] = ld16(blk + 16 + 32 * gg);
                g1[j] = ld16(blk + 32 + 32 * gg);
            }
        }
        DRaw<TD> dsh, drt;
        d_zero(dsh);
        d_zero(drt);
        if (ds < K) d_load<TD>(drt, (const uint8_t *)L.down_exps + (size_t)s_sel[ds] * DN_SLAB, gw, dq);
        if (lane < 8) d_load<TD>(dsh, (const uint8_t *)L.down_shexp, gw, dq);
        if (blockIdx.x != 0) {      // workgroup 0 quantised x itself
            uint32_t v[3];
            auto xi = [&](int k) {
                const int i = (int)threadIdx.x + 256 * k;
                return i < XQ_WORDS ? i : -1;
            };
            // written by workgroup 0 before its selection record: read cached
            ok = read_bulk<3>(tg->xq[l % MAXL], xi, seq, v, abort_flag);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const int i = xi(k);
                if (i < 0) continue;
                if (i < XQ_D) ((uint32_t *)s_xq)[i] = v[k];
                else if (i < XQ_S) s_xd[i - XQ_D] = __uint_as_float(v[k]);
                else s_xs[i - XQ_S] = (int16_t)(int)v[k];
            }
        }
        if (!wg_all(ok, s_vote, 1)) return;
        TR(3);

        // ---- 4. gate/up rows -> h = silu(g) * u, published for the quantisers
        {
            Q4Act a;
            const uint4 *xw = s_xq + (gib * QK_K + 64 * gg) / 16;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint4 w = xw[k];
                a.x[4 * k + 0] = w.x;
                a.x[4 * k + 1] = w.y;
                a.x[4 * k + 2] = w.z;
                a.x[4 * k + 3] = w.w;
            }
            a.xd = s_xd[gib];
            const int16_t *sp = s_xs + gib * 16 + 4 * gg;
            a.sx0 = (float)(sp[0] + sp[1]);
            a.sx1 = (float)(sp[2] + sp[3]);
#pragma unroll
            for (int j = 0; j < MAX_RP; j++) {
                const int rp = gw + j * nw;
                if (rp < S * F) {                       // wave-uniform
                    float v = q4_task(gh[j], g0[j], g1[j], a, gg);
                    v = group_sum<32>(v);
                    auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                               false, false);
                    const float u = __uint_as_float(pr[1]);
                    if (lane == 0) st64(tg->h + rp, __float_as_uint((v / (1.0f + expf(-v))) * u), seq);
                }
            }
        }
        TR(4);

        // ---- 5. quantiser waves publish Q8_K(h) blocks; every workgroup
        // polls the 18 block sentinels, then reads the blocks into LDS
        ok = true;
        if (quantiser && qk < S * NBF) {
            uint32_t v[4];
            ok = poll<4>(tg->h, [&](int k) { return qk * QK_K + 4 * lane + k; }, seq, v, abort_flag);
            const float4 hv = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]),
                                          __uint_as_float(v[2]), __uint_as_float(v[3]));
            *(float4 *)(g_h + qk * QK_K + 4 * lane) = hv;              // stage copy
            const Q8Lane q = q8k_quant_lane(hv);
            unsigned long long *o = tg->hq[l % MAXL] + qk * HQ_BLK;
            st64(o + lane, q.packed, seq);
            if ((lane & 3) == 0) st64(o + 65 + (lane >> 2), (uint32_t)q.gsum, seq);
            if (lane == 0) st64(o + 64, __float_as_uint(q.d), seq);  // sentinel, written last
        }
        if (wv == 0) {
            uint32_t v[1];
            ok = poll<1>(tg->hq[l % MAXL], [&](int) { return lane < S * NBF ? lane * HQ_BLK + 64 : -1; }, seq, v,
                         abort_flag) && ok;
        }
        if (!wg_all(ok, s_vote, 2)) return;
        {
            uint32_t v[HQ_PER_THREAD];
            auto hi = [&](int k) {
                const int i = (int)threadIdx.x + 256 * k;
                return i < S * NBF * HQ_BLK ? i : -1;
            };
            ok = read_bulk<HQ_PER_THREAD>(tg->hq[l % MAXL], hi, seq, v, abort_flag);
#pragma unroll
            for (int k = 0; k < HQ_PER_THREAD; k++) {
                const int i = hi(k);
                if (i < 0) continue;
                const int b = i / HQ_BLK, r = i % HQ_BLK;
                if (r < 64) ((uint32_t *)s_hq)[b * 64 + r] = v[k];
                else if (r == 64) s_hd[b] = __uint_as_float(v[k]);
                else s_hs[b * 16 + r - 65] = (int16_t)(int)v[k];
            }
        }
        if (!wg_all(ok, s_vote, 3)) return;
        TR(5);

        // ---- 6. down row gw of the routed experts (8 lanes each) and of the
        // shared expert (lanes 0-7), combined in the reference order
        {
            const int slot = ds < K ? ds : 0;
            float dr = d_dot<TD>(drt, (const uint32_t *)s_hq + slot * (F / 4), s_hd + slot * NBF,
                                 s_hs + slot * (F / 16), dq);
            dr = group_sum<8>(dr);
            float dsv = d_dot<TD>(dsh, (const uint32_t *)s_hq + K * (F / 4), s_hd + K * NBF,
                                  s_hs + K * (F / 16), dq);
            dsv = group_sum<8>(dsv);
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                const float dk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dr), 8 * k));
                acc = __fadd_rn(acc, __fmul_rn(s_w[k], dk));
            }
            const float dsh0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsv), 0));
            acc = __fadd_rn(acc, __fmul_rn(s_gs, dsh0));
            if (out) {
                if (lane == 0) out[gw] = acc;
            } else {
                xrow = __fadd_rn(acc, xrow);
                if (lane == 0) {
                    if (l + 1 < n_layer) st64(tg->x + gw, __float_as_uint(xrow), seq + 1u);
                    else x[gw] = xrow;
                }
            }
        }
        TR(6);
#undef TR
        // LDS is rewritten next layer only after this barrier
        __syncthreads();
    }
}

}  // namespace fused

// ------------------------------------------------------------------ host --
static qmag_moe_layer *g_dev_layers = nullptr;
static qmag_moe_layer g_host_copy[256];
static int g_host_n = 0;
static fused::Tagged *g_tagged = nullptr;
static int *g_abort = nullptr;
static unsigned g_epoch = 0;        // launches since the tagged buffers were last zeroed
static unsigned long long *g_trace = nullptr;   // phase timestamps of the last launch (optional)
static size_t g_trace_bytes = 0;
static float *g_logits = nullptr, *g_h = nullptr, *g_w = nullptr, *g_gs = nullptr;
static int *g_sel = nullptr;
static int g_coop_ok = -1;

bool fused_eligible(const qmag_moe_layer *L, int n_layer)
{
    if (n_layer < 1 || n_layer > 255) return false;
    for (int l = 0; l < n_layer; l++) {
        const qmag_moe_layer &a = L[l];
        if (a.n_embd != fused::N || a.n_ff != fused::F || a.n_expert < 1 || a.n_expert > 256 ||
            a.n_used < 1 || a.n_used > 8 || a.n_used > a.n_expert)
            return false;
        if (a.t_down_exps != a.t_down_shexp || a.t_down_exps != L[0].t_down_exps) return false;
    }
    if (g_coop_ok < 0) {
        int coop = 0, occ = 0;
        if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, ctx().dev) != hipSuccess) coop = 0;
        const void *k = L[0].t_down_exps == QMAG_TYPE_Q6_K
                            ? (const void *)fused::moe_decode_kernel<QMAG_TYPE_Q6_K>
                            : (const void *)fused::moe_decode_kernel<QMAG_TYPE_Q4_K>;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, 256, 0) != hipSuccess) occ = 0;
        g_coop_ok = (coop && ctx().n_cu * occ >= fused::WGS) ? 1 : 0;
    }
    return g_coop_ok == 1;
}

static int rearm()
{
    QMAG_HIP(hipStreamSynchronize(ctx().stream));
    QMAG_HIP(hipMemset(g_tagged, 0, sizeof(fused::Tagged)));
    QMAG_HIP(hipMemset(g_abort, 0, 128));
    QMAG_HIP(hipDeviceSynchronize());
    g_epoch = 0;
    return QMAG_OK;
}

int fused_status()
{
    if (!g_abort) return QMAG_OK;
    int abort_flag = 0;
    QMAG_HIP(hipMemcpy(&abort_flag, g_abort, sizeof(int), hipMemcpyDeviceToHost));
    if (abort_flag) {
        int st = rearm();
        if (st) return st;
        return fail(QMAG_ERR_KERNEL, "fused MoE decode: a cross-workgroup wait hit its spin limit");
    }
    return QMAG_OK;
}

static int fused_prepare(const qmag_moe_layer *L, int n_layer, hipStream_t s)
{
    if (!g_dev_layers) {
        QMAG_HIP(hipMalloc(&g_dev_layers, sizeof(qmag_moe_layer) * 256));
        QMAG_HIP(hipMalloc(&g_tagged, sizeof(fused::Tagged)));
        QMAG_HIP(hipMalloc(&g_abort, 128));
        QMAG_HIP(hipMalloc(&g_logits, sizeof(float) * 256));
        QMAG_HIP(hipMalloc(&g_h, sizeof(float) * fused::SMAX * fused::F));
        QMAG_HIP(hipMalloc(&g_w, sizeof(float) * 8));
        QMAG_HIP(hipMalloc(&g_gs, sizeof(float) * 8));
        QMAG_HIP(hipMalloc(&g_sel, sizeof(int) * 8));
        int st = rearm();
        if (st) return st;
    }
    if (g_host_n != n_layer || memcmp(g_host_copy, L, sizeof(qmag_moe_layer) * (size_t)n_layer) != 0) {
        QMAG_HIP(hipStreamSynchronize(s));
        QMAG_HIP(hipMemcpy(g_dev_layers, L, sizeof(qmag_moe_layer) * (size_t)n_layer, hipMemcpyHostToDevice));
        memcpy(g_host_copy, L, sizeof(qmag_moe_layer) * (size_t)n_layer);
        g_host_n = n_layer;
    }
    if (g_epoch >= (1u << 24)) {           // tags would wrap: zero the buffers, restart
        int st = rearm();
        if (st) return st;
    }
    if (option(QMAG_OPT_TRACE)) {
        const size_t need = sizeof(unsigned long long) * fused::WGS * (size_t)n_layer * 8;
        if (need > g_trace_bytes) {
            QMAG_HIP(hipStreamSynchronize(s));
            if (g_trace) QMAG_HIP(hipFree(g_trace));
            QMAG_HIP(hipMalloc(&g_trace, need));
            g_trace_bytes = need;
        }
    } else if (g_trace) {
        QMAG_HIP(hipStreamSynchronize(s));
        QMAG_HIP(hipFree(g_trace));
        g_trace = nullptr;
        g_trace_bytes = 0;
    }
    return QMAG_OK;
}

int fused_launch(const qmag_moe_layer *L, int n_layer, float *x, float *out, hipStream_t s)
{
    if (out && n_layer != 1) return fail(QMAG_ERR_ARG, "fused: out mode needs exactly one layer");
    int st = fused_prepare(L, n_layer, s);
    if (st) return st;
    const qmag_moe_layer *dl = g_dev_layers;
    unsigned epoch = g_epoch;
    unsigned long long *trace = option(QMAG_OPT_TRACE) ? g_trace : nullptr;
    void *args[] = {(void *)&dl,      (void *)&n_layer, (void *)&x,     (void *)&out,
                    (void *)&g_tagged, (void *)&g_logits, (void *)&g_h, (void *)&g_sel,
                    (void *)&g_w,     (void *)&g_gs,    (void *)&g_abort, (void *)&epoch,
                    (void *)&trace};
    const void *k = L[0].t_down_exps == QMAG_TYPE_Q6_K
                        ? (const void *)fused::moe_decode_kernel<QMAG_TYPE_Q6_K>
                        : (const void *)fused::moe_decode_kernel<QMAG_TYPE_Q4_K>;
    prof_begin(PROF_FUSED, s);
    if (option(QMAG_OPT_COOP))
        QMAG_HIP(hipLaunchCooperativeKernel(k, dim3(fused::WGS), dim3(256), args, 0, s));
    else       // fused_eligible checked that every workgroup fits at once
        QMAG_HIP(hipLaunchKernel(k, dim3(fused::WGS), dim3(256), args, 0, s));
    prof_end(PROF_FUSED, s);
    g_epoch++;
    return QMAG_OK;
}

int fused_trace_read(void *dst, size_t bytes)
{
    if (!g_trace) return fail(QMAG_ERR_ARG, "no trace recorded (enable QMAG_OPT_TRACE)");
    QMAG_HIP(hipStreamSynchronize(ctx().stream));
    QMAG_HIP(hipMemcpy(dst, g_trace, bytes < g_trace_bytes ? bytes : g_trace_bytes, hipMemcpyDeviceToHost));
    return QMAG_OK;
}

int fused_last_stage(const float **logits, const int **sel, const float **w, const float **gs,
                     const float **h)
{
    if (!g_logits) return fail(QMAG_ERR_ARG, "no fused MoE call yet");
    if (logits) *logits = g_logits;
    if (sel) *sel = g_sel;
    if (w) *w = g_w;
    if (gs) *gs = g_gs;
    if (h) *h = g_h;
    return QMAG_OK;
}

}  // namespace qmag
