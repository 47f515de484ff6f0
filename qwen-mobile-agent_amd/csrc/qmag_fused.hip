// qmag_fused.hip -- one persistent kernel that runs the whole qwen35moe MoE
// FFN decode (batch 1) for a run of layers (src/nn.c:509-707 per layer, the
// residual add of nn.c:2252 between layers).
//
// Shapes are the engine's compile-time ones (src/qma.h:28, 57-60): hidden
// 2048, expert ff 512, up to 256 experts, top-k <= 8, plus the shared
// expert.  512 workgroups x 4 waves, two workgroups per CU, in two roles:
//
//   core workgroups 0..127 (16 per XCD) each own 16 rows of the hidden state.
//     They compute the router logits (2 per workgroup, router rows staged in
//     LDS one layer ahead), Q8_K(x) (workgroups 0..7 publish one 256-block
//     each, with that block's share of the shared-expert gate input; every
//     core workgroup also keeps its own copy) and the combine + residual of
//     their rows from the 9 slots' down outputs.
//   stream workgroups 128..511 run the softmax/top-k themselves.
//   Every wave (2048) takes up to two routed gate/up row pairs (slot s <
//   n_used is expert sel[s]), so each CU carries the same share whichever
//   two workgroups it holds.  The shared expert's 512 row pairs go to waves
//   2, 3 of workgroups 256..511, idle during the top-k: their rows are
//   fetched at layer start and h published as soon as Q8_K(x) is in.
//   Down projection: 32 units of 64 rows per slot.  A unit gathers its slot's
//   h, quantises it (Q8_K(h), two blocks, in LDS) and takes the dots of its
//   down rows, held in registers; routed units sit in workgroups 256..511
//   (one per CU), the shared slot's in 128..159 (its h is out early).
//   Spreading the down dots over 288 workgroups, each needing one slot's h,
//   keeps both the gathers and the integer work per workgroup small.
//
// Hand-offs of one layer (each a set of tagged words, see below):
//   x_l rows      core -> core            (2048 words, read by 128 workgroups)
//   logits        core -> every workgroup (256 words, 8 replicas); every
//                 workgroup runs the softmax/top-k itself, so the selection
//                 needs no further hop
//   Q8_K(x)       core 0..7 -> stream     (656 words, 8 replicas; produced
//                 together with the logits, off the critical path)
//   h             stream -> stream        (512 words of one slot, read by that
//                                          slot's 32 down workgroups)
//   y             stream -> core          (down outputs, 16 rows x 9 slots
//                                          read by each core workgroup)
//
// Every published value is one 64-bit word {32 data bits, 32-bit tag},
// written with a single-copy-atomic device-scope store; the tag is
// epoch*256 + layer + 1 (the epoch counts launches, so no buffer is ever
// cleared between launches).  A consumer reads words with device-scope
// atomic loads and accepts a word only when it carries the current tag: data
// is its own ready flag, and no read-modify-write, barrier or cache
// maintenance is needed.  Each buffer has one slot: a word of layer l+1 is
// written only after every reader of the layer-l word has consumed it (the
// dependency chain of the layer passes through every such reader).
//
// Every poll is bounded: an exhausted waiter raises an abort flag that all
// pollers check, so the grid always drains; qmag_sync() reports it.
#include <limits.h>
#include <string.h>

#include <vector>

#include "qmag_internal.h"

namespace qmag {
namespace fused {

constexpr int N = 2048, F = 512;
constexpr int NBE = N / QK_K, NBF = F / QK_K;     // 8, 2
constexpr int SMAX = 9;                           // 8 routed + shared
constexpr int WGS = 512;
constexpr int CORE = 128;                         // core workgroups
constexpr int CROWS = N / CORE;                   // 16 hidden rows per core workgroup
constexpr int WROWS = CROWS / 4;                  // 4 per core wave
constexpr int NLOG = 256 / CORE;                  // 2 router logits per core workgroup
constexpr int TR_LAYERS = 64;                     // layers a traced launch records
constexpr int GU_WAVES = WGS * 4;                 // every wave takes routed gate/up row pairs
constexpr int MAX_RP = (8 * F + GU_WAVES - 1) / GU_WAVES;      // 2 routed row pairs per wave
// the shared expert's row pair i: workgroup SH_WG0 + i/2, wave 2 + i%2 (the
// second workgroup of every CU when workgroups fill the CUs in order)
constexpr int SH_WG0 = WGS / 2;
static_assert(F <= 2 * (WGS - SH_WG0), "shared row pairs out of range");
constexpr int DROWS = 64;                         // down rows per down unit (one slot)
constexpr int DWG_PER_SLOT = N / DROWS;           // 32
constexpr int DN_ROUNDS = DROWS / 4 / 8;          // 16 rows per wave, 8 lanes per row: 2 rounds
// routed down unit u (slot u/32) in workgroup RDN_WG0 + u, one per CU;
// shared-slot unit r in workgroup SDN_WG0 + r (its h is out early)
constexpr int RDN_WG0 = WGS / 2, SDN_WG0 = CORE;
static_assert(RDN_WG0 + 8 * DWG_PER_SLOT <= WGS && SDN_WG0 + DWG_PER_SLOT <= RDN_WG0,
              "down workgroups out of range");
// Every wait is bounded twice: by wall time (SPIN_TICKS of the 100 MHz
// real-time counter, 50 ms, far beyond any legitimate hand-off of a few
// microseconds) and, as a backstop, by a poll count.
constexpr long SPIN_LIMIT = 1L << 22;
constexpr uint64_t SPIN_TICKS = 5000000;

// Q8_K records are laid out exactly as the LDS copy their readers keep, so a
// reader copies word i to LDS word i:
//   Q8_K(x): 512 packed xq words (block b at 64b), 8 scales d, 128 group
//   sums, 8 partials of the shared-expert gate input (nn.c:452-454)
constexpr int XR_D = N / 4, XR_S = XR_D + NBE, XR_G = XR_S + N / 16, XR_WORDS = XR_G + NBE;   // 656
//   Q8_K(h) of one slot in a down workgroup's LDS, 2 blocks: packed words,
//   scales, group sums
constexpr int HS_D = F / 4, HS_S = HS_D + NBF, HS_WORDS = HS_S + F / 16;                    // 162
constexpr int REP = 8;                            // replicas of the widely read records

struct Tagged {
    unsigned long long logits[REP][256];          // logit e at word logit_pos(e)
    unsigned long long xq[REP][XR_WORDS];
    unsigned long long x[N];
    unsigned long long h[SMAX * F];               // slot s, row i at s*F + i
    unsigned long long y[SMAX * N];               // down output of slot s, row r at s*N + r
};
// word offsets of the arrays (every array starts on a 16-byte boundary)
constexpr int TW_LOGITS = 0, TW_XQ = TW_LOGITS + REP * 256, TW_X = TW_XQ + REP * XR_WORDS,
              TW_H = TW_X + N, TW_Y = TW_H + SMAX * F;
static_assert(offsetof(Tagged, xq) == 8 * TW_XQ && offsetof(Tagged, x) == 8 * TW_X &&
              offsetof(Tagged, h) == 8 * TW_H && offsetof(Tagged, y) == 8 * TW_Y && XR_WORDS % 2 == 0 &&
              XR_G % 2 == 0 && TW_H % 2 == 0 && TW_Y % 2 == 0 && F % 2 == 0,
              "tagged layout");
// Logits are stored so that the 16-byte pair p of lane l (p = l, l + 64)
// holds experts l + 64h + 128(p >= 64), h = the half: a lane then reads
// experts l, l+64, l+128, l+192, the layout the top-k works on.
__device__ __forceinline__ int logit_pos(int e) { return 2 * ((e & 63) + 64 * (e >> 7)) + ((e >> 6) & 1); }

__device__ __forceinline__ unsigned long long ld64(const unsigned long long *p)
{
    return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until all of this wave's outstanding memory operations completed
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ int ld_flag(const int *p)
{
    return __hip_atomic_load(const_cast<int *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The abort word: 0 while every wait has been met; otherwise epoch + 1 of the
// first launch one of whose waits expired (the host replays from that launch
// on).  Every poller checks it, so the grid drains once it is set, and a later
// launch that finds it set exits before writing any output.
struct Abort {
    int *flag;
    int code;       // this launch's epoch + 1
};
__device__ __forceinline__ void raise_abort(const Abort &ab)
{
    int expect = 0;
    __hip_atomic_compare_exchange_strong(ab.flag, &expect, ab.code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}
// true when the wait that started at t0 must give up: another waiter raised
// the abort word, or this one ran out of time (then it raises the word)
__device__ __forceinline__ bool give_up(const Abort &ab, uint64_t t0)
{
    if (ld_flag(ab.flag) != 0) return true;
    if (__builtin_amdgcn_s_memrealtime() - t0 > SPIN_TICKS) {
        raise_abort(ab);
        return true;
    }
    return false;
}

// One wave reads CNT tagged words per lane, p[idx(k)] (idx < 0: no word),
// until every word carries `seq`; the low halves land in val[].  All loads of
// a round are issued together, and a retry reloads only the stale words.
template <int CNT, typename Idx>
__device__ bool poll(const unsigned long long *p, Idx idx, uint32_t seq, uint32_t (&val)[CNT],
                     const Abort &ab)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
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
        if ((it & 31) == 31 && give_up(ab, t0)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    raise_abort(ab);
    return false;
}

// Bulk reads take two tagged words per 16-byte load: a buffer load with the
// same device-coherent cache policy (sc1) as the 8-byte atomic loads.  Each
// 8-byte half is single-copy atomic and checked against its own tag, so the
// pair needs no atomicity as a whole; 16-byte loads halve the requests,
// which is what bounds a workgroup's bulk read rate.
constexpr int CPOL_SC1 = 16;
constexpr int OOB_BYTE = 1 << 30;                 // beyond the Tagged buffer's records
typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Publish one tagged word (index `word` of the Tagged buffer): an aligned
// 8-byte vector store with the device-coherent policy, the instruction a
// relaxed agent-scope atomic store compiles to.  Addressed through the
// buffer resource so the only per-lane state is a 32-bit offset.
__device__ __forceinline__ void st64(Rsrc rs, int word, uint32_t v, uint32_t seq)
{
    const u32x2 d = {v, seq};
    __builtin_amdgcn_raw_buffer_store_b64(d, rs, word * 8, 0, CPOL_SC1);
}

// One wave reads CNT word pairs per lane.  code(k) = pair index * 4 + need
// (need: bit 0 the low word, bit 1 the high word must carry seq), or -1 for
// no pair.  Word offsets are relative to the resource base; the low 32 bits
// of the needed words land in val[k][0..1].
template <int CNT, typename Code>
__device__ bool pollq(Rsrc rs, int base_word, Code code, uint32_t seq, uint32_t (&val)[CNT][2],
                      const Abort &ab)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < CNT; k++)
        if (code(k) >= 0) pending |= 1u << k;
    for (long it = 0; it < SPIN_LIMIT; it++) {
        // one batch of loads, then the checks: a round costs one memory
        // latency, not one per pair.  A pair that is done or absent reads
        // beyond the end of the buffer, which returns zeros without a memory
        // access, so the loads need no branch.
        decltype(__builtin_amdgcn_raw_buffer_load_b128(rs, 0, 0, 0)) v[CNT];
#pragma unroll
        for (int k = 0; k < CNT; k++) {
            const int off = (pending & (1u << k)) ? (base_word + 2 * (code(k) >> 2)) * 8 : OOB_BYTE;
            v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL_SC1);
        }
        // keep the batch together: without these the compiler sinks each load
        // into the branch that checks it, or hoists a check between the
        // loads, one memory latency per pair again
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < CNT; k++) __asm__ volatile("" : "+v"(v[k]));
#pragma unroll
        for (int k = 0; k < CNT; k++) {
            if (pending & (1u << k)) {
                const int c = code(k);
                const bool lo = !(c & 1) || v[k][1] == seq, hi = !(c & 2) || v[k][3] == seq;
                if (lo && hi) {
                    val[k][0] = v[k][0];
                    val[k][1] = v[k][2];
                    pending &= ~(1u << k);
                }
            }
        }
        if (__all(pending == 0)) return true;
        if ((it & 31) == 31 && give_up(ab, t0)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    raise_abort(ab);
    return false;
}

// workgroup-wide AND of one flag per wave (slot: a distinct LDS row per call site)
__device__ __forceinline__ bool wg_all(bool ok, int (*s_vote)[4], int slot)
{
    if (lane_id() == 0) s_vote[slot][threadIdx.x >> 6] = ok ? 1 : 0;
    __syncthreads();
    return (s_vote[slot][0] & s_vote[slot][1] & s_vote[slot][2] & s_vote[slot][3]) != 0;
}

// ---- down-projection task: 8 lanes per (row, slot), lane q of the 8
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

// fp32 contribution of task q against one slot's Q8_K(h) held in LDS; the
// 8 lanes of a (row, slot) pair sum to the row's dot (blocks in order)
template <int TD>
__device__ __forceinline__ float d_dot(const DRaw<TD> &d, const uint32_t *hq, const float *hd,
                                       const int *hs, int q)
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
        const int *s = hs + ib * 16 + 4 * sub;
        a.sx0 = (float)(s[0] + s[1]);
        a.sx1 = (float)(s[2] + s[3]);
        return q4_task(d.hdr, d.q0, d.q1, a, sub);
    }
}

// Order-preserving int32 key of a finite float: a > b as floats exactly when
// key(a) > key(b) as signed ints (-0 is folded to +0 first, so the two zeros,
// equal as floats, get one key).  An integer wave max folds its DPP move into
// the max itself; a float max would first quiet signalling NaNs in both
// operands (three instructions per step instead of one).
__device__ __forceinline__ int f2key(float v)
{
    // (route_topk handles NaN logits before it makes keys; this keeps the
    // order total all the same)
    if (v != v) return INT_MIN;
    const int b = __float_as_int(v + 0.0f);
    return b >= 0 ? b : b ^ 0x7fffffff;
}
__device__ __forceinline__ float key2f(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff); }

// Softmax top-K over E <= 256 logits (4 per lane of one wave: experts
// lane + 64j), in the order nn.c:525-536 picks them: each pick is the largest
// value left, the lowest index among equal values (the reference's strict-`>`
// scan from e = 0).  The selection is made on the logits (softmax is
// monotonic) through their integer keys; each lane sorts its four candidates
// once, and a pick is one wave max over the lane heads and a shift of the
// winning lane's list.  Lane k < K receives pick k: its expert id and its
// weight exp(l_k - l_max) / sum over the K picks, the reference's
// p_k / sum_sel p with the full softmax sum cancelled (summed in pick order).
//
// The picks run a fast path first: the winning lane is the one whose head
// equals the maximum, a vector compare, so no pick waits for a scalar round
// trip.  That is exact unless two heads are equal; every pick's ballot is
// checked off the critical path, and if any pick saw such a tie the picks are
// made again with the tie rule (lowest index among the equal heads).
template <bool EXACT>
__device__ __forceinline__ bool topk_picks(const int (&v0)[4], const int (&id0)[4], int K, int lane, int &sel,
                                           int &my_key)
{
    int v[4] = {v0[0], v0[1], v0[2], v0[3]}, id[4] = {id0[0], id0[1], id0[2], id0[3]};
    unsigned long long tie = 0;
    for (int k = 0; k < K; k++) {
        const int m = group_max_i<64>(v[0]);
        bool me = v[0] == m;
        unsigned long long bal = __ballot(me);
        if constexpr (EXACT) {
            if (bal & (bal - 1)) {              // exact tie: the lowest index wins (one wave min)
                const int best = group_min_i<64>(me ? id[0] : INT_MAX);
                me = me && id[0] == best;
                bal = __ballot(me);
            }
        } else {
            tie |= bal & (bal - 1);
        }
        const int id_head = id[0];
        v[0] = me ? v[1] : v[0];
        v[1] = me ? v[2] : v[1];
        v[2] = me ? v[3] : v[2];
        v[3] = me ? INT_MIN : v[3];
        id[0] = me ? id[1] : id[0];
        id[1] = me ? id[2] : id[1];
        id[2] = me ? id[3] : id[2];
        const int e = __builtin_amdgcn_readlane(id_head, __builtin_ctzll(bal));
        sel = lane == k ? e : sel;
        my_key = lane == k ? m : my_key;
    }
    return tie == 0;
}

__device__ void route_topk(const float (&lg)[4], int E, int K, int &my_sel, float &my_w)
{
    const int lane = lane_id();
    int v[4], id[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[j] = lane + 64 * j < E ? f2key(lg[j]) : INT_MIN;
        id[j] = lane + 64 * j;
    }
    auto cswap = [&](int i, int j) {           // descending; equal keys by index
        const bool sw = v[j] > v[i] || (v[j] == v[i] && id[j] < id[i]);
        const int vi = v[i], vj = v[j], ii = id[i], ij = id[j];
        v[i] = sw ? vj : vi;
        v[j] = sw ? vi : vj;
        id[i] = sw ? ij : ii;
        id[j] = sw ? ii : ij;
    };
    cswap(0, 1);
    cswap(2, 3);
    cswap(0, 2);
    cswap(1, 3);
    cswap(1, 2);
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < 4; j++) nan_here = nan_here || (lane + 64 * j < E && lg[j] != lg[j]);
    const bool any_nan = __ballot(nan_here) != 0;
    int my_key = INT_MIN, sel = 0;
    if (!topk_picks<false>(v, id, K, lane, sel, my_key)) topk_picks<true>(v, id, K, lane, sel, my_key);
    const float l0 = key2f(__builtin_amdgcn_readfirstlane(my_key));
    // the reference's softmax is NaN throughout when a logit is NaN or +Inf,
    // or when every logit is strictly below -1e30 (see route_degenerate):
    // then it picks expert 0 K times
    if (any_nan || !(l0 < INFINITY) || l0 < -1e30f) {
        if (lane < K) my_sel = 0;
        my_w = route_degenerate_weight(K);
        return;
    }
    if (lane < K) my_sel = sel;
    const float ex = lane < K ? expf(key2f(my_key) - l0) : 0.0f;
    my_w = ex / group_sum<8>(ex);
}

template <int TD>
__global__ __launch_bounds__(256, 2) void moe_decode_kernel(const qmag_moe_layer *__restrict__ layers,
                                                            int n_layer, float *x, float *out,
                                                            Tagged *tg, float *g_logits, float *g_h,
                                                            int *g_sel, float *g_w, float *g_gs,
                                                            int *abort_flag, unsigned epoch,
                                                            unsigned long long *trace)
{
    __shared__ float4 s_x[N / 4];                 // core: x_l
    __shared__ float4 s_wr[NLOG][N / 4];          // core: this workgroup's router rows
    __shared__ uint4 s_xrec[(XR_WORDS + 3) / 4];  // the Q8_K(x_l) record
    __shared__ float4 s_hs[F / 4];                // down: h of the slot
    __shared__ uint4 s_hq[(HS_WORDS + 3) / 4];    // down: Q8_K of that h
    __shared__ float s_gsp[NBE];                  // core: shared-gate input partials
    __shared__ float s_dres[CROWS][SMAX + 1];     // core: per (row, slot) down outputs
    __shared__ float s_xout[CROWS];               // core: x_{l+1} rows to publish
    __shared__ int s_sel[8];
    __shared__ float s_w[8];
    __shared__ int s_vote[4][4];
    __shared__ uint32_t s_tr[TR_LAYERS][8];        // traced launches: phase stamps until the end

    const int lane = lane_id(), wv = (int)(threadIdx.x >> 6), tid = (int)threadIdx.x;
    const int b = (int)blockIdx.x;
    const int rep = b % REP;
    const bool core = b < CORE;
    const Rsrc rs = __builtin_amdgcn_make_buffer_rsrc(tg, 0, (int)sizeof(Tagged), 0x00020000);
    const Abort ab{abort_flag, (int)epoch + 1};
    // set by an earlier launch whose wait expired: this launch exits at its
    // first barrier, before any output is written (read now, used there)
    const bool pre_abort = ld_flag(abort_flag) != 0;
    const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
    if (trace && threadIdx.x == 0)
        for (int i = 0; i < TR_LAYERS * 8; i++) s_tr[i / 8][i % 8] = 0;
    // the 256 logits of replica rep, lane's pairs l and l + 64 (experts
    // l + 64j, j = 0..3); a half is needed only for an expert below E
    auto logit_pairs = [&](int E) {
        return [=](int k) {
            const int e0 = lane + 128 * k;
            const int need = (e0 < E ? 1 : 0) | (e0 + 64 < E ? 2 : 0);
            return need ? 4 * (lane + 64 * k) + need : -1;
        };
    };
    auto read_logits = [&](int E, uint32_t seq, float (&lg)[4]) {
        uint32_t v[2][2];
        const bool ok = pollq<2>(rs, TW_LOGITS + rep * 256, logit_pairs(E), seq, v, ab);
#pragma unroll
        for (int j = 0; j < 4; j++)
            lg[j] = lane + 64 * j < E ? __uint_as_float(v[j >> 1][j & 1]) : -INFINITY;
        return ok;
    };
    constexpr size_t GU_ROW = (size_t)NBE * Q4K_BYTES;                 // 1152
    constexpr size_t GU_SLAB = (size_t)F * GU_ROW;                     // 589,824
    constexpr size_t DN_SLAB = (size_t)N * NBF * (TD == QMAG_TYPE_Q6_K ? Q6K_BYTES : Q4K_BYTES);

    // ---- roles shared by both kinds of workgroup
    // routed gate/up row pairs: global wave gw takes rows gw + j*GU_WAVES
    const int gw = b * 4 + wv;
    const int half = lane >> 5, l32 = lane & 31;
    const int gib = l32 >> 2, gg = l32 & 3;       // gate/up task: block, 64-lane group
    // shared-expert row pair (at most one per wave): waves 2, 3 of the
    // workgroups from SH_WG0 on, which are idle while wave 0 runs the top-k
    const int sh_row = b >= SH_WG0 && wv >= 2 ? 2 * (b - SH_WG0) + (wv - 2) : F;
    // down role: a routed unit (slot u/32, rows (u%32)*64 ..) in workgroup
    // RDN_WG0 + u, a shared-slot unit in workgroup SDN_WG0 + r; wave wv takes
    // rows drow0 + 16wv .. +15, 8 lanes per row (lane group dg, sub-task dq)
    const int dunit = b >= RDN_WG0 ? b - RDN_WG0 : -1;
    const bool sh_down = b >= SDN_WG0 && b < SDN_WG0 + DWG_PER_SLOT;
    const int drow0 = (dunit >= 0 ? dunit % DWG_PER_SLOT : b - SDN_WG0) * DROWS;
    const int dq = lane & 7, dg = lane >> 3;

    // optional phase timestamps (100 MHz real-time counter), thread 0 only
    // They collect in LDS (32-bit offsets from the workgroup's start, the
    // first TR_LAYERS layers) and go to memory once, when the workgroup
    // ends: a store to memory inside the layers would sit in the wave's
    // memory counter, which every later wait for a load also waits on.
#define TR(i)                                                                              \
    if (trace && threadIdx.x == 0 && l < TR_LAYERS)                                        \
        s_tr[l][i] = (uint32_t)(__builtin_amdgcn_s_memrealtime() - t_start) | 0x80000000u;

    // core: rows r0 .. r0+15; wave wv owns r0+4wv .. +3, lane i < 4 keeps the
    // residual value of row r0 + 4wv + i
    const int r0 = b * CROWS;
    // core: the router rows of layer l go straight into LDS, issued by wave
    // 3 alone right after it published x_l (layer 0's before the loop): the
    // HBM is idle then, and waves 0-2, which poll x_l, keep no loads in
    // flight ahead of their polls
    auto load_router_rows = [&](const qmag_moe_layer &Ln) {
#pragma unroll
        for (int j = 0; j < NLOG; j++) {
            const int e = NLOG * b + j;
            if (e < Ln.n_expert) {
                const float4 *row = (const float4 *)(Ln.gate_inp + (size_t)e * N);
#pragma unroll
                for (int k = 0; k < N / 4 / 64; k++)
                    __builtin_amdgcn_global_load_lds((const void *)(row + lane + 64 * k),
                                                     (__attribute__((address_space(3))) void *)&s_wr[j][64 * k],
                                                     16, 0, 0);
            }
        }
    };
    // gate/up helpers: the wave's Q8_K(x_l) operand from the record in LDS,
    // one row pair's raw blocks, and h = silu(gate) * up of a row pair (lanes
    // 0-31 hold the gate dot, 32-63 the up dot)
    constexpr size_t GU_ROW_ = GU_ROW;
    auto gu_load = [&](uint4 &rh, uint4 &q0, uint4 &q1, const uint8_t *slab, int row) {
        const uint8_t *blk = slab + (size_t)row * GU_ROW_ + (size_t)gib * Q4K_BYTES;
        rh = ld16(blk);
        q0 = ld16(blk + 16 + 32 * gg);
        q1 = ld16(blk + 32 + 32 * gg);
    };
    auto load_act = [&](Q4Act &a) {
        const uint4 *xw = s_xrec + (gib * QK_K + 64 * gg) / 16;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 w = xw[k];
            a.x[4 * k + 0] = w.x;
            a.x[4 * k + 1] = w.y;
            a.x[4 * k + 2] = w.z;
            a.x[4 * k + 3] = w.w;
        }
        a.xd = ((const float *)s_xrec)[XR_D + gib];
        const int *sp = (const int *)s_xrec + XR_S + gib * 16 + 4 * gg;
        a.sx0 = (float)(sp[0] + sp[1]);
        a.sx1 = (float)(sp[2] + sp[3]);
    };
    auto swiglu = [&](const Q4Act &a, const uint4 &rh, const uint4 &q0, const uint4 &q1) {
        float v = q4_task(rh, q0, q1, a, gg);
        v = group_sum<32>(v);
        auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        const float u = __uint_as_float(pr[1]);
        return (v / (1.0f + expf(-v))) * u;
    };
    // the routed experts' gate/up row pairs of this wave: requested, then
    // computed and published (one store for all)
    auto routed_gate_up = [&](const qmag_moe_layer &L, int K, uint32_t seq) {
        const uint8_t *const ge = (const uint8_t *)L.gate_exps, *const ue = (const uint8_t *)L.up_exps;
        uint4 gh[MAX_RP], g0[MAX_RP], g1[MAX_RP];
#pragma unroll
        for (int j = 0; j < MAX_RP; j++) {
            gh[j] = g0[j] = g1[j] = make_uint4(0, 0, 0, 0);
            const int rp = gw + j * GU_WAVES, slot = rp / F;
            if (rp < K * F) gu_load(gh[j], g0[j], g1[j], (half ? ue : ge) + (size_t)s_sel[slot] * GU_SLAB, rp % F);
        }
        Q4Act a;
        load_act(a);
        float my_h = 0.0f;
#pragma unroll
        for (int j = 0; j < MAX_RP; j++) {
            if (gw + j * GU_WAVES < K * F) {           // wave-uniform
                const float hv = swiglu(a, gh[j], g0[j], g1[j]);
                if (lane == j) my_h = hv;
            }
        }
        if (lane < MAX_RP && gw + lane * GU_WAVES < K * F)
            st64(rs, TW_H + gw + lane * GU_WAVES, __float_as_uint(my_h), seq);
    };

    if (core) {
        // ================================================================ core
        float xres = lane < WROWS ? x[r0 + WROWS * wv + lane] : 0.0f;
        if (wv == 3) load_router_rows(layers[0]);

        for (int l = 0; l < n_layer; l++) {
            const qmag_moe_layer &L = layers[l];
            const int E = L.n_expert, K = L.n_used, S = K + 1;
            const uint32_t seq = epoch * 256u + (uint32_t)l + 1u;
            const bool last = l + 1 == n_layer;
            TR(0);

            // ---- x_l.  Waves 0-2 poll (wave 3 published this workgroup's
            // rows last layer; a wave's loads wait for its earlier stores)
            bool ok = true;
            if (l == 0) {
#pragma unroll
                for (int k = 0; k < 2; k++) s_x[tid + 256 * k] = ((const float4 *)x)[tid + 256 * k];
            } else if (wv < 3) {
                uint32_t v[6][2];
                auto xp = [&](int k) {
                    const int p = tid + 192 * k;         // word pair
                    return p < N / 2 ? 4 * p + 3 : -1;
                };
                // one word of another workgroup's rows first: bulk polls
                // from every core workgroup during the wait would load the
                // memory system the other hand-offs share
                {
                    uint32_t g1[1];
                    ok = poll<1>(tg->x, [&](int) { return lane == 0 ? ((b + CORE / 2) % CORE) * CROWS + CROWS - 1 : -1; },
                                 seq, g1, ab);
                }
                ok = ok && pollq<6>(rs, TW_X, xp, seq, v, ab);
#pragma unroll
                for (int k = 0; k < 6; k++)
                    if (xp(k) >= 0)
                        ((float2 *)s_x)[xp(k) >> 2] = make_float2(__uint_as_float(v[k][0]), __uint_as_float(v[k][1]));
            }
            drain();                 // router rows have landed in LDS
            if (!wg_all(ok && !(l == 0 && pre_abort), s_vote, 0)) return;
            TR(1);

            // ---- logits (waves 0, 1, each published in every replica), then
            // this workgroup's own copy of the Q8_K(x_l) record (4 blocks
            // each); Q8_K(x) block b and its shared-gate partial published
            // (wave 2, b < 8); softmax/top-K (wave 3)
            if (wv < NLOG) {
                const int lw = wv;
                const int e = NLOG * b + lw;
                if (e < E) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float4 xa = s_x[lane + 64 * j], w = s_wr[lw][lane + 64 * j];
                        s += w.x * xa.x + w.y * xa.y + w.z * xa.z + w.w * xa.w;
                    }
                    s = group_sum<64>(s);
                    if (L.router_bias) s += ldg(L.router_bias + e);
                    if (lane < REP) st64(rs, TW_LOGITS + lane * 256 + logit_pos(e), __float_as_uint(s), seq);
                    if (last && lane == 0) g_logits[e] = s;
                }
#pragma unroll
                for (int k = 0; k < NBE / 2; k++) {
                    const int blk = lw * (NBE / 2) + k;
                    const Q8Lane q = q8k_quant_lane(s_x[blk * 64 + lane]);
                    ((uint32_t *)s_xrec)[blk * 64 + lane] = q.packed;
                    if ((lane & 3) == 0) ((int *)s_xrec)[XR_S + blk * 16 + (lane >> 2)] = q.gsum;
                    if (lane == 0) ((float *)s_xrec)[XR_D + blk] = q.d;
                }
            } else if (wv == 2 && b < NBE) {
                const Q8Lane q = q8k_quant_lane(s_x[b * 64 + lane]);
                const float4 wsh = ldg4(L.gate_inp_shexp + 4 * (b * 64 + lane));
                const int8_t *q8 = (const int8_t *)&q.packed;
                float g = wsh.x * (float)q8[0] * q.d + wsh.y * (float)q8[1] * q.d +
                          wsh.z * (float)q8[2] * q.d + wsh.w * (float)q8[3] * q.d;
                g = group_sum<64>(g);
#pragma nounroll
                for (int r = 0; r < REP; r++) {
                    const int o = TW_XQ + r * XR_WORDS;
                    st64(rs, o + b * 64 + lane, q.packed, seq);
                    if ((lane & 3) == 0) st64(rs, o + XR_S + b * 16 + (lane >> 2), (uint32_t)q.gsum, seq);
                    if (lane == 0) st64(rs, o + XR_D + b, __float_as_uint(q.d), seq);
                    if (lane == 1) st64(rs, o + XR_G + b, __float_as_uint(g), seq);
                }
            } else if (wv == 3) {
                float lg[4];
                ok = read_logits(E, seq, lg);
                int my_sel = 0;
                float my_w = 0.0f;
                // the picks are a chain of dependent wave reductions: issue
                // them ahead of the other wave sharing this SIMD
                __builtin_amdgcn_s_setprio(3);
                route_topk(lg, E, K, my_sel, my_w);
                __builtin_amdgcn_s_setprio(0);
                if (lane < K) {
                    s_sel[lane] = my_sel;
                    s_w[lane] = my_w;
                    if (last && b == 0) {
                        g_sel[lane] = my_sel;
                        g_w[lane] = my_w;
                    }
                }
            }
            if (!wg_all(ok, s_vote, 1)) return;
            TR(2);

            routed_gate_up(L, K, seq);
            TR(4);

            // ---- the down outputs of this workgroup's rows, every slot
            // (thread t < 8S: slot t/8, rows r0 + 2(t%8) + {0,1}), and the 8
            // shared-gate partials (4 more pairs)
            if (wv < 2) {
                uint32_t v[1][2];
                auto yp = [&](int) {
                    if (tid < 8 * S) return 4 * ((TW_Y + (tid >> 3) * N + r0) / 2 + (tid & 7)) + 3;
                    if (tid < 8 * S + NBE / 2) return 4 * ((TW_XQ + rep * XR_WORDS + XR_G) / 2 + tid - 8 * S) + 3;
                    return -1;
                };
                ok = pollq<1>(rs, 0, yp, seq, v, ab);
                if (tid < 8 * S) {
                    s_dres[2 * (tid & 7)][tid >> 3] = __uint_as_float(v[0][0]);
                    s_dres[2 * (tid & 7) + 1][tid >> 3] = __uint_as_float(v[0][1]);
                } else if (tid < 8 * S + NBE / 2) {
                    s_gsp[2 * (tid - 8 * S)] = __uint_as_float(v[0][0]);
                    s_gsp[2 * (tid - 8 * S) + 1] = __uint_as_float(v[0][1]);
                }
            }
            if (!wg_all(ok, s_vote, 2)) return;
            TR(5);

            // ---- combine in the reference order (nn.c:614-629)
            if (lane < WROWS) {
                float g = 0.0f;
#pragma unroll
                for (int k = 0; k < NBE; k++) g += s_gsp[k];
                const float gs = 1.0f / (1.0f + expf(-g));
                if (last && b == 0 && wv == 0 && lane == 0) g_gs[0] = gs;
                const float *dres = s_dres[WROWS * wv + lane];
                float acc = 0.0f;
                for (int k = 0; k < K; k++) acc = __fadd_rn(acc, __fmul_rn(s_w[k], dres[k]));
                acc = __fadd_rn(acc, __fmul_rn(gs, dres[K]));
                if (out) {
                    out[r0 + WROWS * wv + lane] = acc;
                } else {
                    xres = __fadd_rn(acc, xres);
                    s_xout[WROWS * wv + lane] = xres;
                }
            }
            __syncthreads();
            // wave 3 publishes the workgroup's 16 rows with one store
            if (!out && wv == 3 && lane < CROWS) {
                if (!last) st64(rs, TW_X + r0 + lane, __float_as_uint(s_xout[lane]), seq + 1u);
                else x[r0 + lane] = s_xout[lane];
            }
            if (!last && wv == 3) load_router_rows(layers[l + 1]);    // this layer's rows are consumed
            TR(6);
        }
    } else {
        // ============================================================== stream
        for (int l = 0; l < n_layer; l++) {
            const qmag_moe_layer &L = layers[l];
            const int E = L.n_expert, K = L.n_used, S = K + 1;
            const uint32_t seq = epoch * 256u + (uint32_t)l + 1u;
            const bool last = l + 1 == n_layer;
            TR(0);

            // ---- rows that do not depend on the selection: in the shared
            // slot's down workgroups their down rows, requested at layer
            // start; the shared expert's gate/up row pairs follow once x_l is
            // published (below), so that they do not compete with the core's
            // reads for the router and the logits
            uint4 sh_h = make_uint4(0, 0, 0, 0), sh_0 = sh_h, sh_1 = sh_h;
            const int dslot = dunit >= 0 ? dunit / DWG_PER_SLOT : sh_down ? K : S;   // S: no down role
            const bool down = dslot < S && (dunit < 0 || dslot < K);
            DRaw<TD> dr[DN_ROUNDS];
            auto dn_load = [&](const uint8_t *slab) {
#pragma unroll
                for (int j = 0; j < DN_ROUNDS; j++) d_load<TD>(dr[j], slab, drow0 + 16 * wv + 8 * j + dg, dq);
            };
            if (sh_down) dn_load((const uint8_t *)L.down_shexp);

            bool ok = true;
            // ---- softmax/top-K (wave 0); meanwhile waves 2, 3 each fetch the
            // whole Q8_K(x_l) record, published with the logits, and the
            // shared-expert row pair among them is computed and published at
            // once.  These workgroups wait here through the core's part of the
            // layer: one word first.
            if (wv == 0) {
                uint32_t g1[1];
                ok = poll<1>(tg->logits[rep], [&](int) { return lane == 0 ? logit_pos((b * 37) % E) : -1; }, seq, g1,
                             ab);
                float lg[4];
                ok = ok && read_logits(E, seq, lg);
                TR(7);
                int my_sel = 0;
                float my_w = 0.0f;
                __builtin_amdgcn_s_setprio(3);        // as in the core workgroups
                route_topk(lg, E, K, my_sel, my_w);
                __builtin_amdgcn_s_setprio(0);
                if (lane < K) s_sel[lane] = my_sel;
                TR(6);
            } else if (wv >= 2) {
                uint32_t g1[1];
                ok = poll<1>(tg->xq[rep], [&](int) { return lane == 0 ? XR_G + (b & 7) : -1; }, seq, g1, ab);
                if (sh_row < F) gu_load(sh_h, sh_0, sh_1, (const uint8_t *)(half ? L.up_shexp : L.gate_shexp), sh_row);
                constexpr int XP = (XR_WORDS / 2 + 63) / 64;   // 6 word pairs per lane
                uint32_t v[XP][2];
                auto xp = [&](int k) {
                    const int p = lane + 64 * k;       // word pair (the whole record is written)
                    return p < XR_WORDS / 2 ? 4 * p + 3 : -1;
                };
                ok = ok && pollq<XP>(rs, TW_XQ + rep * XR_WORDS, xp, seq, v, ab);
#pragma unroll
                for (int k = 0; k < XP; k++)
                    if (xp(k) >= 0) ((uint2 *)s_xrec)[xp(k) >> 2] = make_uint2(v[k][0], v[k][1]);
                if (sh_row < F) {
                    Q4Act a;
                    load_act(a);
                    const float hv = swiglu(a, sh_h, sh_0, sh_1);
                    if (lane == 0) st64(rs, TW_H + K * F + sh_row, __float_as_uint(hv), seq);
                }
            }
            if (!wg_all(ok && !(l == 0 && pre_abort), s_vote, 1)) return;
            TR(2);
            // the shared registers count as read on every path from here on,
            // so no later write into them has to wait for the load queue
            __asm__ volatile("" ::"v"(sh_h.x), "v"(sh_0.x), "v"(sh_1.x));

            routed_gate_up(L, K, seq);
            TR(4);

            if (down) {
                // ---- a routed slot's down rows, requested only now that the
                // gate/up data is in: issued together with it they would share the
                // HBM with the requests h is waiting for.  They land while the
                // slot's h is gathered.
                if (dslot < K) dn_load((const uint8_t *)L.down_exps + (size_t)s_sel[dslot] * DN_SLAB);
                // ---- h of slot dslot: 256 word pairs, one per thread
                {
                    uint32_t v[1][2];
                    if (wv == 0) {                    // one word first, as for x
                        uint32_t g1[1];
                        ok = poll<1>(tg->h + dslot * F, [&](int) { return lane == 0 ? F - 1 - (b % 64) : -1; }, seq, g1,
                                     ab);
                    }
                    if (!wg_all(ok, s_vote, 0)) return;
                    ok = pollq<1>(rs, TW_H + dslot * F, [&](int) { return 4 * tid + 3; }, seq, v, ab);
                    ((float2 *)s_hs)[tid] = make_float2(__uint_as_float(v[0][0]), __uint_as_float(v[0][1]));
                }
                if (!wg_all(ok, s_vote, 3)) return;
                // ---- Q8_K(h): waves 0 and 1 quantise one block each
                if (wv < NBF) {
                    const Q8Lane q = q8k_quant_lane(s_hs[wv * 64 + lane]);
                    ((uint32_t *)s_hq)[wv * 64 + lane] = q.packed;
                    if ((lane & 3) == 0) ((int *)s_hq)[HS_S + wv * 16 + (lane >> 2)] = q.gsum;
                    if (lane == 0) ((float *)s_hq)[HS_D + wv] = q.d;
                }
                if (last && drow0 == 0) ((float2 *)g_h)[dslot * (F / 2) + tid] = ((const float2 *)s_hs)[tid];
                __syncthreads();
                TR(5);
                // ---- down dots of the wave's 16 rows; y published per row
#pragma unroll
                for (int j = 0; j < DN_ROUNDS; j++) {
                    float v = d_dot<TD>(dr[j], (const uint32_t *)s_hq, (const float *)s_hq + HS_D,
                                        (const int *)s_hq + HS_S, dq);
                    v = group_sum<8>(v);
                    if (dq == 0) st64(rs, TW_Y + dslot * N + drow0 + 16 * wv + 8 * j + dg, __float_as_uint(v), seq);
                }
                TR(1);
            }

            // LDS is rewritten next layer only after this barrier
            __syncthreads();
        }
    }
    if (trace && threadIdx.x == 0) {
        const int nl = n_layer < TR_LAYERS ? n_layer : TR_LAYERS;
        for (int l = 0; l < nl; l++)
            for (int i = 0; i < 8; i++) {
                const uint32_t v = s_tr[l][i];        // set stamps have the top bit
                if (v) trace[((size_t)b * n_layer + l) * 8 + i] = t_start + (v & 0x7fffffffu);
            }
    }
#undef TR
}

}  // namespace fused

// ------------------------------------------------------------------ host --
static qmag_moe_layer *g_dev_layers = nullptr;
static qmag_moe_layer g_host_copy[256];
static int g_host_n = 0;
// one-layer calls (the moe_ffn seam, one layer per call, rotating over a
// model's layers) keep every distinct descriptor resident in its own slot:
// uploaded the first time it is seen, found by a hash of its bytes after
constexpr int ONE_SLOTS = 256, ONE_HASH = 1024;
static qmag_moe_layer *g_dev_one = nullptr;
static qmag_moe_layer g_one_host[ONE_SLOTS];
static int g_one_n = 0;
static short g_one_table[ONE_HASH];         // slot + 1, 0 = empty (linear probing)
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
        // One tagged slot per buffer is safe only if every workgroup that
        // reads a layer's words lies on that layer's dependency chain; with
        // n_used >= 4 every wave has a routed gate/up row pair, so it does.
        // With fewer, some workgroups read the logits and feed nothing, and
        // in a multi-layer launch the next layer could overwrite the words
        // before they read them.  One-layer launches are safe for any n_used.
        if (n_layer > 1 && a.n_used < 4) return false;
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

static bool g_pending = false;       // a launch was issued since the last fused_status()
bool fused_pending() { return g_pending; }

// Recovery log: the calls issued since the last status check.  If a wait
// of launch e expired, launch e left its output partly written and every
// later launch exited at its first barrier without writing any; the calls
// are then re-run from launch e on through the launch sequence, in-place
// calls first restored from the copy of their input taken before they ran.
struct FusedCall {
    size_t layer0 = 0;                    // the call's descriptors: g_log_layers[layer0 .. + n_layer)
    int n_layer = 0;
    float *x = nullptr, *out = nullptr;   // out == nullptr: the stack (x updated in place)
    int n_tok = 0;
    int lpt = 1;                          // persistent launches per token (fused runs of a mixed stack)
    unsigned first_epoch = 0;             // epoch of the call's first launch (token 0)
    int snap = -1;                        // snapshot slot holding the input rows, or -1
};
// At most LOG_CALLS calls, SNAP_SLOTS of them in place, between status
// checks; a call that would exceed either first checks (a stream sync, so
// it is kept rare: a one-layer call adds one entry and one descriptor to
// storage whose capacity persists, no allocation per call).
constexpr int LOG_CALLS = 16384, SNAP_SLOTS = 8;
static std::vector<FusedCall> g_log;
static std::vector<qmag_moe_layer> g_log_layers;
static int g_snap_used = 0;
static float *g_snap[SNAP_SLOTS] = {};
static size_t g_snap_bytes[SNAP_SLOTS] = {};
static long g_recovered = 0;
static int g_test_abort = 0;

// append a call to the log; its descriptors are shared with the previous
// entry when they are the same (a stack decoded step after step)
static void log_call(FusedCall &c, const qmag_moe_layer *L, int n_layer)
{
    c.n_layer = n_layer;
    if (!g_log.empty() && g_log.back().n_layer == n_layer &&
        memcmp(g_log_layers.data() + g_log.back().layer0, L, sizeof(qmag_moe_layer) * (size_t)n_layer) == 0) {
        c.layer0 = g_log.back().layer0;
    } else {
        c.layer0 = g_log_layers.size();
        g_log_layers.insert(g_log_layers.end(), L, L + n_layer);
    }
    g_log.push_back(c);
}

static int replay(const std::vector<FusedCall> &log, const std::vector<qmag_moe_layer> &layers, unsigned e,
                  hipStream_t s)
{
    const size_t N = fused::N;
    for (const FusedCall &c : log) {
        if (c.first_epoch + (unsigned)(c.n_tok * c.lpt) <= e) continue;   // finished before launch e
        const int t0 = e > c.first_epoch ? (int)((e - c.first_epoch) / (unsigned)c.lpt) : 0;
        const size_t rows = (size_t)(c.n_tok - t0) * N;
        if (c.snap >= 0)
            QMAG_HIP(hipMemcpyAsync(c.x + t0 * N, g_snap[c.snap] + t0 * N, sizeof(float) * rows,
                                    hipMemcpyDeviceToDevice, s));
        const qmag_moe_layer *cl = layers.data() + c.layer0;
        for (int t = t0; t < c.n_tok; t++) {
            float *xt = c.x + t * N;
            if (!c.out) {
                for (int l = 0; l < c.n_layer; l++) {
                    int st = moe_ffn(&cl[l], xt, xt, 1, xt, s);
                    if (st) return st;
                }
            } else {
                int st = moe_ffn(&cl[0], xt, c.out + t * N, 1, nullptr, s);
                if (st) return st;
            }
        }
    }
    moe_note_sequence_ran();
    QMAG_HIP(hipStreamSynchronize(s));
    return QMAG_OK;
}

// the status once the abort word has been read (the stream synchronised)
static int status_of_word(int word)
{
    g_snap_used = 0;
    if (word == 0) {                 // the common case: keep the storage's capacity
        g_log.clear();
        g_log_layers.clear();
        return QMAG_OK;
    }
    std::vector<FusedCall> log;
    std::vector<qmag_moe_layer> layers;
    log.swap(g_log);
    layers.swap(g_log_layers);
    int st = rearm();
    if (st) return st;
    st = replay(log, layers, (unsigned)word - 1u, ctx().stream);
    if (st) return st;
    g_recovered++;
    return QMAG_OK;
}

int fused_status()
{
    g_pending = false;
    if (!g_abort) {
        g_log.clear();
        g_log_layers.clear();
        g_snap_used = 0;
        return QMAG_OK;
    }
    QMAG_HIP(hipStreamSynchronize(ctx().stream));
    int word = 0;
    QMAG_HIP(hipMemcpy(&word, g_abort, sizeof(int), hipMemcpyDeviceToHost));
    return status_of_word(word);
}

// For a caller that synchronises the stream anyway: the abort word is
// copied into host memory (pinned) on the stream behind the launches, and
// fused_status_word takes it after the synchronisation instead of reading
// it with a second round trip.  No persistent launch yet: the word is 0.
int fused_abort_copy(int *host, hipStream_t s)
{
    if (!g_abort) {
        *host = 0;
        return QMAG_OK;
    }
    QMAG_HIP(hipMemcpyAsync(host, g_abort, sizeof(int), hipMemcpyDeviceToHost, s));
    return QMAG_OK;
}

int fused_status_word(int word)
{
    g_pending = false;
    if (!g_abort) {
        g_log.clear();
        g_log_layers.clear();
        g_snap_used = 0;
        return QMAG_OK;
    }
    return status_of_word(word);
}

long fused_recoveries() { return g_recovered; }
void fused_test_abort_next(int nth) { g_test_abort = nth > 0 ? nth : 0; }

static uint32_t layer_hash(const qmag_moe_layer *L)
{
    const unsigned char *p = (const unsigned char *)L;
    uint32_t h = 2166136261u;                       // FNV-1a over the descriptor bytes
    for (size_t i = 0; i < sizeof(qmag_moe_layer); i++) h = (h ^ p[i]) * 16777619u;
    return h;
}

// device copy of a one-layer descriptor, uploading it on first sight
static int one_layer_slot(const qmag_moe_layer *L, hipStream_t s, const qmag_moe_layer **dl)
{
    uint32_t i = layer_hash(L) % ONE_HASH;
    for (; g_one_table[i]; i = (i + 1) % ONE_HASH) {
        const int slot = g_one_table[i] - 1;
        if (memcmp(&g_one_host[slot], L, sizeof(qmag_moe_layer)) == 0) {
            *dl = g_dev_one + slot;
            return QMAG_OK;
        }
    }
    if (g_one_n == ONE_SLOTS) {                    // full: start over (launches in flight may read slots)
        QMAG_HIP(hipStreamSynchronize(s));
        g_one_n = 0;
        memset(g_one_table, 0, sizeof(g_one_table));
        for (i = layer_hash(L) % ONE_HASH; g_one_table[i]; i = (i + 1) % ONE_HASH) {}
    }
    const int slot = g_one_n++;
    QMAG_HIP(hipMemcpy(g_dev_one + slot, L, sizeof(qmag_moe_layer), hipMemcpyHostToDevice));
    g_one_host[slot] = *L;
    g_one_table[i] = (short)(slot + 1);
    *dl = g_dev_one + slot;
    return QMAG_OK;
}

static int fused_prepare(const qmag_moe_layer *L, int n_layer, hipStream_t s, const qmag_moe_layer **dl)
{
    if (!g_dev_layers) {
        QMAG_HIP(hipMalloc(&g_dev_layers, sizeof(qmag_moe_layer) * 256));
        QMAG_HIP(hipMalloc(&g_dev_one, sizeof(qmag_moe_layer) * ONE_SLOTS));
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
    if (n_layer == 1) {
        int st = one_layer_slot(L, s, dl);
        if (st) return st;
    } else {
        if (g_host_n != n_layer || memcmp(g_host_copy, L, sizeof(qmag_moe_layer) * (size_t)n_layer) != 0) {
            QMAG_HIP(hipStreamSynchronize(s));
            QMAG_HIP(hipMemcpy(g_dev_layers, L, sizeof(qmag_moe_layer) * (size_t)n_layer, hipMemcpyHostToDevice));
            memcpy(g_host_copy, L, sizeof(qmag_moe_layer) * (size_t)n_layer);
            g_host_n = n_layer;
        }
        *dl = g_dev_layers;
    }
    if (option(QMAG_OPT_TRACE)) {
        const size_t need = sizeof(unsigned long long) * fused::WGS * (size_t)n_layer * 8;
        if (need > g_trace_bytes) {
            QMAG_HIP(hipStreamSynchronize(s));
            if (g_trace) QMAG_HIP(hipFree(g_trace));
            QMAG_HIP(hipMalloc(&g_trace, need));
            g_trace_bytes = need;
        }
        // phases a workgroup does not pass through read back as 0
        QMAG_HIP(hipMemsetAsync(g_trace, 0, need, s));
    } else if (g_trace) {
        QMAG_HIP(hipStreamSynchronize(s));
        QMAG_HIP(hipFree(g_trace));
        g_trace = nullptr;
        g_trace_bytes = 0;
    }
    return QMAG_OK;
}

static int fused_launch(const qmag_moe_layer *L, const qmag_moe_layer *dl, int n_layer, float *x, float *out,
                        hipStream_t s)
{
    unsigned epoch = g_epoch;
    if (g_test_abort > 0 && --g_test_abort == 0) {   // test hook: this launch finds the abort word set
        static int code;
        code = (int)epoch + 1;
        QMAG_HIP(hipMemcpyAsync(g_abort, &code, sizeof(int), hipMemcpyHostToDevice, s));
        QMAG_HIP(hipStreamSynchronize(s));
    }
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
    g_pending = true;
    return QMAG_OK;
}

// copy n_tok input rows at x into the next snapshot slot (grown as needed)
static int take_snapshot(const float *x, int n_tok, hipStream_t s, int *slot_out)
{
    const int slot = g_snap_used++;
    const size_t need = sizeof(float) * fused::N * (size_t)n_tok;
    if (need > g_snap_bytes[slot]) {
        QMAG_HIP(hipStreamSynchronize(s));
        if (g_snap[slot]) QMAG_HIP(hipFree(g_snap[slot]));
        g_snap[slot] = nullptr;
        g_snap_bytes[slot] = 0;
        QMAG_HIP(hipMalloc(&g_snap[slot], need));
        g_snap_bytes[slot] = need;
    }
    QMAG_HIP(hipMemcpyAsync(g_snap[slot], x, need, hipMemcpyDeviceToDevice, s));
    *slot_out = slot;
    return QMAG_OK;
}

int fused_call(const qmag_moe_layer *L, int n_layer, float *x, float *out, int n_tok, hipStream_t s)
{
    if (out && n_layer != 1) return fail(QMAG_ERR_ARG, "fused: out mode needs exactly one layer");
    if (n_tok <= 0 || n_tok >= (1 << 23)) return fail(QMAG_ERR_ARG, "fused: n_tok=%d", n_tok);
    const bool wraps = g_epoch + (unsigned)n_tok >= (1u << 24);     // tags would wrap
    const bool in_place = !out || out == x;
    if (g_log.size() >= (size_t)LOG_CALLS || (in_place && g_snap_used == SNAP_SLOTS) || wraps) {
        int st = fused_status();
        if (st) return st;
        if (wraps) {
            st = rearm();
            if (st) return st;
        }
    }
    const qmag_moe_layer *dl = nullptr;
    int st = fused_prepare(L, n_layer, s, &dl);
    if (st) return st;
    FusedCall c;
    c.x = x;
    c.out = out;
    c.n_tok = n_tok;
    c.first_epoch = g_epoch;
    if (in_place) {                     // keep the input to replay from
        st = take_snapshot(x, n_tok, s, &c.snap);
        if (st) return st;
    }
    log_call(c, L, n_layer);
    for (int t = 0; t < n_tok; t++) {
        st = fused_launch(L, dl, n_layer, x + (size_t)t * fused::N, out ? out + (size_t)t * fused::N : nullptr, s);
        if (st) return st;
    }
    return QMAG_OK;
}

// A stack the persistent kernel cannot take whole (down types that change
// from layer to layer, a shared expert typed apart from the routed ones):
// the maximal runs of consecutive layers it can take go through it, the other
// layers through the launch sequence, token by token in layer order.  The
// whole stack's descriptors are uploaded once and each run reads its slice.
// One log entry and one input snapshot cover a whole call (up to 2^22
// persistent launches; a longer call is cut into such chunks of tokens):
// token t's nf persistent launches are consecutive epochs, so an expired wait
// of epoch e replays tokens (e - first) / nf on through the launch sequence,
// each through the whole stack.  Returns 1 (nothing launched) when no layer
// qualifies.
int fused_stack_runs(const qmag_moe_layer *L, int n_layer, float *x, int n_tok, hipStream_t s)
{
    if (n_layer < 2 || n_layer > 256) return 1;
    std::vector<int> rb, re;
    std::vector<char> rf;
    for (int b = 0; b < n_layer;) {
        int e = b + 1;
        const bool f = fused_eligible(L + b, 1);
        if (f)
            while (e < n_layer && fused_eligible(L + b, e + 1 - b)) e++;
        else
            while (e < n_layer && !fused_eligible(L + e, 1)) e++;
        rb.push_back(b);
        re.push_back(e);
        rf.push_back(f);
        b = e;
    }
    int nf = 0;
    for (char f : rf) nf += f;
    if (nf == 0) return 1;
    if (n_tok <= 0 || n_tok >= (1 << 23)) return fail(QMAG_ERR_ARG, "fused: n_tok=%d", n_tok);
    const qmag_moe_layer *dl = nullptr;
    int st = fused_prepare(L, n_layer, s, &dl);
    if (st) return st;
    const int chunk = (1 << 22) / nf;
    for (int t0 = 0; t0 < n_tok; t0 += chunk) {
        const int nt = n_tok - t0 < chunk ? n_tok - t0 : chunk;
        float *xc = x + (size_t)t0 * fused::N;
        const bool wraps = g_epoch + (unsigned)(nt * nf) >= (1u << 24);
        if (g_log.size() >= (size_t)LOG_CALLS || g_snap_used == SNAP_SLOTS || wraps) {
            st = fused_status();
            if (st) return st;
            if (wraps) {
                st = rearm();
                if (st) return st;
            }
        }
        FusedCall c;
        c.x = xc;
        c.n_tok = nt;
        c.lpt = nf;
        c.first_epoch = g_epoch;
        st = take_snapshot(xc, nt, s, &c.snap);
        if (st) return st;
        log_call(c, L, n_layer);
        for (int t = 0; t < nt; t++) {
            float *xt = xc + (size_t)t * fused::N;
            for (size_t r = 0; r < rb.size(); r++) {
                if (rf[r]) {
                    st = fused_launch(L + rb[r], dl + rb[r], re[r] - rb[r], xt, nullptr, s);
                    if (st) return st;
                } else {
                    for (int l = rb[r]; l < re[r]; l++) {
                        st = moe_ffn(&L[l], xt, xt, 1, xt, s);
                        if (st) return st;
                    }
                }
            }
        }
    }
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
