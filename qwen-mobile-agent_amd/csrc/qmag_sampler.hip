// qmag_sampler.hip -- sampling on the device (src/sampler.c:36-134), so the
// LM head's logits (151,936 floats) never leave HBM.
//
// sampler_candidates: the repeat penalty (per occurrence in last_tokens:
// negative logits multiplied, others divided), division by the temperature,
// then the k largest values in descending order.  sampler_pick: the softmax
// over the live candidates with a double sum, the top-p cut, one xorshift64*
// draw and the cumulative pick, and the pick's entry into last_tokens.
//
// One launch of one workgroup per 4096 logits.  Each workgroup applies the
// penalty and the temperature to its logits and selects its k largest over
// unique 64-bit keys (the value's order-preserving bits with -0 folded into
// +0, then the complemented index, so equal values order by ascending index,
// and a bit that restores a zero's sign in the reported value): the value
// half of the k-th largest of the threads' maxima bounds the answer from
// below, and the few keys that reach it are sorted by one wave's bitonic
// network (an exact radix select takes over when more than 128 reach it).
// The last workgroup to finish (a device-scope counter) selects the k
// largest of all chunks' candidates the same way and, in the sampling form,
// makes the pick with the reference's arithmetic, the candidates one per
// lane: the sequential sums become per-lane prefixes in the same order, and
// each cut one ballot.  Results are written straight to pinned host memory.
//
// Among exactly equal values the lower index comes first.  The reference
// keeps its candidates in a min-heap and sorts them with qsort, so which of
// several equal values at the k-th place it keeps, and their order, depends
// on the heap; for distinct values the two agree exactly.  NaN logits sort
// after every number here; the reference's comparisons leave their place to
// the heap's history.
#include <limits.h>
#include <string.h>

#include <mutex>

#include "qmag_internal.h"

namespace qmag {

constexpr int SAMP_CHUNK = 4096;            // logits per workgroup
constexpr int SAMP_PER_THREAD = SAMP_CHUNK / 256;
constexpr int SAMP_MAX_K = 64;
constexpr int SAMP_MERGE_PER_THREAD = 32;   // the last workgroup's share of n_chunks * k
constexpr int SAMP_MAX_CHUNKS = 256 * SAMP_MERGE_PER_THREAD / SAMP_MAX_K;   // 128
constexpr int SAMP_MAX_VOCAB = SAMP_MAX_CHUNKS * SAMP_CHUNK;               // 524,288

// the repeat penalty's distinct last-token ids with their occurrence counts
struct SampParams {
    float temp;
    float repeat_penalty;
    int n_uniq;
    int uniq[64];
    int count[64];
};

// value order as unsigned order: larger key = larger value; NaN lowest of
// the numbers' keys (1), 0 = no element
__device__ __forceinline__ uint32_t samp_key(float v)
{
    if (v != v) return 1u;
    const uint32_t b = __float_as_uint(v + 0.0f);        // -0 folded to +0
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return k < 2u ? 2u : k;
}
__device__ __forceinline__ float samp_val(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// unique selection key: the value half, then the complemented index shifted
// up one bit (ids are below 2^31, so the dropped top bit is 1 for all and the
// order among ids is kept); the low bit is the sign of a zero value, which
// the value half folds into +0 (the reference compares -0 and +0 as equal),
// so it never decides an order and only restores the reported value
__device__ __forceinline__ uint64_t samp_comp(uint32_t key, int id, float v)
{
    const uint32_t neg_zero = __float_as_uint(v) == 0x80000000u ? 1u : 0u;
    return ((uint64_t)key << 32) | ((uint32_t)~(uint32_t)id << 1) | neg_zero;
}
__device__ __forceinline__ int samp_id(uint64_t c) { return (int)~(((uint32_t)c >> 1) | 0x80000000u); }
__device__ __forceinline__ float samp_value(uint64_t c)
{
    return (c & 1u) ? -0.0f : samp_val((uint32_t)(c >> 32));
}

// The value of lane (lane ^ m), m one of 1, 2, 4, 8, 16, 32 (a constant once
// the callers' loops are unrolled), by DPP moves and the gfx950 lane swaps
// instead of the LDS crossbar: xor 4 is a half-row mirror (xor 7) then a
// quad reversal (xor 3), xor 8 a row mirror (xor 15) then a half-row mirror.
constexpr int DPP_XOR3 = 0x1B;          // quad_perm [3,2,1,0]
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int m)
{
    const int x = (int)v;
    switch (m) {
    case 1: return (uint32_t)dpp_i<DPP_XOR1>(x);
    case 2: return (uint32_t)dpp_i<DPP_XOR2>(x);
    case 4: return (uint32_t)dpp_i<DPP_XOR3>(dpp_i<DPP_HALF_MIRROR>(x));
    case 8: return (uint32_t)dpp_i<DPP_HALF_MIRROR>(dpp_i<DPP_MIRROR>(x));
    case 16: {
        // rows 1, 3 of the first result hold rows 0, 2; rows 0, 2 of the
        // second hold rows 1, 3
        auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? p[0] : p[1];
    }
    default: {
        auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? p[0] : p[1];
    }
    }
}
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m)
{
    const uint32_t lo = xor_lane((uint32_t)v, m), hi = xor_lane((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}
// a uniform lane's value
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int src)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}

// inclusive prefix sum over the 64 lanes of a wave: a butterfly in which the
// upper half of each block of 2d lanes adds the lower half's total
__device__ __forceinline__ int wave_incl_scan(int v)
{
    const int lane = lane_id();
    int tot = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = (int)xor_lane((uint32_t)tot, d);
        v += (lane & d) ? o : 0;
        tot += o;
    }
    return v;
}

// exclusive prefix sum over the workgroup's 256 threads; s_w: 4 ints
__device__ __forceinline__ int wg_excl_scan(int v, int *s_w, int *total)
{
    const int t = (int)threadIdx.x, w = t >> 6;
    const int incl = wave_incl_scan(v);
    if ((t & 63) == 63) s_w[w] = incl;
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; i++) base += s_w[i];
    *total = s_w[0] + s_w[1] + s_w[2] + s_w[3];
    __syncthreads();
    return base + incl - v;
}

// Marks the `need` largest nonzero keys held across the workgroup (E per
// thread; all keys distinct): after the call sel[j] is set for exactly
// min(need, nonzero count) of them.  s_hist: 256 uints, s_info: 4 ints.
template <int E>
__device__ void wg_select(const uint64_t (&c)[E], int need, bool (&sel)[E], uint32_t *s_hist, int *s_info)
{
    const int t = (int)threadIdx.x;
    uint64_t prefix = 0;
    int L = 0;
    for (int pass = 0; pass < 8 && need > 0; pass++) {
        const int shift = 56 - 8 * pass;
        s_hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < E; j++)
            if (c[j] && (L == 0 || (c[j] >> (64 - L)) == prefix))
                atomicAdd(&s_hist[(uint32_t)(c[j] >> shift) & 255u], 1u);
        __syncthreads();
        if (t < 64) {
            // lane l owns bins 4l .. 4l+3; counts above a bin run from bin 255 down
            const uint32_t h0 = s_hist[4 * t], h1 = s_hist[4 * t + 1], h2 = s_hist[4 * t + 2],
                           h3 = s_hist[4 * t + 3];
            const int local = (int)(h0 + h1 + h2 + h3);
            const int incl = wave_incl_scan(local);
            const int tot = __builtin_amdgcn_readlane(incl, 63);
            int above = tot - incl;                       // bins of the lanes above
            const uint32_t h[4] = {h0, h1, h2, h3};
#pragma unroll
            for (int i = 3; i >= 0; i--) {
                if (above < need && need <= above + (int)h[i]) {
                    s_info[0] = 4 * t + i;
                    s_info[1] = above;
                    s_info[2] = (int)h[i];
                }
                above += (int)h[i];
            }
            if (t == 0 && tot < need) {                   // fewer candidates than asked: all of them
                s_info[0] = -1;
                s_info[1] = tot;
                s_info[2] = 0;
            }
        }
        __syncthreads();
        const int b = s_info[0], above = s_info[1], cnt = s_info[2];
        __syncthreads();
        if (b < 0) {                                      // take every nonzero key
            prefix = 0;
            L = 0;
            break;
        }
        need -= above;
        prefix = (prefix << 8) | (uint64_t)b;
        L += 8;
        if (cnt == need) break;                           // the boundary group is wholly in
    }
#pragma unroll
    for (int j = 0; j < E; j++) {
        if (!c[j]) {
            sel[j] = false;
        } else if (L == 0) {
            sel[j] = true;
        } else {
            const uint64_t top = c[j] >> (64 - L);
            sel[j] = top >= prefix;
        }
    }
}

// wg_select after a cheap pre-filter: the need-th largest of the threads'
// own maxima is a lower bound on the need-th largest key (need threads hold
// a key at least that large), so keys below it cannot be selected; the exact
// selection then runs on the few that remain, with little contention on the
// histogram bins.  s_m: 4 uint64.
template <int E>
__device__ void wg_topk(uint64_t (&c)[E], int need, bool (&sel)[E], uint32_t *s_hist, int *s_info, uint64_t *s_m)
{
    const int t = (int)threadIdx.x;
    uint64_t m[1] = {0ull};
#pragma unroll
    for (int j = 0; j < E; j++) m[0] = c[j] > m[0] ? c[j] : m[0];
    bool ms[1];
    wg_select<1>(m, need, ms, s_hist, s_info);
    // the bound: the smallest selected maximum
    uint64_t lo = ms[0] ? m[0] : ~0ull;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const uint64_t o = shfl_xor64(lo, d);
        lo = o < lo ? o : lo;
    }
    if ((t & 63) == 0) s_m[t >> 6] = lo;
    __syncthreads();
    uint64_t bound = s_m[0];
    for (int w = 1; w < 4; w++) bound = s_m[w] < bound ? s_m[w] : bound;
    // fewer than `need` threads hold keys: the bound would cut keys the
    // selection needs, so keep every key
    if (__syncthreads_count(m[0] != 0ull) < need) bound = 1ull;
#pragma unroll
    for (int j = 0; j < E; j++) c[j] = c[j] >= bound ? c[j] : 0ull;
    wg_select<E>(c, need, sel, s_hist, s_info);
}

// One compare-exchange step of a bitonic network over keys one per lane
// (element index i): descending order overall.
__device__ __forceinline__ uint64_t bitonic_step(uint64_t v, int i, int size, int stride)
{
    const uint64_t o = shfl_xor64(v, stride);
    const bool keep_max = ((i & stride) == 0) == ((i & size) == 0);
    return (v > o) == keep_max ? v : o;          // one compare: equal keys are equal values
}

// 64 keys, one per lane, sorted descending
__device__ __forceinline__ uint64_t wave_sort64(uint64_t v)
{
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) v = bitonic_step(v, lane, size, stride);
    return v;
}

// a bitonic sequence of 64 keys sorted descending (the merge half of the
// network)
__device__ __forceinline__ uint64_t wave_clean64(uint64_t v)
{
    const int lane = lane_id();
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) v = bitonic_step(v, lane, 64, stride);
    return v;
}

// 128 keys (a: elements 0-63, b: 64-127, element 64r + lane) sorted
// descending
__device__ __forceinline__ void wave_sort128(uint64_t &a, uint64_t &b)
{
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= 128; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride == 64) {
                const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
                a = hi;
                b = lo;
            } else {
                a = bitonic_step(a, lane, size, stride);
                b = bitonic_step(b, 64 + lane, size, stride);
            }
        }
}

// 32-bit forms of the networks above, for keys without the index half
__device__ __forceinline__ uint32_t bitonic_step32(uint32_t v, int i, int size, int stride)
{
    const uint32_t o = xor_lane(v, stride);
    const bool keep_max = ((i & stride) == 0) == ((i & size) == 0);
    return (v > o) == keep_max ? v : o;
}
__device__ __forceinline__ uint32_t wave_sort64_u32(uint32_t v)
{
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) v = bitonic_step32(v, lane, size, stride);
    return v;
}
__device__ __forceinline__ uint32_t wave_clean64_u32(uint32_t v)
{
    const int lane = lane_id();
    v = bitonic_step32(v, lane, 64, 32);
    v = bitonic_step32(v, lane, 64, 16);
    v = bitonic_step32(v, lane, 64, 8);
    v = bitonic_step32(v, lane, 64, 4);
    v = bitonic_step32(v, lane, 64, 2);
    return bitonic_step32(v, lane, 64, 1);
}
// 32 keys in lanes 0-31 sorted descending (lanes 32-63 sort their own 32)
__device__ __forceinline__ uint64_t wave_sort32(uint64_t v)
{
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= 32; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) v = bitonic_step(v, lane, size, stride);
    return v;
}

// The `need` (<= 64) largest nonzero keys held across the workgroup (E per
// thread, all distinct), sorted descending into s_out[0..need), by sorting
// networks instead of radix passes.  The need-th largest of the threads'
// maxima bounds the answer from below (need threads hold a key at least
// that large); only its value half is found (32-bit networks: the four
// waves' sorted maxima merged twice), and every key whose value half reaches
// it is kept -- a superset of the keys at or above the full bound, so it
// holds the answer.  The kept keys are gathered through an LDS counter (in
// no fixed order) and, when at most 128, sorted by one wave: the sorted
// result is the same whatever order they were gathered in.  Returns false
// (nothing written to s_out, c untouched) when more than 128 are kept; the
// caller then takes the radix select.  s_sort: 256 uint64, s_w: 4 ints.
template <int E>
__device__ bool wg_topk_sorted(const uint64_t (&c)[E], int need, uint64_t *s_out, uint64_t *s_sort, int *s_w,
                               uint64_t *s_m)
{
    (void)s_m;
    const int t = (int)threadIdx.x, w = t >> 6, lane = t & 63;
    uint64_t m = 0;
#pragma unroll
    for (int j = 0; j < E; j++) m = c[j] > m ? c[j] : m;
    uint32_t *s_s32 = (uint32_t *)s_sort;
    if (t == 0) s_w[0] = 0;                   // the kept-key counter, used after three barriers
    s_s32[t] = wave_sort64_u32((uint32_t)(m >> 32));
    __syncthreads();
    uint32_t v2 = 0;
    if (w < 2) {                              // top 64 of waves (0, 1) and of (2, 3)
        const uint32_t x = s_s32[128 * w + lane], y = s_s32[128 * w + 127 - lane];
        v2 = wave_clean64_u32(x > y ? x : y);
    }
    __syncthreads();                          // every read above is done
    if (w < 2) s_s32[64 * w + lane] = v2;
    __syncthreads();
    if (w == 0) {                             // top 64 of all the maxima
        const uint32_t x = s_s32[lane], y = s_s32[127 - lane];
        const uint32_t v = wave_clean64_u32(x > y ? x : y);
        const uint32_t bound = (uint32_t)__builtin_amdgcn_readlane((int)v, need - 1);
        if (lane == 0) s_w[1] = (int)bound;
    }
    __syncthreads();
    const uint32_t bound = (uint32_t)s_w[1];  // 0 when fewer than `need` threads hold keys
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < E; j++) cnt += c[j] && (uint32_t)(c[j] >> 32) >= bound;
    int pos = cnt ? atomicAdd(&s_w[0], cnt) : 0;
#pragma unroll
    for (int j = 0; j < E; j++)
        if (c[j] && (uint32_t)(c[j] >> 32) >= bound) {
            if (pos < 128) s_sort[pos] = c[j];
            pos++;
        }
    __syncthreads();
    const int total = s_w[0];
    if (total > 128) return false;            // workgroup-uniform
    if (w == 0) {
        uint64_t a = lane < total ? s_sort[lane] : 0ull;
        if (total <= 32) {                    // the usual case
            a = wave_sort32(a);
        } else if (total <= 64) {
            a = wave_sort64(a);
        } else {
            uint64_t b = 64 + lane < total ? s_sort[64 + lane] : 0ull;
            wave_sort128(a, b);
        }
        if (lane < need) s_out[lane] = a;
    }
    __syncthreads();
    return true;
}

// the reference's xorshift64* (sampler.c:9-14)
__device__ __forceinline__ uint64_t samp_rng(uint64_t &s)
{
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1DULL;
}

__device__ __forceinline__ float readlane_f(float v, int i)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// sampler_pick (sampler.c:100-134) with candidate i in lane i (i < k, in
// descending order); every lane returns the token.  *drew = 1 when a draw
// was made (the seed advanced; the token joins last_tokens).
//
// The reference's three running sums, without a branch per candidate: a
// lane that is not live contributes +0.0, which leaves a sum >= 0 unchanged,
// so z adds every lane's value in index order, and lane i forms its own
// inclusive prefix of p in index order -- the value the reference's acc and
// cum (the same additions in the same order) hold after candidate i.  The
// top-p cut is then the first live lane whose prefix reaches top_p (else the
// last live lane), and the pick the first kept live lane whose prefix
// exceeds the draw (else the last kept one): one ballot each.
__device__ int samp_pick_wave(float lg, int id, int k, float temp, float top_p, uint64_t &seed, int *drew)
{
    const int lane = lane_id();
    *drew = 0;
    const bool live = lane < k && lg > -1e29f;
    const unsigned long long lv = __ballot(live);
    const int id0 = __builtin_amdgcn_readlane(id, 0);
    if (!lv) return id0;                                   // all masked
    const int first_live = __ffsll(lv) - 1;
    if (temp <= 0.0f) return __builtin_amdgcn_readlane(id, first_live);   // greedy: the best live one
    float mx = live ? lg : -INFINITY;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __uint_as_float(xor_lane(__float_as_uint(mx), d)));
    // expf correctly rounded, through double (the device's expf is not)
    const float e = live ? (float)exp((double)__fsub_rn(lg, mx)) : 0.0f;
    double z = 0.0;                                        // summed in index order
    for (int i = first_live; i < k; i++) z += (double)readlane_f(e, i);
    const float inv = (float)(1.0 / z);
    const float p = live ? __fmul_rn(e, inv) : 0.0f;
    float pre = 0.0f;                                      // p[first_live] + ... + p[lane], in order
    for (int j = first_live; j < k; j++) {
        const float s = __fadd_rn(pre, readlane_f(p, j));
        pre = j <= lane ? s : pre;
    }
    const unsigned long long hit = __ballot(live && pre >= top_p);
    const int kept = hit ? __ffsll(hit) : 64 - __clzll(lv);        // the cut lane + 1
    const uint64_t r = samp_rng(seed);
    const float rv = (float)((double)(r >> 11) * (1.0 / 9007199254740992.0));
    const unsigned long long pk = __ballot(live && lane < kept && rv < pre);
    const int pick = pk ? __ffsll(pk) - 1 : kept - 1;
    *drew = 1;
    return __builtin_amdgcn_readlane(id, pick);
}

// The k largest of the chunks' candidates (total_c of them, E per thread),
// sorted descending into s_win, or (return false) selected into s_win in no
// order by the radix select.
template <int E>
__device__ bool samp_merge(const uint64_t *cand, int total_c, int k, uint64_t *s_win, uint64_t *s_sort, int *s_w,
                           uint64_t *s_m, uint32_t *s_hist, int *s_info)
{
    const int t = (int)threadIdx.x;
    uint64_t g[E];
#pragma unroll
    for (int j = 0; j < E; j++) {
        const int i = t + 256 * j;
        g[j] = i < total_c ? __hip_atomic_load(cand + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    }
    const bool sorted = wg_topk_sorted<E>(g, k, s_win, s_sort, s_w, s_m);
    if (!sorted) {
        bool gs[E];
        wg_topk<E>(g, k, gs, s_hist, s_info, s_m);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < E; j++) cnt += gs[j];
        int total;
        int pos = wg_excl_scan(cnt, s_w, &total);
#pragma unroll
        for (int j = 0; j < E; j++)
            if (gs[j]) s_win[pos++] = g[j];
        __syncthreads();
    }
    return sorted;
}

// out (pinned host memory): [0..63] ids, [64..127] values (float bits),
// [128] token, [129] drew, [130..131] new seed (low, high), [132] = seq
// once everything before it is visible to the host
__global__ __launch_bounds__(256) void sampler_kernel(const float *__restrict__ logits, int n, SampParams P, int k,
                                                      int n_chunks, uint64_t *__restrict__ cand,
                                                      unsigned *__restrict__ done, int sample, uint64_t seed,
                                                      float top_p, int *__restrict__ out, int seq)
{
    __shared__ float4 s_v4[SAMP_CHUNK / 4];
    __shared__ uint32_t s_hist[256];
    __shared__ int s_info[4], s_w[4];
    __shared__ uint64_t s_win[SAMP_MAX_K];
    __shared__ int s_last;
    __shared__ uint64_t s_m[4];
    __shared__ uint64_t s_sort[256];
    float *s_v = (float *)s_v4;
    const int t = (int)threadIdx.x;
    const int base = (int)blockIdx.x * SAMP_CHUNK;
    // the repeat penalty's ids and counts (argument memory) requested ahead
    // of the logits, so that their round trip overlaps the logits' own
    int pen_id = -1, pen_cnt = 0;
    if (P.repeat_penalty != 1.0f && t < P.n_uniq) {
        pen_id = P.uniq[t];
        pen_cnt = P.count[t];
    }
    // the temperature in a register now, not reloaded after the barriers
    uint32_t temp_bits = __float_as_uint(P.temp);
    __asm__ volatile("" : "+s"(temp_bits));
    const float temp = __uint_as_float(temp_bits);
    if (base + SAMP_CHUNK <= n) {
        // a whole chunk: every load in flight at once
        float4 v[SAMP_PER_THREAD / 4];
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD / 4; m++) v[m] = ldg4(logits + base + 4 * (t + 256 * m));
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD / 4; m++) s_v4[t + 256 * m] = v[m];
    } else {
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD / 4; m++) {
            const int i = base + 4 * (t + 256 * m);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i + 3 < n) v = ldg4(logits + i);
            else {
                if (i < n) v.x = logits[i];
                if (i + 1 < n) v.y = logits[i + 1];
                if (i + 2 < n) v.z = logits[i + 2];
            }
            s_v4[t + 256 * m] = v;
        }
    }
    __syncthreads();
    // repeat penalty (sampler.c:47-55): each occurrence of an id in
    // last_tokens applies the rule to the current value, in turn
    if (pen_id >= base && pen_id < base + SAMP_CHUNK && pen_id < n) {
        float v = s_v[pen_id - base];
        for (int j = 0; j < pen_cnt; j++) v = v < 0.0f ? v * P.repeat_penalty : v / P.repeat_penalty;
        s_v[pen_id - base] = v;
    }
    __syncthreads();
    // element i = t + 256 m of the chunk: every LDS read issued at once
    // (the chunk's slots past n hold zeros and are masked after)
    float cv[SAMP_PER_THREAD];
#pragma unroll
    for (int m = 0; m < SAMP_PER_THREAD; m++) cv[m] = s_v[t + 256 * m];
    if (temp > 0.0f && temp != 1.0f) {                            // sampler.c:56-58 (x / 1 = x)
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD; m++) cv[m] = cv[m] / temp;
    }
    uint64_t c[SAMP_PER_THREAD];
#pragma unroll
    for (int m = 0; m < SAMP_PER_THREAD; m++) {
        const int i = t + 256 * m;
        c[m] = base + i < n ? samp_comp(samp_key(cv[m]), base + i, cv[m]) : 0ull;
    }
    const int valid = n - base < SAMP_CHUNK ? n - base : SAMP_CHUNK;
    const int kk = k < valid ? k : valid;
    // The candidates go out with device-scope stores (coherent across the
    // XCDs' L2s without a cache write-back), each wave waits for its stores
    // to complete, then one increment of the counter per workgroup: the
    // workgroup that brings it to n_chunks saw every other one's stores done
    // and merges.  No cache-wide fence is needed.
    uint64_t *mine = cand + (size_t)blockIdx.x * k;
    if (wg_topk_sorted<SAMP_PER_THREAD>(c, kk, s_win, s_sort, s_w, s_m)) {
        for (int i = t; i < k; i += 256)
            __hip_atomic_store(mine + i, i < kk ? s_win[i] : 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        bool sel[SAMP_PER_THREAD];
        wg_topk<SAMP_PER_THREAD>(c, kk, sel, s_hist, s_info, s_m);
        int cnt = 0;
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD; m++) cnt += sel[m];
        int total;
        int pos = wg_excl_scan(cnt, s_w, &total);
#pragma unroll
        for (int m = 0; m < SAMP_PER_THREAD; m++)
            if (sel[m]) __hip_atomic_store(mine + pos++, c[m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int i = kk + t; i < k; i += 256)
            __hip_atomic_store(mine + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0)
        s_last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(n_chunks - 1);
    __syncthreads();
    if (!s_last) return;
    // the k largest of all chunks' candidates: 8 per thread when they fit
    // (up to 2,048: 38 chunks of 40 for a 151,936-entry vocabulary), the
    // full 32 otherwise
    const int total_c = n_chunks * k;
    const bool sorted = total_c <= 256 * 8
                            ? samp_merge<8>(cand, total_c, k, s_win, s_sort, s_w, s_m, s_hist, s_info)
                            : samp_merge<SAMP_MERGE_PER_THREAD>(cand, total_c, k, s_win, s_sort, s_w, s_m, s_hist,
                                                                s_info);
    if (t < 64) {
        const int lane = t;
        uint64_t v = lane < k ? s_win[lane] : 0ull;
        if (!sorted) v = wave_sort64(v);
        const int id = samp_id(v);
        const float val = samp_value(v);
        // results to pinned host memory with system-scope stores, waited for
        // before the completion marker is stored
        auto put = [&](int i, int v) { __hip_atomic_store(out + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); };
        if (lane < k) {
            put(lane, id);
            put(64 + lane, __float_as_int(val));
        }
        if (sample) {
            int drew = 0;
            uint64_t sd = seed;
            const int tok = samp_pick_wave(val, id, k, temp, top_p, sd, &drew);
            if (lane == 0) {
                put(128, tok);
                put(129, drew);
                put(130, (int)(uint32_t)sd);
                put(131, (int)(uint32_t)(sd >> 32));
            }
        }
        if (lane == 0) __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // for the next call
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) put(132, seq);
    }
}

// ------------------------------------------------------------------ host --
static int *g_samp_host = nullptr;      // pinned: the kernel's results
static int g_samp_seq = 0;
// one sampling call at a time per process: the pinned results, the marker
// sequence and the workspace are shared
static std::mutex g_samp_mu;

// Wait for the kernel's completion marker in pinned memory: a host spin on
// one word is far quicker than a stream synchronisation.  Every few
// thousand polls the stream is queried, so a launch that failed, or a
// kernel that finished without the marker reaching the host, ends the wait.
// The marker is read with acquire ordering: the results, stored before it
// by the kernel, are read after it.
static int wait_marker(hipStream_t st, int seq)
{
    const int *m = g_samp_host + 132;
    for (long i = 1;; i++) {
        if (__atomic_load_n(m, __ATOMIC_ACQUIRE) == seq) return QMAG_OK;
        if (i % 4096 == 0) {
            const hipError_t e = hipStreamQuery(st);
            if (e == hipSuccess) {
                if (__atomic_load_n(m, __ATOMIC_ACQUIRE) == seq) return QMAG_OK;
                return fail(QMAG_ERR_KERNEL, "sampler: kernel finished without its completion marker");
            }
            if (e != hipErrorNotReady) return hip_fail(e, "sampler wait", __FILE__, __LINE__);
        }
    }
}

static int sample_run(int n_vocab, const float *logits, const qmag_sampler *s, int max_k, bool sample, float top_p,
                      int *ids, float *vals, int res[4])
{
    if (!logits || !s || n_vocab <= 0) return fail(QMAG_ERR_ARG, "sampler: null pointer or n_vocab=%d", n_vocab);
    if (n_vocab > SAMP_MAX_VOCAB) return fail(QMAG_ERR_ARG, "sampler: n_vocab %d above %d", n_vocab, SAMP_MAX_VOCAB);
    if (max_k < 1 || max_k > SAMP_MAX_K) return fail(QMAG_ERR_ARG, "sampler: max_k %d outside 1..%d", max_k, SAMP_MAX_K);
    int k = s->top_k;                                   // sampler.c:63-66
    if (k < 1) k = 1;
    if (k > n_vocab) k = n_vocab;
    if (k > max_k) k = max_k;
    SampParams P;
    P.temp = s->temp;
    P.repeat_penalty = s->repeat_penalty;
    const int n_last = s->n_last < 0 ? 0 : s->n_last > 64 ? 64 : s->n_last;
    // distinct ids in first-occurrence order with their counts, found through
    // a 128-entry open-addressing table (at most 64 ids, so it never fills)
    // instead of a linear search over the ids seen so far (up to ~2,000
    // comparisons per call on the host, ahead of the launch)
    short slot[128];                                    // index into P.uniq + 1, 0 = empty
    int key[128];
    memset(slot, 0, sizeof(slot));
    P.n_uniq = 0;
    for (int i = 0; i < n_last; i++) {
        const int id = s->last_tokens[i];
        if (id < 0 || id >= n_vocab) continue;             // sampler.c:50
        unsigned h = ((unsigned)id * 2654435761u) >> 25;
        while (slot[h] && key[h] != id) h = (h + 1) & 127;
        if (!slot[h]) {
            key[h] = id;
            slot[h] = (short)(P.n_uniq + 1);
            P.uniq[P.n_uniq] = id;
            P.count[P.n_uniq++] = 0;
        }
        P.count[slot[h] - 1]++;
    }
    const int n_chunks = (n_vocab + SAMP_CHUNK - 1) / SAMP_CHUNK;
    hipStream_t st = ctx().stream;
    std::lock_guard<std::mutex> guard(g_samp_mu);
    // Logits computed from persistent-decode outputs: have any expired wait
    // of those launches recovered first (qmag_d2h does the same).  A recovery
    // re-runs the decode calls but not the work queued after them, such as
    // the LM head that produced these logits from their earlier (partly
    // unwritten) outputs: then nothing is sampled and the caller is told to
    // recompute the logits.
    if (fused_pending()) {
        const long r0 = fused_recoveries();
        const int fst = fused_status();
        if (fst) return fst;
        if (fused_recoveries() != r0)
            return fail(QMAG_ERR_REPLAYED,
                        "sampler: persistent decode calls queued before these logits were re-run after an "
                        "expired wait; logits computed from their earlier outputs are stale: recompute them "
                        "and sample again");
    }
    const size_t cand_bytes = sizeof(uint64_t) * (size_t)SAMP_MAX_CHUNKS * SAMP_MAX_K;
    int wst = QMAG_OK;
    uint8_t *ws = (uint8_t *)workspace(WS_SAMP, cand_bytes + 256, &wst);
    if (!ws) return wst;
    unsigned *done = (unsigned *)(ws + cand_bytes);
    static uint8_t *counted = nullptr;
    if (ws != counted) {
        // a new buffer: the completion counter starts at zero; each
        // launch's last workgroup puts it back
        QMAG_HIP(hipMemsetAsync(done, 0, sizeof(unsigned), st));
        counted = ws;
    }
    if (!g_samp_host) {
        QMAG_HIP(hipHostMalloc((void **)&g_samp_host, 136 * sizeof(int), hipHostMallocDefault));
        g_samp_host[132] = 0;
    }
    const int seq = ++g_samp_seq == 0 ? ++g_samp_seq : g_samp_seq;    // never 0, the initial marker
    hipLaunchKernelGGL(sampler_kernel, dim3(n_chunks), dim3(256), 0, st, logits, n_vocab, P, k, n_chunks,
                       (uint64_t *)ws, done, sample ? 1 : 0, s->seed, top_p, g_samp_host, seq);
    QMAG_HIP(hipGetLastError());
    const int wst2 = wait_marker(st, seq);
    if (wst2) return wst2;
    if (ids) memcpy(ids, g_samp_host, sizeof(int) * k);
    if (vals) memcpy(vals, g_samp_host + 64, sizeof(float) * k);
    if (sample) memcpy(res, g_samp_host + 128, sizeof(int) * 4);
    return k;
}

}  // namespace qmag

using namespace qmag;

extern "C" {

int qmag_sampler_candidates_dev(int n_vocab, const float *logits, const qmag_sampler *s, int *ids, float *lgs,
                                int max_k)
{
    int st = require_ready();
    if (st) return st;
    if (!ids || !lgs) return fail(QMAG_ERR_ARG, "sampler: null output");
    int res[4];
    return sample_run(n_vocab, logits, s, max_k, false, 0.0f, ids, lgs, res);
}

int qmag_sampler_sample_dev(int n_vocab, const float *logits, qmag_sampler *s, int max_k, float top_p, int *token)
{
    int st = require_ready();
    if (st) return st;
    if (!token) return fail(QMAG_ERR_ARG, "sampler: null token");
    int res[4] = {0, 0, 0, 0};
    const int k = sample_run(n_vocab, logits, s, max_k, true, top_p, nullptr, nullptr, res);
    if (k < 0) return k;
    *token = res[0];
    if (res[1]) {                  // a draw: the new state, and the pick joins last_tokens
        s->seed = (uint64_t)(uint32_t)res[2] | ((uint64_t)(uint32_t)res[3] << 32);
        if (s->n_last < 64) {
            s->last_tokens[s->n_last++] = res[0];
        } else {
            memmove(s->last_tokens, s->last_tokens + 1, 63 * sizeof(int));
            s->last_tokens[63] = res[0];
        }
    }
    return QMAG_OK;
}

}  // extern "C"
