// qmag_sampler.hip -- sampling on the device (src/sampler.c:36-134), so the
// LM head's logits (151,936 floats) never leave HBM.
//
// sampler_candidates: the repeat penalty (per occurrence in last_tokens:
// negative logits multiplied, others divided), division by the temperature,
// then the k largest values in descending order.  sampler_pick: the softmax
// over the live candidates with a double sum, the top-p cut, one xorshift64*
// draw and the cumulative pick, and the pick's entry into last_tokens.
//
// Two launches.  cand_chunk_kernel: one workgroup per 4096 logits, one wave
// per 1024 of them; each lane holds 16 (indices lane + 64m), sorts them once
// (descending value, ascending index among equal values) and the wave takes
// its top k by k picks, each a wave max over the lane heads; wave 0 then
// merges the four waves' lists the same way.  cand_merge_kernel: one
// workgroup stages the chunks' sorted lists in LDS and one wave merges them
// by k picks over the list heads (each lane owns up to two lists), then, in
// the sampling form, one lane makes the pick with the reference's
// arithmetic.  About 2 * 64 picks of ~0.1 us for k = 64; the logits are read
// once (0.6 MB for the Qwen vocabulary).
//
// Among exactly equal values the lower index comes first.  The reference
// keeps its candidates in a min-heap and sorts them with qsort, so which of
// several equal values at the k-th place it keeps, and their order, depends
// on the heap; for distinct values the two agree exactly.  NaN logits sort
// after every number here; the reference's comparisons leave their place to
// the heap's history.
#include <limits.h>
#include <string.h>

#include "qmag_internal.h"

namespace qmag {

constexpr int SAMP_WAVE_CHUNK = 1024;       // logits per wave in the first launch
constexpr int SAMP_PER_LANE = SAMP_WAVE_CHUNK / 64;
constexpr int SAMP_WAVES = 4;
constexpr int SAMP_CHUNK = SAMP_WAVES * SAMP_WAVE_CHUNK;   // logits per workgroup
constexpr int SAMP_MAX_K = 64;
constexpr int SAMP_LISTS_PER_LANE = 2;      // the merge handles up to 128 chunks
// 127 chunks: the merge's lists (127 * 64 * 8 bytes) and its 512 bytes of
// output staging fill exactly the 64 KiB of LDS a workgroup gets by default
constexpr int SAMP_MAX_VOCAB = 127 * SAMP_CHUNK;    // 520,192

struct SampParams {
    float temp;
    float repeat_penalty;
    int n_last;
    int last[64];
};

// order key: descending float order as ascending unsigned order; 0 marks an
// element past the end, 1 a NaN (after every other value)
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

template <int W>
__device__ __forceinline__ uint32_t group_max_u(uint32_t v)
{
    if constexpr (W >= 2) v = max(v, (uint32_t)dpp_i<DPP_XOR1>((int)v));
    if constexpr (W >= 4) v = max(v, (uint32_t)dpp_i<DPP_XOR2>((int)v));
    if constexpr (W >= 8) v = max(v, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)v));
    if constexpr (W >= 16) v = max(v, (uint32_t)dpp_i<DPP_MIRROR>((int)v));
    if constexpr (W >= 32) {
        auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max(p[0], p[1]);
    }
    if constexpr (W >= 64) {
        auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max(p[0], p[1]);
    }
    return v;
}

// one pick: the largest head key; among equal keys the lowest index.  Returns
// whether this lane's head was picked.
__device__ __forceinline__ bool samp_pick(uint32_t head, int head_id, uint32_t &m)
{
    m = group_max_u<64>(head);
    bool me = head == m;
    const unsigned long long bal = __ballot(me);
    if (bal & (bal - 1)) {
        const int best = group_min_i<64>(me ? head_id : INT_MAX);
        me = me && head_id == best;
    }
    return me;
}

__global__ __launch_bounds__(256) void cand_chunk_kernel(const float *__restrict__ logits, int n, SampParams P, int k,
                                                         uint32_t *__restrict__ ckey, int *__restrict__ cid)
{
    __shared__ float4 s_v4[SAMP_CHUNK / 4];
    __shared__ uint32_t s_key[SAMP_WAVES][64][SAMP_PER_LANE + 1];
    __shared__ int s_id[SAMP_WAVES][64][SAMP_PER_LANE + 1];
    __shared__ uint32_t s_wk[SAMP_WAVES][SAMP_MAX_K + 1];
    __shared__ int s_wi[SAMP_WAVES][SAMP_MAX_K + 1];
    float *s_v = (float *)s_v4;
    const int t = (int)threadIdx.x, lane = lane_id(), w = t >> 6;
    const int base = (int)blockIdx.x * SAMP_CHUNK;
#pragma unroll
    for (int m = 0; m < SAMP_CHUNK / 4 / 256; m++) {
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
    __syncthreads();
    // repeat penalty (sampler.c:47-55): the first occurrence of each
    // last-token id applies every occurrence, in order
    if (P.repeat_penalty != 1.0f && t < P.n_last) {
        const int id = P.last[t];
        bool first = true;
        for (int j = 0; j < t; j++) first = first && P.last[j] != id;
        if (first && id >= base && id < base + SAMP_CHUNK && id < n) {
            float v = s_v[id - base];
            for (int j = t; j < P.n_last; j++)
                if (P.last[j] == id) v = v < 0.0f ? v * P.repeat_penalty : v / P.repeat_penalty;
            s_v[id - base] = v;
        }
    }
    __syncthreads();
    uint32_t key[SAMP_PER_LANE];
    int id[SAMP_PER_LANE];
#pragma unroll
    for (int m = 0; m < SAMP_PER_LANE; m++) {
        const int i = w * SAMP_WAVE_CHUNK + lane + 64 * m;
        float v = s_v[i];
        if (P.temp > 0.0f) v = v / P.temp;                       // sampler.c:56-58
        id[m] = base + i;
        key[m] = base + i < n ? samp_key(v) : 0u;
    }
    // the lane's 16 in descending (key, -index) order: Batcher's odd-even
    // merge sort, unrolled into 63 compare-exchanges on registers
    auto cs = [&](int a, int b) {
        const bool sw = key[b] > key[a] || (key[b] == key[a] && id[b] < id[a]);
        const uint32_t ka = key[a], kb = key[b];
        const int ia = id[a], ib = id[b];
        key[a] = sw ? kb : ka;
        key[b] = sw ? ka : kb;
        id[a] = sw ? ib : ia;
        id[b] = sw ? ia : ib;
    };
#pragma unroll
    for (int p = 1; p < SAMP_PER_LANE; p <<= 1)
#pragma unroll
        for (int q = p; q >= 1; q >>= 1)
#pragma unroll
            for (int j = q % p; j + q < SAMP_PER_LANE; j += 2 * q)
#pragma unroll
                for (int i = 0; i < q; i++)
                    if (i + j + q < SAMP_PER_LANE && (i + j) / (2 * p) == (i + j + q) / (2 * p)) cs(i + j, i + j + q);
#pragma unroll
    for (int m = 0; m < SAMP_PER_LANE; m++) {
        s_key[w][lane][m] = key[m];
        s_id[w][lane][m] = id[m];
    }
    s_key[w][lane][SAMP_PER_LANE] = 0u;          // sentinel past each list
    s_id[w][lane][SAMP_PER_LANE] = INT_MAX;
    // k picks over the lane heads (each lane reads only its own row)
    {
        int h = 0;
        uint32_t head = key[0];
        int head_id = id[0];
        for (int p = 0; p < k; p++) {
            uint32_t m;
            const bool me = samp_pick(head, head_id, m);
            if (me) {
                s_wk[w][p] = head;
                s_wi[w][p] = head_id;
                h = min(h + 1, SAMP_PER_LANE);
                head = s_key[w][lane][h];
                head_id = s_id[w][lane][h];
            }
        }
    }
    if (lane == 0) {
        s_wk[w][k] = 0u;
        s_wi[w][k] = INT_MAX;
    }
    __syncthreads();
    // wave 0 merges the four lists: lane j < 4 holds list j's head
    if (w == 0) {
        int h = 0;
        uint32_t head = lane < SAMP_WAVES ? s_wk[lane][0] : 0u;
        int head_id = lane < SAMP_WAVES ? s_wi[lane][0] : INT_MAX;
        for (int p = 0; p < k; p++) {
            uint32_t m;
            const bool me = samp_pick(head, head_id, m);
            if (me) {
                ckey[(size_t)blockIdx.x * k + p] = head;
                cid[(size_t)blockIdx.x * k + p] = head_id;
                h = min(h + 1, k);
                head = lane < SAMP_WAVES ? s_wk[lane][h] : 0u;
                head_id = lane < SAMP_WAVES ? s_wi[lane][h] : INT_MAX;
            }
        }
    }
}

// the reference's xorshift64* (sampler.c:9-14)
__device__ __forceinline__ uint64_t samp_rng(uint64_t &s)
{
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return s * 0x2545F4914F6CDD1DULL;
}

// sampler_pick (sampler.c:100-134) over k candidates in descending order,
// in one lane.  Returns the token; *drew = 1 if a draw was made (the seed
// advanced and the token joins last_tokens), 0 for the greedy and the
// all-masked answers.
__device__ int samp_pick_token(const int *cid, const float *cval, int k, float temp, float top_p, uint64_t &seed,
                               int *drew)
{
    float lg[SAMP_MAX_K];
    for (int i = 0; i < k; i++) lg[i] = cval[i];
    *drew = 0;
    int first_live = -1;
    for (int i = 0; i < k; i++)
        if (lg[i] > -1e29f) {
            first_live = i;
            break;
        }
    if (first_live < 0) return cid[0];                      // all masked
    if (temp <= 0.0f) return cid[first_live];               // greedy
    float mx = lg[first_live];
    for (int i = first_live; i < k; i++)
        if (lg[i] > -1e29f && lg[i] > mx) mx = lg[i];
    double z = 0.0;
    for (int i = first_live; i < k; i++)
        if (lg[i] > -1e29f) {
            // expf correctly rounded, through double (the device's own expf
            // is not correctly rounded)
            const float e = (float)exp((double)__fsub_rn(lg[i], mx));
            lg[i] = e;
            z += (double)e;
        }
    const float inv = (float)(1.0 / z);
    for (int i = first_live; i < k; i++)
        if (lg[i] > -1e29f) lg[i] = __fmul_rn(lg[i], inv);
    float acc = 0.0f;
    int kept = first_live;
    for (int i = first_live; i < k; i++) {
        if (lg[i] <= -1e29f) continue;
        acc = __fadd_rn(acc, lg[i]);
        kept = i + 1;
        if (acc >= top_p) break;
    }
    const uint64_t r = samp_rng(seed);
    const float rv = (float)((double)(r >> 11) * (1.0 / 9007199254740992.0));
    float cum = 0.0f;
    int pick = cid[kept - 1];
    for (int i = first_live; i < kept; i++) {
        if (lg[i] <= -1e29f) continue;
        cum = __fadd_rn(cum, lg[i]);
        if (rv < cum) {
            pick = cid[i];
            break;
        }
    }
    *drew = 1;
    return pick;
}

// out: ids[k], vals[k]; in the sampling form also res[0] = picked token,
// res[1] = 1 if the pick drew, res[2..3] = the new seed (low, high)
__global__ __launch_bounds__(256) void cand_merge_kernel(const uint32_t *__restrict__ ckey, const int *__restrict__ cid,
                                                         int n_chunks, int k, int *__restrict__ ids,
                                                         float *__restrict__ vals, int sample, uint64_t seed,
                                                         float temp, float top_p, int *__restrict__ res)
{
    extern __shared__ uint32_t s_dyn[];
    uint32_t *s_key = s_dyn;                              // [n_chunks][k]
    int *s_id = (int *)(s_dyn + (size_t)n_chunks * k);
    __shared__ int s_oid[SAMP_MAX_K];
    __shared__ float s_oval[SAMP_MAX_K];
    for (int i = (int)threadIdx.x; i < n_chunks * k; i += (int)blockDim.x) {
        s_key[i] = ckey[i];
        s_id[i] = cid[i];
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = lane_id();
        int hp[SAMP_LISTS_PER_LANE];
        uint32_t hk[SAMP_LISTS_PER_LANE];
        int hi[SAMP_LISTS_PER_LANE];
#pragma unroll
        for (int j = 0; j < SAMP_LISTS_PER_LANE; j++) {
            const int c = lane + 64 * j;
            hp[j] = 0;
            hk[j] = c < n_chunks ? s_key[c * k] : 0u;
            hi[j] = c < n_chunks ? s_id[c * k] : INT_MAX;
        }
        for (int p = 0; p < k; p++) {
            // this lane's best head: the larger key, then the lower index
            const bool second = hk[1] > hk[0] || (hk[1] == hk[0] && hi[1] < hi[0]);
            const uint32_t bk = second ? hk[1] : hk[0];
            const int bi = second ? hi[1] : hi[0];
            uint32_t m;
            const bool me = samp_pick(bk, bi, m);
            if (me) {
                s_oid[p] = bi;
                s_oval[p] = samp_val(bk);
                const int c = lane + (second ? 64 : 0);
                const int np = (second ? hp[1] : hp[0]) + 1;
                const uint32_t nk = np < k ? s_key[c * k + np] : 0u;
                const int ni = np < k ? s_id[c * k + np] : INT_MAX;
                if (second) {
                    hp[1] = np;
                    hk[1] = nk;
                    hi[1] = ni;
                } else {
                    hp[0] = np;
                    hk[0] = nk;
                    hi[0] = ni;
                }
            }
        }
    }
    __syncthreads();
    const int t = (int)threadIdx.x;
    if (t < k) {
        ids[t] = s_oid[t];
        vals[t] = s_oval[t];
    }
    if (sample && t == 0) {
        int drew = 0;
        uint64_t sd = seed;
        res[0] = samp_pick_token(s_oid, s_oval, k, temp, top_p, sd, &drew);
        res[1] = drew;
        res[2] = (int)(uint32_t)sd;
        res[3] = (int)(uint32_t)(sd >> 32);
    }
}

// ------------------------------------------------------------------ host --
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
    P.n_last = s->n_last < 0 ? 0 : s->n_last > 64 ? 64 : s->n_last;
    for (int i = 0; i < 64; i++) P.last[i] = i < P.n_last ? s->last_tokens[i] : -1;
    const int n_chunks = (n_vocab + SAMP_CHUNK - 1) / SAMP_CHUNK;
    const size_t cand = (size_t)n_chunks * k;
    const size_t need = cand * 8 + 256 + SAMP_MAX_K * 8 + 64;
    hipStream_t st = ctx().stream;
    // logits computed from persistent-decode outputs: have any expired wait
    // of those launches recovered first (qmag_d2h does the same)
    if (fused_pending()) {
        const int fst = fused_status();
        if (fst) return fst;
    }
    int wst = QMAG_OK;
    uint8_t *ws = (uint8_t *)workspace(WS_SAMP, need, &wst);
    if (!ws) return wst;
    uint32_t *ckey = (uint32_t *)ws;
    int *cid = (int *)(ws + cand * 4);
    int *d_ids = (int *)(ws + ((cand * 8 + 255) & ~(size_t)255));
    float *d_vals = (float *)(d_ids + SAMP_MAX_K);
    int *d_res = (int *)(d_vals + SAMP_MAX_K);
    const size_t lds = cand * 8;                       // <= 127 chunks * 64 * 8 bytes
    hipLaunchKernelGGL(cand_chunk_kernel, dim3(n_chunks), dim3(256), 0, st, logits, n_vocab, P, k, ckey, cid);
    QMAG_HIP(hipGetLastError());
    hipLaunchKernelGGL(cand_merge_kernel, dim3(1), dim3(256), lds, st, ckey, cid, n_chunks, k, d_ids, d_vals,
                       sample ? 1 : 0, s->seed, s->temp, top_p, d_res);
    QMAG_HIP(hipGetLastError());
    if (ids) QMAG_HIP(hipMemcpyAsync(ids, d_ids, sizeof(int) * k, hipMemcpyDeviceToHost, st));
    if (vals) QMAG_HIP(hipMemcpyAsync(vals, d_vals, sizeof(float) * k, hipMemcpyDeviceToHost, st));
    if (sample) QMAG_HIP(hipMemcpyAsync(res, d_res, sizeof(int) * 4, hipMemcpyDeviceToHost, st));
    QMAG_HIP(hipStreamSynchronize(st));
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
