/*
 * qma_oracle.h -- CPU oracle for the quantized MoE expert-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a scalar C99 restatement of the
 * reference engine's arithmetic (qma: src/q8k.c, src/quants.c, src/qma.h,
 * src/nn.c).  It is used by tests/ as the parity checker, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg
 * as the timed CPU path.  The GPU library never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Where the
 * reference is NEON code, the restatement keeps the NEON lane structure
 * (4 int32 / fp32 lanes per vector, FADDP pairwise horizontal adds) so the
 * fp32 association follows the reference as written; it is compiled with
 * -ffp-contract=off and uses fmaf() exactly where the reference uses a
 * fused vector FMA intrinsic.
 *
 * Pins (see tests/test_oracle_*.py): the numpy restatement in
 * oracle/oracle_np.py (independent code), brute-force integer dots on tiny
 * inputs, closed-form fp64 dots, definition-level known answers for Q8_K,
 * exhaustive scale/min unpack, and the committed fixtures in tests/golden/.
 */
#ifndef QMA_ORACLE_H
#define QMA_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_TYPE_Q4_K 12    /* GGML type ids, qma.h:67-69 */
#define ORC_TYPE_Q6_K 14

/* GGUF super-block layouts, byte-identical to qma.h:77-90. */
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t  scales[12];
    uint8_t  qs[128];
} orc_block_q4k;            /* 144 B */

typedef struct {
    uint8_t  ql[128];
    uint8_t  qh[64];
    int8_t   scales[16];
    uint16_t d;
} orc_block_q6k;            /* 210 B */

/* ---- formats (qma.h, quants.c) ---- */
float    orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
void     orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);
void     orc_dequant_q4k(const void *blocks, float *y, int64_t k);
void     orc_dequant_q6k(const void *blocks, float *y, int64_t k);
float    orc_dot_q4k_f32(const void *row, const float *x, int n);
float    orc_dot_q6k_f32(const void *row, const float *x, int n);

/* ---- Q8_K activation quantization and int8 dots (q8k.c) ---- */
void     orc_q8k_quant(const float *x, int n, int8_t *xq, float *xd, int16_t *xsum);
float    orc_q8k_dot(const void *row, int wtype, const int8_t *xq,
                     const float *xd, const int16_t *xsum, int n);
void     orc_q8k_gateup(const void *g, const void *u, const int8_t *xq,
                        const float *xd, const int16_t *xsum, int n,
                        float *gate, float *up);
/* integer intermediates: Q4_K per-32-lane sub-block sums (n/32 values),
   Q6_K per-super-block sums (n/256 values) */
void     orc_q4k_subsums(const void *row, const int8_t *xq, int n, int32_t *P);
void     orc_q6k_blocksums(const void *row, const int8_t *xq, int n, int32_t *S);

/* ---- drivers (nn.c) ---- */
/* CPU pool that follows pool_run (nn.c:139-175); nthreads<=0 -> 1 */
void     orc_pool_set_threads(int nthreads);
int      orc_pool_threads(void);

void     orc_matmul_q8k(const float *x, const void *W, int n_in, int n_out,
                        int T, int wtype, float *out);

typedef struct {
    int n_embd;               /* 2048 (qma.h:28)                 */
    int n_ff;                 /* 512  (qma.h:59-60)              */
    int n_expert;             /* 256  (qma.h:57)                 */
    int n_used;               /* 8    (qma.h:58)                 */
    const float   *gate_inp;       /* f32 [n_expert][n_embd]          */
    const float   *router_bias;    /* f32 [n_expert] or NULL (synthetic skew) */
    const uint8_t *gate_exps;      /* Q4_K [n_expert][n_ff rows]      */
    const uint8_t *up_exps;        /* Q4_K [n_expert][n_ff rows]      */
    const uint8_t *down_exps;      /* Q4_K/Q6_K [n_expert][n_embd rows] */
    int            t_down_exps;
    const float   *gate_inp_shexp; /* f32 [n_embd]                    */
    const uint8_t *gate_shexp;     /* Q4_K [n_ff rows]                */
    const uint8_t *up_shexp;
    const uint8_t *down_shexp;     /* Q4_K/Q6_K [n_embd rows]         */
    int            t_down_shexp;
} orc_moe_layer;

/* router for one token: softmax, top-n_used (strict >, lowest index wins),
   renormalised weights.  logits_out (optional, n_expert) receives the
   pre-softmax logits (plus bias). */
void     orc_moe_route(const orc_moe_layer *L, const float *x, int *sel,
                       float *w, float *logits_out);
/* full layer, q8k semantics; partial accumulators start at zero */
void     orc_moe_ffn(const orc_moe_layer *L, const float *x, float *out, int T);
/* same, with the routing forced (sel/w: [T][n_used]) */
void     orc_moe_ffn_routed(const orc_moe_layer *L, const float *x, float *out,
                            int T, const int *sel, const float *w);
/* stage outputs of one (token, expert) task: h = silu(g)*u (n_ff floats) */
void     orc_moe_expert_h(const uint8_t *ge, const uint8_t *ue, int n_embd,
                          int n_ff, const int8_t *xq, const float *xd,
                          const int16_t *xsum, float *h);
float    orc_moe_shared_gate(const float *wsh, const int8_t *xq,
                             const float *xd, int n_embd);
/* fp32 twins (QMA_NOQ8K, nn.c:393-407, 475-492, 585): no activation
   quantisation; expert h on fp32 x, the fp32 shared gate, the full layer */
void     orc_moe_expert_h_f32(const uint8_t *ge, const uint8_t *ue, int n_embd,
                              int n_ff, const float *x, float *h);
float    orc_moe_shared_gate_f32(const float *wsh, const float *x, int n_embd);
void     orc_moe_ffn_f32(const orc_moe_layer *L, const float *x, float *out, int T);
/* residual chain used by the layer-stack workload: x <- x + moe_l(x) */
void     orc_moe_stack(const orc_moe_layer *layers, int n_layer, float *x);

/* ---- sampler (sampler.c), state in the layout of sampler_t (qma.h:279-287) ---- */
typedef struct {
    uint64_t seed;
    float    temp;
    int      top_k;
    float    top_p;
    float    repeat_penalty;
    int      last_tokens[64];
    int      n_last;
} orc_sampler;
int      orc_sampler_candidates(int n_vocab, const float *logits, const orc_sampler *s,
                                int *ids, float *lgs, int max_k);
int      orc_sampler_pick(orc_sampler *s, const int *ids, float *lgs, int n, float top_p);

/* ---- synthetic inputs (the build's own generator and quantizers) ---- */
uint64_t orc_splitmix64(uint64_t *state);
void     orc_fill_normal(uint64_t seed, int64_t n, float mean, float std, float *out);
void     orc_quantize_q4k(const float *x, int64_t n, void *out);
void     orc_quantize_q6k(const float *x, int64_t n, void *out);

#ifdef __cplusplus
}
#endif
#endif
