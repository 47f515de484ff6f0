/*
 * qma_gpu.h -- C-ABI of the MI355X (gfx950) quantized MoE expert-matmul
 * library (libqmagpu.so).
 *
 * Two groups of entry points:
 *
 * 1. Reference-compatible: the exact names and signatures the qma engine
 *    binds from src/q8k.c (declared at src/qma.h:358-365).  Host pointers,
 *    caller-owned buffers, no status returns, unknown wtype -> 0.0f.  They
 *    run on the GPU (staged per calling thread) so a build that drops
 *    src/q8k.c and links this library keeps working unchanged; they are
 *    per-row calls and therefore latency-bound.  qma_q8k_available() reports
 *    whether a usable gfx950 device is present; without one the other q8k
 *    entries compute nothing and return zeros, as the reference's build
 *    without dotprod does (q8k.c:280-316), and the quants.c entries abort
 *    with a message (the reference has no unavailable form for them).
 *
 * 2. Device entries (qmag_*): the coarse seams of src/nn.c -- matmul
 *    (nn.c:307) and moe_ffn (nn.c:509) -- over weights resident in HBM in the
 *    GGUF block layout.  All pointers are device pointers, work is ordered on
 *    the library stream, and each returns an int status (0 ok, <0 error;
 *    qmag_last_error() gives the text).  They are called from one host thread
 *    at a time, as the engine calls its seams (from qma_eval on the main
 *    thread, nn.c:2111-2286): they share the stream, workspaces and the
 *    recovery log.  The group 1 entries and the expert cache may be called
 *    from several threads at once.
 *
 * Weight formats: GGML Q4_K (type 12, 144-byte super-blocks) and Q6_K
 * (type 14, 210-byte super-blocks), src/qma.h:67-90.  Activation Q8_K is the
 * planar form of src/q8k.c:32-85: xq int8[n], xd f32[n/256], xsum i16[n/16].
 */
#ifndef QMA_GPU_H
#define QMA_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMAG_TYPE_Q4_K 12
#define QMAG_TYPE_Q6_K 14
/* Q6_K rows repacked by qmag_repack_q6k_dev for the matmul entries (a layout
   of this library with no counterpart in the reference or the GGUF; the same
   bytes per row, the same results as QMAG_TYPE_Q6_K). */
#define QMAG_TYPE_Q6_K_R 270

#define QMAG_OK 0
#define QMAG_ERR_HIP (-1)      /* a HIP runtime call failed                  */
#define QMAG_ERR_ARG (-2)      /* unsupported shape / type / null pointer    */
#define QMAG_ERR_NODEV (-3)    /* no gfx950 device, or qmag_init not called  */
#define QMAG_ERR_KERNEL (-4)   /* a kernel reported an internal guard trip   */
#define QMAG_ERR_REPLAYED (-5) /* decode calls were re-run after an expired
                                  wait; work queued after them (logits) is
                                  stale and must be queued again            */
/* Buffers passed to the MoE device entries must stay allocated, and the
   input of an out-of-place call (x != out) must keep its contents, until the
   next qmag_sync, qmag_d2h, sampler or host-buffer call, which checks for an
   expired wait: the library may re-run the calls issued since the previous
   check (see qmag_fused_recoveries), reading those inputs again.  The input
   of an in-place call (a stack, or x == out) is copied by the library before
   the call and needs no such care.  Only those MoE calls are re-run: other
   device work queued after them that read their outputs (an LM-head matmul,
   say) is re-queued by the caller when qmag_fused_recoveries rises. */

/* ------------------------------------------------------------------------ */
/* Reference-compatible entries                                              */
/* ------------------------------------------------------------------------ */

/* replaces qma_q8k_available, src/q8k.c:271-278 (qma.h:359) */
int qma_q8k_available(void);

/* replaces qma_q8k_quant, src/q8k.c:280-288 (qma.h:360) */
void qma_q8k_quant(const float *x, int n, int8_t *xq, float *xd, int16_t *xsum);

/* replaces qma_q8k_dot, src/q8k.c:305-316 (qma.h:361-362) */
float qma_q8k_dot(const void *row, int wtype, const int8_t *xq, const float *xd,
                  const int16_t *xsum, int n);

/* replaces qma_q8k_gateup, src/q8k.c:291-302 (qma.h:364-365) */
void qma_q8k_gateup(const void *g, const void *u, const int8_t *xq, const float *xd,
                    const int16_t *xsum, int n, float *gate, float *up);

/* The fp32 entries of src/quants.c (qma.h:348-351), same names, argument
   order and host-pointer semantics; the block pointers are raw GGUF bytes
   (the reference types them block_q4_K * / block_q6_K *, which link to the
   same symbols).  Only whole super-blocks are processed (k / 256, n / 256),
   as the reference loops.  They are skipped here when the engine's own
   qma.h, which declares them with its block types, was included first. */
#ifndef QMA_H
/* replaces dequantize_row_q4_K, src/quants.c:29-47 (qma.h:348) */
void dequantize_row_q4_K(const void *x, float *y, int64_t k);
/* replaces dequantize_row_q6_K, src/quants.c:50-75 (qma.h:349) */
void dequantize_row_q6_K(const void *x, float *y, int64_t k);
/* replaces dot_q4_K_f32, src/quants.c:80-105 (qma.h:350) */
float dot_q4_K_f32(const void *W, const float *x, int n);
/* replaces dot_q6_K_f32, src/quants.c:108-133 (qma.h:351) */
float dot_q6_K_f32(const void *W, const float *x, int n);
#endif

/* ------------------------------------------------------------------------ */
/* Runtime                                                                   */
/* ------------------------------------------------------------------------ */

/* Select device `device`, create the library stream.  Idempotent. */
int qmag_init(int device);
const char *qmag_last_error(void);
/* CU count, clock (kHz), HBM bytes, gfx arch name (>= 16 chars buffer). */
int qmag_device_info(int *n_cu, int *clock_khz, size_t *hbm_bytes, char *arch, int arch_len);

int qmag_malloc(void **dptr, size_t bytes);
int qmag_free(void *dptr);
int qmag_h2d(void *dst, const void *src, size_t bytes);      /* synchronous */
int qmag_d2h(void *dst, const void *src, size_t bytes);      /* synchronous */
int qmag_d2d(void *dst, const void *src, size_t bytes);      /* stream-ordered */
int qmag_memset(void *dst, int value, size_t bytes);         /* stream-ordered */
/* Wait for the library stream.  If a bounded wait of the persistent decode
   kernel expired since the last check, the affected calls are re-run first
   (see qmag_fused_recoveries); QMAG_ERR_KERNEL only if that fails too. */
int qmag_sync(void);

/* Timing on the library stream: record event `slot` (0..63) and read the
   elapsed milliseconds between two recorded slots (synchronises on b). */
int qmag_event_record(int slot);
int qmag_event_elapsed(int a, int b, float *ms);

/* Per-kernel timing (the QMA_TIMING role, nn.c:219-259, on the GPU): while
   enabled, every kernel the MoE entries launch is bracketed by HIP events on
   the library stream.  Kernel ids: 0 router, 1 top-k/Q8_K(x), 2 gate/up,
   3 Q8_K(h), 4 down+combine, 5 fused decode, 6 matvec (matmul entries),
   7 Q8_K quantisation (every launch of it), 8 grouping (prefill), 9 combine
   (prefill).  qmag_prof_read synchronises and
   returns the launch count and summed milliseconds of one id. */
int qmag_prof_enable(int on);
int qmag_prof_read(int kernel_id, long *count, double *total_ms);

/* Options.  QMAG_OPT_FUSED (default 1): batch-1 MoE decode of the qwen35moe
   shape (n_embd 2048, n_ff 512, n_used <= 8, equal down types) runs as one
   persistent kernel launch per token through all layers; 0 selects the
   per-stage launch sequence (same results within the fp32 tolerance). */
#define QMAG_OPT_FUSED 1
/* QMAG_OPT_TRACE (default 0): the fused decode kernel records, per
   workgroup and layer (the first 64 layers of a launch), up to 8 phase
   timestamps of the 100 MHz device
   real-time counter (slot 0 is the layer start; the other slots mark the
   phases of the workgroup's role, 0 where it has none); qmag_trace_read
   copies the last launch's [512][n_layer][8] uint64 array to the host. */
#define QMAG_OPT_TRACE 2
/* QMAG_OPT_COOP (default 0): 1 launches the fused decode kernel with
   hipLaunchCooperativeKernel (co-residency of its 512 workgroups guaranteed
   by the runtime); 0 launches it as an ordinary kernel after the occupancy
   check that makes it eligible (two workgroups per CU fit, so all are
   resident when the device is otherwise idle; a workgroup that were not
   would make the others exhaust their bounded waits, reported as
   QMAG_ERR_KERNEL by qmag_sync, never a hang).  The ordinary launch is the
   default: equally fast, and visible to rocprofv3's kernel tracing. */
#define QMAG_OPT_COOP 3
/* QMAG_OPT_GROUPED (default 1): qmag_moe_ffn_dev with T >= 8 tokens (the
   prefill form) runs the grouped expert GEMM: (token, slot) pairs bucketed
   by expert into chunks of up to 64, gate/up and down as int8 MFMA tiles of
   16 pairs, each expert's weights read once per chunk; 0 selects the
   per-token launch sequence (same results within the fp32 tolerance). */
#define QMAG_OPT_GROUPED 4
/* QMAG_OPT_TEST_ABORT (write-only; tests of the recovery path): value n > 0
   makes the n-th persistent decode launch from now find its abort word
   already set, as if its wait had expired, so it and the launches after it
   exit without output and the next qmag_sync / qmag_d2h re-runs them through
   the launch sequence; 0 cancels. */
#define QMAG_OPT_TEST_ABORT 5
int qmag_set_option(int option, int value);
/* Persistent decode launches whose bounded cross-workgroup wait expired (50 ms
   each; a workgroup that is not resident, e.g. CUs held by another process,
   is the one way to get there) are reported at the next qmag_sync or
   qmag_d2h, which then re-run the affected calls -- every call issued since
   the previous status check, from the failing launch on -- through the
   per-stage launch sequence, restoring in-place inputs from copies taken
   before the calls ran, and return QMAG_OK.  This counts such recoveries. */
int qmag_fused_recoveries(long *count);
int qmag_trace_read(void *dst, size_t bytes);

/* ------------------------------------------------------------------------ */
/* Device entries                                                            */
/* ------------------------------------------------------------------------ */

/* Q8_K quantization of T rows of n floats (n % 256 == 0); q8k.c:34-85. */
int qmag_q8k_quant_dev(const float *x, int n, int T, int8_t *xq, float *xd, int16_t *xsum);

/* out[t][r] = row_r(W) . Q8_K(x[t]) for pre-quantised activations;
   mm_worker, nn.c:276-289.  n_in: any multiple of 256 (powers of two up to
   8192 run the tiled kernel, other lengths a kernel of one wave per row). */
int qmag_matmul_q8k_dev(const int8_t *xq, const float *xd, const int16_t *xsum,
                        const void *W, int n_in, int n_out, int T, int wtype, float *out);

/* matmul seam, nn.c:307-345: quantise each x[t] once, then the matvec (for
   T = 1 and n_in a power of two up to 8192 a single launch: the matvec
   quantises x itself, bit-identically).  n_in: any multiple of 256. */
int qmag_matmul_dev(const float *x, const void *W, int n_in, int n_out, int T, int wtype,
                    float *out);

/* Several matmuls over one activation vector in one launch (T = 1): out[i]
   = W[i] . Q8_K(x) for i < n_mat <= QMAG_MV_GROUP_MAX, every matrix n_in
   wide (a power of two from 256 to 8192) and of its own wtype (Q4_K, Q6_K or
   QMAG_TYPE_Q6_K_R).  For the projections the engine computes from the same
   x, one matmul() call each in the reference: q, k and v (nn.c:2111-2113),
   and qkv, the attention gate and beta / alpha of the recurrent layers
   (nn.c:2162, 2165-2170).  No counterpart in the reference: it saves the
   per-launch cost of the separate calls.  W, n_out, wtype and out are host
   arrays of n_mat entries (W and out holding device pointers).  Results are
   bit-identical to separate qmag_matmul_dev calls.  QMAG_ERR_ARG when the
   matrices need more than 65,536 waves together (call them separately).
   It allocates nothing: x is quantised inside the kernel and the matrix
   table travels as kernel arguments. */
#define QMAG_MV_GROUP_MAX 4
int qmag_matmul_group_dev(const float *x, int n_in, int n_mat, const void *const *W, const int *n_out,
                          const int *wtype, float *const *out);

/* Repack n_out Q6_K rows of n_in weights (n_in a multiple of 2048) from the
   block layout (block_q6_K, qma.h; what the GGUF holds) into the row layout
   the matmul entries read fastest, for wtype QMAG_TYPE_Q6_K_R: per row, each
   super-block's 16-byte low ql task pieces, then the high ones, then the qh
   bytes, the scales and the d values of every super-block (n_out * n_in / 256
   * 210 bytes, as before).  No counterpart in the reference: a one-time
   transform at weight upload for large Q6_K matrices such as the LM head
   (nn.c:2243).  dst: device memory of the same size, 16-byte aligned, either
   src itself (the rows are repacked in place, each through LDS, so no second
   copy of the matrix is needed; rows of at most 65,536 bytes, n_in <= 79,872)
   or not overlapping it.  Results of qmag_matmul_dev / qmag_matmul_q8k_dev /
   qmag_matmul_noalloc_dev on the repacked rows are bit-identical to those on
   the block layout. */
int qmag_repack_q6k_dev(const void *src, void *dst, int n_in, int n_out);

/* The matmul seam without any allocation (no counterpart in the reference):
   for callers that cannot allocate -- code under HIP graph capture, serving
   loops that forbid hipMalloc.  Same arguments and results as
   qmag_matmul_dev (the same kernels; bit-identical output), but the Q8_K
   staging of the T activation rows lives in a fixed 2.4 MB array of device
   memory each GPU holds for the life of the process, instead of a workspace
   grown with hipMalloc.  Limit: T * n_in <= 2^21 (QMAG_ERR_ARG beyond).
   Calls that overlap on one GPU share that array and race; issue them on the
   library stream (every qmag entry does) and not from several threads at
   once. */
#define QMAG_NOALLOC_MAX_VALUES (1 << 21)
int qmag_matmul_noalloc_dev(const float *x, const void *W, int n_in, int n_out, int T, int wtype,
                            float *out);

/* Dequantisation of n weights (n % 256 == 0) to f32, bit-identical to
   dequantize_row_q4_K / dequantize_row_q6_K (src/quants.c:29-75); the weight
   definition embed_row uses (nn.c:2044-2054). */
int qmag_dequant_dev(const void *W, int wtype, int64_t n, float *y);

/* The fp32 dequantise-then-dot matmul (dot_q4_K_f32 / dot_q6_K_f32 per row,
   src/quants.c:80-133; the QMA_NOQ8K path, nn.c:393-407, 475-492):
   out[t][r] = sum_i deq(W_r)_i * x[t][i], no activation quantisation.
   n_in: any multiple of 256 (rows longer than 8192 values are taken in
   8192-value chunks whose partial sums are added in chunk order). */
int qmag_matmul_f32_dev(const float *x, const void *W, int n_in, int n_out, int T, int wtype,
                        float *out);

/* One MoE FFN layer's tensors, resident in HBM (device pointers).  Field
   meaning follows qma_t.layers[il] (src/qma.h:202-218); expert slabs are
   expert-major as in the GGUF (src/gguf.c:268-271, nn.c:668-674). */
typedef struct qmag_moe_layer {
    int n_embd;                 /* 2048 */
    int n_ff;                   /* 512  */
    int n_expert;               /* 256  */
    int n_used;                 /* 8    */
    const float *gate_inp;      /* f32 [n_expert][n_embd] router (ffn_gate_inp)       */
    const float *router_bias;   /* f32 [n_expert] or NULL: synthetic logit skew        */
    const void *gate_exps;      /* Q4_K, n_expert x n_ff rows of n_embd               */
    const void *up_exps;        /* Q4_K, same shape                                   */
    const void *down_exps;      /* Q4_K/Q6_K, n_expert x n_embd rows of n_ff          */
    int t_down_exps;
    const float *gate_inp_shexp;/* f32 [n_embd] shared-expert gate                    */
    const void *gate_shexp;     /* Q4_K, n_ff rows of n_embd                          */
    const void *up_shexp;
    const void *down_shexp;     /* Q4_K/Q6_K, n_embd rows of n_ff                     */
    int t_down_shexp;
} qmag_moe_layer;

/* moe_ffn seam, nn.c:509-649: out[t] = sum_k w_k * expert_k(x[t]) +
   sigmoid(gs) * shared(x[t]) for T tokens (x, out: f32 [T][n_embd]). */
int qmag_moe_ffn_dev(const qmag_moe_layer *L, const float *x, float *out, int T);

/* The moe_ffn seam on host buffers, as the engine calls it (nn.c:2246-2252:
   moe_ffn(m, il, x, ..., out, T) with host pointers, out read at once): x and
   out are host memory, f32 [T][n_embd].  x goes to the device through pinned
   staging on the library stream, the layer runs as qmag_moe_ffn_dev, out
   comes back the same way, and the call returns after one stream
   synchronisation (the persistent decode kernel's status read in the same
   pass; an expired wait is recovered before out is returned).  Synchronous;
   one call at a time (an internal lock). */
int qmag_moe_ffn_host(const qmag_moe_layer *L, const float *x, float *out, int T);

/* The moe_ffn seam with q8k off (QMA_NOQ8K, or no q8k; nn.c:585): the same
   routing, then moe_expert_one and moe_shared (nn.c:393-407, 475-492) --
   expert h on fp32 x, the shared gate sigmoid(wsh . x) on fp32 x, every dot
   dequantise-then-dot in fp32 -- and the combine in the reference's order.
   Replaces the per-row dot_q4_K_f32 / dot_q6_K_f32 calls of that path with
   three launches per call.  Same shapes and stage buffers
   (qmag_moe_last_stage) as qmag_moe_ffn_dev; T <= 65535. */
int qmag_moe_ffn_f32_dev(const qmag_moe_layer *L, const float *x, float *out, int T);

/* Decode over a stack of MoE layers: for each of n_tok tokens in turn,
   x[t] <- x[t] + moe_l(x[t]) for l = 0..n_layer-1 (the residual add of
   qma_eval, nn.c:2252).  x: f32 [n_tok][n_embd], updated in place.  Layers
   may differ in down type (Q4_K/Q6_K per tensor, as GGUF quant mixes have
   them): the persistent decode kernel takes each run of consecutive layers
   it can, the launch sequence the others. */
int qmag_moe_stack_dev(const qmag_moe_layer *layers, int n_layer, float *x, int n_tok);

/* Stage outputs of the last qmag_moe_ffn_dev / qmag_moe_stack_dev layer
   (device pointers the library owns, valid until the next call):
   logits f32[n_expert], sel i32[n_used], w f32[n_used], gs f32[1],
   h f32[(n_used+1)][n_ff] (slot n_used = shared expert) for token 0; after
   a qmag_moe_ffn_dev call on T > 1 tokens each array holds all T tokens,
   token-major ([T][n_expert], [T][n_used], ..., [T][n_used+1][n_ff]). */
int qmag_moe_last_stage(const float **logits, const int **sel, const float **w,
                        const float **gs, const float **h);

/* ------------------------------------------------------------------------ */
/* GGUF v3 weights into HBM residency (the loader role of src/gguf.c)        */
/* ------------------------------------------------------------------------ */

/* An opened, indexed GGUF file: mapped read-only; tensor data is not read
   until a tensor is uploaded. */
typedef struct qmag_gguf qmag_gguf;

/* Open and index a GGUF (v2/v3) file: header, integer metadata (keys with the
   qwen35moe./qwen35. architecture prefix stripped, gguf.c:146-153), the tensor
   table and the aligned data section (general.alignment, default 32).  As
   qma_load (gguf.c:104-283) it fails (QMAG_ERR_ARG, message in
   qmag_last_error) on a bad magic, truncated or corrupt tables, a tensor
   outside the file, a first dimension that is not a whole number of blocks,
   or a tensor type other than F32 (0), Q4_K (12) and Q6_K (14).  Needs no
   GPU. */
int qmag_gguf_open(const char *path, qmag_gguf **out);
void qmag_gguf_close(qmag_gguf *g);
/* An integer metadata value ("block_count", "expert_count", ...; the
   architecture prefix is optional). */
int qmag_gguf_meta_u64(const qmag_gguf *g, const char *key, uint64_t *val);
/* A tensor's GGML type, dimensions (ne[0] fastest) and host bytes in the
   mapping (valid until qmag_gguf_close). */
int qmag_gguf_tensor(const qmag_gguf *g, const char *name, int *type, int64_t ne[3], const void **data,
                     size_t *nbytes);
/* Copy one tensor to a new device allocation (free with qmag_free), e.g.
   output.weight for the LM-head matmul (nn.c:2286). */
int qmag_gguf_upload_tensor(const qmag_gguf *g, const char *name, void **dptr, int *type, int64_t ne[3]);
/* Upload layer il's MoE FFN tensors -- blk.<il>.ffn_{gate_inp, gate_exps,
   up_exps, down_exps, gate_inp_shexp, gate_shexp, up_shexp, down_shexp}
   (gguf.c:318-326) -- each as one contiguous copy (expert-major slabs,
   gguf.c:268-271), and fill *L with the device pointers, the shapes from the
   tensor dimensions, the per-layer down types, and n_used from
   expert_used_count (8 if absent, qma.h:58).  Gate/up must be Q4_K and the
   expert and shared hidden sizes equal. */
int qmag_gguf_upload_moe_layer(const qmag_gguf *g, int il, qmag_moe_layer *L);
/* Free the device tensors of a layer filled by qmag_gguf_upload_moe_layer. */
int qmag_gguf_free_moe_layer(qmag_moe_layer *L);
/* The expert cache's fetch callback over an opened file (user = the
   qmag_gguf *): the record of (layer, expert) copied from the mapping, as
   expert_fetch (nn.c:1564-1595) preads it; -1 when the layer or expert does
   not exist.  qmag_gguf_expert_record_bytes gives the largest layer's record
   size (down types vary per layer, nn.c:1601-1605); a cache given this
   callback must have records at least that large, and refuses it otherwise
   (io_start returns QMAG_ERR_ARG, a get that would read returns NULL). */
int qmag_gguf_fetch_expert(void *user, int layer, int expert, uint8_t *dst);
int qmag_gguf_expert_record_bytes(const qmag_gguf *g, size_t *rec);

/* ------------------------------------------------------------------------ */
/* Expert paging: a bounded cache of expert records in HBM (the role of      */
/* qma_ecache, src/ecache.h:95-123, for models larger than the device)       */
/* ------------------------------------------------------------------------ */

/* The reference's fetch callback type (qma_fetch_fn, ecache.h:29-32): fill
   dst (host memory, rec_bytes) with the record of (layer, expert) -- gate,
   up and down slabs back to back (expert_fetch, nn.c:1564-1595) -- and
   return 0.  Called from the reader threads and the calling thread, so it
   must be safe to enter concurrently. */
typedef int (*qmag_fetch_fn)(void *user, int layer, int expert, uint8_t *dst);
typedef struct qmag_ecache qmag_ecache;
typedef struct {
    uint64_t hits, misses, bytes_read, evictions, prefetched, spec_issued;
    int n_slots;
    size_t rec_bytes, slot_bytes;
} qmag_ecache_counters;

/* replaces qma_ecache_init (ecache.h:95-96): budget / rec_bytes slots of
   device memory (at least 4; none when the budget holds no record), policy
   0 LFRU, 1 LRU.  The cache is allocated by the library (*c). */
int qmag_ecache_init(qmag_ecache **c, size_t budget_bytes, size_t rec_bytes, int policy);
/* replaces qma_ecache_free / qma_ecache_clear (ecache.h:97-98) */
void qmag_ecache_free(qmag_ecache *c);
void qmag_ecache_clear(qmag_ecache *c);
/* replaces qma_ecache_get (ecache.h:100-105): the record's DEVICE address,
   reading it through fetch on a miss or waiting for a read a hint started;
   NULL on failure.  The bytes are in place when it returns; they stay valid
   for work queued on the library stream before the next get. */
const uint8_t *qmag_ecache_get(qmag_ecache *c, int layer, int expert, qmag_fetch_fn fetch, void *user);
/* replaces qma_ecache_hold / qma_ecache_release (ecache.h:107-114): held
   records stay valid for work queued before the release. */
const uint8_t *qmag_ecache_hold(qmag_ecache *c, int layer, int expert, qmag_fetch_fn fetch, void *user);
void qmag_ecache_release(qmag_ecache *c);
/* replaces qma_ecache_io_start / _io_stop (ecache.h:116-123): nthreads
   (<= 8) reader threads, each with pinned staging; depth reads in flight. */
int qmag_ecache_io_start(qmag_ecache *c, qmag_fetch_fn fetch, void *user, int nthreads, int depth);
void qmag_ecache_io_stop(qmag_ecache *c);
/* replaces qma_ecache_hint / qma_ecache_prefetch (ecache.h:125-134) */
void qmag_ecache_hint(qmag_ecache *c, int layer, const int *ids, int n);
void qmag_ecache_prefetch(qmag_ecache *c, int layer, const int *ids, int n);
/* No counterpart in the reference (its tests read the struct): wait until
   every queued read has landed; the counters of qma_ecache; the slot that
   holds (layer, expert) or -1; a slot's device address. */
int qmag_ecache_drain(qmag_ecache *c);
int qmag_ecache_stats(const qmag_ecache *c, qmag_ecache_counters *out);
int qmag_ecache_slot_of(const qmag_ecache *c, int layer, int expert);
const uint8_t *qmag_ecache_slot_ptr(const qmag_ecache *c, int slot);

/* moe_ffn with the expert cache on (nn.c:553-571, 677-694): the router and
   top-k on the device, the distinct selected experts hinted to the cache in
   (token, slot) order, then per token its n_used records held, the expert
   stages run on them, and released.  L's gate_exps/up_exps/down_exps are not
   used (may be NULL); the router and the shared expert are resident.  One
   host synchronisation per call (the selection). */
int qmag_moe_ffn_paged_dev(const qmag_moe_layer *L, qmag_ecache *c, int il, qmag_fetch_fn fetch, void *user,
                           const float *x, float *out, int T);

/* ------------------------------------------------------------------------ */
/* Sampling on the device (src/sampler.c), logits resident in HBM            */
/* ------------------------------------------------------------------------ */

/* The sampler state, field for field the layout of sampler_t (qma.h:279-287),
   so a sampler_t * may be passed where a qmag_sampler * is expected. */
typedef struct qmag_sampler {
    uint64_t seed;
    float temp;
    int top_k;
    float top_p;
    float repeat_penalty;
    int last_tokens[64];
    int n_last;
} qmag_sampler;

/* sampler_candidates (sampler.c:36-95, qma.h:338) on device logits: the
   repeat penalty per occurrence in last_tokens, division by temp when
   temp > 0, and the k = clamp(top_k, 1, min(n_vocab, max_k)) largest values
   in descending order, ids and values copied to the host arrays ids[k],
   lgs[k] (agent.c:935 asks for 40).  Returns k (>= 1) or a negative status.  max_k <= 64,
   n_vocab <= 524288.  Equal values are ordered by ascending id (the
   reference's order among exact ties follows its heap). */
int qmag_sampler_candidates_dev(int n_vocab, const float *logits, const qmag_sampler *s, int *ids, float *lgs,
                                int max_k);
/* sampler_candidates followed by sampler_pick (sampler.c:100-134) on the
   unmasked candidates, both on the device; only the token id comes back.
   Matches the reference call pair with no grammar mask between them: the
   greedy answer at temp <= 0; otherwise the softmax with a double sum, the
   top-p cut, one xorshift64* draw (s->seed advances) and the pick joining
   s->last_tokens (the last 64 kept).  Replaces the pair at agent.c:935-955
   when no grammar mask runs (tool_mode off); with the mask, call
   qmag_sampler_candidates_dev and the host's sampler_pick on its 40.
   Both sampler entries first settle persistent decode calls still pending
   (as qmag_sync does); if that re-ran any of them after an expired wait,
   the logits, computed on the stream from their earlier outputs, are stale:
   the call then samples nothing, leaves *s unchanged and returns
   QMAG_ERR_REPLAYED, and the caller recomputes the logits (the LM head) and
   calls again. */
int qmag_sampler_sample_dev(int n_vocab, const float *logits, qmag_sampler *s, int max_k, float top_p,
                            int *token);

/* ------------------------------------------------------------------------ */
/* Synthetic inputs (bench/test utilities; not part of the reference)        */
/* ------------------------------------------------------------------------ */

/* f32 ~ N(mean, std) from a counter-based generator keyed by seed. */
int qmag_synth_normal(uint64_t seed, size_t n, float mean, float std, float *out);
/* N(0, std) weights generated and quantised to Q4_K / Q6_K in one pass
   (n % 256 == 0); same quantiser as qmag_quantize_dev. */
int qmag_synth_weights(uint64_t seed, size_t n, float std, int wtype, void *out);
/* fp32 -> Q4_K / Q6_K with the build's quantiser (n % 256 == 0). */
int qmag_quantize_dev(const float *x, size_t n, int wtype, void *out);

#ifdef __cplusplus
}
#endif
#endif
