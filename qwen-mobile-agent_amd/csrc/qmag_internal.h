// qmag_internal.h -- host-side internals shared by the library's units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

#include "../../include/qma_gpu.h"
#include "qmag_device.h"

namespace qmag {

struct Ctx {
    // set (release) once the fields below are filled in; read with acquire
    // by every entry point, from any thread
    std::atomic<bool> ready{false};
    int dev = -1;
    hipStream_t stream = nullptr;
    hipEvent_t ev[64] = {};
    int n_cu = 0;
    int clock_khz = 0;
    size_t hbm = 0;
    char arch[64] = {0};
};

Ctx &ctx();
// status helpers: record a message for qmag_last_error() and return code
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char *what, const char *file, int line);
int require_ready();

#define QMAG_HIP(call)                                                        \
    do {                                                                      \
        hipError_t _e = (call);                                               \
        if (_e != hipSuccess) return qmag::hip_fail(_e, #call, __FILE__, __LINE__); \
    } while (0)

// Grow-on-demand device workspace, one buffer per slot (never shrinks).
enum WsSlot {
    WS_XQ = 0, WS_XD, WS_XS,        // Q8_K of the layer input(s)
    WS_LOGITS, WS_SEL, WS_W, WS_GS, // router outputs
    WS_H, WS_HQ, WS_HD, WS_HS,      // expert hidden state and its Q8_K
    WS_LAYERS,                      // device copy of layer descriptors
    WS_OUT,                         // layer output scratch
    WS_FLAGS,                       // kernel status / counters
    WS_GRP,                         // grouped prefill: bucket counts/offsets, pair permutation
    WS_Y,                           // grouped prefill: per-pair down outputs
    WS_XMB,                         // grouped prefill: Q8_K(x) sub-block sums times the block scale
    WS_SAMP,                        // sampler: per-chunk candidates and the merged list
    WS_HOSTIO,                      // qmag_moe_ffn_host: the device copies of x and out
    WS_F32PART,                     // fp32 matmul rows longer than one LDS chunk: per-chunk partials
    WS_COUNT
};
void *workspace(int slot, size_t bytes, int *status);

// ---- per-kernel event timing (qmag_prof_*) ----
enum ProfId {
    PROF_ROUTER = 0, PROF_TOPK, PROF_GATEUP, PROF_HQUANT, PROF_DOWN, PROF_FUSED, PROF_MATVEC, PROF_Q8K,
    PROF_GROUP, PROF_COMBINE,
    PROF_COUNT
};
bool prof_on();
void prof_begin(int id, hipStream_t s);
void prof_end(int id, hipStream_t s);
// while one is alive on a thread, that thread's launches are not timed
struct ProfSuspend {
    ProfSuspend();
    ~ProfSuspend();
};
// the allocation-free matmul's scratch address, looked up per device
int noalloc_setup(int dev);

// ---- launchers (all stream-ordered on s) ----
int launch_q8k_quant(const float *x, int nblocks, int8_t *xq, float *xd, int16_t *xsum,
                     hipStream_t s);
int launch_matvec(const int8_t *xq, const float *xd, const int16_t *xsum, const void *W,
                  int n_in, int n_out, int T, int wtype, float *out, hipStream_t s);
// T = 1 with x in f32: the matvec quantises x to Q8_K itself (bit-identical);
// available for the row lengths matvec_x_supported() accepts
bool matvec_x_supported(int n_in);
int launch_repack_q6k(const void *src, void *dst, int n_in, int n_out, hipStream_t s);
// up to QMAG_MV_GROUP_MAX matrices over one x at T = 1, one launch
struct MvGroup {
    const uint8_t *W[QMAG_MV_GROUP_MAX];
    float *out[QMAG_MV_GROUP_MAX];
    int n_out[QMAG_MV_GROUP_MAX];
    int wtype[QMAG_MV_GROUP_MAX];
    int wave0[QMAG_MV_GROUP_MAX + 1];   // first wave of each matrix; wave0[n] = all waves
    int n;
};
constexpr int QMAG_MV_GROUP_MAX_WAVES = 1 << 16;
int launch_matvec_group(const float *x, int n_in, int n_mat, const void *const *W, const int *n_out,
                        const int *wtype, float *const *out, hipStream_t s);
int launch_matvec_x(const float *x, const void *W, int n_in, int n_out, int wtype, float *out, hipStream_t s);
// fp32 path of quants.c (qmag_quants.hip)
int launch_dequant(const void *W, int wtype, long n, float *y, hipStream_t s);
int launch_f32dot(const float *x, const void *W, int n_in, int n_out, int T, int wtype, float *out,
                  hipStream_t s);
int moe_ffn(const qmag_moe_layer *L, const float *x, float *out, int T, const float *resid,
            hipStream_t s);
// need_exps = false: the routed expert slabs may be null (paged experts)
int moe_check_layer(const qmag_moe_layer *L, bool need_exps = true);

// grouped prefill (qmag_prefill.hip)
// part[kc][T][E]: x . Wr^T over 256-wide k chunk kc (no bias)
int launch_router_mfma(const qmag_moe_layer *L, const float *x, int T, float *part, hipStream_t s);
int moe_grouped(const qmag_moe_layer *L, int T, const int *sel, const float *w, const float *gs,
                const int8_t *xq, const float *xd, const float *xmb, float *h, int8_t *hq, float *hd,
                int16_t *hs, const float *resid, float *out, hipStream_t s);

// persistent single-launch decode (qmag_fused.hip)
bool fused_eligible(const qmag_moe_layer *L, int n_layer);
// n_tok tokens through n_layer layers, one launch per token: x (and out,
// when not null: one layer, out = moe(x)) are [n_tok][2048]
int fused_call(const qmag_moe_layer *L, int n_layer, float *x, float *out, int n_tok, hipStream_t s);
// a stack fused_eligible refuses as a whole: its eligible runs fused, the rest
// through the launch sequence; 1 when no layer qualifies (nothing launched)
int fused_stack_runs(const qmag_moe_layer *L, int n_layer, float *x, int n_tok, hipStream_t s);
long fused_recoveries();
void fused_test_abort_next(int nth);
// the launch sequence wrote the latest stage outputs (qmag_moe_last_stage)
void moe_note_sequence_ran();
int fused_status();
int fused_abort_copy(int *host, hipStream_t s);
int fused_status_word(int word);
// true when a persistent decode launch was issued since the last status check
bool fused_pending();
int fused_trace_read(void *dst, size_t bytes);
int fused_last_stage(const float **logits, const int **sel, const float **w, const float **gs,
                     const float **h);

// library options (qmag_set_option)
int option(int id);

}  // namespace qmag
