// qmag_quants.hip -- the fp32 half of the k-quant path (src/quants.c):
// Q4_K / Q6_K dequantisation (quants.c:29-75, the closed-form weight
// definition, also what embed_row uses, nn.c:2044-2054) and the
// dequantise-then-dot fp32 matvec (quants.c:80-133; the QMA_NOQ8K path of
// moe_expert_one / moe_shared, nn.c:393-407, 475-492).
//
// Both are HBM-bound streams over the GGUF block bytes.  Dequantisation is
// bit-identical to the reference's unfused fp32 form: w = d1*q - m1 with
// d1 = d*sc and m1 = dmin*m rounded separately (Q4_K), w = (d*sc)*q (Q6_K);
// the multiplies and the subtraction are issued as separately rounded
// operations so the compiler cannot contract them into an FMA.
#include "qmag_internal.h"

namespace qmag {

// ------------------------------------------------------------ dequant ----
// One wave per 256-value super-block; lane l writes elements 4l..4l+3.
template <int WT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ W, long nblocks,
                                                      float *__restrict__ y)
{
    const long blk = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (blk >= nblocks) return;                 // wave-uniform
    const int lane = lane_id();
    const int e0 = 4 * lane;
    float4 o;
    if constexpr (WT == QMAG_TYPE_Q4_K) {
        const uint8_t *b = W + blk * Q4K_BYTES;
        const uint4 hdr = ld16(b);
        const int j = e0 >> 5;                  // sub-block 0..7
        const int g = j >> 1;                   // 64-value group: bytes qs[32g..32g+31]
        const uint32_t qw = ld4(b + 16 + 32 * g + (e0 & 31));
        uint32_t sc, m;
        q4_scale_min(j, hdr.y, hdr.z, hdr.w, sc, m);
        const float d = h2f(hdr.x & 0xffff), dmin = h2f(hdr.x >> 16);
        const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
        const uint32_t nib = (j & 1) ? (qw >> 4) & 0x0F0F0F0Fu : qw & 0x0F0F0F0Fu;
        o.x = __fsub_rn(__fmul_rn(d1, (float)(nib & 255)), m1);
        o.y = __fsub_rn(__fmul_rn(d1, (float)((nib >> 8) & 255)), m1);
        o.z = __fsub_rn(__fmul_rn(d1, (float)((nib >> 16) & 255)), m1);
        o.w = __fsub_rn(__fmul_rn(d1, (float)(nib >> 24)), m1);
    } else {
        const uint8_t *b = W + blk * Q6K_BYTES;
        const int n = e0 >> 7, r = e0 & 127, Q = r >> 5, l = r & 31;
        const uint32_t lw = ld4(b + 64 * n + 32 * (Q & 1) + l);
        const uint32_t hw = ld4(b + 128 + 32 * n + l);
        const int sc = (int)(int8_t)b[192 + 8 * n + (l >> 4) + 2 * Q];
        const float d = h2f(ld2(b + 208));
        const float ds = __fmul_rn(d, (float)sc);
        const uint32_t lo = (Q >= 2 ? lw >> 4 : lw) & 0x0F0F0F0Fu;
        const uint32_t hi = (hw >> (2 * Q)) & 0x03030303u;
        const uint32_t q = lo | (hi << 4);
        o.x = __fmul_rn(ds, (float)((int)(q & 255) - 32));
        o.y = __fmul_rn(ds, (float)((int)((q >> 8) & 255) - 32));
        o.z = __fmul_rn(ds, (float)((int)((q >> 16) & 255) - 32));
        o.w = __fmul_rn(ds, (float)((int)(q >> 24) - 32));
    }
    ((float4 *)(y + blk * QK_K))[lane] = o;
}

int launch_dequant(const void *W, int wtype, long n, float *y, hipStream_t s)
{
    if (n <= 0 || n % QK_K) return fail(QMAG_ERR_ARG, "dequant: n=%ld is not a positive multiple of 256", n);
    if (!W || !y) return fail(QMAG_ERR_ARG, "dequant: null pointer");
    const long nb = n / QK_K;
    const long wgs = (nb + 3) / 4;
    if (wtype == QMAG_TYPE_Q4_K)
        hipLaunchKernelGGL(dequant_kernel<QMAG_TYPE_Q4_K>, dim3((unsigned)wgs), dim3(256), 0, s,
                           (const uint8_t *)W, nb, y);
    else if (wtype == QMAG_TYPE_Q6_K)
        hipLaunchKernelGGL(dequant_kernel<QMAG_TYPE_Q6_K>, dim3((unsigned)wgs), dim3(256), 0, s,
                           (const uint8_t *)W, nb, y);
    else
        return fail(QMAG_ERR_ARG, "dequant: unsupported wtype %d", wtype);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// ------------------------------------------------------ fp32 matvec ----
// out[t][r] = sum_i deq(W[r])_i * x[t][i].  x of one token sits in LDS; a row
// is split into 64-value tasks (f32_task) spread over LPR lanes, each lane
// looping over its tasks.  Grid: (row chunks, T).  A launch covers nb
// super-blocks of each row: the whole row, or for rows longer than the LDS
// chunk one chunk of it (x_stride and rb then give the full rows' strides).
constexpr int F32_MAX_IN = 8192;

template <int WT, int LPR>
__global__ __launch_bounds__(256) void f32dot_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                     float *__restrict__ out, int nb, int n_out, int x_stride,
                                                     size_t rb)
{
    __shared__ __align__(16) float s_x[F32_MAX_IN];
    const int t = (int)blockIdx.y;
    const int n_in = nb * QK_K;
    const float *xt = x + (size_t)t * x_stride;
    for (int i = (int)threadIdx.x; i < n_in / 4; i += (int)blockDim.x)
        ((float4 *)s_x)[i] = ldg4(xt + 4 * i);
    __syncthreads();
    const int lane = lane_id(), sub = lane % LPR;
    const int rows_per_wave = 64 / LPR;
    const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nwave = (int)((gridDim.x * blockDim.x) >> 6);
    const int ntask = 4 * nb;
    for (int base = wave * rows_per_wave; base < n_out; base += nwave * rows_per_wave) {
        const int row = base + lane / LPR;
        float v = 0.0f;
        if (row < n_out)
            for (int tk = sub; tk < ntask; tk += LPR) v += f32_task<WT>(W + (size_t)row * rb, tk, s_x);
        v = group_sum<LPR>(v);
        if (sub == 0 && row < n_out) out[(size_t)t * n_out + row] = v;
    }
}

template <int WT>
static int launch_f32dot_t(const float *x, const void *W, int nb, int n_out, int T, float *out, hipStream_t s,
                           int x_stride, size_t rb)
{
    const int ntask = 4 * nb;
    const int lpr = ntask >= 64 ? 64 : ntask > 16 ? 32 : ntask > 8 ? 16 : ntask > 4 ? 8 : 4;
    const long rows_per_wg = 4L * (64 / lpr);
    long wgs = ((long)n_out + rows_per_wg - 1) / rows_per_wg;
    const long cap = (long)(ctx().n_cu > 0 ? ctx().n_cu : 256) * 8 / (T < 8 ? T : 8);
    if (wgs > cap) wgs = cap;
    const dim3 grid((unsigned)wgs, (unsigned)T);
    const uint8_t *w = (const uint8_t *)W;
    switch (lpr) {
    case 4: hipLaunchKernelGGL((f32dot_kernel<WT, 4>), grid, dim3(256), 0, s, w, x, out, nb, n_out, x_stride, rb); break;
    case 8: hipLaunchKernelGGL((f32dot_kernel<WT, 8>), grid, dim3(256), 0, s, w, x, out, nb, n_out, x_stride, rb); break;
    case 16: hipLaunchKernelGGL((f32dot_kernel<WT, 16>), grid, dim3(256), 0, s, w, x, out, nb, n_out, x_stride, rb); break;
    case 32: hipLaunchKernelGGL((f32dot_kernel<WT, 32>), grid, dim3(256), 0, s, w, x, out, nb, n_out, x_stride, rb); break;
    default: hipLaunchKernelGGL((f32dot_kernel<WT, 64>), grid, dim3(256), 0, s, w, x, out, nb, n_out, x_stride, rb); break;
    }
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

// out[i] = part[0][i] + part[1][i] + ... in chunk order, from 0.0f: the order
// in which the host-pointer entries add their chunks
__global__ __launch_bounds__(256) void f32_chunk_sum_kernel(const float *__restrict__ part, int nch, long n,
                                                            float *__restrict__ out)
{
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
        float v = 0.0f;
        for (int c = 0; c < nch; c++) v += part[(size_t)c * n + i];
        out[i] = v;
    }
}

int launch_f32dot(const float *x, const void *W, int n_in, int n_out, int T, int wtype, float *out,
                  hipStream_t s)
{
    if (n_in <= 0 || n_in % QK_K || n_out <= 0 || T <= 0 || T > 65535)
        return fail(QMAG_ERR_ARG, "f32 matvec: n_in=%d (a multiple of 256) n_out=%d T=%d", n_in, n_out, T);
    if (!x || !W || !out) return fail(QMAG_ERR_ARG, "f32 matvec: null pointer");
    if (wtype != QMAG_TYPE_Q4_K && wtype != QMAG_TYPE_Q6_K)
        return fail(QMAG_ERR_ARG, "f32 matvec: unsupported wtype %d", wtype);
    const size_t bb = wtype == QMAG_TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES, rb = (size_t)(n_in / QK_K) * bb;
    auto launch = [&](const float *xc, const uint8_t *wc, int nbc, float *o) {
        return wtype == QMAG_TYPE_Q4_K ? launch_f32dot_t<QMAG_TYPE_Q4_K>(xc, wc, nbc, n_out, T, o, s, n_in, rb)
                                       : launch_f32dot_t<QMAG_TYPE_Q6_K>(xc, wc, nbc, n_out, T, o, s, n_in, rb);
    };
    if (n_in <= F32_MAX_IN) return launch(x, (const uint8_t *)W, n_in / QK_K, out);
    // longer rows: one launch per chunk of F32_MAX_IN values into partials,
    // then their sum in chunk order
    const int nch = (n_in + F32_MAX_IN - 1) / F32_MAX_IN;
    const size_t n = (size_t)T * n_out;
    int st = QMAG_OK;
    float *part = (float *)workspace(WS_F32PART, sizeof(float) * n * (size_t)nch, &st);
    if (!part) return st;
    for (int c = 0; c < nch; c++) {
        const int c0 = c * F32_MAX_IN, cn = n_in - c0 < F32_MAX_IN ? n_in - c0 : F32_MAX_IN;
        st = launch(x + c0, (const uint8_t *)W + (size_t)(c0 / QK_K) * bb, cn / QK_K, part + (size_t)c * n);
        if (st) return st;
    }
    const long wgs = (long)((n + 255) / 256) < 4096 ? (long)((n + 255) / 256) : 4096;
    hipLaunchKernelGGL(f32_chunk_sum_kernel, dim3((unsigned)wgs), dim3(256), 0, s, part, nch, (long)n, out);
    QMAG_HIP(hipGetLastError());
    return QMAG_OK;
}

}  // namespace qmag

using namespace qmag;

extern "C" {

int qmag_dequant_dev(const void *W, int wtype, int64_t n, float *y)
{
    int st = require_ready();
    if (st) return st;
    return launch_dequant(W, wtype, (long)n, y, ctx().stream);
}

int qmag_matmul_f32_dev(const float *x, const void *W, int n_in, int n_out, int T, int wtype, float *out)
{
    int st = require_ready();
    if (st) return st;
    return launch_f32dot(x, W, n_in, n_out, T, wtype, out, ctx().stream);
}

}  // extern "C"
