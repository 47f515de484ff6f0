// qmag_noalloc.hip -- the matmul seam (nn.c:307-345) without any allocation,
// for callers that cannot call hipMalloc (graph capture, tight serving loops).
//
// qmag_matmul_dev stages the Q8_K form of T > 1 activation rows in a
// workspace it grows with hipMalloc.  This variant stages them in `scratch`,
// a fixed array in device memory that every GPU the library runs on holds for
// the life of the process.  Its device address is looked up once per device
// at qmag_init (hipGetSymbolAddress); host code uses only that address, never
// the array's name, which on the host is a stand-in and not a device pointer.
// Calls that overlap on one GPU share the array and race; the kernels write
// every scratch value they later read, so nothing needs clearing.
#include "qmag_internal.h"

namespace qmag {

// T * n_in activation values at most: xq (1 B each), xd (4 B per 256),
// xsum (2 B per 16), each part starting on a 256-byte boundary
constexpr size_t NOALLOC_MAX_VALUES = (size_t)1 << 21;
constexpr size_t NA_XQ = 0;
constexpr size_t NA_XD = NA_XQ + NOALLOC_MAX_VALUES;
constexpr size_t NA_XS = NA_XD + NOALLOC_MAX_VALUES / QK_K * 4;
constexpr size_t NA_BYTES = NA_XS + NOALLOC_MAX_VALUES / 16 * 2;
static_assert(NA_XD % 256 == 0 && NA_XS % 256 == 0, "scratch layout");

static __device__ __align__(256) uint8_t scratch[NA_BYTES];

constexpr int MAX_DEV = 64;
static uint8_t *g_scratch_ptr[MAX_DEV] = {};

// once per device, with that device current (called from qmag_init)
int noalloc_setup(int dev)
{
    if (dev < 0 || dev >= MAX_DEV) return fail(QMAG_ERR_ARG, "noalloc: device %d out of range", dev);
    if (g_scratch_ptr[dev]) return QMAG_OK;
    void *p = nullptr;
    QMAG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = (uint8_t *)p;
    return QMAG_OK;
}

}  // namespace qmag

using namespace qmag;

extern "C" int qmag_matmul_noalloc_dev(const float *x, const void *W, int n_in, int n_out, int T, int wtype,
                                       float *out)
{
    int st = require_ready();
    if (st) return st;
    if (n_in <= 0 || n_in % QK_K || T <= 0) return fail(QMAG_ERR_ARG, "matmul_noalloc: n_in=%d T=%d", n_in, T);
    if ((size_t)T * (size_t)n_in > NOALLOC_MAX_VALUES)
        return fail(QMAG_ERR_ARG, "matmul_noalloc: T * n_in = %zu exceeds the fixed scratch of %zu values",
                    (size_t)T * (size_t)n_in, NOALLOC_MAX_VALUES);
    uint8_t *sp = g_scratch_ptr[ctx().dev];
    if (!sp) return fail(QMAG_ERR_NODEV, "matmul_noalloc: scratch address not set up");
    ProfSuspend quiet;        // per-kernel event timing allocates events: off here
    hipStream_t s = ctx().stream;
    if (T == 1 && matvec_x_supported(n_in)) return launch_matvec_x(x, W, n_in, n_out, wtype, out, s);
    int8_t *xq = (int8_t *)(sp + NA_XQ);
    float *xd = (float *)(sp + NA_XD);
    int16_t *xs = (int16_t *)(sp + NA_XS);
    st = launch_q8k_quant(x, (n_in / QK_K) * T, xq, xd, xs, s);
    if (st) return st;
    return launch_matvec(xq, xd, xs, W, n_in, n_out, T, wtype, out, s);
}
