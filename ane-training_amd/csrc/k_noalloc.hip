/*
 * k_noalloc.hip — the allocation-free classifier GEMM + greedy pick
 * (lm_gemm_argmax_noalloc, stories_lm.h), for callers that cannot allocate
 * device memory: code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc.
 *
 * It runs the same two kernels as the allocating path (lm_selftest_gemm's
 * tiled GEMM with the argmax-partials epilogue, then the greedy loop's
 * partials reduction), on the caller's device buffers, with the per-(row,
 * 32-column block) argmax partials in `scratch`: a file-scope device array of
 * NOALLOC_MAX_PARTS entries (512 KiB) that each GPU holds until the process
 * ends.  Host code never passes the array's name to a kernel (on the host it
 * is only a stand-in for the symbol): lm_init looks up its device address once
 * per device (lmk_noalloc_setup, with that device current) and the entry point
 * passes that address.  The GEMM writes every partial the reduction reads, so
 * nothing in the array needs clearing between calls; calls that overlap on one
 * GPU share the array and race.
 */
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "lm_internal.h"

#define NOALLOC_MAX_PARTS 65536                /* rows x ceil(N / 32), at most */
#define NOALLOC_MAX_DEVICES 64

static __device__ __attribute__((aligned(256))) LMArgPart scratch[NOALLOC_MAX_PARTS];

/* device address of `scratch`, per device: written once under the mutex with
 * release order, read by the entry point with acquire order (no lock there) */
static std::atomic<LMArgPart *> g_scratch[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

extern "C" int lmk_noalloc_setup(void)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev].load(std::memory_order_relaxed)) return hipSuccess;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch[dev].store((LMArgPart *)p, std::memory_order_release);
    return hipSuccess;
}

extern "C" int lm_gemm_argmax_noalloc(int M, int N, int K, const uint16_t *A, const uint16_t *W,
                                      float *C, int *ids, void *stream)
{
    if (M < 1 || N < 1 || K < 64 || K % 64 || !A || !W || !ids) {
        fprintf(stderr, "stories_lm: lm_gemm_argmax_noalloc: invalid arguments (M %d, N %d, K %d; "
                "K must be a multiple of 64, A, W and ids non-NULL)\n", M, N, K);
        return LM_ERR_INVALID;
    }
    const int nblk = (N + 31) / 32;
    if ((long)M * nblk > NOALLOC_MAX_PARTS) {
        fprintf(stderr, "stories_lm: lm_gemm_argmax_noalloc: %d rows x %d column blocks of 32 "
                "exceed the %d argmax partials of its static scratch\n", M, nblk, NOALLOC_MAX_PARTS);
        return LM_ERR_RANGE;
    }
    int dev = -1;
    LMArgPart *part = nullptr;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < NOALLOC_MAX_DEVICES)
        part = g_scratch[dev].load(std::memory_order_acquire);
    if (!part) {
        fprintf(stderr, "stories_lm: lm_gemm_argmax_noalloc: lm_init has not set up this device\n");
        return LM_ERR_NOT_INIT;
    }
    hipStream_t s = (hipStream_t)stream;
    LMEpilogue ep;
    memset(&ep, 0, sizeof(ep));
    ep.out = C;
    ep.ldc = N;
    ep.part = part;
    int e = lmk_gemm(s, A, K, W, M, N, K, LMK_EPI_ARGMAX, &ep);
    if (e == 0) e = lmk_argmax_final(s, part, nblk, M, ids, nullptr, nullptr, 0, nullptr);
    if (e != 0) {
        fprintf(stderr, "stories_lm: lm_gemm_argmax_noalloc: launch failed: %s\n",
                hipGetErrorString((hipError_t)e));
        return LM_ERR_HIP;
    }
    return LM_OK;
}
