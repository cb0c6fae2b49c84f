// The LM-head argmax entry point that allocates nothing: the per-block
// partials it merges live in a file-scope device array instead of a handle's
// scratch area, and it runs on a stream the caller passes, so it needs no
// handle (whose creation allocates) and makes no device allocation at all.
// For callers that cannot allocate: code under HIP graph capture, serving
// loops that forbid hipMalloc.
#include "kernels.h"
#include "model.h"

#include <mutex>

using namespace qasr;

// One (value, index) pair per block of the argmax grid: the largest grid the
// kernels use (QASR_ARGMAX_MAX_BLOCKS, 4096) times 8 bytes = 32 KiB, held by
// every GPU this library runs on until the process ends.
#define NOALLOC_SCRATCH_BYTES ((size_t)QASR_ARGMAX_MAX_BLOCKS * 8)
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

// device address of `scratch` per device (the host-side name is not a device
// address), resolved once per device with that device current: by
// qasr_hip_create for its device (the library's set-up call), so that a call
// under HIP graph capture finds it resolved, else by the first call there
#define NOALLOC_MAX_DEVICES 64
static void *g_scratch_dev[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_for_current_device(void **ptr) {
    int dev = -1;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8_noalloc: device index beyond 63");
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return qasr_fail(QASR_ERR_HIP, std::string("argmax_int8_noalloc: hipGetSymbolAddress: ") +
                                               hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *ptr = g_scratch_dev[dev];
    return QASR_OK;
}

int noalloc_init_device() {
    void *p = nullptr;
    return scratch_for_current_device(&p);
}

extern "C" int qasr_hip_argmax_int8_noalloc(void *stream, const float *x, const float *norm_w, float eps,
                                            const int8_t *w, const float *ws, int64_t in_dim, int64_t out_dim,
                                            int32_t *idx) {
    if (in_dim <= 0 || in_dim % 64 != 0 || in_dim > 4096)
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8_noalloc: in_dim must be a positive multiple of 64 and <= 4096");
    if (!x || !w || !ws || !idx || out_dim <= 0 || out_dim > (1 << 30))
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8_noalloc: bad arguments");
    const int blocks = argmax_blocks(out_dim);
    if ((size_t)blocks * 8 > NOALLOC_SCRATCH_BYTES)
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8_noalloc: more block partials than the 32 KiB scratch holds");
    void *s = nullptr;
    if (int rc = scratch_for_current_device(&s)) return rc;
    ArgmaxArgs a{};
    a.x = x; a.norm_w = norm_w; a.eps = eps; a.K = (int)in_dim; a.N = (int)out_dim;
    a.w = w; a.ws = ws;
    a.part_val = reinterpret_cast<float *>(s);
    a.part_idx = reinterpret_cast<int *>(reinterpret_cast<char *>(s) + (size_t)QASR_ARGMAX_MAX_BLOCKS * 4);
    a.out_idx = idx;
    LAUNCHCHK(launch_argmax(a, norm_w != nullptr, blocks, reinterpret_cast<hipStream_t>(stream)),
              "argmax_int8_noalloc");
    return QASR_OK;
}
