// cputier_gpu.hip - the GPU side of the host-CPU expert tier's hand-off, as two kernels so that a hipGraph can hold
// them: cpu_handoff_kernel copies the job's rows and routing into the pinned, device-mapped mailbox and raises the flag
// with a system-scope release (runtime/tier/moe4/moe4.cu:719-738 moe4_handoff_kernel); cpu_collect_kernel waits for
// the pool to lower it and adds the CPU partial into y (runtime/tier/tier_split.py:577-644 tier_combine, whose graph
// form spins on the band's DONE flag in its combine kernel). Every wait here is bounded by the wall clock: past the
// bound the kernel records the error in the mailbox's gpu_err word and returns, so no launch outlives a stalled pool.
// The pool itself is cputier.cpp.
#include "cputier_dev.h"

#include <cstring>

namespace hmoe {

// one workgroup: x bf16 [R][H], sel int64 [R][8], rw f16 [R][8] into the mailbox, once the previous job is done
__global__ void __launch_bounds__(1024) cpu_handoff_kernel(const uint4* __restrict__ x, const uint4* __restrict__ sel,
                                                           const uint4* __restrict__ rw, hmoe_cpu_mailbox* mb, int R,
                                                           int layer, long long ticks)
{
    __shared__ int ready;
    __shared__ uint32_t gen;
    if (threadIdx.x == 0) {
        uint32_t g;
        ready = post_begin(mb, ticks, g);
        gen = g;
    }
    __syncthreads();
    if (!ready) return;
    post_job(mb, x, sel, rw, R, layer, gen, 1024);
}

// one workgroup per row: y[r] += out[r] once the pool has finished the generation the hand-off posted (issue); with
// gpu_err set (a hand-off that found the pool busy posted nothing) the partial in the mailbox is not this step's, and
// nothing is added
__global__ void __launch_bounds__(256) cpu_collect_kernel(hmoe_cpu_mailbox* mb, float* __restrict__ y, long long ticks)
{
    __shared__ int done;
    if (threadIdx.x == 0) done = collect_ready(mb, ticks);
    __syncthreads();
    if (!done) return;
    // every wave reads out after the pool's release of the flag
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    const f32x4* o = (const f32x4*) (mb->out + (size_t) blockIdx.x * H);
    f32x4* yp = (f32x4*) (y + (size_t) blockIdx.x * H);
    for (int i = threadIdx.x; i < H / 4; i += 256) yp[i] = yp[i] + o[i];
}

int cpu_mailbox_device(hmoe_cpu_mailbox* mb, hmoe_cpu_mailbox** d, long long* ticks)
{
    hipError_t e = hipHostGetDevicePointer((void**) d, mb, 0);
    if (e != hipSuccess) return set_error(HMOE_ERR_HIP, "cpu tier: the mailbox is not device-mapped (%s)", hipGetErrorString(e));
    int dev = 0, khz = 0;
    e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess || khz <= 0) return set_error(HMOE_ERR_HIP, "cpu tier: wall clock rate (%s)", hipGetErrorString(e));
    *ticks = 2000LL * khz;
    return HMOE_OK;
}

}  // namespace hmoe

using namespace hmoe;

static_assert(offsetof(hmoe_cpu_mailbox, sel) % 16 == 0 && offsetof(hmoe_cpu_mailbox, rw) % 16 == 0 &&
              offsetof(hmoe_cpu_mailbox, x) % 16 == 0 && offsetof(hmoe_cpu_mailbox, out) % 16 == 0,
              "mailbox arrays are copied in 16-byte units");

extern "C" int hmoe_cpu_mailbox_alloc(hmoe_cpu_mailbox** mb)
{
    HMOE_REQUIRE(mb, "cpu_mailbox_alloc: null");
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, sizeof(hmoe_cpu_mailbox), hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess) return set_error(HMOE_ERR_HIP, "cpu_mailbox_alloc: %s", hipGetErrorString(e));
    std::memset(p, 0, sizeof(hmoe_cpu_mailbox));
    *mb = (hmoe_cpu_mailbox*) p;
    return HMOE_OK;
}

extern "C" int hmoe_cpu_mailbox_free(hmoe_cpu_mailbox* mb)
{
    if (!mb) return HMOE_OK;
    hipError_t e = hipHostFree(mb);
    if (e != hipSuccess) return set_error(HMOE_ERR_HIP, "cpu_mailbox_free: %s", hipGetErrorString(e));
    return HMOE_OK;
}

extern "C" int hmoe_cpu_submit(hmoe_cpu_mailbox* mb, const void* x, const int64_t* sel, const uint16_t* rw, int R,
                               int layer, void* stream)
{
    HMOE_REQUIRE(mb && x && sel && rw && R >= 1 && R <= HMOE_CPU_MAXR && layer >= 0, "cpu_submit: arguments (rows %d)", R);
    HMOE_REQUIRE((((uintptr_t) x | (uintptr_t) sel | (uintptr_t) rw) & 15) == 0, "cpu_submit: x / sel / rw not 16-byte aligned");
    hmoe_cpu_mailbox* d = nullptr;
    long long ticks = 0;
    if (int rc = cpu_mailbox_device(mb, &d, &ticks)) return rc;
    cpu_handoff_kernel<<<1, 1024, 0, (hipStream_t) stream>>>((const uint4*) x, (const uint4*) sel, (const uint4*) rw, d,
                                                             R, layer, ticks);
    return HMOE_LAUNCHED("cpu_submit");
}

extern "C" int hmoe_cpu_collect(hmoe_cpu_mailbox* mb, float* y, int R, void* stream)
{
    HMOE_REQUIRE(mb && y && R >= 1 && R <= HMOE_CPU_MAXR && ((uintptr_t) y & 15) == 0, "cpu_collect: arguments");
    hmoe_cpu_mailbox* d = nullptr;
    long long ticks = 0;
    if (int rc = cpu_mailbox_device(mb, &d, &ticks)) return rc;
    cpu_collect_kernel<<<R, 256, 0, (hipStream_t) stream>>>(d, y, ticks);
    return HMOE_LAUNCHED("cpu_collect");
}
