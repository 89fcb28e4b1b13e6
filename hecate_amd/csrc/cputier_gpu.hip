// cputier_gpu.hip - the GPU side of the host-CPU expert tier's hand-off, as two kernels so that a hipGraph can hold
// them: cpu_handoff_kernel copies the job's rows and routing into the pinned, device-mapped mailbox and raises the flag
// with a system-scope release (runtime/tier/moe4/moe4.cu:719-738 moe4_handoff_kernel); cpu_collect_kernel waits for
// the pool to lower it and adds the CPU partial into y (runtime/tier/tier_split.py:577-644 tier_combine, whose graph
// form spins on the band's DONE flag in its combine kernel). Every wait here is bounded by the wall clock: past the
// bound the kernel records the error in the mailbox's gpu_err word and returns, so no launch outlives a stalled pool.
// The pool itself is cputier.cpp.
#include "hmoe_dev.h"

#include <cstring>

namespace hmoe {

__device__ __forceinline__ uint32_t load_sys(const uint32_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// thread 0 polls the pool's done generation until it equals `want` or `ticks` wall-clock ticks pass; true when it did
__device__ bool wait_done(const hmoe_cpu_mailbox* mb, uint32_t want, long long ticks)
{
    const long long t0 = wall_clock64();
    for (;;) {
        if (load_sys(&mb->done) == want) return true;
        if (wall_clock64() - t0 > ticks) return false;
        __builtin_amdgcn_s_sleep(16);
    }
}

// one workgroup: x bf16 [R][H] (R * 768 uint4), sel int64 [R][8] (R * 4 uint4), rw f16 [R][8] (R uint4)
__global__ void __launch_bounds__(1024) cpu_handoff_kernel(const uint4* __restrict__ x, const uint4* __restrict__ sel,
                                                           const uint4* __restrict__ rw, hmoe_cpu_mailbox* mb, int R,
                                                           int layer, long long ticks)
{
    __shared__ int ready;
    __shared__ uint32_t gen;
    if (threadIdx.x == 0) {
        // the previous job is done (its collect waited for it, unless that wait ran out)
        const uint32_t g = load_sys(&mb->issue);
        ready = wait_done(mb, g, ticks);
        if (!ready) __hip_atomic_store(&mb->gpu_err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        gen = g + 1u == 0u ? 1u : g + 1u;                       // (0 is skipped on wrap-around)
    }
    __syncthreads();
    if (!ready) return;
    uint4* dx = (uint4*) mb->x;
    uint4* ds = (uint4*) mb->sel;
    uint4* dw = (uint4*) mb->rw;
    for (int i = threadIdx.x; i < R * (H / 8); i += 1024) dx[i] = x[i];
    for (int i = threadIdx.x; i < R * 4; i += 1024) ds[i] = sel[i];
    for (int i = threadIdx.x; i < R; i += 1024) dw[i] = rw[i];
    if (threadIdx.x == 0) {
        mb->rows = R;
        mb->layer = layer;
        mb->err = 0;
    }
    // each wave's mailbox stores reach the host before the barrier, the flag after it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(&mb->issue, gen, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// one workgroup per row: y[r] += out[r] once the pool has finished the generation the hand-off posted (issue); with
// gpu_err set (a hand-off that found the pool busy posted nothing) the partial in the mailbox is not this step's, and
// nothing is added
__global__ void __launch_bounds__(256) cpu_collect_kernel(const hmoe_cpu_mailbox* mb, float* __restrict__ y,
                                                          int32_t* gpu_err, long long ticks)
{
    __shared__ int done;
    if (threadIdx.x == 0) {
        const int e0 = __hip_atomic_load(gpu_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        done = e0 == 0 && wait_done(mb, load_sys(&mb->issue), ticks);
        if (!done && e0 == 0) __hip_atomic_store(gpu_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
    if (!done) return;
    // every wave reads out after the pool's release of the flag
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
    const f32x4* o = (const f32x4*) (mb->out + (size_t) blockIdx.x * H);
    f32x4* yp = (f32x4*) (y + (size_t) blockIdx.x * H);
    for (int i = threadIdx.x; i < H / 4; i += 256) yp[i] = yp[i] + o[i];
}

// wall-clock ticks of the kernels' bounded waits on the current device: 2 s
static int wait_ticks(long long* ticks)
{
    int dev = 0, khz = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess || khz <= 0) return set_error(HMOE_ERR_HIP, "cpu tier: wall clock rate (%s)", hipGetErrorString(e));
    *ticks = 2000LL * khz;
    return HMOE_OK;
}

static int device_mailbox(hmoe_cpu_mailbox* mb, hmoe_cpu_mailbox** d)
{
    hipError_t e = hipHostGetDevicePointer((void**) d, mb, 0);
    if (e != hipSuccess) return set_error(HMOE_ERR_HIP, "cpu tier: the mailbox is not device-mapped (%s)", hipGetErrorString(e));
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
    if (int rc = device_mailbox(mb, &d)) return rc;
    if (int rc = wait_ticks(&ticks)) return rc;
    cpu_handoff_kernel<<<1, 1024, 0, (hipStream_t) stream>>>((const uint4*) x, (const uint4*) sel, (const uint4*) rw, d,
                                                             R, layer, ticks);
    return HMOE_LAUNCHED("cpu_submit");
}

extern "C" int hmoe_cpu_collect(hmoe_cpu_mailbox* mb, float* y, int R, void* stream)
{
    HMOE_REQUIRE(mb && y && R >= 1 && R <= HMOE_CPU_MAXR && ((uintptr_t) y & 15) == 0, "cpu_collect: arguments");
    hmoe_cpu_mailbox* d = nullptr;
    long long ticks = 0;
    if (int rc = device_mailbox(mb, &d)) return rc;
    if (int rc = wait_ticks(&ticks)) return rc;
    cpu_collect_kernel<<<R, 256, 0, (hipStream_t) stream>>>(d, y, &d->gpu_err, ticks);
    return HMOE_LAUNCHED("cpu_collect");
}
