// cputier_dev.h - the GPU side of the host-CPU tier's mailbox protocol (include/hecate_moe.h hmoe_cpu_mailbox), shared
// by the hand-off and collect kernels (cputier_gpu.hip) and the launches that fold them in (norm.hip: the norm +
// router that posts the job, as nr4_kernel.cuh:360-378 writes the band slot and releases ISSUE; the combine + norm that
// waits for it and adds the CPU partial, as cn.cu:108-142 waits for CPU_DONE).
//
// Protocol: a job is posted by filling the mailbox and then storing issue = g + 1 (a generation, 0 skipped) with a
// system-scope release; the pool stores done = issue when the job's partial is in out. A poster first waits for done
// == issue (the previous job finished). Every GPU wait is bounded by the wall clock: past the bound the kernel sets the
// sticky gpu_err word and goes on without the pool (nothing posted, or nothing added).
#pragma once
#include "hmoe_dev.h"

namespace hmoe {

__device__ __forceinline__ uint32_t load_sys(const uint32_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// thread 0 polls the pool's done generation until it equals `want` or `ticks` wall-clock ticks pass; true when it did
__device__ inline bool wait_done(const hmoe_cpu_mailbox* mb, uint32_t want, long long ticks)
{
    const long long t0 = wall_clock64();
    for (;;) {
        if (load_sys(&mb->done) == want) return true;
        if (wall_clock64() - t0 > ticks) return false;
        __builtin_amdgcn_s_sleep(16);
    }
}

// thread 0, before a post: waits for the previous job; returns whether the mailbox is free, and the generation to post
__device__ inline bool post_begin(hmoe_cpu_mailbox* mb, long long ticks, uint32_t& gen)
{
    const uint32_t g = load_sys(&mb->issue);
    const bool ready = wait_done(mb, g, ticks);
    if (!ready) __hip_atomic_store(&mb->gpu_err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    gen = g + 1u == 0u ? 1u : g + 1u;                           // (0 is skipped on wrap-around)
    return ready;
}

// every thread of one workgroup of nt threads: the job's rows x bf16 [R][H] (R * 768 uint4), sel int64 [R][8]
// (R * 4 uint4), rw f16 [R][8] (R uint4) into the mailbox, the header, then (after the workgroup's barrier, by thread
// 0) issue = gen with a system-scope release
__device__ inline void post_job(hmoe_cpu_mailbox* mb, const uint4* __restrict__ x, const uint4* __restrict__ sel,
                                const uint4* __restrict__ rw, int R, int layer, uint32_t gen, int nt)
{
    uint4* dx = (uint4*) mb->x;
    uint4* ds = (uint4*) mb->sel;
    uint4* dw = (uint4*) mb->rw;
    for (int i = threadIdx.x; i < R * (H / 8); i += nt) dx[i] = x[i];
    for (int i = threadIdx.x; i < R * 4; i += nt) ds[i] = sel[i];
    for (int i = threadIdx.x; i < R; i += nt) dw[i] = rw[i];
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

// thread 0, before the CPU partial is read: whether the job the last post issued has finished (false, with gpu_err
// set, when the wait ran out; false without waiting when gpu_err is already set: no job of this step was posted)
__device__ inline bool collect_ready(hmoe_cpu_mailbox* mb, long long ticks)
{
    const int e0 = __hip_atomic_load(&mb->gpu_err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const bool done = e0 == 0 && wait_done(mb, load_sys(&mb->issue), ticks);
    if (!done && e0 == 0) __hip_atomic_store(&mb->gpu_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return done;
}

// host: the device address of a mapped mailbox and the kernels' wait bound (2 s of wall clock on the current device)
int cpu_mailbox_device(hmoe_cpu_mailbox* mb, hmoe_cpu_mailbox** d, long long* ticks);

}  // namespace hmoe
