// cputier.cpp - the host-CPU expert tier (runtime/tier/cpuband.cpp: the Grace band) for x86 hosts: a persistent
// pool of threads that serves decode jobs (<= 8 rows) from a mailbox in pinned, device-mapped host memory, runs the
// cold experts (ids in [lo, lo + n)) with q8_0 activations and int4 x int8 dot products, and leaves an fp32 partial
// for the GPU to add (the GPU side of the hand-off is in cputier_gpu.hip).
//
// Arithmetic, as cpuband.cpp with group-128 bf16 scales:
//   * picks in first appearance over rows, then top-k order; wgt[p][r] = sum of the f16 routing weights (:151-178);
//   * x rows and each pick's activation quantised per 32: s = absmax / 127 (1 if 0), q = lrintf(v / s) (:106-111);
//   * y[n] over groups g of 128: four fp32 lanes accumulate float(dot) * xs per 32-block (lane i takes the products
//     of k + 4i..+4 and k + 16 + 4i..+4), fold (a0 + a1) + (a2 + a3), y = fma(s[n][g], fold, y) (:80-104);
//   * act = g / (1 + expf(-g)) * u * wgt, then q8_0 (:201-207);
//   * out[r][n] = sum over picks in pick order of the down rows, from 0 (:210-218).
// Threads split the output rows of every GEMV; a job is a fixed sequence of barriers, so results do not depend on
// the thread count.
#include "hecate_moe.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <immintrin.h>
#include <memory>
#include <mutex>
#include <sched.h>
#include <thread>
#include <vector>

namespace hmoe_cpu {

constexpr int H = HMOE_H, I = HMOE_I, TOPK = HMOE_TOPK;
constexpr int CMAXR = HMOE_CPU_MAXR;

static inline float bf2f(uint16_t b) { uint32_t u = (uint32_t) b << 16; float f; std::memcpy(&f, &u, 4); return f; }
static inline float h2f(uint16_t h) { return (float) _cvtsh_ss(h); }

// one expert matrix on the host: codes [N][K / 2] (row-major, low nibble first), bf16 scales [N][K / 128]
struct Mat { const uint8_t* q = nullptr; const uint16_t* s = nullptr; };
struct Expert { Mat gate, up, down; };
struct Layer { int lo = 0; std::vector<Expert> ex; };

// the job's work arrays (sized for CMAXR rows and up to MAXP = CMAXR * TOPK picks)
constexpr int MAXP = CMAXR * TOPK;
struct Work
{
    int P = 0, R = 0;
    const Layer* ly = nullptr;     // the job's layer (thread 0 reads it in the parse; the others after the barrier)
    int32_t pick[MAXP];
    float wgt[MAXP][CMAXR];
    int nrows[MAXP], rows[MAXP][CMAXR];
    std::vector<int8_t> xq;        // [R][H]
    std::vector<float> xs;         // [R][H / 32]
    std::vector<int8_t> xqp;       // [P][CMAXR][H]: each pick's rows of xq, compacted
    std::vector<float> xsp;        // [P][CMAXR][H / 32]
    std::vector<float> gy, uy;     // [P][CMAXR][I]
    std::vector<int8_t> aq;        // [P][CMAXR][I]
    std::vector<float> as;         // [P][CMAXR][I / 32]
    Work() : xq(CMAXR * H), xs(CMAXR * H / 32), xqp((size_t) MAXP * CMAXR * H), xsp((size_t) MAXP * CMAXR * H / 32),
             gy((size_t) MAXP * CMAXR * I), uy((size_t) MAXP * CMAXR * I), aq((size_t) MAXP * CMAXR * I),
             as((size_t) MAXP * CMAXR * I / 32) {}
};

constexpr int MAX_LAYERS = 4097;                     // layer ids 0 .. 4096
constexpr int MAX_THREADS = 256;

struct Pool
{
    std::vector<std::thread> th;
    // the layers, each published once complete through an atomic pointer and never changed after (add_layer of an id
    // that exists publishes a new record; the old ones are kept until the pool stops), so a job that reads a layer
    // while the host adds another (or replaces this one) reads a whole, unchanging record
    std::atomic<const Layer*> layer[MAX_LAYERS];
    std::vector<std::unique_ptr<Layer>> owned;        // every record published (freed at stop)
    hmoe_cpu_mailbox* mb = nullptr;
    std::atomic<int> stop{0};
    // gather barrier (cpuband.cpp:62-75): thread t > 0 releases its own 128-byte line with its barrier count, thread
    // 0 acquires them all and releases the sense line; no line is written by more than one thread
    struct alignas(128) Flag { std::atomic<uint32_t> v{0}; };
    Flag flag[MAX_THREADS];
    alignas(128) std::atomic<uint32_t> sense{0};
    int nthr = 0;
    uint32_t start_gen = 0;                           // the mailbox's issue at start: taken as served
    bool skip = false;                                // HMOE_CPU_SKIP: acknowledge jobs with a zero partial
    int hold_t = -1, hold_us = 0;                     // HMOE_CPU_HOLD test hook
    Work w;
    std::atomic<long long> jobs{0}, picks{0};
};

static Pool* g_pool = nullptr;
static std::mutex g_mu;

// the pool's barrier: gen is the calling thread's own count of barriers passed (every thread passes the same
// sequence, so the counts agree); false when the pool is stopping (a thread that never arrives, e.g. one held back or
// gone, must not keep the others here past hmoe_cpu_stop)
static bool barrier(Pool& p, int t, uint32_t& gen)
{
    ++gen;
    if (t == 0)
    {
        for (int i = 1; i < p.nthr; ++i)
            while (p.flag[i].v.load(std::memory_order_acquire) != gen)
            {
                if (p.stop.load(std::memory_order_acquire)) return false;
                _mm_pause();
            }
        p.sense.store(gen, std::memory_order_release);
        return true;
    }
    p.flag[t].v.store(gen, std::memory_order_release);
    while (p.sense.load(std::memory_order_acquire) != gen)
    {
        if (p.stop.load(std::memory_order_acquire)) return false;
        _mm_pause();
    }
    return true;
}

// q8_0 of a 32-element group
static void quant_group(const float* v, int8_t* q, float* sc)
{
    float m = 0.0f;
    for (int k = 0; k < 32; ++k) m = std::fmax(m, std::fabs(v[k]));
    const float s = m > 0 ? m / 127.0f : 1.0f;
    *sc = s;
    const float inv = 1.0f / s;
    for (int k = 0; k < 32; ++k) q[k] = (int8_t) lrintf(v[k] * inv);
}

// the four lane sums of one 32-block: lane i = sum of z * x over k 4i..4i+3 and 16 + 4i..16 + 4i + 3
static inline __m128i block_dot(__m256i z, const int8_t* x)
{
    const __m256i xv = _mm256_loadu_si256((const __m256i*) x);
    // |z| (u8) times x with z's sign, summed in pairs (int16), then in fours (int32)
    const __m256i pr = _mm256_maddubs_epi16(_mm256_sign_epi8(z, z), _mm256_sign_epi8(xv, z));
    const __m256i q4 = _mm256_madd_epi16(pr, _mm256_set1_epi16(1));       // sums of k 4m..4m+3, m = 0..7
    return _mm_add_epi32(_mm256_castsi256_si128(q4), _mm256_extracti128_si256(q4, 1));
}

// rows [n0, n1) of y[r][n] = W x[r] for nr rows (xq [nr][K], xs [nr][K / 32]), y row stride ys
static void gemv(const Mat& m, int K, const int8_t* xq, const float* xs, int nr, int n0, int n1, float* y, int ys)
{
    const __m256i lo4 = _mm256_set1_epi8(0x0f), eight = _mm256_set1_epi8(8);
    for (int n = n0; n < n1; ++n)
    {
        const uint8_t* qr = m.q + (size_t) n * (K / 2);
        const uint16_t* sr = m.s + (size_t) n * (K / 128);
        float yr[CMAXR];
        for (int r = 0; r < nr; ++r) yr[r] = 0.0f;
        for (int g = 0; g < K / 128; ++g)
        {
            __m128 acc[CMAXR];
            for (int r = 0; r < nr; ++r) acc[r] = _mm_setzero_ps();
            for (int b = 0; b < 4; ++b)
            {
                const int k = g * 128 + b * 32;
                // the block's 32 codes in k order, minus 8: byte j = code(k + 2j) | code(k + 2j + 1) << 4
                const __m128i raw = _mm_loadu_si128((const __m128i*) (qr + k / 2));
                const __m128i lo = _mm_and_si128(raw, _mm256_castsi256_si128(lo4));
                const __m128i hi = _mm_and_si128(_mm_srli_epi16(raw, 4), _mm256_castsi256_si128(lo4));
                const __m256i z = _mm256_sub_epi8(
                    _mm256_set_m128i(_mm_unpackhi_epi8(lo, hi), _mm_unpacklo_epi8(lo, hi)), eight);
                for (int r = 0; r < nr; ++r)
                {
                    const __m128 d = _mm_cvtepi32_ps(block_dot(z, xq + (size_t) r * K + k));
                    acc[r] = _mm_fmadd_ps(d, _mm_set1_ps(xs[(size_t) r * (K / 32) + k / 32]), acc[r]);
                }
            }
            const float sc = bf2f(sr[g]);
            for (int r = 0; r < nr; ++r)
            {
                alignas(16) float a[4];
                _mm_store_ps(a, acc[r]);
                yr[r] = std::fma(sc, (a[0] + a[1]) + (a[2] + a[3]), yr[r]);
            }
        }
        for (int r = 0; r < nr; ++r) y[(size_t) r * ys + n] = yr[r];
    }
}

// ---- the same GEMV with AVX-512 VNNI (used when the host has it; same integer lane sums, same bits) ----
// The input rows are first laid out per group of 128 as VG bytes: xa (k 0..15 of blocks 0..3, 16 bytes each), xb (k
// 16..31 of each block), then 16 int32 init[4 b + i] = -8 * (the sum of x over lane i of block b). vpdpbusd of the
// unsigned codes (z + 8) against xa and xb, started from init, leaves in dword 4 b + i exactly block_dot's lane i of
// block b: sum z x = sum (z + 8) x - 8 sum x, all in int32.
constexpr int VG = 192;

#define HMOE_VNNI __attribute__((target("avx512f,avx512bw,avx512vnni")))

HMOE_VNNI static void to_vnni(const int8_t* xq, int K, uint8_t* out)
{
    const __m512i ones = _mm512_set1_epi8(1);
    for (int g = 0; g < K / 128; ++g)
    {
        const __m512i b01 = _mm512_loadu_si512(xq + (size_t) g * 128);        // [b0 lo, b0 hi, b1 lo, b1 hi]
        const __m512i b23 = _mm512_loadu_si512(xq + (size_t) g * 128 + 64);
        const __m512i xa = _mm512_shuffle_i64x2(b01, b23, 0x88), xb = _mm512_shuffle_i64x2(b01, b23, 0xdd);
        const __m512i sx = _mm512_dpbusd_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), ones, xa), ones, xb);
        uint8_t* o = out + (size_t) g * VG;
        _mm512_storeu_si512(o, xa);
        _mm512_storeu_si512(o + 64, xb);
        _mm512_storeu_si512(o + 128, _mm512_sub_epi32(_mm512_setzero_si512(), _mm512_slli_epi32(sx, 3)));
    }
}

HMOE_VNNI static void gemv_vnni(const Mat& m, int K, const int8_t* xq, const float* xs, int nr, int n0, int n1, float* y,
                                int ys)
{
    const int NG = K / 128;
    static thread_local std::vector<uint8_t> xv((size_t) CMAXR * (H / 128) * VG);
    for (int r = 0; r < nr; ++r) to_vnni(xq + (size_t) r * K, K, xv.data() + (size_t) r * NG * VG);
    const __m512i lo4 = _mm512_set1_epi8(0x0f);
    for (int n = n0; n < n1; ++n)
    {
        const uint8_t* qr = m.q + (size_t) n * (K / 2);
        const uint16_t* sr = m.s + (size_t) n * NG;
        float yr[CMAXR];
        for (int r = 0; r < nr; ++r) yr[r] = 0.0f;
        for (int g = 0; g < NG; ++g)
        {
            // the group's 4 blocks, one per 128-bit lane: k 0..15 and k 16..31 of each as unsigned codes
            const __m512i raw = _mm512_loadu_si512(qr + (size_t) g * 64);
            const __m512i lo = _mm512_and_si512(raw, lo4), hi = _mm512_and_si512(_mm512_srli_epi16(raw, 4), lo4);
            const __m512i za = _mm512_unpacklo_epi8(lo, hi), zb = _mm512_unpackhi_epi8(lo, hi);
            const float sc = bf2f(sr[g]);
            for (int r = 0; r < nr; ++r)
            {
                const uint8_t* xg = xv.data() + ((size_t) r * NG + g) * VG;
                __m512i d = _mm512_dpbusd_epi32(_mm512_loadu_si512(xg + 128), za, _mm512_loadu_si512(xg));
                d = _mm512_dpbusd_epi32(d, zb, _mm512_loadu_si512(xg + 64));
                const __m512 f = _mm512_cvtepi32_ps(d);
                const float* xsr = xs + (size_t) r * (K / 32) + 4 * g;
                __m128 acc = _mm_fmadd_ps(_mm512_castps512_ps128(f), _mm_set1_ps(xsr[0]), _mm_setzero_ps());
                acc = _mm_fmadd_ps(_mm512_extractf32x4_ps(f, 1), _mm_set1_ps(xsr[1]), acc);
                acc = _mm_fmadd_ps(_mm512_extractf32x4_ps(f, 2), _mm_set1_ps(xsr[2]), acc);
                acc = _mm_fmadd_ps(_mm512_extractf32x4_ps(f, 3), _mm_set1_ps(xsr[3]), acc);
                alignas(16) float a[4];
                _mm_store_ps(a, acc);
                yr[r] = std::fma(sc, (a[0] + a[1]) + (a[2] + a[3]), yr[r]);
            }
        }
        for (int r = 0; r < nr; ++r) y[(size_t) r * ys + n] = yr[r];
    }
}

static bool g_vnni = false;                         // the host has AVX-512 VNNI (decided at pool start)

static void gemv_any(const Mat& m, int K, const int8_t* xq, const float* xs, int nr, int n0, int n1, float* y, int ys)
{
    if (g_vnni) gemv_vnni(m, K, xq, xs, nr, n0, n1, y, ys);
    else gemv(m, K, xq, xs, nr, n0, n1, y, ys);
}

static void range(int total, int t, int T, int& a, int& b)
{
    a = (int) ((long long) total * t / T);
    b = (int) ((long long) total * (t + 1) / T);
}

// one job (generation g), by every thread of the pool (t = 0 .. nthr - 1), in the phases of cpuband.cpp:137-218, each
// ended by a barrier: thread 0 parses the picks while the others quantise every row of x (:137-179), then the rows of
// each pick are gathered, the gate and up rows of every pick are split over the threads (one phase for all picks), the
// activations are quantised, and the down rows are split (each output summed over the picks in order). False when the
// pool stopped inside it.
static bool run_job(Pool& p, int t, uint32_t g, uint32_t& gen)
{
    hmoe_cpu_mailbox* mb = p.mb;
    Work& w = p.w;
    const int T = p.nthr;
    const int R0 = mb->rows, L0 = mb->layer;
    const bool rows_ok = R0 >= 1 && R0 <= CMAXR;
    if (t == 0)
    {
        w.R = rows_ok ? R0 : 0;
        w.P = 0;
        w.ly = (w.R && L0 >= 0 && L0 < MAX_LAYERS) ? p.layer[L0].load(std::memory_order_acquire) : nullptr;
        if (w.ly && !p.skip)
        {
            const Layer& ly = *w.ly;
            const int n = (int) ly.ex.size();
            for (int i = 0; i < w.R * TOPK; ++i)
            {
                const int64_t e = mb->sel[i] - ly.lo;
                if (e < 0 || e >= n) continue;
                int j = 0;
                while (j < w.P && w.pick[j] != (int32_t) e) ++j;
                if (j == w.P) { w.pick[w.P] = (int32_t) e; for (int r = 0; r < w.R; ++r) w.wgt[w.P][r] = 0.0f; ++w.P; }
                w.wgt[j][i / TOPK] += h2f(mb->rw[i]);
            }
            for (int q = 0; q < w.P; ++q)
            {
                int nr = 0;
                for (int r = 0; r < w.R; ++r) if (w.wgt[q][r] != 0.0f) w.rows[q][nr++] = r;
                w.nrows[q] = nr;
            }
        }
    }
    // q8_0 of every row of x, by threads 1 .. T - 1 (all of it by thread 0 when it is alone)
    if (rows_ok && (t != 0 || T == 1))
    {
        int a, b;
        range(R0 * H / 32, T == 1 ? 0 : t - 1, T == 1 ? 1 : T - 1, a, b);
        for (int gi = a; gi < b; ++gi)
        {
            float v[32];
            for (int k = 0; k < 32; ++k) v[k] = bf2f(mb->x[(size_t) gi * 32 + k]);
            quant_group(v, w.xq.data() + (size_t) gi * 32, w.xs.data() + gi);
        }
    }
    if (!barrier(p, t, gen)) return false;
    const int R = w.R, P = w.P;
    if (R && P)
    {
        const Layer& ly = *w.ly;
        // each pick's rows of x, compacted
        {
            int a, b;
            range(P * CMAXR, t, T, a, b);
            for (int i = a; i < b; ++i)
            {
                const int q = i / CMAXR, j = i % CMAXR;
                if (j >= w.nrows[q]) continue;
                const int r = w.rows[q][j];
                std::memcpy(w.xqp.data() + ((size_t) q * CMAXR + j) * H, w.xq.data() + (size_t) r * H, H);
                std::memcpy(w.xsp.data() + ((size_t) q * CMAXR + j) * (H / 32), w.xs.data() + (size_t) r * (H / 32),
                            sizeof(float) * (H / 32));
            }
        }
        if (!barrier(p, t, gen)) return false;
        // gate and up rows of every pick: the (pick, matrix, row) range split over the threads
        {
            int a, b;
            range(P * 2 * I, t, T, a, b);
            for (int i = a; i < b;)
            {
                const int q = i / (2 * I), m = (i / I) % 2, n0 = i % I, n1 = std::min(I, n0 + (b - i));
                const Expert& ex = ly.ex[w.pick[q]];
                gemv_any(m ? ex.up : ex.gate, H, w.xqp.data() + (size_t) q * CMAXR * H,
                         w.xsp.data() + (size_t) q * CMAXR * (H / 32), w.nrows[q], n0, n1,
                         (m ? w.uy : w.gy).data() + (size_t) q * CMAXR * I, I);
                i += n1 - n0;
            }
        }
        if (!barrier(p, t, gen)) return false;
        // act = silu(g) u wgt -> q8_0, every pick's rows
        {
            int a, b;
            range(P * CMAXR * (I / 32), t, T, a, b);
            for (int gi = a; gi < b; ++gi)
            {
                const int q = gi / (CMAXR * (I / 32)), j = (gi / (I / 32)) % CMAXR, k0 = (gi % (I / 32)) * 32;
                if (j >= w.nrows[q]) continue;
                const float wt = w.wgt[q][w.rows[q][j]];
                const size_t o = ((size_t) q * CMAXR + j) * I + k0;
                float v[32];
                for (int k = 0; k < 32; ++k)
                {
                    const float gg = w.gy[o + k];
                    v[k] = gg / (1.0f + expf(-gg)) * w.uy[o + k] * wt;
                }
                quant_group(v, w.aq.data() + o, w.as.data() + o / 32);
            }
        }
        if (!barrier(p, t, gen)) return false;
    }
    // down: output rows split over the threads, picks in order, summed into out from 0 (out zero when no pick runs)
    {
        int a, b;
        range(H, t, T, a, b);
        for (int r = 0; r < R; ++r) std::memset(mb->out + (size_t) r * H + a, 0, sizeof(float) * (size_t) (b - a));
        static thread_local std::vector<float> y1(CMAXR * H);
        for (int q = 0; q < (R ? P : 0); ++q)
        {
            const Expert& ex = w.ly->ex[w.pick[q]];
            const int nr = w.nrows[q];
            gemv_any(ex.down, I, w.aq.data() + (size_t) q * CMAXR * I, w.as.data() + (size_t) q * CMAXR * I / 32, nr, a, b,
                     y1.data(), H);
            for (int j = 0; j < nr; ++j)
            {
                float* o = mb->out + (size_t) w.rows[q][j] * H;
                for (int n = a; n < b; ++n) o[n] += y1[(size_t) j * H + n];
            }
        }
    }
    if (!barrier(p, t, gen)) return false;
    if (t == 0)
    {
        p.jobs.fetch_add(1, std::memory_order_relaxed);
        p.picks.fetch_add(P, std::memory_order_relaxed);
        mb->err = !R ? 1 : (w.ly || p.skip ? 0 : 2);        // 1: bad row count, 2: no such layer
        __atomic_store_n(&mb->done, g, __ATOMIC_RELEASE);
    }
    return true;
}

static void worker(Pool* p, int t, int core)
{
    if (core >= 0)
    {
        cpu_set_t cs;
        CPU_ZERO(&cs);
        CPU_SET(core, &cs);
        sched_setaffinity(0, sizeof(cs), &cs);       // best effort
    }
    int idle = 0;
    uint32_t gen = 0;                                // barriers this thread has passed
    uint32_t last = p->start_gen;                    // the generation this thread served last
    while (true)
    {
        // every thread watches issue and runs each generation once: a poster may post the next job only when done
        // equals issue, and done is written after the job's last barrier, which every thread passes, so no thread can
        // miss a generation or see a job's inputs change under it (the 0/1 flag this replaces let a slow thread take a
        // re-raised flag for the job it had just finished)
        if (p->stop.load(std::memory_order_acquire)) return;
        const uint32_t g = __atomic_load_n(&p->mb->issue, __ATOMIC_ACQUIRE);
        if (g != last)
        {
            idle = 0;
            last = g;
            if (!run_job(*p, t, g, gen)) return;
            if (t == p->hold_t)
                for (int us = 0; us < p->hold_us && !p->stop.load(std::memory_order_acquire); us += 1000)
                    std::this_thread::sleep_for(std::chrono::microseconds(std::min(1000, p->hold_us - us)));
            continue;
        }
        if (++idle < 4096) _mm_pause();
        else std::this_thread::yield();
    }
}

}  // namespace hmoe_cpu

namespace hmoe { int set_error(int code, const char* fmt, ...); }    // the library's error record (hmoe_last_error)

using namespace hmoe_cpu;

extern "C" int hmoe_cpu_start(hmoe_cpu_mailbox* mb, int threads, int first_core)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_pool) return hmoe::set_error(HMOE_ERR_ARG, "cpu_start: the pool is running");
    if (!mb || threads < 1 || threads > MAX_THREADS) return hmoe::set_error(HMOE_ERR_ARG, "cpu_start: mailbox / threads");
    // the dot kernel: AVX-512 VNNI where the host has it, unless HMOE_CPU_ISA=avx2 asks for the AVX2 one (both give
    // the same bits)
    const char* isa = std::getenv("HMOE_CPU_ISA");
    g_vnni = __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw") &&
             !(isa && std::strcmp(isa, "avx2") == 0);
    Pool* p = new Pool();
    for (auto& l : p->layer) l.store(nullptr, std::memory_order_relaxed);
    p->mb = mb;
    p->nthr = threads;
    p->start_gen = __atomic_load_n(&mb->issue, __ATOMIC_ACQUIRE);
    __atomic_store_n(&mb->done, p->start_gen, __ATOMIC_RELEASE);     // nothing in flight
    const char* skip = std::getenv("HMOE_CPU_SKIP");
    p->skip = skip && std::atoi(skip) != 0;
    if (const char* hold = std::getenv("HMOE_CPU_HOLD"))
        if (std::sscanf(hold, "%d,%d", &p->hold_t, &p->hold_us) != 2) p->hold_t = -1;
    g_pool = p;
    for (int t = 0; t < threads; ++t) p->th.emplace_back(worker, p, t, first_core >= 0 ? first_core + t : -1);
    return 0;
}

extern "C" int hmoe_cpu_add_layer(int layer, int lo, int n, const uint8_t* const* q, const uint16_t* const* s)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_pool) return hmoe::set_error(HMOE_ERR_ARG, "cpu_add_layer: no pool");
    if (layer < 0 || layer >= MAX_LAYERS || lo < 0 || n < 0 || n > 256 || (n && (!q || !s)))
        return hmoe::set_error(HMOE_ERR_ARG, "cpu_add_layer: arguments");
    hmoe_cpu_mailbox* mb = g_pool->mb;
    if (__atomic_load_n(&mb->issue, __ATOMIC_ACQUIRE) != __atomic_load_n(&mb->done, __ATOMIC_ACQUIRE))
        return hmoe::set_error(HMOE_ERR_ARG, "cpu_add_layer: a job is in flight");
    // every pointer is checked before the pool's layers change
    for (int i = 0; i < 3 * n; ++i)
        if (!q[i] || !s[i]) return hmoe::set_error(HMOE_ERR_ARG, "cpu_add_layer: null matrix (expert %d)", i / 3);
    std::unique_ptr<Layer> L(new Layer());
    L->lo = lo;
    L->ex.assign(n, Expert{});
    for (int e = 0; e < n; ++e)
    {
        // q / s: per expert the gate, up and down pointers (3 n each)
        L->ex[e].gate = {q[3 * e + 0], s[3 * e + 0]};
        L->ex[e].up = {q[3 * e + 1], s[3 * e + 1]};
        L->ex[e].down = {q[3 * e + 2], s[3 * e + 2]};
    }
    g_pool->layer[layer].store(L.get(), std::memory_order_release);
    g_pool->owned.push_back(std::move(L));
    return 0;
}

extern "C" int hmoe_cpu_stats(long long* jobs, long long* picks)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_pool) return hmoe::set_error(HMOE_ERR_ARG, "cpu_stats: no pool");
    if (jobs) *jobs = g_pool->jobs.load();
    if (picks) *picks = g_pool->picks.load();
    return 0;
}

extern "C" int hmoe_cpu_stop(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_pool) return 0;
    g_pool->stop.store(1, std::memory_order_release);
    for (auto& t : g_pool->th) t.join();
    delete g_pool;
    g_pool = nullptr;
    return 0;
}
