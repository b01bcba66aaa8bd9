// gemv.hip -- decode GEMV over GGUF blocks for gfx950.
//
// y[n] = W[n x k] . x[k] with x first quantised to per-32 int8 blocks exactly
// as the reference does (csrc/gncx_llm_kernels.cpp:955-995), then integer
// block dots (v_dot4_i32_i8) with fp32 per-block scaling:
//   Q4_0  cpp:1362-1382   Q4_K  cpp:1383-1397 (+ dot cpp:1127-1205)
//   Q6_K  cpp:1398-1412 (+ dot cpp:1211-1321)   Q8_0  cpp:1413-1431
//   BF16  cpp:1432-1461 (fp32 activations, no quantisation)
//
// Layout of the work: every work-group first quantises x into LDS (the
// activation vector is at most 40960 values, 60 KB with its block records),
// then each wave owns whole rows.  A row is split into "slots" that map one
// lane to a fixed byte range of one block:
//   Q4_K  4 lanes per 144 B super-block: 16 B header + 32 B of nibbles each
//   Q6_K  4 lanes per 210 B super-block: (half, 16-group) -> 3 x 16 B + scales
//   Q4_0  1 lane per 18 B block,  Q8_0  1 lane per 34 B block,  BF16 16 B
// so consecutive lanes read consecutive bytes of the row (coalesced 16 B
// loads) and the only cross-lane step is one wave reduction per row.
#include <hip/hip_runtime.h>

#include "gncx_device.h"
#include "gncx_launch.h"
#include "gncx_slots.h"

namespace gncx {
namespace {

using namespace dev;

constexpr int kThreads = 256;  // 4 waves per work-group

// Resident waves the grid is sized for (256 CUs x this many).
#ifndef GNCX_GEMV_WAVES_PER_CU
#define GNCX_GEMV_WAVES_PER_CU 16
#endif

// One wave owns groups of R consecutive rows.  A row's slots are consumed in
// batches of P passes (64 slots per pass).  The loads of one batch are always
// in flight while the previous batch is being reduced (double buffering in
// registers, across batches of a row and across groups), and the first batch
// is issued before the work-group quantises x into LDS, so the activation
// pass hides under the first HBM round trip.  With AREG (a row fits in one
// batch) each lane's activation slice is the same for every row, so it is
// read from LDS once into registers.
template <int TYPE, int P, int R, bool AREG>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint8_t* __restrict w, size_t rbytes,
                                                        const float* __restrict x, int32_t k, int32_t n,
                                                        float* __restrict y) {
    using S = Slot<TYPE>;
    using Frag = typename S::Frag;
    using Act = typename S::Act;
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t* q = reinterpret_cast<int8_t*>(lds);
    ActMeta* meta = reinterpret_cast<ActMeta*>(lds + k);
    const int lane = threadIdx.x & 63;
    const int32_t wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int32_t nwaves = gridDim.x * (kThreads / 64);
    const int32_t slots = S::slots(k);
    const int32_t ngroups = (n + R - 1) / R;
    const int32_t nbatch = (slots + 64 * P - 1) / (64 * P);

    Frag cur[R][P];
    Frag nxt[R][P];
    auto issue = [&](Frag (&f)[R][P], int32_t grp, int32_t b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int32_t row = grp * R + r;
            if (row < n) {
                const uint8_t* rp = w + static_cast<size_t>(row) * rbytes;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const int s = lane + 64 * (b * P + p);
                    if (s < slots) S::load(f[r][p], PtrRow{rp}, s);
                }
            }
        }
    };

    int32_t g = wave;
    if (g < ngroups) issue(cur, g, 0);
    if (TYPE != kBF16) {
        quantize_block8(x, k / 32, threadIdx.x, kThreads, q, meta);
        __syncthreads();
    }
    Act areg[AREG ? P : 1];
    if constexpr (AREG) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int s = lane + 64 * p;
            if (s < slots) slot_act<TYPE>(areg[p], s, q, meta, x);
        }
    }
    for (; g < ngroups; g += nwaves) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        for (int32_t b = 0; b < nbatch; ++b) {
            if (b + 1 < nbatch) issue(nxt, g, b + 1);
            else if (g + nwaves < ngroups) issue(nxt, g + nwaves, 0);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int32_t row = g * R + r;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const int s = lane + 64 * (b * P + p);
                    if (s < slots && row < n) {
                        if constexpr (AREG) {
                            acc[r] += S::dot(cur[r][p], areg[p], s);
                        } else {
                            Act a;
                            slot_act<TYPE>(a, s, q, meta, x);
                            acc[r] += S::dot(cur[r][p], a, s);
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int p = 0; p < P; ++p) cur[r][p] = nxt[r][p];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[r]);
            const int32_t row = g * R + r;
            if (lane == 0 && row < n) y[row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Band kernel (the main path): one work-group per CU, so x is quantised into
// LDS only 256 times per call.  Work-group g owns rows g, g + G, g + 2G, ...
// (G = number of work-groups): at any moment the whole GPU is sweeping one
// contiguous stretch of the matrix, which keeps HBM pages and channels busy
// the way a plain streaming read does (a contiguous band per work-group
// measured 2x slower).
//
// Waves are arranged nwk x nwr: wave (kw, rw) covers slots [64 kw, 64 kw + 64)
// of a row (one K-slice, its activations kept in registers).  Rows are handed
// out one at a time from an LDS counter per K-slice, so waves the memory
// system serves first take more rows (with a static split the last of a CU's
// 16 waves finished up to 15% after the first).  Results never depend on
// which wave took which row: K-slice partials meet in LDS and are added in a
// fixed order.
//
// Two schedules, picked per shape from measurements on Q4_K / Q6_K / Q8_0 /
// Q4_0 / BF16 at K = 4096 and 14336:
//
//   ONE (at least 8 row-waves, i.e. K up to 128 slots with 16 waves): each
//   wave keeps one row in flight.  With 16 rows of ~2-4 KB in flight per CU a
//   plain read of the matrix streams fastest (33 MB read in 6.4 us against
//   6.9 us with two rows per wave).  The single row leaves nothing to cover
//   the quantisation of x, so the first nqw waves (at least 4, one per SIMD)
//   issue their x loads first, then their first two rows, then quantise (the
//   waitcnt for x does not wait for the rows), and every wave starts with two
//   rows in flight.  Loads are plain global loads: rows past the end and lanes
//   without a slot re-read valid bytes (local row 0, slot 0) whose results
//   are unused, so no load sits behind a branch and each waitcnt counts
//   exactly the loads issued after the one it needs.  With one K-slice per
//   row each wave keeps its results in registers and stores them once it has
//   no loads left (0.1-0.3 us faster than writing y from LDS after a barrier);
//   K-split rows meet in LDS and y is written once all rows are done.
//
//   TWO (K-split rows, or 8 waves per CU): each wave keeps two rows in flight
//   in two register buffers used in turn; the first nqw waves quantise x
//   before they touch weights and the other waves issue their first two rows
//   at once.  Loads go through a per-row buffer resource whose past-the-end
//   form (num_records 0) reads zeros and makes no memory request, so the
//   steady loop issues the same loads every turn.  With one K-slice per row
//   the wave writes y itself.
//
// The quantised-x count is an LDS counter with relaxed atomics: writers wait
// for their own q / meta writes (lgkmcnt(0)) before the increment and readers
// read q only after seeing the count, so LDS ordering is explicit (the
// release / acquire forms made the compiler wait for every weight load too).
//
// Two block sizes: 16 waves per CU for matrices up to kBandStreamBytes per
// work-group (more loads in flight ramp a short call up faster), 8 waves
// above that (fewer rows in flight keep the swept window of the matrix small:
// Q6_K 4096 x 128256 measured 80 us with 8 waves against 98 us with 16).
#ifndef GNCX_BAND_THREADS
#define GNCX_BAND_THREADS 1024
#endif
#ifndef GNCX_BAND_THREADS_STREAM
#define GNCX_BAND_THREADS_STREAM 512
#endif
#ifndef GNCX_BAND_STREAM_KB
#define GNCX_BAND_STREAM_KB 256
#endif
#ifndef GNCX_BAND_GROUPS
#define GNCX_BAND_GROUPS 256
#endif
constexpr int kBandThreads = GNCX_BAND_THREADS;
constexpr int kBandThreadsStream = GNCX_BAND_THREADS_STREAM;
constexpr size_t kBandStreamBytes = static_cast<size_t>(GNCX_BAND_STREAM_KB) * 1024;
constexpr int32_t kBandGroups = GNCX_BAND_GROUPS;  // one work-group per CU of an MI355X
constexpr size_t kBandLds = 64 * 1024;
constexpr size_t kBandCtl = 256;    // LDS head: per-K-slice row counters, the quantised count, norm partials
constexpr int kCtlQuantised = 31;   // index of the count of waves done quantising
constexpr int kCtlNormPart = 32;    // [16] per-wave sums of squares of the add+RMSNorm prologue
constexpr int kCtlNormCount = 48;   // count of waves that stored their sum of squares
constexpr int kOneMinRowWaves = 8;  // ONE schedule from this many row-waves (16-wave groups only)
#ifndef GNCX_NORM_WAVES
#define GNCX_NORM_WAVES 8
#endif
constexpr int kNormWaves = GNCX_NORM_WAVES;  // waves forming x in the add+RMSNorm prologue (k <= 4096)
constexpr int kNormU = 16 / kNormWaves;  // float4 of x per thread of those waves
constexpr int kNormStride = 64 * kNormWaves;

enum BandSched { kSchedOne = 1, kSchedTwo = 2 };

// x tasks (4 values) per quantising thread with loads in flight together,
// and the least number of quantising waves
template <int SCHED>
struct BandQuant {
    static constexpr int kU = SCHED == kSchedOne ? 4 : 8;
    static constexpr int kMinWaves = SCHED == kSchedOne ? 4 : 1;
};

// The matrices of one launch: rows [end[i-1], end[i]) of the launch's row
// space are rows of W_i, written to y_i (end[] < 2^31).  MULTI = false is
// the single matrix of a plain matvec, with no lookup at all; with MULTI a
// row lookup is a chain of 32-bit scalar compares and selects over kernel
// arguments at fixed offsets (an indexed w[m] became a scalar memory load per
// row, and 64-bit select chains at every lookup cost 0.5-1.5 us on short
// rows, hence the separate instantiation).
struct BandMats {
    const uint8_t* w[kMaxGemvMats];
    float* y[kMaxGemvMats];
    int32_t end[kMaxGemvMats];
    int32_t count;
    template <bool MULTI, class P>
    __device__ __forceinline__ P pick(size_t g, const P (&a)[kMaxGemvMats], size_t& first) const {
        P p = a[0];
        first = 0;
        if constexpr (MULTI) {
            const int32_t gi = static_cast<int32_t>(g);
#pragma unroll
            for (int m = 1; m < kMaxGemvMats; ++m) {
                if (count > m && gi >= end[m - 1]) {
                    p = a[m];
                    first = static_cast<size_t>(end[m - 1]);
                }
            }
        }
        return p;
    }
    template <bool MULTI>
    __device__ __forceinline__ const uint8_t* row(size_t g, uint32_t rbytes) const {
        size_t first;
        const uint8_t* p = pick<MULTI>(g, w, first);
        return p + (g - first) * rbytes;
    }
    template <bool MULTI>
    __device__ __forceinline__ float* out(size_t g) const {
        size_t first;
        float* p = pick<MULTI>(g, y, first);
        return p + (g - first);
    }
};

// Fused prologue / epilogue of the decode chain (ONE schedule, 1024 threads,
// one K-slice per row, k <= 4096):
//   kExtNorm    x = RMSNorm(h + r) * gamma, formed by every work-group from h,
//               r and gamma with the arithmetic of rmsnorm_kernel<true> (the
//               same per-thread float4, wave sums and ordered sum of the 16
//               wave partials), so the quantised x is the one the separate
//               add+RMSNorm kernel feeds a plain matvec; work-group 0 stores
//               h + r to h_out (h_out != h: other work-groups still read h);
//   kExtSwiglu  two matrices of N rows each (gate, up) with N a multiple of the
//               grid: work-group g holds gate row i and up row i in its LDS
//               results and writes act[i] = SiLU(gate[i]) * up[i] with the
//               arithmetic of swiglu_kernel; gate and up are not stored.
enum BandExt { kExtNone = 0, kExtNorm = 1, kExtSwiglu = 2 };
struct BandExtra {
    const float* h;
    const float* r;  // may be null: x = RMSNorm(h) * gamma
    const float* gamma;
    float* h_out;    // may be null
    float* act;
    float eps;
};

template <int TYPE, int THREADS, int SCHED, bool MULTI, int EXT = kExtNone>
__global__ __launch_bounds__(THREADS) void gemv_band_kernel(BandMats mats, uint32_t rbytes,
                                                                 const float* __restrict x, int32_t k,
                                                                 int32_t n, int32_t nwk, int32_t nwr, int32_t nqw,
                                                                 BandExtra ex) {
    static_assert(EXT == kExtNone || (SCHED == kSchedOne && THREADS == 1024 && TYPE != kBF16),
                  "fused prologue / epilogue: ONE schedule, 1024 threads, quantised weights");
    using S = Slot<TYPE>;
    using Frag = typename S::Frag;
    using Act = typename S::Act;
    constexpr bool kQuant = TYPE != kBF16;
    constexpr int kU = BandQuant<SCHED>::kU;
    extern __shared__ __align__(16) uint8_t lds[];
    int32_t* ctl = reinterpret_cast<int32_t*>(lds);
    int8_t* q = reinterpret_cast<int8_t*>(lds + kBandCtl);
    ActMeta* meta = reinterpret_cast<ActMeta*>(lds + kBandCtl + k);
    const size_t qbytes = kQuant ? static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta) : 0;
    float* part = reinterpret_cast<float*>(lds + kBandCtl + qbytes);  // [local row][nwk]

    const int lane = threadIdx.x & 63;
    // ONE branches on the wave index around loads, where a uniform branch keeps
    // each waitcnt exact; TWO measured faster with the index in a vector register
    const int wv = SCHED == kSchedOne ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)
                                      : static_cast<int>(threadIdx.x >> 6);
    const int kw = wv % nwk, rw = wv / nwk;
    const bool active = rw < nwr;
    const bool qwave = kQuant && wv < nqw;
    const int32_t slots = S::slots(k);
    const int s = kw * 64 + lane;
    const bool has_slot = active && s < slots;
    const int32_t groups = gridDim.x;
    // local row li of this work-group is global row li * groups + blockIdx.x
    const int32_t rows_here = (n - static_cast<int32_t>(blockIdx.x) + groups - 1) / groups;
    auto grow = [&](int32_t li) { return static_cast<size_t>(li) * groups + blockIdx.x; };
    // whole rows (one K-slice): under TWO the wave stores y itself after each
    // row; under ONE it keeps its results in registers (lane i: its i-th row)
    // and stores them with one instruction once it has no loads left, since a
    // store issued between loads holds up the vmcnt wait of every later load
    const bool direct = SCHED == kSchedTwo && nwk == 1;
    const bool wstore = SCHED == kSchedOne && nwk == 1 && !(EXT & kExtSwiglu);
    int32_t nres = 0;
    float res = 0.0f;
    int32_t res_row = 0;
    auto flush = [&]() {
        if (lane < nres) *mats.template out<MULTI>(grow(res_row)) = res;
        nres = 0;
    };

    if (threadIdx.x < kBandCtl / sizeof(int32_t)) ctl[threadIdx.x] = 0;
    __syncthreads();

    auto grab = [&]() -> int32_t {
        int32_t g = 0;
        if (lane == 0) g = __hip_atomic_fetch_add(&ctl[kw], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        return __builtin_amdgcn_readfirstlane(g);
    };
    auto issue = [&](Frag& f, int32_t li) {
        const bool ok = li < rows_here;
        if constexpr (SCHED == kSchedOne)
            S::load(f, PtrRow{mats.template row<MULTI>(grow(ok ? li : 0), rbytes)}, has_slot ? s : 0);
        else
            S::load(f, BufRow(mats.template row<MULTI>(ok ? grow(li) : 0, rbytes), rbytes, ok), s);
    };
    auto reduce = [&](const Frag& f, const Act& a, int32_t li) {
        float v = has_slot ? S::dot(f, a, s) : 0.0f;
        v = wave_sum_lane63(v);
        if (wstore) {
            const float sv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
            const bool mine = lane == nres;
            res = mine ? sv : res;
            res_row = mine ? li : res_row;
            if (++nres == 64) flush();
            return;
        }
        if (lane == 63) {
            if (direct) *mats.template out<MULTI>(grow(li)) = v;
            else part[li * nwk + kw] = v;
        }
    };
    auto quantise = [&](const float4 (&xv)[kU]) {
        quant_finish<kU>(xv, x, k / 32, threadIdx.x, nqw * 64, q, meta);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's q / meta writes are done
        asm volatile("" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(&ctl[kCtlQuantised], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    auto act = [&](Act& a) {
        if (kQuant) {
            // the quantising waves depend on nothing but their own x loads
            while (__hip_atomic_load(&ctl[kCtlQuantised], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < nqw)
                __builtin_amdgcn_s_sleep(1);
            asm volatile("" ::: "memory");
        }
        if (has_slot) slot_act<TYPE>(a, s, q, meta, x);
    };

    Frag fa, fb;
    int32_t ja = rows_here, jb = rows_here;
    if constexpr (SCHED == kSchedOne) {
        auto start = [&]() {
            if (active) {
                ja = grab();
                jb = grab();
            }
            issue(fa, ja);
            issue(fb, jb);
        };
        // kExtNorm: h + r of float4 vt = threadIdx.x + 256 u of a quantising thread
        float4 hsum[kNormU];
        const int32_t n4 = k / 4;
        if constexpr ((EXT & kExtNorm) != 0) {
#pragma clang fp contract(off)
            // The first kNormWaves waves form x as 1024 threads of one float4
            // each would: thread threadIdx.x stands for the threads vt =
            // threadIdx.x + kNormStride u, of "virtual wave" wv + kNormWaves u,
            // whose wave sum goes to partial wv + kNormWaves u, and the 16
            // partials are added in order -- the association of
            // rmsnorm_kernel<true> -- so x is bit-identical with it.  The
            // other waves issue their rows at once; h, r and gamma go first,
            // so their waitcnt does not wait for the rows (the loads are
            // unconditional, clamped to the last float4 of x: a load behind a
            // branch made the compiler wait for every row, +2.5 us).
            if (qwave) {
                float4 hv[kNormU], rv[kNormU], gv[kNormU];
#pragma unroll
                for (int u = 0; u < kNormU; ++u) {
                    const int32_t vt = static_cast<int32_t>(threadIdx.x) + kNormStride * u;
                    const int32_t t4 = vt < n4 ? vt : n4 - 1;
                    hv[u] = reinterpret_cast<const float4*>(ex.h)[t4];
                    rv[u] = ex.r ? reinterpret_cast<const float4*>(ex.r)[t4] : make_float4(0.f, 0.f, 0.f, 0.f);
                    gv[u] = reinterpret_cast<const float4*>(ex.gamma)[t4];
                }
                start();
                float* npart = reinterpret_cast<float*>(ctl + kCtlNormPart);
#pragma unroll
                for (int u = 0; u < kNormU; ++u) {
                    hsum[u] = ex.r ? make_float4(hv[u].x + rv[u].x, hv[u].y + rv[u].y, hv[u].z + rv[u].z,
                                                 hv[u].w + rv[u].w)
                                   : hv[u];
                    const bool mine = static_cast<int32_t>(threadIdx.x) + kNormStride * u < n4;
                    float ss = mine ? hsum[u].x * hsum[u].x + hsum[u].y * hsum[u].y + hsum[u].z * hsum[u].z +
                                          hsum[u].w * hsum[u].w
                                    : 0.0f;
                    ss = wave_sum(ss);
                    if (lane == 0) npart[wv + kNormWaves * u] = ss;
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                asm volatile("" ::: "memory");
                if (lane == 0)
                    __hip_atomic_fetch_add(&ctl[kCtlNormCount], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                while (__hip_atomic_load(&ctl[kCtlNormCount], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <
                       kNormWaves)
                    __builtin_amdgcn_s_sleep(1);
                asm volatile("" ::: "memory");
                float tot = 0.0f;
#pragma unroll
                for (int w = 0; w < 16; ++w) tot += npart[w];
                const float inv = 1.0f / sqrtf(tot / static_cast<float>(k) + ex.eps);
#pragma unroll
                for (int u = 0; u < kNormU; ++u) {
                    const int32_t vt = static_cast<int32_t>(threadIdx.x) + kNormStride * u;
                    const float4 xn = make_float4(hsum[u].x * inv * gv[u].x, hsum[u].y * inv * gv[u].y,
                                                  hsum[u].z * inv * gv[u].z, hsum[u].w * inv * gv[u].w);
                    if (vt < n4) quantize_task(xn, vt >> 3, vt & 7, q, meta);
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);
                asm volatile("" ::: "memory");
                if (lane == 0)
                    __hip_atomic_fetch_add(&ctl[kCtlQuantised], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
                start();
            }
        } else if (qwave) {
            float4 xv[kU];
            quant_load<kU>(xv, x, k / 32, threadIdx.x, nqw * 64);
            start();
            quantise(xv);
        } else {
            start();
        }
        if (active) {
            Act a;
            act(a);
            if (ja < rows_here) reduce(fa, a, ja);
            if (jb < rows_here) reduce(fb, a, jb);
            for (int32_t li = jb < rows_here ? grab() : rows_here; li < rows_here; li = grab()) {
                issue(fa, li);
                reduce(fa, a, li);
            }
        }
        if constexpr ((EXT & kExtNorm) != 0) {
            if (blockIdx.x == 0 && ex.h_out && qwave) {
#pragma unroll
                for (int u = 0; u < kNormU; ++u) {
                    const int32_t vt = static_cast<int32_t>(threadIdx.x) + kNormStride * u;
                    if (vt < n4) reinterpret_cast<float4*>(ex.h_out)[vt] = hsum[u];
                }
            }
        }
    } else {
        if (qwave) {
            float4 xv[kU];
            quant_load<kU>(xv, x, k / 32, threadIdx.x, nqw * 64);
            quantise(xv);
        }
        if (active) {
            ja = grab();
            issue(fa, ja);
            jb = grab();
            issue(fb, jb);
            Act a;
            act(a);
            while (ja < rows_here || jb < rows_here) {  // wave-uniform
                if (ja < rows_here) {
                    reduce(fa, a, ja);
                    ja = grab();
                }
                issue(fa, ja);
                if (jb < rows_here) {
                    reduce(fb, a, jb);
                    jb = grab();
                }
                issue(fb, jb);
            }
        }
    }
    if (direct) return;
    if (wstore) {
        flush();
        return;
    }
    __syncthreads();
    if constexpr ((EXT & kExtSwiglu) != 0) {
#pragma clang fp contract(off)
        const int32_t half = rows_here / 2;  // local row li + half is up row li
        for (int32_t li = threadIdx.x; li < half; li += THREADS) {
            const float g = part[li], u = part[li + half];
            ex.act[grow(li)] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
        }
        return;
    }
    for (int32_t li = threadIdx.x; li < rows_here; li += THREADS) {
        float acc = 0.0f;
        for (int j = 0; j < nwk; ++j) acc += part[li * nwk + j];
        *mats.template out<MULTI>(grow(li)) = acc;
    }
}

__global__ __launch_bounds__(kThreads) void act_quant_kernel(const float* __restrict x, int32_t k,
                                                             int8_t* __restrict q, ActMeta* __restrict meta) {
    const int32_t row = blockIdx.y;
    const int32_t nb = k / 32;
    // blocks of this row handled by this work-group: 32 per group
    const int32_t b0 = blockIdx.x * (kThreads / 8);
    const int32_t nb_here = min(nb - b0, kThreads / 8);
    if (nb_here <= 0) return;
    dev::quantize_block8(x + static_cast<size_t>(row) * k + static_cast<size_t>(b0) * 32, nb_here,
                         threadIdx.x, kThreads, q + static_cast<size_t>(row) * k + static_cast<size_t>(b0) * 32,
                         meta + static_cast<size_t>(row) * nb + b0);
}

template <int TYPE, int P, int R, bool AREG>
hipError_t launch_shape(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y, hipStream_t stream) {
    const size_t rb = row_bytes(TYPE, k);
    const size_t lds = TYPE == kBF16 ? 0 : static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta);
    const int32_t ngroups = (n + R - 1) / R;
    int32_t waves = 256 * GNCX_GEMV_WAVES_PER_CU;
    if (waves > ngroups) waves = ngroups;
    const int32_t groups = (waves + kThreads / 64 - 1) / (kThreads / 64);
    hipLaunchKernelGGL((gemv_kernel<TYPE, P, R, AREG>), dim3(groups), dim3(kThreads), lds, stream, w, rb, x, k, n, y);
    return hipGetLastError();
}

// Rows of one pass (<= 64 slots) go two to a wave; longer rows one to a wave,
// in batches of up to PMAX passes (register budget of the format's slot).
template <int TYPE, int PMAX>
hipError_t launch_gemv_t(const uint8_t* w, const float* x, int32_t k, int32_t n, float* y, hipStream_t stream) {
    const int32_t passes = (Slot<TYPE>::slots(k) + 63) / 64;
    if (passes <= 1) return launch_shape<TYPE, 1, 2, true>(w, x, k, n, y, stream);
    if (passes == 2) return launch_shape<TYPE, 2, 1, true>(w, x, k, n, y, stream);
    if (PMAX == 2) return launch_shape<TYPE, 2, 1, false>(w, x, k, n, y, stream);
    if (passes <= PMAX) return launch_shape<TYPE, (PMAX > 2 ? PMAX : 2), 1, true>(w, x, k, n, y, stream);
    return launch_shape<TYPE, (PMAX > 2 ? PMAX : 2), 1, false>(w, x, k, n, y, stream);
}


// Band kernel geometry for (type, k, n) with `waves` waves per work-group
// under schedule `sched`; false when the shape does not fit it.
bool band_plan(int32_t slots, int32_t k, int32_t n, bool quantised, int32_t waves, int sched, int32_t& groups,
               int32_t& nwk, int32_t& nwr, int32_t& nqw, size_t& lds) {
    nwk = (slots + 63) / 64;
    if (nwk < 1 || nwk > waves) return false;
    nwr = waves / nwk;
    groups = n < kBandGroups ? n : kBandGroups;
    const int32_t rows_per_wg = (n + groups - 1) / groups;
    groups = (n + rows_per_wg - 1) / rows_per_wg;
    const int32_t tasks = k / 4;  // 4 values of x per quantisation task
    const int u = sched == kSchedOne ? BandQuant<kSchedOne>::kU : BandQuant<kSchedTwo>::kU;
    const int min_waves = sched == kSchedOne ? BandQuant<kSchedOne>::kMinWaves : BandQuant<kSchedTwo>::kMinWaves;
    nqw = quantised ? (tasks + 64 * u - 1) / (64 * u) : 0;
    if (quantised && nqw < min_waves) nqw = min_waves;
    if (nqw > waves) nqw = waves;
    const size_t qbytes = quantised ? static_cast<size_t>(k) + static_cast<size_t>(k / 32) * sizeof(ActMeta) : 0;
    const bool direct = sched == kSchedTwo && nwk == 1;
    lds = kBandCtl + qbytes + (direct ? 0 : sizeof(float) * static_cast<size_t>(rows_per_wg) * nwk);
    return lds <= kBandLds && nwk <= static_cast<int32_t>(kCtlQuantised);
}

template <int TYPE, int THREADS, int SCHED>
bool try_band_sched(const BandMats& m, const float* x, int32_t k, int32_t n, hipStream_t stream) {
    int32_t groups, nwk, nwr, nqw;
    size_t lds;
    if (!band_plan(Slot<TYPE>::slots(k), k, n, TYPE != kBF16, THREADS / 64, SCHED, groups, nwk, nwr, nqw, lds))
        return false;
    const uint32_t rb = static_cast<uint32_t>(row_bytes(TYPE, k));
    if (m.count > 1)
        hipLaunchKernelGGL((gemv_band_kernel<TYPE, THREADS, SCHED, true>), dim3(groups), dim3(THREADS), lds, stream, m,
                           rb, x, k, n, nwk, nwr, nqw, BandExtra{});
    else
        hipLaunchKernelGGL((gemv_band_kernel<TYPE, THREADS, SCHED, false>), dim3(groups), dim3(THREADS), lds, stream,
                           m, rb, x, k, n, nwk, nwr, nqw, BandExtra{});
    return true;
}

// The fused forms (BandExt): ONE schedule with 16 waves and whole rows only;
// false when the shape does not fit (the caller runs the separate kernels).
template <int TYPE, int EXT>
bool try_band_ext(const BandMats& m, const float* x, int32_t k, int32_t n, const BandExtra& ex, hipStream_t stream) {
    int32_t groups, nwk, nwr, nqw;
    size_t lds;
    if (!band_plan(Slot<TYPE>::slots(k), k, n, true, 16, kSchedOne, groups, nwk, nwr, nqw, lds)) return false;
    if (nwk != 1 || nwr < kOneMinRowWaves) return false;
    if constexpr ((EXT & kExtNorm) != 0) {
        if (k % 4 != 0 || k > 4 * 1024) return false;
        nqw = kNormWaves;  // kNormU float4 of x per thread of these waves
    }
    if constexpr ((EXT & kExtSwiglu) != 0) {
        if (m.count != 2 || 2 * m.end[0] != n || m.end[0] % groups != 0) return false;
    }
    const uint32_t rb = static_cast<uint32_t>(row_bytes(TYPE, k));
    if (m.count > 1)
        hipLaunchKernelGGL((gemv_band_kernel<TYPE, 1024, kSchedOne, true, EXT>), dim3(groups), dim3(1024), lds, stream,
                           m, rb, x, k, n, nwk, nwr, nqw, ex);
    else if constexpr ((EXT & kExtSwiglu) == 0)
        hipLaunchKernelGGL((gemv_band_kernel<TYPE, 1024, kSchedOne, false, EXT>), dim3(groups), dim3(1024), lds,
                           stream, m, rb, x, k, n, nwk, nwr, nqw, ex);
    else
        return false;
    return true;
}

template <int EXT>
bool try_band_ext_type(int32_t type, const BandMats& m, const float* x, int32_t k, int32_t n, const BandExtra& ex,
                       hipStream_t stream) {
    switch (type) {
    case kQ4_0: return try_band_ext<kQ4_0, EXT>(m, x, k, n, ex, stream);
    case kQ8_0: return try_band_ext<kQ8_0, EXT>(m, x, k, n, ex, stream);
    case kQ4_K: return try_band_ext<kQ4_K, EXT>(m, x, k, n, ex, stream);
    case kQ6_K: return try_band_ext<kQ6_K, EXT>(m, x, k, n, ex, stream);
    default: return false;
    }
}

// ONE for 16-wave groups with at least kOneMinRowWaves row-waves, and for
// Q4_K / Q8_0 rows split into three or more K-slices (Q4_K 12288 x 4096:
// 8.2 vs 8.8 us under TWO; Q8_0 14336 x 4096: 14.3 vs 15.5 us); TWO otherwise
template <int TYPE, int THREADS>
bool try_band(const BandMats& m, const float* x, int32_t k, int32_t n, hipStream_t stream) {
    const int32_t nwk = (Slot<TYPE>::slots(k) + 63) / 64;
    const bool one = nwk >= 1 && ((THREADS / 64) / nwk >= kOneMinRowWaves ||
                                  (nwk >= 3 && (TYPE == kQ4_K || TYPE == kQ8_0)));
    if (THREADS == 1024 && one && try_band_sched<TYPE, THREADS, kSchedOne>(m, x, k, n, stream)) return true;
    return try_band_sched<TYPE, THREADS, kSchedTwo>(m, x, k, n, stream);
}

// n = total rows of the matrices in m
template <int TYPE>
hipError_t launch_band(const BandMats& m, const float* x, int32_t k, int32_t n, hipStream_t stream, bool& used) {
    const int32_t groups = n < kBandGroups ? n : kBandGroups;
    const size_t per_group = row_bytes(TYPE, k) * static_cast<size_t>(n) / static_cast<size_t>(groups);
    // Long-K Q6_K (three or more K-slices) also streams best with 16 waves:
    // 14336 x 4096 12.5-12.7 us against 13.3-13.7 with 8, 12288 x 4096 11.1
    // against 12.0-12.3 (the same boxes, back-to-back calls on 16 copies)
    used = (per_group > kBandStreamBytes && try_band<TYPE, kBandThreadsStream>(m, x, k, n, stream)) ||
           try_band<TYPE, kBandThreads>(m, x, k, n, stream);
    return used ? hipGetLastError() : hipSuccess;
}

hipError_t launch_band_type(int32_t type, const BandMats& m, const float* x, int32_t k, int32_t n,
                            hipStream_t stream, bool& used) {
    switch (type) {
    case kQ4_0: return launch_band<kQ4_0>(m, x, k, n, stream, used);
    case kQ8_0: return launch_band<kQ8_0>(m, x, k, n, stream, used);
    case kQ4_K: return launch_band<kQ4_K>(m, x, k, n, stream, used);
    case kQ6_K: return launch_band<kQ6_K>(m, x, k, n, stream, used);
    case kBF16: return launch_band<kBF16>(m, x, k, n, stream, used);
    default: used = false; return hipErrorInvalidValue;
    }
}

// shape and alignment rules shared by the single and multi launchers
hipError_t check_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k) {
    if (k <= 0 || k > kMaxGemvK) return hipErrorInvalidValue;
    if (type != kBF16 && (k % 32) != 0) return hipErrorInvalidValue;
    if ((type == kQ4_K || type == kQ6_K) && (k % 256) != 0) return hipErrorInvalidValue;
    if (type == kBF16 && (k % 8) != 0) return hipErrorInvalidValue;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
    if ((xa & 15u) != 0) return hipErrorInvalidValue;
    if (type == kQ4_K || type == kBF16) {
        if ((wa & 15u) != 0 || (row_bytes(type, k) & 15u) != 0) return hipErrorInvalidValue;
    } else if ((wa & 3u) != 0) {
        return hipErrorInvalidValue;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y,
                       hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipError_t e = check_gemv(type, w, x, k);
    if (e != hipSuccess) return e;
    BandMats m{};
    m.w[0] = w;
    m.y[0] = y;
    m.end[0] = n;
    m.count = 1;
    bool used = false;
    e = launch_band_type(type, m, x, k, n, stream, used);
    if (used || e != hipSuccess) return e;
    switch (type) {
    case kQ4_0: return launch_gemv_t<kQ4_0, 4>(w, x, k, n, y, stream);
    case kQ8_0: return launch_gemv_t<kQ8_0, 2>(w, x, k, n, y, stream);
    case kQ4_K: return launch_gemv_t<kQ4_K, 2>(w, x, k, n, y, stream);
    case kQ6_K: return launch_gemv_t<kQ6_K, 2>(w, x, k, n, y, stream);
    case kBF16: return launch_gemv_t<kBF16, 4>(w, x, k, n, y, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_multi(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                             const float* x, int32_t k, float* const* ys, hipStream_t stream) {
    if (count <= 0 || count > kMaxGemvMats) return hipErrorInvalidValue;
    BandMats m{};
    int64_t total = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (ns[i] < 0) return hipErrorInvalidValue;
        hipError_t e = check_gemv(type, ws[i], x, k);
        if (e != hipSuccess) return e;
        total += ns[i];
        m.w[i] = ws[i];
        m.y[i] = ys[i];
        m.end[i] = static_cast<int32_t>(total);
    }
    if (total == 0) return hipSuccess;
    if (total > INT32_MAX) return hipErrorInvalidValue;
    m.count = count;
    bool used = false;
    hipError_t e = launch_band_type(type, m, x, k, static_cast<int32_t>(total), stream, used);
    if (used || e != hipSuccess) return e;
    for (int32_t i = 0; i < count; ++i) {
        e = launch_gemv(type, ws[i], x, k, ns[i], ys[i], stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemv_fused(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns, int32_t k,
                             float* const* ys, const GemvFusion& f, hipStream_t stream) {
    const bool norm = f.gamma != nullptr, glu = f.act != nullptr;
    if (count <= 0 || count > kMaxGemvMats || (!norm && !glu)) return hipErrorInvalidValue;
    if (norm && (!f.h || f.h == f.h_out)) return hipErrorInvalidValue;
    if (!norm && !f.x) return hipErrorInvalidValue;
    const float* xin = norm ? f.h : f.x;  // alignment and shape checks
    const uintptr_t al = reinterpret_cast<uintptr_t>(f.h) | reinterpret_cast<uintptr_t>(f.r) |
                         reinterpret_cast<uintptr_t>(f.gamma) | reinterpret_cast<uintptr_t>(f.h_out);
    if (norm && (al & 15u) != 0) return hipErrorInvalidValue;
    BandMats m{};
    int64_t total = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (ns[i] <= 0) return hipErrorInvalidValue;
        hipError_t e = check_gemv(type, ws[i], xin, k);
        if (e != hipSuccess) return e;
        total += ns[i];
        m.w[i] = ws[i];
        m.y[i] = ys ? ys[i] : nullptr;
        m.end[i] = static_cast<int32_t>(total);
    }
    if (total > INT32_MAX) return hipErrorInvalidValue;
    if (glu && (count != 2 || ns[0] != ns[1])) return hipErrorInvalidValue;
    if (!glu && !ys) return hipErrorInvalidValue;
    m.count = count;
    const BandExtra ex{f.h, f.r, f.gamma, f.h_out, f.act, f.eps};
    const int32_t n = static_cast<int32_t>(total);
    bool ok;
    if (norm && glu) ok = try_band_ext_type<kExtNorm | kExtSwiglu>(type, m, nullptr, k, n, ex, stream);
    else if (norm) ok = try_band_ext_type<kExtNorm>(type, m, nullptr, k, n, ex, stream);
    else ok = try_band_ext_type<kExtSwiglu>(type, m, f.x, k, n, ex, stream);
    return ok ? hipGetLastError() : hipErrorNotSupported;
}

hipError_t launch_act_quant(const float* x, int32_t rows, int32_t k, int8_t* q, ActMeta* meta,
                            hipStream_t stream) {
    if (rows <= 0 || k <= 0) return hipSuccess;
    if ((k % 32) != 0 || (reinterpret_cast<uintptr_t>(x) & 15u) != 0) return hipErrorInvalidValue;
    const int32_t nb = k / 32;
    const int32_t gx = (nb + kThreads / 8 - 1) / (kThreads / 8);
    hipLaunchKernelGGL(act_quant_kernel, dim3(gx, rows), dim3(kThreads), 0, stream, x, k, q, meta);
    return hipGetLastError();
}

}  // namespace gncx
