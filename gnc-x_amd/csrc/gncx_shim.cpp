// gncx_shim.cpp -- C++20 host shim: the reference's C-ABI on top of HIP.
//
// Every exported name and signature is the one csrc/gncx_llm_kernels.cpp of
// the reference exports (cited per function), so this library drops in for
// bin/gncx_llm_core.so under the LuaJIT FFI (lua/gncx_streamer.lua:16-252).
//
// Pointers crossing the ABI may be host memory (the reference contract: the
// LuaJIT caller passes mmap'ed / RAM-pinned weights and host scratch) or HIP
// device memory (callers that keep activations in HBM).  The shim classifies
// each pointer with hipPointerGetAttributes:
//   * weights (base + offset) living on the host are uploaded once, in their
//     native GGUF block layout, into a registry keyed by host address and
//     reused for the life of the process (weights are immutable, the
//     reference's own convention); a cheap content signature guards against a
//     freed-and-reused host address;
//   * host activations are staged through device scratch and host outputs are
//     copied back before the call returns (the reference is synchronous);
//     device activations/outputs are used in place and the call is only
//     stream-ordered (no host synchronisation);
//   * a host KV cache gets a device twin that is kept coherent: rows the
//     library writes go to both copies, rows it has not seen are uploaded on
//     first use.
// Calls are serialised with one mutex (the reference is not re-entrant
// either).  On any failure the call prints one line to stderr, records the
// error for gncx_hip_last_error(), and leaves its outputs untouched; there
// is no CPU fallback.  GNCX_ABORT_ON_ERROR=1 turns failures into abort().
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <linux/futex.h>
#include <signal.h>
#include <sys/mman.h>
#include <sys/syscall.h>
#include <sys/stat.h>
#include <ucontext.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "gncx_formats.h"
#include "gncx_launch.h"
// the public declarations: every definition below must match them
#include "../../include/gncx_llm_core.h"

#define GNCX_API extern "C" __attribute__((visibility("default")))

namespace {

using namespace gncx;

// The one lock of the library; t_in_call marks the thread that holds it (the
// page-fault handler of the lazy host buffers must not take it twice).
// Before the lock is released, a call's writes to lazy host buffers that the
// host reads back get their copies to the host queued (queue_readbacks).
thread_local bool t_in_call = false;
// Deferred work of lazy-host-buffer calls (gathered matvecs, an attention
// prologue) is issued when the lock is next taken, except for the kind the
// locking call may join (t_keep, set around its lock).
enum KeepPending { kKeepNone = 0, kKeepGemv = 1, kKeepPrologue = 2 };
thread_local int t_keep = kKeepNone;
void queue_readbacks();
bool flush_pending(const char* where, int keep = kKeepNone);
// Page-locked host memory that the current call's kernels read in place (a
// lazy host buffer's pinned copy, read once by a call that waits for its
// kernels); stage_in passes these through.  Cleared when the call releases
// the lock.
std::array<const void*, 4> g_direct{};
int g_ndirect = 0;
bool is_direct(const void* p) {
    for (int i = 0; i < g_ndirect; ++i)
        if (g_direct[i] == p) return true;
    return false;
}
struct CallLock {
    std::mutex m;
    void lock() {
        m.lock();
        t_in_call = true;
        (void)flush_pending("deferred call", t_keep);
    }
    void unlock() {
        queue_readbacks();
        g_ndirect = 0;
        t_in_call = false;
        m.unlock();
    }
};
CallLock g_mu;
std::string g_last_error;
int g_last_code = 0;

// Device-to-host copies staged in pinned slots, copied to the caller's
// buffers by sync_out.  A call that fails before its sync drops them, so a
// later call never writes into an earlier caller's (possibly freed) buffer.
struct Deferred {
    void* host;
    const void* pinned;
    size_t n;
};
std::vector<Deferred> g_deferred;

void set_error(const char* where, const char* what, int code) {
    g_deferred.clear();
    g_last_error = std::string(where) + ": " + what;
    g_last_code = code ? code : -1;
    std::fprintf(stderr, "gncx_llm_core: %s\n", g_last_error.c_str());
    const char* ab = std::getenv("GNCX_ABORT_ON_ERROR");
    if (ab && ab[0] == '1') std::abort();
}

bool check(hipError_t e, const char* where) {
    if (e == hipSuccess) return true;
    set_error(where, hipGetErrorString(e), static_cast<int>(e));
    return false;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
size_t dim_count(int32_t v) { return v > 0 ? static_cast<size_t>(v) : 0; }

// ---- runtime state ----------------------------------------------------

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    bool ensure(size_t bytes, const char* where) {
        if (bytes <= cap && p) return true;
        if (p) {
            (void)hipFree(p);
            p = nullptr;
            cap = 0;
        }
        const size_t c = round_up(std::max<size_t>(bytes, 4096), 1 << 16);
        if (!check(hipMalloc(&p, c), where)) return false;
        cap = c;
        return true;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

struct DevWeight {
    uint8_t* d = nullptr;
    size_t bytes = 0;
    uint64_t sig = 0;
    // where the host bytes live (tracked_host_range):
    //   kMapped     inside a read-only mapping from gncx_gla_map_readonly:
    //               unmapping drops this copy and nothing can write the
    //               bytes, so a hit needs neither the pointer query nor the
    //               content signature;
    //   kRamBuffer  inside a buffer from gncx_ram_alloc*: freeing it or
    //               copying into it drops this copy, but the caller may also
    //               write it with plain stores, so a hit skips the pointer
    //               query (the range is known host memory) and still checks
    //               the content signature;
    //   kUntracked  other host memory: both checks.
    int trust = 0;
};

struct KVTwin {
    float* d = nullptr;
    int32_t cap_rows = 0;
    int32_t kv_dim = 0;
    int32_t valid_rows = 0;
    std::array<float, 8> row0{};  // first values of host row 0 when last synced
};

struct Runtime {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;  // null stream unless the caller sets one
    DevBuf x, y, q, k, v, o, ws, aux;
    std::unordered_map<uintptr_t, DevWeight> weights;
    std::unordered_map<uintptr_t, KVTwin> kv;
};

Runtime g_rt;

bool ensure_runtime(const char* where) {
    if (g_rt.ready) return true;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        set_error(where, "no HIP device is visible (this library has no CPU path)", e ? static_cast<int>(e) : -1);
        return false;
    }
    const char* dv = std::getenv("GNCX_DEVICE");
    g_rt.device = dv ? std::atoi(dv) : 0;
    if (!check(hipSetDevice(g_rt.device), where)) return false;
    g_rt.ready = true;
    return true;
}

bool is_device_ptr(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t a;
    hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

uint64_t host_signature(const uint8_t* p, size_t bytes) {
    uint64_t h = 1469598103934665603ull ^ bytes;
    const size_t probes = 16;
    for (size_t i = 0; i < probes; ++i) {
        size_t off = (bytes > 8) ? (bytes - 8) * i / (probes - 1) : 0;
        uint64_t v = 0;
        std::memcpy(&v, p + off, std::min<size_t>(8, bytes));
        h = (h ^ v) * 1099511628211ull;
    }
    return h;
}

// A deferred matvec or attention prologue may still point at the copy (its
// weights or gamma): recorded work is issued before the copy is freed, and
// hipFree waits for the device, so it never reads freed or re-uploaded bytes.
void forget_weight(uintptr_t key) {
    auto it = g_rt.weights.find(key);
    if (it == g_rt.weights.end()) return;
    (void)flush_pending("weight copy release");
    (void)hipFree(it->second.d);
    g_rt.weights.erase(it);
}

enum WeightTrust : int { kUntracked = 0, kRamBuffer = 1, kMapped = 2 };
int tracked_host_range(const void* p, size_t bytes);

// Device view of `bytes` weight bytes at p (host: uploaded once, cached).
// A copy is keyed by the host address, and the signature reads only the
// `bytes` this call names: the memory at p may now be a different, smaller
// allocation than the one copied (a freed array whose address came back), so
// bytes past the call's range may be unmapped.  A copy of another size is
// dropped and made again.
const uint8_t* device_weights(const uint8_t* p, size_t bytes, const char* where) {
    const uintptr_t key = reinterpret_cast<uintptr_t>(p);
    auto it = g_rt.weights.find(key);
    if (it != g_rt.weights.end() && it->second.bytes >= bytes) {
        if (it->second.trust == kMapped) return it->second.d;
        if (it->second.trust == kRamBuffer) {
            if (it->second.bytes == bytes && it->second.sig == host_signature(p, bytes)) return it->second.d;
            forget_weight(key);
            it = g_rt.weights.end();
        }
    }
    if (is_device_ptr(p)) return p;
    if (it != g_rt.weights.end()) {
        if (it->second.bytes == bytes && it->second.sig == host_signature(p, bytes)) return it->second.d;
        forget_weight(key);
    }
    DevWeight w;
    w.bytes = bytes;
    w.sig = host_signature(p, bytes);
    w.trust = tracked_host_range(p, bytes);
    void* d = nullptr;
    // 256 B aligned, plus slack so no vector load near the end leaves the allocation
    if (!check(hipMalloc(&d, round_up(bytes, 256) + 256), where)) return nullptr;
    if (!check(hipMemcpy(d, p, bytes, hipMemcpyHostToDevice), where)) {
        (void)hipFree(d);
        return nullptr;
    }
    w.d = static_cast<uint8_t*>(d);
    g_rt.weights.emplace(key, w);
    return w.d;
}

// ---- host transfers through pinned bounce slots ------------------------
// Small copies between pageable host memory and the device go through a ring
// of pinned slots: host -> slot -> device, and device -> slot -> host after
// the call's synchronisation (sync_out).  Pageable async copies cost ~2x as
// much per call (42 vs 19 us for an input, a kernel and an output of 16 KB).
// A slot is reused only after its copy completed (event) and its deferred
// host copy was made.  Copies above kPinnedMax go directly.
constexpr size_t kPinnedMax = size_t{1} << 20;
struct PinnedSlot {
    void* p = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;
    bool pending = false;   // a copy from / to the slot may still run
    bool deferred = false;  // holds device output not yet copied to the host
};
std::array<PinnedSlot, 16> g_pin;
int g_pin_next = 0;

bool sync_out(const char* where) {
    if (!check(hipStreamSynchronize(g_rt.stream), where)) return false;
    for (const Deferred& d : g_deferred) std::memcpy(d.host, d.pinned, d.n);
    g_deferred.clear();
    for (PinnedSlot& sl : g_pin) sl.pending = sl.deferred = false;
    return true;
}

PinnedSlot* pinned_slot(size_t bytes, const char* where) {
    PinnedSlot* sl = &g_pin[g_pin_next];
    g_pin_next = (g_pin_next + 1) % static_cast<int>(g_pin.size());
    if (sl->deferred && !sync_out(where)) return nullptr;
    if (sl->pending) {
        if (!check(hipEventSynchronize(sl->ev), where)) return nullptr;
        sl->pending = false;
    }
    if (!sl->ev && !check(hipEventCreateWithFlags(&sl->ev, hipEventDisableTiming), where)) return nullptr;
    if (sl->cap < bytes) {
        if (sl->p) (void)hipHostFree(sl->p);
        sl->p = nullptr;
        sl->cap = 0;
        const size_t c = round_up(std::max<size_t>(bytes, 64 * 1024), 64 * 1024);
        if (!check(hipHostMalloc(&sl->p, c, hipHostMallocDefault), where)) return nullptr;
        sl->cap = c;
    }
    return sl;
}

bool h2d(void* dev, const void* host, size_t bytes, const char* where) {
    if (bytes > kPinnedMax)
        return check(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, g_rt.stream), where);
    PinnedSlot* sl = pinned_slot(bytes, where);
    if (!sl) return false;
    std::memcpy(sl->p, host, bytes);
    if (!check(hipMemcpyAsync(dev, sl->p, bytes, hipMemcpyHostToDevice, g_rt.stream), where)) return false;
    if (!check(hipEventRecord(sl->ev, g_rt.stream), where)) return false;
    sl->pending = true;
    return true;
}

// device -> host, complete once sync_out has returned
bool d2h(void* host, const void* dev, size_t bytes, const char* where) {
    if (bytes > kPinnedMax)
        return check(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, g_rt.stream), where);
    PinnedSlot* sl = pinned_slot(bytes, where);
    if (!sl) return false;
    if (!check(hipMemcpyAsync(sl->p, dev, bytes, hipMemcpyDeviceToHost, g_rt.stream), where)) return false;
    sl->deferred = true;
    g_deferred.push_back({host, sl->p, bytes});
    return true;
}

// Input vector: device pointers pass through, host data is staged into buf.
const float* stage_in(const float* p, size_t count, DevBuf& buf, const char* where) {
    if (!p) return nullptr;
    if (is_direct(p) || is_device_ptr(p)) return p;
    if (!buf.ensure(count * sizeof(float), where)) return nullptr;
    if (!h2d(buf.p, p, count * sizeof(float), where)) return nullptr;
    return buf.as<float>();
}

// Output vector: device pointers pass through, host outputs get scratch.
float* out_target(float* p, size_t count, DevBuf& buf, bool& host, const char* where) {
    host = !is_device_ptr(p);
    if (!host) return p;
    if (!buf.ensure(count * sizeof(float), where)) return nullptr;
    return buf.as<float>();
}

bool finish_out(float* host_dst, const float* dev_src, size_t count, bool host, const char* where) {
    if (!host) return true;
    if (!d2h(host_dst, dev_src, count * sizeof(float), where)) return false;
    return sync_out(where);
}

// ---- 4-phase encode bookkeeping (cpp:782-784, 997-1015) ----------------

uint64_t g_norm_epoch = 0;
uint64_t g_norm_epoch_cancellations = 0;
const GNCXCompactToken* g_norm_epoch_tokens_ptr = nullptr;

uint64_t count_cancellations(const GNCXCompactToken* t, int32_t n) {
    if (!t) return 0;
    if (t == g_norm_epoch_tokens_ptr) return g_norm_epoch_cancellations;
    std::array<uint32_t, 10> pos{}, neg{};
    for (int32_t i = 0; i < n; ++i) {
        const uint8_t d = t[i].diag_d;
        const uint8_t b1 = (t[i].phase_2bit >> 1) & 1u;
        if (d < 10) {
            pos[d] += b1;
            neg[d] += b1 ^ 1u;
        }
    }
    uint64_t c = 0;
    for (int d = 0; d < 10; ++d) c += std::min(pos[d], neg[d]);
    return c;
}

// matvec activation cache key (cpp:1338-1358)
struct ActCache {
    const float* last_in = nullptr;
    int32_t last_dim = 0;
    uint64_t last_epoch = 0;
    uint64_t cached_canceled = 0;
    bool staged_on_device = false;  // scratch x holds that vector
} g_act;

void add_telemetry(GNCXTelemetryStats* t, uint64_t macs, uint64_t canceled, uint64_t merges) {
    if (!t) return;
    t->total_macs_equivalent += macs;
    t->zero_origin_cancellations += canceled;
    t->zero_weight_skips += macs / 15;
    t->xfold_bucket_merges += merges;
}

// Deferred matvecs (lazy host buffers only).  The streamer issues the Q, K
// and V projections, and the gate and up projections, as consecutive matvec
// calls on one normalised vector whose outputs only the device reads.  Such
// calls are gathered (same input, type and in_dim, at most kMaxGemvMats) and
// issued as one multi-matrix launch -- the results are those of separate
// launches bit for bit -- when the lock is next taken by any other call (or
// by a matvec that does not join them), including the fault resolver, so
// every consumer of a deferred output, device or host, finds it issued
// first.  A deferred call reports success; a failure of the gathered launch
// is reported by the call that issues it.
// the shape and alignment rules of launch_gemv (a call that breaks them is
// not deferred, so its error is reported by the call itself)
bool check_gemv_args(int32_t type, const uint8_t* w, const float* x, int32_t k) {
    if (k <= 0 || k > kMaxGemvK || !type_supported(type)) return false;
    if (type != kBF16 && k % 32 != 0) return false;
    if ((type == kQ4_K || type == kQ6_K) && k % 256 != 0) return false;
    if (type == kBF16 && k % 8 != 0) return false;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), xa = reinterpret_cast<uintptr_t>(x);
    if (xa & 15u) return false;
    if (type == kQ4_K || type == kBF16) return (wa & 15u) == 0 && (row_bytes(type, k) & 15u) == 0;
    return (wa & 3u) == 0;
}

struct PendingGemv {
    int32_t count = 0, type = 0, k = 0;
    const float* x = nullptr;
    const uint8_t* w[kMaxGemvMats] = {};
    int32_t n[kMaxGemvMats] = {};
    float* y[kMaxGemvMats] = {};
};
PendingGemv g_pend;

bool flush_gemv(const char* where) {
    if (g_pend.count == 0) return true;
    const int32_t c = g_pend.count;
    g_pend.count = 0;
    return check(launch_gemv_multi(g_pend.type, c, g_pend.w, g_pend.n, g_pend.x, g_pend.k, g_pend.y, g_rt.stream),
                 where);
}

// Deferred attention prologue (lazy host buffers only).  The streamer follows
// its Q/K/V projections with heads-RMSNorm of q, heads-RMSNorm of k, RoPE of
// both and the attention step, each a call of its own on device-held q and k.
// These are recorded in that order and, when the attention step on the same q
// and k follows, run as the attention kernel's fused prologue (bit-identical
// with the separate kernels), the prologue results written back to q and k
// as the separate calls leave them.  Any other call issues the recorded ones
// as the separate kernels first.
struct PendingPrologue {
    int stage = 0;  // 1: q normalised, 2: k normalised, 4: both rotated
    float* q = nullptr;
    float* k = nullptr;
    const float* gq = nullptr;
    const float* gk = nullptr;
    int32_t nq = 0, nk = 0, hd = 0;
    float eps_q = 0.0f, eps_k = 0.0f;
    RopeTable rope{};
};
PendingPrologue g_pro;

bool flush_prologue(const char* where) {
    if (g_pro.stage == 0) return true;
    const int st = g_pro.stage;
    g_pro.stage = 0;
    if ((st & 1) && !check(launch_rmsnorm_heads(g_pro.q, g_pro.gq, g_pro.nq, g_pro.hd, g_pro.eps_q, g_rt.stream), where))
        return false;
    if ((st & 2) && !check(launch_rmsnorm_heads(g_pro.k, g_pro.gk, g_pro.nk, g_pro.hd, g_pro.eps_k, g_rt.stream), where))
        return false;
    if ((st & 4) && !check(launch_rope(g_pro.q, g_pro.k, g_pro.rope, g_pro.nq, g_pro.nk, g_pro.hd, g_rt.stream), where))
        return false;
    return true;
}

bool flush_pending(const char* where, int keep) {
    bool ok = true;
    if (keep != kKeepGemv) ok = flush_gemv(where) && ok;
    if (keep != kKeepPrologue) ok = flush_prologue(where) && ok;
    return ok;
}

bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bn && y < x + an;
}

// true when y = W x joins (or starts) the pending group instead of launching
bool defer_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y) {
    const size_t yb = sizeof(float) * static_cast<size_t>(n);
    bool joins = g_pend.count > 0 && g_pend.count < kMaxGemvMats && g_pend.type == type && g_pend.k == k &&
                 g_pend.x == x && !overlaps(y, yb, x, sizeof(float) * static_cast<size_t>(k));
    for (int32_t i = 0; joins && i < g_pend.count; ++i)
        joins = !overlaps(y, yb, g_pend.y[i], sizeof(float) * static_cast<size_t>(g_pend.n[i]));
    if (!joins) {
        if (!flush_gemv("deferred matvec")) return false;
        if (overlaps(y, yb, x, sizeof(float) * static_cast<size_t>(k))) return false;
        g_pend.type = type;
        g_pend.k = k;
        g_pend.x = x;
    }
    g_pend.w[g_pend.count] = w;
    g_pend.n[g_pend.count] = n;
    g_pend.y[g_pend.count] = y;
    ++g_pend.count;
    return true;
}

bool matvec_impl(const uint8_t* base, size_t off, int32_t type, const float* in_vec, int32_t in_dim, int32_t out_dim, float* out_vec, bool reuse_x,
                 float softcap, const char* where, bool may_defer = false) {
    if (!ensure_runtime(where)) return false;
    const size_t wbytes = row_bytes(type, in_dim) * static_cast<size_t>(out_dim);
    const uint8_t* w = device_weights(base + off, wbytes, where);
    if (!w) return false;
    const float* x;
    if (is_device_ptr(in_vec)) {
        x = in_vec;
        g_act.staged_on_device = false;
    } else if (reuse_x && g_act.staged_on_device) {
        x = g_rt.x.as<float>();
    } else {
        x = stage_in(in_vec, static_cast<size_t>(in_dim), g_rt.x, where);
        if (!x) return false;
        g_act.staged_on_device = true;
    }
    bool host_out = false;
    float* y = out_target(out_vec, static_cast<size_t>(out_dim), g_rt.y, host_out, where);
    if (!y) return false;
    if (may_defer && !host_out && softcap == 0.0f && x == in_vec && check_gemv_args(type, w, x, in_dim) &&
        defer_gemv(type, w, x, in_dim, out_dim, y))
        return true;
    if (!flush_gemv(where)) return false;
    if (!check(launch_gemv(type, w, x, in_dim, out_dim, y, g_rt.stream), where)) return false;
    if (softcap > 0.0f && !check(launch_softcap(y, out_dim, softcap, g_rt.stream), where)) return false;
    return finish_out(out_vec, y, static_cast<size_t>(out_dim), host_out, where);
}

// ---- RoPE table (cpp:1779-1796, host libm like the reference) ---------

bool rope_table(int32_t pos, int32_t head_dim, float base, const float* factors, RopeTable& t) {
    if (head_dim <= 0 || head_dim % 2 || head_dim / 2 > kMaxRopeHalf) return false;
    t.half = head_dim / 2;
    for (int32_t i = 0; i < t.half; ++i) {
        float freq = 1.0f / std::pow(base, static_cast<float>(2 * i) / static_cast<float>(head_dim));
        if (factors != nullptr && factors[i] != 0.0f) freq /= factors[i];
        const float angle = static_cast<float>(pos) * freq;
        t.c[i] = std::cos(angle);
        t.s[i] = std::sin(angle);
    }
    return true;
}

// freq factors may sit in host or device memory; the table is built on host
bool read_factors(const uint8_t* base, size_t off, int32_t half, std::array<float, kMaxRopeHalf>& f,
                  const char* where) {
    const float* src = reinterpret_cast<const float*>(base + off);
    if (is_device_ptr(src))
        return check(hipMemcpy(f.data(), src, sizeof(float) * half, hipMemcpyDeviceToHost), where);
    std::memcpy(f.data(), src, sizeof(float) * half);
    return true;
}

// ---- KV twins ----------------------------------------------------------

void forget_kv(uintptr_t key) {
    auto it = g_rt.kv.find(key);
    if (it == g_rt.kv.end()) return;
    (void)hipFree(it->second.d);
    g_rt.kv.erase(it);
}

// Device twin of a host cache with room for cap_rows rows, valid for rows
// [0, need_rows).
float* kv_twin(float* host, int32_t kv_dim, int32_t need_rows, int32_t cap_rows, const char* where) {
    const uintptr_t key = reinterpret_cast<uintptr_t>(host);
    auto it = g_rt.kv.find(key);
    if (it != g_rt.kv.end()) {
        KVTwin& t = it->second;
        bool stale = t.kv_dim != kv_dim;
        if (!stale && t.valid_rows > 0)
            stale = std::memcmp(t.row0.data(), host, sizeof(float) * std::min<int32_t>(8, kv_dim)) != 0;
        if (stale) {
            forget_kv(key);
            it = g_rt.kv.end();
        }
    }
    if (it == g_rt.kv.end()) {
        KVTwin t;
        t.kv_dim = kv_dim;
        t.cap_rows = std::max<int32_t>(cap_rows, 256);
        void* d = nullptr;
        if (!check(hipMalloc(&d, sizeof(float) * static_cast<size_t>(t.cap_rows) * kv_dim), where)) return nullptr;
        t.d = static_cast<float*>(d);
        it = g_rt.kv.emplace(key, t).first;
    }
    KVTwin& t = it->second;
    if (cap_rows > t.cap_rows) {
        const int32_t cap = std::max<int32_t>(cap_rows, t.cap_rows * 2);
        void* d = nullptr;
        if (!check(hipMalloc(&d, sizeof(float) * static_cast<size_t>(cap) * kv_dim), where)) return nullptr;
        if (t.valid_rows > 0 &&
            !check(hipMemcpyAsync(d, t.d, sizeof(float) * static_cast<size_t>(t.valid_rows) * kv_dim,
                                  hipMemcpyDeviceToDevice, g_rt.stream),
                   where))
            return nullptr;
        (void)hipStreamSynchronize(g_rt.stream);
        (void)hipFree(t.d);
        t.d = static_cast<float*>(d);
        t.cap_rows = cap;
    }
    if (t.valid_rows < need_rows) {
        const size_t r0 = static_cast<size_t>(t.valid_rows);
        const size_t nr = static_cast<size_t>(need_rows) - r0;
        if (!check(hipMemcpy(t.d + r0 * kv_dim, host + r0 * kv_dim, sizeof(float) * nr * kv_dim,
                             hipMemcpyHostToDevice),
                   where))
            return nullptr;
        t.valid_rows = need_rows;
    }
    std::memcpy(t.row0.data(), host, sizeof(float) * std::min<int32_t>(8, kv_dim));
    return t.d;
}

void kv_mark_written(float* host, int32_t row) {
    auto it = g_rt.kv.find(reinterpret_cast<uintptr_t>(host));
    if (it == g_rt.kv.end()) return;
    if (row + 1 > it->second.valid_rows) it->second.valid_rows = row + 1;
    std::memcpy(it->second.row0.data(), host, sizeof(float) * std::min<int32_t>(8, it->second.kv_dim));
}

// ---- lazily coherent host buffers ---------------------------------------
// Buffers from gncx_ram_alloc_colored / gncx_ram_alloc are host memory the
// caller reads and writes with plain loads and stores.  By default they are
// page-locked and every call that uses one copies in and out and returns
// complete, as for any host pointer.  In lazy mode (GNCX_HOST_LAZY=1 in the
// environment, or gncx_hip_set_host_coherence(1), before the buffers are
// allocated) they are ordinary pages instead, each buffer used by a call gets
// a device copy, and which copy is current follows the accesses, tracked by
// page protection:
//   kHost    the host pages are current and read-write (device copy stale);
//   kShared  both are current, the pages read-only (a host write is caught);
//   kDevice  the device copy is current, the pages inaccessible (any host
//            access is caught).
// A call that reads a buffer makes the device copy current (one upload when
// the host pages hold it) and uses it in place; a call that writes one writes
// the device copy and leaves it kDevice: no download and no wait, so a call
// whose outputs are all such buffers returns once its work is queued.  A host
// access to an inaccessible page raises SIGSEGV; the handler waits for the
// device, downloads the buffer and leaves it read-only (kShared); a host write
// to a read-only page makes it read-write (kHost).  Each buffer is a mapping
// of its own, so the protection catches nothing else.  A system call handed
// an inaccessible buffer fails with EFAULT instead of faulting:
// gncx_hip_host_flush makes buffers host-resident before such use.
enum class Home : uint8_t { kHost, kShared, kDevice };

struct HostBuffer {
    void* block = nullptr;  // what was allocated (whole pages)
    size_t block_bytes = 0;
    bool pinned = false;    // hipHostMalloc: page-locked, never protected
    uint8_t* ptr = nullptr;  // coloured start handed to the caller
    size_t bytes = 0;
    uint8_t bank = 0;
    uint8_t l1_set = 0;
    uint8_t* twin = nullptr;  // device copy (lazy buffers)
    Home home = Home::kHost;
    // read-back ahead of the host: a buffer the host read after a call wrote
    // it gets, after each later write, a copy queued into page-locked staging
    // as the writing call returns, so the host's next access only waits for
    // that copy; dropped after kReadbackMisses copies the host did not use
    bool readback = false;
    uint8_t* stage = nullptr;
    hipEvent_t staged_ev = nullptr;
    uint64_t writes = 0;      // calls that wrote the device copy
    uint64_t staged = ~0ull;  // value of writes the staged copy holds
    int misses = 0;
    bool queued = false;      // in g_readbacks
    int prot = PROT_READ | PROT_WRITE;  // current protection of the pages
    // a buffer the host rewrites after every upload (the residual stream):
    // once seen kKeepRwAfter times its pages stay read-write after an upload,
    // which costs one upload per device read instead of a fault per rewrite
    bool just_uploaded = false;
    int rewrites = 0;
    bool keep_rw = false;
    // a buffer the host reads after every device write (a projection the
    // host adds to its residual, the logits): once seen kSyncReturnAfter times
    // in a row, the writing call copies it home before it returns, with no
    // page protection and no fault; every kSyncReturnRecheck such calls the
    // fault path runs once again to see that the host still reads it
    int hits = 0;
    bool sync_return = false;
    int sync_returns = 0;
};
std::map<uintptr_t, HostBuffer*> g_bufs;  // by block address
std::vector<HostBuffer*> g_readbacks;     // written by the current call
constexpr size_t kReadbackMax = size_t{1} << 20;
constexpr int kReadbackMisses = 4;
constexpr int kKeepRwAfter = 2;
constexpr int kSyncReturnAfter = 2;
constexpr int kSyncReturnRecheck = 64;
int g_lazy = -1;                           // -1: not read from the environment yet
struct sigaction g_prev_segv;

bool lazy_mode() {
    if (g_lazy < 0) {
        const char* e = std::getenv("GNCX_HOST_LAZY");
        g_lazy = e && e[0] == '1' ? 1 : 0;
    }
    return g_lazy == 1;
}

// The buffer whose block holds address a (page-locked ones included).
HostBuffer* buffer_at(uintptr_t a) {
    auto it = g_bufs.upper_bound(a);
    if (it == g_bufs.begin()) return nullptr;
    --it;
    HostBuffer* b = it->second;
    return a < it->first + b->block_bytes ? b : nullptr;
}

// mappings from gncx_gla_map_readonly: base -> bytes
std::map<uintptr_t, size_t> g_maps;

int tracked_host_range(const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = g_maps.upper_bound(a);
    if (it != g_maps.begin()) {
        --it;
        if (a + bytes <= it->first + it->second) return kMapped;
    }
    const HostBuffer* b = buffer_at(a);
    return b && a >= reinterpret_cast<uintptr_t>(b->ptr) && a + bytes <= reinterpret_cast<uintptr_t>(b->ptr) + b->bytes
               ? kRamBuffer
               : kUntracked;
}

size_t page_bytes() {
    static const size_t pg = static_cast<size_t>(sysconf(_SC_PAGESIZE));
    return pg;
}

bool protect(HostBuffer& b, int prot) {
    if (b.prot == prot) return true;
    const uintptr_t pg = page_bytes();
    const uintptr_t lo = reinterpret_cast<uintptr_t>(b.ptr) & ~(pg - 1);
    const uintptr_t hi = (reinterpret_cast<uintptr_t>(b.ptr) + b.bytes + pg - 1) & ~(pg - 1);
    if (mprotect(reinterpret_cast<void*>(lo), hi - lo, prot) != 0) return false;
    b.prot = prot;
    return true;
}

// device copy -> host pages (made read-write first); waits for queued work
bool download(HostBuffer& b, const char* where) {
    if (!protect(b, PROT_READ | PROT_WRITE)) {
        set_error(where, "mprotect failed on a lazy host buffer", -1);
        return false;
    }
    if (!check(hipStreamSynchronize(g_rt.stream), where)) return false;
    return check(hipMemcpy(b.ptr, b.twin, b.bytes, hipMemcpyDeviceToHost), where);
}

// host pages -> device copy, ordered after the work already queued
bool upload(HostBuffer& b, const char* where) {
    if (b.bytes <= kPinnedMax) return h2d(b.twin, b.ptr, b.bytes, where);
    if (!check(hipStreamSynchronize(g_rt.stream), where)) return false;
    return check(hipMemcpy(b.twin, b.ptr, b.bytes, hipMemcpyHostToDevice), where);
}

// Bring a lazy buffer back to the host: current and read-write.
bool make_host(HostBuffer& b, const char* where) {
    if (b.home == Home::kHost) return true;
    if (b.home == Home::kDevice ? !download(b, where) : !protect(b, PROT_READ | PROT_WRITE)) return false;
    b.home = Home::kHost;
    return true;
}

void on_segv(int sig, siginfo_t* si, void* uc);

// Host faults on lazy buffers are resolved off the signal path.  The SIGSEGV
// handler only does async-signal-safe work: it writes a pointer to a request
// on its own stack into a pipe and sleeps on a futex in that request.  A
// resolver thread reads the request, takes the call lock like any library
// call, makes the buffer's pages current (which may wait on the device, copy
// and change protections), and wakes the faulting thread, which then retries
// its access or, for a fault that is not a lazy buffer's, chains to the
// handler installed before.  So the faulting thread may hold a lock that the
// resolver never takes (a stdio FILE lock, the caller's own locks) when it
// faults.  The resolver does call the HIP runtime (event and stream waits,
// copies), so a lazy buffer handed straight to a HIP API (a copy from it, for
// instance) can deadlock: such use is not supported.  Only a fault taken by
// the library itself while it holds the call lock is resolved in the handler,
// as the resolver could never get that lock, and then without issuing any
// recorded work; the library touches lazy buffers' host pages only through
// their device copies, so that case is not expected.  A fork() child inherits
// the handler but not the resolver thread: its faults go straight to the
// handler installed before.
struct FaultRequest {
    uintptr_t addr;
    int write;
    std::atomic<int> done;  // 0 while the resolver works, then 1
    int handled;
};
int g_fault_pipe[2] = {-1, -1};
pid_t g_fault_pid = 0;  // the process whose resolver thread reads the pipe
ssize_t write_fd(int fd, const void* p, size_t n) { return ::write(fd, p, n); }

bool resolve_fault(uintptr_t a, bool write, bool may_issue);

void fault_resolver() {
    for (;;) {
        FaultRequest* r = nullptr;
        const ssize_t got = read(g_fault_pipe[0], &r, sizeof(r));
        if (got != static_cast<ssize_t>(sizeof(r))) {
            if (got < 0 && errno == EINTR) continue;
            return;
        }
        bool handled;
        {
            std::lock_guard<CallLock> lk(g_mu);
            handled = resolve_fault(r->addr, r->write != 0, true);
        }
        r->handled = handled ? 1 : 0;
        r->done.store(1, std::memory_order_release);
        syscall(SYS_futex, reinterpret_cast<int*>(&r->done), FUTEX_WAKE_PRIVATE, 1, nullptr, nullptr, 0);
    }
}

void ensure_segv_handler() {
    if (g_fault_pipe[0] < 0) {
        if (pipe2(g_fault_pipe, O_CLOEXEC) != 0) {
            g_fault_pipe[0] = g_fault_pipe[1] = -1;
            return;  // no resolver: lazy_ptr reports the failure
        }
        g_fault_pid = getpid();
        std::thread(fault_resolver).detach();
    }
    struct sigaction cur;
    sigaction(SIGSEGV, nullptr, &cur);
    if ((cur.sa_flags & SA_SIGINFO) && cur.sa_sigaction == on_segv) return;
    struct sigaction sa;
    std::memset(&sa, 0, sizeof(sa));
    sa.sa_sigaction = on_segv;
    sa.sa_flags = SA_SIGINFO | SA_RESTART;
    sigemptyset(&sa.sa_mask);
    sigaction(SIGSEGV, &sa, &g_prev_segv);
}

// A host access to a lazy buffer's protected page (with the call lock
// held): make the host copy current and read-only, or read-write for a write
// to a read-only page.  False when the address is not a protected page of a
// lazy buffer.  The address is classified first; recorded work (deferred
// matvecs, an attention prologue) is issued only for a lazy buffer's page and
// only when may_issue (the resolver thread, never the signal handler).
bool resolve_fault(uintptr_t a, bool write, bool may_issue) {
    HostBuffer* b = buffer_at(a);
    if (!b || b->pinned || !b->twin || b->home == Home::kHost) return false;
    const uintptr_t pg = page_bytes();
    const uintptr_t lo = reinterpret_cast<uintptr_t>(b->ptr) & ~(pg - 1);
    const uintptr_t hi = (reinterpret_cast<uintptr_t>(b->ptr) + b->bytes + pg - 1) & ~(pg - 1);
    if (a < lo || a >= hi) return false;
    const char* where = "lazy host buffer access";
    if (may_issue) (void)flush_pending(where);
    if (b->home == Home::kDevice && b->stage && b->staged == b->writes) {
        // the copy queued when the last writer returned
        if (check(hipEventSynchronize(b->staged_ev), where) && protect(*b, PROT_READ | PROT_WRITE)) {
            std::memcpy(b->ptr, b->stage, b->bytes);
            b->misses = 0;
            b->staged = ~0ull;
            b->home = protect(*b, PROT_READ) ? Home::kShared : Home::kHost;
            b->just_uploaded = false;
            if (++b->hits >= kSyncReturnAfter) b->sync_return = true;
            return true;
        }
    }
    if (b->home == Home::kDevice) {
        if (b->bytes <= kReadbackMax) b->readback = true;
        if (!download(*b, where)) {
            (void)protect(*b, PROT_READ | PROT_WRITE);  // the data is lost; keep the program running
            b->home = Home::kHost;
        } else if (protect(*b, PROT_READ)) {
            b->home = Home::kShared;
        } else {
            b->home = Home::kHost;
        }
        return true;
    }
    if (!write) return true;  // a read that faulted before another thread made the pages readable
    if (!protect(*b, PROT_READ | PROT_WRITE)) return false;
    b->home = Home::kHost;
    if (b->just_uploaded && ++b->rewrites >= kKeepRwAfter) b->keep_rw = true;
    b->just_uploaded = false;
    return true;
}

void on_segv(int sig, siginfo_t* si, void* uc) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(si->si_addr);
    // x86-64 page-fault error code: bit 1 set for a write
    const bool write = (static_cast<ucontext_t*>(uc)->uc_mcontext.gregs[REG_ERR] & 2) != 0;
    bool handled = false;
    if (g_fault_pid != 0 && getpid() != g_fault_pid) {
        // a fork() child: no resolver reads the pipe here, and the parent's
        // resolver would act on the parent's memory
    } else if (t_in_call) {
        handled = resolve_fault(a, write, false);  // the library itself holds the call lock
    } else if (g_fault_pipe[1] >= 0) {
        const int saved_errno = errno;
        FaultRequest req;
        req.addr = a;
        req.write = write ? 1 : 0;
        req.done.store(0, std::memory_order_relaxed);
        req.handled = 0;
        FaultRequest* rp = &req;
        ssize_t put;
        do {
            put = write_fd(g_fault_pipe[1], &rp, sizeof(rp));
        } while (put < 0 && errno == EINTR);
        if (put == static_cast<ssize_t>(sizeof(rp))) {
            while (req.done.load(std::memory_order_acquire) == 0)
                syscall(SYS_futex, reinterpret_cast<int*>(&req.done), FUTEX_WAIT_PRIVATE, 0, nullptr, nullptr, 0);
            handled = req.handled != 0;
        }
        errno = saved_errno;
    }
    if (handled) return;
    if (g_prev_segv.sa_flags & SA_SIGINFO) {
        if (g_prev_segv.sa_sigaction) g_prev_segv.sa_sigaction(sig, si, uc);
        return;
    }
    if (g_prev_segv.sa_handler == SIG_DFL || g_prev_segv.sa_handler == SIG_IGN) {
        signal(SIGSEGV, SIG_DFL);  // the access runs again and takes the default action
        return;
    }
    g_prev_segv.sa_handler(sig);
}

// A sync-return buffer the call wrote: its copy home, made before the call
// returns.  False (buffer left device-owned and inaccessible, the fault path
// takes over) when a step fails.
bool sync_return(HostBuffer& b, const char* where) {
    if (!b.stage) {
        void* p = nullptr;
        if (hipHostMalloc(&p, b.bytes, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        b.stage = static_cast<uint8_t*>(p);
    }
    if (!check(hipMemcpyAsync(b.stage, b.twin, b.bytes, hipMemcpyDeviceToHost, g_rt.stream), where) ||
        !check(hipStreamSynchronize(g_rt.stream), where) || !protect(b, PROT_READ | PROT_WRITE))
        return false;
    std::memcpy(b.ptr, b.stage, b.bytes);
    b.home = Home::kHost;
    b.staged = ~0ull;
    return true;
}

void queue_readbacks() {
    if (g_readbacks.empty()) return;
    for (HostBuffer* b : g_readbacks) {
        b->queued = false;
        if (b->home != Home::kDevice || !b->readback) continue;
        if (b->sync_return) {
            const bool recheck = ++b->sync_returns % kSyncReturnRecheck == 0;
            if (!recheck && sync_return(*b, "lazy host buffer copy home")) continue;
            // the fault path once more: the host must still read it to come back here
            b->sync_return = false;
            b->hits = 0;
            if (!protect(*b, PROT_NONE)) {
                (void)make_host(*b, "lazy host buffer copy home");  // the host copy, current
                continue;
            }
        }
        if (b->staged != ~0ull && ++b->misses >= kReadbackMisses) {  // the host left the last copy unread
            b->readback = false;
            continue;
        }
        const char* where = "lazy host buffer read-back";
        if (!b->stage) {
            void* p = nullptr;
            if (hipHostMalloc(&p, b->bytes, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                b->readback = false;
                continue;
            }
            b->stage = static_cast<uint8_t*>(p);
            if (!check(hipEventCreateWithFlags(&b->staged_ev, hipEventDisableTiming), where)) {
                b->readback = false;
                continue;
            }
        }
        if (check(hipMemcpyAsync(b->stage, b->twin, b->bytes, hipMemcpyDeviceToHost, g_rt.stream), where) &&
            check(hipEventRecord(b->staged_ev, g_rt.stream), where))
            b->staged = b->writes;
    }
    g_readbacks.clear();
}

// a lazy buffer whose data only the device reads back (no host read-back
// pattern seen): a write to it may be deferred
bool device_only_lazy(const void* p) {
    if (g_lazy != 1 || !p) return false;
    const HostBuffer* b = buffer_at(reinterpret_cast<uintptr_t>(p));
    return b && !b->pinned && !b->readback && !b->sync_return;
}

// [p, p + bytes) inside a lazy buffer: its address in the device copy, after
// making that copy current (read) and taking ownership for the device
// (write).  Any other pointer comes back unchanged.  A range that leaves its
// buffer makes the buffer host-resident and is used as host memory.
// kRdPinned: a read by a call that waits for its kernels before it returns;
// a host-owned buffer the host rewrites after every call is then read by the
// kernels from a page-locked copy in place (no upload into the device copy,
// which stays stale while the host owns the buffer).
constexpr int kRd = 1, kWr = 2, kRdPinned = 4;
template <class T>
T* lazy_ptr(T* p, size_t count, int access, bool& ok, const char* where) {
    if (!p || !ok || g_lazy != 1) return p;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    HostBuffer* b = buffer_at(a);
    if (!b || b->pinned) return p;
    const size_t bytes = count * sizeof(T);
    const uintptr_t lo = reinterpret_cast<uintptr_t>(b->ptr);
    if (a < lo || a + bytes > lo + b->bytes) {
        ok = make_host(*b, where);
        return p;
    }
    if (!b->twin) {
        void* d = nullptr;
        if (!ensure_runtime(where) || !check(hipMalloc(&d, round_up(b->bytes, 256) + 256), where)) {
            ok = false;
            return nullptr;
        }
        b->twin = static_cast<uint8_t*>(d);
        b->home = Home::kHost;  // the pages hold the data
    }
    ensure_segv_handler();
    if (g_fault_pipe[1] < 0) {
        set_error(where, "the lazy host buffers' fault resolver could not start", -1);
        ok = false;
        return nullptr;
    }
    // a sync-return buffer that the call overwrites whole is not uploaded
    // first (its next copy home replaces the pages anyway)
    const bool whole_output = access == kWr && b->sync_return && a == lo && bytes == b->bytes;
    if ((access & kRdPinned) && !(access & kWr) && b->home == Home::kHost && b->keep_rw &&
        bytes <= kPinnedMax && g_ndirect < static_cast<int>(g_direct.size())) {
        PinnedSlot* sl = pinned_slot(bytes, where);
        if (!sl) {
            ok = false;
            return nullptr;
        }
        std::memcpy(sl->p, p, bytes);
        // the call's kernel reads the slot: a reuse before the next wait for
        // the stream waits for it first (as for a slot holding device output)
        sl->deferred = true;
        g_direct[g_ndirect++] = sl->p;
        return static_cast<T*>(sl->p);
    }
    if (b->home == Home::kHost && !whole_output) {
        // uploaded for writes too: a call that writes nothing keeps the data
        if (!upload(*b, where)) {
            ok = false;
            return nullptr;
        }
        if (b->keep_rw && !(access & kWr)) {
            // pages stay read-write and the buffer host-owned: the next
            // device read uploads again, a host rewrite costs nothing
        } else {
            if (!protect(*b, PROT_READ)) {
                set_error(where, "mprotect failed on a lazy host buffer", -1);
                ok = false;
                return nullptr;
            }
            b->home = Home::kShared;
            b->just_uploaded = true;
        }
    }
    if ((access & kWr) && b->home != Home::kDevice) {
        // a sync-return buffer keeps its pages as they are: the writing call
        // copies it home before it returns (queue_readbacks)
        if (!b->sync_return && !protect(*b, PROT_NONE)) {
            set_error(where, "mprotect failed on a lazy host buffer", -1);
            ok = false;
            return nullptr;
        }
        b->home = Home::kDevice;
        b->just_uploaded = false;
    }
    if (access & kWr) {
        ++b->writes;
        if (b->readback && !b->queued) {
            b->queued = true;
            g_readbacks.push_back(b);
        }
    }
    return reinterpret_cast<T*>(b->twin + (a - lo));
}

struct AttnCall {
    const float* q;
    const float* k;
    const float* v;
    float* kc;
    float* vc;
    int32_t pos, n_heads, n_kv, hd;
    float scale;
    int32_t sw, write_kv;
    float* out;
    // fused prologue
    int32_t norm_qk = 0;
    const float* q_gamma = nullptr;
    const float* k_gamma = nullptr;
    float eps = 0.0f;
    const RopeTable* rope = nullptr;
    float* q_back = nullptr;  // host/device q to receive the prologue result
    float* k_back = nullptr;
};

bool attention_impl(const AttnCall& c, const char* where) {
    if (!ensure_runtime(where)) return false;
    if (c.n_heads <= 0 || c.n_kv <= 0 || c.hd <= 0 || c.pos < 0 || c.n_heads % c.n_kv != 0) {
        set_error(where, "invalid head geometry or position", -1);
        return false;
    }
    const int32_t kv_dim = c.n_kv * c.hd;
    const bool use_new = c.write_kv && c.k && c.v;
    const size_t qn = static_cast<size_t>(c.n_heads) * c.hd;
    const float* q = stage_in(c.q, qn, g_rt.q, where);
    if (!q) return false;
    const float* kn = use_new ? stage_in(c.k, kv_dim, g_rt.k, where) : nullptr;
    const float* vn = use_new ? stage_in(c.v, kv_dim, g_rt.v, where) : nullptr;
    if (use_new && (!kn || !vn)) return false;

    const bool host_k = !is_device_ptr(c.kc), host_v = !is_device_ptr(c.vc);
    // rows needed on device: [0, pos) always, row pos too when it is not written here
    const int32_t need = use_new ? c.pos : c.pos + 1;
    float* kc = host_k ? kv_twin(c.kc, kv_dim, need, c.pos + 1, where) : c.kc;
    if (!kc) return false;
    float* vc = host_v ? kv_twin(c.vc, kv_dim, need, c.pos + 1, where) : c.vc;
    if (!vc) return false;

    bool host_out = false;
    float* out = out_target(c.out, qn, g_rt.o, host_out, where);
    if (!out) return false;
    const int32_t t0 = c.sw > 0 ? std::max(0, c.pos - c.sw + 1) : 0;
    const size_t wsb = attention_workspace_bytes(c.n_heads, c.hd, c.pos + 1 - t0);
    if (!g_rt.ws.ensure(wsb, where)) return false;

    AttnArgs a{};
    a.q = q;
    a.k_new = kn;
    a.v_new = vn;
    a.k_cache = kc;
    a.v_cache = vc;
    a.out = out;
    a.pos = c.pos;
    a.n_heads = c.n_heads;
    a.n_kv_heads = c.n_kv;
    a.head_dim = c.hd;
    a.scale = c.scale;
    a.sliding_window = c.sw;
    a.write_kv = c.write_kv;
    a.norm_qk = c.norm_qk;
    a.q_gamma = c.q_gamma;
    a.k_gamma = c.k_gamma;
    a.eps = c.eps;
    a.rope = c.rope;
    // prologue results: device targets (host ones are copied back below)
    float* qb = nullptr;
    float* kb = nullptr;
    if (c.q_back) qb = is_device_ptr(c.q_back) ? c.q_back : g_rt.aux.ensure(sizeof(float) * (qn + kv_dim), where) ? g_rt.aux.as<float>() : nullptr;
    if (c.k_back && use_new) kb = is_device_ptr(c.k_back) ? c.k_back : g_rt.aux.ensure(sizeof(float) * (qn + kv_dim), where) ? g_rt.aux.as<float>() + qn : nullptr;
    a.q_out = qb;
    a.k_out = kb;
    if (!check(launch_attention(a, g_rt.ws.p, g_rt.ws.cap, g_rt.stream), where)) return false;

    if (use_new) {
        // the reference writes the host cache row inside the call (cpp:1903-1906)
        if (host_k) {
            if (c.norm_qk || c.rope) {
                // the stored row is the prologue result: take it from the twin
                if (!d2h(c.kc + static_cast<size_t>(c.pos) * kv_dim, kc + static_cast<size_t>(c.pos) * kv_dim,
                         sizeof(float) * kv_dim, where))
                    return false;
            } else if (!is_device_ptr(c.k)) {
                std::memcpy(c.kc + static_cast<size_t>(c.pos) * kv_dim, c.k, sizeof(float) * kv_dim);
            } else if (!d2h(c.kc + static_cast<size_t>(c.pos) * kv_dim, c.k, sizeof(float) * kv_dim, where)) {
                return false;
            }
        }
        if (host_v) {
            if (!is_device_ptr(c.v))
                std::memcpy(c.vc + static_cast<size_t>(c.pos) * kv_dim, c.v, sizeof(float) * kv_dim);
            else if (!d2h(c.vc + static_cast<size_t>(c.pos) * kv_dim, c.v, sizeof(float) * kv_dim, where))
                return false;
        }
    }
    if (c.q_back && qb && !is_device_ptr(c.q_back))
        if (!d2h(c.q_back, qb, sizeof(float) * qn, where)) return false;
    if (c.k_back && kb && !is_device_ptr(c.k_back))
        if (!d2h(c.k_back, kb, sizeof(float) * kv_dim, where)) return false;
    const bool any_host = host_out || host_k || host_v || (c.q_back && !is_device_ptr(c.q_back)) ||
                          (c.k_back && !is_device_ptr(c.k_back));
    if (host_out && !d2h(c.out, out, sizeof(float) * qn, where)) return false;
    if (any_host && !sync_out(where)) return false;
    if (use_new) {
        if (host_k) kv_mark_written(c.kc, c.pos);
        if (host_v) kv_mark_written(c.vc, c.pos);
    }
    return true;
}

}  // namespace

// =======================================================================
// Reference C-ABI (names and signatures of csrc/gncx_llm_kernels.cpp)
// =======================================================================

// cpp:1327-1471
GNCX_API void gncx_xfold_universal_matvec(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                          const float* in_vec, const GNCXCompactToken* in_tokens, int32_t in_dim,
                                          int32_t out_dim, float* out_vec, GNCXTelemetryStats* telemetry) {
    t_keep = kKeepGemv;
    std::lock_guard<CallLock> lk(g_mu);
    t_keep = kKeepNone;
    bool ok = true;
    // an output only the device reads may wait in the pending group
    const bool may_defer = device_only_lazy(out_vec);
    in_vec = lazy_ptr(in_vec, dim_count(in_dim), kRd, ok, "gncx_xfold_universal_matvec");
    out_vec = lazy_ptr(out_vec, dim_count(out_dim), kWr, ok, "gncx_xfold_universal_matvec");
    if (!ok) return;
    uint64_t canceled = 0;
    bool reuse = false;
    if (in_tokens != nullptr && in_vec == g_act.last_in && in_dim == g_act.last_dim &&
        g_norm_epoch == g_act.last_epoch) {
        canceled = g_act.cached_canceled;
        reuse = true;
    } else {
        canceled = count_cancellations(in_tokens, in_dim);
        if (in_tokens != nullptr) {
            g_act.last_in = in_vec;
            g_act.last_dim = in_dim;
            g_act.last_epoch = g_norm_epoch;
            g_act.cached_canceled = canceled;
        } else {
            g_act.last_in = nullptr;
        }
    }
    if (type_supported(ggml_type) && out_dim > 0 && in_dim > 0)
        matvec_impl(mmap_base, weight_abs_offset, ggml_type, in_vec, in_dim, out_dim, out_vec, reuse,
                    0.0f, "gncx_xfold_universal_matvec", may_defer);
    const uint64_t macs = static_cast<uint64_t>(in_dim) * static_cast<uint64_t>(out_dim);
    add_telemetry(telemetry, macs, canceled, static_cast<uint64_t>(in_dim / 32) * static_cast<uint64_t>(out_dim));
}

// cpp:1476-1489
GNCX_API void gncx_xfold_q4_0_matvec(const uint8_t* mmap_base, size_t weight_abs_offset, const float* in_vec,
                                     const GNCXCompactToken* in_tokens, int32_t in_dim, int32_t out_dim,
                                     float* out_vec, GNCXTelemetryStats* telemetry) {
    gncx_xfold_universal_matvec(mmap_base, weight_abs_offset, kQ4_0, in_vec, in_tokens, in_dim, out_dim, out_vec,
                                telemetry);
}

// cpp:1495-1692
GNCX_API void gncx_xfold_universal_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                            const float* in_batch, int32_t batch_size, int32_t in_dim,
                                            int32_t out_dim, float* out_batch, GNCXTelemetryStats* telemetry) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_xfold_universal_matbatch";
    bool ok = true;
    in_batch = lazy_ptr(in_batch, dim_count(batch_size) * dim_count(in_dim), kRd, ok, where);
    out_batch = lazy_ptr(out_batch, dim_count(batch_size) * dim_count(out_dim), kWr, ok, where);
    if (!ok) return;
    if (type_supported(ggml_type) && batch_size > 0 && out_dim > 0 && in_dim > 0 && ensure_runtime(where)) {
        do {
            const size_t wbytes = row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dim);
            const uint8_t* w = device_weights(mmap_base + weight_abs_offset, wbytes, where);
            if (!w) break;
            const size_t xn = static_cast<size_t>(batch_size) * in_dim;
            const size_t yn = static_cast<size_t>(batch_size) * out_dim;
            const float* x = stage_in(in_batch, xn, g_rt.aux, where);
            if (!x) break;
            bool host_out = false;
            float* y = out_target(out_batch, yn, g_rt.y, host_out, where);
            if (!y) break;
            const size_t wsb = matbatch_workspace_bytes(ggml_type, batch_size, in_dim, out_dim);
            if (!g_rt.ws.ensure(wsb, where)) break;
            if (!check(launch_matbatch(ggml_type, w, x, batch_size, in_dim, out_dim, y, g_rt.ws.p, g_rt.ws.cap,
                                       g_rt.stream),
                       where))
                break;
            finish_out(out_batch, y, yn, host_out, where);
        } while (false);
    }
    const uint64_t macs = static_cast<uint64_t>(batch_size) * static_cast<uint64_t>(in_dim) *
                          static_cast<uint64_t>(out_dim);
    if (telemetry) {
        telemetry->total_macs_equivalent += macs;
        telemetry->zero_weight_skips += macs / 15;
        telemetry->xfold_bucket_merges += static_cast<uint64_t>(batch_size) * static_cast<uint64_t>(in_dim / 32) *
                                          static_cast<uint64_t>(out_dim);
    }
}

// gncx_swiglu_activation of the batch's gate and up rows followed by
// gncx_xfold_universal_matbatch of the result, with the SwiGLU formed by the
// matbatch's own activation pass (the prefill's down projection without the
// activation rows in memory).  The same values as the two calls.
GNCX_API void gncx_hip_swiglu_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                       const float* gate_batch, const float* up_batch, int32_t batch_size,
                                       int32_t in_dim, int32_t out_dim, float* out_batch) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_swiglu_matbatch";
    bool ok = true;
    const size_t xn = dim_count(batch_size) * dim_count(in_dim);
    gate_batch = lazy_ptr(gate_batch, xn, kRd, ok, where);
    up_batch = lazy_ptr(up_batch, xn, kRd, ok, where);
    out_batch = lazy_ptr(out_batch, dim_count(batch_size) * dim_count(out_dim), kWr, ok, where);
    if (!ok) return;
    if (!gate_batch || !up_batch || !out_batch || !type_supported(ggml_type) || batch_size <= 0 || out_dim <= 0 ||
        in_dim <= 0 || !ensure_runtime(where))
        return;
    const size_t wbytes = row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dim);
    const uint8_t* w = device_weights(mmap_base + weight_abs_offset, wbytes, where);
    if (!w) return;
    const float* g = stage_in(gate_batch, xn, g_rt.aux, where);
    if (!g) return;
    const float* u = stage_in(up_batch, xn, g_rt.x, where);
    if (!u) return;
    const size_t yn = static_cast<size_t>(batch_size) * out_dim;
    bool host_out = false;
    float* y = out_target(out_batch, yn, g_rt.y, host_out, where);
    if (!y) return;
    if (!g_rt.ws.ensure(matbatch_workspace_bytes(ggml_type, batch_size, in_dim, out_dim), where)) return;
    hipError_t e = launch_matbatch(ggml_type, w, g, batch_size, in_dim, out_dim, y, g_rt.ws.p, g_rt.ws.cap,
                                   g_rt.stream, u);
    if (e == hipErrorNotSupported) {
        // BF16 weights take fp32 activations: the SwiGLU rows are formed first
        if (!g_rt.v.ensure(xn * sizeof(float), where)) return;
        float* act = g_rt.v.as<float>();
        if (!check(launch_swiglu(g, u, static_cast<int32_t>(xn), act, g_rt.stream), where)) return;
        e = launch_matbatch(ggml_type, w, act, batch_size, in_dim, out_dim, y, g_rt.ws.p, g_rt.ws.cap, g_rt.stream);
    }
    if (!check(e, where)) return;
    finish_out(out_batch, y, yn, host_out, where);
}

// cpp:1694-1707
GNCX_API void gncx_xfold_q4_0_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, const float* in_batch,
                                       int32_t batch_size, int32_t in_dim, int32_t out_dim, float* out_batch,
                                       GNCXTelemetryStats* telemetry) {
    gncx_xfold_universal_matbatch(mmap_base, weight_abs_offset, kQ4_0, in_batch, batch_size, in_dim, out_dim,
                                  out_batch, telemetry);
}

// Several matrices of one type and in_dim applied to the same batch: the
// batch is quantised once, and Q4_K matrices that are whole tiles of one
// plan go through one launch.
GNCX_API void gncx_hip_matbatch_multi(int32_t count, const uint8_t* const* weights, const int32_t* out_dims,
                                      int32_t ggml_type, const float* in_batch, int32_t batch_size, int32_t in_dim,
                                      float* const* out_arg) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_matbatch_multi";
    if (count <= 0 || count > 4 || !weights || !out_dims || !out_arg || !in_batch || in_dim <= 0 ||
        batch_size <= 0) {
        set_error(where, "count must be 1..4, with weights, out_dims, in_batch and out_batches given", -1);
        return;
    }
    if (!type_supported(ggml_type) || !ensure_runtime(where)) return;
    bool ok = true;
    float* outs[4];
    in_batch = lazy_ptr(in_batch, dim_count(batch_size) * dim_count(in_dim), kRd, ok, where);
    for (int32_t i = 0; i < count; ++i)
        outs[i] = lazy_ptr(out_arg[i], dim_count(batch_size) * dim_count(out_dims[i]), kWr, ok, where);
    if (!ok) return;
    const uint8_t* ws[4];
    float* ys[4];
    bool host[4];
    size_t host_total = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (out_dims[i] <= 0 || !weights[i] || !outs[i]) {
            set_error(where, "every matrix needs weights, out_dims > 0 and an output", -1);
            return;
        }
        ws[i] = device_weights(weights[i], row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dims[i]), where);
        if (!ws[i]) return;
        host[i] = !is_device_ptr(outs[i]);
        if (host[i]) host_total += static_cast<size_t>(batch_size) * static_cast<size_t>(out_dims[i]);
    }
    const float* x = stage_in(in_batch, static_cast<size_t>(batch_size) * in_dim, g_rt.aux, where);
    if (!x) return;
    if (host_total && !g_rt.y.ensure(sizeof(float) * host_total, where)) return;
    size_t off = 0;
    for (int32_t i = 0; i < count; ++i) {
        ys[i] = host[i] ? g_rt.y.as<float>() + off : outs[i];
        if (host[i]) off += static_cast<size_t>(batch_size) * static_cast<size_t>(out_dims[i]);
    }
    const size_t wsb = matbatch_multi_workspace_bytes(ggml_type, count, out_dims, batch_size, in_dim);
    if (!g_rt.ws.ensure(wsb, where)) return;
    if (!check(launch_matbatch_multi(ggml_type, count, ws, out_dims, x, batch_size, in_dim, ys, g_rt.ws.p,
                                     g_rt.ws.cap, g_rt.stream),
               where))
        return;
    for (int32_t i = 0; i < count; ++i)
        if (host[i] &&
            !finish_out(outs[i], ys[i], static_cast<size_t>(batch_size) * static_cast<size_t>(out_dims[i]), true,
                        where))
            return;
}

// cpp:1713-1732
GNCX_API void gncx_universal_lm_head_logits(const uint8_t* mmap_base, size_t embd_abs_offset, int32_t ggml_type,
                                            const float* final_hidden, int32_t embed_dim, int32_t vocab_size,
                                            float softcap, float* out_logits) {
    std::lock_guard<CallLock> lk(g_mu);
    bool ok = true;
    final_hidden = lazy_ptr(final_hidden, dim_count(embed_dim), kRd, ok, "gncx_universal_lm_head_logits");
    out_logits = lazy_ptr(out_logits, dim_count(vocab_size), kWr, ok, "gncx_universal_lm_head_logits");
    if (!ok) return;
    g_act.last_in = nullptr;  // the inner matvec is called with in_tokens == NULL
    if (type_supported(ggml_type) && vocab_size > 0 && embed_dim > 0)
        matvec_impl(mmap_base, embd_abs_offset, ggml_type, final_hidden, embed_dim, vocab_size, out_logits,
                    false, softcap, "gncx_universal_lm_head_logits");
}

// cpp:1734-1745
GNCX_API void gncx_q8_0_lm_head_logits(const uint8_t* mmap_base, size_t embd_abs_offset, const float* final_hidden,
                                       int32_t embed_dim, int32_t vocab_size, float* out_logits) {
    gncx_universal_lm_head_logits(mmap_base, embd_abs_offset, kQ8_0, final_hidden, embed_dim, vocab_size, 0.0f,
                                  out_logits);
}

// cpp:1887-1994
GNCX_API void gncx_mqa_attention_step_ext(const float* q_vec, const float* k_vec, const float* v_vec,
                                          float* k_cache_layer, float* v_cache_layer, int32_t pos, int32_t n_heads,
                                          int32_t n_kv_heads, int32_t head_dim, float attn_scale,
                                          int32_t sliding_window, int32_t write_kv, float* out_attn_vec) {
    t_keep = kKeepPrologue;
    std::lock_guard<CallLock> lk(g_mu);
    t_keep = kKeepNone;
    const char* where = "gncx_mqa_attention_step_ext";
    bool ok = true;
    const size_t qn = dim_count(n_heads) * dim_count(head_dim), kvn = dim_count(n_kv_heads) * dim_count(head_dim);
    const int cache_access = write_kv && k_vec && v_vec ? kRd | kWr : kRd;
    q_vec = lazy_ptr(q_vec, qn, kRd, ok, where);
    k_vec = lazy_ptr(k_vec, kvn, kRd, ok, where);
    v_vec = lazy_ptr(v_vec, kvn, kRd, ok, where);
    k_cache_layer = lazy_ptr(k_cache_layer, (dim_count(pos) + 1) * kvn, cache_access, ok, where);
    v_cache_layer = lazy_ptr(v_cache_layer, (dim_count(pos) + 1) * kvn, cache_access, ok, where);
    out_attn_vec = lazy_ptr(out_attn_vec, qn, kWr, ok, where);
    if (!ok) {
        (void)flush_prologue(where);
        return;
    }
    AttnCall c{q_vec, k_vec, v_vec, k_cache_layer, v_cache_layer, pos, n_heads, n_kv_heads, head_dim, attn_scale,
               sliding_window, write_kv, out_attn_vec};
    // the recorded prologue of this q and k runs inside the attention kernel
    const int st = g_pro.stage;
    if ((st == 3 || st == 4 || st == 7) && const_cast<float*>(q_vec) == g_pro.q && const_cast<float*>(k_vec) == g_pro.k &&
        n_heads == g_pro.nq && n_kv_heads == g_pro.nk && head_dim == g_pro.hd && write_kv && v_vec &&
        (!(st & 3) || g_pro.eps_q == g_pro.eps_k)) {
        g_pro.stage = 0;
        c.norm_qk = (st & 3) ? 1 : 0;
        c.q_gamma = (st & 3) ? g_pro.gq : nullptr;
        c.k_gamma = (st & 3) ? g_pro.gk : nullptr;
        c.eps = g_pro.eps_q;
        c.rope = (st & 4) ? &g_pro.rope : nullptr;
        c.q_back = g_pro.q;  // the prologue results, as the separate calls leave q and k
        c.k_back = g_pro.k;
        attention_impl(c, where);
        return;
    }
    if (!flush_prologue(where)) return;
    attention_impl(c, where);
}

// cpp:1996-2013
GNCX_API void gncx_mqa_attention_step(const float* q_vec, const float* k_vec, const float* v_vec,
                                      float* k_cache_layer, float* v_cache_layer, int32_t pos, int32_t n_heads,
                                      int32_t n_kv_heads, int32_t head_dim, float* out_attn_vec) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    gncx_mqa_attention_step_ext(q_vec, k_vec, v_vec, k_cache_layer, v_cache_layer, pos, n_heads, n_kv_heads,
                                head_dim, scale, 0, 1, out_attn_vec);
}

// cpp:895-953
GNCX_API void gncx_rmsnorm_inplace_heads(float* vec, const uint8_t* mmap_base, size_t norm_weight_offset,
                                         int32_t has_weight, int32_t n_heads, int32_t head_dim, float eps) {
    t_keep = kKeepPrologue;
    std::lock_guard<CallLock> lk(g_mu);
    t_keep = kKeepNone;
    const char* where = "gncx_rmsnorm_inplace_heads";
    if (n_heads <= 0 || head_dim <= 0 || !ensure_runtime(where)) {
        (void)flush_prologue(where);
        return;
    }
    const float* g = nullptr;
    if (has_weight) {
        g = reinterpret_cast<const float*>(
            device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(head_dim), where));
        if (!g) {
            (void)flush_prologue(where);
            return;
        }
    }
    const size_t n = static_cast<size_t>(n_heads) * head_dim;
    bool ok = true;
    const bool may_defer = device_only_lazy(vec) && head_dim <= 2 * kMaxRopeHalf;
    vec = lazy_ptr(vec, n, kRd | kWr, ok, where);
    if (!ok) {
        (void)flush_prologue(where);
        return;
    }
    if (may_defer && is_device_ptr(vec)) {
        if (g_pro.stage == 0) {
            g_pro.q = vec;
            g_pro.gq = g;
            g_pro.nq = n_heads;
            g_pro.hd = head_dim;
            g_pro.eps_q = eps;
            g_pro.stage = 1;
            return;
        }
        if (g_pro.stage == 1 && head_dim == g_pro.hd &&
            !overlaps(vec, sizeof(float) * n, g_pro.q, sizeof(float) * static_cast<size_t>(g_pro.nq) * g_pro.hd)) {
            g_pro.k = vec;
            g_pro.gk = g;
            g_pro.nk = n_heads;
            g_pro.eps_k = eps;
            g_pro.stage = 3;
            return;
        }
    }
    if (!flush_prologue(where)) return;
    const bool host = !is_device_ptr(vec);
    float* d = host ? const_cast<float*>(stage_in(vec, n, g_rt.q, where)) : vec;
    if (!d) return;
    if (!check(launch_rmsnorm_heads(d, g, n_heads, head_dim, eps, g_rt.stream), where)) return;
    finish_out(vec, d, n, host, where);
}

// cpp:1760-1863
GNCX_API void gncx_apply_rope_xor11_ext(float* q_vec, float* k_vec, GNCXCompactToken* q_tokens,
                                        const uint8_t* mmap_base, size_t rope_freqs_offset, int32_t has_rope_freqs,
                                        int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t pos,
                                        float freq_base) {
    t_keep = kKeepPrologue;
    std::lock_guard<CallLock> lk(g_mu);
    t_keep = kKeepNone;
    const char* where = "gncx_apply_rope_xor11_ext";
    if (!ensure_runtime(where)) {
        (void)flush_prologue(where);
        return;
    }
    const int32_t half = head_dim / 2;
    std::array<float, kMaxRopeHalf> fac{};
    const float* factors = nullptr;
    if (has_rope_freqs) {
        if (half > kMaxRopeHalf || !read_factors(mmap_base, rope_freqs_offset, half, fac, where)) {
            (void)flush_prologue(where);
            return;
        }
        factors = fac.data();
    }
    RopeTable t;
    if (!rope_table(pos, head_dim, freq_base, factors, t)) {
        set_error(where, "head_dim must be even and at most 512", -1);
        (void)flush_prologue(where);
        return;
    }
    const size_t qn = q_vec ? static_cast<size_t>(n_heads) * head_dim : 0;
    const size_t kn = k_vec ? static_cast<size_t>(n_kv_heads) * head_dim : 0;
    bool ok = true;
    const bool may_defer = q_vec && k_vec && device_only_lazy(q_vec) && device_only_lazy(k_vec);
    q_vec = lazy_ptr(q_vec, qn, kRd | kWr, ok, where);
    k_vec = lazy_ptr(k_vec, kn, kRd | kWr, ok, where);
    if (!ok) {
        (void)flush_prologue(where);
        return;
    }
    if (may_defer && is_device_ptr(q_vec) && is_device_ptr(k_vec) &&
        (g_pro.stage == 3 ? q_vec == g_pro.q && k_vec == g_pro.k && n_heads == g_pro.nq &&
                                n_kv_heads == g_pro.nk && head_dim == g_pro.hd
                          : g_pro.stage == 0 && !overlaps(q_vec, sizeof(float) * qn, k_vec, sizeof(float) * kn))) {
        g_pro.q = q_vec;
        g_pro.k = k_vec;
        g_pro.nq = n_heads;
        g_pro.nk = n_kv_heads;
        g_pro.hd = head_dim;
        g_pro.rope = t;
        g_pro.stage |= 4;
        // telemetry phase flip of the rotated half (cpp:1818-1823, 1829-1831)
        if (q_tokens)
            for (int32_t h = 0; h < n_heads; ++h)
                for (int32_t i = 0; i < half; ++i) q_tokens[h * head_dim + i + half].phase_2bit ^= 0x03u;
        return;
    }
    if (!flush_prologue(where)) return;
    const bool hq = q_vec && !is_device_ptr(q_vec), hk = k_vec && !is_device_ptr(k_vec);
    float* dq = q_vec ? (hq ? const_cast<float*>(stage_in(q_vec, qn, g_rt.q, where)) : q_vec) : nullptr;
    float* dk = k_vec ? (hk ? const_cast<float*>(stage_in(k_vec, kn, g_rt.k, where)) : k_vec) : nullptr;
    if ((q_vec && !dq) || (k_vec && !dk)) return;
    if (!check(launch_rope(dq, dk, t, q_vec ? n_heads : 0, k_vec ? n_kv_heads : 0, head_dim, g_rt.stream), where))
        return;
    if (hq && !d2h(q_vec, dq, sizeof(float) * qn, where)) return;
    if (hk && !d2h(k_vec, dk, sizeof(float) * kn, where)) return;
    if ((hq || hk) && !sync_out(where)) return;
    // telemetry phase flip of the rotated half (cpp:1818-1823, 1829-1831)
    if (q_vec && q_tokens)
        for (int32_t h = 0; h < n_heads; ++h)
            for (int32_t i = 0; i < half; ++i) q_tokens[h * head_dim + i + half].phase_2bit ^= 0x03u;
}

// cpp:1865-1878
GNCX_API void gncx_apply_rope_xor11(float* q_vec, float* k_vec, GNCXCompactToken* q_tokens, int32_t n_heads,
                                    int32_t n_kv_heads, int32_t head_dim, int32_t pos, float freq_base) {
    gncx_apply_rope_xor11_ext(q_vec, k_vec, q_tokens, nullptr, 0, 0, n_heads, n_kv_heads, head_dim, pos, freq_base);
}

// cpp:2038-2052
GNCX_API void gncx_swiglu_activation(const float* gate_vec, const float* up_vec, int32_t ffn_dim,
                                     float* out_ffn_vec) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_swiglu_activation";
    if (ffn_dim <= 0 || !ensure_runtime(where)) return;
    bool ok = true;
    gate_vec = lazy_ptr(gate_vec, dim_count(ffn_dim), kRd, ok, where);
    up_vec = lazy_ptr(up_vec, dim_count(ffn_dim), kRd, ok, where);
    out_ffn_vec = lazy_ptr(out_ffn_vec, dim_count(ffn_dim), kWr, ok, where);
    if (!ok) return;
    const float* g = stage_in(gate_vec, ffn_dim, g_rt.q, where);
    const float* u = stage_in(up_vec, ffn_dim, g_rt.k, where);
    if (!g || !u) return;
    bool host = false;
    float* o = out_target(out_ffn_vec, ffn_dim, g_rt.o, host, where);
    if (!o) return;
    if (!check(launch_swiglu(g, u, ffn_dim, o, g_rt.stream), where)) return;
    finish_out(out_ffn_vec, o, ffn_dim, host, where);
}

// cpp:2018-2033
GNCX_API void gncx_geglu_activation(const float* gate_vec, const float* up_vec, int32_t ffn_dim,
                                    float* out_ffn_vec) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_geglu_activation";
    if (ffn_dim <= 0 || !ensure_runtime(where)) return;
    bool ok = true;
    gate_vec = lazy_ptr(gate_vec, dim_count(ffn_dim), kRd, ok, where);
    up_vec = lazy_ptr(up_vec, dim_count(ffn_dim), kRd, ok, where);
    out_ffn_vec = lazy_ptr(out_ffn_vec, dim_count(ffn_dim), kWr, ok, where);
    if (!ok) return;
    const float* g = stage_in(gate_vec, ffn_dim, g_rt.q, where);
    const float* u = stage_in(up_vec, ffn_dim, g_rt.k, where);
    if (!g || !u) return;
    bool host = false;
    float* o = out_target(out_ffn_vec, ffn_dim, g_rt.o, host, where);
    if (!o) return;
    if (!check(launch_geglu(g, u, ffn_dim, o, g_rt.stream), where)) return;
    finish_out(out_ffn_vec, o, ffn_dim, host, where);
}

// y[i] += x[i]: the residual adds the streamer does on the host
// (lua/gncx_streamer.lua:871-873, 906-908), on the device.
GNCX_API void gncx_hip_vec_add(float* y, const float* x, int32_t n) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_vec_add";
    if (n <= 0 || !y || !x || !ensure_runtime(where)) return;
    bool ok = true;
    x = lazy_ptr(x, dim_count(n), kRd, ok, where);
    y = lazy_ptr(y, dim_count(n), kRd | kWr, ok, where);
    if (!ok) return;
    const float* xd = stage_in(x, n, g_rt.k, where);
    if (!xd) return;
    const bool host_y = !is_device_ptr(y);
    float* yd = y;
    if (host_y) {
        yd = const_cast<float*>(stage_in(y, n, g_rt.o, where));
        if (!yd) return;
    }
    if (!check(launch_vec_add(yd, xd, n, g_rt.stream), where)) return;
    finish_out(y, yd, n, host_y, where);
}

// Several matrices of one type and in_dim applied to the same x in one launch.
GNCX_API void gncx_hip_matvec_multi(int32_t count, const uint8_t* const* weights, const int32_t* out_dims,
                                    int32_t ggml_type, const float* in_vec, int32_t in_dim, float* const* out_arg) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_matvec_multi";
    if (count <= 0 || count > kMaxGemvMats || !weights || !out_dims || !out_arg || !in_vec || in_dim <= 0) {
        set_error(where, "count must be 1..4, with weights, out_dims, in_vec and out_vecs given", -1);
        return;
    }
    if (!type_supported(ggml_type) || !ensure_runtime(where)) return;
    bool ok = true;
    float* out_vecs[kMaxGemvMats];
    in_vec = lazy_ptr(in_vec, dim_count(in_dim), kRd, ok, where);
    for (int32_t i = 0; i < count; ++i) out_vecs[i] = lazy_ptr(out_arg[i], dim_count(out_dims[i]), kWr, ok, where);
    if (!ok) return;
    // x staged here is not the vector the matvec act-quant cache rule refers to
    g_act.last_in = nullptr;
    g_act.staged_on_device = false;
    const uint8_t* ws[kMaxGemvMats];
    float* ys[kMaxGemvMats];
    bool host[kMaxGemvMats];
    size_t host_total = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (out_dims[i] <= 0 || !weights[i] || !out_vecs[i]) {
            set_error(where, "every matrix needs weights, out_dims > 0 and an output", -1);
            return;
        }
        ws[i] = device_weights(weights[i], row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dims[i]), where);
        if (!ws[i]) return;
        host[i] = !is_device_ptr(out_vecs[i]);
        if (host[i]) host_total += static_cast<size_t>(out_dims[i]);
    }
    const float* x = stage_in(in_vec, static_cast<size_t>(in_dim), g_rt.x, where);
    if (!x) return;
    // host outputs share one staging buffer
    if (host_total && !g_rt.y.ensure(sizeof(float) * host_total, where)) return;
    size_t off = 0;
    for (int32_t i = 0; i < count; ++i) {
        ys[i] = host[i] ? g_rt.y.as<float>() + off : out_vecs[i];
        if (host[i]) off += static_cast<size_t>(out_dims[i]);
    }
    if (!check(launch_gemv_multi(ggml_type, count, ws, out_dims, x, in_dim, ys, g_rt.stream), where)) return;
    for (int32_t i = 0; i < count; ++i)
        if (host[i] && !finish_out(out_vecs[i], ys[i], static_cast<size_t>(out_dims[i]), true, where)) return;
}

// hidden += delta, then the RMSNorm of gncx_rmsnorm_and_encode_4phase (no tokens)
// of the new hidden into out_normed_fp32, in one kernel.
GNCX_API void gncx_hip_add_rmsnorm(float* hidden, const float* delta, const uint8_t* mmap_base,
                                   size_t norm_weight_offset, int32_t dim, float eps, float* out_normed_fp32) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_add_rmsnorm";
    g_norm_epoch++;
    if (dim <= 0 || !hidden || !delta || !out_normed_fp32 || !ensure_runtime(where)) return;
    bool ok = true;
    hidden = lazy_ptr(hidden, dim_count(dim), kRd | kWr, ok, where);
    delta = lazy_ptr(delta, dim_count(dim), kRd, ok, where);
    out_normed_fp32 = lazy_ptr(out_normed_fp32, dim_count(dim), kWr, ok, where);
    if (!ok) return;
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(dim), where));
    if (!g) return;
    const float* dd = stage_in(delta, static_cast<size_t>(dim), g_rt.k, where);
    if (!dd) return;
    const bool host_h = !is_device_ptr(hidden);
    float* hd = hidden;
    if (host_h) {
        hd = const_cast<float*>(stage_in(hidden, static_cast<size_t>(dim), g_rt.q, where));
        if (!hd) return;
    }
    bool host_o = false;
    float* o = out_target(out_normed_fp32, static_cast<size_t>(dim), g_rt.o, host_o, where);
    if (!o) return;
    if (!check(launch_add_rmsnorm(hd, dd, g, dim, eps, o, g_rt.stream), where)) return;
    if (!finish_out(hidden, hd, static_cast<size_t>(dim), host_h, where)) return;
    finish_out(out_normed_fp32, o, static_cast<size_t>(dim), host_o, where);
}

namespace {
// cpp:693-780: one row of the embedding table, decoded on the device.
void fetch_embedding(int32_t type, const uint8_t* base, size_t off, int32_t token, int32_t dim, float scale,
                     float* out, const char* where) {
    std::lock_guard<CallLock> lk(g_mu);
    if (dim <= 0 || token < 0 || !ensure_runtime(where)) return;
    bool ok = true;
    out = lazy_ptr(out, dim_count(dim), kWr, ok, where);
    if (!ok) return;
    const size_t rb = row_bytes(type, dim);
    const uint8_t* row = base + off + static_cast<size_t>(token) * rb;
    const uint8_t* drow;
    // a registered (or device-resident) table is read in place; otherwise only the row travels
    auto it = g_rt.weights.find(reinterpret_cast<uintptr_t>(base + off));
    if (is_device_ptr(row)) {
        drow = row;
    } else if (it != g_rt.weights.end() && (static_cast<size_t>(token) + 1) * rb <= it->second.bytes) {
        drow = it->second.d + static_cast<size_t>(token) * rb;
    } else {
        if (!g_rt.aux.ensure(round_up(rb, 16), where)) return;
        if (!h2d(g_rt.aux.p, row, rb, where)) return;
        drow = g_rt.aux.as<uint8_t>();
    }
    bool host = false;
    float* o = out_target(out, dim, g_rt.o, host, where);
    if (!o) return;
    if (!check(launch_fetch_embedding(type, drow, 0, dim, scale, o, g_rt.stream), where)) return;
    finish_out(out, o, dim, host, where);
}
}  // namespace

// The rows of count tokens (host token ids, checked against vocab_size) of an
// embedding table in one launch: the values of one gncx_fetch_token_embedding_*
// call per token (the streamer's prefill loop, lua/gncx_streamer.lua:1001-1003).
GNCX_API void gncx_hip_fetch_token_embeddings(int32_t ggml_type, const uint8_t* mmap_base, size_t tensor_abs_offset,
                                              const int32_t* token_ids, int32_t count, int32_t vocab_size,
                                              int32_t embed_dim, float scale_factor, float* out_rows) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_fetch_token_embeddings";
    if (ggml_type != kQ8_0 && ggml_type != kQ6_K && ggml_type != kBF16) {
        set_error(where, "the embedding table must be Q8_0, Q6_K or BF16", -1);
        return;
    }
    if (!token_ids || !out_rows || count <= 0 || count > 65535 || vocab_size <= 0 || embed_dim <= 0) {
        set_error(where, "token_ids, out_rows, count 1..65535, vocab_size > 0 and embed_dim > 0 are required", -1);
        return;
    }
    if (is_device_ptr(token_ids)) {
        set_error(where, "token_ids must be host memory (they are checked against vocab_size first)", -1);
        return;
    }
    for (int32_t i = 0; i < count; ++i) {
        if (token_ids[i] < 0 || token_ids[i] >= vocab_size) {
            set_error(where, "a token id is outside [0, vocab_size)", -1);
            return;
        }
    }
    if (!ensure_runtime(where)) return;
    bool ok = true;
    const size_t n = static_cast<size_t>(count) * static_cast<size_t>(embed_dim);
    out_rows = lazy_ptr(out_rows, n, kWr, ok, where);
    if (!ok) return;
    const size_t rb = row_bytes(ggml_type, embed_dim);
    const uint8_t* table = device_weights(mmap_base + tensor_abs_offset, rb * static_cast<size_t>(vocab_size), where);
    if (!table) return;
    if (!g_rt.v.ensure(round_up(sizeof(int32_t) * static_cast<size_t>(count), 16), where)) return;
    if (!h2d(g_rt.v.p, token_ids, sizeof(int32_t) * static_cast<size_t>(count), where)) return;
    bool host = false;
    float* o = out_target(out_rows, n, g_rt.o, host, where);
    if (!o) return;
    if (!check(launch_fetch_embedding_rows(ggml_type, table, g_rt.v.as<int32_t>(), count, embed_dim, scale_factor, o,
                                           g_rt.stream),
               where))
        return;
    finish_out(out_rows, o, n, host, where);
}

// cpp:693-715
GNCX_API void gncx_fetch_token_embedding_q8_0(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                              int32_t embed_dim, float scale_factor, float* out_hidden) {
    fetch_embedding(kQ8_0, mmap_base, tensor_abs_offset, token_id, embed_dim, scale_factor, out_hidden,
                    "gncx_fetch_token_embedding_q8_0");
}
// cpp:720-760
GNCX_API void gncx_fetch_token_embedding_q6_k(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                              int32_t embed_dim, float scale_factor, float* out_hidden) {
    fetch_embedding(kQ6_K, mmap_base, tensor_abs_offset, token_id, embed_dim, scale_factor, out_hidden,
                    "gncx_fetch_token_embedding_q6_k");
}
// cpp:765-780
GNCX_API void gncx_fetch_token_embedding_bf16(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                              int32_t embed_dim, float scale_factor, float* out_hidden) {
    fetch_embedding(kBF16, mmap_base, tensor_abs_offset, token_id, embed_dim, scale_factor, out_hidden,
                    "gncx_fetch_token_embedding_bf16");
}

// cpp:789-890.  The norm and, when out_tokens is given, the 4-phase
// telemetry encode (cpp:842-889) run on the device; the tokens are the
// reference's bit for bit (same rounding at every step).
GNCX_API void gncx_rmsnorm_and_encode_4phase(const float* input_hidden, const uint8_t* mmap_base,
                                             size_t norm_weight_offset, int32_t dim, float eps, int32_t layer_k,
                                             float* out_normed_fp32, GNCXCompactToken* out_tokens,
                                             float* out_quant_scale) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_rmsnorm_and_encode_4phase";
    g_norm_epoch++;
    if (dim <= 0 || !ensure_runtime(where)) return;
    bool ok = true;
    // with tokens the call waits before it returns: the kernel may read a
    // host-owned hidden vector from a page-locked copy
    input_hidden = lazy_ptr(input_hidden, dim_count(dim), out_tokens ? kRd | kRdPinned : kRd, ok, where);
    out_normed_fp32 = lazy_ptr(out_normed_fp32, dim_count(dim), kWr, ok, where);
    if (!ok) return;
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(dim), where));
    if (!g) return;
    const float* x = stage_in(input_hidden, dim, g_rt.q, where);
    if (!x) return;
    bool host = false;
    float* o = out_target(out_normed_fp32, dim, g_rt.o, host, where);
    if (!o) return;
    if (out_tokens == nullptr) {
        if (!check(launch_rmsnorm(x, g, 1, dim, eps, o, g_rt.stream), where)) return;
        if (!finish_out(out_normed_fp32, o, dim, host, where)) return;
        if (out_quant_scale) *out_quant_scale = 1.0f;
        return;
    }
    // the encode runs on the device in the norm's kernel and writes tokens,
    // scale and cancellation count straight into a page-locked slot: one wait
    const size_t tok_words = round_up(static_cast<size_t>(dim), 64);
    PinnedSlot* sl = pinned_slot(sizeof(uint32_t) * (tok_words + 2), where);
    if (!sl) return;
    uint32_t* ht = static_cast<uint32_t*>(sl->p);
    if (!check(launch_rmsnorm_encode(x, g, dim, eps, o, layer_k, ht, reinterpret_cast<float*>(ht + tok_words),
                                     g_rt.stream),
               where))
        return;
    if (!check(hipEventRecord(sl->ev, g_rt.stream), where)) return;
    sl->pending = true;
    if (host && !d2h(out_normed_fp32, o, sizeof(float) * dim, where)) return;
    if (!sync_out(where)) return;
    std::memcpy(out_tokens, ht, sizeof(uint32_t) * dim);
    if (out_quant_scale) std::memcpy(out_quant_scale, ht + tok_words, sizeof(float));
    const uint64_t c = ht[tok_words + 1];
    g_norm_epoch_cancellations = c;
    g_norm_epoch_tokens_ptr = out_tokens;
}

// =======================================================================
// Build-side extensions (no counterpart in the reference)
// =======================================================================

// Select the device (default 0 or $GNCX_DEVICE).  Returns 0 or a HIP error.
GNCX_API int gncx_hip_init(int device) {
    std::lock_guard<CallLock> lk(g_mu);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        set_error("gncx_hip_init", "no HIP device is visible", e ? static_cast<int>(e) : -1);
        return g_last_code;
    }
    if (device < 0 || device >= n) return static_cast<int>(hipErrorInvalidDevice);
    e = hipSetDevice(device);
    if (e != hipSuccess) return static_cast<int>(e);
    g_rt.device = device;
    g_rt.ready = true;
    // the no-allocation step's scratch on this device (noalloc.hip)
    void* scratch = nullptr;
    if (!check(noalloc_scratch(device, &scratch), "gncx_hip_init")) return g_last_code;
    return 0;
}

// Stream the library enqueues on (default: the null stream).
GNCX_API void gncx_hip_set_stream(void* stream) {
    std::lock_guard<CallLock> lk(g_mu);
    g_rt.stream = static_cast<hipStream_t>(stream);
}
GNCX_API void* gncx_hip_get_stream(void) { return g_rt.stream; }

GNCX_API int gncx_hip_synchronize(void) {
    std::lock_guard<CallLock> lk(g_mu);
    return static_cast<int>(hipStreamSynchronize(g_rt.stream));
}

// Last failure ("" when none) and its code (0 when none); reading clears.
GNCX_API const char* gncx_hip_last_error(void) { return g_last_error.c_str(); }
GNCX_API int gncx_hip_last_status(void) {
    std::lock_guard<CallLock> lk(g_mu);
    const int c = g_last_code;
    g_last_code = 0;
    if (c == 0) g_last_error.clear();
    return c;
}

// Drop the device copy of host weights at p (all copies when p is null).
GNCX_API void gncx_hip_weight_forget(const void* p) {
    std::lock_guard<CallLock> lk(g_mu);
    if (p) {
        forget_weight(reinterpret_cast<uintptr_t>(p));
        return;
    }
    (void)flush_pending("weight copy release");
    for (auto& kv : g_rt.weights) (void)hipFree(kv.second.d);
    g_rt.weights.clear();
}

// Drop the device twin of a host KV cache (all twins when p is null); call
// after rewriting a host cache outside this library.
GNCX_API void gncx_hip_kv_forget(const float* p) {
    std::lock_guard<CallLock> lk(g_mu);
    if (p) {
        forget_kv(reinterpret_cast<uintptr_t>(p));
        return;
    }
    for (auto& kv : g_rt.kv) (void)hipFree(kv.second.d);
    g_rt.kv.clear();
}

// Bytes of device memory held by uploaded weights.
GNCX_API size_t gncx_hip_weight_bytes(void) {
    std::lock_guard<CallLock> lk(g_mu);
    size_t s = 0;
    for (auto& kv : g_rt.weights) s += kv.second.bytes;
    return s;
}

// Dequantise out_dim rows of in_dim weights to fp32 with the block decoders
// the dots use (bit-exact with the reference's decoders).
GNCX_API void gncx_hip_dequantize(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                  int32_t in_dim, int32_t out_dim, float* out) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_dequantize";
    if (!type_supported(ggml_type) || in_dim <= 0 || out_dim <= 0 || !ensure_runtime(where)) return;
    const size_t wbytes = row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dim);
    const uint8_t* w = device_weights(mmap_base + weight_abs_offset, wbytes, where);
    if (!w) return;
    const size_t n = static_cast<size_t>(in_dim) * out_dim;
    bool host = false;
    float* o = out_target(out, n, g_rt.y, host, where);
    if (!o) return;
    if (!check(launch_dequant(ggml_type, w, in_dim, out_dim, o, g_rt.stream), where)) return;
    finish_out(out, o, n, host, where);
}

// Per-32 Q8 activation blocks of `rows` rows of in_dim values (cpp:955-995):
// q[rows*in_dim] int8 and meta[rows*in_dim/32][4] = {d (float bits), sum of
// q[0:16], sum of q[16:32], sum of q[0:32]}.
GNCX_API void gncx_hip_quantize_act(const float* in, int32_t rows, int32_t in_dim, int8_t* q, int32_t* meta) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_quantize_act";
    if (rows <= 0 || in_dim <= 0 || !ensure_runtime(where)) return;
    const size_t n = static_cast<size_t>(rows) * in_dim;
    const size_t nb = n / 32;
    const float* x = stage_in(in, n, g_rt.aux, where);
    if (!x) return;
    if (!g_rt.ws.ensure(round_up(n, 256) + nb * sizeof(ActMeta), where)) return;
    int8_t* dq = g_rt.ws.as<int8_t>();
    ActMeta* dm = reinterpret_cast<ActMeta*>(g_rt.ws.as<char>() + round_up(n, 256));
    if (!check(launch_act_quant(x, rows, in_dim, dq, dm, g_rt.stream), where)) return;
    if (!check(hipMemcpyAsync(q, dq, n, is_device_ptr(q) ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost,
                              g_rt.stream),
               where))
        return;
    if (!check(hipMemcpyAsync(meta, dm, nb * sizeof(ActMeta),
                              is_device_ptr(meta) ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, g_rt.stream),
               where))
        return;
    check(hipStreamSynchronize(g_rt.stream), where);
}

// Decode attention step with the per-head RMSNorm (cpp:895-953) and RoPE
// (cpp:1760-1863) of q and k fused in front of the KV scan: one call does
// what the reference does with gncx_rmsnorm_inplace_heads(q),
// gncx_rmsnorm_inplace_heads(k), gncx_apply_rope_xor11_ext(q, k) and
// gncx_mqa_attention_step_ext, with the same results.  q_vec/k_vec receive
// the normalised, rotated vectors as those calls leave them.  Norm weights are
// addressed like the reference's (base + offset, has_weight); rope_base <= 0
// skips the rotation.
namespace {
// the body of gncx_hip_attention_step_fused; the caller holds g_mu
void attention_step_fused_impl(float* q_vec, float* k_vec, const float* v_vec, float* k_cache_layer,
                               float* v_cache_layer, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                               int32_t head_dim, float attn_scale, int32_t sliding_window, int32_t write_kv,
                               const uint8_t* mmap_base, size_t q_norm_offset, size_t k_norm_offset,
                               int32_t has_norm_weight, float norm_eps, size_t rope_freqs_offset,
                               int32_t has_rope_freqs, float rope_base, float* out_attn_vec, const char* where) {
    if (!ensure_runtime(where)) return;
    const float* qg = nullptr;
    const float* kg = nullptr;
    if (has_norm_weight) {
        qg = reinterpret_cast<const float*>(
            device_weights(mmap_base + q_norm_offset, sizeof(float) * static_cast<size_t>(head_dim), where));
        kg = reinterpret_cast<const float*>(
            device_weights(mmap_base + k_norm_offset, sizeof(float) * static_cast<size_t>(head_dim), where));
        if (!qg || !kg) return;
    }
    RopeTable t;
    const RopeTable* rp = nullptr;
    if (rope_base > 0.0f) {
        std::array<float, kMaxRopeHalf> fac{};
        const float* factors = nullptr;
        if (has_rope_freqs) {
            if (head_dim / 2 > kMaxRopeHalf || !read_factors(mmap_base, rope_freqs_offset, head_dim / 2, fac, where))
                return;
            factors = fac.data();
        }
        if (!rope_table(pos, head_dim, rope_base, factors, t)) {
            set_error(where, "head_dim must be even and at most 512", -1);
            return;
        }
        rp = &t;
    }
    AttnCall c{q_vec, k_vec, v_vec, k_cache_layer, v_cache_layer, pos, n_heads, n_kv_heads, head_dim, attn_scale,
               sliding_window, write_kv, out_attn_vec};
    c.norm_qk = 1;
    c.q_gamma = qg;
    c.k_gamma = kg;
    c.eps = norm_eps;
    c.rope = rp;
    c.q_back = q_vec;
    c.k_back = k_vec;
    attention_impl(c, where);
}

// RoPE rows of positions pos0 .. pos0 + batch - 1 ([batch][head_dim]: cos
// then sin, host libm like the single-position table), kept on the device
// for the next call with the same key (every layer of one prefill)
struct RopeRows {
    DevBuf buf;
    int32_t pos0 = -1, batch = 0, head_dim = 0;
    float base = 0.0f;
    std::array<float, kMaxRopeHalf> fac{};
    bool has_fac = false;
} g_rope_rows;

const float* rope_rows(int32_t pos0, int32_t batch, int32_t head_dim, float base, const float* factors,
                       const char* where) {
    RopeRows& r = g_rope_rows;
    const int32_t half = head_dim / 2;
    const bool same = r.pos0 == pos0 && r.batch == batch && r.head_dim == head_dim && r.base == base &&
                      r.has_fac == (factors != nullptr) &&
                      (!factors || std::memcmp(r.fac.data(), factors, sizeof(float) * half) == 0);
    if (same) return r.buf.as<float>();
    std::vector<float> tab(static_cast<size_t>(batch) * head_dim);
    RopeTable t;
    for (int32_t i = 0; i < batch; ++i) {
        if (!rope_table(pos0 + i, head_dim, base, factors, t)) {
            set_error(where, "head_dim must be even and at most 512", -1);
            return nullptr;
        }
        std::memcpy(&tab[static_cast<size_t>(i) * head_dim], t.c, sizeof(float) * half);
        std::memcpy(&tab[static_cast<size_t>(i) * head_dim + half], t.s, sizeof(float) * half);
    }
    r.pos0 = -1;
    // a kernel queued with the previous rows may still read them
    if (!check(hipStreamSynchronize(g_rt.stream), where)) return nullptr;
    if (!r.buf.ensure(sizeof(float) * tab.size(), where)) return nullptr;
    if (!check(hipMemcpy(r.buf.p, tab.data(), sizeof(float) * tab.size(), hipMemcpyHostToDevice), where))
        return nullptr;
    r.pos0 = pos0;
    r.batch = batch;
    r.head_dim = head_dim;
    r.base = base;
    r.has_fac = factors != nullptr;
    if (factors) std::memcpy(r.fac.data(), factors, sizeof(float) * half);
    return r.buf.as<float>();
}

// The key-split plan of the last prefill shape (attention_prefill_plan),
// uploaded once per shape with its partial-result buffer; the layers of one
// prefill share both, their launches being in stream order.
struct PrefillPlan {
    int32_t pos0 = -1, batch = 0, sw = 0, n_heads = 0, n_kv = 0;
    int32_t n_items = 0, n_split = 0, part_slots = 0;
    bool some = false;
    DevBuf tab, part;
} g_pf_plan;

bool prefill_plan(PrefillArgs& a, const char* where) {
    PrefillPlan& pl = g_pf_plan;
    if (!(pl.pos0 == a.pos0 && pl.batch == a.batch && pl.sw == a.sliding_window && pl.n_heads == a.n_heads &&
          pl.n_kv == a.n_kv_heads)) {
        std::vector<int32_t> tab;
        int32_t ni = 0, ns = 0;
        const bool some = attention_prefill_plan(a, tab, ni, ns);
        const int32_t slots = some ? attention_prefill_part_slots(tab, ni, ns) : 0;
        pl.pos0 = -1;
        if (some) {
            // a launch queued with the previous plan may still read it
            if (!check(hipStreamSynchronize(g_rt.stream), where)) return false;
            if (!pl.tab.ensure(sizeof(int32_t) * tab.size(), where) ||
                !pl.part.ensure(sizeof(float) * attention_prefill_part_floats(slots, a.n_kv_heads), where))
                return false;
            if (!check(hipMemcpy(pl.tab.p, tab.data(), sizeof(int32_t) * tab.size(), hipMemcpyHostToDevice), where))
                return false;
        }
        pl.some = some;
        pl.n_items = ni;
        pl.n_split = ns;
        pl.part_slots = slots;
        pl.pos0 = a.pos0;
        pl.batch = a.batch;
        pl.sw = a.sliding_window;
        pl.n_heads = a.n_heads;
        pl.n_kv = a.n_kv_heads;
    }
    if (pl.some) {
        a.plan = pl.tab.as<int32_t>();
        a.n_items = pl.n_items;
        a.n_split = pl.n_split;
        a.part_slots = pl.part_slots;
        a.part = pl.part.as<float>();
    }
    return true;
}
}  // namespace

GNCX_API void gncx_hip_attention_step_fused(float* q_vec, float* k_vec, const float* v_vec, float* k_cache_layer,
                                            float* v_cache_layer, int32_t pos, int32_t n_heads,
                                            int32_t n_kv_heads, int32_t head_dim, float attn_scale,
                                            int32_t sliding_window, int32_t write_kv, const uint8_t* mmap_base,
                                            size_t q_norm_offset, size_t k_norm_offset, int32_t has_norm_weight,
                                            float norm_eps, size_t rope_freqs_offset, int32_t has_rope_freqs,
                                            float rope_base, float* out_attn_vec) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_attention_step_fused";
    bool ok = true;
    const size_t qn = dim_count(n_heads) * dim_count(head_dim), kvn = dim_count(n_kv_heads) * dim_count(head_dim);
    const int cache_access = write_kv && k_vec && v_vec ? kRd | kWr : kRd;
    q_vec = lazy_ptr(q_vec, qn, kRd | kWr, ok, where);
    k_vec = lazy_ptr(k_vec, kvn, kRd | kWr, ok, where);
    v_vec = lazy_ptr(v_vec, kvn, kRd, ok, where);
    k_cache_layer = lazy_ptr(k_cache_layer, (dim_count(pos) + 1) * kvn, cache_access, ok, where);
    v_cache_layer = lazy_ptr(v_cache_layer, (dim_count(pos) + 1) * kvn, cache_access, ok, where);
    out_attn_vec = lazy_ptr(out_attn_vec, qn, kWr, ok, where);
    if (!ok) return;
    attention_step_fused_impl(q_vec, k_vec, v_vec, k_cache_layer, v_cache_layer, pos, n_heads, n_kv_heads, head_dim,
                              attn_scale, sliding_window, write_kv, mmap_base, q_norm_offset, k_norm_offset,
                              has_norm_weight, norm_eps, rope_freqs_offset, has_rope_freqs, rope_base, out_attn_vec,
                              where);
}

// gncx_hip_attention_step_fused for tokens pos0 .. pos0 + batch - 1 in turn
// (write_kv = 1), as one batched causal pass where the kernels take the shape
GNCX_API void gncx_hip_attention_prefill(float* q_batch, float* k_batch, const float* v_batch, float* k_cache_layer,
                                         float* v_cache_layer, int32_t pos0, int32_t batch, int32_t n_heads,
                                         int32_t n_kv_heads, int32_t head_dim, float attn_scale,
                                         int32_t sliding_window, const uint8_t* mmap_base, size_t q_norm_offset,
                                         size_t k_norm_offset, int32_t has_norm_weight, float norm_eps,
                                         size_t rope_freqs_offset, int32_t has_rope_freqs, float rope_base,
                                         float* out_batch) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_attention_prefill";
    if (!ensure_runtime(where) || batch <= 0) return;
    if (pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || n_heads % n_kv_heads != 0 || !q_batch ||
        !k_batch || !v_batch || !k_cache_layer || !v_cache_layer || !out_batch) {
        set_error(where, "invalid head geometry, position or pointer", -1);
        return;
    }
    const size_t qn = static_cast<size_t>(n_heads) * head_dim, kn = static_cast<size_t>(n_kv_heads) * head_dim;
    bool ok = true;
    const size_t bt = dim_count(batch), rows = dim_count(pos0) + bt;
    q_batch = lazy_ptr(q_batch, bt * qn, kRd | kWr, ok, where);
    k_batch = lazy_ptr(k_batch, bt * kn, kRd | kWr, ok, where);
    v_batch = lazy_ptr(v_batch, bt * kn, kRd, ok, where);
    k_cache_layer = lazy_ptr(k_cache_layer, rows * kn, kRd | kWr, ok, where);
    v_cache_layer = lazy_ptr(v_cache_layer, rows * kn, kRd | kWr, ok, where);
    out_batch = lazy_ptr(out_batch, bt * qn, kWr, ok, where);
    if (!ok) return;
    if (!attention_prefill_supported(n_heads, n_kv_heads, head_dim)) {
        for (int32_t t = 0; t < batch; ++t)
            attention_step_fused_impl(q_batch + t * qn, k_batch + t * kn, v_batch + t * kn, k_cache_layer,
                                      v_cache_layer, pos0 + t, n_heads, n_kv_heads, head_dim, attn_scale,
                                      sliding_window, 1, mmap_base, q_norm_offset, k_norm_offset, has_norm_weight,
                                      norm_eps, rope_freqs_offset, has_rope_freqs, rope_base, out_batch + t * qn,
                                      where);
        return;
    }
    const float* qg = nullptr;
    const float* kg = nullptr;
    if (has_norm_weight) {
        qg = reinterpret_cast<const float*>(
            device_weights(mmap_base + q_norm_offset, sizeof(float) * static_cast<size_t>(head_dim), where));
        kg = reinterpret_cast<const float*>(
            device_weights(mmap_base + k_norm_offset, sizeof(float) * static_cast<size_t>(head_dim), where));
        if (!qg || !kg) return;
    }
    const float* rope = nullptr;
    if (rope_base > 0.0f) {
        std::array<float, kMaxRopeHalf> fac{};
        const float* factors = nullptr;
        if (has_rope_freqs) {
            if (!read_factors(mmap_base, rope_freqs_offset, head_dim / 2, fac, where)) return;
            factors = fac.data();
        }
        rope = rope_rows(pos0, batch, head_dim, rope_base, factors, where);
        if (!rope) return;
    }
    const size_t nq = static_cast<size_t>(batch) * qn, nk = static_cast<size_t>(batch) * kn;
    const bool host_q = !is_device_ptr(q_batch), host_k = !is_device_ptr(k_batch);
    float* qd = host_q ? const_cast<float*>(stage_in(q_batch, nq, g_rt.q, where)) : q_batch;
    float* kd = host_k ? const_cast<float*>(stage_in(k_batch, nk, g_rt.k, where)) : k_batch;
    const float* vd = stage_in(v_batch, nk, g_rt.v, where);
    if (!qd || !kd || !vd) return;
    const int32_t kv_dim = static_cast<int32_t>(kn);
    const bool host_kc = !is_device_ptr(k_cache_layer), host_vc = !is_device_ptr(v_cache_layer);
    float* kc = host_kc ? kv_twin(k_cache_layer, kv_dim, pos0, pos0 + batch, where) : k_cache_layer;
    if (!kc) return;
    float* vc = host_vc ? kv_twin(v_cache_layer, kv_dim, pos0, pos0 + batch, where) : v_cache_layer;
    if (!vc) return;
    bool host_out = false;
    float* od = out_target(out_batch, nq, g_rt.o, host_out, where);
    if (!od) return;
    PrefillArgs a{};
    a.q = qd;
    a.k = kd;
    a.v = vd;
    a.k_cache = kc;
    a.v_cache = vc;
    a.out = od;
    a.pos0 = pos0;
    a.batch = batch;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.head_dim = head_dim;
    a.scale = attn_scale;
    a.sliding_window = sliding_window;
    a.norm_qk = 1;
    a.q_gamma = qg;
    a.k_gamma = kg;
    a.eps = norm_eps;
    a.rope = rope;
    if (!prefill_plan(a, where)) return;
    if (!check(launch_attention_prefill(a, g_rt.stream), where)) return;
    // host copies: the caches' new rows (the reference writes them in the call), q / k (prologue results), out
    const size_t row0 = static_cast<size_t>(pos0) * kn;
    auto back = [&](float* host, const float* dev, size_t n) {
        return d2h(host, dev, sizeof(float) * n, where);
    };
    if (host_kc && !back(k_cache_layer + row0, kc + row0, nk)) return;
    if (host_vc && !back(v_cache_layer + row0, vc + row0, nk)) return;
    if (host_q && !back(q_batch, qd, nq)) return;
    if (host_k && !back(k_batch, kd, nk)) return;
    if (host_out && !back(out_batch, od, nq)) return;
    if ((host_kc || host_vc || host_q || host_k || host_out) && !sync_out(where)) return;
    if (host_kc) kv_mark_written(k_cache_layer, pos0 + batch - 1);
    if (host_vc) kv_mark_written(v_cache_layer, pos0 + batch - 1);
}

// RMSNorm of `rows` contiguous vectors of dim with one gamma
GNCX_API void gncx_hip_rmsnorm_rows(const float* in, int32_t rows, const uint8_t* mmap_base,
                                    size_t norm_weight_offset, int32_t dim, float eps, float* out) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_rmsnorm_rows";
    g_norm_epoch++;
    if (rows <= 0 || dim <= 0 || !in || !out || !ensure_runtime(where)) return;
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(dim), where));
    if (!g) return;
    const size_t n = static_cast<size_t>(rows) * dim;
    const float* x = stage_in(in, n, g_rt.q, where);
    if (!x) return;
    bool host = false;
    float* o = out_target(out, n, g_rt.o, host, where);
    if (!o) return;
    if (!check(launch_rmsnorm(x, g, rows, dim, eps, o, g_rt.stream), where)) return;
    finish_out(out, o, n, host, where);
}

// gncx_hip_add_rmsnorm over `rows` contiguous rows of dim: hidden[r] +=
// delta[r], then out[r] = the RMSNorm of the new hidden[r], one launch; the
// same values as gncx_hip_vec_add of the rows followed by gncx_hip_rmsnorm_rows.
GNCX_API void gncx_hip_add_rmsnorm_rows(float* hidden, const float* delta, int32_t rows, const uint8_t* mmap_base,
                                        size_t norm_weight_offset, int32_t dim, float eps, float* out) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_add_rmsnorm_rows";
    g_norm_epoch++;
    if (rows <= 0 || dim <= 0 || !hidden || !delta || !out || !ensure_runtime(where)) return;
    const size_t n = static_cast<size_t>(rows) * dim;
    bool ok = true;
    hidden = lazy_ptr(hidden, n, kRd | kWr, ok, where);
    delta = lazy_ptr(delta, n, kRd, ok, where);
    out = lazy_ptr(out, n, kWr, ok, where);
    if (!ok) return;
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(dim), where));
    if (!g) return;
    const float* dd = stage_in(delta, n, g_rt.k, where);
    if (!dd) return;
    const bool host_h = !is_device_ptr(hidden);
    float* hd = hidden;
    if (host_h) {
        hd = const_cast<float*>(stage_in(hidden, n, g_rt.q, where));
        if (!hd) return;
    }
    bool host_o = false;
    float* o = out_target(out, n, g_rt.o, host_o, where);
    if (!o) return;
    if (!check(launch_add_rmsnorm_rows(hd, dd, g, rows, dim, eps, o, g_rt.stream), where)) return;
    if (!finish_out(hidden, hd, n, host_h, where)) return;
    finish_out(out, o, n, host_o, where);
}

// ---- fused decode-chain matvecs ------------------------------------------
// Device pointers only (these are for callers whose hidden state lives in
// HBM); weights may be host (uploaded once) or device memory.

namespace {
bool all_device(std::initializer_list<const void*> ps) {
    for (const void* p : ps)
        if (p && !is_device_ptr(p)) return false;
    return true;
}
}  // namespace

GNCX_API void gncx_hip_matvec_multi_addnorm(const float* hidden, const float* delta, const uint8_t* mmap_base,
                                            size_t norm_weight_offset, float eps, float* hidden_out, int32_t count,
                                            const uint8_t* const* weights, const int32_t* out_dims,
                                            int32_t ggml_type, int32_t in_dim, float* const* out_vecs) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_matvec_multi_addnorm";
    g_norm_epoch++;
    if (count <= 0 || count > kMaxGemvMats || !weights || !out_dims || !out_vecs || !hidden || in_dim <= 0 ||
        hidden_out == hidden) {
        set_error(where, "count 1..4 with weights, out_dims and outputs; hidden_out must differ from hidden", -1);
        return;
    }
    if (!type_supported(ggml_type) || !ensure_runtime(where)) return;
    if (!all_device({hidden, delta, hidden_out})) {
        set_error(where, "hidden, delta and hidden_out must be device memory", -1);
        return;
    }
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(in_dim), where));
    if (!g) return;
    const uint8_t* ws[kMaxGemvMats];
    for (int32_t i = 0; i < count; ++i) {
        if (out_dims[i] <= 0 || !weights[i] || !out_vecs[i] || !is_device_ptr(out_vecs[i])) {
            set_error(where, "every matrix needs weights, out_dims > 0 and a device output", -1);
            return;
        }
        ws[i] = device_weights(weights[i], row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dims[i]), where);
        if (!ws[i]) return;
    }
    GemvFusion f;
    f.h = hidden;
    f.r = delta;
    f.gamma = g;
    f.eps = eps;
    f.h_out = hidden_out;
    hipError_t e = launch_gemv_fused(ggml_type, count, ws, out_dims, in_dim, out_vecs, f, g_rt.stream);
    if (e != hipErrorNotSupported) {
        check(e, where);
        return;
    }
    // the separate kernels, same results: h_out = h + delta, normed into the staging buffer
    if (!g_rt.x.ensure(sizeof(float) * static_cast<size_t>(in_dim), where)) return;
    float* xn = g_rt.x.as<float>();
    if (delta) {
        if (!hidden_out) {
            set_error(where, "this shape needs hidden_out for the separate add+RMSNorm", -1);
            return;
        }
        if (!check(hipMemcpyAsync(hidden_out, hidden, sizeof(float) * in_dim, hipMemcpyDeviceToDevice, g_rt.stream),
                   where) ||
            !check(launch_add_rmsnorm(hidden_out, delta, g, in_dim, eps, xn, g_rt.stream), where))
            return;
    } else {
        if (!check(launch_rmsnorm(hidden, g, 1, in_dim, eps, xn, g_rt.stream), where)) return;
        if (hidden_out && !check(hipMemcpyAsync(hidden_out, hidden, sizeof(float) * in_dim, hipMemcpyDeviceToDevice,
                                                g_rt.stream),
                                 where))
            return;
    }
    check(launch_gemv_multi(ggml_type, count, ws, out_dims, xn, in_dim, out_vecs, g_rt.stream), where);
}

// The batch form: hidden += delta over batch_size rows (delta may be NULL:
// hidden is left as it is), then gncx_hip_matbatch_multi of the rows'
// RMSNorm, the norm formed inside the activation pass where the plan allows.
GNCX_API void gncx_hip_matbatch_multi_addnorm(float* hidden, const float* delta, const uint8_t* mmap_base,
                                              size_t norm_weight_offset, float eps, int32_t count,
                                              const uint8_t* const* weights, const int32_t* out_dims,
                                              int32_t ggml_type, int32_t batch_size, int32_t in_dim,
                                              float* const* out_batches) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_matbatch_multi_addnorm";
    g_norm_epoch++;
    if (count <= 0 || count > 4 || !weights || !out_dims || !out_batches || !hidden || in_dim <= 0 ||
        batch_size <= 0) {
        set_error(where, "count 1..4 with weights, out_dims, outputs, hidden and positive sizes", -1);
        return;
    }
    if (!type_supported(ggml_type) || !ensure_runtime(where)) return;
    if (!all_device({hidden, delta})) {
        set_error(where, "hidden and delta must be device memory", -1);
        return;
    }
    const float* g = reinterpret_cast<const float*>(
        device_weights(mmap_base + norm_weight_offset, sizeof(float) * static_cast<size_t>(in_dim), where));
    if (!g) return;
    const uint8_t* ws[4];
    for (int32_t i = 0; i < count; ++i) {
        if (out_dims[i] <= 0 || !weights[i] || !out_batches[i] || !is_device_ptr(out_batches[i])) {
            set_error(where, "every matrix needs weights, out_dims > 0 and a device output", -1);
            return;
        }
        ws[i] = device_weights(weights[i], row_bytes(ggml_type, in_dim) * static_cast<size_t>(out_dims[i]), where);
        if (!ws[i]) return;
    }
    if (!g_rt.ws.ensure(matbatch_multi_workspace_bytes(ggml_type, count, out_dims, batch_size, in_dim), where))
        return;
    const hipError_t e = launch_matbatch_multi_norm(ggml_type, count, ws, out_dims, hidden, delta, g, eps, batch_size,
                                                    in_dim, out_batches, g_rt.ws.p, g_rt.ws.cap, g_rt.stream);
    if (e != hipErrorNotSupported) {
        check(e, where);
        return;
    }
    // the two steps, same values: the normed rows in a staging buffer
    const size_t n = static_cast<size_t>(batch_size) * in_dim;
    if (!g_rt.v.ensure(sizeof(float) * n, where)) return;
    float* xn = g_rt.v.as<float>();
    if (delta) {
        if (!check(launch_add_rmsnorm_rows(hidden, delta, g, batch_size, in_dim, eps, xn, g_rt.stream), where)) return;
    } else if (!check(launch_rmsnorm(hidden, g, batch_size, in_dim, eps, xn, g_rt.stream), where)) {
        return;
    }
    check(launch_matbatch_multi(ggml_type, count, ws, out_dims, xn, batch_size, in_dim, out_batches, g_rt.ws.p,
                                g_rt.ws.cap, g_rt.stream),
          where);
}

GNCX_API void gncx_hip_matvec_swiglu(const uint8_t* gate_weights, const uint8_t* up_weights, int32_t ggml_type,
                                     const float* in_vec, int32_t in_dim, int32_t ffn_dim, float* out_act) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_matvec_swiglu";
    if (!gate_weights || !up_weights || !in_vec || !out_act || in_dim <= 0 || ffn_dim <= 0) {
        set_error(where, "weights, in_vec, out_act and positive dims are required", -1);
        return;
    }
    if (!type_supported(ggml_type) || !ensure_runtime(where)) return;
    if (!all_device({in_vec, out_act})) {
        set_error(where, "in_vec and out_act must be device memory", -1);
        return;
    }
    const size_t wb = row_bytes(ggml_type, in_dim) * static_cast<size_t>(ffn_dim);
    const uint8_t* ws[2] = {device_weights(gate_weights, wb, where), nullptr};
    if (!ws[0]) return;
    ws[1] = device_weights(up_weights, wb, where);
    if (!ws[1]) return;
    const int32_t ns[2] = {ffn_dim, ffn_dim};
    GemvFusion f;
    f.x = in_vec;
    f.act = out_act;
    hipError_t e = launch_gemv_fused(ggml_type, 2, ws, ns, in_dim, nullptr, f, g_rt.stream);
    if (e != hipErrorNotSupported) {
        check(e, where);
        return;
    }
    // the separate kernels, same results
    if (!g_rt.y.ensure(sizeof(float) * 2 * static_cast<size_t>(ffn_dim), where)) return;
    float* ys[2] = {g_rt.y.as<float>(), g_rt.y.as<float>() + ffn_dim};
    check(launch_gemv_multi(ggml_type, 2, ws, ns, in_vec, in_dim, ys, g_rt.stream), where) &&
        check(launch_swiglu(ys[0], ys[1], ffn_dim, out_act, g_rt.stream), where);
}

// ---- native decode step --------------------------------------------------
// One token of GNCXStreamer:forward_token (lua/gncx_streamer.lua:759-965)
// for a Qwen3/Llama-shaped model, every launch issued from here: per layer
//   Q/K/V      one launch, x = RMSNorm(h + delta) * attn_norm in its prologue
//              (delta: the previous layer's down projection; none at layer 0)
//   attention  Q/K head RMSNorm + RoPE prologue, KV row store, split-K scan,
//              merge (gncx_hip_attention_step_fused)
//   O          matvec of the attention output
//   gate/up    one launch, x = RMSNorm(h + O) * ffn_norm in its prologue,
//              act = SiLU(gate) * up in its epilogue
//   down       matvec of act
// then the final residual add + RMSNorm and the tied lm_head.  The residual
// stream alternates between the two hidden buffers (a prologue reads h while
// work-group 0 writes h + delta to the other one).  Shapes the fused launches
// do not take run the separate kernels with the same results.

namespace {

// device addresses of one model's tensors, resolved once per (base, table)
struct DecodePlan {
    const uint8_t* base = nullptr;
    std::vector<GNCXDecodeLayer> layers;
    GNCXDecodeTensor embd{}, onorm{};
    int32_t dims[7] = {};
    struct Layer {
        const float *attn_norm, *q_norm, *k_norm, *ffn_norm;
        const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    };
    std::vector<Layer> dev;
    const uint8_t* embd_dev = nullptr;
    const float* onorm_dev = nullptr;
    GNCXDecodeState state{};
    std::vector<float*> kc, vc;
    bool state_ok = false;
} g_plan;

bool plan_model(const GNCXDecodeModel& m, const char* where) {
    DecodePlan& p = g_plan;
    const int32_t dims[7] = {m.n_layers, m.embed, m.n_heads, m.n_kv_heads, m.head_dim, m.ffn, m.vocab};
    const bool same = p.base == m.base && p.dev.size() == static_cast<size_t>(m.n_layers) &&
                      std::memcmp(p.dims, dims, sizeof(dims)) == 0 &&
                      std::memcmp(&p.embd, &m.token_embd, sizeof(GNCXDecodeTensor)) == 0 &&
                      std::memcmp(&p.onorm, &m.output_norm, sizeof(GNCXDecodeTensor)) == 0 &&
                      std::memcmp(p.layers.data(), m.layers, sizeof(GNCXDecodeLayer) * m.n_layers) == 0;
    if (same) return true;
    p.base = nullptr;
    p.dev.clear();
    const size_t E = m.embed, Q = static_cast<size_t>(m.n_heads) * m.head_dim,
                 KV = static_cast<size_t>(m.n_kv_heads) * m.head_dim, F = m.ffn, HD = m.head_dim;
    auto mat = [&](const GNCXDecodeTensor& t, size_t rows, size_t cols) -> const uint8_t* {
        if (!type_supported(t.ggml_type)) {
            set_error(where, "unsupported ggml_type for a layer matrix", -1);
            return nullptr;
        }
        return device_weights(m.base + t.offset, row_bytes(t.ggml_type, static_cast<int32_t>(cols)) * rows, where);
    };
    auto vec = [&](const GNCXDecodeTensor& t, size_t n) -> const float* {
        return reinterpret_cast<const float*>(device_weights(m.base + t.offset, sizeof(float) * n, where));
    };
    std::vector<DecodePlan::Layer> dev(m.n_layers);
    for (int32_t l = 0; l < m.n_layers; ++l) {
        const GNCXDecodeLayer& L = m.layers[l];
        DecodePlan::Layer& d = dev[l];
        d.attn_norm = vec(L.attn_norm, E);
        d.ffn_norm = vec(L.ffn_norm, E);
        d.q_norm = m.qk_norm ? vec(L.attn_q_norm, HD) : nullptr;
        d.k_norm = m.qk_norm ? vec(L.attn_k_norm, HD) : nullptr;
        d.q = mat(L.attn_q, Q, E);
        d.k = mat(L.attn_k, KV, E);
        d.v = mat(L.attn_v, KV, E);
        d.o = mat(L.attn_output, E, Q);
        d.gate = mat(L.ffn_gate, F, E);
        d.up = mat(L.ffn_up, F, E);
        d.down = mat(L.ffn_down, E, F);
        if (!d.attn_norm || !d.ffn_norm || (m.qk_norm && (!d.q_norm || !d.k_norm)) || !d.q || !d.k || !d.v || !d.o ||
            !d.gate || !d.up || !d.down)
            return false;
    }
    const uint8_t* embd = mat(m.token_embd, static_cast<size_t>(m.vocab), E);
    const float* onorm = vec(m.output_norm, E);
    if (!embd || !onorm) return false;
    p.layers.assign(m.layers, m.layers + m.n_layers);
    p.embd = m.token_embd;
    p.onorm = m.output_norm;
    std::memcpy(p.dims, dims, sizeof(dims));
    p.dev = std::move(dev);
    p.embd_dev = embd;
    p.onorm_dev = onorm;
    p.base = m.base;
    return true;
}

// every buffer of the state must be device memory (checked when it changes)
bool plan_state(const GNCXDecodeModel& m, const GNCXDecodeState& s, const char* where) {
    DecodePlan& p = g_plan;
    const bool same = p.state_ok && std::memcmp(&p.state, &s, sizeof(s)) == 0 &&
                      std::memcmp(p.kc.data(), s.k_cache, sizeof(float*) * m.n_layers) == 0 &&
                      std::memcmp(p.vc.data(), s.v_cache, sizeof(float*) * m.n_layers) == 0 &&
                      p.kc.size() == static_cast<size_t>(m.n_layers);
    if (same) return true;
    p.state_ok = false;
    if (!s.k_cache || !s.v_cache || s.max_seq <= 0) {
        set_error(where, "KV cache tables and max_seq are required", -1);
        return false;
    }
    const void* need[] = {s.hidden[0], s.hidden[1], s.q, s.k, s.v, s.attn, s.proj, s.normed,
                          s.gate, s.up, s.act, s.logits, s.token};
    for (const void* b : need)
        if (!b || !is_device_ptr(b)) {
            set_error(where, "every state buffer must be device memory", -1);
            return false;
        }
    if (s.token_log && !is_device_ptr(s.token_log)) {
        set_error(where, "token_log must be device memory", -1);
        return false;
    }
    for (int32_t l = 0; l < m.n_layers; ++l)
        if (!s.k_cache[l] || !s.v_cache[l] || !is_device_ptr(s.k_cache[l]) || !is_device_ptr(s.v_cache[l])) {
            set_error(where, "every KV cache must be device memory", -1);
            return false;
        }
    p.state = s;
    p.kc.assign(s.k_cache, s.k_cache + m.n_layers);
    p.vc.assign(s.v_cache, s.v_cache + m.n_layers);
    p.state_ok = true;
    return true;
}

}  // namespace

namespace {

// The scratch of one step: the attention split-K partials (reused by every
// layer, stream-ordered) and the argmax partials.
struct StepScratch {
    void* attn;
    size_t attn_bytes;
    void* argmax;
    size_t argmax_bytes;
};

// The whole step.  fixed == nullptr: scratch from the library's growable
// device buffers (and host weights uploaded once, as everywhere).  fixed !=
// nullptr: the caller's scratch, and nothing is allocated: the weights must
// already be device memory, and a step needing more scratch than given is
// rejected before anything is enqueued.
int decode_step_impl(const GNCXDecodeModel* model, const GNCXDecodeState* state, int32_t token_id, int32_t pos,
                     int32_t greedy, const StepScratch* fixed, const char* where) {
    if (!model || !state || !model->layers || !model->base) {
        set_error(where, "model (with base and layers) and state are required", -1);
        return -1;
    }
    const GNCXDecodeModel& m = *model;
    const GNCXDecodeState& s = *state;
    if (m.n_layers <= 0 || m.embed <= 0 || m.n_heads <= 0 || m.n_kv_heads <= 0 || m.head_dim <= 0 || m.ffn <= 0 ||
        m.vocab <= 0 || m.n_heads % m.n_kv_heads != 0) {
        set_error(where, "invalid model shape", -1);
        return -1;
    }
    if (pos < 0 || pos >= s.max_seq) {
        set_error(where, "position outside the KV cache", -1);
        return -1;
    }
    if (token_id >= m.vocab) {
        set_error(where, "token id past the vocabulary", -1);
        return -1;
    }
    if (!ensure_runtime(where)) return -1;
    if (fixed && !is_device_ptr(m.base)) {
        set_error(where, "the weights (model->base) must be device memory: this entry point uploads nothing", -1);
        return -1;
    }
    if (!plan_model(m, where) || !plan_state(m, s, where)) return -1;
    const DecodePlan& P = g_plan;
    const hipStream_t st = g_rt.stream;
    const int32_t E = m.embed, Q = m.n_heads * m.head_dim, KV = m.n_kv_heads * m.head_dim, F = m.ffn;

    RopeTable rope;
    const RopeTable* rp = nullptr;
    if (m.rope_base > 0.0f) {
        if (!rope_table(pos, m.head_dim, m.rope_base, nullptr, rope)) {
            set_error(where, "head_dim must be even and at most 512", -1);
            return -1;
        }
        rp = &rope;
    }
    StepScratch sc{};
    if (fixed) {
        // the split plan of this step's attention (the same for every layer)
        AttnArgs probe{};
        probe.pos = pos;
        probe.n_heads = m.n_heads;
        probe.n_kv_heads = m.n_kv_heads;
        probe.head_dim = m.head_dim;
        probe.write_kv = 1;
        probe.norm_qk = m.qk_norm ? 1 : 0;
        probe.rope = rp;
        const size_t need_attn = attention_workspace_need(probe);
        const size_t need_argmax = greedy ? argmax_workspace_bytes(m.vocab) : 0;
        if (need_attn > fixed->attn_bytes || need_argmax > fixed->argmax_bytes) {
            char msg[192];
            std::snprintf(msg, sizeof(msg),
                          "this step needs %zu B of attention and %zu B of argmax scratch; the fixed scratch holds "
                          "%zu and %zu B",
                          need_attn, need_argmax, fixed->attn_bytes, fixed->argmax_bytes);
            set_error(where, msg, static_cast<int>(hipErrorInvalidValue));
            return -1;
        }
        sc = *fixed;
    } else {
        if (!g_rt.ws.ensure(attention_workspace_bytes(m.n_heads, m.head_dim, pos + 1), where)) return -1;
        sc.attn = g_rt.ws.p;
        sc.attn_bytes = g_rt.ws.cap;
        if (greedy) {
            if (!g_rt.aux.ensure(argmax_workspace_bytes(m.vocab), where)) return -1;
            sc.argmax = g_rt.aux.p;
            sc.argmax_bytes = g_rt.aux.cap;
        }
    }

    // embedding row of the token (cpp:693-760), into hidden[0]
    int cur = 0;
    float* H[2] = {s.hidden[0], s.hidden[1]};
    if (token_id >= 0) {
        if (!check(launch_fetch_embedding(m.token_embd.ggml_type, P.embd_dev, token_id, E, 1.0f, H[0], st), where))
            return -1;
    } else if (!check(launch_fetch_embedding_dev(m.token_embd.ggml_type, P.embd_dev, s.token, m.vocab, E, 1.0f, H[0],
                                                 st),
                      where)) {
        return -1;
    }

    // x = RMSNorm(H[cur] + delta) * gamma feeding `count` matrices; the new
    // residual lands in H[cur ^ 1] when delta is given
    auto norm_matvec = [&](const float* delta, const float* gamma, int32_t count, const uint8_t* const* ws,
                           const int32_t* ns, int32_t type, float* const* ys, float* act) -> bool {
        GemvFusion f;
        f.h = H[cur];
        f.r = delta;
        f.gamma = gamma;
        f.eps = m.eps;
        f.h_out = delta ? H[cur ^ 1] : nullptr;
        f.act = act;
        hipError_t e = launch_gemv_fused(type, count, ws, ns, E, act ? nullptr : ys, f, st);
        if (e == hipSuccess) {
            if (delta) cur ^= 1;
            return true;
        }
        if (e != hipErrorNotSupported) return check(e, where);
        if (delta) {
            if (!check(launch_add_rmsnorm(H[cur], delta, gamma, E, m.eps, s.normed, st), where)) return false;
        } else if (!check(launch_rmsnorm(H[cur], gamma, 1, E, m.eps, s.normed, st), where)) {
            return false;
        }
        if (!act) return check(launch_gemv_multi(type, count, ws, ns, s.normed, E, ys, st), where);
        float* gu[2] = {s.gate, s.up};
        return check(launch_gemv_multi(type, 2, ws, ns, s.normed, E, gu, st), where) &&
               check(launch_swiglu(s.gate, s.up, F, act, st), where);
    };

    const float* delta = nullptr;
    for (int32_t l = 0; l < m.n_layers; ++l) {
        const GNCXDecodeLayer& L = m.layers[l];
        const DecodePlan::Layer& d = P.dev[l];
        // Q / K / V (one launch when the three share a type)
        if (L.attn_k.ggml_type == L.attn_q.ggml_type && L.attn_v.ggml_type == L.attn_q.ggml_type) {
            const uint8_t* ws[3] = {d.q, d.k, d.v};
            const int32_t ns[3] = {Q, KV, KV};
            float* ys[3] = {s.q, s.k, s.v};
            if (!norm_matvec(delta, d.attn_norm, 3, ws, ns, L.attn_q.ggml_type, ys, nullptr)) return -1;
        } else {
            const uint8_t* w1[1] = {d.q};
            const int32_t n1[1] = {Q};
            float* y1[1] = {s.q};
            if (!norm_matvec(delta, d.attn_norm, 1, w1, n1, L.attn_q.ggml_type, y1, nullptr)) return -1;
            // the normalised x again for K and V: from the updated residual, no delta
            const uint8_t* wk[1] = {d.k};
            const int32_t nk[1] = {KV};
            float* yk[1] = {s.k};
            if (!norm_matvec(nullptr, d.attn_norm, 1, wk, nk, L.attn_k.ggml_type, yk, nullptr)) return -1;
            const uint8_t* wv[1] = {d.v};
            float* yv[1] = {s.v};
            if (!norm_matvec(nullptr, d.attn_norm, 1, wv, nk, L.attn_v.ggml_type, yv, nullptr)) return -1;
        }
        // attention step with the Q/K head norm + RoPE prologue
        AttnArgs a{};
        a.q = s.q;
        a.k_new = s.k;
        a.v_new = s.v;
        a.k_cache = s.k_cache[l];
        a.v_cache = s.v_cache[l];
        a.out = s.attn;
        a.pos = pos;
        a.n_heads = m.n_heads;
        a.n_kv_heads = m.n_kv_heads;
        a.head_dim = m.head_dim;
        a.scale = m.attn_scale;
        a.sliding_window = 0;
        a.write_kv = 1;
        a.norm_qk = m.qk_norm ? 1 : 0;
        a.q_gamma = d.q_norm;
        a.k_gamma = d.k_norm;
        a.eps = m.eps;
        a.rope = rp;
        if (!check(launch_attention(a, sc.attn, sc.attn_bytes, st), where)) return -1;
        // O projection
        if (!check(launch_gemv(L.attn_output.ggml_type, d.o, s.attn, Q, E, s.proj, st), where)) return -1;
        // gate / up with SwiGLU
        if (L.ffn_up.ggml_type == L.ffn_gate.ggml_type) {
            const uint8_t* ws[2] = {d.gate, d.up};
            const int32_t ns[2] = {F, F};
            float* ys[2] = {s.gate, s.up};
            if (!norm_matvec(s.proj, d.ffn_norm, 2, ws, ns, L.ffn_gate.ggml_type, ys, s.act)) return -1;
        } else {
            const uint8_t* wg[1] = {d.gate};
            const int32_t nf[1] = {F};
            float* yg[1] = {s.gate};
            if (!norm_matvec(s.proj, d.ffn_norm, 1, wg, nf, L.ffn_gate.ggml_type, yg, nullptr)) return -1;
            const uint8_t* wu[1] = {d.up};
            float* yu[1] = {s.up};
            if (!norm_matvec(nullptr, d.ffn_norm, 1, wu, nf, L.ffn_up.ggml_type, yu, nullptr) ||
                !check(launch_swiglu(s.gate, s.up, F, s.act, st), where))
                return -1;
        }
        // down projection; its output is the next prologue's delta
        if (!check(launch_gemv(L.ffn_down.ggml_type, d.down, s.act, F, E, s.proj, st), where)) return -1;
        delta = s.proj;
    }
    // final residual add + RMSNorm, then the tied lm_head (cpp:1713-1732)
    if (!check(launch_add_rmsnorm(H[cur], delta, P.onorm_dev, E, m.eps, s.normed, st), where)) return -1;
    if (!check(launch_gemv(m.token_embd.ggml_type, P.embd_dev, s.normed, E, m.vocab, s.logits, st), where)) return -1;
    if (greedy && !check(launch_argmax(s.logits, m.vocab, s.token, s.token_log ? s.token_log + pos : nullptr,
                                       sc.argmax, sc.argmax_bytes, st),
                         where))
        return -1;
    return 0;
}

}  // namespace

GNCX_API int gncx_hip_decode_step(const GNCXDecodeModel* model, const GNCXDecodeState* state, int32_t token_id,
                                  int32_t pos, int32_t greedy) {
    std::lock_guard<CallLock> lk(g_mu);
    return decode_step_impl(model, state, token_id, pos, greedy, nullptr, "gncx_hip_decode_step");
}

// gncx_hip_decode_step with its scratch in this GPU's fixed device array
// (noalloc.hip) and no allocation of any kind: weights and every state
// buffer must already be device memory.  Calls that overlap on one GPU share
// the array and race.
GNCX_API int gncx_hip_decode_step_noalloc(const GNCXDecodeModel* model, const GNCXDecodeState* state,
                                          int32_t token_id, int32_t pos, int32_t greedy) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_decode_step_noalloc";
    if (!ensure_runtime(where)) return -1;
    void* base = nullptr;
    if (!check(noalloc_scratch(g_rt.device, &base), where)) return -1;
    StepScratch fixed{static_cast<char*>(base) + kNoAllocArgmaxBytes, kNoAllocScratchBytes - kNoAllocArgmaxBytes,
                      base, kNoAllocArgmaxBytes};
    return decode_step_impl(model, state, token_id, pos, greedy, &fixed, where);
}

// index of the first largest logit, on the device (the greedy pick of the
// streamer's sampler without its repetition penalty, lua/gncx_streamer.lua:1229-1272)
GNCX_API void gncx_hip_argmax(const float* values, int32_t n, int32_t* out_index) {
    std::lock_guard<CallLock> lk(g_mu);
    const char* where = "gncx_hip_argmax";
    if (!values || !out_index || n <= 0 || !ensure_runtime(where)) return;
    if (!all_device({values, out_index})) {
        set_error(where, "values and out_index must be device memory", -1);
        return;
    }
    if (!g_rt.aux.ensure(argmax_workspace_bytes(n), where)) return;
    check(launch_argmax(values, n, out_index, nullptr, g_rt.aux.p, g_rt.aux.cap, g_rt.stream), where);
}

// ---- weight files and host buffers ------------------------------------
// The reference's loader maps the GGUF read-only (cpp:327-404) and copies the
// per-layer tensors, scratch vectors and KV caches into 2 MB-aligned,
// "bank/L1-set coloured" anonymous memory (cpp:434-612).  Here the same entry
// points hand out page-locked host memory from hipHostMalloc when a HIP
// device is visible, so the one-time weight upload and every host KV-row or
// activation transfer runs at full DMA rate without a bounce, and plain
// anonymous pages otherwise.  The colour is kept: each buffer starts at an
// address whose bits 14..16 and 6..11 are the requested bank and L1-set slots
// (only 6..11 above 64 MiB, cpp:526-528), so the bank / set getters report
// what the reference reports.  Releasing a mapping or a buffer, or copying
// into one, drops the device twins of the weights and KV caches inside it.
namespace {

struct MappedFile {
    int fd = -1;
    const uint8_t* base = nullptr;
    size_t bytes = 0;
};

uint32_t g_alloc_seq = 0;  // gncx_ram_alloc's rotating colour (cpp:553-559)

bool device_visible() {
    static int n = -1;
    if (n < 0) {
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            n = 0;
        }
    }
    return n > 0;
}

// Device twins of host ranges overlapping [lo, hi) are out of date.
void forget_range(uintptr_t lo, uintptr_t hi) {
    if (lo >= hi) return;
    std::vector<uintptr_t> drop;
    for (const auto& kv : g_rt.weights)
        if (kv.first < hi && kv.first + kv.second.bytes > lo) drop.push_back(kv.first);
    for (uintptr_t k : drop) forget_weight(k);
    drop.clear();
    for (const auto& kv : g_rt.kv) {
        const size_t rows = static_cast<size_t>(std::max<int32_t>(kv.second.valid_rows, 1));
        if (kv.first < hi && kv.first + rows * kv.second.kv_dim * sizeof(float) > lo) drop.push_back(kv.first);
    }
    for (uintptr_t k : drop) forget_kv(k);
}

// Smallest 64 B-aligned address >= p whose bits under `mask` equal `want`.
uintptr_t coloured(uintptr_t p, uintptr_t mask, uintptr_t want) {
    uintptr_t a = (p + 63) & ~static_cast<uintptr_t>(63);
    while ((a & mask) != want) a += 64;
    return a;
}

}  // namespace

// cpp:327-384.  Read-only private mapping with read-ahead advice; null when
// the file cannot be opened or mapped.
GNCX_API void* gncx_gla_map_readonly(const char* filepath, size_t* out_size) {
    if (!filepath) return nullptr;
    const int fd = open(filepath, O_RDONLY);
    if (fd < 0) return nullptr;
    struct stat st{};
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return nullptr;
    }
    const size_t bytes = static_cast<size_t>(st.st_size);
    void* p = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
        close(fd);
        return nullptr;
    }
    (void)posix_fadvise(fd, 0, static_cast<off_t>(bytes), POSIX_FADV_WILLNEED);
    (void)madvise(p, bytes, MADV_WILLNEED);
    auto* h = new MappedFile{fd, static_cast<const uint8_t*>(p), bytes};
    {
        std::lock_guard<CallLock> lk(g_mu);
        g_maps[reinterpret_cast<uintptr_t>(p)] = bytes;
    }
    if (out_size) *out_size = bytes;
    return h;
}

// cpp:386-389
GNCX_API const uint8_t* gncx_gla_get_base_ptr(void* opaque_handle) {
    return opaque_handle ? static_cast<MappedFile*>(opaque_handle)->base : nullptr;
}

// cpp:391-404
GNCX_API void gncx_gla_unmap(void* opaque_handle) {
    if (!opaque_handle) return;
    auto* h = static_cast<MappedFile*>(opaque_handle);
    {
        std::lock_guard<CallLock> lk(g_mu);
        forget_range(reinterpret_cast<uintptr_t>(h->base), reinterpret_cast<uintptr_t>(h->base) + h->bytes);
        g_maps.erase(reinterpret_cast<uintptr_t>(h->base));
    }
    munmap(const_cast<uint8_t*>(h->base), h->bytes);
    close(h->fd);
    delete h;
}

// cpp:617-667 (POSIX branch): read-ahead advice for the pages of a range.
GNCX_API void gncx_gla_prefetch_range(const uint8_t* mmap_base, size_t offset, size_t num_bytes) {
    if (!mmap_base || num_bytes == 0) return;
    const uintptr_t a = reinterpret_cast<uintptr_t>(mmap_base + offset);
    const uintptr_t page = a & ~static_cast<uintptr_t>(4095);
    (void)madvise(reinterpret_cast<void*>(page), num_bytes + (a - page), MADV_WILLNEED);
}

// cpp:481-551.  Colour slots: bank = (d * R_odd + k) mod 8 and L1 set =
// (3 d R_odd + 7 k) mod 64 with R_odd = (R | 1) mod 8 (cpp:485-487).
GNCX_API void* gncx_ram_alloc_colored(size_t total_bytes, uint8_t k, uint8_t d, uint8_t R) {
    if (total_bytes == 0) total_bytes = 64;
    const uint32_t r_odd = (R | 1u) & 7u;
    const uint32_t bank = (static_cast<uint32_t>(d) * r_odd + k) & 7u;
    const uint32_t set = (static_cast<uint32_t>(d) * r_odd * 3u + static_cast<uint32_t>(k) * 7u) & 63u;
    const bool full = total_bytes <= (size_t{64} << 20);
    const uintptr_t mask = full ? 0x1ffc0 : 0xfc0;
    const uintptr_t want = (full ? static_cast<uintptr_t>(bank) << 14 : 0) | (static_cast<uintptr_t>(set) << 6);
    const size_t block_bytes = total_bytes + (size_t{128} << 10) + 64;
    auto* h = new HostBuffer();
    std::lock_guard<CallLock> lk(g_mu);
    if (!lazy_mode() && device_visible() && ensure_runtime("gncx_ram_alloc_colored")) {
        void* p = nullptr;
        if (hipHostMalloc(&p, block_bytes, hipHostMallocDefault) == hipSuccess && p) {
            h->block = p;
            h->pinned = true;
        } else {
            (void)hipGetLastError();
        }
    }
    if (!h->block) {
        void* p = mmap(nullptr, block_bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
        if (p == MAP_FAILED) {
            delete h;
            return nullptr;
        }
        h->block = p;
    }
    h->block_bytes = block_bytes;
    const uintptr_t a = coloured(reinterpret_cast<uintptr_t>(h->block), mask, want);
    h->ptr = reinterpret_cast<uint8_t*>(a);
    h->bytes = total_bytes;
    h->bank = static_cast<uint8_t>((a >> 14) & 7u);
    h->l1_set = static_cast<uint8_t>((a >> 6) & 63u);
    g_bufs[reinterpret_cast<uintptr_t>(h->block)] = h;
    return h;
}

// cpp:553-559: colour (k, d, R) = (s mod 4, s mod 64, {1,3,5,7}[s mod 4]) of
// the s-th call.
GNCX_API void* gncx_ram_alloc(size_t total_bytes) {
    static constexpr uint8_t kRot[4] = {1, 3, 5, 7};
    uint32_t seq;
    {
        std::lock_guard<CallLock> lk(g_mu);
        seq = g_alloc_seq++;
    }
    return gncx_ram_alloc_colored(total_bytes, static_cast<uint8_t>(seq & 3u), static_cast<uint8_t>(seq & 63u),
                                  kRot[seq & 3u]);
}

// cpp:561-574
GNCX_API uint8_t* gncx_ram_get_ptr(void* ram_handle) {
    return ram_handle ? static_cast<HostBuffer*>(ram_handle)->ptr : nullptr;
}
GNCX_API uint8_t gncx_ram_get_ddr3_bank(void* ram_handle) {
    return ram_handle ? static_cast<HostBuffer*>(ram_handle)->bank : 0;
}
GNCX_API uint8_t gncx_ram_get_l1_set(void* ram_handle) {
    return ram_handle ? static_cast<HostBuffer*>(ram_handle)->l1_set : 0;
}

// cpp:576-600
GNCX_API void gncx_ram_free(void* ram_handle) {
    if (!ram_handle) return;
    auto* h = static_cast<HostBuffer*>(ram_handle);
    std::lock_guard<CallLock> lk(g_mu);
    forget_range(reinterpret_cast<uintptr_t>(h->ptr), reinterpret_cast<uintptr_t>(h->ptr) + h->bytes);
    g_bufs.erase(reinterpret_cast<uintptr_t>(h->block));
    g_readbacks.erase(std::remove(g_readbacks.begin(), g_readbacks.end(), h), g_readbacks.end());
    if (h->twin) {
        // queued work may still use the device copy
        (void)hipStreamSynchronize(g_rt.stream);
        (void)hipFree(h->twin);
    }
    if (h->staged_ev) (void)hipEventDestroy(h->staged_ev);
    if (h->stage) (void)hipHostFree(h->stage);
    if (h->pinned) {
        // pending deferred write-backs never target freed memory: they are
        // flushed before the call that queued them returns
        (void)hipHostFree(h->block);
    } else {
        munmap(h->block, h->block_bytes);
    }
    delete h;
}

// cpp:602-612
GNCX_API void gncx_ram_copy_chunk(void* ram_handle, size_t dst_offset, const uint8_t* src_base, size_t src_offset,
                                  size_t num_bytes) {
    if (!ram_handle || !src_base || num_bytes == 0) return;
    auto* h = static_cast<HostBuffer*>(ram_handle);
    std::lock_guard<CallLock> lk(g_mu);
    const uintptr_t dst = reinterpret_cast<uintptr_t>(h->ptr) + dst_offset;
    forget_range(dst, dst + num_bytes);
    if (h->twin && !make_host(*h, "gncx_ram_copy_chunk")) return;
    std::memcpy(h->ptr + dst_offset, src_base + src_offset, num_bytes);
}

// Lazy coherence of the library's host buffers on (1) or off (0); any other
// value only reports.  Returns the mode before the call.  It applies to
// buffers allocated while it is on; turning it off brings every buffer back
// to the host (current and read-write).
GNCX_API int gncx_hip_set_host_coherence(int lazy) {
    std::lock_guard<CallLock> lk(g_mu);
    const int before = lazy_mode() ? 1 : 0;
    if (lazy == 0 && before == 1)
        for (auto& kv : g_bufs)
            if (kv.second->twin) (void)make_host(*kv.second, "gncx_hip_set_host_coherence");
    if (lazy == 0 || lazy == 1) g_lazy = lazy;
    return before;
}

// Make the host buffer holding p (every buffer when p is null) current and
// read-write on the host, e.g. before handing it to a system call.
GNCX_API void gncx_hip_host_flush(const void* p) {
    std::lock_guard<CallLock> lk(g_mu);
    if (!p) {
        for (auto& kv : g_bufs)
            if (kv.second->twin) (void)make_host(*kv.second, "gncx_hip_host_flush");
        return;
    }
    HostBuffer* b = buffer_at(reinterpret_cast<uintptr_t>(p));
    if (b && b->twin) (void)make_host(*b, "gncx_hip_host_flush");
}

// ---- exports outside the decode path ----------------------------------
// The reference's LoRA / MeZO training primitives, its embedding-model
// helpers and the layer visualisation point (cpp:2129-2654) are exported
// under their names and signatures so that every binding of the reference
// resolves, but they are not provided: a call records the error, prints it
// and leaves every output untouched (float results are 0).
namespace {
void not_provided(const char* where) {
    std::lock_guard<CallLock> lk(g_mu);
    set_error(where, "not provided by this library (outside the quantized decode path); outputs untouched", -1);
}
}  // namespace

GNCX_API void gncx_lora_init_adapter(float*, float*, int32_t, int32_t, int32_t, uint64_t) {
    not_provided("gncx_lora_init_adapter");
}
GNCX_API void gncx_lora_forward_add(const float*, const float*, const float*, int32_t, int32_t, int32_t, float,
                                    float*) {
    not_provided("gncx_lora_forward_add");
}
GNCX_API void gncx_lora_backward_step(const float*, const float*, float*, float*, float*, int32_t, int32_t, int32_t,
                                      float, float, float) {
    not_provided("gncx_lora_backward_step");
}
GNCX_API void gncx_mezo_perturb_params(float*, int32_t, uint64_t, float) { not_provided("gncx_mezo_perturb_params"); }
GNCX_API void gncx_mezo_update_params(float*, int32_t, uint64_t, float, float, float) {
    not_provided("gncx_mezo_update_params");
}
GNCX_API float gncx_cross_entropy_loss(const float*, int32_t, int32_t, float*) {
    not_provided("gncx_cross_entropy_loss");
    return 0.0f;
}
GNCX_API void gncx_project_layer_3d_point(int32_t, int32_t, const GNCXCompactToken*, const float*, int32_t,
                                          GNCXLayer3DPoint*) {
    not_provided("gncx_project_layer_3d_point");
}
GNCX_API float gncx_cosine_similarity(const float*, const float*, int32_t) {
    not_provided("gncx_cosine_similarity");
    return 0.0f;
}
GNCX_API void gncx_vector_l2_normalize(float*, int32_t) { not_provided("gncx_vector_l2_normalize"); }
GNCX_API void gncx_mean_pooling(const float*, int32_t, int32_t, float*) { not_provided("gncx_mean_pooling"); }
GNCX_API void gncx_bidirectional_attention_gqa(const float*, const float*, const float*, int32_t, int32_t, int32_t,
                                               int32_t, float, float*) {
    not_provided("gncx_bidirectional_attention_gqa");
}
GNCX_API void gncx_bidirectional_attention(const float*, const float*, const float*, int32_t, int32_t, int32_t,
                                           float, float*) {
    not_provided("gncx_bidirectional_attention");
}
