// attention.hip -- GQA/MQA/SWA decode attention step for gfx950.
//
// Semantics of the reference's gncx_mqa_attention_step_ext
// (csrc/gncx_llm_kernels.cpp:1887-1994): optionally store k_new/v_new at row
// `pos` of the layer's KV cache, then for every query head h (KV head
// h / (n_heads / n_kv_heads)) softmax((q . k_t) * scale) over the window
// [max(0, pos - sw + 1), pos] and o = sum_t p_t v_t with the reference's
// normaliser 1 / (sum + 1e-12).
//
// MI355X design (flash-decoding): the window is cut into chunks; one
// work-group owns (KV head, chunk) and serves all query heads of its group, so
// each KV row is read from HBM once (the reference re-reads it per query
// head).  A token row of one KV head is read by hd/16 lanes with coalesced
// 16-byte loads; scores go to LDS, each wave reduces one head's max/sum, the
// V pass accumulates in registers and the waves combine through LDS.  A
// second small kernel merges the chunk partials with the log-sum-exp rule.
//
// Optional fused prologue (cpp:895-953 per-head RMSNorm, then cpp:1797-1862
// NEOX RoPE with a host-computed cos/sin table) is applied to q and k_new in
// LDS before the scan, with the same arithmetic as the stand-alone kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "gncx_device.h"
#include "gncx_launch.h"

namespace gncx {
namespace {

using namespace dev;

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kHeadBlock = 4;     // query heads handled per pass (one wave each in the softmax)
constexpr int kMaxChunk = 1024;   // tokens per work-group
// Work-groups a call aims for: windows that fit 32-token chunks at kTargetGroups
// keep those (one pass per work-group, K/V loaded up front); longer windows
// take about half as many, longer chunks.  Measured per call, GQA 32/8 x 128
// (chunk + merge), 1024 / 512 target work-groups: ctx 2100: 13.8 / 18.0 us;
// ctx 4096: 16.1 / 17.3; ctx 8192: 27.6 / 26.5; ctx 16384: 42.5 / 34.5;
// ctx 32768: 63.2 / 56.4; ctx 65536: 110 / 101; GQA 32/4 ctx 32768: 60.7 /
// 52.6 us.
constexpr int kTargetGroups = 1024;
constexpr int kTargetGroupsLong = 512;

struct AttnParams {
    const float* q;
    const float* k_new;
    const float* v_new;
    float* k_cache;
    float* v_cache;
    float* part_o;  // [n_split][n_heads][hd]
    float* part_ml; // [n_split][n_heads][2]  (max, sum)
    float* q_out;
    float* k_out;
    const float* q_gamma;
    const float* k_gamma;
    int32_t pos, n_heads, n_kv, t0, t1, chunk, use_new, norm_qk, has_rope;
    float scale, eps;
    RopeTable rope;
};


// Per-head RMSNorm then RoPE of one head held in LDS; one wave.
template <int HD>
__device__ void prologue_head(float* v, const float* gamma, bool norm, bool rope, float eps,
                              const float* __restrict rc, const float* __restrict rs, int lane) {
#pragma clang fp contract(off)
    if (norm) {
        const float inv = head_inv_rms(v, HD, eps, lane);
        for (int i = lane; i < HD; i += 64) {
            const float x = v[i] * inv;
            v[i] = gamma ? x * gamma[i] : x;
        }
    }
    if (rope) {
        constexpr int H = HD / 2;
        for (int i = lane; i < H; i += 64) {
            const float x1 = v[i], x2 = v[i + H];
            v[i] = x1 * rc[i] - x2 * rs[i];
            v[i + H] = x2 * rc[i] + x1 * rs[i];
        }
    }
}

// The prologue's per-lane operands (norm weights of the elements a lane
// normalises, the RoPE rows of the pairs it rotates), loaded into registers
// with the other small operands before the K/V rows, so the prologue waits
// for no memory.
template <int HD>
struct ProRegs {
    static constexpr int NE = HD / 64 > 0 ? HD / 64 : 1;  // elements per lane
    static constexpr int NR = (HD / 2 + 63) / 64;         // rotated pairs per lane
    float gq[NE], gk[NE], c[NR], s[NR];
    // unconditional loads (a missing weight reads q, whose first HD values
    // exist, and is never used: prologue_head_r takes has_gamma): with no load
    // behind a branch the compiler counts them exactly and waits for these
    // alone, not for the K/V rows issued after them
    __device__ __forceinline__ void load(const AttnParams& p, int lane) {
        const float* gqp = p.q_gamma ? p.q_gamma : p.q;
        const float* gkp = p.k_gamma ? p.k_gamma : p.q;
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int i = lane + 64 * e < HD ? lane + 64 * e : 0;
            gq[e] = gqp[i];
            gk[e] = gkp[i];
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int i = lane + 64 * r < HD / 2 ? lane + 64 * r : 0;
            c[r] = p.rope.c[i];
            s[r] = p.rope.s[i];
        }
    }
};

// prologue_head with the operands in registers; gamma == nullptr means no weight
template <int HD>
__device__ __forceinline__ void prologue_head_r(float* v, const float* g, bool has_gamma, bool norm, bool rope,
                                                float eps, const ProRegs<HD>& pr, int lane) {
#pragma clang fp contract(off)
    if (norm) {
        const float inv = head_inv_rms(v, HD, eps, lane);
#pragma unroll
        for (int e = 0; e < ProRegs<HD>::NE; ++e) {
            const int i = lane + 64 * e;
            if (i < HD) {
                const float x = v[i] * inv;
                v[i] = has_gamma ? x * g[e] : x;
            }
        }
    }
    if (rope) {
        constexpr int H = HD / 2;
#pragma unroll
        for (int r = 0; r < ProRegs<HD>::NR; ++r) {
            const int i = lane + 64 * r;
            if (i < H) {
                const float x1 = v[i], x2 = v[i + H];
                v[i] = x1 * pr.c[r] - x2 * pr.s[r];
                v[i + H] = x2 * pr.c[r] + x1 * pr.s[r];
            }
        }
    }
}

// SHORT: the chunk fits one pass (chunk <= TPP tokens).  Each thread's K and V
// slices are then loaded at the start, ahead of q, so a work-group waits for
// HBM once instead of three times in a row (q, then K, then V after the
// softmax), and head blocks after the first re-read nothing.
template <int HD, bool SHORT>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(AttnParams p) {
    constexpr int LPT = HD / 16;          // lanes per token row (16 dims each)
    constexpr int TPP = kThreads / LPT;   // tokens per pass
    extern __shared__ __align__(16) float smem[];
    const int G = p.n_heads / p.n_kv;
    float* sc = smem;                                   // [kHeadBlock][chunk]
    float* red = sc + kHeadBlock * p.chunk;             // [kWaves][kHeadBlock][HD]
    float* qs = red + kWaves * kHeadBlock * HD;         // [G][HD]  (prologue result)
    float* ks = qs + G * HD;                            // [HD]
    float* vs = ks + HD;                                // SHORT: [TPP][HD], the chunk's V rows

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int hk = blockIdx.x;
    const int split = blockIdx.y;
    const int ta = p.t0 + split * p.chunk;
    const int tb = min(p.t1, ta + p.chunk);
    const int j = tid % LPT;       // 16-dim slice of the row
    const int ts = tid / LPT;      // token slot within a pass
    const size_t kv_dim = static_cast<size_t>(p.n_kv) * HD;
    const bool have_new = p.use_new != 0;

    // q rows of this KV head's query heads, k_new and the prologue operands
    // first: the prologue then runs while the K/V rows are still in flight.
    // Every early load is unconditional (indices clamped, pointers selected,
    // unused values replaced afterwards), so the compiler counts them exactly
    // and the prologue waits for these loads alone: a load behind a branch made
    // it wait for every load issued so far, the K/V rows included.
    constexpr int kQRegs = 8;  // q values per thread held across the K/V issue
    const int gq_n = G * HD;
    const float* qg = p.q + static_cast<size_t>(hk) * G * HD;
    float qreg[kQRegs];
#pragma unroll
    for (int u = 0; u < kQRegs; ++u) {
        const int i = tid + u * kThreads;
        qreg[u] = qg[i < gq_n ? i : gq_n - 1];
    }
    // without a new row, q (at least n_kv HD values) stands in for k_new
    const float* knp = have_new ? p.k_new : p.q;
    const float kreg = knp[static_cast<size_t>(hk) * HD + (tid < HD ? tid : 0)];  // used where have_new && tid < HD
    const bool pro = p.norm_qk || p.has_rope;
    ProRegs<HD> pr;
    if (pro) pr.load(p, lane);

    // SHORT: this thread's token is ta + ts; its K / V slices are loaded now
    // (the new token's K comes from LDS after the prologue, its V from v_new);
    // a slot past the chunk reads row ta, and neither its score nor its V row
    // is used
    // (native vectors: float4 copies are memcpys, and a V slice copied that
    // way went through scratch memory on its way to LDS)
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    float4 kpre[4];
    f32x4 vpre[4];
    const int tok0 = ta + ts;
    const bool valid0 = tok0 < tb;
    const bool new0 = have_new && tok0 == p.pos;
    if constexpr (SHORT) {
        const int tokc = valid0 ? tok0 : ta;
        const float* ksrc = p.k_cache + static_cast<size_t>(tokc) * kv_dim + static_cast<size_t>(hk) * HD;
        const float* vsrc = new0 ? p.v_new + static_cast<size_t>(hk) * HD
                                 : p.v_cache + static_cast<size_t>(tokc) * kv_dim + static_cast<size_t>(hk) * HD;
#pragma unroll
        for (int c = 0; c < 4; ++c) kpre[c] = *reinterpret_cast<const float4*>(ksrc + 4 * (j + LPT * c));
#pragma unroll
        for (int c = 0; c < 4; ++c) vpre[c] = *reinterpret_cast<const f32x4*>(vsrc + 4 * (j + LPT * c));
    }

    // ---- q (and k_new) into LDS, with the optional prologue ----
#pragma unroll
    for (int u = 0; u < kQRegs; ++u) {
        const int i = tid + u * kThreads;
        if (i < G * HD) qs[i] = qreg[u];
    }
    for (int i = tid + kQRegs * kThreads; i < G * HD; i += kThreads) qs[i] = qg[i];
    if (have_new && tid < HD) ks[tid] = kreg;
    __syncthreads();
    // The work-group whose chunk holds `pos` (the last one) is the only one
    // that reads the new k: it alone runs k's prologue and writes the
    // prologue results back to q_out / k_out.
    const bool owner = p.pos >= ta && p.pos < tb;
    if (pro) {
        for (int h = wv; h < G + (have_new && owner ? 1 : 0); h += kWaves) {
            if (h < G) prologue_head_r<HD>(qs + h * HD, pr.gq, p.q_gamma != nullptr, p.norm_qk, p.has_rope, p.eps, pr, lane);
            else prologue_head_r<HD>(ks, pr.gk, p.k_gamma != nullptr, p.norm_qk, p.has_rope, p.eps, pr, lane);
        }
        __syncthreads();
        if (owner) {
            if (p.q_out)
                for (int i = tid; i < G * HD; i += kThreads) p.q_out[static_cast<size_t>(hk) * G * HD + i] = qs[i];
            if (p.k_out && have_new)
                for (int i = tid; i < HD; i += kThreads) p.k_out[static_cast<size_t>(hk) * HD + i] = ks[i];
        }
    }
    // the work-group whose chunk holds `pos` stores the new K/V row of its head
    if (have_new && p.pos >= ta && p.pos < tb) {
        float* kd = p.k_cache + static_cast<size_t>(p.pos) * kv_dim + static_cast<size_t>(hk) * HD;
        float* vd = p.v_cache + static_cast<size_t>(p.pos) * kv_dim + static_cast<size_t>(hk) * HD;
        const float* vn = p.v_new + static_cast<size_t>(hk) * HD;
        for (int i = tid; i < HD; i += kThreads) {
            kd[i] = ks[i];
            vd[i] = vn[i];
        }
    }

    // SHORT: the chunk's V rows into LDS for pass 2 (their last use of
    // registers: held across the head-block loop they went to scratch memory)
    if constexpr (SHORT) {
#pragma unroll
        for (int c = 0; c < 4; ++c) *reinterpret_cast<f32x4*>(vs + ts * HD + 4 * (j + LPT * c)) = vpre[c];
    }

    for (int hb = 0; hb < G; hb += kHeadBlock) {
        const int nh = min(kHeadBlock, G - hb);
        // q slices of this lane: kept in registers across the token passes of
        // a long chunk; a one-pass chunk reads each head's slices from LDS where
        // it uses them (64 registers fewer: four work-groups per CU)
        float4 qf[SHORT ? 1 : kHeadBlock][4];
        if constexpr (!SHORT) {
#pragma unroll
            for (int h = 0; h < kHeadBlock; ++h)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    qf[h][c] = h < nh ? *reinterpret_cast<const float4*>(qs + (hb + h) * HD + 4 * (j + LPT * c))
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
        }

        // ---- pass 1: scores ----
        for (int t = ta; t < tb; t += TPP) {
            const int tok = t + ts;
            const bool valid = tok < tb;
            float4 kf[4];
            if (SHORT) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    kf[c] = new0 ? *reinterpret_cast<const float4*>(ks + 4 * (j + LPT * c)) : kpre[c];
            } else if (valid) {
                const float* src = (have_new && tok == p.pos)
                                       ? ks
                                       : p.k_cache + static_cast<size_t>(tok) * kv_dim + static_cast<size_t>(hk) * HD;
#pragma unroll
                for (int c = 0; c < 4; ++c) kf[c] = *reinterpret_cast<const float4*>(src + 4 * (j + LPT * c));
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) kf[c] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int h = 0; h < kHeadBlock; ++h) {
                float s = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float4 qv;
                    if constexpr (SHORT)
                        qv = h < nh ? *reinterpret_cast<const float4*>(qs + (hb + h) * HD + 4 * (j + LPT * c))
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
                    else
                        qv = qf[h][c];
                    s += qv.x * kf[c].x + qv.y * kf[c].y + qv.z * kf[c].z + qv.w * kf[c].w;
                }
                s = group_sum<LPT>(s);
                if (valid && j == 0 && h < nh) sc[h * p.chunk + (tok - ta)] = s * p.scale;
            }
        }
        __syncthreads();

        // ---- per-head max / exp / sum: wave h owns head h ----
        const int len = tb - ta;
        float mx = -1e30f, sum = 0.0f;
        if (wv < nh) {
            float* row = sc + wv * p.chunk;
            for (int i = lane; i < len; i += 64) mx = fmaxf(mx, row[i]);
            mx = wave_max(mx);
            for (int i = lane; i < len; i += 64) {
                const float e = expf(row[i] - mx);
                row[i] = e;
                sum += e;
            }
            sum = wave_sum(sum);
        }
        __syncthreads();

        // ---- pass 2: o = sum_t e_t v_t ----
        if constexpr (SHORT) {
            // V is in LDS: thread (f, tg) sums float4 f of the head block over
            // tokens tg, tg + NTG, ...; the NTG partials meet in LDS
            constexpr int NF = kHeadBlock * HD / 4;
            constexpr int NTG = kThreads / NF;
            const int f = tid % NF, tg = tid / NF;
            const int h = f / (HD / 4), d4 = f % (HD / 4);
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            if (h < nh) {
                const float* prow = sc + h * p.chunk;
                for (int tl = tg; tl < len; tl += NTG) {
                    const float w = prow[tl];
                    const float4 v = *reinterpret_cast<const float4*>(vs + tl * HD + 4 * d4);
                    acc.x += w * v.x;
                    acc.y += w * v.y;
                    acc.z += w * v.z;
                    acc.w += w * v.w;
                }
            }
            float4* r4 = reinterpret_cast<float4*>(red);
            r4[tg * NF + f] = acc;
            if (wv < nh && lane == 0) {
                float* ml = p.part_ml + (static_cast<size_t>(split) * p.n_heads + hk * G + hb + wv) * 2;
                ml[0] = mx;
                ml[1] = sum;
            }
            __syncthreads();
            if (tid < NF && h < nh) {
                float4 t = r4[f];
#pragma unroll
                for (int g = 1; g < NTG; ++g) {
                    const float4 v = r4[g * NF + f];
                    t.x += v.x;
                    t.y += v.y;
                    t.z += v.z;
                    t.w += v.w;
                }
                *reinterpret_cast<float4*>(p.part_o + (static_cast<size_t>(split) * p.n_heads + hk * G + hb + h) * HD +
                                           4 * d4) = t;
            }
            __syncthreads();
            continue;
        }
        float4 of[kHeadBlock][4];
#pragma unroll
        for (int h = 0; h < kHeadBlock; ++h)
#pragma unroll
            for (int c = 0; c < 4; ++c) of[h][c] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int t = ta; t < tb; t += TPP) {
            const int tok = t + ts;
            if (tok < tb) {
                float4 vf[4];
                if (SHORT) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) vf[c] = make_float4(vpre[c].x, vpre[c].y, vpre[c].z, vpre[c].w);
                } else {
                    const float* src = (have_new && tok == p.pos)
                                           ? p.v_new + static_cast<size_t>(hk) * HD
                                           : p.v_cache + static_cast<size_t>(tok) * kv_dim + static_cast<size_t>(hk) * HD;
#pragma unroll
                    for (int c = 0; c < 4; ++c) vf[c] = *reinterpret_cast<const float4*>(src + 4 * (j + LPT * c));
                }
#pragma unroll
                for (int h = 0; h < kHeadBlock; ++h) {
                    const float w = h < nh ? sc[h * p.chunk + (tok - ta)] : 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        of[h][c].x += w * vf[c].x;
                        of[h][c].y += w * vf[c].y;
                        of[h][c].z += w * vf[c].z;
                        of[h][c].w += w * vf[c].w;
                    }
                }
            }
        }
        // reduce over the token slots of this wave (lanes with equal j)
#pragma unroll
        for (int h = 0; h < kHeadBlock; ++h)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int o = LPT; o < 64; o <<= 1) {
                    of[h][c].x += __shfl_xor(of[h][c].x, o, 64);
                    of[h][c].y += __shfl_xor(of[h][c].y, o, 64);
                    of[h][c].z += __shfl_xor(of[h][c].z, o, 64);
                    of[h][c].w += __shfl_xor(of[h][c].w, o, 64);
                }
        if (lane < LPT) {
#pragma unroll
            for (int h = 0; h < kHeadBlock; ++h)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    *reinterpret_cast<float4*>(red + (wv * kHeadBlock + h) * HD + 4 * (j + LPT * c)) = of[h][c];
        }
        // per-head (max, sum) from the owning wave
        if (wv < nh && lane == 0) {
            float* ml = p.part_ml + (static_cast<size_t>(split) * p.n_heads + hk * G + hb + wv) * 2;
            ml[0] = mx;
            ml[1] = sum;
        }
        __syncthreads();
        for (int i = tid; i < nh * HD; i += kThreads) {
            const int h = i / HD, d = i % HD;
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) acc += red[(w * kHeadBlock + h) * HD + d];
            p.part_o[(static_cast<size_t>(split) * p.n_heads + hk * G + hb + h) * HD + d] = acc;
        }
        __syncthreads();
    }
}

// Large query-head groups (G = n_heads / n_kv_heads >= 16, head_dim 128),
// e.g. MQA: the G query heads of one KV head are the M dimension of two small
// fp32 matrix products per 64-token sub-chunk, S = Q K^T and O += P V
// (v_mfma_f32_32x32x2f32, fp32 throughout like the reference), so every K/V
// row is read from HBM once.  One work-group (4 waves) owns (KV head, chunk);
// it walks the chunk in sub-chunks with an online softmax (running max and sum
// per head, O rescaled by e^(m_old - m_new)) and leaves the same (o, max, sum)
// partials as attn_chunk_kernel for attn_merge_kernel.
//   S: wave w computes tokens 32 (w % 2) .. + 32 over dims 64 (w / 2) .. + 64;
//      lane l holds Q[l % 32][d] and K[t][d] for the 32 dims d of its half
//      (the order of d inside a dot is free: half g = l / 32 takes dims
//      64 (w / 2) + 32 g .. + 32), the two dim halves meet in LDS.
//   softmax: wave w takes heads 8 w .. 8 w + 7 with lane = token; the eight
//      heads go through each step together (independent DPP max / sum
//      reductions, no LDS round trips), then lane i < 8 updates the running
//      max and sum of head 8 w + i.
//   P V: wave w owns output dims 32 w .. + 32; lane l reads P[l % 32][t] from
//      LDS and V[t][32 w + l % 32] from HBM for tokens t = 32 g + kk.
// MFMA layouts (32x32x2 f32): A[l % 32][l / 32], B[l / 32][l % 32], accumulator
// register r of lane l is D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
constexpr int kMqSub = 64;
constexpr int kMqHeads = 32;
constexpr int kMqLd = kMqSub + 4;

__global__ __launch_bounds__(kThreads) void attn_mq_kernel(AttnParams p) {
    constexpr int HD = 128;
    __shared__ __align__(16) float spart[2][kMqHeads][kMqLd];
    __shared__ __align__(16) float pl[kMqHeads][kMqLd];
    __shared__ float alpha_s[kMqHeads], m_s[kMqHeads], l_s[kMqHeads];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 31, g = lane >> 5;
    const int G = p.n_heads / p.n_kv;
    const int hk = blockIdx.x, split = blockIdx.y;
    const int ta = p.t0 + split * p.chunk;
    const int tb = min(p.t1, ta + p.chunk);
    const size_t kv_dim = static_cast<size_t>(p.n_kv) * HD;
    const bool have_new = p.use_new != 0;

    // the work-group whose chunk holds `pos` stores the new K/V row; its own
    // reads of token pos below take k_new / v_new directly
    if (have_new && p.pos >= ta && p.pos < tb) {
        float* kd = p.k_cache + static_cast<size_t>(p.pos) * kv_dim + static_cast<size_t>(hk) * HD;
        float* vd = p.v_cache + static_cast<size_t>(p.pos) * kv_dim + static_cast<size_t>(hk) * HD;
        for (int i = tid; i < HD; i += kThreads) {
            kd[i] = p.k_new[static_cast<size_t>(hk) * HD + i];
            vd[i] = p.v_new[static_cast<size_t>(hk) * HD + i];
        }
    }
    auto krow = [&](int t) -> const float* {
        return (have_new && t == p.pos) ? p.k_new + static_cast<size_t>(hk) * HD
                                        : p.k_cache + static_cast<size_t>(t) * kv_dim + static_cast<size_t>(hk) * HD;
    };
    auto vrow = [&](int t) -> const float* {
        return (have_new && t == p.pos) ? p.v_new + static_cast<size_t>(hk) * HD
                                        : p.v_cache + static_cast<size_t>(t) * kv_dim + static_cast<size_t>(hk) * HD;
    };

    const int tt = wv & 1, dh = wv >> 1;
    const int dq = 64 * dh + 32 * g;  // first dim of this lane's half in the S phase
    float qa[32];
    if (li < G) {
        const float* qr = p.q + (static_cast<size_t>(hk) * G + li) * HD + dq;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(qr + 4 * i);
            qa[4 * i] = v.x; qa[4 * i + 1] = v.y; qa[4 * i + 2] = v.z; qa[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) qa[i] = 0.0f;
    }
    if (tid < kMqHeads) {
        m_s[tid] = -1e30f;
        l_s[tid] = 0.0f;
    }
    floatx16 o;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] = 0.0f;
    __syncthreads();

    // Loads run one phase ahead: a sub-chunk's V rows are issued before its
    // S products and the next sub-chunk's K rows right after them, so they
    // arrive while the softmax and P V run.
    float kb[32];
    auto load_k = [&](int sa_) {
        const int tok = sa_ + 32 * tt + li;
        const float* kr = krow(tok < tb ? tok : tb - 1) + dq;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(kr + 4 * i);
            kb[4 * i] = v.x; kb[4 * i + 1] = v.y; kb[4 * i + 2] = v.z; kb[4 * i + 3] = v.w;
        }
    };
    if (ta < tb) load_k(ta);
    for (int sa = ta; sa < tb; sa += kMqSub) {
        float vb[32];
#pragma unroll
        for (int kk = 0; kk < 32; ++kk) {
            const int t = sa + 32 * g + kk;
            vb[kk] = vrow(t < tb ? t : tb - 1)[32 * wv + li];
        }
        // ---- S partials over this wave's dim half ----
        {
            floatx16 sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 32; ++kk) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[kk], kb[kk], sacc, 0, 0, 0);
            if (sa + kMqSub < tb) load_k(sa + kMqSub);
#pragma unroll
            for (int r = 0; r < 16; ++r) spart[dh][8 * (r >> 2) + 4 * g + (r & 3)][32 * tt + li] = sacc[r];
        }
        __syncthreads();
        // ---- online softmax ----
        {
            const bool valid = sa + lane < tb;
            float sv[8], mo[8], mn[8], su[8];
#pragma unroll
            for (int hh = 0; hh < 8; ++hh) {
                const int h = 8 * wv + hh;
                sv[hh] = valid ? (spart[0][h][lane] + spart[1][h][lane]) * p.scale : -1e30f;
                mo[hh] = m_s[h];
            }
#pragma unroll
            for (int hh = 0; hh < 8; ++hh) mn[hh] = fmaxf(mo[hh], wave_max(sv[hh]));
#pragma unroll
            for (int hh = 0; hh < 8; ++hh) {
                const float e = valid ? expf(sv[hh] - mn[hh]) : 0.0f;
                pl[8 * wv + hh][lane] = e;
                su[hh] = wave_sum(e);
            }
            float m_old = mo[0], m_new = mn[0], sum = su[0];
#pragma unroll
            for (int hh = 1; hh < 8; ++hh) {
                m_old = lane == hh ? mo[hh] : m_old;
                m_new = lane == hh ? mn[hh] : m_new;
                sum = lane == hh ? su[hh] : sum;
            }
            if (lane < 8) {
                const int h = 8 * wv + lane;
                const float a = expf(m_old - m_new);
                alpha_s[h] = a;
                l_s[h] = l_s[h] * a + sum;
                m_s[h] = m_new;
            }
        }
        __syncthreads();
        // ---- O = O e^(m_old - m_new) + P V over this wave's 32 dims ----
        {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[r] *= alpha_s[8 * (r >> 2) + 4 * g + (r & 3)];
            float pa[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(&pl[li][32 * g + 4 * i]);
                pa[4 * i] = v.x; pa[4 * i + 1] = v.y; pa[4 * i + 2] = v.z; pa[4 * i + 3] = v.w;
            }
#pragma unroll
            for (int kk = 0; kk < 32; ++kk) o = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[kk], vb[kk], o, 0, 0, 0);
        }
        __syncthreads();  // spart / pl / alpha are rewritten by the next sub-chunk
    }
    // partials: unnormalised o, and (max, sum) per head
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int h = 8 * (r >> 2) + 4 * g + (r & 3);
        if (h < G) p.part_o[(static_cast<size_t>(split) * p.n_heads + hk * G + h) * HD + 32 * wv + li] = o[r];
    }
    if (tid < G) {
        float* ml = p.part_ml + (static_cast<size_t>(split) * p.n_heads + hk * G + tid) * 2;
        ml[0] = m_s[tid];
        ml[1] = l_s[tid];
    }
}

// ---------------------------------------------------------------------------
// Causal prefill: B query tokens at positions pos0 .. pos0 + B - 1, each with
// the semantics of one decode step at its position (write its K/V row, then
// attend over its window).  Two launches:
//   attn_prefill_prologue_kernel: per token, the heads-RMSNorm + RoPE
//     prologue of q and k in LDS (the decode prologue's arithmetic, with the
//     token's own host-made cos/sin row), q written back, K/V rows stored;
//   attn_prefill_kernel (head_dim 128, G = n_heads / n_kv dividing 32): a
//     work-group owns 128 query rows, 128 / G tokens x the G heads of one KV
//     head, and walks the block's whole key range in 32-key sub-chunks with
//     S^T = K Q^T, online softmax and O += P V (fp16 matrix cores, fp16-pair
//     operands), masking each row to its own causal window, and writes
//     out = O / (l + 1e-12) directly (no split, no merge).
struct PrefillParams {
    float* q;             // [B][n_heads * HD], prologue result in place
    float* k;             // [B][n_kv * HD], prologue result in place
    const float* v;       // [B][n_kv * HD]
    float* k_cache;
    float* v_cache;
    float* out;           // [B][n_heads * HD]
    const float* q_gamma;
    const float* k_gamma;
    const float* rope;    // [B][2][HD / 2] cos then sin rows, or null
    int32_t pos0, batch, n_heads, n_kv, sw, norm_qk;
    float scale, eps;
    // key-split plan (null: one work-group per block, longest first):
    // plan[4 y .. 4 y + 3] = (block, slot, first key, last key) of grid row
    // y, slot -1 for a whole block, else the partial slot of that part of a
    // split block, whose (unnormalised o, max, sum) go to part_o / part_ml
    const int32_t* plan;
    float* part_o;   // [slots][n_kv][128 rows][HD]
    float* part_ml;  // [slots][n_kv][128 rows][2]
};

template <int HD>
__global__ __launch_bounds__(kThreads) void attn_prefill_prologue_kernel(PrefillParams p) {
    extern __shared__ __align__(16) float smem[];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int qn = p.n_heads * HD, kn = p.n_kv * HD;
    float* qr = p.q + static_cast<size_t>(t) * qn;
    float* kr = p.k + static_cast<size_t>(t) * kn;
    const float* vr = p.v + static_cast<size_t>(t) * kn;
    float* qs = smem;        // [n_heads][HD]
    float* ks = smem + qn;   // [n_kv][HD]
    const bool rope = p.rope != nullptr;
    if (p.norm_qk || rope) {
        for (int i = tid; i < qn; i += kThreads) qs[i] = qr[i];
        for (int i = tid; i < kn; i += kThreads) ks[i] = kr[i];
        __syncthreads();
        const float* rc = rope ? p.rope + static_cast<size_t>(t) * HD : nullptr;
        const float* rs = rope ? rc + HD / 2 : nullptr;
        for (int h = wv; h < p.n_heads + p.n_kv; h += kWaves) {
            if (h < p.n_heads) prologue_head<HD>(qs + h * HD, p.q_gamma, p.norm_qk, rope, p.eps, rc, rs, lane);
            else prologue_head<HD>(ks + (h - p.n_heads) * HD, p.k_gamma, p.norm_qk, rope, p.eps, rc, rs, lane);
        }
        __syncthreads();
        for (int i = tid; i < qn; i += kThreads) qr[i] = qs[i];
        for (int i = tid; i < kn; i += kThreads) kr[i] = ks[i];
    } else {
        ks = kr;  // K unchanged: stored straight from the input
    }
    const size_t row = static_cast<size_t>(p.pos0 + t) * kn;
    for (int i = tid; i < kn; i += kThreads) {
        p.k_cache[row + i] = ks[i];
        p.v_cache[row + i] = vr[i];
    }
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// 8 floats as an fp16 pair: hi = fp16(v), lo = fp16(v - hi) (v - hi is exact
// in fp32), so hi + lo carries about 22 significant bits of v.  Below fp16's
// normal range lo keeps an absolute step of 2^-24, far below what these
// attention sums resolve.
__device__ __forceinline__ void split8(const float (&v)[8], half8_t& hi, half8_t& lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const _Float16 h = static_cast<_Float16>(v[i]);
        hi[i] = h;
        lo[i] = static_cast<_Float16>(v[i] - static_cast<float>(h));
    }
}

// The causal batch on the fp16 matrix cores.  A work-group owns 128 query rows
// (128 / G tokens x the G heads of one KV head), a wave 32 of them, and walks
// the rows' key range in 32-key sub-chunks:
//   stage   the sub-chunk's K and V rows are loaded once per work-group (the
//           next sub-chunk's loads are in flight during this one's products),
//           split into fp16 pairs (hi = fp16(v), lo = fp16(v - hi): about 22
//           significant bits) and written to LDS in MFMA operand order;
//   S^T     = K Q^T on v_mfma_f32_32x32x16_f16, three products per K16 slice
//           (hi hi, hi lo, lo hi; the lo lo term is below 2^-22 of the
//           product), Q split once at the start: lane (i, g) ends up holding
//           the scores of query row i (of its wave) for the 16 keys
//           8 a + 4 g + b (a, b = 0..3) of the sub-chunk;
//   softmax the online update of each row's max and sum in registers (the two
//           lane halves of a row meet with one exchange each);
//   O += P V with P straight from those registers as the MFMA's A operand:
//           its K16 slice c holds keys 16 c + 4 g + {0..3, 8..11} in lane half
//           g, and the staged V fragments take the same key order.  O rows
//           are rescaled by the rows' factors through a 32-float LDS array.
// A 64-key sub-chunk of 32 rows with operands from registers and S transposed
// through LDS (the fp32-MFMA form before this) read each K/V row once per 32
// rows instead of once per 128.
// Operands hold |values| < 65504 (fp16's range): q and k after the
// heads-RMSNorm, v and the probabilities in [0, 1].
constexpr int kPfRows = 128;  // query rows (token, head) per work-group
constexpr int kPfKeys = 32;   // keys per sub-chunk

__global__ __launch_bounds__(kThreads, 2) void attn_prefill_kernel(PrefillParams p) {
    constexpr int HD = 128;
    // operand fragments: 8 halves per lane, [slice][lane] for K (A of S^T),
    // [N tile][slice][lane] for V (B of P V)
    __shared__ __align__(16) half8_t khi[HD / 16][64], klo[HD / 16][64];
    __shared__ __align__(16) half8_t vhi[HD / 32][kPfKeys / 16][64], vlo[HD / 32][kPfKeys / 16][64];
    __shared__ __align__(16) float rowf[kWaves][32];  // per-row factors on their way to the O layout
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int li = lane & 31, g = lane >> 5;
    const int G = p.n_heads / p.n_kv, TQ = kPfRows / G;
    const int hk = blockIdx.x;
    int blk = static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y);  // longest key ranges first
    int slot = -1;
    if (p.plan) {
        const int4 it = reinterpret_cast<const int4*>(p.plan)[blockIdx.y];
        blk = it.x;
        slot = it.y;
    }
    const int q0 = blk * TQ;
    const int nq = min(TQ, p.batch - q0);
    const int hi_block = p.pos0 + q0 + nq - 1;
    const int lo_block = p.sw > 0 ? max(0, p.pos0 + q0 - p.sw + 1) : 0;
    // this work-group's keys: the block's range, or one half of it
    const int lo_first = p.plan ? reinterpret_cast<const int4*>(p.plan)[blockIdx.y].z : lo_block;
    const int hi_last = p.plan ? reinterpret_cast<const int4*>(p.plan)[blockIdx.y].w : hi_block;
    const size_t kv_dim = static_cast<size_t>(p.n_kv) * HD;
    const size_t q_dim = static_cast<size_t>(p.n_heads) * HD;
    const float* kbase = p.k_cache + static_cast<size_t>(hk) * HD;
    const float* vbase = p.v_cache + static_cast<size_t>(hk) * HD;

    // this lane's query row: row 32 wv + li of the work-group, token
    // (32 wv + li) / G of the block, head (32 wv + li) % G of KV head hk
    const int qrow = 32 * wv + li;
    const int qt = qrow / G;
    const bool qvalid = qt < nq;
    const int q_hi = p.pos0 + q0 + qt;                          // last key of its window
    const int q_lo = p.sw > 0 ? max(0, q_hi - p.sw + 1) : 0;    // first key
    half8_t qh[HD / 16], ql[HD / 16];
    {
        const float* qr = p.q + static_cast<size_t>(q0 + (qvalid ? qt : 0)) * q_dim +
                          (static_cast<size_t>(hk) * G + qrow % G) * HD + 8 * g;
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 16 * c);
            const float4 b = *reinterpret_cast<const float4*>(qr + 16 * c + 4);
            float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            if (!qvalid)
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            split8(v, qh[c], ql[c]);
        }
    }

    // staging slots of this thread: K slots tid, tid + 256 (slot s: slice
    // s / 64, lane s % 64 -> key s % 32, dims 16 slice + 8 ((s % 64) / 32));
    // V slots tid, tid + 256 (slot s: N tile s / 128, slice (s / 64) % 2,
    // lane s % 64 -> dim 32 tile + s % 32, keys 16 slice + 4 half + {0..3, 8..11})
    float4 kst[2][2];
    float vst[2][8];
    auto prefetch = [&](int sa) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int sl = tid + 256 * u;
            const int c = sl >> 6, L = sl & 63;
            int key = sa + (L & 31);
            key = key <= hi_last ? key : hi_last;
            const float* kr = kbase + static_cast<size_t>(key) * kv_dim + 16 * c + 8 * (L >> 5);
            kst[u][0] = *reinterpret_cast<const float4*>(kr);
            kst[u][1] = *reinterpret_cast<const float4*>(kr + 4);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int sl = tid + 256 * u;
            const int n = sl >> 7, c = (sl >> 6) & 1, L = sl & 63;
            const int d = 32 * n + (L & 31);
            const int k0 = sa + 16 * c + 4 * (L >> 5);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                int key = k0 + (i & 3) + 8 * (i >> 2);
                key = key <= hi_last ? key : hi_last;
                vst[u][i] = vbase[static_cast<size_t>(key) * kv_dim + d];
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int sl = tid + 256 * u;
            const float kv[8] = {kst[u][0].x, kst[u][0].y, kst[u][0].z, kst[u][0].w,
                                 kst[u][1].x, kst[u][1].y, kst[u][1].z, kst[u][1].w};
            half8_t h, l;
            split8(kv, h, l);
            khi[sl >> 6][sl & 63] = h;
            klo[sl >> 6][sl & 63] = l;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int sl = tid + 256 * u;
            half8_t h, l;
            split8(vst[u], h, l);
            vhi[sl >> 7][(sl >> 6) & 1][sl & 63] = h;
            vlo[sl >> 7][(sl >> 6) & 1][sl & 63] = l;
        }
    };

    float m_run = -1e30f, l_run = 0.0f;  // row qrow's running max and sum
    floatx16 o[HD / 32];
#pragma unroll
    for (int n = 0; n < HD / 32; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[n][r] = 0.0f;

    prefetch(lo_first);
    for (int sa = lo_first; sa <= hi_last; sa += kPfKeys) {
        stage();
        __syncthreads();
        if (sa + kPfKeys <= hi_last) prefetch(sa + kPfKeys);
        // S^T for the sub-chunk: rows = keys, columns = this wave's query rows
        floatx16 st;
#pragma unroll
        for (int r = 0; r < 16; ++r) st[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < HD / 16; ++c) {
            const half8_t kh = khi[c][lane], kl = klo[c][lane];
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[c], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[c], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[c], st, 0, 0, 0);
        }
        // online softmax of row qrow over keys sa + 8 a + 4 g + b (r = 4 a + b),
        // in base 2: scores scaled by scale log2(e), e^(s - m) as one
        // v_exp_f32 of the difference (expf's range reduction took 12% of
        // the kernel; the results move by about 1e-7 relative)
        float mx = -1e30f;
        bool valid[16];
        const float scale2 = p.scale * 1.4426950408889634f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = sa + 8 * (r >> 2) + 4 * g + (r & 3);
            valid[r] = qvalid && key >= q_lo && key <= q_hi;
            st[r] = valid[r] ? st[r] * scale2 : -1e30f;
            mx = fmaxf(mx, st[r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        float e[16], sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            e[r] = valid[r] ? __builtin_amdgcn_exp2f(st[r] - m_new) : 0.0f;
            sum += e[r];
        }
        sum += __shfl_xor(sum, 32, 64);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run = l_run * alpha + sum;
        m_run = m_new;
        // O rows are 8 (r / 4) + 4 g + r % 4 of the wave: their factors via LDS
        if (g == 0) rowf[wv][li] = alpha;
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's own writes, read back below
        asm volatile("" ::: "memory");
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            const float4 f = *reinterpret_cast<const float4*>(&rowf[wv][8 * a4 + 4 * g]);
#pragma unroll
            for (int n = 0; n < HD / 32; ++n) {
                o[n][4 * a4] *= f.x;
                o[n][4 * a4 + 1] *= f.y;
                o[n][4 * a4 + 2] *= f.z;
                o[n][4 * a4 + 3] *= f.w;
            }
        }
        // O += P V: slice c takes the exponentials e[8 c .. 8 c + 7]
#pragma unroll
        for (int c = 0; c < kPfKeys / 16; ++c) {
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) pv[i] = e[8 * c + i];
            half8_t ph, plo;
            split8(pv, ph, plo);
#pragma unroll
            for (int n = 0; n < HD / 32; ++n) {
                const half8_t vh = vhi[n][c][lane], vl = vlo[n][c][lane];
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, vh, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, vl, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(plo, vh, o[n], 0, 0, 0);
            }
        }
        __syncthreads();  // every wave is done with this sub-chunk's K / V fragments
    }
    if (slot >= 0) {
        // half of a split block: the unnormalised O and the row's (max, sum)
        // for attn_prefill_merge_kernel
        const size_t base = (static_cast<size_t>(slot) * p.n_kv + hk) * kPfRows;
        if (g == 0)
            reinterpret_cast<float2*>(p.part_ml)[base + qrow] = make_float2(m_run, l_run);
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int row = 32 * wv + 8 * a4 + 4 * g + b;
#pragma unroll
                for (int n = 0; n < HD / 32; ++n) p.part_o[(base + row) * HD + 32 * n + li] = o[n][4 * a4 + b];
            }
        return;
    }
    // out = O / (l + 1e-12), the rows' sums through LDS like the factors
    if (g == 0) rowf[wv][li] = 1.0f / (l_run + 1e-12f);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
        const float4 f = *reinterpret_cast<const float4*>(&rowf[wv][8 * a4 + 4 * g]);
        const float fr[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int row = 32 * wv + 8 * a4 + 4 * g + b;
            const int t = row / G, h = row % G;
            if (t < nq) {
                float* dst = p.out + static_cast<size_t>(q0 + t) * q_dim + (static_cast<size_t>(hk) * G + h) * HD;
#pragma unroll
                for (int n = 0; n < HD / 32; ++n) dst[32 * n + li] = o[n][4 * a4 + b] * fr[b];
            }
        }
    }
}

// The parts of split block j = blockIdx.y (plan_split[3 j ..]: block, first
// partial slot, parts) for KV head blockIdx.x, a slice of its rows per
// blockIdx.z:
// out = sum_i o_i 2^(m_i - M) / (sum_i l_i 2^(m_i - M) + 1e-12), M = max_i m_i
// (the maxima are in base-2 units, the scores having been scaled by log2 e);
// a part with no key in a row's window has m = -1e30 and weight 0.
constexpr int kPfMaxParts = 8;
__global__ __launch_bounds__(kThreads) void attn_prefill_merge_kernel(PrefillParams p, const int32_t* plan_split) {
    constexpr int HD = 128;
    const int hk = blockIdx.x, j = blockIdx.y;
    const int G = p.n_heads / p.n_kv, TQ = kPfRows / G;
    const int blk = plan_split[3 * j], slot0 = plan_split[3 * j + 1], parts = plan_split[3 * j + 2];
    const int q0 = blk * TQ, nq = min(TQ, p.batch - q0);
    const size_t q_dim = static_cast<size_t>(p.n_heads) * HD;
    // one float4 of one row per thread (grid z: kPfRows HD / 4 / kThreads
    // slices), every part's loads issued together
    {
        const int it = static_cast<int>(blockIdx.z) * kThreads + static_cast<int>(threadIdx.x);
        const int row = it / (HD / 4), d4 = it % (HD / 4);
        const int t = row / G, h = row % G;
        if (t >= nq) return;
        float2 ml[kPfMaxParts];
        float M = -1e30f;
#pragma unroll
        for (int i = 0; i < kPfMaxParts; ++i) {
            if (i < parts) {
                ml[i] = reinterpret_cast<const float2*>(p.part_ml)[(static_cast<size_t>(slot0 + i) * p.n_kv + hk) * kPfRows + row];
                M = fmaxf(M, ml[i].x);
            }
        }
        float l = 0.0f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < kPfMaxParts; ++i) {
            if (i < parts) {
                const float a = __builtin_amdgcn_exp2f(ml[i].x - M);
                const float4 o = reinterpret_cast<const float4*>(
                    p.part_o + ((static_cast<size_t>(slot0 + i) * p.n_kv + hk) * kPfRows + row) * HD)[d4];
                l += ml[i].y * a;
                acc.x += o.x * a;
                acc.y += o.y * a;
                acc.z += o.z * a;
                acc.w += o.w * a;
            }
        }
        const float inv = 1.0f / (l + 1e-12f);
        reinterpret_cast<float4*>(p.out + static_cast<size_t>(q0 + t) * q_dim + (static_cast<size_t>(hk) * G + h) * HD)[d4] =
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
}

// out[h] = (sum_j o_j e^(m_j - M)) / (sum_j l_j e^(m_j - M) + 1e-12).  Work-
// group (h, y) of a (heads, ny) grid writes float4 columns y nd4 .. + nd4 of
// head h (nd4 = hd / 4 / ny): every work-group forms M and the sum from the
// (max, sum) pairs of all splits and reads only its columns of the partial
// o, so a long window's partials are read by ny times as many CUs.  Thread
// (d4, g) owns column d4 and splits g, g + ng, ...; its first U partial
// loads are issued before the max / sum pass, so the work-group waits on
// memory about once.  U is the smallest of 4, 8, 16 and 32 that covers the
// thread's splits (more loads in flight than needed cost registers and
// occupancy).  The ng per-thread sums of a column meet in an LDS tree.
constexpr int kMergeThreads = 256;
constexpr int kMergeMaxSplit = 4096;
#ifndef GNCX_MERGE_KB
#define GNCX_MERGE_KB 32
#endif
constexpr size_t kMergeBytesPerGroup = static_cast<size_t>(GNCX_MERGE_KB) * 1024;  // partial o per work-group
template <int U>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(const float* __restrict part_o,
                                                                   const float* __restrict part_ml, int32_t n_split,
                                                                   int32_t n_heads, int32_t hd,
                                                                   float* __restrict out) {
    __shared__ float wgt[kMergeMaxSplit];
    __shared__ float red[2][kMergeThreads / 64];
    __shared__ float4 accs[kMergeThreads];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nd4 = hd / 4 / static_cast<int>(gridDim.y);  // a power of two from 4 to 64
    const int ng = kMergeThreads / nd4;
    const int d4 = static_cast<int>(blockIdx.y) * nd4 + tid % nd4, g = tid / nd4;
    auto po_at = [&](int s) {
        return *reinterpret_cast<const float4*>(part_o + (static_cast<size_t>(s) * n_heads + h) * hd + 4 * d4);
    };
    // Every load a thread needs is issued here, unconditionally (split
    // indices clamped to the last split, whose weight is then not used), so
    // the kernel waits on memory once: this thread's (max, sum) pair of split
    // tid and its U partial-o float4.
    // (more than kMergeThreads splits: the pairs are read again where used)
    const bool one_ml = n_split <= kMergeThreads;
    auto ml_at = [&](int sp) {
        return *reinterpret_cast<const float2*>(part_ml + (static_cast<size_t>(sp) * n_heads + h) * 2);
    };
    const float2 ml0 = ml_at(tid < n_split ? tid : n_split - 1);
    float4 po[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sp = g + u * ng;
        po[u] = po_at(sp < n_split ? sp : n_split - 1);
    }
    float m = tid < n_split ? ml0.x : -1e30f;
    if (!one_ml)
        for (int sp = tid + kMergeThreads; sp < n_split; sp += kMergeThreads) m = fmaxf(m, ml_at(sp).x);
    m = wave_max(m);
    if (lane == 0) red[0][wv] = m;
    __syncthreads();
    float M = red[0][0];
    for (int w = 1; w < kMergeThreads / 64; ++w) M = fmaxf(M, red[0][w]);
    float l = 0.0f;
    if (tid < n_split) {
        const float e = expf(ml0.x - M);
        wgt[tid] = e;
        l += ml0.y * e;
    }
    if (!one_ml)
        for (int sp = tid + kMergeThreads; sp < n_split; sp += kMergeThreads) {
            const float2 v = ml_at(sp);
            const float e = expf(v.x - M);
            wgt[sp] = e;
            l += v.y * e;
        }
    l = wave_sum(l);
    if (lane == 0) red[1][wv] = l;
    __syncthreads();
    float lt = 0.0f;
    for (int w = 0; w < kMergeThreads / 64; ++w) lt += red[1][w];
    const float inv = 1.0f / (lt + 1e-12f);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sp = g + u * ng;
        const float w = sp < n_split ? wgt[sp] : 0.0f;
        a.x += po[u].x * w;
        a.y += po[u].y * w;
        a.z += po[u].z * w;
        a.w += po[u].w * w;
    }
    for (int sp = g + U * ng; sp < n_split; sp += ng) {
        const float4 v = po_at(sp);
        const float w = wgt[sp];
        a.x += v.x * w;
        a.y += v.y * w;
        a.z += v.z * w;
        a.w += v.w * w;
    }
    accs[tid] = a;
    __syncthreads();
    for (int half = ng / 2; half > 0; half /= 2) {
        if (g < half) {
            const float4 v = accs[tid + half * nd4];
            a.x += v.x;
            a.y += v.y;
            a.z += v.z;
            a.w += v.w;
            accs[tid] = a;
        }
        __syncthreads();
    }
    if (g == 0) {
        float4 r;
        r.x = a.x * inv;
        r.y = a.y * inv;
        r.z = a.z * inv;
        r.w = a.w * inv;
        *reinterpret_cast<float4*>(out + static_cast<size_t>(h) * hd + 4 * d4) = r;
    }
}

hipError_t launch_merge(const float* part_o, const float* part_ml, int32_t n_split, int32_t n_heads, int32_t hd,
                        float* out, hipStream_t stream) {
    // column slices per head: the smallest count that keeps a work-group's
    // share of the partial o within kMergeBytesPerGroup (at least 4 columns each)
    int32_t ny = 1;
    const size_t head_bytes = sizeof(float) * static_cast<size_t>(n_split) * hd;
    while (ny < 16 && hd / 4 / ny > 4 && head_bytes / ny > kMergeBytesPerGroup) ny *= 2;
    const int32_t ng = kMergeThreads / (hd / 4 / ny);  // split groups per column
    const int32_t per = (n_split + ng - 1) / ng;       // splits per thread
    const dim3 grid(n_heads, ny);
    if (per <= 4)
        hipLaunchKernelGGL(attn_merge_kernel<4>, grid, dim3(kMergeThreads), 0, stream, part_o, part_ml, n_split,
                           n_heads, hd, out);
    else if (per <= 8)
        hipLaunchKernelGGL(attn_merge_kernel<8>, grid, dim3(kMergeThreads), 0, stream, part_o, part_ml, n_split,
                           n_heads, hd, out);
    else if (per <= 16)
        hipLaunchKernelGGL(attn_merge_kernel<16>, grid, dim3(kMergeThreads), 0, stream, part_o, part_ml, n_split,
                           n_heads, hd, out);
    else
        hipLaunchKernelGGL(attn_merge_kernel<32>, grid, dim3(kMergeThreads), 0, stream, part_o, part_ml, n_split,
                           n_heads, hd, out);
    return hipGetLastError();
}

struct Plan {
    int32_t t0, t1, chunk, n_split;
};

// LDS per work-group: scores [kHeadBlock][chunk] + wave partials + q + k_new,
// plus the chunk's V rows for a one-pass chunk (kThreads * 16 floats), kept
// within 64 KB by capping the chunk.
constexpr size_t kLdsBudget = 64 * 1024;

size_t lds_base(int32_t chunk, int32_t G, int32_t hd) {
    return sizeof(float) * (static_cast<size_t>(kHeadBlock) * chunk + static_cast<size_t>(kWaves) * kHeadBlock * hd +
                            static_cast<size_t>(G) * hd + hd);
}

// the chunk fits one pass of the work-group and its V rows fit beside the rest
bool one_pass(int32_t chunk, int32_t G, int32_t hd) {
    return chunk <= kThreads / (hd / 16) && lds_base(chunk, G, hd) + sizeof(float) * kThreads * 16 <= kLdsBudget;
}

size_t lds_bytes(int32_t chunk, int32_t G, int32_t hd) {
    return lds_base(chunk, G, hd) + (one_pass(chunk, G, hd) ? sizeof(float) * kThreads * 16 : 0);
}

Plan make_plan(int32_t pos, int32_t sw, int32_t n_kv, int32_t G, int32_t hd) {
    Plan pl;
    pl.t0 = sw > 0 ? (pos - sw + 1 > 0 ? pos - sw + 1 : 0) : 0;
    pl.t1 = pos + 1;
    const int32_t win = pl.t1 - pl.t0;
    auto chunk_for = [&](int32_t groups) {
        int32_t want = groups / (n_kv > 0 ? n_kv : 1);
        if (want < 1) want = 1;
        int32_t c = (win + want - 1) / want;
        c = ((c + 31) / 32) * 32;
        if (c < 32) c = 32;
        return c > kMaxChunk ? kMaxChunk : c;
    };
    int32_t chunk = chunk_for(kTargetGroups);
    if (chunk > 32) chunk = chunk_for(kTargetGroupsLong);
    while (chunk > 32 && lds_bytes(chunk, G, hd) > kLdsBudget) chunk -= 32;
    // the merge weighs at most kMergeMaxSplit chunks
    while ((win + chunk - 1) / chunk > kMergeMaxSplit) chunk += 32;
    pl.chunk = chunk;
    pl.n_split = (win + chunk - 1) / chunk;
    return pl;
}

template <int HD>
hipError_t launch_hd(const AttnArgs& a, const Plan& pl, float* part_o, float* part_ml, hipStream_t stream) {
    AttnParams p{};
    p.q = a.q;
    p.k_new = a.k_new;
    p.v_new = a.v_new;
    p.k_cache = a.k_cache;
    p.v_cache = a.v_cache;
    p.part_o = part_o;
    p.part_ml = part_ml;
    p.q_out = a.q_out;
    p.k_out = a.k_out;
    p.q_gamma = a.q_gamma;
    p.k_gamma = a.k_gamma;
    p.pos = a.pos;
    p.n_heads = a.n_heads;
    p.n_kv = a.n_kv_heads;
    p.t0 = pl.t0;
    p.t1 = pl.t1;
    p.chunk = pl.chunk;
    p.use_new = (a.write_kv && a.k_new && a.v_new) ? 1 : 0;
    p.norm_qk = a.norm_qk;
    p.has_rope = a.rope ? 1 : 0;
    p.scale = a.scale;
    p.eps = a.eps;
    if (a.rope) p.rope = *a.rope;
    else p.rope.half = 0;
    const int G = a.n_heads / a.n_kv_heads;
    const size_t lds = lds_bytes(pl.chunk, G, HD);
    if (lds > kLdsBudget || pl.chunk > kMaxChunk) return hipErrorInvalidValue;  // window too long for one step
    if (one_pass(pl.chunk, G, HD))
        hipLaunchKernelGGL((attn_chunk_kernel<HD, true>), dim3(a.n_kv_heads, pl.n_split), dim3(kThreads), lds, stream,
                           p);
    else
        hipLaunchKernelGGL((attn_chunk_kernel<HD, false>), dim3(a.n_kv_heads, pl.n_split), dim3(kThreads), lds,
                           stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge(part_o, part_ml, pl.n_split, a.n_heads, HD, a.out, stream);
}

// Chunks of whole 64-token sub-chunks, about one work-group per CU.
Plan make_mq_plan(int32_t pos, int32_t sw, int32_t n_kv) {
    Plan pl;
    pl.t0 = sw > 0 ? (pos - sw + 1 > 0 ? pos - sw + 1 : 0) : 0;
    pl.t1 = pos + 1;
    const int32_t win = pl.t1 - pl.t0;
    int32_t want = 256 / (n_kv > 0 ? n_kv : 1);
    if (want < 1) want = 1;
    int32_t chunk = (win + want - 1) / want;
    chunk = ((chunk + kMqSub - 1) / kMqSub) * kMqSub;
    while ((win + chunk - 1) / chunk > kMergeMaxSplit) chunk += kMqSub;
    pl.chunk = chunk;
    pl.n_split = (win + chunk - 1) / chunk;
    return pl;
}

hipError_t launch_mq(const AttnArgs& a, const Plan& pl, float* part_o, float* part_ml, hipStream_t stream) {
    AttnParams p{};
    p.q = a.q;
    p.k_new = a.k_new;
    p.v_new = a.v_new;
    p.k_cache = a.k_cache;
    p.v_cache = a.v_cache;
    p.part_o = part_o;
    p.part_ml = part_ml;
    p.pos = a.pos;
    p.n_heads = a.n_heads;
    p.n_kv = a.n_kv_heads;
    p.t0 = pl.t0;
    p.t1 = pl.t1;
    p.chunk = pl.chunk;
    p.use_new = (a.write_kv && a.k_new && a.v_new) ? 1 : 0;
    p.scale = a.scale;
    hipLaunchKernelGGL(attn_mq_kernel, dim3(a.n_kv_heads, pl.n_split), dim3(kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_merge(part_o, part_ml, pl.n_split, a.n_heads, 128, a.out, stream);
}

}  // namespace

bool attention_prefill_supported(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0) return false;
    const int32_t G = n_heads / n_kv_heads;
    if (G > 32 || 32 % G != 0) return false;
    return sizeof(float) * static_cast<size_t>(n_heads + n_kv_heads) * head_dim <= kLdsBudget;
}

size_t attention_prefill_part_floats(int32_t part_slots, int32_t n_kv_heads) {
    return static_cast<size_t>(part_slots) * n_kv_heads * kPfRows * (128 + 2);
}
constexpr size_t kPfPartMax = size_t{128} << 20;

// The key-split plan of a prefill call.  A block's work is its number of
// 32-key sub-chunks, and two work-groups share a CU, so the kernel's time is
// about the larger of its longest work-group and the total work over the
// resident work-groups.  Blocks longer than a third of the longest (and than
// 8 sub-chunks) are cut into parts of their key range of at most that
// length, each a work-group, whose partial results attn_prefill_merge_kernel
// combines; grid rows are ordered longest first.  (2048 tokens, 32/8 heads:
// kernel + merge 200 us per layer unsplit; halves 163 + 12, thirds best,
// quarters 149 + 21: the partials' traffic grows with the parts.)  Up to 8
// sub-chunks in the longest block there is nothing worth a second launch: no
// plan.
// Table: n_items rows of (block, slot, first key, last key), slot -1 for a
// whole block, else its part's index in the partial buffers; then per split
// block (block, first slot, parts).
bool attention_prefill_plan(const PrefillArgs& a, std::vector<int32_t>& tab, int32_t& n_items, int32_t& n_split) {
    n_items = n_split = 0;
    tab.clear();
    if (a.batch <= 0 || a.n_kv_heads <= 0 || a.n_heads % a.n_kv_heads != 0) return false;
    const int32_t G = a.n_heads / a.n_kv_heads, TQ = kPfRows / G;
    const int32_t nblk = (a.batch + TQ - 1) / TQ;
    struct Item {
        int32_t blk, slot, ks, ke;
    };
    std::vector<Item> items;
    std::vector<int32_t> split;
    int32_t maxsub = 0;
    auto range = [&](int32_t blk, int32_t& lo, int32_t& hi) {
        const int32_t q0 = blk * TQ, nq = std::min(TQ, a.batch - q0);
        hi = a.pos0 + q0 + nq - 1;
        lo = a.sliding_window > 0 ? std::max(0, a.pos0 + q0 - a.sliding_window + 1) : 0;
    };
    for (int32_t blk = 0; blk < nblk; ++blk) {
        int32_t lo, hi;
        range(blk, lo, hi);
        maxsub = std::max(maxsub, (hi - lo) / kPfKeys + 1);
    }
    if (maxsub <= 8) return false;
    const int32_t cut = std::max<int32_t>(8, (maxsub + 2) / 3);
    int32_t slots = 0;
    for (int32_t blk = nblk - 1; blk >= 0; --blk) {
        int32_t lo, hi;
        range(blk, lo, hi);
        const int32_t nsub = (hi - lo) / kPfKeys + 1;
        if (nsub > cut) {
            const int32_t parts = (nsub + cut - 1) / cut;  // at most 3 (cut >= maxsub / 3)
            if (parts > kPfMaxParts) return false;
            split.insert(split.end(), {blk, slots, parts});
            for (int32_t q = 0; q < parts; ++q) {
                const int32_t s0 = nsub * q / parts, s1 = nsub * (q + 1) / parts;  // sub-chunks [s0, s1)
                items.push_back({blk, slots + q, lo + kPfKeys * s0, q + 1 == parts ? hi : lo + kPfKeys * s1 - 1});
            }
            slots += parts;
        } else {
            items.push_back({blk, -1, lo, hi});
        }
    }
    // the partial buffers stay within kPfPartMax (a long prompt's plan would
    // need them per 128 rows of every part: it runs unsplit instead)
    if (attention_prefill_part_floats(slots, a.n_kv_heads) * sizeof(float) > kPfPartMax) return false;
    std::stable_sort(items.begin(), items.end(),
                     [](const Item& x, const Item& y) { return x.ke - x.ks > y.ke - y.ks; });
    if (items.size() > 65535 || split.size() / 3 > 65535) return false;
    for (const Item& it : items) tab.insert(tab.end(), {it.blk, it.slot, it.ks, it.ke});
    tab.insert(tab.end(), split.begin(), split.end());
    n_items = static_cast<int32_t>(items.size());
    n_split = static_cast<int32_t>(split.size() / 3);
    return true;
}

// partial slots of a plan: the parts of its split blocks (the last table
// entries: block, first slot, parts)
int32_t attention_prefill_part_slots(const std::vector<int32_t>& tab, int32_t n_items, int32_t n_split) {
    if (n_split <= 0) return 0;
    const size_t last = 4 * static_cast<size_t>(n_items) + 3 * static_cast<size_t>(n_split - 1);
    return tab[last + 1] + tab[last + 2];
}

hipError_t launch_attention_prefill(const PrefillArgs& a, hipStream_t stream) {
    if (a.batch <= 0) return hipSuccess;
    if (!attention_prefill_supported(a.n_heads, a.n_kv_heads, a.head_dim) || a.pos0 < 0) return hipErrorInvalidValue;
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                         reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.out) |
                         reinterpret_cast<uintptr_t>(a.k_cache) | reinterpret_cast<uintptr_t>(a.v_cache);
    if (al & 15u) return hipErrorInvalidValue;
    const int32_t G = a.n_heads / a.n_kv_heads, TQ = kPfRows / G;
    const int32_t nblk = (a.batch + TQ - 1) / TQ;
    if (nblk > 65535) return hipErrorInvalidValue;
    PrefillParams p{};
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.k_cache = a.k_cache;
    p.v_cache = a.v_cache;
    p.out = a.out;
    p.q_gamma = a.q_gamma;
    p.k_gamma = a.k_gamma;
    p.rope = a.rope;
    p.pos0 = a.pos0;
    p.batch = a.batch;
    p.n_heads = a.n_heads;
    p.n_kv = a.n_kv_heads;
    p.sw = a.sliding_window;
    p.norm_qk = a.norm_qk;
    p.scale = a.scale;
    p.eps = a.eps;
    const size_t lds = (a.norm_qk || a.rope) ? sizeof(float) * static_cast<size_t>(a.n_heads + a.n_kv_heads) * 128 : 0;
    hipLaunchKernelGGL(attn_prefill_prologue_kernel<128>, dim3(a.batch), dim3(kThreads), lds, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!a.plan || a.n_items <= 0) {
        hipLaunchKernelGGL(attn_prefill_kernel, dim3(a.n_kv_heads, nblk), dim3(kThreads), 0, stream, p);
        return hipGetLastError();
    }
    p.plan = a.plan;
    p.part_o = a.part;
    p.part_ml = a.part + static_cast<size_t>(a.part_slots) * a.n_kv_heads * kPfRows * 128;
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(a.n_kv_heads, a.n_items), dim3(kThreads), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess || a.n_split == 0) return e;
    hipLaunchKernelGGL(attn_prefill_merge_kernel, dim3(a.n_kv_heads, a.n_split, kPfRows * 128 / 4 / kThreads),
                       dim3(kThreads), 0, stream, p, a.plan + 4 * a.n_items);
    return hipGetLastError();
}

size_t attention_workspace_bytes(int32_t n_heads, int32_t head_dim, int32_t window) {
    // upper bound over n_kv: chunks of at least 32 tokens, at most kMergeMaxSplit of them
    int32_t n_split = (window + 31) / 32;
    if (n_split > kMergeMaxSplit) n_split = kMergeMaxSplit;
    return sizeof(float) * static_cast<size_t>(n_split) * n_heads * (head_dim + 2) + 256;
}

size_t attention_workspace_need(const AttnArgs& a) {
    if (a.n_heads <= 0 || a.n_kv_heads <= 0 || a.pos < 0 || a.n_heads % a.n_kv_heads != 0) return 0;
    const int32_t G = a.n_heads / a.n_kv_heads;
    const bool mq = a.head_dim == 128 && G >= 16 && G <= kMqHeads && !a.norm_qk && !a.rope;
    const Plan pl = mq ? make_mq_plan(a.pos, a.sliding_window, a.n_kv_heads)
                       : make_plan(a.pos, a.sliding_window, a.n_kv_heads, G, a.head_dim);
    return sizeof(float) * static_cast<size_t>(pl.n_split) * a.n_heads * (a.head_dim + 2);
}

hipError_t launch_attention(const AttnArgs& a, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (a.n_heads <= 0 || a.n_kv_heads <= 0 || a.pos < 0) return hipErrorInvalidValue;
    if (a.n_heads % a.n_kv_heads != 0) return hipErrorInvalidValue;
    if (a.rope && a.rope->half * 2 != a.head_dim) return hipErrorInvalidValue;
    const uintptr_t al = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k_cache) |
                         reinterpret_cast<uintptr_t>(a.v_cache) | reinterpret_cast<uintptr_t>(a.out);
    if (al & 15u) return hipErrorInvalidValue;
    const int32_t G = a.n_heads / a.n_kv_heads;
    const bool mq = a.head_dim == 128 && G >= 16 && G <= kMqHeads && !a.norm_qk && !a.rope;
    const Plan pl = mq ? make_mq_plan(a.pos, a.sliding_window, a.n_kv_heads)
                       : make_plan(a.pos, a.sliding_window, a.n_kv_heads, G, a.head_dim);
    const size_t need_o = sizeof(float) * static_cast<size_t>(pl.n_split) * a.n_heads * a.head_dim;
    const size_t need_ml = sizeof(float) * static_cast<size_t>(pl.n_split) * a.n_heads * 2;
    if (need_o + need_ml > workspace_bytes) return hipErrorInvalidValue;
    float* part_o = static_cast<float*>(workspace);
    float* part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + need_o);
    if (mq) return launch_mq(a, pl, part_o, part_ml, stream);
    switch (a.head_dim) {
    case 64: return launch_hd<64>(a, pl, part_o, part_ml, stream);
    case 128: return launch_hd<128>(a, pl, part_o, part_ml, stream);
    case 256: return launch_hd<256>(a, pl, part_o, part_ml, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace gncx
