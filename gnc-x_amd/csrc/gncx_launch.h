// gncx_launch.h -- host-callable launchers for the HIP kernels.
//
// Every launcher takes device pointers only, enqueues on `stream` and returns
// hipSuccess or the error of the failed check/launch; none synchronises.  The
// host shim (gncx_shim.cpp) owns pointer classification, staging and the
// reference-compatible C-ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "gncx_formats.h"

namespace gncx {

// Largest in_dim the fused GEMV accepts (its quantised activations live in LDS).
constexpr int32_t kMaxGemvK = 40960;

// y[n] = W[n x k] . Q8(x[k])   (BF16: fp32 x)  -- quantises x inside the kernel.
hipError_t launch_gemv(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n,
                       float* y, hipStream_t stream);

// ys[i][ns[i]] = W_i[ns[i] x k] . Q8(x[k]) for up to kMaxGemvMats matrices of one
// type and k, in one launch when the band kernel takes the shape (x is
// quantised once per work-group for all of them); otherwise one launch each.
constexpr int32_t kMaxGemvMats = 4;
hipError_t launch_gemv_multi(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                             const float* x, int32_t k, float* const* ys, hipStream_t stream);

// A matvec(_multi) with the decode chain's neighbours fused in (ONE schedule
// shapes: 16 waves, whole rows, k <= 4096 for the prologue):
//   gamma != null  x = RMSNorm(h + r) * gamma (r may be null) is formed in
//                  every work-group, bit-identical with launch_add_rmsnorm;
//                  h + r is stored to h_out when given (h_out != h);
//   gamma == null  x is the input vector, as for launch_gemv_multi;
//   act != null    two matrices (gate, up) of equal rows: act = SiLU(gate.x) *
//                  (up.x), bit-identical with launch_swiglu; ys may be null.
// Returns hipErrorNotSupported when the shape does not fit (nothing launched).
struct GemvFusion {
    const float* x = nullptr;
    const float* h = nullptr;
    const float* r = nullptr;
    const float* gamma = nullptr;
    float eps = 0.0f;
    float* h_out = nullptr;
    float* act = nullptr;
};
hipError_t launch_gemv_fused(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns, int32_t k,
                             float* const* ys, const GemvFusion& f, hipStream_t stream);

// Per-32 Q8 quantisation of `rows` rows of k floats into q[rows*k] and
// meta[rows*k/32] (used by matbatch and the dequant tests).
hipError_t launch_act_quant(const float* x, int32_t rows, int32_t k, int8_t* q, ActMeta* meta,
                            hipStream_t stream);

// Dequantise n rows of k weights to fp32 (bit-exact block decoders).
hipError_t launch_dequant(int32_t type, const uint8_t* w, int32_t k, int32_t n, float* out,
                          hipStream_t stream);

// Y[b x n] = Q8(X[b x k]) . W^T  (per-row activation quantisation).  With up
// non-null, X is SwiGLU(x, up) (the values of gncx_swiglu_activation), formed
// by the quantisation pass (quantised types; BF16 weights: hipErrorNotSupported).
size_t matbatch_workspace_bytes(int32_t type, int32_t b, int32_t k, int32_t n);
hipError_t launch_matbatch(int32_t type, const uint8_t* w, const float* x, int32_t b, int32_t k,
                           int32_t n, float* y, void* workspace, size_t workspace_bytes,
                           hipStream_t stream, const float* up = nullptr);
// ys[i][b x ns[i]] = Q8(X) . W_i^T for count (1..4) matrices of one type
// sharing X: the activations are quantised once, and Q4_K matrices whose rows
// are whole tiles of the summed plan run as one launch.  Each output equals
// launch_matbatch's for that matrix.
size_t matbatch_multi_workspace_bytes(int32_t type, int32_t count, const int32_t* ns, int32_t b, int32_t k);
hipError_t launch_matbatch_multi(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                                 const float* x, int32_t b, int32_t k, float* const* ys, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream);
// launch_matbatch_multi of the RMSNorm (gamma, eps) of the rows h after the
// optional residual add h += r (r may be null; h is updated in place), the
// norm and the quantisation in one kernel: the outputs of
// launch_add_rmsnorm_rows (or launch_rmsnorm) into a buffer followed by
// launch_matbatch_multi on it.  hipErrorNotSupported where the fused form does
// not apply (not a one-launch Q4_K plan, K over 16384, unaligned rows): the
// caller then runs the two steps.
hipError_t launch_matbatch_multi_norm(int32_t type, int32_t count, const uint8_t* const* ws, const int32_t* ns,
                                      float* h, const float* r, const float* gamma, float eps, int32_t b, int32_t k,
                                      float* const* ys, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream);

// cos/sin of one RoPE position, computed on the host with the C library's
// powf/cosf/sinf exactly as the reference does (cpp:1779-1796), passed to
// the kernels by value.
constexpr int32_t kMaxRopeHalf = 256;
struct RopeTable {
    int32_t half;  // head_dim / 2
    float c[kMaxRopeHalf];
    float s[kMaxRopeHalf];
};

// Decode attention step (reference cpp:1887-1994) with split-K softmax.
struct AttnArgs {
    const float* q;        // [n_heads*hd]
    const float* k_new;    // [n_kv*hd] or null
    const float* v_new;    // [n_kv*hd] or null
    float* k_cache;        // [rows*n_kv*hd]
    float* v_cache;
    float* out;            // [n_heads*hd]
    int32_t pos, n_heads, n_kv_heads, head_dim;
    float scale;
    int32_t sliding_window, write_kv;
    // optional fused prologue applied to q and k_new before the scan:
    // per-head RMSNorm (cpp:895-953) then NEOX RoPE (cpp:1797-1862)
    int32_t norm_qk;          // 1 = RMSNorm q and k_new per head
    const float* q_gamma;     // may be null (no weight)
    const float* k_gamma;
    float eps;
    const RopeTable* rope;    // host table, null = no rotation
    float* q_out;             // prologue result for q written back (optional)
    float* k_out;             // prologue result for k_new written back (optional)
};
size_t attention_workspace_bytes(int32_t n_heads, int32_t head_dim, int32_t window);
// The workspace launch_attention(a, ...) uses for its split plan (at most
// attention_workspace_bytes); 0 for arguments it rejects.
size_t attention_workspace_need(const AttnArgs& a);

// Causal prefill of `batch` tokens at positions pos0 .. pos0 + batch - 1: per
// token the heads-RMSNorm + RoPE prologue (q and k in place), its K/V row
// stored, then attention over its own window, all tokens at once.
struct PrefillArgs {
    float* q;        // [batch][n_heads * head_dim]
    float* k;        // [batch][n_kv_heads * head_dim]
    const float* v;  // [batch][n_kv_heads * head_dim]
    float* k_cache;  // rows [0, pos0) already filled
    float* v_cache;
    float* out;      // [batch][n_heads * head_dim]
    int32_t pos0, batch, n_heads, n_kv_heads, head_dim;
    float scale;
    int32_t sliding_window;
    int32_t norm_qk;
    const float* q_gamma;
    const float* k_gamma;
    float eps;
    const float* rope;  // device [batch][head_dim]: cos[head_dim / 2] then sin, or null
    // key-split plan from attention_prefill_plan (device copy of its table),
    // or null; part: attention_prefill_part_floats(part_slots, n_kv_heads) floats
    const int32_t* plan = nullptr;
    int32_t n_items = 0, n_split = 0, part_slots = 0;
    float* part = nullptr;
};
// shapes the batched kernels take: head_dim 128, n_heads / n_kv_heads dividing 32
bool attention_prefill_supported(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim);
// host: the key-split plan of a call (n_items rows of 4 ints, then n_split
// block indices); false when the call takes no plan
bool attention_prefill_plan(const PrefillArgs& a, std::vector<int32_t>& tab, int32_t& n_items, int32_t& n_split);
int32_t attention_prefill_part_slots(const std::vector<int32_t>& tab, int32_t n_items, int32_t n_split);
size_t attention_prefill_part_floats(int32_t part_slots, int32_t n_kv_heads);
hipError_t launch_attention_prefill(const PrefillArgs& a, hipStream_t stream);
hipError_t launch_attention(const AttnArgs& a, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

// Per-head RMSNorm in place (reference cpp:895-953); gamma may be null.
hipError_t launch_rmsnorm_heads(float* v, const float* gamma, int32_t n_heads, int32_t head_dim,
                                float eps, hipStream_t stream);
// RMSNorm of `rows` vectors of dim (reference cpp:789-833).
hipError_t launch_rmsnorm(const float* x, const float* gamma, int32_t rows, int32_t dim, float eps,
                          float* out, hipStream_t stream);
// h += r, then out = RMSNorm(h) * gamma, one row of dim, in one kernel (the
// same arithmetic as launch_vec_add followed by launch_rmsnorm).
// rows contiguous rows: h[r] += d[r], out[r] = RMSNorm(h[r]) (as launch_add_rmsnorm per row)
hipError_t launch_add_rmsnorm_rows(float* h, const float* r, const float* gamma, int32_t rows, int32_t dim, float eps,
                                   float* out, hipStream_t stream);
hipError_t launch_add_rmsnorm(float* h, const float* r, const float* gamma, int32_t dim, float eps, float* out,
                              hipStream_t stream);
// NEOX RoPE with a host-computed cos/sin table (reference cpp:1797-1862).
hipError_t launch_rope(float* q, float* k, const RopeTable& table, int32_t n_heads,
                       int32_t n_kv_heads, int32_t head_dim, hipStream_t stream);
// SiLU(gate)*up (reference cpp:2038-2052).
hipError_t launch_vec_add(float* y, const float* x, int32_t n, hipStream_t stream);
hipError_t launch_swiglu(const float* gate, const float* up, int32_t n, float* out,
                         hipStream_t stream);
// GELU(tanh approximation)(gate)*up (reference cpp:2018-2033).
hipError_t launch_geglu(const float* gate, const float* up, int32_t n, float* out, hipStream_t stream);
// launch_rmsnorm of one row, then in the same kernel the 4-phase telemetry
// tokens of the result (reference cpp:842-889) as packed {phase, d,
// |residual|} words, the quant scale in qscale[0] and the cancellation count
// (uint32) in qscale[1]; layer_k clamped to [0, 17].  tokens and qscale may
// be page-locked host memory.
hipError_t launch_rmsnorm_encode(const float* x, const float* gamma, int32_t dim, float eps, float* out,
                                 int32_t layer_k, uint32_t* tokens, float* qscale, hipStream_t stream);
// tanh softcap in place (reference cpp:1726-1731).
hipError_t launch_softcap(float* y, int32_t n, float softcap, hipStream_t stream);
// One embedding row (reference cpp:693-780), scale folded like the reference.
hipError_t launch_fetch_embedding(int32_t type, const uint8_t* table, int32_t token, int32_t dim,
                                  float scale, float* out, hipStream_t stream);
// The same with the token read from device memory (tokens outside [0, vocab)
// leave out untouched).
// Rows of count tokens of a device table (ids checked by the caller) into
// out[count][dim], one launch.
hipError_t launch_fetch_embedding_rows(int32_t type, const uint8_t* table, const int32_t* tokens, int32_t count,
                                       int32_t dim, float scale, float* out, hipStream_t stream);
hipError_t launch_fetch_embedding_dev(int32_t type, const uint8_t* table, const int32_t* token, int32_t vocab,
                                      int32_t dim, float scale, float* out, hipStream_t stream);
// *out = index of the first largest of x[0..n) (NaN never wins); also *log when
// given.  x 16-byte aligned, n up to 4M; workspace of argmax_workspace_bytes(n).
size_t argmax_workspace_bytes(int32_t n);
hipError_t launch_argmax(const float* x, int32_t n, int32_t* out, int32_t* log, void* workspace, size_t ws_bytes,
                         hipStream_t stream);

// Fixed device scratch of the no-allocation decode step (noalloc.hip): a
// file-scope device array of kNoAllocScratchBytes per GPU.  The argmax
// partials use its first kNoAllocArgmaxBytes, the attention partials the
// rest.  noalloc_scratch returns this device's copy's address, looked up once
// per device (with that device current) and kept.
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
constexpr size_t kNoAllocArgmaxBytes = size_t{64} << 10;
hipError_t noalloc_scratch(int device, void** out);

}  // namespace gncx
