/*
 * gncx_llm_core.h -- C-ABI of gnc-x_amd/bin/gncx_llm_core.so, the MI355X
 * (gfx950) drop-in for the reference's bin/gncx_llm_core.so.
 *
 * Part 1 declares, with identical names and signatures, the reference entry
 * points of the quantized linear-algebra path; each cites the definition it
 * replaces in csrc/gncx_llm_kernels.cpp and the LuaJIT FFI declaration that
 * binds it in lua/gncx_streamer.lua.  Part 2 declares build-side extensions
 * that have no counterpart in the reference.
 *
 * Pointer rules (both parts): any pointer may be host memory (the reference
 * contract) or HIP device memory.  Host weights are uploaded once and cached
 * by address (weights are immutable for the life of the process, as in the
 * reference); host inputs are staged and host outputs are complete when the
 * call returns.  With device inputs and outputs the call is stream-ordered on
 * the library stream (gncx_hip_set_stream) and does not synchronise the host.
 * Calls are serialised internally; the library keeps the reference's one
 * piece of cross-call state, the matvec activation cache (cpp:1338-1358).
 *
 * Failures (no GPU, out of device memory, unsupported shape) print one line
 * to stderr, leave the outputs untouched and are reported by
 * gncx_hip_last_status()/gncx_hip_last_error().  Unknown ggml types leave the
 * output untouched, as in the reference (cpp:1362-1462).
 */
#ifndef GNCX_LLM_CORE_H
#define GNCX_LLM_CORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma pack(push, 1)
/* cpp:267-271; streamer.lua:17-21 */
typedef struct GNCXCompactToken {
    uint8_t phase_2bit;
    uint8_t diag_d;
    uint16_t abs_delta;
} GNCXCompactToken;

/* cpp:308-313; streamer.lua:23-28 */
typedef struct GNCXTelemetryStats {
    uint64_t total_macs_equivalent;
    uint64_t zero_origin_cancellations;
    uint64_t zero_weight_skips;
    uint64_t xfold_bucket_merges;
} GNCXTelemetryStats;
#pragma pack(pop)

/* ggml type ids accepted by the matvec/matbatch family (cpp:1362-1462) */
enum { GNCX_Q4_0 = 2, GNCX_Q8_0 = 8, GNCX_Q4_K = 12, GNCX_Q6_K = 14, GNCX_BF16 = 30 };

/* ---------------- Part 1: reference entry points ---------------------- */

/* y[out_dim] = W[out_dim x in_dim] . Q8(x).  Replaces cpp:1327-1471
 * (FFI: streamer.lua:108-118, called at streamer.lua:664-680). */
void gncx_xfold_universal_matvec(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                 const float* in_vec, const GNCXCompactToken* in_tokens, int32_t in_dim,
                                 int32_t out_dim, float* out_vec, GNCXTelemetryStats* telemetry);

/* Q4_0 alias of the above.  Replaces cpp:1476-1489. */
void gncx_xfold_q4_0_matvec(const uint8_t* mmap_base, size_t weight_abs_offset, const float* in_vec,
                            const GNCXCompactToken* in_tokens, int32_t in_dim, int32_t out_dim, float* out_vec,
                            GNCXTelemetryStats* telemetry);

/* Y[b x out_dim] = Q8(X[b x in_dim]) . W^T, row-major.  Replaces cpp:1495-1692
 * (FFI: streamer.lua:120-130, called at streamer.lua:682-696). */
void gncx_xfold_universal_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                                   const float* in_batch, int32_t batch_size, int32_t in_dim, int32_t out_dim,
                                   float* out_batch, GNCXTelemetryStats* telemetry);

/* Q4_0 alias.  Replaces cpp:1694-1707. */
void gncx_xfold_q4_0_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, const float* in_batch,
                              int32_t batch_size, int32_t in_dim, int32_t out_dim, float* out_batch,
                              GNCXTelemetryStats* telemetry);

/* matvec on the tied embedding + optional tanh softcap.  Replaces
 * cpp:1713-1732 (called at streamer.lua:953-962). */
void gncx_universal_lm_head_logits(const uint8_t* mmap_base, size_t embd_abs_offset, int32_t ggml_type,
                                   const float* final_hidden, int32_t embed_dim, int32_t vocab_size, float softcap,
                                   float* out_logits);

/* Q8_0 alias.  Replaces cpp:1734-1745. */
void gncx_q8_0_lm_head_logits(const uint8_t* mmap_base, size_t embd_abs_offset, const float* final_hidden,
                              int32_t embed_dim, int32_t vocab_size, float* out_logits);

/* GQA/MQA/SWA decode attention step with KV write at pos.  Replaces
 * cpp:1887-1994 (called at streamer.lua:848-862 and :1104-1108). */
void gncx_mqa_attention_step_ext(const float* q_vec, const float* k_vec, const float* v_vec, float* k_cache_layer,
                                 float* v_cache_layer, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                                 int32_t head_dim, float attn_scale, int32_t sliding_window, int32_t write_kv,
                                 float* out_attn_vec);

/* scale = 1/sqrt(head_dim), no window, write_kv = 1.  Replaces cpp:1996-2013. */
void gncx_mqa_attention_step(const float* q_vec, const float* k_vec, const float* v_vec, float* k_cache_layer,
                             float* v_cache_layer, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                             int32_t head_dim, float* out_attn_vec);

/* Per-head RMSNorm in place, optional fp32 gamma at base + offset.
 * Replaces cpp:895-953 (called at streamer.lua:817, :823). */
void gncx_rmsnorm_inplace_heads(float* vec, const uint8_t* mmap_base, size_t norm_weight_offset,
                                int32_t has_weight, int32_t n_heads, int32_t head_dim, float eps);

/* NEOX RoPE of q and k at pos; cos/sin built on the host with the C
 * library as the reference does.  Replaces cpp:1760-1863 (streamer.lua:831-843). */
void gncx_apply_rope_xor11_ext(float* q_vec, float* k_vec, GNCXCompactToken* q_tokens, const uint8_t* mmap_base,
                               size_t rope_freqs_offset, int32_t has_rope_freqs, int32_t n_heads,
                               int32_t n_kv_heads, int32_t head_dim, int32_t pos, float freq_base);

/* Replaces cpp:1865-1878. */
void gncx_apply_rope_xor11(float* q_vec, float* k_vec, GNCXCompactToken* q_tokens, int32_t n_heads,
                           int32_t n_kv_heads, int32_t head_dim, int32_t pos, float freq_base);

/* RMSNorm + optional 4-phase telemetry encode, both on the device.  Replaces
 * cpp:789-890 (called at streamer.lua:793-803, 877-887, 939-949). */
void gncx_rmsnorm_and_encode_4phase(const float* input_hidden, const uint8_t* mmap_base, size_t norm_weight_offset,
                                    int32_t dim, float eps, int32_t layer_k, float* out_normed_fp32,
                                    GNCXCompactToken* out_tokens, float* out_quant_scale);

/* SiLU(gate) * up.  Replaces cpp:2038-2052 (called at streamer.lua:894). */
void gncx_swiglu_activation(const float* gate_vec, const float* up_vec, int32_t ffn_dim, float* out_ffn_vec);

/* GELU (tanh approximation)(gate) * up.  Replaces cpp:2018-2033 (FFI:
 * streamer.lua:172-177, called at streamer.lua:896). */
void gncx_geglu_activation(const float* gate_vec, const float* up_vec, int32_t ffn_dim, float* out_ffn_vec);

/* One dequantised embedding row times scale_factor.  Replace cpp:693-715,
 * cpp:720-760 and cpp:765-780 (called at streamer.lua:698-713). */
void gncx_fetch_token_embedding_q8_0(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                     int32_t embed_dim, float scale_factor, float* out_hidden);
void gncx_fetch_token_embedding_q6_k(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                     int32_t embed_dim, float scale_factor, float* out_hidden);
void gncx_fetch_token_embedding_bf16(const uint8_t* mmap_base, size_t tensor_abs_offset, int32_t token_id,
                                     int32_t embed_dim, float scale_factor, float* out_hidden);

/* Weight file and host buffers (FFI: streamer.lua:30-47).  The file is
 * mapped read-only with read-ahead advice; buffers are page-locked host
 * memory (hipHostMalloc) when a HIP device is visible, anonymous pages
 * otherwise, starting at the address bits of the requested bank / L1-set
 * colour.  Unmapping, freeing or copying into a range drops the device
 * copies of weights and KV caches that live inside it.
 * Replace cpp:327-384, 386-389, 391-404, 617-667, 481-551, 553-559,
 * 561-574, 576-600 and 602-612 in that order. */
void* gncx_gla_map_readonly(const char* filepath, size_t* out_size);
const uint8_t* gncx_gla_get_base_ptr(void* opaque_handle);
void gncx_gla_unmap(void* opaque_handle);
void gncx_gla_prefetch_range(const uint8_t* mmap_base, size_t offset, size_t num_bytes);
void* gncx_ram_alloc_colored(size_t total_bytes, uint8_t k, uint8_t d, uint8_t R);
void* gncx_ram_alloc(size_t total_bytes);
uint8_t* gncx_ram_get_ptr(void* ram_handle);
uint8_t gncx_ram_get_ddr3_bank(void* ram_handle);
uint8_t gncx_ram_get_l1_set(void* ram_handle);
void gncx_ram_free(void* ram_handle);
void gncx_ram_copy_chunk(void* ram_handle, size_t dst_offset, const uint8_t* src_base, size_t src_offset,
                         size_t num_bytes);

/* Centre-relative layer coordinate.  Replaces cpp:672-686 with
 * gncx_genome_vm.hpp:35-60 (FFI: streamer.lua:49-57, called at
 * streamer.lua:502-511). */
void gncx_genome_get_layer_coordinate(int32_t layer_index, int32_t total_layers, int32_t base_k,
                                      int32_t* out_rel_layer, int32_t* out_dist_centro, int32_t* out_crivo_k,
                                      int32_t* out_hemisferio);

/* Diagonal slot manager that colours the KV-cache buffers.  Replaces
 * cpp:2059-2111 with gncx_geometric_mm.hpp (FFI: streamer.lua:188-194,
 * called at streamer.lua:514-564). */
void* gncx_geo_mm_create(uint32_t min_frames);
void gncx_geo_mm_destroy(void* handle);
int32_t gncx_geo_alloc(void* handle, uint8_t k_hint, uint8_t* out_k, uint8_t* out_d, uint8_t* out_R,
                       uint32_t* out_linear_idx);
void gncx_geo_free(void* handle, uint8_t k, uint8_t d, uint8_t R, uint32_t linear_idx);
float gncx_geo_fragmentation(void* handle);
size_t gncx_geo_used(void* handle);
size_t gncx_geo_capacity(void* handle);

/* Exported under the reference's names and signatures so that every binding
 * resolves, but NOT provided: a call records an error (gncx_hip_last_status),
 * prints it and leaves all outputs untouched; float results are 0.  They are
 * the LoRA / MeZO training primitives (cpp:2129-2331), the layer
 * visualisation point (cpp:2348-2435) and the embedding-model helpers
 * (cpp:2443-2654), none of which the quantized decode path calls
 * (FFI: streamer.lua:211-250). */
typedef struct GNCXLayer3DPoint GNCXLayer3DPoint; /* layout: streamer.lua:196-209 */
void gncx_lora_init_adapter(float* a_ptr, float* b_ptr, int32_t in_dim, int32_t out_dim, int32_t rank,
                            uint64_t seed);
void gncx_lora_forward_add(const float* in_vec, const float* a_ptr, const float* b_ptr, int32_t in_dim,
                           int32_t out_dim, int32_t rank, float scale, float* io_out_vec);
void gncx_lora_backward_step(const float* in_vec, const float* grad_out, float* a_ptr, float* b_ptr,
                             float* grad_in_accum, int32_t in_dim, int32_t out_dim, int32_t rank, float scale,
                             float lr, float weight_decay);
void gncx_mezo_perturb_params(float* params, int32_t num_params, uint64_t seed, float epsilon);
void gncx_mezo_update_params(float* params, int32_t num_params, uint64_t seed, float projected_grad, float lr,
                             float weight_decay);
float gncx_cross_entropy_loss(const float* logits, int32_t vocab_size, int32_t target_token_id,
                              float* out_grad_logits);
void gncx_project_layer_3d_point(int32_t layer_index, int32_t total_layers, const GNCXCompactToken* in_tokens,
                                 const float* normed_fp32, int32_t dim, GNCXLayer3DPoint* out_point);
float gncx_cosine_similarity(const float* u, const float* v, int32_t dim);
void gncx_vector_l2_normalize(float* vec, int32_t dim);
void gncx_mean_pooling(const float* hidden_batch, int32_t batch_size, int32_t dim, float* out_pooled);
void gncx_bidirectional_attention_gqa(const float* q_batch, const float* k_batch, const float* v_batch,
                                      int32_t batch_size, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                      float attn_scale, float* out_attn_batch);
void gncx_bidirectional_attention(const float* q_batch, const float* k_batch, const float* v_batch,
                                  int32_t batch_size, int32_t n_heads, int32_t head_dim, float attn_scale,
                                  float* out_attn_batch);

/* ---------------- Part 2: build-side extensions ----------------------- */
/* No counterpart in the reference. */

/* Select the HIP device (default: 0 or $GNCX_DEVICE).  0 or a HIP error. */
int gncx_hip_init(int device);
/* Stream the library enqueues on (hipStream_t; default: the null stream). */
void gncx_hip_set_stream(void* stream);
void* gncx_hip_get_stream(void);
/* hipStreamSynchronize of the library stream; 0 or a HIP error. */
int gncx_hip_synchronize(void);
/* Last failure message ("" when none). */
const char* gncx_hip_last_error(void);
/* Last failure code (0 when none); reading it clears it. */
int gncx_hip_last_status(void);
/* Drop the device copy of host weights at p (every copy when p is NULL). */
void gncx_hip_weight_forget(const void* p);
/* Drop the device twin of a host KV cache (every twin when p is NULL); call
 * after rewriting a host cache outside this library. */
void gncx_hip_kv_forget(const float* p);
/* Lazy coherence of the buffers from gncx_ram_alloc(_colored): 1 on, 0 off,
 * anything else only reports; returns the mode before the call (the initial
 * mode is 1 when the environment has GNCX_HOST_LAZY=1).  Buffers allocated
 * while it is on are ordinary pages with a device copy each: a call that
 * reads one uses the device copy in place (uploaded once when the host wrote
 * it), a call that writes one writes only the device copy and, when all its
 * outputs are such buffers or device memory, returns without waiting for
 * the device.  The host copy is brought back on the host's first access
 * (caught by page protection; a SIGSEGV handler is installed and chains to
 * the previous one).  A system call given a buffer the device holds fails
 * with EFAULT: call gncx_hip_host_flush first.  Turning the mode off brings
 * every buffer back to the host.  Off (the default), buffers are page-locked
 * and every call copies in and out and returns complete. */
int gncx_hip_set_host_coherence(int lazy);
/* Bring the buffer holding p (all buffers when p is NULL) back to the host:
 * current and read-write. */
void gncx_hip_host_flush(const void* p);
/* Device bytes held by uploaded weights. */
size_t gncx_hip_weight_bytes(void);
/* out[out_dim x in_dim] = fp32 decode of the weights with the block decoders
 * the dots use (bit-exact with cpp:85-112, 707-714, 734-759 and the implicit
 * Q4_0/Q4_K decoders of cpp:1023-1030, 1127-1178). */
void gncx_hip_dequantize(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type, int32_t in_dim,
                         int32_t out_dim, float* out);
/* Per-32 Q8 activation blocks of rows x in_dim values (cpp:955-995):
 * q[rows*in_dim] and meta[rows*in_dim/32][4] = {d as float bits, sum q[0:16],
 * sum q[16:32], sum q[0:32]}. */
void gncx_hip_quantize_act(const float* in, int32_t rows, int32_t in_dim, int8_t* q, int32_t* meta);
/* y[i] += x[i] for i < n: the residual adds that lua/gncx_streamer.lua:871-873
 * and :906-908 do on the host, for callers whose hidden state stays on the
 * device. */
void gncx_hip_vec_add(float* y, const float* x, int32_t n);
/* One launch doing gncx_rmsnorm_inplace_heads(q), gncx_rmsnorm_inplace_heads(k),
 * gncx_apply_rope_xor11_ext(q, k) and gncx_mqa_attention_step_ext with the
 * same results; q_vec/k_vec receive the normalised, rotated vectors.
 * rope_base <= 0 skips the rotation.  With write_kv == 0, k_vec is unused. */
void gncx_hip_attention_step_fused(float* q_vec, float* k_vec, const float* v_vec, float* k_cache_layer,
                                   float* v_cache_layer, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                                   int32_t head_dim, float attn_scale, int32_t sliding_window, int32_t write_kv,
                                   const uint8_t* mmap_base, size_t q_norm_offset, size_t k_norm_offset,
                                   int32_t has_norm_weight, float norm_eps, size_t rope_freqs_offset,
                                   int32_t has_rope_freqs, float rope_base, float* out_attn_vec);

/* Extensions with no counterpart in the reference, for callers that keep the
 * hidden state on the device and want fewer launches per token (the streamer
 * issues one gncx_xfold_universal_matvec per matrix, lua/gncx_streamer.lua:
 * 806-809 and 890-891, and adds residuals on the host, :871-873 and :906-908).
 *
 * out_vecs[i][out_dims[i]] = W_i . x for count (1..4) matrices of one
 * ggml_type and in_dim, e.g. Q/K/V or gate/up; weights[i] points at each
 * tensor (host or device, like mmap_base + offset), x is quantised once.  Each
 * output equals what gncx_xfold_universal_matvec gives for that matrix. */
void gncx_hip_matvec_multi(int32_t count, const uint8_t* const* weights, const int32_t* out_dims,
                           int32_t ggml_type, const float* in_vec, int32_t in_dim, float* const* out_vecs);
/* out_batches[i][batch][out_dims[i]] = the gncx_xfold_universal_matbatch
 * product of W_i and in_batch [batch][in_dim] for count (1..4) matrices of
 * one ggml_type, e.g. Q/K/V or gate/up of a prefill (lua/gncx_streamer.lua
 * 1068-1071 and 1135-1136 issue them one call each).  Q4_K matrices whose rows
 * are whole tiles of one launch plan share one launch, and the batch is then
 * quantised once; otherwise each matrix is a call of its own, which quantises
 * the batch again.  Each output is the single call's result to within fp32
 * summation order (a single call may split K for a small matrix). */
void gncx_hip_matbatch_multi(int32_t count, const uint8_t* const* weights, const int32_t* out_dims,
                             int32_t ggml_type, const float* in_batch, int32_t batch_size, int32_t in_dim,
                             float* const* out_batches);
/* out_rows[count][embed_dim] = the rows of token_ids[0..count) (host memory,
 * each in [0, vocab_size)) of the embedding table at mmap_base +
 * tensor_abs_offset (Q8_0, Q6_K or BF16) times scale_factor, in one launch:
 * the values of gncx_fetch_token_embedding_* per token (the streamer's prefill
 * fetches one row per call, lua/gncx_streamer.lua:1001-1003). */
void gncx_hip_fetch_token_embeddings(int32_t ggml_type, const uint8_t* mmap_base, size_t tensor_abs_offset,
                                     const int32_t* token_ids, int32_t count, int32_t vocab_size, int32_t embed_dim,
                                     float scale_factor, float* out_rows);
/* gncx_hip_attention_step_fused (write_kv = 1) for tokens pos0 .. pos0 +
 * batch - 1 in turn, as one causal batch: q_batch [batch][n_heads*head_dim],
 * k_batch / v_batch [batch][n_kv_heads*head_dim] (q and k receive the
 * normalised, rotated rows), out_batch [batch][n_heads*head_dim], cache rows
 * [0, pos0) already filled.  For the streamer's per-token prefill loop
 * (lua/gncx_streamer.lua:1079-1109). */
void gncx_hip_attention_prefill(float* q_batch, float* k_batch, const float* v_batch, float* k_cache_layer,
                                float* v_cache_layer, int32_t pos0, int32_t batch, int32_t n_heads,
                                int32_t n_kv_heads, int32_t head_dim, float attn_scale, int32_t sliding_window,
                                const uint8_t* mmap_base, size_t q_norm_offset, size_t k_norm_offset,
                                int32_t has_norm_weight, float norm_eps, size_t rope_freqs_offset,
                                int32_t has_rope_freqs, float rope_base, float* out_batch);
/* The RMSNorm of gncx_rmsnorm_and_encode_4phase (no tokens) of each of `rows`
 * contiguous vectors of dim, one launch (the streamer normalises prefill
 * rows one call each, lua/gncx_streamer.lua:1059-1065 and 1126-1132). */
void gncx_hip_rmsnorm_rows(const float* in, int32_t rows, const uint8_t* mmap_base, size_t norm_weight_offset,
                           int32_t dim, float eps, float* out);
/* hidden[i] += delta[i], then out_normed_fp32 = the RMSNorm of
 * gncx_rmsnorm_and_encode_4phase (cpp:789-833) of the new hidden, in one
 * kernel; the same values as gncx_hip_vec_add followed by that call. */
void gncx_hip_add_rmsnorm(float* hidden, const float* delta, const uint8_t* mmap_base, size_t norm_weight_offset,
                          int32_t dim, float eps, float* out_normed_fp32);
/* gncx_hip_add_rmsnorm over `rows` contiguous rows of dim in one launch: the
 * prefill's residual add followed by the next RMSNorm of every batch row
 * (lua/gncx_streamer.lua:1122 then :1126-1132, and :1153 then the next
 * layer's :1059-1065); the same values as gncx_hip_vec_add of the rows
 * followed by gncx_hip_rmsnorm_rows. */
void gncx_hip_add_rmsnorm_rows(float* hidden, const float* delta, int32_t rows, const uint8_t* mmap_base,
                               size_t norm_weight_offset, int32_t dim, float eps, float* out);
/* out_batch = gncx_xfold_universal_matbatch of W over the rows
 * gncx_swiglu_activation(gate_batch, up_batch) would write, with the SwiGLU
 * formed inside the matbatch's activation pass (the prefill's down
 * projection, lua/gncx_streamer.lua:1138-1142); the same values as the two
 * calls.  Inputs of batch_size x in_dim, output batch_size x out_dim. */
void gncx_hip_swiglu_matbatch(const uint8_t* mmap_base, size_t weight_abs_offset, int32_t ggml_type,
                              const float* gate_batch, const float* up_batch, int32_t batch_size, int32_t in_dim,
                              int32_t out_dim, float* out_batch);

/* The decode chain's neighbours fused into a matvec launch, for callers whose
 * activations are device memory (weights may be host or device memory, as
 * mmap_base + offset).
 *
 * out_vecs[i] = W_i . x with x = the RMSNorm of gncx_rmsnorm_and_encode_4phase
 * (no tokens) of hidden + delta (delta may be NULL), formed inside the launch;
 * hidden_out (NULL, or a buffer other than hidden) receives hidden + delta.
 * The same values as gncx_hip_add_rmsnorm followed by gncx_hip_matvec_multi
 * (lua/gncx_streamer.lua:871-880 then :806-809). */
void gncx_hip_matvec_multi_addnorm(const float* hidden, const float* delta, const uint8_t* mmap_base,
                                   size_t norm_weight_offset, float eps, float* hidden_out, int32_t count,
                                   const uint8_t* const* weights, const int32_t* out_dims, int32_t ggml_type,
                                   int32_t in_dim, float* const* out_vecs);
/* The prefill's form over batch_size rows (device memory): hidden += delta
 * (delta may be NULL, leaving hidden as it is), then out_batches[i] = W_i . x
 * with x the rows' RMSNorm, formed inside the matbatch's activation pass where
 * its plan allows (Q4_K matrices of one launch, in_dim up to 16384).  The
 * same values as gncx_hip_add_rmsnorm_rows (or gncx_hip_rmsnorm_rows) into a
 * buffer followed by gncx_hip_matbatch_multi of it (lua/gncx_streamer.lua
 * 1122 then 1126-1132 and 1135-1136; 1059-1065 then 1068-1071). */
void gncx_hip_matbatch_multi_addnorm(float* hidden, const float* delta, const uint8_t* mmap_base,
                                     size_t norm_weight_offset, float eps, int32_t count,
                                     const uint8_t* const* weights, const int32_t* out_dims, int32_t ggml_type,
                                     int32_t batch_size, int32_t in_dim, float* const* out_batches);
/* out_act = SiLU(W_gate . x) * (W_up . x) in one launch: the values of two
 * gncx_xfold_universal_matvec calls followed by gncx_swiglu_activation
 * (lua/gncx_streamer.lua:890-894). */
void gncx_hip_matvec_swiglu(const uint8_t* gate_weights, const uint8_t* up_weights, int32_t ggml_type,
                            const float* in_vec, int32_t in_dim, int32_t ffn_dim, float* out_act);

/* Native decode step: one token of GNCXStreamer:forward_token
 * (lua/gncx_streamer.lua:759-965) for a Qwen3/Llama-shaped model, every
 * launch issued by the library with the chain fused (per layer: Q/K/V with the
 * residual add + RMSNorm in its prologue; the attention step with the Q/K head
 * RMSNorm + RoPE prologue; O; gate/up with the add + RMSNorm prologue and the
 * SwiGLU epilogue; down), then the final RMSNorm and the tied lm_head into
 * state->logits.  Stream-ordered: nothing synchronises with the host.
 * token_id >= 0 is the input token; token_id < 0 reads it from
 * state->token.  greedy != 0 writes the argmax of the logits to
 * state->token (and to state->token_log[pos] when token_log is given), so a
 * loop of steps with token_id = -1 decodes greedily without host round trips.
 * Tensors are addressed like the streamer's (base + offset); every state
 * buffer is device memory.  Returns 0, or -1 with gncx_hip_last_error set. */
typedef struct GNCXDecodeTensor {
    size_t offset;
    int32_t ggml_type; /* layer matrices and token_embd; ignored for fp32 norms */
} GNCXDecodeTensor;
typedef struct GNCXDecodeLayer {
    GNCXDecodeTensor attn_norm, attn_q, attn_k, attn_v, attn_q_norm, attn_k_norm, attn_output, ffn_norm, ffn_gate,
        ffn_up, ffn_down;
} GNCXDecodeLayer;
typedef struct GNCXDecodeModel {
    const uint8_t* base;
    const GNCXDecodeLayer* layers; /* [n_layers] */
    GNCXDecodeTensor token_embd;   /* embedding table and tied lm_head */
    GNCXDecodeTensor output_norm;
    int32_t n_layers, embed, n_heads, n_kv_heads, head_dim, ffn, vocab;
    int32_t qk_norm; /* 1: per-head RMSNorm of q and k (Qwen3) */
    float eps, rope_base, attn_scale;
} GNCXDecodeModel;
typedef struct GNCXDecodeState {
    float* hidden[2]; /* [embed] each: the residual stream alternates between them */
    float* q;         /* [n_heads * head_dim] */
    float* k;         /* [n_kv_heads * head_dim] */
    float* v;
    float* attn;      /* [n_heads * head_dim] */
    float* proj;      /* [embed] */
    float* normed;    /* [embed] */
    float* gate;      /* [ffn] */
    float* up;
    float* act;
    float* logits;    /* [vocab] */
    float* const* k_cache; /* [n_layers] of [max_seq][n_kv_heads * head_dim] */
    float* const* v_cache;
    int32_t max_seq;
    int32_t* token;     /* [1] */
    int32_t* token_log; /* NULL or [max_seq] */
} GNCXDecodeState;
int gncx_hip_decode_step(const GNCXDecodeModel* model, const GNCXDecodeState* state, int32_t token_id, int32_t pos,
                         int32_t greedy);
/* gncx_hip_decode_step without any allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid it).  No counterpart in the reference.  Its scratch (attention
 * split-K partials and argmax partials) lives in a fixed device array of
 * 8 MiB per GPU, held until the process ends, instead of device memory the
 * library allocates; model->base and every state buffer must already be
 * device memory (nothing is uploaded).  A step needing more scratch than the
 * array holds (split plans of more than about 500 chunks, e.g. one KV head
 * at a context past 16k) is rejected with an error before anything is
 * enqueued.  Results are bit-identical with gncx_hip_decode_step.  Calls that
 * overlap on one GPU share the array and race; serialise them.  Returns 0, or
 * -1 with gncx_hip_last_error set. */
int gncx_hip_decode_step_noalloc(const GNCXDecodeModel* model, const GNCXDecodeState* state, int32_t token_id,
                                 int32_t pos, int32_t greedy);
/* *out_index = index of the first largest of values[0..n) (NaN never wins):
 * the greedy pick of the streamer's sampler without its repetition penalty
 * (lua/gncx_streamer.lua:1229-1272), on the device.  Device pointers; values
 * 16-byte aligned; n up to 4194304. */
void gncx_hip_argmax(const float* values, int32_t n, int32_t* out_index);

#ifdef __cplusplus
}
#endif
#endif
