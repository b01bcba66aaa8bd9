/*
 * gncx_oracle.h -- CPU restatement of GNC-X's quantized linear-algebra path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (gnc-x_amd/) never links, loads or falls back to it.
 *
 * Every function restates one reference routine of
 * csrc/gncx_llm_kernels.cpp (cited per function in gncx_oracle.c) as plain
 * scalar C compiled with -ffp-contract=off; matvec / matbatch / lm_head split
 * their output rows over pthreads, each row computed by one thread, so the
 * results do not depend on the thread count.  Integer and byte
 * work (fp16 decode, block dequantisation, Q8 activation quantisation, block
 * integer dots) is bit-exact with the reference; float accumulation follows
 * the reference's association but not its compiler's FMA contraction.
 */
#ifndef GNCX_ORACLE_H
#define GNCX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids understood by the path (cpp:1362-1462). */
enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14, ORC_BF16 = 30 };

/* One quantised 32-wide activation block (cpp:299-306, without the pad). */
typedef struct {
    float   d;
    int32_t sum;
    int32_t sum_lo16;
    int32_t sum_hi16;
    int8_t  qs[32];
} orc_act_q8;

float    orc_fp16_to_fp32(uint16_t h);
float    orc_bf16_to_fp32(uint16_t b);
size_t   orc_row_bytes(int32_t type, int32_t k);
/* Threads used by the row-parallel functions ($ORC_THREADS, else the online
 * CPUs, at most 16). */
int32_t  orc_threads(void);

void     orc_quantize_act_q8(const float* x, int32_t k, orc_act_q8* out);

/* Dequantise one row of k weights of the given type into fp32. */
void     orc_dequant_row(int32_t type, const uint8_t* row, int32_t k, float* out);

/* Block dots against quantised activations. */
float    orc_dot_row(int32_t type, const uint8_t* row, const orc_act_q8* act, int32_t k,
                     const float* x_fp32);

void     orc_matvec(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t n, float* y);
void     orc_matbatch(int32_t type, const uint8_t* w, const float* x, int32_t b, int32_t k,
                      int32_t n, float* y);
void     orc_lm_head(int32_t type, const uint8_t* w, const float* x, int32_t k, int32_t vocab,
                     float softcap, float* y);

void     orc_rmsnorm(const float* x, const float* gamma, int32_t dim, float eps, float* out);
void     orc_rmsnorm_heads(float* v, const float* gamma, int32_t n_heads, int32_t head_dim,
                           float eps);
void     orc_rope_table(int32_t pos, int32_t head_dim, float freq_base, const float* freq_factors,
                        float* cos_t, float* sin_t);
void     orc_rope(float* q, float* k, const float* freq_factors, int32_t n_heads,
                  int32_t n_kv_heads, int32_t head_dim, int32_t pos, float freq_base);
void     orc_attention_step(const float* q, const float* k_new, const float* v_new, float* k_cache,
                            float* v_cache, int32_t pos, int32_t n_heads, int32_t n_kv_heads,
                            int32_t head_dim, float scale, int32_t sliding_window,
                            int32_t write_kv, float* out);
/* b consecutive attention steps at pos0 .. pos0 + b - 1 over caches that
 * already hold those rows; q and out are [b][n_heads * head_dim]. */
void     orc_attention_prefill(const float* q, const float* k_cache, const float* v_cache, int32_t pos0,
                               int32_t b, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                               int32_t sliding_window, float* out);
void     orc_swiglu(const float* gate, const float* up, int32_t n, float* out);
void     orc_geglu(const float* gate, const float* up, int32_t n, float* out);
float    orc_encode_4phase(const float* v, int32_t dim, int32_t layer_k, uint32_t* tokens);
void     orc_fetch_embedding(int32_t type, const uint8_t* table, int32_t token, int32_t dim,
                             float scale, float* out);

#ifdef __cplusplus
}
#endif
#endif
