// streamer_replay.cpp -- GNCXStreamer:forward_token for a Qwen3 model
// (lua/gncx_streamer.lua:759-965), issued call for call through the C-ABI
// of gncx_llm_core.so from native code, the way LuaJIT's FFI issues it: the
// same entry points, arguments and buffers, the residual loops on the host
// buffers, no interpreter between the calls.  It is a caller of the library
// (a separate shared object that links against it), used to measure what the
// unchanged streamer gets; it is not part of the drop-in.
#include <cstdint>

#include "../../include/gncx_llm_core.h"

#define REPLAY_API extern "C" __attribute__((visibility("default")))

// One token at pos.  s->hidden[0] .. s->logits are the streamer's scratch
// buffers (lua/gncx_streamer.lua:461-477), s->k_cache / v_cache its per-layer
// caches; tokens / quant_scale its 4-phase arrays (:486-487); crivo_k[l] each
// layer's sieve order (:502-511) and layer_k the final norm's.  Returns
// gncx_hip_last_status() (0 when every call succeeded).
REPLAY_API int gncx_replay_forward_token(const GNCXDecodeModel* m, const GNCXDecodeState* s,
                                         GNCXCompactToken* tokens, float* quant_scale, GNCXTelemetryStats* telemetry,
                                         const int32_t* crivo_k, int32_t layer_k, int32_t token, int32_t pos,
                                         int32_t compute_logits) {
    const uint8_t* base = static_cast<const uint8_t*>(m->base);
    const int32_t E = m->embed, H = m->n_heads, KV = m->n_kv_heads, hd = m->head_dim, F = m->ffn;
    const int32_t qd = H * hd, kvd = KV * hd;
    float* h = static_cast<float*>(s->hidden[0]);
    float* nrm = static_cast<float*>(s->normed);
    float* q = static_cast<float*>(s->q);
    float* k = static_cast<float*>(s->k);
    float* v = static_cast<float*>(s->v);
    float* at = static_cast<float*>(s->attn);
    float* pr = static_cast<float*>(s->proj);
    float* ga = static_cast<float*>(s->gate);
    float* up = static_cast<float*>(s->up);
    float* ac = static_cast<float*>(s->act);
    // 1. the token's embedding row (:766, :698-713; scale 1 for Qwen3)
    switch (m->token_embd.ggml_type) {
    case GNCX_Q8_0: gncx_fetch_token_embedding_q8_0(base, m->token_embd.offset, token, E, 1.0f, h); break;
    case GNCX_Q6_K: gncx_fetch_token_embedding_q6_k(base, m->token_embd.offset, token, E, 1.0f, h); break;
    case GNCX_BF16: gncx_fetch_token_embedding_bf16(base, m->token_embd.offset, token, E, 1.0f, h); break;
    default: return -1;
    }
    auto matvec = [&](const GNCXDecodeTensor& t, const float* x, const GNCXCompactToken* tk, int32_t in_dim,
                      int32_t out_dim, float* y) {
        gncx_xfold_universal_matvec(base, t.offset, t.ggml_type, x, tk, in_dim, out_dim, y, telemetry);
    };
    // 2. the layers (:780-957)
    for (int32_t l = 0; l < m->n_layers; ++l) {
        const GNCXDecodeLayer& L = m->layers[l];
        gncx_rmsnorm_and_encode_4phase(h, base, L.attn_norm.offset, E, m->eps, crivo_k[l], nrm, tokens, quant_scale);
        matvec(L.attn_q, nrm, tokens, E, qd, q);
        matvec(L.attn_k, nrm, tokens, E, kvd, k);
        matvec(L.attn_v, nrm, tokens, E, kvd, v);
        if (m->qk_norm) {
            gncx_rmsnorm_inplace_heads(q, base, L.attn_q_norm.offset, 1, H, hd, m->eps);
            gncx_rmsnorm_inplace_heads(k, base, L.attn_k_norm.offset, 1, KV, hd, m->eps);
        }
        gncx_apply_rope_xor11_ext(q, k, tokens, nullptr, 0, 0, H, KV, hd, pos, m->rope_base);
        gncx_mqa_attention_step_ext(q, k, v, static_cast<float*>(s->k_cache[l]), static_cast<float*>(s->v_cache[l]),
                                    pos, H, KV, hd, m->attn_scale, 0, 1, at);
        matvec(L.attn_output, at, nullptr, qd, E, pr);
        for (int32_t i = 0; i < E; ++i) h[i] = h[i] + pr[i];
        gncx_rmsnorm_and_encode_4phase(h, base, L.ffn_norm.offset, E, m->eps, crivo_k[l], nrm, tokens, quant_scale);
        matvec(L.ffn_gate, nrm, tokens, E, F, ga);
        matvec(L.ffn_up, nrm, tokens, E, F, up);
        gncx_swiglu_activation(ga, up, F, ac);
        matvec(L.ffn_down, ac, nullptr, F, E, pr);
        for (int32_t i = 0; i < E; ++i) h[i] = h[i] + pr[i];
    }
    // 3. the final norm and the tied lm_head (:936-962)
    if (compute_logits) {
        gncx_rmsnorm_and_encode_4phase(h, base, m->output_norm.offset, E, m->eps, layer_k, nrm, tokens, quant_scale);
        gncx_universal_lm_head_logits(base, m->token_embd.offset, m->token_embd.ggml_type, nrm, E, m->vocab, 0.0f,
                                      static_cast<float*>(s->logits));
    }
    return gncx_hip_last_status();
}
