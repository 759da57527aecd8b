/* gpt_capi.h - C ABI of the GPT training-step harness around the attention path.
 *
 * The harness is the caller of the attention path in the reference: TransformerModel's
 * forward and backward (src/model.cu:248-704) with embedding, pre-LN blocks (LayerNorm, QKV
 * projection, causal attention, out projection + residual, LayerNorm, FFN with tanh GELU +
 * residual), final LayerNorm, LM head, mean cross-entropy, and the fused clip + AdamW +
 * zero-grad optimizer step (src/optimizer.cu:117-154, driven as in src/benchmark.cu:195).
 * fp32 throughout; GEMMs on rocBLAS; the attention through libtcamd_attn (attn_capi.h).
 *
 * Parameters live in one flat buffer in the reference's order (src/model.cu:185-217):
 * tok_emb (V,C), pos_emb (T,C), per layer [ln1 gamma, beta (C), qkv_w (C,3C), qkv_b (3C),
 * proj_w (C,C), proj_b (C), ln2 gamma, beta (C), ffn1_w (C,F), ffn1_b (F), ffn2_w (F,C),
 * ffn2_b (C)], ln_f gamma, beta (C), head_w (C,V); weights stored (in, out), row-major.
 * The gradient buffer has the same layout.  Every call returns 0 or an attn status code.
 * No counterpart in the reference as a C ABI (the reference drives the model from C++).
 */
#ifndef TCAMD_GPT_CAPI_H
#define TCAMD_GPT_CAPI_H

#include <hip/hip_runtime.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpt_model gpt_model;

/* Attention used inside the blocks. */
enum {
    GPT_ATTN_FUSED = 0,        /* attn_fused_causal_*: qkv in, merged heads out (3 launches) */
    GPT_ATTN_TILED_SPLIT = 1,  /* the reference's tiled sequence: split, tiled, head merge */
    GPT_ATTN_MATERIALIZED = 2, /* the reference's default: T x T scores and probabilities */
    GPT_ATTN_FUSED_X3 = 3      /* attn_fused_causal_*_f32x3: fp32 on the bf16 MFMA (three
                                  bf16 planes per operand); d_head 32 or 64 */
};

/* Mirrors TransformerConfig (include/config.h). */
typedef struct {
    int vocab_size, max_seq_len, d_model, num_layers, num_heads, d_ff, batch_size;
    float layernorm_eps, learning_rate, weight_decay, beta1, beta2, adam_eps, grad_clip;
    int attention_mode;
} gpt_config;

/* Fills the reference defaults (include/config.h) for the given shape. */
void gpt_default_config(gpt_config* cfg, int vocab_size, int max_seq_len, int d_model,
                        int num_layers, int num_heads, int d_ff, int batch_size);

/* Allocates parameters (zero), gradients, optimizer state and activations. */
int gpt_create(const gpt_config* cfg, gpt_model** out);
void gpt_destroy(gpt_model* model);
long long gpt_num_parameters(const gpt_model* model);

/* Host <-> device copies of the flat parameter / gradient buffers (synchronous). */
int gpt_set_parameters(gpt_model* model, const float* host, long long n);
int gpt_get_parameters(const gpt_model* model, float* host, long long n);
int gpt_get_gradients(const gpt_model* model, float* host, long long n);

/* The logits (B*T, V) of the last forward (synchronous copy). */
int gpt_get_logits(const gpt_model* model, float* host, long long n);

/* Forward + backward for tokens / targets (device int32, B*T each): the mean loss into
 * *loss_dev (device float) and every parameter gradient (overwritten). */
int gpt_forward_backward(gpt_model* model, const int* tokens, const int* targets,
                         float* loss_dev, hipStream_t stream);
/* Global-norm clip (grad_clip) + AdamW at learning_rate + zero the gradients. */
int gpt_optimizer_step(gpt_model* model, hipStream_t stream);

/* Record HIP events around every attention launch of the following steps (on = 1) and
 * report their summed duration of the last step in ms (synchronises on the events). */
int gpt_set_attention_timing(gpt_model* model, int on);
int gpt_last_attention_ms(gpt_model* model, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* TCAMD_GPT_CAPI_H */
