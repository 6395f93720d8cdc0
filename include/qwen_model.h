/* Model description shared by the host engine, the CPU oracle and the Python
 * harness: the text config of a Qwen3.5 hybrid (Gated DeltaNet + gated GQA
 * attention) and the fixed order in which its tensors are handed over.
 *
 * The fields are the subset of the reference's `TextConfig`
 * (src/weights.rs:27-45) that the forward pass reads, already resolved the way
 * `model_from_tensors` resolves them (src/weights.rs:187-337): rotary_dim =
 * head_dim * partial_rotary_factor, one flag per layer for
 * "full_attention" versus "linear_attention".
 *
 * Tensors are row-major fp32 host arrays ([out, in] for matrices, as
 * `Matrix`, src/tensor.rs:138-146). They are passed as an array of
 * QW_SLOTS_BASE + num_layers * QW_SLOTS_LAYER pointers in this order:
 *
 *   0  model.language_model.embed_tokens.weight      [vocab, hidden] (tied lm_head)
 *   1  model.language_model.norm.weight              [hidden]
 *   then per layer L, at 2 + L * QW_SLOTS_LAYER + slot:
 *   0  input_layernorm.weight                        [hidden]
 *   1  post_attention_layernorm.weight               [hidden]
 *   2  mlp.gate_proj.weight                          [intermediate, hidden]
 *   3  mlp.up_proj.weight                            [intermediate, hidden]
 *   4  mlp.down_proj.weight                          [hidden, intermediate]
 *   full_attention layers:
 *   5  self_attn.q_proj.weight   [2*heads*head_dim, hidden]  (per head [Q | gate])
 *   6  self_attn.k_proj.weight   [kv_heads*head_dim, hidden]
 *   7  self_attn.v_proj.weight   [kv_heads*head_dim, hidden]
 *   8  self_attn.o_proj.weight   [hidden, heads*head_dim]
 *   9  self_attn.q_norm.weight   [head_dim]
 *   10 self_attn.k_norm.weight   [head_dim]
 *   linear_attention (Gated DeltaNet) layers:
 *   5  linear_attn.in_proj_qkv.weight [channels, hidden], channels = 2*kh*dk + vh*dv
 *   6  linear_attn.in_proj_z.weight   [vh*dv, hidden]
 *   7  linear_attn.in_proj_a.weight   [vh, hidden]
 *   8  linear_attn.in_proj_b.weight   [vh, hidden]
 *   9  linear_attn.conv1d.weight      [channels, conv_kernel]
 *   10 linear_attn.dt_bias           [vh]
 *   11 linear_attn.A_log             [vh]
 *   12 linear_attn.norm.weight       [dv]
 *   13 linear_attn.out_proj.weight   [hidden, vh*dv]
 * Unused slots are NULL.
 */
#ifndef QWEN_MODEL_H
#define QWEN_MODEL_H
#include <stdint.h>

#define QW_MAX_LAYERS 256
#define QW_SLOTS_BASE 2
#define QW_SLOTS_LAYER 15

enum QwSlot {
    QW_INPUT_NORM = 0, QW_POST_NORM = 1, QW_GATE = 2, QW_UP = 3, QW_DOWN = 4,
    QW_Q = 5, QW_K = 6, QW_V = 7, QW_O = 8, QW_Q_NORM = 9, QW_K_NORM = 10,
    QW_QKV = 5, QW_Z = 6, QW_A = 7, QW_B = 8, QW_CONV = 9, QW_DT = 10, QW_A_LOG = 11,
    QW_DELTA_NORM = 12, QW_OUT = 13
};

typedef struct QwConfig {
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t num_layers;
    int32_t vocab_size;
    int32_t num_heads;      /* attention query heads */
    int32_t num_kv_heads;   /* attention KV heads (GQA) */
    int32_t head_dim;
    int32_t rotary_dim;     /* partial RoPE: first rotary_dim dims of each head */
    int32_t key_heads;      /* DeltaNet key heads */
    int32_t value_heads;    /* DeltaNet value heads */
    int32_t key_dim;
    int32_t value_dim;
    int32_t conv_kernel;
    int32_t max_positions;
    float rms_norm_eps;
    float rope_theta;
    uint8_t attention[QW_MAX_LAYERS]; /* 1 = full_attention, 0 = linear_attention */
} QwConfig;

#endif
