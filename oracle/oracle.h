/*
 * CPU oracle for scry-llm's int8 Llama forward path -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference CPU backend
 * (crates/scry-llm/src/backend/cpu.rs), the quantizer
 * (crates/scry-llm/src/quantize.rs), the Llama model
 * (crates/scry-llm/src/nn/llama.rs), the init helpers
 * (crates/scry-llm/src/nn/init.rs) and greedy generation
 * (crates/scry-llm/src/generate.rs).  Every function cites the reference
 * lines it follows.  It is compiled with -ffp-contract=off and no fast-math
 * against glibc libm so each f32/f64 operation happens in the same order and
 * precision as the Rust source.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / CPU baseline.  The product
 * (esolearn_amd/) never links or calls it.
 *
 * Parity status per function (how each is pinned) is listed in the header of
 * oracle.c.  The fastrand 2.3.0 stream (orc_rng_*) is "parity unpinned": no
 * reference test fixes any of its output values.
 */
#ifndef SCRY_ORACLE_H
#define SCRY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fastrand 2.3.0 (wyrand) restatement: parity unpinned ---- */
uint64_t orc_rng_u64_at(uint64_t seed, uint64_t call_index);
void orc_rng_fill_u64(uint64_t seed, uint64_t start_call, size_t n, uint64_t *out);
void orc_rng_fill_f64(uint64_t seed, uint64_t start_call, size_t n, double *out);

/* init.rs:2-14 -- n samples starting at stream call `start_call`
 * (sample j consumes calls start_call+2j and start_call+2j+1). */
void orc_normal_vec(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                    float *out);
/* same values, computed in parallel by jumping ahead in the additive state */
void orc_normal_vec_par(uint64_t seed, uint64_t start_call, size_t n, float mean, float stdv,
                        float *out);

/* ---- quantize.rs ---- */
void orc_quantize_symmetric(const float *w, size_t n, int8_t *q, float *scale);
void orc_dequantize(const int8_t *q, size_t n, float scale, float *out);
/* builder-defined block-32 variant: quantize_symmetric on each 32-long
 * k-block of each output column of W[k,n]; scales laid out [n][ceil(k/32)] */
void orc_quantize_block32(const float *w, int k, int n, int8_t *q, float *scales);

/* ---- cpu.rs int8 matmul ---- */
void orc_matmul_i8_f32_tiled(const float *a, const int8_t *bq, float scale, int m, int k, int n,
                             float *c);
void orc_matmul_i8_f32_par(const float *a, const int8_t *bq, float scale, int m, int k, int n,
                           float *c);
void orc_matmul_i8_f32_tb(const float *a, const int8_t *bq_nk, float scale, int m, int k, int n,
                          float *c);
void orc_matmul_i8_f32_b32(const float *a, const int8_t *bq, const float *scales, int m, int k,
                           int n, float *c);
void orc_matmul_i8_f32_bias(const float *a, const int8_t *bq, float scale, const float *bias,
                            int m, int k, int n, float *c);

/* ---- cpu.rs f32 matmul family ---- */
void orc_gemv_f32(const float *vec, const float *mat, int k, int n, float *out);
void orc_gemv_trans_b(const float *vec, const float *mat_t, int k, int n, float *out);
void orc_gemv_into(const float *vec, const float *mat, int k, int n, float *out);
void orc_matmul_f32(const float *a, const float *b, int m, int k, int n, int trans_a,
                    int trans_b, float *c);
void orc_matmul_strided_batched(const float *a, const float *b, int batch, int m, int k, int n,
                                int trans_a, int trans_b, float *c);
/* ---- the bf16 feature (kernels.rs:629-633, cuda.rs:1226-1290) ---- */
uint16_t orc_f32_to_bf16(float x);
void orc_f32_to_bf16_vec(const float *x, size_t n, uint16_t *out);
void orc_matmul_bf16(const float *a, const float *b, int m, int k, int n, int trans_a, int trans_b,
                     float *c);
/* the same (trans_a = 0) on all cores, bit-identical */
void orc_matmul_bf16_par(const float *a, const float *b, int m, int k, int n, int trans_b, float *c);

/* ---- cpu.rs glue ops ---- */
void orc_rmsnorm(const float *x, const float *w, int rows, int d, float eps, float *out);
void orc_rope_with_freqs_preloaded(const float *x, int seq, int n_heads, int head_dim,
                                   int start_pos, const float *freqs, float *out);
void orc_scale(const float *x, size_t n, float s, float *out);
void orc_softmax(const float *x, int rows, int cols, float *out);
float orc_silu(float x);
void orc_swiglu(const float *gate, const float *up, size_t n, float *out);
void orc_add(const float *a, const float *b, size_t n, float *out);
int orc_embedding(const float *weight, const int64_t *idx, int n_idx, int vocab, int dim,
                  float *out);
void orc_repeat_kv(const float *x, int n_kv, int n_q, int seq, int d_head, float *out);
void orc_gather_reshape_repeat_kv(const float *cache, int max_seq, int cached_len, int n_kv,
                                  int n_q, int head_dim, float *out);
void orc_scatter_rows(float *dst, const float *src, int total_rows, int cols, int row_start,
                      int row_count);
void orc_causal_mask_scale(float *scores, int n_mat, int seq, float scale, float mask_value);
int64_t orc_argmax(const float *logits, int64_t n);
/* generate.rs:92-165 sample_token; *rng_state is a fastrand state
 * (Rng::with_seed(s) starts at s), advanced once per sampled token. */
int64_t orc_sample_token(const float *logits, int64_t n, float temperature, int64_t top_k, float top_p,
                         uint64_t *rng_state);
void orc_compute_rope_freqs(int head_dim, float theta, int has_scaling, double factor,
                            double low_freq_factor, double high_freq_factor,
                            int64_t original_max_pos, double *out);

/* ---- the rest of the trait surface (cpu.rs, mod.rs default bodies) ---- */
void orc_layernorm(const float *x, const float *gamma, const float *beta, int rows, int d, float eps,
                   float *out, float *mean_out, float *rstd_out);
float orc_gelu(float x);
void orc_gelu_vec(const float *x, size_t n, float *out);
float orc_sum(const float *x, size_t n);
void orc_mul(const float *a, const float *b, size_t n, float *out);
void orc_rope_rows(const float *x, size_t rows, int last_dim, int pos, int head_dim, float theta, float *out);
void orc_gather_columns(const float *x, int rows, int total, int start, int count, float *out);
void orc_scatter_columns(float *dst, const float *src, int rows, int total, int start, int count);
void orc_add_broadcast(const float *a, const size_t *ad, int an, const float *b, const size_t *bd, int bn,
                       const size_t *od, int on, float *out);
void orc_scaled_softmax(const float *x, int rows, int cols, float scale, float *out);
void orc_split_qkv_reshape_heads(const float *qkv, int seq, int n_heads, int d_head, float *q, float *k,
                                 float *v);
void orc_reshape_heads(const float *x, int batch, int seq, int n_heads, int d_head, int dir, float *out);

/* ---- llama.rs model ---- */
typedef struct {
    int32_t vocab_size, hidden_size, intermediate_size, n_layers, n_heads, n_kv_heads,
        max_seq_len;
    float rms_norm_eps, rope_theta;
    int32_t tie_word_embeddings;
    int32_t has_rope_scaling;
    double rs_factor, rs_low_freq_factor, rs_high_freq_factor;
    int64_t rs_original_max_pos;
} orc_llama_config;

/* tensor ids for orc_llama_tensor / orc_llama_qtensor */
enum {
    ORC_T_EMBED = 0,   /* [V,h] f32 */
    ORC_T_QKV = 1,     /* [h, q+2kv] */
    ORC_T_O = 2,       /* [q_dim, h] */
    ORC_T_GATE = 3,    /* [h, ffn] */
    ORC_T_UP = 4,      /* [h, ffn] */
    ORC_T_DOWN = 5,    /* [ffn, h] */
    ORC_T_LM_HEAD = 6, /* [V, h]; tied -> int8 copy of the embedding */
    ORC_T_ROPE_FREQS = 7 /* [hd/2] f32 */
};

typedef struct orc_llama orc_llama;
typedef struct orc_cache orc_cache;

/* LlamaModel::new (llama.rs:593-680) with fastrand::Rng::with_seed(seed);
 * quantize != 0 additionally builds the int8 copy of every projection
 * (build-defined composition: quantize_symmetric per tensor).
 * keep_f32 == 0 frees the f32 projection weights after quantizing. */
orc_llama *orc_llama_new(const orc_llama_config *cfg, uint64_t seed, int quantize, int keep_f32,
                         int block32);
void orc_llama_free(orc_llama *m);
orc_llama *orc_llama_new_empty(const orc_llama_config *cfg);
int orc_llama_set_qtensor(orc_llama *m, int id, int layer, const int8_t *q, float scale);
int orc_llama_set_qtensor_b32(orc_llama *m, int id, int layer, const int8_t *q32, const float *s32);
int orc_llama_set_embed(orc_llama *m, const float *w);
/* RMSNorm weight `which` (0 input, 1 post-attention: of `layer`; 2 final) and
 * the eps of every norm, as from_safetensors loads them (llama.rs:880-914). */
int orc_llama_set_norm(orc_llama *m, int which, int layer, const float *w, float eps);
uint64_t orc_llama_rng_calls(const orc_llama *m);
/* copies a tensor out; returns element count (0 if absent) */
size_t orc_llama_tensor(const orc_llama *m, int id, int layer, float *out);
size_t orc_llama_qtensor(const orc_llama *m, int id, int layer, int8_t *out, float *scale);
size_t orc_llama_qscales_b32(const orc_llama *m, int id, int layer, float *out);

orc_cache *orc_cache_new(const orc_llama *m, int max_seq);
void orc_cache_free(orc_cache *c);
int orc_cache_len(const orc_cache *c, int layer);
void orc_cache_layer(const orc_cache *c, int layer, float *k_out, float *v_out);

/* LlamaModel::forward_with_llama_cache (llama.rs:744-763);
 * mode 0 = reference f32 weights, 1 = int8 per-tensor, 2 = int8 block-32,
 * 3 = the bf16 feature (bf16 weights and activations, f32 result) */
int orc_llama_forward_with_cache(const orc_llama *m, orc_cache *c, int64_t token, int pos,
                                 int mode, float *logits);
/* LlamaModel::forward (llama.rs:683-700): logits [seq, V] */
int orc_llama_forward(const orc_llama *m, const int64_t *tokens, int seq, int mode,
                      float *logits);
/* generate() greedy (generate.rs:51-89 with temperature 0) */
/* generate.rs:51-89 generate(): returns the token count or < 0 on error. */
int orc_generate(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens, float temperature,
                 int64_t top_k, float top_p, uint64_t seed, int mode, int64_t *out_tokens, float *step_logits);
int orc_generate_greedy(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens,
                        int mode, int64_t *out_tokens, float *step_logits);

/* The cache path evaluated layer by layer (per-tensor int8, mode 1 only):
 * n tokens at positions pos0.. are appended to c, bit-identical to n calls of
 * orc_llama_forward_with_cache; logits (if n_logits > 0) receives the last
 * n_logits rows' logits [n_logits, V].  Returns 0, -1 (token out of range),
 * -2 (cache full), -3 (a projection has no per-tensor int8 weights) or -4. */
int orc_llama_forward_cache_seq(const orc_llama *m, orc_cache *c, const int64_t *tokens, int n,
                                int pos0, int n_logits, float *logits);
/* orc_generate_greedy(mode 1) on the layer-major path: same tokens,
 * bit-identical step logits. */
int orc_generate_greedy_fast(const orc_llama *m, const int64_t *prompt, int n_prompt, int max_tokens,
                             int64_t *out_tokens, float *step_logits);

/* threading: 0 = reference-faithful single-threaded loops; n>0 = bit-identical
 * parallel variants on n threads */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
