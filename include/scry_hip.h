/*
 * scry_hip -- C ABI of the MI355X (gfx950) backend for scry-llm's int8 Llama
 * forward path.
 *
 * The reference boundary is Rust: `trait DeviceBackend` + `trait MathBackend`
 * (crates/scry-llm/src/backend/mod.rs:12-45, 48-622) behind the `quantize`
 * Cargo feature, with the Llama model in crates/scry-llm/src/nn/llama.rs and
 * the sampling loop in crates/scry-llm/src/generate.rs.  Each entry point
 * below names the reference item it replaces.  A Rust `HipBackend` maps
 * `Storage` to `scry_buf`, `I8Storage` to `scry_i8buf`, and panics on a
 * non-zero status, which is the reference's error behaviour (ops panic).
 *
 * Conventions
 *  - Every call returns 0 on success or a SCRY_ERR_* code; it never aborts.
 *    scry_hip_last_error() gives the message of the last failure on the
 *    calling thread.
 *  - Storage handles own device memory; the caller frees them.  Ops return
 *    newly allocated storage (the reference's functional style), except
 *    scatter_rows which writes in place like its `&mut` counterpart.
 *  - All work is queued on one HIP stream per process; to_vec calls
 *    synchronise, as the reference's to_vec does.  Calls from several host
 *    threads are serialised internally.
 *  - Only float32 storage and int8 weight storage exist, as in the
 *    reference's `quantize` feature (W8A32).
 */
#ifndef SCRY_HIP_H
#define SCRY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SCRY_OK = 0,
    SCRY_ERR_INVALID = 1,     /* bad argument or shape (the reference panics) */
    SCRY_ERR_HIP = 2,         /* HIP runtime error */
    SCRY_ERR_OOM = 3,         /* device allocation failed */
    SCRY_ERR_NOT_INIT = 4,    /* scry_hip_init not called / no device */
    SCRY_ERR_RANGE = 5,       /* index out of range (embedding id, cache full) */
    SCRY_ERR_UNSUPPORTED = 6  /* shape outside what the kernels implement */
};

typedef struct scry_buf_s *scry_buf;     /* f32 device storage (Storage)       */
typedef struct scry_i8buf_s *scry_i8buf; /* int8 weight storage (I8Storage)    */
typedef struct scry_llama_s *scry_llama; /* LlamaModel with int8 projections   */
typedef struct scry_kv_cache_s *scry_kv_cache; /* LlamaKvCache (device)        */

/* SamplingConfig (generate.rs:24-45): temperature (< 1e-8 means greedy),
 * top_k (0 or >= vocab: off), top_p (outside (0, 1): off), max_tokens. */
typedef struct {
    float temperature;
    int32_t top_k;
    float top_p;
    int32_t max_tokens;
} scry_sampling_config;

/* ---------------------------------------------------------------- runtime */
/* replaces cuda.rs:39-52 init_gpu (context, stream, kernel set) */
int scry_hip_init(int device);
int scry_hip_shutdown(void);
const char *scry_hip_last_error(void);
/* replaces cuda.rs:1193-1197 CudaBackend::synchronize */
int scry_hip_synchronize(void);
int scry_hip_device_count(int *count);
/* device name / CU count / gcnArch of the initialised device */
int scry_hip_device_info(char *name, size_t name_len, int *cu_count, char *arch,
                         size_t arch_len);

/* -------------------------------------------- DeviceBackend (mod.rs:12-45) */
/* DeviceBackend::zeros (mod.rs:23) */
int scry_hip_zeros(size_t n, scry_buf *out);
/* DeviceBackend::from_vec (mod.rs:25) */
int scry_hip_from_vec(const float *host, size_t n, scry_buf *out);
/* bf16 mode (the `bf16` feature): init_gpu_bf16 (cuda.rs:55-59) is
 * scry_hip_init + mode on.  In bf16 mode scry_hip_from_vec_with_bf16 keeps
 * the bf16 bytes only; scry_hip_matmul rounds both operands to bf16 with the
 * reference's cast and accumulates in f32 (bf16_ops::matmul_bf16,
 * cuda.rs:1226-1290); to_vec and embedding widen bf16-only storage; other
 * ops refuse it.  set_bf16_mode toggles the mode (tests). */
int scry_hip_init_bf16(int device);
int scry_hip_set_bf16_mode(int on);
int scry_hip_bf16_mode(int *on);
/* DeviceBackend::from_vec_with_bf16 (mod.rs:28-32, cuda.rs:230-240): bf16 is
 * n little-endian bf16 words; outside bf16 mode it is from_vec(host). */
int scry_hip_from_vec_with_bf16(const float *host, const uint16_t *bf16, size_t n, scry_buf *out);
/* DeviceBackend::to_vec (mod.rs:33); n must equal the storage length */
int scry_hip_to_vec(scry_buf b, float *host, size_t n);
/* DeviceBackend::clone_storage (mod.rs:44) */
int scry_hip_clone_storage(scry_buf src, scry_buf *out);
int scry_hip_buf_len(scry_buf b, size_t *n);
int scry_hip_free(scry_buf b);

/* DeviceBackend::i8_from_vec (mod.rs:17-18, `quantize` feature) */
int scry_hip_i8_from_vec(const int8_t *host, size_t n, scry_i8buf *out);
/* DeviceBackend::i8_to_vec (mod.rs:19-20); takes the storage handle, which is
 * what the trait needs (the reference signature takes &[i8]) */
int scry_hip_i8_to_vec(scry_i8buf b, int8_t *host, size_t n);
int scry_hip_i8_len(scry_i8buf b, size_t *n);
int scry_hip_i8_free(scry_i8buf b);

/* --------------------------------------------------- quantize.rs on device */
/* quantize_symmetric (quantize.rs:16-32): per-tensor, bit-exact */
int scry_hip_quantize_symmetric(scry_buf w, scry_i8buf *q_out, float *scale_out);
/* dequantize (quantize.rs:35-40) */
int scry_hip_dequantize(scry_i8buf q, float scale, scry_buf *out);
/* Block-32 variant (no reference counterpart; builder-defined): quantize_symmetric
 * on each 32-long k-block of each output column of W[k,n]; scales [n][ceil(k/32)] */
int scry_hip_quantize_block32(scry_buf w, int k, int n, scry_i8buf *q_out, scry_buf *scales_out);

/* ------------------------------------ MathBackend int8 (mod.rs:512-557) */
/* MathBackend::matmul_i8_f32 (mod.rs:520-533; CPU cpu.rs:541-551 ->
 * matmul_i8_f32_tiled cpu.rs:1128-1160): C[m,n] = A[m,k] . (f32(Bq[k,n]) * scale) */
int scry_hip_matmul_i8_f32(scry_buf a, scry_i8buf b_q, float scale, int m, int k, int n,
                           scry_buf *out);
/* MathBackend::matmul_i8_f32_bias (mod.rs:536-557; cpu.rs:553-570) */
int scry_hip_matmul_i8_f32_bias(scry_buf a, scry_i8buf b_q, float scale, scry_buf bias, int m,
                                int k, int n, scry_buf *out);
/* block-32 counterpart of matmul_i8_f32 (builder-defined) */
int scry_hip_matmul_i8_f32_block32(scry_buf a, scry_i8buf b_q, scry_buf scales, int m, int k,
                                   int n, scry_buf *out);

/* --------------------------------------- MathBackend glue on the path */
/* MathBackend::matmul (mod.rs:54-63; cpu.rs:924-961): f32 GEMM/GEMV; in bf16
 * mode bf16 operands, f32 accumulation (cuda.rs:274-277) */
int scry_hip_matmul(scry_buf a, scry_buf b, int m, int k, int n, int trans_a, int trans_b,
                    scry_buf *out);
/* MathBackend::matmul_bias (mod.rs:62-86; ops::matmul_bias, ops.rs:21-35):
 * scry_hip_matmul, then the f32 bias row [n] added to every row of [m, n] */
int scry_hip_matmul_bias(scry_buf a, scry_buf b, scry_buf bias, int m, int k, int n, int trans_a,
                         int trans_b, scry_buf *out);
/* MathBackend::matmul_strided_batched (mod.rs:561-591; cpu.rs:1321-1350) */
int scry_hip_matmul_strided_batched(scry_buf a, scry_buf b, int batch, int m, int k, int n,
                                    int trans_a, int trans_b, scry_buf *out);
/* MathBackend::rmsnorm (cpu.rs:574-599): rows x d */
int scry_hip_rmsnorm(scry_buf x, scry_buf w, int rows, int d, float eps, scry_buf *out);
/* MathBackend::rope_with_freqs_preloaded (mod.rs:203-211; cpu.rs:635-664) */
int scry_hip_rope_with_freqs_preloaded(scry_buf x, int seq, int n_heads, int head_dim,
                                       int start_pos, scry_buf freqs, scry_buf *out);
/* MathBackend::rope_with_freqs_scaled_preloaded (mod.rs:219-230) */
int scry_hip_rope_with_freqs_scaled_preloaded(scry_buf x, int seq, int n_heads, int head_dim,
                                              int start_pos, scry_buf freqs, float scale,
                                              scry_buf *out);
/* MathBackend::scale (cpu.rs:509-511) */
int scry_hip_scale(scry_buf x, float s, scry_buf *out);
/* MathBackend::softmax over the last axis (cpu.rs:336-366): rows x cols */
int scry_hip_softmax(scry_buf x, int rows, int cols, scry_buf *out);
/* MathBackend::swiglu (cpu.rs:666-678) */
int scry_hip_swiglu(scry_buf gate, scry_buf up, scry_buf *out);
/* MathBackend::add, same-shape path (cpu.rs:104-113) */
int scry_hip_add(scry_buf a, scry_buf b, scry_buf *out);
/* MathBackend::embedding (cpu.rs:485-498); SCRY_ERR_RANGE for id >= vocab */
int scry_hip_embedding(scry_buf weight, const int64_t *ids, int n_ids, int vocab, int dim,
                       scry_buf *out);
/* MathBackend::gather_reshape_repeat_kv (mod.rs:297-311; cpu.rs:707-730) */
int scry_hip_gather_reshape_repeat_kv(scry_buf cache, int max_seq, int cached_len, int n_kv,
                                      int n_q, int head_dim, scry_buf *out);
/* MathBackend::repeat_kv (cpu.rs:680-705) */
int scry_hip_repeat_kv(scry_buf x, int n_kv, int n_q, int seq, int d_head, scry_buf *out);
/* MathBackend::scatter_rows (mod.rs:368-381): in place */
int scry_hip_scatter_rows(scry_buf dst, scry_buf src, int total_rows, int cols, int row_start,
                          int row_count);
/* generate.rs:167-173 argmax (Iterator::max_by semantics), on device */
int scry_hip_argmax(scry_buf logits, int64_t *out);
/* init::normal_vec (init.rs:12-14): n samples of N(mean, std) by Box-Muller
 * from the fastrand::Rng state *rng_state (two Rng::f64 per sample, advanced
 * by 2n steps), computed on the host with glibc libm as the reference, then
 * stored to new device storage (Linear::new, linear.rs:28-39). */
int scry_hip_normal_vec(uint64_t *rng_state, size_t n, float mean, float std_dev, scry_buf *out);
/* sample_token (generate.rs:92-186) on device: the step sampler of
 * scry_hip_llama_generate on one logits vector (temperature < 1e-8: argmax).
 * *rng_state is the fastrand::Rng state, advanced by the one draw. */
int scry_hip_sample_token(scry_buf logits, const scry_sampling_config *cfg, uint64_t *rng_state,
                          int64_t *out);
/* No counterpart in the reference: scry_hip_sample_token without any device
 * allocation, for callers that must not allocate device memory (between
 * replays of a captured graph, tight serving loops).  Same arguments, results
 * and rng advance.  It waits for the stream and copies the token and the rng
 * state back to the host, so it must be called outside stream capture.  Its
 * scratch is a static device array of about 2 MiB per GPU, held until the
 * process ends; vocabularies above 262144 entries are refused
 * (SCRY_ERR_UNSUPPORTED).  All calls on one GPU share that array: calls that
 * overlap on one GPU race. */
int scry_hip_sample_token_noalloc(scry_buf logits, const scry_sampling_config *cfg, uint64_t *rng_state,
                                  int64_t *out);

/* ------------------------------------ the rest of the trait surface
 * Every other required method of DeviceBackend / MathBackend, and the
 * defaulted ones whose default body is a host round trip (to_vec, loop,
 * from_vec), run on the device.  Arithmetic as the CPU backend's (cpu.rs). */
/* DeviceBackend::ones (mod.rs:24; cpu.rs:37-39) */
int scry_hip_ones(size_t n, scry_buf *out);
/* MathBackend::add with broadcasting (mod.rs:89-95; cpu.rs:94-188): shapes as
 * dims arrays (1 to 6 dims, Shape MAX_DIMS); out_dims must be
 * Shape::broadcast(a, b) (ops::add, ops.rs:38-42), else SCRY_ERR_INVALID (the
 * reference panics "broadcast failed"). */
int scry_hip_add_broadcast(scry_buf a, const size_t *a_dims, int a_ndim, scry_buf b, const size_t *b_dims,
                           int b_ndim, const size_t *out_dims, int out_ndim, scry_buf *out);
/* MathBackend::add_inplace (mod.rs:99-107; cpu.rs:88-92): dst[i] += src[i] over
 * the shorter of the two */
int scry_hip_add_inplace(scry_buf dst, scry_buf src);
/* MathBackend::scaled_softmax (mod.rs:114-117; cpu.rs:300-334): rows x cols */
int scry_hip_scaled_softmax(scry_buf x, float scale, int rows, int cols, scry_buf *out);
/* MathBackend::layernorm (mod.rs:121-127; cpu.rs:416-475): rows x d; also the
 * per-row mean and rstd [rows] */
int scry_hip_layernorm(scry_buf x, scry_buf gamma, scry_buf beta, int rows, int d, float eps, scry_buf *out,
                       scry_buf *mean, scry_buf *rstd);
/* MathBackend::layernorm_inference (mod.rs:130-139; cpu.rs:368-414) */
int scry_hip_layernorm_inference(scry_buf x, scry_buf gamma, scry_buf beta, int rows, int d, float eps,
                                 scry_buf *out);
/* MathBackend::gelu, tanh approximation (mod.rs:142; cpu.rs:477-483, 1110-1116) */
int scry_hip_gelu(scry_buf x, scry_buf *out);
/* MathBackend::sum (mod.rs:153; cpu.rs:500-503): f64 sum rounded to f32 */
int scry_hip_sum(scry_buf x, float *out);
/* MathBackend::mul_elementwise (mod.rs:156; cpu.rs:505-507) */
int scry_hip_mul_elementwise(scry_buf a, scry_buf b, scry_buf *out);
/* MathBackend::concat_rows (mod.rs:162-168; cpu.rs:526-539): a then b */
int scry_hip_concat_rows(scry_buf a, scry_buf b, int a_rows, int b_rows, int cols, scry_buf *out);
/* MathBackend::rope (mod.rs:194-200; cpu.rs:601-633): rows of last_dim values
 * (the shape's last axis), heads of head_dim inside each row, position pos,
 * frequencies 1/theta^(2i/head_dim) */
int scry_hip_rope(scry_buf x, size_t rows, int last_dim, int pos, int head_dim, float theta, scry_buf *out);
/* MathBackend::gather_columns (mod.rs:316-331): [rows, total_cols] ->
 * [rows, col_count] from col_start; llama.rs:389-391 calls it every layer */
int scry_hip_gather_columns(scry_buf x, int rows, int total_cols, int col_start, int col_count, scry_buf *out);
/* MathBackend::scatter_columns (mod.rs:334-350): additive, in place */
int scry_hip_scatter_columns(scry_buf dst, scry_buf src, int rows, int total_cols, int col_start, int col_count);
/* MathBackend::gather_rows (mod.rs:353-365) */
int scry_hip_gather_rows(scry_buf x, int total_rows, int cols, int row_start, int row_count, scry_buf *out);
/* MathBackend::apply_causal_mask_and_scale (mod.rs:384-401): in place */
int scry_hip_apply_causal_mask_and_scale(scry_buf scores, int seq, float scale, float mask_value);
/* MathBackend::apply_batched_causal_mask_and_scale (mod.rs:595-621): every
 * whole [seq, seq] matrix of the storage, in place */
int scry_hip_apply_batched_causal_mask_and_scale(scry_buf scores, int num_matrices, int seq, float scale,
                                                 float mask_value);
/* MathBackend::split_qkv_reshape_heads (mod.rs:408-438): [seq, 3*d_model] ->
 * three [n_heads, seq, d_head] */
int scry_hip_split_qkv_reshape_heads(scry_buf qkv, int seq, int n_heads, int d_head, scry_buf *q, scry_buf *k,
                                     scry_buf *v);
/* MathBackend::reshape_for_heads (mod.rs:441-467): [B*S, H*d] -> [B*H, S, d] */
int scry_hip_reshape_for_heads(scry_buf x, int batch, int seq, int n_heads, int d_head, scry_buf *out);
/* MathBackend::reshape_from_heads (mod.rs:484-510): the inverse */
int scry_hip_reshape_from_heads(scry_buf x, int batch, int seq, int n_heads, int d_head, scry_buf *out);

/* ------------------------------------------------------ Llama (llama.rs) */
typedef struct {
    int32_t vocab_size, hidden_size, intermediate_size, n_layers, n_heads, n_kv_heads,
        max_seq_len;
    float rms_norm_eps, rope_theta;
    int32_t tie_word_embeddings;
    int32_t has_rope_scaling;
    double rs_factor, rs_low_freq_factor, rs_high_freq_factor;
    int64_t rs_original_max_pos;
} scry_llama_config; /* LlamaConfig (llama.rs:20-34) */

/* SCRY_QUANT_BF16: no int8 step -- every projection is kept as bf16 (the
 * reference's cast of the f32 weight) and each matmul rounds its activation
 * to bf16 and accumulates in f32, as the reference's bf16 feature does
 * (cuda.rs:1206-1290); attention, norms and the residual stream stay f32.
 * Decode (forward_with_cache, generate) runs on it; the batched prefill and
 * the per-tensor int8 readback refuse it (SCRY_ERR_UNSUPPORTED). */
enum { SCRY_QUANT_PER_TENSOR = 0, SCRY_QUANT_BLOCK32 = 1, SCRY_QUANT_BF16 = 2 };

enum {
    SCRY_T_EMBED = 0,
    SCRY_T_QKV = 1,
    SCRY_T_O = 2,
    SCRY_T_GATE = 3,
    SCRY_T_UP = 4,
    SCRY_T_DOWN = 5,
    SCRY_T_LM_HEAD = 6
};

/* LlamaModel::new (llama.rs:593-680) with fastrand::Rng::with_seed(seed),
 * followed by the int8 layout step: every projection (fused qkv, o, gate, up,
 * down, lm_head; a tied lm_head gets its own int8 copy of embed_tokens) is
 * quantized per tensor (quantize.rs:16-32) on the device and repacked into the
 * GEMV stream layout.  quant_mode: SCRY_QUANT_PER_TENSOR or SCRY_QUANT_BLOCK32.
 * init_on_device = 0 draws the N(0, 0.02) samples on the host with glibc libm
 * (the reference's arithmetic); 1 draws the same stream on the GPU with the
 * device libm (identical except where the two libms differ in the last bit). */
int scry_hip_llama_new_random(const scry_llama_config *cfg, uint64_t seed, int quant_mode,
                              int init_on_device, scry_llama *out);
/* LlamaModel::from_safetensors (llama.rs:765-958): weights from HuggingFace
 * safetensors shards (F32 / BF16 / F16; the first shard holding a name wins):
 * model.embed_tokens.weight, model.layers.{i}.self_attn.{q,k,v,o}_proj.weight,
 * model.layers.{i}.mlp.{gate,up,down}_proj.weight,
 * model.layers.{i}.{input,post_attention}_layernorm.weight, model.norm.weight
 * and, when not tied, lm_head.weight, in HF's [out, in] layout.  The
 * projections are quantized with quant_mode as by new_random; the RMSNorms
 * use the loaded weights and cfg->rms_norm_eps.  Errors (status, message):
 * a missing tensor, an unsupported dtype, a shape that does not match cfg, an
 * unreadable or malformed shard. */
int scry_hip_llama_from_safetensors(const scry_llama_config *cfg, const char *const *paths, int n_paths,
                                    int quant_mode, scry_llama *out);
int scry_hip_llama_free(scry_llama m);
/* Replace one tensor from host f32 data in the reference layout ([in,out]
 * row-major; embed/lm_head [V,h]); it is quantized and repacked on device.
 * This is the hook a safetensors loader (llama.rs:768-958) feeds. */
int scry_hip_llama_set_tensor(scry_llama m, int tensor_id, int layer, const float *host,
                              size_t n);
/* Read back a projection's int8 weights in the reference layout (inverse of
 * the repack) plus its per-tensor scale -- the i8_to_vec of a model tensor. */
int scry_hip_llama_get_qtensor(scry_llama m, int tensor_id, int layer, int8_t *host, size_t n,
                               float *scale);
/* f32 embedding table back to host (V*h floats) */
int scry_hip_llama_get_embed(scry_llama m, float *host, size_t n);

/* LlamaModel::new_llama_kv_cache (llama.rs:712-719; kv_cache.rs:134-145) */
int scry_hip_llama_kv_cache_new(scry_llama m, int max_seq, scry_kv_cache *out);
int scry_hip_kv_cache_free(scry_kv_cache c);
int scry_hip_kv_cache_seq_len(scry_kv_cache c, int *seq_len);
/* K and V rows [max_seq, n_kv*hd] of one layer back to host */
int scry_hip_kv_cache_layer_to_vec(scry_kv_cache c, int layer, float *k_host, float *v_host,
                                   size_t n);

/* LlamaModel::forward_with_llama_cache (llama.rs:744-763): one token through
 * all layers, appending K/V at the cache's current length; logits [V] to host
 * (logits may be NULL).  The device greedy token (argmax) is returned in
 * *argmax_out when non-NULL. */
int scry_hip_llama_forward_with_cache(scry_llama m, scry_kv_cache c, int64_t token, int pos,
                                      float *logits, int64_t *argmax_out);

/* generate() with temperature 0 (generate.rs:51-89, 92-98): the prompt is fed
 * token by token through the cache path, then greedy tokens follow.  The whole
 * loop runs on the device (one replay of the captured per-kernel step graph
 * per token); only the token ids come back.  Writes max(1, max_tokens) ids to
 * out_tokens and the count to *n_out.  step_logits (optional) receives [n_out, V] logits. */
int scry_hip_llama_generate_greedy(scry_llama m, const int64_t *prompt, int n_prompt,
                                   int max_tokens, int64_t *out_tokens, int *n_out,
                                   float *step_logits);

/* generate() as above, with the prompt prefilled: its first n_prompt - 1
 * tokens go through one batched prefill (GEMMs on the matrix cores), then the
 * decode loop starts at the last prompt token.  Same tokens as
 * scry_hip_llama_generate_greedy; logits agree within float rounding.  (No
 * counterpart in the reference, whose generate feeds the prompt token by
 * token, generate.rs:69-76.) */
int scry_hip_llama_generate_greedy_prefill(scry_llama m, const int64_t *prompt, int n_prompt,
                                           int max_tokens, int64_t *out_tokens, int *n_out,
                                           float *step_logits);

/* generate() (generate.rs:51-89) with sample_token (generate.rs:92-186) on the
 * device.  *rng_state is the fastrand::Rng (wyrand) state, as the reference's
 * `rng: &mut fastrand::Rng` (Rng::with_seed(s) sets it to s); it is advanced
 * by the draws made (one Rng::f64 per sampled token, none when greedy).
 * Temperature < 1e-8 is scry_hip_llama_generate_greedy.
 * Otherwise each step's LM head is followed by one sampling workgroup (top-k
 * by radix select, f64 softmax, top-p cut, weighted draw) inside the captured
 * step graph; only the token ids come back.  prefill != 0 runs the first
 * n_prompt - 1 prompt tokens through the batched prefill (as
 * scry_hip_llama_generate_greedy_prefill).  Outputs as
 * scry_hip_llama_generate_greedy. */
int scry_hip_llama_generate(scry_llama m, const int64_t *prompt, int n_prompt,
                            const scry_sampling_config *cfg, uint64_t *rng_state, int prefill,
                            int64_t *out_tokens, int *n_out, float *step_logits);

/* LlamaModel::forward (llama.rs:683-700; attention llama.rs:162-266): logits
 * [seq, V] (host) for every position of one sequence, causal attention, no
 * cache kept.  Projections run as GEMMs on the matrix cores. */
int scry_hip_llama_forward(scry_llama m, const int64_t *tokens, int seq, float *logits);

/* Batched prefill (the forward above over several sequences, continuing KV
 * caches; the reference has no batched cache path): tokens [n_seq, seq] run
 * at positions caches[s]->seq_len .. of their caches, whose K/V rows are
 * appended (seq_len advances by seq).  last_logits (host, may be NULL)
 * receives [n_seq, V]: each sequence's last position.  1 <= n_seq <= 16,
 * distinct caches, head_dim <= 128. */
int scry_hip_llama_prefill(scry_llama m, scry_kv_cache *caches, int n_seq, const int64_t *tokens,
                           int seq, float *last_logits);

/* Batched greedy decode.  The reference has no counterpart: it decodes one
 * sequence at a time (generate.rs:51-89, llama.rs:744-763), and each
 * sequence's step here computes that step.  n_seq sequences advance `steps`
 * tokens together; every projection reads its weights once per step for all
 * of them.  tokens[i] (host) is the token at position caches[i]->seq_len (the
 * last one fed: after a prefill of all but the last prompt token, that
 * token).  out_tokens (host, [n_seq][steps]) receives the argmax tokens that
 * follow (generate.rs:167-173); logits (host, may be NULL) [steps][n_seq][V]
 * every step's logits.  K/V rows seq_len .. seq_len + steps - 1 are appended
 * (seq_len advances by steps).  1 <= n_seq <= 16, distinct caches, int8
 * models (per-tensor or block-32 scales; a bf16 model returns
 * SCRY_ERR_UNSUPPORTED), hidden, q and ffn sizes multiples of 8, hidden at
 * most 8192. */
int scry_hip_llama_decode_batch(scry_llama m, scry_kv_cache *caches, int n_seq, const int64_t *tokens,
                                int steps, int64_t *out_tokens, float *logits);

/* ------------------------------------------------ measurement helpers */
/* No counterpart in the reference: 1 when decode steps replay their captured
 * graphs, 0 when they are direct launches (SCRY_HIP_NO_GRAPH set, or a
 * rocprofiler tool attached: ROCP_TOOL_LIBRARIES non-empty, as rocprofv3
 * sets it).  Needs no device. */
int scry_hip_graph_replay(void);
/* No counterpart in the reference: step profile of the graph-replayed decode
 * step.  Feeds the prompt, then replays `steps` decode steps captured with
 * per-workgroup stamps of the 100 MHz constant clock.  Launch i of step t
 * (per layer qkv, attention, o, gate/up, down; then the LM head and the
 * argmax finish: 5 L + 2 launches) gets its earliest workgroup start and
 * latest end, in us from the step's first start, at start_us / end_us
 * [t * max_launches + i].  *n_launches = 5 L + 2. */
int scry_hip_llama_profile_step(scry_llama m, const int64_t *prompt, int n_prompt, int steps, int max_launches,
                                int *n_launches, double *start_us, double *end_us);
/* Decode-step session for benchmarks: binds a model and cache, feeds the
 * prompt, then runs `steps` greedy decode steps as graph replays.  The time of
 * the decode steps (HIP events on the launch stream) is returned in *ms. */
int scry_hip_llama_bench_decode(scry_llama m, const int64_t *prompt, int n_prompt, int warmup,
                                int steps, int64_t *out_tokens, double *ms);
/* The same session with the device sampler (scry_hip_llama_generate's step:
 * LM head, then top-k / softmax / top-p / draw) after each LM head; rng state
 * starts at seed.  For the sampler's share of the step time. */
int scry_hip_llama_bench_decode_sampled(scry_llama m, const int64_t *prompt, int n_prompt, int warmup,
                                        int steps, const scry_sampling_config *cfg, uint64_t seed,
                                        int64_t *out_tokens, double *ms);
/* Average device time (HIP events on the launch stream) of `iters` launches
 * of one projection kernel of the model, with the same arguments the decode
 * step uses.  tensor_id: SCRY_T_QKV / O / GATE (fused gate+up) / DOWN / LM_HEAD. */
int scry_hip_llama_time_projection(scry_llama m, int tensor_id, int layer, int iters,
                                   double *avg_us, double *bytes_per_launch);
/* Average device time of `iters` launches of the decode attention kernel
 * (one query token against ctx_len cached positions, every layer's cache in
 * turn) with the decode step's launch shape.  The reference's counterpart is
 * the per-token attention sequence of llama.rs:411-455; this entry is timing
 * only. */
int scry_hip_llama_time_attention(scry_llama m, int ctx_len, int iters, double *avg_us,
                                  double *bytes_per_launch);
/* Prefill then decode, timed: prompts [n_seq, n_prompt]; the first
 * n_prompt - 1 tokens of every sequence go through one batched prefill
 * (*prefill_ms, after an untimed pass), then each sequence runs decode_steps
 * greedy steps in turn (*decode_ms, all sequences).  out_tokens (may be NULL)
 * receives [n_seq, decode_steps]. */
int scry_hip_llama_bench_prefill(scry_llama m, const int64_t *prompts, int n_seq, int n_prompt,
                                 int decode_steps, int64_t *out_tokens, double *prefill_ms,
                                 double *decode_ms);
/* The same with the decode steps of all sequences batched
 * (scry_hip_llama_decode_batch); *decode_ms covers the step replays (the
 * step's graph capture, once per call, is outside). */
int scry_hip_llama_bench_prefill_batch(scry_llama m, const int64_t *prompts, int n_seq, int n_prompt,
                                       int decode_steps, int64_t *out_tokens, double *prefill_ms,
                                       double *decode_ms);
/* Average device time of matmul_i8_f32 at m,k,n rotating over `n_bufs`
 * distinct weight copies (defeats the 256 MB Infinity Cache). */
int scry_hip_bench_qgemv(int m, int k, int n, int quant_mode, int n_bufs, int warmup, int iters,
                         double *avg_us, double *bytes_per_launch);
/* matmul_i8_f32 (m, k, n) launched `iters` times over n_bufs weight copies:
 * *avg_us from back-to-back launches, and (if per_group_us is not NULL) the
 * per-launch device time of each group of `group` consecutive launches
 * (iters / group entries; iters a multiple of group), for the distribution.
 * path 0: the route matmul_i8_f32 takes (the skinny MFMA kernel for 3..16
 * activation rows when k % 8 == 0, k >= 256 and n >= 256, else the GEMV up to
 * 16 rows, the MFMA GEMM above); 1: the GEMV; 2: the MFMA GEMM (with its
 * input pass: int8 digit planes for per-tensor scales and k <= 16384, else the
 * bf16 activation split); 3: the skinny MFMA kernel (with its split reduction).
 * quant_mode: per-tensor or block-32 scales. */
int scry_hip_bench_qgemv_dist(int m, int k, int n, int quant_mode, int path, int n_bufs, int warmup, int iters,
                              int group, double *per_group_us, double *avg_us, double *bytes_per_launch);
/* The same with a bias row (matmul_i8_f32_bias, cpu.rs:553-570; the quantized
 * Linear::forward, linear.rs:67-94): per-tensor int8, bias added in the
 * GEMV's store epilogue. */
int scry_hip_bench_qgemv_bias(int m_rows, int k, int n, int n_bufs, int warmup, int iters,
                              double *avg_us, double *bytes_per_launch);
/* The bf16-mode GEMV (1-16 rows, bf16 weight rows [n][kp]) over n_bufs
 * weight copies: average device time and algorithmic bytes per launch. */
int scry_hip_bench_gemv_bf16(int m_rows, int k, int n, int n_bufs, int warmup, int iters, double *avg_us,
                             double *bytes_per_launch);

#ifdef __cplusplus
}
#endif
#endif /* SCRY_HIP_H */
