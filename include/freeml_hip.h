/*
 * freeml_hip.h — C ABI of the MI355X (gfx950) backend for FreeML's NanoLLM token loop.
 *
 * Two groups of entry points, both plain C: device pointers are `float*` / `int32_t*`
 * obtained from fmlh_malloc, host pointers are ordinary memory, sizes are element counts.
 *
 *  1. Matrix ops: one entry point per free function of FreeML's operator API that the NanoLLM
 *     forward reaches (the overload set a `MatrixHIP<float>` backend binds, next to the
 *     reference's MatrixCPU and MatrixDX11 overloads).  Each comment names the reference
 *     routine (path:line relative to the FreeML root) whose meaning it keeps.  Matrices are
 *     row-major: element (x, y, z) of a (dimsX, dimsY, dimsZ) matrix sits at
 *     z*dimsX*dimsY + y*dimsX + x (MatrixLibrary/CPU/MatrixCPU.h:84-112).
 *  2. The NanoLLM token loop (fmlh_nanollm_*): the graph built by Examples/NanoLLM/NanoLLM.cpp
 *     (:255-376) run greedily with a device-resident KV cache, MFMA/GEMV projections, fused
 *     causal attention and a device argmax.  Its results follow the reference loop: the logits
 *     of step s are those Model::Run (ModelLibrary/Model.h:764-788) gives for the token window
 *     at row len-1, and the next token is their first maximum (NanoLLM.cpp:189-205).
 *
 * Errors: every function returns 0 on success or a negative FMLH_E* code; the message of the
 * last failure on the calling thread is fmlh_last_error().  Nothing is printed.  (The
 * reference's own convention is assert + log + silent return, ToolsLibrary/Logger.h and
 * MatrixLibrary/GPU/DirectX11/MatrixDX11_Functions.h:92-120; the C++ host binding turns these
 * codes back into that convention.)
 *
 * Ordering: all work is enqueued on one HIP stream per process (fmlh_get_stream); calls return
 * before the device finishes unless they hand data to host memory.  No call allocates device
 * memory while a token loop runs except where noted.
 */
#ifndef FREEML_HIP_H
#define FREEML_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMLH_OK 0
#define FMLH_E_INVALID (-1)   /* bad argument / shape mismatch */
#define FMLH_E_HIP (-2)       /* HIP runtime failure (launch, copy, allocation) */
#define FMLH_E_NODEVICE (-3)  /* no usable gfx950 device */
#define FMLH_E_STATE (-4)     /* call not valid in the object's current state */

/* ---- runtime ------------------------------------------------------------------------- */

/* Selects the device, creates the library stream (default priority).  Idempotent.
 * Replaces DirectX11Manager::Init (MatrixLibrary/GPU/DirectX11/DirectX11Manager.h:49-165). */
int fmlh_init(int device);
/* Releases everything the library holds: waits for enqueued work, destroys every token-loop
 * engine still alive (their handles become invalid; fmlh_nanollm_destroy refuses them), the
 * process-wide split-K workspace and the library stream.  Memory from fmlh_malloc is not
 * tracked and must be freed before.  Afterwards every call but fmlh_init fails with
 * FMLH_E_STATE; fmlh_init starts the library again.  Call it before the process exits, while
 * the HIP runtime is still alive (the Python binding does so from an atexit handler).
 * Replaces DirectX11Manager's teardown (MatrixLibrary/GPU/DirectX11/DirectX11Manager.h). */
int fmlh_shutdown(void);
/* Device arch name (e.g. "gfx950") and CU count of the initialised device. */
int fmlh_device_info(char* arch, size_t arch_len, int* cu_count);
const char* fmlh_last_error(void);
/* The HIP stream (hipStream_t) every call enqueues on. */
void* fmlh_get_stream(void);

/* Device memory.  Replaces MatrixDX11::AllocateMemory/FreeMemory (MatrixDX11.h:48-75) and
 * the staging copies behind DataRead/DataWrite (MatrixDX11.h:190-226).  d2h blocks until the
 * data is on the host; h2d returns once the source may be reused. */
int fmlh_malloc(void** dptr, size_t bytes);
int fmlh_free(void* dptr);
int fmlh_memcpy_h2d(void* dst, const void* src, size_t bytes);
int fmlh_memcpy_d2h(void* dst, const void* src, size_t bytes);
int fmlh_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Waits for all enqueued work (DirectX11Manager::WaitForGPU, DirectX11Manager.h:650). */
int fmlh_synchronize(void);

/* Events on the library stream, for timing enqueued work. */
int fmlh_event_create(void** ev);
int fmlh_event_destroy(void* ev);
int fmlh_event_record(void* ev);
int fmlh_event_elapsed_ms(void* start, void* stop, float* ms); /* synchronizes on stop */

/* ---- matrix ops (MatrixHIP<float> overload set) ------------------------------------- */

/* TransposeMode (MatrixLibrary/MatrixBase_Mul.h:27). */
#define FMLH_TRANSPOSE_NONE 0
#define FMLH_TRANSPOSE_LEFT 1
#define FMLH_TRANSPOSE_RIGHT 2
#define FMLH_TRANSPOSE_BOTH 3

/* Mul<Mode>(out, L, R) (MatrixBase_Mul.h:591-615).  out is M x N; L is M x K (K x M with
 * Left); R is K x N (N x K with Right).  Dense::Forward calls it with None (QKV, MLP FC, MLP
 * proj; Dense.h:207) and Right (attention proj, lm_head; Dense.h:203). */
int fmlh_mul(int mode, float* out, const float* L, const float* R,
             uint32_t M, uint32_t N, uint32_t K);

/* Dense::Forward with its epilogue fused (Dense.h:179-222, and the block's residual Add,
 * TransformerBlock.h:382/:400): C = epi(A op(B)), A M x K (row stride lda), B K x N (ldb) or,
 * with b_trans = 1, N x K (ldb, the `TransposedWeights` Dense layout).  epilogue 0: none,
 * 1: GeluMat (Gelu.h:32-38), 2: C = R + A op(B) (R row stride ldr; R may alias C). */
#define FMLH_EPILOGUE_NONE 0
#define FMLH_EPILOGUE_GELU 1
#define FMLH_EPILOGUE_RESIDUAL 2
int fmlh_gemm_ex(const float* A, int lda, const float* B, int ldb, int b_trans, float* C, int ldc,
                 int M, int N, int K, int epilogue, const float* R, int ldr);

/* fmlh_gemm_ex for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc); no counterpart in the reference.  Same
 * arguments, kernels and results as fmlh_gemm_ex, but the split-K partial sums go to a fixed
 * 16 MiB device array (4 Mi floats, one per device, held until the process ends) instead of the
 * library's grow-on-demand workspace; nothing is allocated or freed.  A product whose partials
 * need more is refused with FMLH_E_INVALID; before fmlh_init, FMLH_E_STATE.  All calls on a
 * device share its array: they are ordered on the library stream, and work that overlaps them
 * on another stream of the same device races on the partials. */
int fmlh_gemm_ex_noalloc(const float* A, int lda, const float* B, int ldb, int b_trans, float* C, int ldc,
                         int M, int N, int K, int epilogue, const float* R, int ldr);

/* MatMul_Strided<Mode> (MatrixBase_Mul.h:617-722): `batch` planes; plane z reads
 * L + z*l_plane, R + z*r_plane and writes out + z*o_plane.  Element strides as in
 * MulStrided (:88-144): A(i,k) = L[i*l_rs + k*l_cs] (transposed: L[k*l_rs + i*l_cs]). */
int fmlh_matmul_strided(int mode, float* out, const float* L, const float* R,
                        uint32_t M, uint32_t N, uint32_t K,
                        uint32_t l_rs, uint32_t l_cs, uint32_t r_rs, uint32_t r_cs,
                        uint32_t o_rs, uint32_t o_cs, uint32_t batch,
                        size_t l_plane, size_t r_plane, size_t o_plane);

/* Softmax (MatrixBase_Functions.h:49-80): per row max, exp(x - max), sum, divide. */
int fmlh_softmax(float* out, const float* in, uint32_t rows, uint32_t cols);

/* LayerNormOp (MatrixBase_Functions.h:481-549): mean, two-pass variance,
 * invStd = 1 / sqrt(var + eps), out = (x - mean) * invStd * gamma (+ beta).
 * beta and xhat may be NULL. */
int fmlh_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps);

/* GeluMat (MatrixBase_Functions.h:988-1000): 0.5 * x * (1 + erf(x / sqrt(2))). */
int fmlh_gelu(float* out, const float* in, size_t n);

/* Add (MatrixBase_Functions.h:470-479): out = a + b, n elements (out may alias a or b). */
int fmlh_add(float* out, const float* a, const float* b, size_t n);

/* Copy (MatrixBase_Functions.h:156-161). */
int fmlh_copy(float* out, const float* in, size_t n);

/* GatherRows (MatrixBase_Functions.h:202-242): out[z][r][:] = src[zs][idx[z][r]][:] with
 * zs = 0 when src_batch == 1; ids are float (truncated).  An id outside [0, src_rows) gives a
 * zero row, as the reference's DX11 gather_rows shader does (its CPU path asserts). */
int fmlh_gather_rows(float* out, const float* src, const float* idx, uint32_t width,
                     uint32_t out_rows, uint32_t out_batch, uint32_t src_rows,
                     uint32_t src_batch);

/* SplitQKV (MatrixBase_Functions.h:329-367): packed rows [Q | K | V] of width 3*dC. */
int fmlh_split_qkv(float* q, float* k, float* v, const float* packed, uint32_t rows,
                   uint32_t dC);

/* ScaleAdd(out, in, Mat* scale, add) (MatrixBase_Functions.h:1055-1070):
 * out = in * scale[0] + add, scale read from device memory. */
int fmlh_scale_add(float* out, const float* in, const float* scale, const float* add, size_t n);

/* BroadcastAdd (MatrixBase_Functions.h:716-730): out[i] = L[i] + R[i % dims_x]. */
int fmlh_broadcast_add(float* out, const float* L, const float* R, size_t n, uint32_t dims_x);

/* Fill(out, float) (MatrixBase_Functions.h:1078-1085) and Fill(out, Mat*) (:1087-1095, value
 * read from device memory). */
int fmlh_fill(float* out, float value, size_t n);
int fmlh_fill_from(float* out, const float* value, size_t n);

/* PerElementMul (MatrixBase_Functions.h:847-854). */
int fmlh_per_element_mul(float* out, const float* a, const float* b, size_t n);

/* Scale(out, in, Mat* val) (MatrixBase_Functions.h:1020-1029) and Scale(out, in, float)
 * (:1031-1038). */
int fmlh_scale(float* out, const float* in, const float* value, size_t n);
int fmlh_scale_scalar(float* out, const float* in, float value, size_t n);

/* Row-wise first maximum (strict '>'), as DecodeMatrixTokens / CountCorrectTokensBatch
 * (Examples/NanoLLM/NanoLLM.cpp:189-205, :236-246).  out_idx: rows int32 (device). */
int fmlh_row_argmax(int32_t* out_idx, const float* in, uint32_t rows, uint32_t cols);

/* ---- training step (Model::Run with a target, ModelLibrary/Model.h:790-878) ---------- */

/* SoftmaxBackwards (MatrixBase_Functions.h:83-111): per row out = p * (dp - sum(dp * p)).
 * Called per head by CausalSelfAttentionLayer::Backwards (CausalSelfAttentionLayer.h:640).
 * out may alias grad_in. */
int fmlh_softmax_backward(float* out, const float* softmax_out, const float* grad_in, uint32_t rows,
                          uint32_t cols);

/* LayerNormBackwardsOp (MatrixBase_Functions.h:552-705), as LayerNorm::Backwards calls it
 * (LayerNorm.h): dx from dy, the input and gamma; dgamma = sum over rows of dy * xhat and
 * (when dbeta is non-NULL) dbeta = sum of dy.  With xhat NULL the normalised input is
 * recomputed and ws (2 * rows floats, device) holds each row's mean and 1/std.  dx must not
 * alias dy or in. */
int fmlh_layernorm_backward(float* dx, const float* dy, const float* in, const float* gamma,
                            float* dgamma, float* dbeta, const float* xhat, float* ws,
                            uint32_t rows, uint32_t cols, float eps);

/* GeluDerivtiveMat (MatrixBase_Functions.h:1002-1017), the derivative Gelu::derivativeMat
 * passes to Dense::Backwards (ActivationLibrary/Gelu.h:40-46, Dense.h:246-250). */
int fmlh_gelu_derivative(float* out, const float* in, size_t n);

/* ScatterAddRows (MatrixBase_Functions.h:285-327), Embedding::Backwards' weight gradient
 * (Embedding.h:174-194): out[oz][idx[z][r]] += src[z][r] for src_batch planes of src_rows
 * rows, oz = 0 when out_batch == 1.  Each destination row receives its sources in (z, r)
 * order, as the reference adds them (bit-identical sums).  Ids are float, truncated; an id
 * outside [0, out_rows) is skipped. */
int fmlh_scatter_add_rows(float* out, const float* src, const float* idx, uint32_t width,
                          uint32_t src_rows, uint32_t src_batch, uint32_t out_rows,
                          uint32_t out_batch);

/* CategoricalCrossEntropyWithLogits::Gradient and ::Loss (LossLibrary/
 * CategoricalCrossEntropyWithLogits.h:29-208) over logits [batch][steps][vocab].  target is
 * either index targets (target_cols 1: [target_batch][steps] ids, -1 ignored; gradient
 * (onehot - softmax) / valid rows, loss = mean over valid rows of logsumexp - z[id]) or one-hot
 * (target_cols == vocab: gradient onehot - softmax, loss = summed over rows).  target_batch is
 * 1 (shared) or batch.  grad (NULL: skip) is written on the device; loss (NULL: skip) is one
 * device float and needs ws of steps * batch floats. */
int fmlh_cce_logits(float* grad, float* loss, float* ws, const float* target, const float* logits,
                    uint32_t vocab, uint32_t steps, uint32_t batch, uint32_t target_cols,
                    uint32_t target_batch);

/* AdamWUpdate (MatrixBase_Functions.h:1497-1545), AdamWOptimiser::Step's update
 * (OptimiserLibrary/AdamWOptimiser.h:131-193), element-wise in the reference's operation order
 * (no FMA contraction): m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g g,
 * p = p + lr (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps) - lr wd p. */
int fmlh_adamw_update(float* param, const float* grad, float* mt, float* vt, size_t n, float lr,
                      float beta1, float beta2, float beta1_pow_t, float beta2_pow_t, float eps,
                      float weight_decay);

/* CausalSelfAttentionLayer's per-head score-to-probability steps for all heads at once
 * (CausalSelfAttentionLayer.h:453-458): for head h and row i, ScaleAdd by *scale (device
 * scalar, the layer's ScalarScale) plus the causal mask (0 on and below the diagonal, -inf
 * above), then Softmax.  scores: [n_head][T][T]; the probabilities are written to head h's
 * matrix p_heads[h] (device pointers, at element offset p_offset: the batch plane) and to
 * p_all [n_head][T][T].  n_head <= 32. */
int fmlh_attention_softmax_heads(float* const* p_heads, size_t p_offset, float* p_all, const float* scores,
                                 const float* scale, uint32_t n_head, uint32_t T);

/* The matching backward step for all heads (CausalSelfAttentionLayer.h:640-642):
 * ds = ((p (da - sum(da p))) * causal 0/1 mask) * *scale, p from p_heads[h] (batch plane 0),
 * da and ds [n_head][T][T]. */
int fmlh_attention_softmax_backward_heads(float* ds_all, float* const* p_heads, const float* datt_all,
                                          const float* scale, uint32_t n_head, uint32_t T);

/* MergeQKV (MatrixBase_Functions.h:369-431): per-head gradients q/k/v [n_head][tokens][head_dim]
 * into the packed [tokens][3 C] layout (CausalSelfAttentionLayer.h:663). */
int fmlh_merge_qkv(float* packed, const float* q, const float* k, const float* v, uint32_t head_dim,
                   uint32_t tokens, uint32_t n_head);

/* SumColumns (MatrixBase_Functions.h:1098-1118), the Dense bias gradient (Dense.h:263, :272):
 * out[c] = in[0][c] + in[1][c] + ... + in[rows-1][c], added in row order (bit-identical to the
 * reference's loop); in is rows x cols, row-major. */
int fmlh_sum_columns(float* out, const float* in, uint32_t rows, uint32_t cols);

/* DropoutLayer::UpdateMask for 0 < prob < 1 (DropoutLayer.h:97-123): mask[i] = 0 where
 * uniforms[(start + i) mod count] < prob, else 1 -- the draws RandomUtils::
 * random_uniform_buffered (ToolsLibrary/Tools.h:63-69) makes from its buffer of count uniforms
 * when its running index is at start. */
int fmlh_dropout_mask(float* mask, uint64_t n, const float* uniforms, uint64_t count, uint64_t start,
                      float prob);

/* ---- NanoLLM token loop ------------------------------------------------------------- */

typedef struct fmlh_nanollm fmlh_nanollm;

/* NanoLLMConfig (NanoLLM.cpp:47-66) plus the number of sequences decoded together. */
typedef struct fmlh_nanollm_config {
    uint32_t vocab;      /* V: vocabulary (Embedding rows, lm_head outputs) */
    uint32_t block_size; /* T: context length; positions 0 .. T-1 */
    uint32_t n_embed;    /* C */
    uint32_t n_head;     /* H; C % H == 0 */
    uint32_t n_layer;    /* L TransformerBlocks */
    uint32_t max_batch;  /* B: independent sequences (the reference is batch 1 per run) */
} fmlh_nanollm_config;

/* Parameters in FreeML's storage layout (row-major, fp32), i.e. the contents of the blob
 * matrices named in the comments.  `layers` points to n_layer groups of 8 pointers:
 *   [0] w_qkv   C x 3C  CSA_AttentionLayer/Dense_Weights (CausalSelfAttentionLayer.h:47)
 *   [1] w_proj  C x C   CSA_ProjLayer/Dense_Weights, out-rows x in-cols (:51, Dense.h:203)
 *   [2] w_fc    C x 4C  DenseFCData/Dense_Weights (TransformerBlock.h:288)
 *   [3] w_proj2 4C x C  DenseProjData/Dense_Weights (TransformerBlock.h:316)
 *   [4] ln0 gamma, [5] ln0 beta or NULL, [6] ln1 gamma, [7] ln1 beta or NULL (LayerNorm.h:111-121)
 * lm_head (V x C, ln_f -> lm_head Dense_Weights) NULL or equal to tok_emb means tied
 * (NanoLLM.cpp:333-345). */
typedef struct fmlh_nanollm_weights {
    const float* tok_emb; /* V x C  embedding_token/Embedding_Weights */
    const float* pos_emb; /* T x C  embedding_pos/Embedding_Weights */
    const float* const* layers;
    const float* lnf_gamma;
    const float* lnf_beta; /* NULL: no BetaShift (use_bias = false) */
    const float* lm_head;
} fmlh_nanollm_weights;

/* Builds the engine and allocates the KV cache and activations for max_batch sequences of
 * block_size tokens.  weights_on_device = 0: host pointers; every parameter is copied to the
 * device.  weights_on_device = 1: device pointers; W_qkv, W_fc and W_proj2 are copied once,
 * transposed (one output per row, the layout every decode kernel reads), and the other
 * parameters (embeddings, W_proj, LayerNorm gains/shifts, lm_head) are referenced and must
 * outlive the engine.  After the caller updates referenced parameters in place (e.g. an AdamW
 * step on the blobs), fmlh_nanollm_refresh_weights must be called before the next prefill or
 * decode so that the transposed copies follow. */
int fmlh_nanollm_create(const fmlh_nanollm_config* cfg, const fmlh_nanollm_weights* w,
                        int weights_on_device, fmlh_nanollm** out);
/* Re-takes the transposed copies of W_qkv, W_fc and W_proj2 from the device parameters given
 * to fmlh_nanollm_create (weights_on_device = 1 only; FMLH_E_STATE otherwise, where the engine
 * owns all its weights).  Enqueued on the library stream, ordered before later calls.  No
 * counterpart in the reference, whose MatrixCPU layers read their blobs directly. */
int fmlh_nanollm_refresh_weights(fmlh_nanollm* m);
int fmlh_nanollm_destroy(fmlh_nanollm* m);

/* Prefill: `batch` prompts of prompt_len ids each (host, batch x prompt_len, row-major) are
 * embedded, run through every block (K/V written to the cache) and the first token of every
 * sequence is chosen on the device from logits row prompt_len-1.  Starts a new loop. */
int fmlh_nanollm_prefill(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch,
                         uint32_t prompt_len);

/* n_steps greedy decode steps after a prefill: each embeds the last chosen token at the next
 * position, attends to the cache and picks the next token, all on the device (no host
 * round trip).  Fails with FMLH_E_STATE if the loop would pass position block_size - 1. */
int fmlh_nanollm_decode(fmlh_nanollm* m, uint32_t n_steps);

/* Device-to-host reads of the loop's state (blocking).  Tokens chosen so far: generated
 * token g of sequence b is out[b * count + (g - first)], g counted from the prefill's (0). */
int fmlh_nanollm_read_tokens(fmlh_nanollm* m, int32_t* out, uint32_t first, uint32_t count);
/* Logits of the most recent step: batch x vocab. */
int fmlh_nanollm_read_logits(fmlh_nanollm* m, float* out);
/* Number of tokens generated so far (per sequence) and current batch. */
int fmlh_nanollm_status(fmlh_nanollm* m, uint32_t* generated, uint32_t* batch);
/* Which implementation fmlh_nanollm_decode uses for `batch` sequences: FMLH_DECODE_RELAY
 * (greedy batches of up to 56 sequences of the compiled shapes, 64 with FMLH_RELAY=1,
 * block_size <= 256: one
 * cooperative launch per decode call, each product computed by its own small team of
 * workgroups whose weights stay on the chip, the batch's sequences flowing through the teams
 * as a pipeline; FMLH_RELAY=0 turns it off), FMLH_DECODE_PERSISTENT (one cooperative kernel
 * launch per decode call, `workgroups` workgroups exchanging each step's activations through
 * global memory; up to 8 sequences, or two groups of 8 where the per-workgroup weight slices
 * fit in LDS), FMLH_DECODE_GROUPED (more than 8 sequences, up to 64: one cooperative launch per
 * decode call, groups of up to 8 sequences on their own workgroups, matrix-core products;
 * block_size <= 256 and the compiled head_dim / n_embed pairs), FMLH_DECODE_WIDE (up to 8
 * sequences of shapes none of those take -- head_dim 64, n_embed 256 / 512 / 768 / 1024,
 * block_size <= 4096: one cooperative launch per decode call, every workgroup streaming its
 * slice of each product's weights, key-sliced attention items; FMLH_WIDE=0 turns it off) or
 * FMLH_DECODE_GRAPH (one HIP graph of ~5 kernels per layer per step; `workgroups` = 0).
 * No counterpart in the reference, whose NanoLLM loop re-runs the whole window per token
 * (NanoLLM.cpp:150-205). */
#define FMLH_DECODE_GRAPH 0
#define FMLH_DECODE_PERSISTENT 1
#define FMLH_DECODE_GROUPED 2
#define FMLH_DECODE_RELAY 3
#define FMLH_DECODE_WIDE 4
int fmlh_nanollm_decode_path(fmlh_nanollm* m, uint32_t batch, int* path, int* workgroups);

/* Sampling for the picks of later prefill / decode calls (no counterpart in the reference,
 * whose NanoLLM decodes greedily).  temperature 0 (the default): greedy, first maximum.
 * temperature > 0: token i is drawn with probability proportional to
 * exp((z_i - max z) / temperature) over the top_k largest logits (ties at the k-th value go to
 * the lower indices; top_k 0 or >= vocab keeps all), by inverse CDF in index order at u * total,
 * u = (splitmix64(seed ^ splitmix64(sequence << 32 | position)) >> 40) / 2^24 for the position
 * being filled.  Decode then takes the graph path. */
int fmlh_nanollm_set_sampling(fmlh_nanollm* m, float temperature, uint32_t top_k, unsigned long long seed);

/* Convenience: prefill + (n_gen - 1) decode steps; copies tokens (batch x n_gen) and, if
 * logits_out is not NULL, every step's logits (batch x n_gen x vocab) to host memory. */
int fmlh_nanollm_generate(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch,
                          uint32_t prompt_len, uint32_t n_gen, int32_t* tokens_out,
                          float* logits_out);

/* Measurement hook: replays one op of the decode step (layer 0 for per-layer ops) `iters`
 * times between two events on the library stream and reports the mean time per launch and the
 * op's algorithmic HBM bytes per launch (weights + activations + KV read; no reuse credit).
 * The op runs the kernels a decode step of the current batch runs: where batched decode fuses
 * the QKV projection with the cache write and the residual projections with the following
 * LayerNorm, the op includes them.
 * Needs a prefilled loop; afterwards the loop state is undefined (prefill again).  No
 * counterpart in the reference, which has no device timing (Model::PrintTimings, Model.h:633,
 * measures host wall-clock). */
#define FMLH_OP_QKV 0
#define FMLH_OP_ATTENTION 1
#define FMLH_OP_ATTN_PROJ 2
#define FMLH_OP_MLP_FC 3
#define FMLH_OP_MLP_PROJ 4
#define FMLH_OP_LM_HEAD 5
int fmlh_nanollm_profile_op(fmlh_nanollm* m, int op, uint32_t iters, float* avg_ms,
                            double* bytes);

/* Full-window forward (Model::Run on a block_size window, Model.h:764-788): ids (host,
 * batch x block_size, positions 0..T-1) -> logits (host, batch x block_size x vocab).
 * Uses the prefill kernels; the KV cache is overwritten. */
int fmlh_nanollm_forward_window(fmlh_nanollm* m, const int32_t* ids, uint32_t batch,
                                float* logits_out);

#ifdef __cplusplus
}
#endif

#endif /* FREEML_HIP_H */
