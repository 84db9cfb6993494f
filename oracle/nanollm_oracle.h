/*
 * CPU oracle for the FreeML NanoLLM token loop — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference arithmetic (MatrixCPU<float> path) used as the
 * checker for the HIP backend.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never does.
 *
 * Every function follows a reference routine (paths relative to the FreeML root) and keeps
 * its floating-point evaluation order, so that results are bit-identical to the reference
 * compiled with the same libm (pinned by tests/test_oracle.py against the compiled reference
 * in oracle/_ref and against fixtures in tests/golden/).
 */
#ifndef FREEML_NANOLLM_ORACLE_H
#define FREEML_NANOLLM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TransposeMode (MatrixLibrary/MatrixBase_Mul.h:27). */
enum { ORC_NONE = 0, ORC_LEFT = 1, ORC_RIGHT = 2, ORC_BOTH = 3 };

/* ---- per-op restatements ------------------------------------------------------------ */

/* Mul<Mode>(out, L, R) (MatrixBase_Mul.h:592-615 -> MulBlock :478-589 / MulNoDynamicAlloc
 * :36-86).  L is M x K (K x M when mode has Left), R is K x N (N x K when mode has Right),
 * out is M x N.  Each output is the sequential k = 0..K-1 fp32 sum (no FMA).  Rows are
 * split over nthreads workers as MulBlock does; the split does not change any result. */
void orc_mul(int mode, float* out, const float* L, const float* R,
             uint32_t M, uint32_t N, uint32_t K, int nthreads);

/* MulStrided<Mode> (MatrixBase_Mul.h:88-144): general strided single-plane product. */
void orc_mul_strided(int mode, float* C, const float* A, const float* B,
                     uint32_t M, uint32_t N, uint32_t K,
                     uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs,
                     uint32_t c_rs, uint32_t c_cs);

/* LayerNormOp (MatrixBase_Functions.h:481-549).  beta and xhat may be NULL. */
void orc_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps);

/* Softmax (MatrixBase_Functions.h:49-80): max, exp(x - max), sequential sum, divide. */
void orc_softmax(float* out, const float* in, uint32_t rows, uint32_t cols);

/* ScaleAdd(out, in, scale, add) (MatrixBase_Functions.h:1055-1070): out = in*scale + add. */
void orc_scale_add(float* out, const float* in, float scale, const float* add, uint32_t n);

/* GeluMat (MatrixBase_Functions.h:988-1000): 0.5*x*(1 + erf(x / sqrt(2))). */
void orc_gelu(float* out, const float* in, uint32_t n);

/* Add (MatrixBase_Functions.h:470-479). */
void orc_add(float* out, const float* a, const float* b, uint32_t n);

/* GatherRows (MatrixBase_Functions.h:202-242) for one plane: float ids truncated to uint. */
void orc_gather_rows(float* out, const float* src, const float* ids, uint32_t width,
                     uint32_t rows);

/* SplitQKV (MatrixBase_Functions.h:329-367). */
void orc_split_qkv(float* q, float* k, float* v, const float* packed, uint32_t rows,
                   uint32_t dC);

/* TriangleMatrix Lower (MatrixBase_Functions.h:113-139). */
void orc_triangle_lower(float* out, uint32_t rows, uint32_t cols, float true_val,
                        float false_val);

/* First-max argmax with strict '>' (Examples/NanoLLM/NanoLLM.cpp:189-205). */
uint32_t orc_argmax(const float* row, uint32_t n);

/* ---- model -------------------------------------------------------------------------- */

typedef struct orc_model orc_model;

/* Builds a NanoLLM graph description (NanoLLM.cpp:255-376) over caller-owned fp32 weights.
 * layer_ptrs holds n_layer groups of 8 pointers:
 *   {w_qkv (C x 3C), w_proj (C x C, out-rows x in-cols), w_fc (C x 4C), w_proj2 (4C x C),
 *    ln0_gamma, ln0_beta|NULL, ln1_gamma, ln1_beta|NULL}.
 * lm_head (V x C) may equal tok_emb (tied, NanoLLM.cpp:333-345).  Returns NULL on bad shape. */
orc_model* orc_model_create(uint32_t vocab, uint32_t block_size, uint32_t n_embed,
                            uint32_t n_head, uint32_t n_layer,
                            const float* tok_emb, const float* pos_emb,
                            const float* const* layer_ptrs,
                            const float* lnf_gamma, const float* lnf_beta,
                            const float* lm_head, int nthreads);
void orc_model_destroy(orc_model* m);

/* Model::Run forward on one full block_size window (Model.h:764-788 over the layer
 * Forward()s in NanoLLM order), reference-faithful: full T x T scores, additive -inf mask,
 * full-row softmax and P.V.  ids: T token ids.  logits: T x V.  Returns 0 on success. */
int orc_forward_window(orc_model* m, const int32_t* ids, float* logits);

/* Greedy token loop (NanoLLM.cpp:189-205): for each step the window is the token history padded
 * with id 0 to block_size, logits row len-1 is taken, argmax appended.  Full-window
 * recompute per step (the reference cost).  tokens_out: n_gen ids; logits_out (nullable):
 * n_gen x V rows.  Requires prompt_len + n_gen - 1 <= block_size. */
int orc_greedy_window(orc_model* m, const int32_t* prompt, uint32_t prompt_len,
                      uint32_t n_gen, int32_t* tokens_out, float* logits_out);

/* Same loop computed incrementally: each new row attends to the cached K/V of earlier rows.
 * Row r of every layer depends only on rows <= r and keeps the reference's per-output
 * summation order, so logits and tokens are bit-identical to orc_greedy_window. */
int orc_greedy_cached(orc_model* m, const int32_t* prompt, uint32_t prompt_len,
                      uint32_t n_gen, int32_t* tokens_out, float* logits_out);


/* ---- training-step restatements (Model::Run with a target, ModelLibrary/Model.h:790-878) */

/* SoftmaxBackwards (MatrixBase_Functions.h:83-111): per row dot = sequential sum of
 * dp*p, out = p * (dp - dot). */
void orc_softmax_backward(float* out, const float* p, const float* dp, uint32_t rows, uint32_t cols);

/* LayerNormBackwardsOp (MatrixBase_Functions.h:552-705).  dbeta and xhat may be NULL (xhat
 * NULL: recomputed from in, :624-654). */
void orc_layernorm_backward(float* dx, const float* dy, const float* in, const float* gamma,
                            float* dgamma, float* dbeta, const float* xhat, uint32_t rows,
                            uint32_t cols, float eps);

/* GeluDerivtiveMat (MatrixBase_Functions.h:1002-1017). */
void orc_gelu_derivative(float* out, const float* in, uint32_t n);

/* ScatterAddRows (MatrixBase_Functions.h:285-327): out += rows of src at float ids, in
 * (z, r) order.  Ids must be in range (the reference asserts). */
void orc_scatter_add_rows(float* out, const float* src, const float* idx, uint32_t width,
                          uint32_t src_rows, uint32_t src_batch, uint32_t out_rows,
                          uint32_t out_batch);

/* MergeQKV (MatrixBase_Functions.h:369-431). */
void orc_merge_qkv(float* packed, const float* q, const float* k, const float* v,
                   uint32_t head_dim, uint32_t tokens, uint32_t n_head);

/* CategoricalCrossEntropyWithLogits::Gradient / ::Loss (LossLibrary/
 * CategoricalCrossEntropyWithLogits.h:29-208).  target_cols 1: index targets (-1 ignored),
 * else one-hot rows of width vocab.  grad may be NULL; returns the loss. */
float orc_cce_logits(float* grad, const float* target, const float* logits, uint32_t vocab,
                     uint32_t steps, uint32_t batch, uint32_t target_cols, uint32_t target_batch);

/* AdamWUpdate (MatrixBase_Functions.h:1497-1545). */
void orc_adamw_update(float* param, const float* grad, float* mt, float* vt, uint32_t n, float lr,
                      float beta1, float beta2, float beta1_pow_t, float beta2_pow_t, float eps,
                      float weight_decay);

/* SumColumns (MatrixBase_Functions.h:1098-1118): out[c] = sum of in[r][c] over r in row order. */
void orc_sum_columns(float* out, const float* in, uint32_t rows, uint32_t cols);

/* DropoutLayer::UpdateMask (DropoutLayer.h:97-123) with the draws of
 * RandomUtils::random_uniform_buffered (ToolsLibrary/Tools.h:63-69) read from `uniforms`
 * (count floats) starting at running index `start`: prob <= 0 gives ones, prob >= 1 zeros (no
 * draws), else mask[i] = uniforms[(start + i) mod count] < prob ? 0 : 1.  Returns the draws made. */
uint64_t orc_dropout_mask(float* mask, uint64_t n, const float* uniforms, uint64_t count, uint64_t start,
                          float prob);

#ifdef __cplusplus
}
#endif

#endif
