// Harness around the compiled FreeML reference — TEST INFRASTRUCTURE ONLY.
//
// Compiled by oracle/Makefile from the reference sources where they lie (FREEML_REFERENCE_DIR,
// default /root/reference) into oracle/_ref/libfreeml_ref.so.  It includes the reference's own
// Examples/NanoLLM/NanoLLM.cpp so the graph comes from the reference's BuildOrLoadModel
// (NanoLLM.cpp:255-376) and runs through Model::Run on MatrixCPU<float> (Model.h:764-788).
// Nothing of the reference is copied: this file only drives it.  Weights are written into the
// blobs' matrices after the build, so the reference's non-reproducible random init
// (ToolsLibrary/Tools.h:15-27) and residProjScale (TransformerBlock.h:247-256) do not matter.
#define main freeml_reference_nanollm_main
#include <Examples/NanoLLM/NanoLLM.cpp>
#undef main
#undef T

#include <cstring>
#include <memory>

namespace {

struct RefModel {
    NanoLLMConfig cfg;
    uint32_t vocab = 0;
    std::unique_ptr<Model<float, MatType>> model;
    TrainingMatrices tensors;
    MatrixRef input;
    MatrixRef untiedHead;
};

void Write(MatType* m, const float* src, size_t count) {
    assert(m && m->GetElementCount() == count);
    std::memcpy(m->DataWrite(), src, count * sizeof(float));
}

}  // namespace

extern "C" {

// layer_ptrs: n_layer groups of 8 pointers, same order as oracle/nanollm_oracle.h.
// lm_head == tok_emb keeps the reference's tie; any other pointer unties lm_head.
void* ref_create(uint32_t vocab, uint32_t block_size, uint32_t n_embed, uint32_t n_head,
                 uint32_t n_layer, const float* tok_emb, const float* pos_emb,
                 const float* const* layer_ptrs, const float* lnf_gamma,
                 const float* lm_head) {
    Tools::Logger::EnableConsole(false);
    auto* r = new RefModel();
    r->cfg.block_size = block_size;
    r->cfg.batch_size = 1u;
    r->cfg.n_layer = n_layer;
    r->cfg.n_head = n_head;
    r->cfg.n_embed = n_embed;
    r->cfg.dropout = 0.0f;
    r->cfg.use_bias = false;
    r->cfg.model_name = "/nonexistent/freeml_ref_harness_model";  // forces the build branch
    r->vocab = vocab;
    if (!ValidateConfig(r->cfg)) { delete r; return nullptr; }
    Vocab v;
    v.unique.resize(vocab);
    auto& inst = MatrixManager<float, MatType>::Instance();
    r->model = BuildOrLoadModel(r->cfg, v, inst);
    r->tensors = AllocateTrainingMatrices(r->model.get(), r->cfg, inst);
    r->input = inst.AllocateMatrix({1u, block_size, 1u}, "Ref_Input");

    const size_t C = n_embed;
    Model<float, MatType>* m = r->model.get();
    Write(m->GetLayerBlob("embedding_token")->GetMatrix("Embedding_Weights"), tok_emb, vocab * C);
    Write(m->GetLayerBlob("embedding_pos")->GetMatrix("Embedding_Weights"), pos_emb, block_size * C);
    for (uint32_t l = 0; l < n_layer; ++l) {
        const float* const* p = layer_ptrs + 8u * l;
        auto* blk = m->GetLayerBlob("block_" + std::to_string(l));
        auto* att = blk->GetBlob("AttentionLayerData");
        Write(blk->GetBlob("LayerNorm0Data")->GetMatrix("GammaScale"), p[4], C);
        Write(att->GetBlob("CSA_AttentionLayer")->GetMatrix("Dense_Weights"), p[0], C * 3 * C);
        Write(att->GetBlob("CSA_ProjLayer")->GetMatrix("Dense_Weights"), p[1], C * C);
        Write(blk->GetBlob("LayerNorm1Data")->GetMatrix("GammaScale"), p[6], C);
        Write(blk->GetBlob("DenseFCData")->GetMatrix("Dense_Weights"), p[2], C * 4 * C);
        Write(blk->GetBlob("DenseProjData")->GetMatrix("Dense_Weights"), p[3], 4 * C * C);
    }
    Write(m->GetLayerBlob("ln_f")->GetMatrix("GammaScale"), lnf_gamma, C);
    if (lm_head != tok_emb) {
        r->untiedHead = inst.AllocateMatrix({n_embed, vocab}, "Dense_Weights");
        Write(r->untiedHead.get(), lm_head, vocab * C);
        m->GetLayerBlob("lm_head")->Set("Dense_Weights", r->untiedHead);
    }
    return r;
}

// Model::Run on one window of block_size ids; logits: block_size x vocab.
int ref_forward_window(void* h, const int32_t* ids, float* logits) {
    auto* r = static_cast<RefModel*>(h);
    const uint32_t T = r->cfg.block_size;
    for (uint32_t t = 0; t < T; ++t) r->input->SetValue(0u, t, 0u, static_cast<float>(ids[t]));
    r->model->Run(r->input.get(), nullptr);
    MatType* out = r->model->GetOutput();
    if (!out || out->GetDimsX() != r->vocab || out->GetDimsY() != T) return -1;
    std::memcpy(logits, out->DataRead(), sizeof(float) * T * r->vocab);
    return 0;
}

// Greedy loop over full-window recomputes; argmax is the reference's first-max rule
// (NanoLLM.cpp:192-201) applied to logits row len-1.
int ref_greedy(void* h, const int32_t* prompt, uint32_t prompt_len, uint32_t n_gen,
               int32_t* tokens_out, float* logits_out) {
    auto* r = static_cast<RefModel*>(h);
    const uint32_t T = r->cfg.block_size, V = r->vocab;
    if (prompt_len == 0 || prompt_len + n_gen - 1 > T) return -2;
    std::vector<int32_t> hist(prompt, prompt + prompt_len);
    std::vector<float> logits(static_cast<size_t>(T) * V);
    for (uint32_t s = 0; s < n_gen; ++s) {
        std::vector<int32_t> window(T, 0);
        std::copy(hist.begin(), hist.end(), window.begin());
        if (ref_forward_window(h, window.data(), logits.data())) return -1;
        const float* row = logits.data() + static_cast<size_t>(hist.size() - 1) * V;
        if (logits_out) std::memcpy(logits_out + static_cast<size_t>(s) * V, row, sizeof(float) * V);
        uint32_t best = 0;
        float bv = row[0];
        for (uint32_t v = 1; v < V; ++v)
            if (row[v] > bv) { bv = row[v]; best = v; }
        tokens_out[s] = static_cast<int32_t>(best);
        if (hist.size() < T) hist.push_back(static_cast<int32_t>(best));
    }
    return 0;
}

uint32_t ref_thread_count() { return static_cast<uint32_t>(GetGlobalThreadPool()->GetThreadCount()); }

}  // extern "C"

// ---- single reference routines on caller memory (MatrixCPU views, no copies) ------------
// The training-step ops, for pinning the oracle's restatements bit for bit.

namespace {
MatType View(const float* p, uint32_t x, uint32_t y = 1u, uint32_t z = 1u) {
    return MatType(const_cast<float*>(p), Dims3D(x, y, z));
}
}  // namespace

extern "C" {

void ref_softmax_backward(float* out, const float* p, const float* dp, uint32_t rows, uint32_t cols) {
    MatType o = View(out, cols, rows), s = View(p, cols, rows), g = View(dp, cols, rows);
    SoftmaxBackwards(&o, &s, &g);
}

void ref_layernorm_backward(float* dx, const float* dy, const float* in, const float* gamma,
                            float* dgamma, float* dbeta, const float* xhat, uint32_t rows,
                            uint32_t cols, float eps) {
    MatType mdx = View(dx, cols, rows), mdy = View(dy, cols, rows), min = View(in, cols, rows);
    MatType mg = View(gamma, cols), mdg = View(dgamma, cols), mdb = View(dbeta, cols);
    MatType mxh = View(xhat, cols, rows);
    LayerNormBackwardsOp<float>(&mdx, &mdy, &min, &mg, &mdg, dbeta ? &mdb : nullptr,
                                xhat ? &mxh : nullptr, eps);
}

void ref_gelu_derivative(float* out, const float* in, uint32_t n) {
    MatType o = View(out, n), i = View(in, n);
    GeluDerivtiveMat(&o, &i);
}

void ref_scatter_add_rows(float* out, const float* src, const float* idx, uint32_t width,
                          uint32_t src_rows, uint32_t src_batch, uint32_t out_rows,
                          uint32_t out_batch) {
    MatType o = View(out, width, out_rows, out_batch), s = View(src, width, src_rows, src_batch);
    MatType ix = View(idx, 1u, src_rows, src_batch);
    ScatterAddRows(&o, &s, &ix);
}

void ref_merge_qkv(float* packed, const float* q, const float* k, const float* v, uint32_t head_dim,
                   uint32_t tokens, uint32_t n_head) {
    MatType p = View(packed, 3u * head_dim * n_head, tokens);
    MatType mq = View(q, head_dim, tokens, n_head), mk = View(k, head_dim, tokens, n_head);
    MatType mv = View(v, head_dim, tokens, n_head);
    MergeQKV(&p, &mq, &mk, &mv);
}

float ref_cce_logits(float* grad, const float* target, const float* logits, uint32_t vocab,
                     uint32_t steps, uint32_t batch, uint32_t target_cols, uint32_t target_batch) {
    CategoricalCrossEntropyWithLogits<float, MatType> loss;
    MatType t = View(target, target_cols, steps, target_batch), z = View(logits, vocab, steps, batch);
    MatType g = View(grad, vocab, steps, batch);
    if (grad) loss.Gradient(&g, &t, &z);
    return loss.Loss(&t, &z);
}

// GatherRows (MatrixBase_Functions.h:202-242): one plane of `rows` ids (float) into out.
void ref_gather_rows(float* out, const float* src, const float* ids, uint32_t width, uint32_t rows,
                     uint32_t src_rows) {
    MatType o = View(out, width, rows), s = View(src, width, src_rows), ix = View(ids, 1u, rows);
    GatherRows(&o, &s, &ix);
}

// MulStrided<Mode> on raw pointers (MatrixBase_Mul.h:88-144): C (M x N) = op(A) op(B) with
// element strides; A is stored K x M under Left/Both, B N x K under Right/Both.
void ref_mul_strided(int mode, float* C, const float* A, const float* B, uint32_t M, uint32_t N,
                     uint32_t K, uint32_t a_rs, uint32_t a_cs, uint32_t b_rs, uint32_t b_cs,
                     uint32_t c_rs, uint32_t c_cs) {
    const bool tl = mode == 1 || mode == 3, tr = mode == 2 || mode == 3;
    const uint32_t a_rows = tl ? K : M, a_cols = tl ? M : K;
    const uint32_t b_rows = tr ? N : K, b_cols = tr ? K : N;
    switch (mode) {
        case 0: MulStrided<TransposeMode::None>(A, a_rows, a_cols, a_rs, a_cs, B, b_rows, b_cols, b_rs, b_cs, C, c_rs, c_cs); break;
        case 1: MulStrided<TransposeMode::Left>(A, a_rows, a_cols, a_rs, a_cs, B, b_rows, b_cols, b_rs, b_cs, C, c_rs, c_cs); break;
        case 2: MulStrided<TransposeMode::Right>(A, a_rows, a_cols, a_rs, a_cs, B, b_rows, b_cols, b_rs, b_cs, C, c_rs, c_cs); break;
        default: MulStrided<TransposeMode::Both>(A, a_rows, a_cols, a_rs, a_cs, B, b_rows, b_cols, b_rs, b_cs, C, c_rs, c_cs); break;
    }
}

// SumColumns (MatrixBase_Functions.h:1098-1118) of a rows x cols matrix into out (cols).
void ref_sum_columns(float* out, const float* in, uint32_t rows, uint32_t cols) {
    MatType o = View(out, cols, 1u), i = View(in, cols, rows);
    SumColumns(&o, &i);
}

// The first n floats of RandomUtils' uniform buffer (ToolsLibrary/Tools.h:36-50; built on its
// first use in this process); returns its size.
uint64_t ref_uniform_buffer(float* out, uint64_t n) {
    const uint64_t count = RandomUtils::GetUniformBufferCount();
    std::memcpy(out, RandomUtils::GetUniformBufferData(), sizeof(float) * (n < count ? n : count));
    return count;
}

// DropoutLayer::UpdateMask (DropoutLayer.h:97-123) into mask (n floats): its draws advance the
// process-wide buffered-uniform index.
void ref_dropout_mask(float* mask, uint32_t n, float prob) {
    DropoutLayer<float, MatType> layer;
    float zero_v = 0.0f, one_v = 1.0f;
    MatType m = View(mask, n), z = View(&zero_v, 1u), o = View(&one_v, 1u);
    layer.UpdateMask(&m, prob, &z, &o);
}

void ref_adamw_update(float* param, const float* grad, float* mt, float* vt, uint32_t n, float lr,
                      float beta1, float beta2, float beta1_pow_t, float beta2_pow_t, float eps,
                      float weight_decay) {
    MatType p = View(param, n), g = View(grad, n), m = View(mt, n), v = View(vt, n);
    AdamWUpdate<float>(&p, &g, &m, &v, lr, beta1, beta2, beta1_pow_t, beta2_pow_t, eps, weight_decay);
}

}  // extern "C"

// ---- the NanoLLM example's text front end (NanoLLM.cpp:95-252), on caller buffers ---------

extern "C" {

// BuildVocab (NanoLLM.cpp:121-144): unique_out (256 bytes) gets the sorted unique chars,
// ids_out (n) the id of every input char.  Returns the vocabulary size.
uint32_t ref_build_vocab(const char* data, size_t n, char* unique_out, uint32_t* ids_out) {
    Tools::Logger::EnableConsole(false);  // BuildVocab logs the vocabulary
    Vocab v = BuildVocab(std::vector<char>(data, data + n));
    std::memcpy(unique_out, v.unique.data(), v.unique.size());
    std::memcpy(ids_out, v.ids.data(), v.ids.size() * sizeof(uint32_t));
    return static_cast<uint32_t>(v.unique.size());
}

// encode (NanoLLM.cpp:146-155) with the map BuildVocab makes from `unique`.
void ref_encode(const char* unique, uint32_t n_unique, const char* s, size_t n, uint32_t* ids_out) {
    std::map<char, uint32_t> toId;
    for (uint32_t i = 0; i < n_unique; ++i) toId[unique[i]] = i;
    std::vector<uint32_t> ids = encode(std::string(s, n), toId);
    std::memcpy(ids_out, ids.data(), ids.size() * sizeof(uint32_t));
}

// decode (NanoLLM.cpp:157-166).
void ref_decode(const char* unique, uint32_t n_unique, const uint32_t* ids, size_t n, char* out) {
    std::map<uint32_t, char> toChar;
    for (uint32_t i = 0; i < n_unique; ++i) toChar[i] = unique[i];
    std::vector<char> c = decode(std::vector<uint32_t>(ids, ids + n), toChar);
    std::memcpy(out, c.data(), c.size());
}

// DecodeMatrixTokens (NanoLLM.cpp:168-206) of a {cols, steps} matrix: cols == 1 reads ids,
// otherwise the first maximum of each row.
void ref_decode_matrix_tokens(const float* mat, uint32_t cols, uint32_t steps, const char* unique,
                              uint32_t n_unique, char* out) {
    MatType m = View(mat, cols, steps);
    const std::string s = DecodeMatrixTokens(&m, std::vector<char>(unique, unique + n_unique));
    std::memcpy(out, s.data(), s.size());
}

// CountCorrectTokensBatch (NanoLLM.cpp:226-252) for batch index 0.
uint32_t ref_count_correct(const float* logits, const float* target, uint32_t block, uint32_t vocab) {
    MatType o = View(logits, vocab, block), t = View(target, 1u, block);
    return CountCorrectTokensBatch(&o, &t, block, vocab, 0u);
}

}  // extern "C"
