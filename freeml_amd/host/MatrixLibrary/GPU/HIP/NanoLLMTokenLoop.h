#pragma once
// Greedy token loop over a NanoLLM Model<float, MatrixHIP<float>>.
//
// The reference builds NanoLLM with BuildOrLoadModel (Examples/NanoLLM/NanoLLM.cpp:255-376)
// and has no autoregressive loop; its per-step semantics are Model::Run over the padded
// window, logits row len-1, first-max argmax (NanoLLM.cpp:189-205).  This helper reads the
// parameters straight from the model's blobs (the keys of Embedding.h:30-43, Dense.h:36-72,
// LayerNorm.h:111-121, CausalSelfAttentionLayer.h:47-51, TransformerBlock.h:222-333) as device
// pointers and drives the fmlh_nanollm_* loop of freeml_hip.h, which keeps a KV cache on the
// device and picks tokens without host round trips.  The engine references the embeddings,
// W_proj, the LayerNorm parameters and lm_head in the blobs, and keeps transposed copies of
// W_qkv, W_fc and W_proj2 taken at Create: after the model's parameters change (a training
// step), call Refresh() before the next Generate.
#include <MatrixLibrary/GPU/HIP/MatrixHIP.h>
#include <ModelLibrary/Model.h>

#include <cstdint>
#include <string>
#include <vector>

namespace freeml_hip {

class NanoLLMTokenLoop {
public:
    NanoLLMTokenLoop() = default;
    ~NanoLLMTokenLoop() { Destroy(); }
    NanoLLMTokenLoop(const NanoLLMTokenLoop&) = delete;
    NanoLLMTokenLoop& operator=(const NanoLLMTokenLoop&) = delete;

    // Layer names as NanoLLM.cpp names them; maxBatch independent sequences.
    bool Create(Model<float, MatrixHIP<float>>* model, uint32_t maxBatch = 1) {
        Destroy();
        auto dev = [](MatrixHIP<float>* m) -> const float* { return m ? m->DeviceIn() : nullptr; };
        auto* tokBlob = model->GetLayerBlob("embedding_token");
        auto* posBlob = model->GetLayerBlob("embedding_pos");
        auto* lnfBlob = model->GetLayerBlob("ln_f");
        auto* headBlob = model->GetLayerBlob("lm_head");
        if (!tokBlob || !posBlob || !lnfBlob || !headBlob) return Fail("not a NanoLLM graph (missing layers)");
        MatrixHIP<float>* tok = tokBlob->GetMatrix("Embedding_Weights");
        MatrixHIP<float>* pos = posBlob->GetMatrix("Embedding_Weights");
        MatrixHIP<float>* head = headBlob->GetMatrix("Dense_Weights");
        if (!tok || !pos || !head) return Fail("missing embedding or lm_head weights");
        fmlh_nanollm_config cfg{};
        cfg.n_embed = tok->GetDimsX();
        cfg.vocab = tok->GetDimsY();
        cfg.block_size = pos->GetDimsY();
        cfg.max_batch = maxBatch;
        uint32_t L = 0;
        while (model->GetLayerBlob("block_" + std::to_string(L))) ++L;
        if (L == 0) return Fail("no TransformerBlock layers");
        cfg.n_layer = L;
        m_layerPtrs.assign(8u * L, nullptr);
        for (uint32_t l = 0; l < L; ++l) {
            auto* blk = model->GetLayerBlob("block_" + std::to_string(l));
            auto* att = blk->GetBlob("AttentionLayerData");
            auto* ln0 = blk->GetBlob("LayerNorm0Data");
            auto* ln1 = blk->GetBlob("LayerNorm1Data");
            auto* fc = blk->GetBlob("DenseFCData");
            auto* pr = blk->GetBlob("DenseProjData");
            if (!att || !ln0 || !ln1 || !fc || !pr) return Fail("block blobs not allocated (Model::Init not run?)");
            if (att->GetBlob("CSA_AttentionLayer")->GetMatrix("Dense_Bias") || fc->GetMatrix("Dense_Bias"))
                return Fail("Dense biases (use_bias = true) are not supported by the token loop");
            cfg.n_head = att->GetUInt("NumHeads");
            const float** p = m_layerPtrs.data() + 8u * l;
            p[0] = dev(att->GetBlob("CSA_AttentionLayer")->GetMatrix("Dense_Weights"));
            p[1] = dev(att->GetBlob("CSA_ProjLayer")->GetMatrix("Dense_Weights"));
            p[2] = dev(fc->GetMatrix("Dense_Weights"));
            p[3] = dev(pr->GetMatrix("Dense_Weights"));
            p[4] = dev(ln0->GetMatrix("GammaScale"));
            p[5] = dev(ln0->GetMatrix("BetaShift"));
            p[6] = dev(ln1->GetMatrix("GammaScale"));
            p[7] = dev(ln1->GetMatrix("BetaShift"));
        }
        fmlh_nanollm_weights w{};
        w.tok_emb = dev(tok);
        w.pos_emb = dev(pos);
        w.layers = m_layerPtrs.data();
        w.lnf_gamma = dev(lnfBlob->GetMatrix("GammaScale"));
        w.lnf_beta = dev(lnfBlob->GetMatrix("BetaShift"));
        w.lm_head = head->GetStorage() == tok->GetStorage() ? w.tok_emb : dev(head);
        m_vocab = cfg.vocab;
        return Check(fmlh_nanollm_create(&cfg, &w, 1, &m_loop), "fmlh_nanollm_create");
    }

    // prompts: batch x promptLen ids.  tokens: batch x nGen; logits (optional): batch x nGen x V.
    bool Generate(const std::vector<int32_t>& prompts, uint32_t batch, uint32_t nGen,
                  std::vector<int32_t>& tokens, std::vector<float>* logits = nullptr) {
        if (!m_loop || batch == 0 || prompts.size() % batch) return Fail("bad Generate arguments");
        const uint32_t promptLen = static_cast<uint32_t>(prompts.size() / batch);
        tokens.assign(static_cast<size_t>(batch) * nGen, 0);
        float* lg = nullptr;
        if (logits) {
            logits->assign(static_cast<size_t>(batch) * nGen * m_vocab, 0.f);
            lg = logits->data();
        }
        return Check(fmlh_nanollm_generate(m_loop, prompts.data(), batch, promptLen, nGen, tokens.data(), lg),
                      "fmlh_nanollm_generate");
    }

    // Re-takes the transposed weight copies after the blobs' parameters were updated in place.
    bool Refresh() {
        if (!m_loop) return Fail("Refresh before Create");
        return Check(fmlh_nanollm_refresh_weights(m_loop), "fmlh_nanollm_refresh_weights");
    }

    fmlh_nanollm* Handle() { return m_loop; }

    void Destroy() {
        if (m_loop) fmlh_nanollm_destroy(m_loop);
        m_loop = nullptr;
    }

private:
    bool Fail(const char* why) {
        LOG_ERROR() << "NanoLLMTokenLoop: " << why;
        return false;
    }

    fmlh_nanollm* m_loop = nullptr;
    std::vector<const float*> m_layerPtrs;
    uint32_t m_vocab = 0;
};

}  // namespace freeml_hip
