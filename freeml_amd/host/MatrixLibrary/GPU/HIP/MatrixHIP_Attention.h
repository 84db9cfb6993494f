#pragma once
// CausalSelfAttentionLayer on MatrixHIP<float>: Forward and Backwards specialised for this
// backend (explicit specialisations of the two member functions, the class-specialisation
// route FreeML itself takes for backend-specific code, cf. the DX11 loss at
// LossLibrary/CategoricalCrossEntropyWithLogits.h:216-218).  Everything else of the layer --
// blob layout, sublayers, weights, gradients, save/load -- is the reference's.
//
// The reference processes heads one at a time (CausalSelfAttentionLayer.h:424-499 forward,
// :578-660 backward): per head a scores product, ScaleAdd, Softmax, a dropout copy and a P V
// product, and five products plus three element ops backwards -- ~30 and ~50 small launches per
// layer.  Here every step covers all heads at once: the products are batched over heads (one
// strided launch each, the head's column slice selected by the plane offset) and the
// scale/mask/softmax and softmax-backward/mask/scale chains are one kernel each.  The same
// blob matrices are read and written (Scratch_Q/K/V/Y, Scratch_dScores, Scratch_AttHead_h,
// Scratch_dAtt, Scratch_dQh/dKh/dVh, Scratch_QKVGrad, ErrorOutput_0), so the reference's other
// layers and its backward see the state they expect.
//
// The batched path runs when the attention dropout is off (Probability 0, NanoLLM's setting),
// there are at most 32 heads and, backwards, one sequence (TransformerBlock supports only
// that).  Otherwise the layer runs head by head with the dropout sublayers, in the reference's
// order of steps (also when FMLH_ATTENTION_PER_HEAD is set, for comparison).  At dropout 0 the
// per-head dropout sublayers are an identity (mask of ones, scale 1) and are skipped: their
// Output_0 / Mask matrices are then not refreshed.
#include <LayerLibrary/CausalSelfAttentionLayer.h>
#include <MatrixLibrary/GPU/HIP/MatrixHIP.h>

#include <cstdint>
#include <cstdlib>
#include <vector>

namespace freeml_hip {

// How often the batched (all-heads) attention path ran, for tests and diagnostics.
struct AttentionCounts {
    uint64_t batchedForward = 0, perHeadForward = 0, batchedBackward = 0, perHeadBackward = 0;
};
inline AttentionCounts& AttnCounts() {
    static AttentionCounts c;
    return c;
}

constexpr uint32_t kMaxBatchedHeads = 32;

inline bool PerHeadForced() {
    static const bool forced = std::getenv("FMLH_ATTENTION_PER_HEAD") != nullptr;
    return forced;
}

// Probability > 0 in any per-head attention dropout blob of this layer.
inline bool AnyHeadDropout(Datablob<float, MatrixHIP<float>>* blob, uint32_t nHead) {
    for (uint32_t h = 0; h < nHead; ++h) {
        auto* d = blob->GetBlob("CSA_AttentionDropout_" + std::to_string(h));
        if (d && d->GetFloat("Probability") > 0.f) return true;
    }
    return false;
}

}  // namespace freeml_hip

template <>
inline void CausalSelfAttentionLayer<float, Identity<float>, MatrixHIP<float>>::Forward(
    Datablob<float, MatrixHIP<float>>* _blob) {
    using Mat = MatrixHIP<float>;
    auto inputRef = _blob->AcquireMatrix("Input_0");
    Mat* input = inputRef.get();
    auto outputRef = _blob->AcquireMatrix("Output_0");
    Mat* output = outputRef.get();
    auto qRef = _blob->AcquireMatrix("Scratch_Q");
    auto kRef = _blob->AcquireMatrix("Scratch_K");
    auto vRef = _blob->AcquireMatrix("Scratch_V");
    auto triMaskRef = _blob->AcquireMatrix("TriangleMatrix");
    auto scaleRef = _blob->AcquireMatrix("ScalarScale");
    auto scoresRef = _blob->AcquireMatrix("Scratch_dScores");
    auto yRef = _blob->AcquireMatrix("Scratch_Y");
    auto pAllRef = _blob->AcquireMatrix("Scratch_dAtt");
    Datablob<float, Mat>* attBlob = _blob->GetBlob("CSA_AttentionLayer");
    auto attOutRef = attBlob->AcquireMatrix("Output_0");
    Datablob<float, Mat>* residBlob = _blob->GetBlob("CSA_ResidualDropout");
    Datablob<float, Mat>* projBlob = _blob->GetBlob("CSA_ProjLayer");
    auto projOutRef = projBlob->AcquireMatrix("Output_0");

    const AttentionDims dims = GetDims(_blob, input);
    const uint32_t nHead = dims.nHead, dT = dims.T_block_size, dB = dims.B_batch;
    const uint32_t dC = dims.C_EmbedDims, hd = dims.headDim;

    // Packed QKV projection and split (CausalSelfAttentionLayer.h:416-422).
    attBlob->Set("Input_0", input);
    m_attention->Forward(attBlob);
    SplitQKV(qRef.get(), kRef.get(), vRef.get(), attOutRef.get());

    const bool batched = !freeml_hip::PerHeadForced() && nHead <= freeml_hip::kMaxBatchedHeads &&
                         !freeml_hip::AnyHeadDropout(_blob, nHead) && pAllRef.get() && pAllRef->GetDimsZ() >= nHead && pAllRef->GetDimsX() == dT;
    if (batched) {
        std::vector<float*> pHeads(nHead);
        for (uint32_t h = 0; h < nHead; ++h) pHeads[h] = _blob->AcquireMatrix(HeadAttKey(h).c_str())->DeviceOut();
        const float* q = qRef->DeviceIn();
        const float* k = kRef->DeviceIn();
        const float* v = vRef->DeviceIn();
        const float* scale = scaleRef->DeviceIn();
        float* scores = scoresRef->DeviceOut();
        float* pAll = pAllRef->DeviceOut();
        float* y = yRef->DeviceOut();
        const size_t plane = static_cast<size_t>(dT) * dC, tt = static_cast<size_t>(dT) * dT;
        for (uint32_t b = 0; b < dB; ++b) {
            // S_h = Q_h K_h^T for every head (:445-450): head h's columns start at h * hd.
            freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_RIGHT, scores, q + b * plane, k + b * plane, dT, dT, hd,
                                                  dC, 1, dC, 1, dT, 1, nHead, hd, hd, tt),
                              "attention scores");
            freeml_hip::Check(fmlh_attention_softmax_heads(pHeads.data(), b * tt, pAll, scores, scale, nHead, dT),
                              "attention softmax");
            // Y_h = P_h V_h into head h's column slice of Y (:492-497).
            freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_NONE, y + b * plane, pAll, v + b * plane, dT, hd, dT,
                                                  dT, 1, dC, 1, dC, 1, nHead, tt, hd, hd),
                              "attention P V");
        }
        ++freeml_hip::AttnCounts().batchedForward;
    } else {
        // Head by head with the dropout sublayers, the reference's sequence of steps.
        Mat* Q = qRef.get();
        Mat* K = kRef.get();
        Mat* V = vRef.get();
        for (uint32_t h = 0; h < nHead; ++h) {
            Mat* probs = _blob->AcquireMatrix(HeadAttKey(h).c_str()).get();
            for (uint32_t b = 0; b < dB; ++b) {
                Mat qb, kb, qh, kh, s, p;
                Q->GetSliceZ(&qb, b);
                K->GetSliceZ(&kb, b);
                qh.SetData(qb.GetData(), qb.GetOffset() + h * hd);
                qh.SetDims({hd, dT});
                kh.SetData(kb.GetData(), kb.GetOffset() + h * hd);
                kh.SetDims({hd, dT});
                scoresRef->GetSliceZ(&s, h);
                MatMul_Strided<TransposeMode::Right>(&s, &qh, &kh, dC, 1u, dC, 1u, dT, 1u);
                ScaleAdd(&s, &s, scaleRef.get(), triMaskRef.get());
                probs->GetSliceZ(&p, b);
                Softmax(&p, &s);
            }
            Mat* dropped = probs;
            if (Datablob<float, Mat>* dropBlob = GetAttentionDropoutBlob(_blob, h)) {
                m_attentionDropout->SetInput(dropBlob, probs);
                m_attentionDropout->Forward(dropBlob);
                if (Mat* d = m_attentionDropout->GetOutput(dropBlob).get()) dropped = d;
            }
            for (uint32_t b = 0; b < dB; ++b) {
                Mat vb, vh, yb, yh, pb;
                V->GetSliceZ(&vb, b);
                vh.SetData(vb.GetData(), vb.GetOffset() + h * hd);
                vh.SetDims({hd, dT});
                yRef->GetSliceZ(&yb, b);
                yh.SetData(yb.GetData(), yb.GetOffset() + h * hd);
                yh.SetDims({hd, dT});
                dropped->GetSliceZ(&pb, b);
                MatMul_Strided<TransposeMode::None>(&yh, &pb, &vh, dT, 1u, dC, 1u, dC, 1u);
            }
        }
        ++freeml_hip::AttnCounts().perHeadForward;
    }

    // Output projection, then the residual dropout when it is on (:501-513).
    m_proj->SetInput(projBlob, yRef.get());
    m_proj->Forward(projBlob);
    if (residBlob && residBlob->GetFloat("Probability") > 0.f) {
        m_residualDropout->SetInput(residBlob, projOutRef.get());
        m_residualDropout->Forward(residBlob);
        Copy(output, residBlob->AcquireMatrix("Output_0").get());
    } else {
        Copy(output, m_proj->GetOutput(projBlob).get());
    }
}

template <>
inline void CausalSelfAttentionLayer<float, Identity<float>, MatrixHIP<float>>::Backwards(
    Datablob<float, MatrixHIP<float>>* _blob) {
    using Mat = MatrixHIP<float>;
    auto errorRef = _blob->AcquireMatrix("ErrorInput_0");
    Mat* error = errorRef.get();
    auto errorOutRef = _blob->AcquireMatrix("ErrorOutput_0");
    auto inputRef = _blob->AcquireMatrix("Input_0");
    Mat* input = inputRef.get();
    const AttentionDims dims = GetDims(_blob, input);
    const uint32_t nHead = dims.nHead, dT = dims.T_block_size, dC = dims.C_EmbedDims, hd = dims.headDim;
    auto scaleRef = _blob->AcquireMatrix("ScalarScale");
    auto vRef = _blob->AcquireMatrix("Scratch_V");
    auto dAttRef = _blob->AcquireMatrix("Scratch_dAtt");
    auto dScoresRef = _blob->AcquireMatrix("Scratch_dScores");
    auto qRef = _blob->AcquireMatrix("Scratch_Q");
    auto kRef = _blob->AcquireMatrix("Scratch_K");
    auto qkvGradRef = _blob->AcquireMatrix("Scratch_QKVGrad");
    auto dQhRef = _blob->AcquireMatrix("Scratch_dQh");
    auto dKhRef = _blob->AcquireMatrix("Scratch_dKh");
    auto dVhRef = _blob->AcquireMatrix("Scratch_dVh");
    auto finiteMaskRef = _blob->AcquireMatrix("TriangleFiniteMask");

    // Residual dropout, then the output projection's backward (:561-577).
    Mat* projErrorIn = error;
    Datablob<float, Mat>* residBlob = _blob->GetBlob("CSA_ResidualDropout");
    if (residBlob && residBlob->GetFloat("Probability") > 0.f) {
        m_residualDropout->SetErrorInput(residBlob, error);
        m_residualDropout->Backwards(residBlob);
        projErrorIn = m_residualDropout->GetOutputError(residBlob).get();
    }
    Datablob<float, Mat>* projBlob = _blob->GetBlob("CSA_ProjLayer");
    auto yRef = _blob->AcquireMatrix("Scratch_Y");
    auto dYRef = _blob->AcquireMatrix("Scratch_dY");
    m_proj->SetInput(projBlob, yRef);
    m_proj->SetErrorInput(projBlob, projErrorIn);
    m_proj->Backwards(projBlob);
    Copy(dYRef.get(), m_proj->GetOutputError(projBlob).get());

    // Under the same conditions the forward took its batched path, which left P of every head
    // in Scratch_dAtt; it is read (dV) before dAtt overwrites it.
    const bool batched = !freeml_hip::PerHeadForced() && nHead <= freeml_hip::kMaxBatchedHeads && dims.B_batch == 1 &&
                         !freeml_hip::AnyHeadDropout(_blob, nHead) && dAttRef.get() &&
                         dAttRef->GetDimsZ() >= nHead && dAttRef->GetDimsX() == dT;
    if (batched) {
        std::vector<float*> pHeads(nHead);
        for (uint32_t h = 0; h < nHead; ++h)
            pHeads[h] = const_cast<float*>(_blob->AcquireMatrix(HeadAttKey(h).c_str())->DeviceIn());
        const float* dY = dYRef->DeviceIn();
        const float* v = vRef->DeviceIn();
        const float* q = qRef->DeviceIn();
        const float* k = kRef->DeviceIn();
        const float* scale = scaleRef->DeviceIn();
        float* att = dAttRef->DeviceOut();  // holds P (all heads) on entry
        float* dS = dScoresRef->DeviceOut();
        float* dQ = dQhRef->DeviceOut();
        float* dK = dKhRef->DeviceOut();
        float* dV = dVhRef->DeviceOut();
        const size_t tt = static_cast<size_t>(dT) * dT, th = static_cast<size_t>(dT) * hd;
        // dV_h = P_h^T dY_h (:619-624).
        freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_LEFT, dV, att, dY, dT, hd, dT, dT, 1, dC, 1, hd, 1, nHead,
                                              tt, hd, th),
                          "attention dV");
        // dAtt_h = dY_h V_h^T (:612-617), over P now that dV has read it.
        freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_RIGHT, att, dY, v, dT, dT, hd, dC, 1, dC, 1, dT, 1, nHead,
                                              hd, hd, tt),
                          "attention dAtt");
        // dS_h = ((SoftmaxBackwards) * finite mask) * scale (:640-642).
        freeml_hip::Check(fmlh_attention_softmax_backward_heads(dS, pHeads.data(), att, scale, nHead, dT),
                          "attention softmax backward");
        // dQ_h = dS_h K_h, dK_h = dS_h^T Q_h (:645-660).
        freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_NONE, dQ, dS, k, dT, hd, dT, dT, 1, dC, 1, hd, 1, nHead, tt,
                                              hd, th),
                          "attention dQ");
        freeml_hip::Check(fmlh_matmul_strided(FMLH_TRANSPOSE_LEFT, dK, dS, q, dT, hd, dT, dT, 1, dC, 1, hd, 1, nHead, tt,
                                              hd, th),
                          "attention dK");
        ++freeml_hip::AttnCounts().batchedBackward;
    } else {
        // Head by head with the dropout sublayers, the reference's sequence of steps.
        Mat* Q = qRef.get();
        Mat* K = kRef.get();
        Mat* V = vRef.get();
        Mat* dY = dYRef.get();
        for (uint32_t h = 0; h < nHead; ++h) {
            Mat* probs = _blob->AcquireMatrix(HeadAttKey(h).c_str()).get();
            Datablob<float, Mat>* dropBlob = GetAttentionDropoutBlob(_blob, h);
            Mat* dropped = probs;
            if (dropBlob) {
                dropped = m_attentionDropout->GetOutput(dropBlob).get();
                if (!dropped) dropped = dropBlob->GetMatrix("Output_0");
            }
            Mat dAtt, dS, dQh, dKh, dVh, qh, kh, vh, yh;
            dAttRef->GetSliceZ(&dAtt, h);
            dScoresRef->GetSliceZ(&dS, h);
            dQhRef->GetSliceZ(&dQh, h);
            dKhRef->GetSliceZ(&dKh, h);
            dVhRef->GetSliceZ(&dVh, h);
            qh.SetData(Q->GetData(), Q->GetOffset() + h * hd);
            qh.SetDims({hd, dT});
            kh.SetData(K->GetData(), K->GetOffset() + h * hd);
            kh.SetDims({hd, dT});
            vh.SetData(V->GetData(), V->GetOffset() + h * hd);
            vh.SetDims({hd, dT});
            yh.SetData(dY->GetData(), dY->GetOffset() + h * hd);
            yh.SetDims({hd, dT});
            MatMul_Strided<TransposeMode::Right>(&dAtt, &yh, &vh, dC, 1u, dC, 1u, dT, 1u);
            MatMul_Strided<TransposeMode::Left>(&dVh, dropped, &yh, dT, 1u, dC, 1u, hd, 1u);
            if (dropBlob && dropBlob->GetFloat("Probability") > 0.f) {
                m_attentionDropout->SetErrorInput(dropBlob, &dAtt);
                m_attentionDropout->Backwards(dropBlob);
                Copy(&dAtt, m_attentionDropout->GetOutputError(dropBlob).get());
            }
            SoftmaxBackwards(&dS, probs, &dAtt);
            PerElementMul(&dS, &dS, finiteMaskRef.get());
            Scale(&dS, &dS, scaleRef.get());
            MatMul_Strided<TransposeMode::None>(&dQh, &dS, &kh, dT, 1u, dC, 1u, hd, 1u);
            MatMul_Strided<TransposeMode::Left>(&dKh, &dS, &qh, dT, 1u, dC, 1u, hd, 1u);
        }
        ++freeml_hip::AttnCounts().perHeadBackward;
    }

    // Per-head gradients back into the packed layout, then the QKV projection's backward
    // (:662-673).
    MergeQKV(qkvGradRef.get(), dQhRef.get(), dKhRef.get(), dVhRef.get());
    Datablob<float, Mat>* attBlob = _blob->GetBlob("CSA_AttentionLayer");
    m_attention->SetInput(attBlob, input);
    m_attention->SetErrorInput(attBlob, qkvGradRef.get());
    m_attention->Backwards(attBlob);
    Copy(errorOutRef.get(), m_attention->GetOutputError(attBlob).get());
}
