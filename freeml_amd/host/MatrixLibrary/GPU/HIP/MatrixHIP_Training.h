#pragma once
// Training-step overloads for MatrixHIP<float>: the routines Model::Run(input, target)
// reaches after the forward (ModelLibrary/Model.h:790-878) -- the loss gradient, every layer's
// Backwards and the optimiser step -- plus the TrainLoop's window copy.  Like the forward set
// in MatrixHIP_Functions.h they are found by overload resolution (or, for the loss, by class
// template specialisation, as the DX11 backend does at
// LossLibrary/CategoricalCrossEntropyWithLogits.h:216-400), so FreeML's layer code runs
// unchanged and every matrix stays on the device through the step.
//
// Covered here: SoftmaxBackwards, LayerNormBackwardsOp, GeluDerivtiveMat, ScatterAddRows,
// MergeQKV, CopyRange, AdamWUpdate, CategoricalCrossEntropyWithLogits, SumColumns (the Dense
// bias gradient) and DropoutLayer::UpdateMask (the dropout mask, drawn on the device from the
// reference's own uniform buffer).  The backward's
// products (Mul<Left/None/Right>, MatMul_Strided) and element ops (Copy, Add, PerElementMul,
// Scale, Clear) are the forward set's overloads.  Included by MatrixHIP_Functions.h.
#include <LayerLibrary/DropoutLayer.h>
#include <LossLibrary/CategoricalCrossEntropyWithLogits.h>
#include <MatrixLibrary/GPU/HIP/MatrixHIP.h>
#include <ToolsLibrary/Tools.h>
#include <MatrixLibrary/MatrixBase_Functions.h>

#include <cstdint>

namespace freeml_hip {

// A device buffer of at least `floats` floats for routines that need scratch space (row
// statistics, per-row losses).  One per process, grown on demand; calls are stream-ordered, so
// consecutive users do not overlap.
inline float* Scratch(size_t floats) {
    static float* buf = nullptr;
    static size_t have = 0;
    if (floats > have) {
        if (buf) Check(fmlh_free(buf), "fmlh_free");
        void* p = nullptr;
        have = 0;
        buf = nullptr;
        if (!Check(fmlh_malloc(&p, floats * sizeof(float)), "fmlh_malloc")) return nullptr;
        buf = static_cast<float*>(p);
        have = floats;
    }
    return buf;
}

inline bool SameDims(const Dims3D& a, const Dims3D& b) { return a.x == b.x && a.y == b.y && a.z == b.z; }

// RandomUtils' buffer of uniforms (ToolsLibrary/Tools.h:36-50) on the device, copied once per
// process at the first dropout mask, and this backend's running index into it.
// random_uniform_buffered (Tools.h:63-69) reads that buffer at a process-wide index that
// starts at 0; MatrixHIP keeps its own index, also from 0, so a process that trains on
// MatrixHIP draws exactly the masks a MatrixCPU process would draw from the same buffer, in
// the same order of UpdateMask calls (a process that also draws on MatrixCPU keeps the two
// indices apart).
struct DeviceUniforms {
    float* dev = nullptr;
    uint64_t count = 0;
    uint64_t next = 0;
};

inline DeviceUniforms* Uniforms() {
    static DeviceUniforms u;
    if (!u.dev) {
        const uint64_t n = RandomUtils::GetUniformBufferCount();
        void* p = nullptr;
        if (n == 0 || !Check(fmlh_malloc(&p, n * sizeof(float)), "fmlh_malloc")) return nullptr;
        if (!Check(fmlh_memcpy_h2d(p, RandomUtils::GetUniformBufferData(), n * sizeof(float)), "fmlh_memcpy_h2d")) {
            Check(fmlh_free(p), "fmlh_free");
            return nullptr;
        }
        ++Stats().toDevice;
        u.dev = static_cast<float*>(p);
        u.count = n;
    }
    return &u;
}

}  // namespace freeml_hip

// SumColumns (MatrixBase_Functions.h:1098-1118): the column sums of _in's first plane into row
// 0 of _out, each column's rows added in order (Dense::Backwards' bias gradient,
// Dense.h:263, :272).
template <class T>
void SumColumns(MatrixHIP<T>* _out, MatrixHIP<T>* _in) {
    if (!freeml_hip::Require(_out->GetDimsX() == _in->GetDimsX() && _out->GetDimsY() > 0, "SumColumns: dims"))
        return;
    const float* in = _in->DeviceIn();
    float* out = _out->DeviceOut();
    freeml_hip::Check(fmlh_sum_columns(out, in, _in->GetDimsY(), _in->GetDimsX()), "SumColumns");
}

// DropoutLayer::UpdateMask (DropoutLayer.h:97-123) on the device: the same three branches
// (ones for prob <= 0, zeros for prob >= 1, else one buffered uniform per element in element
// order, 0 where it is below prob), with the draws read from the device copy of the
// reference's uniform buffer.  An explicit specialisation of the member, as
// MatrixHIP_Attention.h specialises the attention layer's; the rest of the layer is the
// reference's.
template <>
inline void DropoutLayer<float, MatrixHIP<float>>::UpdateMask(MatrixHIP<float>* _mask, float _prob,
                                                               MatrixHIP<float>* _zero, MatrixHIP<float>* _one) {
    assert(_mask);
    assert(_zero);
    assert(_one);
    const uint64_t n = _mask->GetElementCount();
    if (n == 0) return;
    if (_prob <= 0.0f) {
        Fill(_mask, _one);
        return;
    }
    if (_prob >= 1.0f) {
        Fill(_mask, _zero);
        return;
    }
    freeml_hip::DeviceUniforms* u = freeml_hip::Uniforms();
    if (!freeml_hip::Require(u != nullptr, "UpdateMask: no device copy of the uniform buffer")) return;
    freeml_hip::Check(fmlh_dropout_mask(_mask->DeviceOut(), n, u->dev, u->count, u->next, _prob), "UpdateMask");
    u->next += n;
}

// SoftmaxBackwards (MatrixBase_Functions.h:83-111): rows = DimsY of the softmax output, as
// the reference iterates them.
template <class T>
void SoftmaxBackwards(MatrixHIP<T>* _out, MatrixHIP<T>* _softmaxOut, MatrixHIP<T>* _gradIn) {
    const uint32_t cols = _softmaxOut->GetDimsX(), rows = _softmaxOut->GetDimsY();
    if (!freeml_hip::Require(_out->GetDimsX() == cols && _out->GetDimsY() == rows,
                             "SoftmaxBackwards: output dims") ||
        !freeml_hip::Require(_gradIn->GetDimsX() == cols && _gradIn->GetDimsY() == rows,
                             "SoftmaxBackwards: gradient dims"))
        return;
    const float* p = _softmaxOut->DeviceIn();
    const float* g = _gradIn->DeviceIn();
    freeml_hip::Check(fmlh_softmax_backward(_out->DeviceOut(), p, g, rows, cols), "SoftmaxBackwards");
}

// LayerNormBackwardsOp (MatrixBase_Functions.h:552-705), called as LayerNorm::Backwards does
// (LayerNormBackwardsOp<T>(errorOut, error, input, gamma, gammaGrad, betaGrad, xHat, eps)).
template <class T>
void LayerNormBackwardsOp(MatrixHIP<T>* _dX, MatrixHIP<T>* _dY, MatrixHIP<T>* _in,
                          MatrixHIP<T>* _gamma, MatrixHIP<T>* _dGamma, MatrixHIP<T>* _dBeta = nullptr,
                          MatrixHIP<T>* _xHat = nullptr, T _eps = static_cast<T>(1e-5)) {
    const uint32_t cols = _in->GetDimsX();
    const uint32_t rows = _in->GetDimsY() * _in->GetDimsZ();
    if (!freeml_hip::Require(_dX && _dY && _gamma && _dGamma, "LayerNormBackwardsOp: null operand") ||
        !freeml_hip::Require(freeml_hip::SameDims(_dX->GetDims(), _in->GetDims()) && freeml_hip::SameDims(_dY->GetDims(), _in->GetDims()),
                             "LayerNormBackwardsOp: dX/dY dims") ||
        !freeml_hip::Require(_gamma->GetDimsX() == cols && _dGamma->GetDimsX() == cols,
                             "LayerNormBackwardsOp: gamma dims") ||
        !freeml_hip::Require(!_dBeta || _dBeta->GetDimsX() == cols, "LayerNormBackwardsOp: beta dims") ||
        !freeml_hip::Require(!_xHat || freeml_hip::SameDims(_xHat->GetDims(), _in->GetDims()), "LayerNormBackwardsOp: xHat dims"))
        return;
    const float* dy = _dY->DeviceIn();
    const float* in = _in->DeviceIn();
    const float* g = _gamma->DeviceIn();
    const float* xh = _xHat ? _xHat->DeviceIn() : nullptr;
    float* ws = xh ? nullptr : freeml_hip::Scratch(2 * static_cast<size_t>(rows));
    float* db = _dBeta ? _dBeta->DeviceOut() : nullptr;
    float* dg = _dGamma->DeviceOut();
    freeml_hip::Check(fmlh_layernorm_backward(_dX->DeviceOut(), dy, in, g, dg, db, xh, ws, rows, cols,
                                              static_cast<float>(_eps)),
                      "LayerNormBackwardsOp");
}

// GeluDerivtiveMat (MatrixBase_Functions.h:1002-1017), via Gelu::derivativeMat.
template <class T>
void GeluDerivtiveMat(MatrixHIP<T>* _out, MatrixHIP<T>* _in) {
    if (!freeml_hip::Require(_out->GetElementCount() >= _in->GetElementCount(), "GeluDerivtiveMat: output size"))
        return;
    const float* in = _in->DeviceIn();
    freeml_hip::Check(fmlh_gelu_derivative(_out->DeviceOut(), in, _in->GetElementCount()), "GeluDerivtiveMat");
}

// ScatterAddRows (MatrixBase_Functions.h:285-327), via Embedding::Backwards.
template <class T>
void ScatterAddRows(MatrixHIP<T>* _out, MatrixHIP<T>* _src, MatrixHIP<T>* _indices) {
    if (!freeml_hip::Require(_indices->GetDimsX() == 1u, "ScatterAddRows: indices must be one column") ||
        !freeml_hip::Require(_src->GetDimsX() == _out->GetDimsX(), "ScatterAddRows: row widths differ") ||
        !freeml_hip::Require(_src->GetDimsY() == _indices->GetDimsY() && _src->GetDimsZ() == _indices->GetDimsZ(),
                             "ScatterAddRows: one index per source row") ||
        !freeml_hip::Require(_out->GetDimsZ() == 1u || _out->GetDimsZ() == _src->GetDimsZ(),
                             "ScatterAddRows: output batch"))
        return;
    const float* src = _src->DeviceIn();
    const float* idx = _indices->DeviceIn();
    freeml_hip::Check(fmlh_scatter_add_rows(_out->DeviceOut(), src, idx, _src->GetDimsX(), _src->GetDimsY(),
                                            _src->GetDimsZ(), _out->GetDimsY(), _out->GetDimsZ()),
                      "ScatterAddRows");
}

// MergeQKV (MatrixBase_Functions.h:369-431), via CausalSelfAttentionLayer::Backwards.
template <class T>
void MergeQKV(MatrixHIP<T>* _packedQKV, MatrixHIP<T>* _qHeads, MatrixHIP<T>* _kHeads, MatrixHIP<T>* _vHeads) {
    const uint32_t hd = _qHeads->GetDimsX(), tokens = _qHeads->GetDimsY(), nHead = _qHeads->GetDimsZ();
    if (!freeml_hip::Require(freeml_hip::SameDims(_kHeads->GetDims(), _qHeads->GetDims()) && freeml_hip::SameDims(_vHeads->GetDims(), _qHeads->GetDims()),
                             "MergeQKV: head dims differ") ||
        !freeml_hip::Require(_packedQKV->GetDimsX() == 3u * hd * nHead && _packedQKV->GetDimsY() == tokens &&
                                 _packedQKV->GetDimsZ() == 1u,
                             "MergeQKV: packed dims"))
        return;
    const float* q = _qHeads->DeviceIn();
    const float* k = _kHeads->DeviceIn();
    const float* v = _vHeads->DeviceIn();
    freeml_hip::Check(fmlh_merge_qkv(_packedQKV->DeviceOut(), q, k, v, hd, tokens, nHead), "MergeQKV");
}

// CopyRange (MatrixBase_Functions.h:163-181): the TrainLoop's window and target copies out of
// the corpus matrix (Examples/NanoLLM/NanoLLM.cpp:441-442).
template <class T>
void CopyRange(MatrixHIP<T>* _out, MatrixHIP<T>* _in, uint32_t outOffset, uint32_t inOffset, uint32_t count) {
    if (count == 0u) return;
    if (!freeml_hip::Require(static_cast<uint64_t>(outOffset) + count <= _out->GetElementCount() &&
                                 static_cast<uint64_t>(inOffset) + count <= _in->GetElementCount(),
                             "CopyRange: range outside a matrix"))
        return;
    const float* in = _in->DeviceIn() + inOffset;
    freeml_hip::Check(fmlh_copy(_out->DeviceOut() + outOffset, in, count), "CopyRange");
}

// AdamWUpdate (MatrixBase_Functions.h:1497-1545).  AdamWOptimiser::Step calls it with every
// operand cast to MatrixBase<T>* (OptimiserLibrary/AdamWOptimiser.h:175-187), so this is a
// non-template MatrixBase<float> overload (preferred over the reference template): MatrixHIP
// operands update on the device, any other backend goes to the reference routine.
inline void AdamWUpdate(MatrixBase<float>* param, MatrixBase<float>* grad, MatrixBase<float>* mt,
                        MatrixBase<float>* vt, float lr, float beta1, float beta2, float beta1_pow_t,
                        float beta2_pow_t, float eps, float weightDecay) {
    auto* p = dynamic_cast<MatrixHIP<float>*>(param);
    auto* g = dynamic_cast<MatrixHIP<float>*>(grad);
    auto* m = dynamic_cast<MatrixHIP<float>*>(mt);
    auto* v = dynamic_cast<MatrixHIP<float>*>(vt);
    if (!(p && g && m && v)) {
        AdamWUpdate<float>(param, grad, mt, vt, lr, beta1, beta2, beta1_pow_t, beta2_pow_t, eps, weightDecay);
        return;
    }
    const size_t n = p->GetElementCount();
    if (!freeml_hip::Require(g->GetElementCount() == n && m->GetElementCount() == n && v->GetElementCount() == n,
                             "AdamWUpdate: element counts differ"))
        return;
    const float* gd = g->DeviceIn();
    float* md = m->DeviceOut();
    float* vd = v->DeviceOut();
    freeml_hip::Check(fmlh_adamw_update(p->DeviceOut(), gd, md, vd, n, lr, beta1, beta2, beta1_pow_t,
                                        beta2_pow_t, eps, weightDecay),
                      "AdamWUpdate");
}

// CategoricalCrossEntropyWithLogits on MatrixHIP (LossLibrary/CategoricalCrossEntropyWithLogits.h:
// 29-208): same targets (index with -1 ignored, or one-hot), same gradient sign and scaling.
// Gradient stays on the device; Loss returns the scalar, one 4-byte readback.
template <class T>
class CategoricalCrossEntropyWithLogits<T, MatrixHIP<T>> : public LossBase<T, MatrixHIP<T>> {
public:
    const char* GetName() const override { return "CategoricalCrossEntropyWithLogits"; }

    T Loss(MatrixHIP<T>* target, MatrixHIP<T>* logits) override {
        Shape s;
        if (!Check(target, logits, s)) return T(0);
        float* ws = freeml_hip::Scratch(static_cast<size_t>(s.steps) * s.batch + 1);
        const float* tg = target->DeviceIn();
        const float* lg = logits->DeviceIn();
        if (!freeml_hip::Check(fmlh_cce_logits(nullptr, ws, ws + 1, tg, lg, s.vocab, s.steps, s.batch,
                                               target->GetDimsX(), target->GetDimsZ()),
                               "CategoricalCrossEntropyWithLogits::Loss"))
            return T(0);
        float loss = 0.0f;
        freeml_hip::Check(fmlh_memcpy_d2h(&loss, ws, sizeof(float)), "fmlh_memcpy_d2h");
        ++freeml_hip::Stats().toHost;
        return static_cast<T>(loss);
    }

    void Gradient(MatrixHIP<T>* out, MatrixHIP<T>* target, MatrixHIP<T>* logits) override {
        Shape s;
        if (!Check(target, logits, s)) return;
        if (!freeml_hip::Require(freeml_hip::SameDims(out->GetDims(), logits->GetDims()), "CategoricalCrossEntropyWithLogits: gradient dims"))
            return;
        const float* tg = target->DeviceIn();
        const float* lg = logits->DeviceIn();
        freeml_hip::Check(fmlh_cce_logits(out->DeviceOut(), nullptr, nullptr, tg, lg, s.vocab, s.steps, s.batch,
                                          target->GetDimsX(), target->GetDimsZ()),
                          "CategoricalCrossEntropyWithLogits::Gradient");
    }

private:
    struct Shape {
        uint32_t vocab = 0, steps = 0, batch = 0;
    };

    static bool Check(MatrixHIP<T>* target, MatrixHIP<T>* logits, Shape& s) {
        s.vocab = logits->GetDimsX();
        s.steps = logits->GetDimsY();
        s.batch = logits->GetDimsZ();
        if (s.vocab == 0 || s.steps == 0 || s.batch == 0) return false;
        return freeml_hip::Require(target->GetDimsX() == 1u || target->GetDimsX() == s.vocab,
                                   "CategoricalCrossEntropyWithLogits: target width") &&
               freeml_hip::Require(target->GetDimsY() == s.steps, "CategoricalCrossEntropyWithLogits: target steps") &&
               freeml_hip::Require(target->GetDimsZ() == 1u || target->GetDimsZ() == s.batch,
                                   "CategoricalCrossEntropyWithLogits: target batch");
    }
};
