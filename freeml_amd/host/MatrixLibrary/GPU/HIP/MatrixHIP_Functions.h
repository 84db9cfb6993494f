#pragma once
// Op overloads for MatrixHIP<float>: the free functions FreeML's layers call unqualified
// (e.g. Mul<Mode>(out, in, w) in Dense.h:201-208).  Overload resolution prefers these exact
// MatrixHIP<T>* matches over the generic MatrixBase<T>* templates (MatrixBase_Functions.h,
// MatrixBase_Mul.h), exactly as it picks the MatrixDX11<T>* overloads of
// MatrixDX11_Functions.h on Windows.  Include this header before the model is instantiated.
//
// Covered: the NanoLLM forward set (Mul, MatMul_Strided, SplitQKV, ScaleAdd, Softmax,
// LayerNormOp, GeluMat, Add, Copy, GatherRows, BroadcastAdd) plus the ops the forward of
// training-mode blobs reaches (Fill, PerElementMul, Scale, Clear).  Every other generic
// FreeML routine still works on MatrixHIP through DataRead/DataWrite on the host mirror.
//
// Argument checks follow the reference: assert on shape mismatch (and, in release builds,
// log and return without computing, the DX11 backend's convention).
#include <MatrixLibrary/GPU/HIP/MatrixHIP.h>
#include <MatrixLibrary/MatrixBase_Functions.h>
#include <MatrixLibrary/MatrixBase_Mul.h>
#include <ToolsLibrary/ThreadPool.h>

#include <cstdint>

namespace freeml_hip {

inline bool Require(bool ok, const char* what) {
    if (!ok) {
        LOG_ERROR() << "freeml_hip: " << what;
        assert(ok);
    }
    return ok;
}

template <class T>
inline bool Same(MatrixHIP<T>* a, MatrixHIP<T>* b) {
    return a->GetElementCount() == b->GetElementCount();
}

}  // namespace freeml_hip

// Mul<Mode> (MatrixBase_Mul.h:591-615).
template <TransposeMode Mode = TransposeMode::None, class T>
void Mul(MatrixHIP<T>* _out, MatrixHIP<T>* _L, MatrixHIP<T>* _R, uint32_t = 32, uint32_t = 12,
         ThreadPool* = nullptr) {
    constexpr bool TL = (Mode == TransposeMode::Left) || (Mode == TransposeMode::Both);
    constexpr bool TR = (Mode == TransposeMode::Right) || (Mode == TransposeMode::Both);
    const uint32_t M = TL ? _L->GetDimsX() : _L->GetDimsY();
    const uint32_t K = TL ? _L->GetDimsY() : _L->GetDimsX();
    const uint32_t N = TR ? _R->GetDimsY() : _R->GetDimsX();
    if (!freeml_hip::Require(_L->GetDimsZ() == 1 && _R->GetDimsZ() == 1, "Mul: batched operand") ||
        !freeml_hip::Require(K == (TR ? _R->GetDimsX() : _R->GetDimsY()), "Mul: inner dims differ") ||
        !freeml_hip::Require(_out->GetDimsY() == M && _out->GetDimsX() == N, "Mul: output dims"))
        return;
    const float* l = _L->DeviceIn();
    const float* r = _R->DeviceIn();
    float* o = _out->DeviceOut();
    freeml_hip::Check(fmlh_mul(static_cast<int>(Mode), o, l, r, M, N, K), "Mul");
}

// MatMul_Strided<Mode> (MatrixBase_Mul.h:617-722), including its batched planes (:678-680).
template <TransposeMode Mode = TransposeMode::None, class T>
void MatMul_Strided(MatrixHIP<T>* _out, MatrixHIP<T>* _L, MatrixHIP<T>* _R, uint32_t L_rowStride,
                    uint32_t L_colStride, uint32_t R_rowStride, uint32_t R_colStride,
                    uint32_t outRowStride, uint32_t outColStride, uint32_t = 32, uint32_t = 12,
                    ThreadPool* = nullptr) {
    constexpr bool TL = (Mode == TransposeMode::Left) || (Mode == TransposeMode::Both);
    constexpr bool TR = (Mode == TransposeMode::Right) || (Mode == TransposeMode::Both);
    if (!freeml_hip::Require(_L->GetDimsZ() == _R->GetDimsZ() && _out->GetDimsZ() == _L->GetDimsZ(),
                             "MatMul_Strided: batch dims differ"))
        return;
    const uint32_t L_rows = _L->GetDimsY(), L_cols = _L->GetDimsX();
    const uint32_t R_rows = _R->GetDimsY(), R_cols = _R->GetDimsX();
    const uint32_t M = TL ? L_cols : L_rows;
    const uint32_t K = TL ? L_rows : L_cols;
    const uint32_t N = TR ? R_rows : R_cols;
    if (!freeml_hip::Require(K == (TR ? R_cols : R_rows), "MatMul_Strided: inner dims differ")) return;
    const uint32_t batch = _L->GetDimsZ();
    const size_t lp = static_cast<size_t>(L_rowStride) * L_rows;
    const size_t rp = static_cast<size_t>(R_rowStride) * R_rows;
    const size_t op = static_cast<size_t>(outRowStride) * _out->GetDimsY();
    const float* l = _L->DeviceIn();
    const float* r = _R->DeviceIn();
    float* o = _out->DeviceOut();
    freeml_hip::Check(fmlh_matmul_strided(static_cast<int>(Mode), o, l, r, M, N, K, L_rowStride,
                                          L_colStride, R_rowStride, R_colStride, outRowStride,
                                          outColStride, batch, lp, rp, op),
                      "MatMul_Strided");
}

// SplitQKV (MatrixBase_Functions.h:329-367).
template <class T>
void SplitQKV(MatrixHIP<T>* _q, MatrixHIP<T>* _k, MatrixHIP<T>* _v, MatrixHIP<T>* _packed) {
    const uint32_t dC = _q->GetDimsX();
    const uint32_t rows = _q->GetDimsY() * _q->GetDimsZ();
    if (_q->GetElementCount() == 0u) return;
    if (!freeml_hip::Require(_packed->GetDimsX() == 3u * dC && _packed->GetElementCount() == 3u * _q->GetElementCount(),
                             "SplitQKV: packed dims"))
        return;
    const float* p = _packed->DeviceIn();
    freeml_hip::Check(fmlh_split_qkv(_q->DeviceOut(), _k->DeviceOut(), _v->DeviceOut(), p, rows, dC),
                      "SplitQKV");
}

// ScaleAdd(out, in, Mat* scale, add) (MatrixBase_Functions.h:1055-1070).
template <class T>
void ScaleAdd(MatrixHIP<T>* _out, MatrixHIP<T>* _in, MatrixHIP<T>* _scale, MatrixHIP<T>* _add) {
    if (!freeml_hip::Require(freeml_hip::Same(_out, _in) && freeml_hip::Same(_out, _add),
                             "ScaleAdd: element counts differ"))
        return;
    const float* in = _in->DeviceIn();
    const float* s = _scale->DeviceIn();
    const float* a = _add->DeviceIn();
    freeml_hip::Check(fmlh_scale_add(_out->DeviceOut(), in, s, a, _out->GetElementCount()), "ScaleAdd");
}

// ScaleAdd(out, in, float scale, add) (MatrixBase_Functions.h:1040-1053).
template <class T>
void ScaleAdd(MatrixHIP<T>* _out, MatrixHIP<T>* _in, float _scale, MatrixHIP<T>* _add) {
    if (!freeml_hip::Require(freeml_hip::Same(_out, _in) && freeml_hip::Same(_out, _add),
                             "ScaleAdd: element counts differ"))
        return;
    // out = in * scale, then out = out * 1 + add keeps the reference's two roundings.
    const float* in = _in->DeviceIn();
    const float* a = _add->DeviceIn();
    float* o = _out->DeviceOut();
    if (!freeml_hip::Check(fmlh_scale_scalar(o, in, _scale, _out->GetElementCount()), "ScaleAdd")) return;
    freeml_hip::Check(fmlh_add(o, o, a, _out->GetElementCount()), "ScaleAdd");
}

// Softmax (MatrixBase_Functions.h:49-80): rows of the (x, y) plane.
template <class T>
void Softmax(MatrixHIP<T>* _out, MatrixHIP<T>* _in) {
    if (!freeml_hip::Require(_out->GetDimsX() == _in->GetDimsX() && _out->GetDimsY() == _in->GetDimsY(),
                             "Softmax: dims differ"))
        return;
    const float* in = _in->DeviceIn();
    freeml_hip::Check(fmlh_softmax(_out->DeviceOut(), in, _in->GetDimsY(), _in->GetDimsX()), "Softmax");
}

// LayerNormOp (MatrixBase_Functions.h:481-549).
template <class T>
void LayerNormOp(MatrixHIP<T>* _out, MatrixHIP<T>* _in, MatrixHIP<T>* _gamma,
                 MatrixHIP<T>* _beta = nullptr, MatrixHIP<T>* _xHat = nullptr,
                 T _eps = static_cast<T>(1e-5)) {
    if (!freeml_hip::Require(_out->GetDimsX() == _in->GetDimsX() && _out->GetDimsY() == _in->GetDimsY() &&
                                 _out->GetDimsZ() == _in->GetDimsZ() && _gamma->GetDimsX() == _in->GetDimsX(),
                             "LayerNormOp: dims differ"))
        return;
    const uint32_t cols = _in->GetDimsX();
    const uint32_t rows = _in->GetDimsY() * _in->GetDimsZ();
    const float* in = _in->DeviceIn();
    const float* g = _gamma->DeviceIn();
    const float* b = _beta ? _beta->DeviceIn() : nullptr;
    float* xh = _xHat ? _xHat->DeviceOut() : nullptr;
    freeml_hip::Check(fmlh_layernorm(_out->DeviceOut(), in, g, b, xh, rows, cols, _eps), "LayerNormOp");
}

// GeluMat (MatrixBase_Functions.h:988-1000), reached from Gelu::activateMat (Gelu.h:32-38).
template <class T>
void GeluMat(MatrixHIP<T>* _out, MatrixHIP<T>* _in) {
    if (!freeml_hip::Require(freeml_hip::Same(_out, _in), "GeluMat: element counts differ")) return;
    const float* in = _in->DeviceIn();
    freeml_hip::Check(fmlh_gelu(_out->DeviceOut(), in, _in->GetElementCount()), "GeluMat");
}

// Add (MatrixBase_Functions.h:470-479).
template <class T>
void Add(MatrixHIP<T>* _out, MatrixHIP<T>* _L, MatrixHIP<T>* _R) {
    const uint32_t n = _R->GetElementCount();
    if (!freeml_hip::Require(_L->GetElementCount() >= n && _out->GetElementCount() >= n, "Add: sizes"))
        return;
    const float* l = _L->DeviceIn();
    const float* r = _R->DeviceIn();
    freeml_hip::Check(fmlh_add(_out->DeviceOut(), l, r, n), "Add");
}

// Copy (MatrixBase_Functions.h:156-161).
template <class T>
void Copy(MatrixHIP<T>* _out, MatrixHIP<T>* _in) {
    if (!freeml_hip::Require(freeml_hip::Same(_out, _in), "Copy: element counts differ")) return;
    const float* in = _in->DeviceIn();
    freeml_hip::Check(fmlh_copy(_out->DeviceOut(), in, _in->GetElementCount()), "Copy");
}

// GatherRows (MatrixBase_Functions.h:202-242).
template <class T>
void GatherRows(MatrixHIP<T>* _out, MatrixHIP<T>* _src, MatrixHIP<T>* _indices) {
    const uint32_t width = _src->GetDimsX();
    if (!freeml_hip::Require(_indices->GetDimsX() == 1u && _out->GetDimsX() == width &&
                                 _indices->GetDimsY() == _out->GetDimsY() &&
                                 _indices->GetDimsZ() == _out->GetDimsZ(),
                             "GatherRows: dims"))
        return;
    const float* s = _src->DeviceIn();
    const float* idx = _indices->DeviceIn();
    freeml_hip::Check(fmlh_gather_rows(_out->DeviceOut(), s, idx, width, _out->GetDimsY(), _out->GetDimsZ(),
                                       _src->GetDimsY(), _src->GetDimsZ()),
                      "GatherRows");
}

// BroadcastAdd (MatrixBase_Functions.h:716-730): the Dense bias.
template <class T>
void BroadcastAdd(MatrixHIP<T>* _out, MatrixHIP<T>* _L, MatrixHIP<T>* _R) {
    if (!freeml_hip::Require(_L->GetDimsZ() == 1 && _R->GetDimsZ() == 1, "BroadcastAdd: batched")) return;
    const float* l = _L->DeviceIn();
    const float* r = _R->DeviceIn();
    freeml_hip::Check(fmlh_broadcast_add(_out->DeviceOut(), l, r, _L->GetElementCount(), _L->GetDimsX()),
                      "BroadcastAdd");
}

// Fill(out, float) (MatrixBase_Functions.h:1078-1085).
template <class T>
void Fill(MatrixHIP<T>* _out, float _val) {
    freeml_hip::Check(fmlh_fill(_out->DeviceOut(), _val, _out->GetElementCount()), "Fill");
}

// Fill(out, Mat* val) (MatrixBase_Functions.h:1087-1095).
template <class T>
void Fill(MatrixHIP<T>* _out, MatrixHIP<T>* _val) {
    const float* v = _val->DeviceIn();
    freeml_hip::Check(fmlh_fill_from(_out->DeviceOut(), v, _out->GetElementCount()), "Fill");
}

// Clear (MatrixBase_Functions.h:1072-1076).
template <class T>
void Clear(MatrixHIP<T>* _out) {
    freeml_hip::Check(fmlh_fill(_out->DeviceOut(), 0.0f, _out->GetElementCount()), "Clear");
}

// PerElementMul (MatrixBase_Functions.h:847-854).
template <class T>
void PerElementMul(MatrixHIP<T>* _out, MatrixHIP<T>* _L, MatrixHIP<T>* _R) {
    const uint32_t n = _R->GetElementCount();
    const float* l = _L->DeviceIn();
    const float* r = _R->DeviceIn();
    freeml_hip::Check(fmlh_per_element_mul(_out->DeviceOut(), l, r, n), "PerElementMul");
}

// Scale(out, in, Mat* val) (MatrixBase_Functions.h:1020-1029).
template <class T>
void Scale(MatrixHIP<T>* _out, MatrixHIP<T>* _in, MatrixHIP<T>* _val) {
    const float* in = _in->DeviceIn();
    const float* v = _val->DeviceIn();
    freeml_hip::Check(fmlh_scale(_out->DeviceOut(), in, v, _in->GetElementCount()), "Scale");
}

// Scale(out, in, float) (MatrixBase_Functions.h:1031-1038).
template <class T>
void Scale(MatrixHIP<T>* _out, MatrixHIP<T>* _in, float _val) {
    const float* in = _in->DeviceIn();
    freeml_hip::Check(fmlh_scale_scalar(_out->DeviceOut(), in, _val, _in->GetElementCount()), "Scale");
}
#include <MatrixLibrary/GPU/HIP/MatrixHIP_Training.h>
#include <MatrixLibrary/GPU/HIP/MatrixHIP_Attention.h>
