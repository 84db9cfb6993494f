#pragma once
// MatrixHIP<float>: FreeML matrix backend whose storage lives in MI355X device memory.
//
// It derives from the reference's MatrixBase<T> (MatrixLibrary/MatrixBase.h:33-160) so that
// Model<float, MatrixHIP<float>>, Datablob, MatrixManager and every Layer instantiate on it
// unchanged (the static_assert at LayerLibrary/Layer.h:40-41).  All device work goes through
// the C ABI in freeml_hip.h; this header contains no HIP code.
//
// Storage and views.  AllocateMemory creates a Storage (device buffer + lazily allocated host
// mirror).  A matrix either owns a Storage or views one at an element offset:
// SetData(src.GetData(), src.GetOffset() + k) makes a view k elements further on, which is
// how CausalSelfAttentionLayer.h:430-440/:477-487, AddLayer.h:155-162 and Model::Run's input
// skeleton (Model.h:773-777) address sub-matrices -- the same contract as MatrixCPU (raw
// pointer, MatrixCPU.h:56-64) and MatrixDX11 (buffer handle + offset, MatrixDX11.h:114-139).
// Views own nothing; only the allocating matrix frees, in FreeMemory (MatrixManager.h:462-486
// calls it once, and never for skeletons).
//
// Coherence.  Each Storage records which copy is current: device, host, or both.
// DataRead/DataWrite (the host-pointer accessors generic FreeML code uses, e.g. init-time
// fills and the NanoLLM argmax) copy device -> host when the host copy is stale, and
// DataWrite marks the device copy stale.  Every op overload first makes its inputs current on
// the device (uploading host edits) and marks its outputs device-current.  This is the role
// of MatrixDX11's Map/Unmap staging (MatrixDX11.h:190-259).  On the forward path every matrix
// stays device-current, so no copy happens between ops.
#include <MatrixLibrary/MatrixBase.h>
#include <ToolsLibrary/Logger.h>

#include <freeml_hip.h>

#include <cassert>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

namespace freeml_hip {

// Reports a failed C-ABI call in the reference's style (log + assert) and returns false.  The
// message also goes to stderr, which stays visible when a program turns the logger's console
// output off.
inline bool Check(int rc, const char* what) {
    if (rc == FMLH_OK) return true;
    LOG_ERROR() << "freeml_hip: " << what << " failed (" << rc << "): " << fmlh_last_error();
    std::fprintf(stderr, "freeml_hip: %s failed (%d): %s\n", what, rc, fmlh_last_error());
    assert(rc == FMLH_OK);
    return false;
}

// Counts device<->host transfers so tests can assert that a forward pass made none.
struct TransferStats {
    uint64_t toHost = 0;
    uint64_t toDevice = 0;
};
inline TransferStats& Stats() {
    static TransferStats s;
    return s;
}

struct Storage {
    enum State : int { kBoth = 0, kDevice = 1, kHost = 2 };
    float* dev = nullptr;
    float* host = nullptr;
    size_t count = 0;
    State state = kDevice;

    ~Storage() { Release(); }

    bool Allocate(size_t n) {
        count = n;
        void* p = nullptr;
        if (!Check(fmlh_malloc(&p, n * sizeof(float)), "fmlh_malloc")) return false;
        dev = static_cast<float*>(p);
        state = kDevice;
        return true;
    }

    void Release() {
        if (dev) Check(fmlh_free(dev), "fmlh_free");
        std::free(host);
        dev = nullptr;
        host = nullptr;
        count = 0;
    }

    float* HostCurrent() {
        if (!host) {
            host = static_cast<float*>(std::aligned_alloc(64, ((count * sizeof(float) + 63) / 64) * 64));
            if (state == kHost) state = kDevice;  // nothing was ever written on the host
        }
        if (state == kDevice) {
            Check(fmlh_memcpy_d2h(host, dev, count * sizeof(float)), "fmlh_memcpy_d2h");
            ++Stats().toHost;
            state = kBoth;
        }
        return host;
    }

    float* DeviceCurrent() {
        if (state == kHost) {
            Check(fmlh_memcpy_h2d(dev, host, count * sizeof(float)), "fmlh_memcpy_h2d");
            ++Stats().toDevice;
            state = kBoth;
        }
        return dev;
    }
};

}  // namespace freeml_hip

template <class T>
class MatrixHIP : public MatrixBase<T> {
    static_assert(std::is_same_v<T, float>, "MatrixHIP implements the fp32 path only");

public:
    MatrixHIP(void* _data = nullptr) {
        MatrixBase<T>::m_hardwareName = "HIP";
        SetData(_data);
    }

    // MatrixManager constructs with null data (MatrixManager.h:200, :270).  Non-null data is
    // taken as a Storage of another MatrixHIP (what GetData() returns).
    MatrixHIP(T* _data, Dims3D _dims, std::string _name = "NoName") : MatrixHIP(static_cast<void*>(_data)) {
        MatrixBase<T>::m_name = _name;
        MatrixBase<T>::m_dims = _dims;
    }

    ~MatrixHIP() override = default;  // views never free; the owner frees in FreeMemory

    MatrixHIP(const MatrixHIP&) = delete;
    MatrixHIP& operator=(const MatrixHIP&) = delete;

    bool AllocateMemory(uint32_t _elementCount) override {
        auto* s = new freeml_hip::Storage();
        if (!s->Allocate(_elementCount)) {
            delete s;
            return false;
        }
        m_storage = s;
        m_offset = 0;
        m_owner = true;
        return true;
    }

    void FreeMemory() override {
        if (m_owner && m_storage) delete m_storage;
        m_storage = nullptr;
        m_owner = false;
    }

    void SetData(void* _ptr, uint32_t _offset = 0u) override {
        if (m_owner && m_storage && m_storage != _ptr) {
            LOG_WARNING() << "MatrixHIP::SetData on an owning matrix (" << MatrixBase<T>::m_name
                          << ") drops its storage reference";
        }
        m_storage = static_cast<freeml_hip::Storage*>(_ptr);
        m_offset = _offset;
        m_owner = false;
    }

    void* GetData() override { return m_storage; }
    uint32_t GetOffset() override { return m_offset; }

    void GetSliceZ(MatrixBase<T>* _matrixOut, uint32_t _zIndex) override {
        auto* out = static_cast<MatrixHIP<T>*>(_matrixOut);
        out->SetData(m_storage, m_offset + this->GetDimsX() * this->GetDimsY() * _zIndex);
        out->SetDims({this->GetDimsX(), this->GetDimsY(), 1});
    }

    // ---- host access (MatrixBase virtuals) -----------------------------------------------
    T* DataWrite() override {
        if (!m_storage) return nullptr;
        float* h = m_storage->HostCurrent();
        m_storage->state = freeml_hip::Storage::kHost;
        return h + m_offset;
    }

    const T* DataRead() override {
        if (!m_storage) return nullptr;
        return m_storage->HostCurrent() + m_offset;
    }

    T GetValue(uint32_t _x, uint32_t _y) override {
        assert(_x < this->GetDimsX() && _y < this->GetDimsY());
        return DataRead()[_y * this->GetDimsX() + _x];
    }

    T GetValue(uint32_t _x, uint32_t _y, uint32_t _z) override {
        assert(_x < this->GetDimsX() && _y < this->GetDimsY() && _z < this->GetDimsZ());
        return DataRead()[this->GetDimsX() * this->GetDimsY() * _z + _y * this->GetDimsX() + _x];
    }

    void SetValue(uint32_t _x, uint32_t _y, T _val) override {
        assert(_x < this->GetDimsX() && _y < this->GetDimsY());
        DataWrite()[_y * this->GetDimsX() + _x] = _val;
    }

    void SetValue(uint32_t _x, uint32_t _y, uint32_t _z, T _val) override {
        assert(_x < this->GetDimsX() && _y < this->GetDimsY() && _z < this->GetDimsZ());
        DataWrite()[this->GetDimsX() * this->GetDimsY() * _z + _y * this->GetDimsX() + _x] = _val;
    }

    std::vector<T> GetRow(uint32_t _r) override {
        const T* start = DataRead() + _r * this->GetDimsX();
        return std::vector<T>(start, start + this->GetDimsX());
    }

    std::vector<T> GetColumn(uint32_t _c) override {
        std::vector<T> col;
        col.reserve(this->GetDimsY());
        const T* d = DataRead();
        for (uint32_t y = 0; y < this->GetDimsY(); ++y) col.push_back(d[y * this->GetDimsX() + _c]);
        return col;
    }

    uint32_t GetElementCount() const override {
        return this->GetDimsX() * this->GetDimsY() * this->GetDimsZ();
    }

    void GetRawData(std::vector<char>& _out) override {
        const uint32_t count = GetElementCount();
        if (count == 0u || !m_storage) {
            _out.clear();
            return;
        }
        _out.resize(static_cast<size_t>(count) * sizeof(T));
        std::memcpy(_out.data(), DataRead(), _out.size());
    }

    // ---- device access (used by the op overloads) ----------------------------------------
    // Input operand: device copy made current (host edits uploaded).
    const float* DeviceIn() { return m_storage ? m_storage->DeviceCurrent() + m_offset : nullptr; }
    // Output operand: device copy current first (a view may write only part of the storage),
    // then the host copy is marked stale.
    float* DeviceOut() {
        if (!m_storage) return nullptr;
        float* d = m_storage->DeviceCurrent() + m_offset;
        m_storage->state = freeml_hip::Storage::kDevice;
        return d;
    }

    freeml_hip::Storage* GetStorage() { return m_storage; }
    bool IsOwner() const { return m_owner; }

private:
    freeml_hip::Storage* m_storage = nullptr;
    uint32_t m_offset = 0;
    bool m_owner = false;
};
