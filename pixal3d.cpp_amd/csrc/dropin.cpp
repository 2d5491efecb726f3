// The reference's sparse CPU API (include/pixal3d/sparse.h and
// include/pixal3d/sparse_transformer.h of Pixal3D.cpp) implemented on the
// MI355X through the pxs C ABI.
//
// Each call keeps the reference contract: host std::vector tensors in and
// out, `false` plus a message in *error on failure, the reference's argument
// checks in the reference's order with its error strings, and alias safety
// (output may be the same object as an input).  Inputs are copied to HBM
// once, validated there (SparseTensorF32::valid runs as a voxel-hash build
// plus one validation kernel instead of a host unordered_map), computed by
// the HIP kernels in fp32, and the result copied back.
//
// Device memory: each host thread owns one HIP stream and a set of
// grow-only device buffers that later calls on that thread reuse; nothing is
// shared between threads, so calls are reentrant like the reference's.

#include "pixal3d/flow_sampler.h"
#include "pixal3d/sparse.h"
#include "pixal3d/sparse_transformer.h"
#include "pxs.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <limits>
#include <sstream>
#include <string>
#include <vector>

namespace pixal3d {
namespace {

void set_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

// ---- per-thread device state ----------------------------------------------

enum Slot {
    kInCoords, kInFeats, kTable, kStatus, kNbr, kMasks, kWeight, kBias, kOut, kOutCoords,
    kWork, kAuxCoords, kAuxFeats, kAux2Feats, kCuQ, kCuK, kOffsets, kRows, kGamma, kBeta,
    kCount, kFlowState, kFlowPos, kFlowNeg, kFlowPred, kFlowX0, kFlowCu, kFlowWork,
    kTraceStats, kTraceWork, kSlotCount
};

class Device {
public:
    ~Device() {
        for (auto & b : buffers_) {
            if (b.ptr) (void)hipFree(b.ptr);
        }
        if (stream_) (void)hipStreamDestroy(stream_);
    }

    bool ready(std::string * error) {
        if (stream_) return true;
        // Default-priority stream, non-blocking with respect to the null stream.
        const hipError_t e = hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking);
        if (e != hipSuccess) {
            stream_ = nullptr;
            set_error(error, std::string("HIP stream creation failed: ") + hipGetErrorString(e));
            return false;
        }
        return true;
    }

    hipStream_t stream() const { return stream_; }

    // Device buffer `slot` with at least `bytes` bytes (grow-only).
    void * buffer(std::size_t slot, std::size_t bytes, std::string * error) {
        if (slot >= buffers_.size()) buffers_.resize(slot + 1);
        Buf & b = buffers_[slot];
        const std::size_t want = bytes == 0 ? 256 : (bytes + 255) / 256 * 256;
        if (b.bytes < want) {
            if (b.ptr) {
                (void)hipStreamSynchronize(stream_);
                (void)hipFree(b.ptr);
                b.ptr = nullptr;
                b.bytes = 0;
            }
            const hipError_t e = hipMalloc(&b.ptr, want);
            if (e != hipSuccess) {
                b.ptr = nullptr;
                set_error(error, std::string("device allocation failed: ") + hipGetErrorString(e));
                return nullptr;
            }
            b.bytes = want;
        }
        return b.ptr;
    }

private:
    struct Buf {
        void * ptr = nullptr;
        std::size_t bytes = 0;
    };
    hipStream_t stream_ = nullptr;
    std::vector<Buf> buffers_;
};

Device & device() {
    thread_local Device d;
    return d;
}

bool pxs_ok(int rc, std::string * error) {
    if (rc == PXS_OK) return true;
    set_error(error, std::string("MI355X sparse kernel failed: ") + pxs_last_error());
    return false;
}

bool hip_ok(hipError_t e, const char * what, std::string * error) {
    if (e == hipSuccess) return true;
    set_error(error, std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

template <typename T>
T * upload(std::size_t slot, const T * host, std::size_t count, std::string * error) {
    Device & d = device();
    void * p = d.buffer(slot, count * sizeof(T), error);
    if (!p) return nullptr;
    if (count > 0 &&
        !hip_ok(hipMemcpyAsync(p, host, count * sizeof(T), hipMemcpyHostToDevice, d.stream()),
                "host to device copy", error)) {
        return nullptr;
    }
    return static_cast<T *>(p);
}

template <typename T>
T * scratch(std::size_t slot, std::size_t count, std::string * error) {
    return static_cast<T *>(device().buffer(slot, count * sizeof(T), error));
}

template <typename T>
bool download(T * host, const T * dev, std::size_t count, std::string * error) {
    Device & d = device();
    if (count > 0 &&
        !hip_ok(hipMemcpyAsync(host, dev, count * sizeof(T), hipMemcpyDeviceToHost, d.stream()),
                "device to host copy", error)) {
        return false;
    }
    return hip_ok(hipStreamSynchronize(d.stream()), "stream synchronize", error);
}

// ---- validation ---------------------------------------------------------------

bool checked_product(std::size_t a, std::size_t b, std::size_t & result) {
    if (b != 0 && a > std::numeric_limits<std::size_t>::max() / b) return false;
    result = a * b;
    return true;
}

struct DevSparse {
    const int32_t * coords = nullptr;
    const float * feats = nullptr;
    int64_t n = 0;
};

// SparseTensorF32::valid (src/sparse.cpp:241-335): the cheap shape checks on
// the host in the reference's order, then the per-row checks (range,
// duplicate, batch contiguity, finiteness; first failing row wins) on the
// device over the uploaded copy.
bool upload_valid_sparse(const SparseTensorF32 & t, std::size_t coord_slot, std::size_t feat_slot,
                         DevSparse & out, std::string * error) {
    if (t.batch_size <= 0 || t.channels <= 0 || t.spatial_x <= 0 || t.spatial_y <= 0 ||
        t.spatial_z <= 0) {
        set_error(error, "invalid sparse tensor shape");
        return false;
    }
    if (t.coords.size() % 4 != 0) {
        set_error(error, "sparse coordinates must have four columns");
        return false;
    }
    std::size_t expected = 0;
    if (!checked_product(t.points(), static_cast<std::size_t>(t.channels), expected) ||
        t.feats.size() != expected) {
        set_error(error, "sparse feature count does not match coordinates");
        return false;
    }
    if (t.batch_size > PXS_MAX_EXTENT || t.spatial_x > PXS_MAX_EXTENT ||
        t.spatial_y > PXS_MAX_EXTENT || t.spatial_z > PXS_MAX_EXTENT) {
        set_error(error, "sparse tensor shape exceeds the device voxel key range (32768)");
        return false;
    }
    if (t.points() > static_cast<std::size_t>(INT_MAX)) {
        set_error(error, "sparse tensor has more than 2^31 - 1 points");
        return false;
    }
    Device & d = device();
    if (!d.ready(error)) return false;
    const int64_t n = static_cast<int64_t>(t.points());
    out.n = n;
    out.coords = upload(coord_slot, t.coords.data(), t.coords.size(), error);
    if (!out.coords) return false;
    out.feats = upload(feat_slot, t.feats.data(), t.feats.size(), error);
    if (!out.feats) return false;
    if (n == 0) return true;
    void * table = device().buffer(kTable, pxs_voxel_hash_bytes(n), error);
    int64_t * status = scratch<int64_t>(kStatus, 1, error);
    if (!table || !status) return false;
    if (!pxs_ok(pxs_voxel_hash_build(out.coords, n, table, d.stream()), error)) return false;
    if (!pxs_ok(pxs_sparse_validate(out.coords, n, t.batch_size, t.spatial_x, t.spatial_y,
                                    t.spatial_z, PXS_F32, out.feats, t.channels, table, status,
                                    d.stream()),
                error)) {
        return false;
    }
    int64_t host_status = 0;
    if (!download(&host_status, status, 1, error)) return false;
    if (host_status != std::numeric_limits<int64_t>::max()) {
        set_error(error, pxs_validation_message(static_cast<int>(host_status & 7)));
        return false;
    }
    return true;
}

struct DevVarLen {
    const float * feats = nullptr;
    int64_t tokens = 0;
};

// VarLenTensorF32::valid (src/sparse.cpp:214-239).
bool upload_valid_varlen(const VarLenTensorF32 & t, std::size_t feat_slot, DevVarLen & out,
                         std::string * error) {
    if (t.batch_size <= 0 || t.channels <= 0 ||
        t.offsets.size() != static_cast<std::size_t>(t.batch_size + 1) || t.offsets.front() != 0) {
        set_error(error, "invalid variable-length tensor shape");
        return false;
    }
    for (std::size_t i = 1; i < t.offsets.size(); ++i) {
        if (t.offsets[i] < t.offsets[i - 1]) {
            set_error(error, "variable-length tensor offsets are not monotonic");
            return false;
        }
    }
    std::size_t expected = 0;
    if (!checked_product(t.offsets.back(), static_cast<std::size_t>(t.channels), expected) ||
        expected != t.feats.size()) {
        set_error(error, "variable-length tensor feature count does not match offsets");
        return false;
    }
    Device & d = device();
    if (!d.ready(error)) return false;
    out.tokens = static_cast<int64_t>(t.offsets.back());
    out.feats = upload(feat_slot, t.feats.data(), t.feats.size(), error);
    if (!out.feats) return false;
    if (out.tokens == 0) return true;
    int64_t * status = scratch<int64_t>(kStatus, 1, error);
    if (!status) return false;
    if (!pxs_ok(pxs_status_reset(status, d.stream()), error) ||
        !pxs_ok(pxs_check_finite(PXS_F32, out.feats, out.tokens, t.channels, t.channels, status,
                                 d.stream()),
                error)) {
        return false;
    }
    int64_t host_status = 0;
    if (!download(&host_status, status, 1, error)) return false;
    if (host_status != std::numeric_limits<int64_t>::max()) {
        set_error(error, "variable-length tensor contains a non-finite value");
        return false;
    }
    return true;
}

bool check_output_channels(int channels, std::string * error) {
    if (channels <= 0) {
        set_error(error, "sparse output channel count must be positive");
        return false;
    }
    return true;
}

void copy_shape(const SparseTensorF32 & input, int channels, SparseTensorF32 & output) {
    output.batch_size = input.batch_size;
    output.channels = channels;
    output.spatial_x = input.spatial_x;
    output.spatial_y = input.spatial_y;
    output.spatial_z = input.spatial_z;
    output.coords = input.coords;
}

// Per-batch row bounds of a tensor contiguous by batch, as cu_seqlens.
std::vector<int64_t> batch_bounds(const SparseTensorF32 & t) {
    std::vector<int64_t> cu(static_cast<std::size_t>(t.batch_size) + 1, 0);
    const std::size_t n = t.points();
    std::size_t p = 0;
    for (int b = 0; b < t.batch_size; ++b) {
        while (p < n && t.coords[p * 4] < b) ++p;
        cu[static_cast<std::size_t>(b)] = static_cast<int64_t>(p);
        while (p < n && t.coords[p * 4] == b) ++p;
        cu[static_cast<std::size_t>(b) + 1] = static_cast<int64_t>(p);
    }
    return cu;
}

std::vector<int64_t> to_i64(const std::vector<std::size_t> & v) {
    return std::vector<int64_t>(v.begin(), v.end());
}

// Row-wise GEMM shared by sparse_linear and varlen_linear.
bool device_linear(const float * x, int64_t rows, int cin, const float * weight,
                   const float * bias, int cout, std::vector<float> & result,
                   std::string * error) {
    Device & d = device();
    const float * w = upload(kWeight, weight, static_cast<std::size_t>(cout) * cin, error);
    const float * b = w ? upload(kBias, bias, static_cast<std::size_t>(cout), error) : nullptr;
    float * y = b ? scratch<float>(kOut, static_cast<std::size_t>(rows) * cout, error) : nullptr;
    if (!y) return false;
    if (!pxs_ok(pxs_linear(PXS_F32, x, rows, cin, w, b, cout, PXS_ACT_NONE, y, d.stream()), error)) {
        return false;
    }
    result.resize(static_cast<std::size_t>(rows) * cout);
    return download(result.data(), y, result.size(), error);
}

} // namespace

// ---- tensor validation ----------------------------------------------------------

bool VarLenTensorF32::valid(std::string * error) const {
    DevVarLen d;
    return upload_valid_varlen(*this, kInFeats, d, error);
}

bool SparseTensorF32::valid(std::string * error) const {
    DevSparse d;
    return upload_valid_sparse(*this, kInCoords, kInFeats, d, error);
}

// ---- a6: linear ------------------------------------------------------------------

// src/sparse.cpp:337-451
bool sparse_linear(const SparseTensorF32 & input, const float * weight, const float * bias,
                   int out_channels, SparseTensorF32 & output, std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (!check_output_channels(out_channels, error)) return false;
    if (!weight) {
        set_error(error, "sparse weight pointer is null");
        return false;
    }
    if (!bias) {
        set_error(error, "sparse bias pointer is null");
        return false;
    }
    std::size_t count = 0;
    if (!checked_product(input.points(), static_cast<std::size_t>(out_channels), count)) {
        set_error(error, "sparse linear output size overflows size_t");
        return false;
    }
    SparseTensorF32 result;
    copy_shape(input, out_channels, result);
    if (!device_linear(in.feats, in.n, input.channels, weight, bias, out_channels, result.feats,
                       error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// src/sparse.cpp:453-488
bool varlen_linear(const VarLenTensorF32 & input, const float * weight, const float * bias,
                   int out_channels, VarLenTensorF32 & output, std::string * error) {
    DevVarLen in;
    if (!upload_valid_varlen(input, kInFeats, in, error) ||
        !check_output_channels(out_channels, error)) {
        return false;
    }
    if (!weight || !bias) {
        set_error(error, "variable-length linear weight or bias pointer is null");
        return false;
    }
    std::size_t count = 0;
    if (!checked_product(input.tokens(), static_cast<std::size_t>(out_channels), count)) {
        set_error(error, "variable-length linear output size overflows size_t");
        return false;
    }
    VarLenTensorF32 result;
    result.batch_size = input.batch_size;
    result.channels = out_channels;
    result.offsets = input.offsets;
    if (!device_linear(in.feats, in.tokens, input.channels, weight, bias, out_channels,
                       result.feats, error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// ---- a12: layer norm ---------------------------------------------------------------

// src/sparse.cpp:490-534
bool sparse_layer_norm(const SparseTensorF32 & input, float epsilon, const float * gamma,
                       const float * beta, SparseTensorF32 & output, std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (!(epsilon > 0.0f) || !std::isfinite(epsilon)) {
        set_error(error, "sparse layer norm epsilon must be finite and positive");
        return false;
    }
    if ((gamma == nullptr) != (beta == nullptr)) {
        set_error(error, "sparse layer norm affine parameters must be both null or non-null");
        return false;
    }
    Device & d = device();
    const std::size_t C = static_cast<std::size_t>(input.channels);
    const float * g = gamma ? upload(kGamma, gamma, C, error) : nullptr;
    const float * b = beta ? upload(kBeta, beta, C, error) : nullptr;
    if ((gamma && !g) || (beta && !b)) return false;
    float * y = scratch<float>(kOut, input.feats.size(), error);
    if (!y) return false;
    if (!pxs_ok(pxs_layer_norm(PXS_F32, in.feats, in.n, input.channels, epsilon, g, b, PXS_F32, y,
                               d.stream()),
                error)) {
        return false;
    }
    SparseTensorF32 result;
    copy_shape(input, input.channels, result);
    result.feats.resize(input.feats.size());
    if (!download(result.feats.data(), y, result.feats.size(), error)) return false;
    output = std::move(result);
    return true;
}

// ---- a15: mean downsample ------------------------------------------------------------

// src/sparse.cpp:536-602
bool sparse_downsample_mean(const SparseTensorF32 & input, int factor, SparseTensorF32 & output,
                            std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (factor <= 0) {
        set_error(error, "sparse downsample factor must be positive");
        return false;
    }
    Device & d = device();
    const int64_t n = in.n;
    const std::size_t rows = static_cast<std::size_t>(std::max<int64_t>(n, 1));
    void * ws = device().buffer(kWork, pxs_downsample_workspace_bytes(n, input.batch_size,
                                                                      input.spatial_x,
                                                                      input.spatial_y,
                                                                      input.spatial_z, factor),
                                error);
    int32_t * oc = scratch<int32_t>(kOutCoords, rows * 4, error);
    int64_t * off = scratch<int64_t>(kOffsets, rows + 1, error);
    int32_t * grows = scratch<int32_t>(kRows, rows, error);
    int64_t * m_dev = scratch<int64_t>(kCount, 1, error);
    if (!ws || !oc || !off || !grows || !m_dev) return false;
    if (!pxs_ok(pxs_downsample_topology(in.coords, n, input.batch_size, input.spatial_x,
                                        input.spatial_y, input.spatial_z, factor, oc, off, grows,
                                        m_dev, ws, d.stream()),
                error)) {
        return false;
    }
    int64_t m = 0;
    if (!download(&m, m_dev, 1, error)) return false;
    float * y = scratch<float>(kOut, static_cast<std::size_t>(std::max<int64_t>(m, 1)) *
                                         input.channels, error);
    if (!y) return false;
    if (!pxs_ok(pxs_downsample_mean(PXS_F32, in.feats, input.channels, off, grows, m, y,
                                    d.stream()),
                error)) {
        return false;
    }
    SparseTensorF32 result;
    result.batch_size = input.batch_size;
    result.channels = input.channels;
    result.spatial_x = (input.spatial_x + factor - 1) / factor;
    result.spatial_y = (input.spatial_y + factor - 1) / factor;
    result.spatial_z = (input.spatial_z + factor - 1) / factor;
    result.coords.resize(static_cast<std::size_t>(m) * 4);
    result.feats.resize(static_cast<std::size_t>(m) * input.channels);
    if (!download(result.coords.data(), oc, result.coords.size(), error) ||
        !download(result.feats.data(), y, result.feats.size(), error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// ---- a5: channel to spatial ------------------------------------------------------------

// src/sparse.cpp:604-702
bool sparse_channel_to_spatial(const SparseTensorF32 & input, int factor,
                               const SparseTensorF32 * subdivision, SparseTensorF32 & output,
                               std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (factor <= 0) {
        set_error(error, "sparse channel-to-spatial factor must be positive");
        return false;
    }
    std::size_t child_count = 1;
    for (int axis = 0; axis < 3; ++axis) {
        if (child_count > std::numeric_limits<std::size_t>::max() / static_cast<std::size_t>(factor)) {
            set_error(error, "sparse channel-to-spatial factor overflows size_t");
            return false;
        }
        child_count *= static_cast<std::size_t>(factor);
    }
    if (input.channels <= 0 || child_count > static_cast<std::size_t>(INT_MAX) ||
        input.channels % static_cast<int>(child_count) != 0) {
        set_error(error, "sparse channel-to-spatial channels are not divisible by factor^3");
        return false;
    }
    const float * sub = nullptr;
    if (subdivision) {
        DevSparse sd;
        std::string ignored;
        if (!upload_valid_sparse(*subdivision, kAuxCoords, kAuxFeats, sd, &ignored) ||
            subdivision->batch_size != input.batch_size ||
            subdivision->channels != static_cast<int>(child_count) ||
            subdivision->coords != input.coords) {
            set_error(error, "sparse subdivision shape or coordinates do not match input");
            return false;
        }
        sub = sd.feats;
    }
    const long long f = factor;
    if (static_cast<long long>(input.spatial_x) * f > std::numeric_limits<int>::max() ||
        static_cast<long long>(input.spatial_y) * f > std::numeric_limits<int>::max() ||
        static_cast<long long>(input.spatial_z) * f > std::numeric_limits<int>::max()) {
        set_error(error, "sparse channel-to-spatial output shape overflows int");
        return false;
    }
    if (!subdivision &&
        input.points() > std::numeric_limits<std::size_t>::max() / child_count) {
        set_error(error, "sparse channel-to-spatial output point count overflows size_t");
        return false;
    }
    const int c_out = input.channels / static_cast<int>(child_count);
    Device & d = device();
    const int64_t n = in.n;
    const std::size_t cap = static_cast<std::size_t>(std::max<int64_t>(n, 1)) * child_count;
    void * ws = device().buffer(kWork, pxs_channel_to_spatial_workspace_bytes(n, factor), error);
    int32_t * oc = scratch<int32_t>(kOutCoords, cap * 4, error);
    float * y = scratch<float>(kOut, cap * c_out, error);
    int64_t * m_dev = scratch<int64_t>(kCount, 1, error);
    if (!ws || !oc || !y || !m_dev) return false;
    if (!pxs_ok(pxs_channel_to_spatial(PXS_F32, in.coords, n, in.feats, input.channels, factor,
                                       sub, oc, y, m_dev, ws, d.stream()),
                error)) {
        return false;
    }
    int64_t m = 0;
    if (!download(&m, m_dev, 1, error)) return false;
    SparseTensorF32 result;
    result.batch_size = input.batch_size;
    result.channels = c_out;
    result.spatial_x = input.spatial_x * factor;
    result.spatial_y = input.spatial_y * factor;
    result.spatial_z = input.spatial_z * factor;
    result.coords.resize(static_cast<std::size_t>(m) * 4);
    result.feats.resize(static_cast<std::size_t>(m) * c_out);
    if (!download(result.coords.data(), oc, result.coords.size(), error) ||
        !download(result.feats.data(), y, result.feats.size(), error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// ---- a7, a9: attention -----------------------------------------------------------------

namespace {

bool device_attention(const float * q, int64_t q_rows, const float * k, const float * v,
                      int k_channels, int v_channels, const std::vector<int64_t> & cu_q,
                      const std::vector<int64_t> & cu_k, int heads, int head_dim, float scale,
                      std::vector<float> & result, std::string * error) {
    Device & d = device();
    const int nseg = static_cast<int>(cu_q.size()) - 1;
    const int64_t * dq = upload(kCuQ, cu_q.data(), cu_q.size(), error);
    const int64_t * dk = dq ? upload(kCuK, cu_k.data(), cu_k.size(), error) : nullptr;
    const int value_dim = v_channels / heads;
    float * o = dk ? scratch<float>(kOut, static_cast<std::size_t>(std::max<int64_t>(q_rows, 1)) *
                                              v_channels, error)
                   : nullptr;
    void * ws = o ? device().buffer(kWork, pxs_attention_workspace_bytes(nseg), error) : nullptr;
    if (!ws) return false;
    if (!pxs_ok(pxs_varlen_attention(PXS_F32, q, heads * head_dim, k, k_channels, v, v_channels,
                                     dq, dk, nseg, q_rows, nullptr, heads, head_dim, value_dim,
                                     scale, o, v_channels, ws, d.stream()),
                error)) {
        return false;
    }
    result.resize(static_cast<std::size_t>(q_rows) * v_channels);
    return download(result.data(), o, result.size(), error);
}

} // namespace

// src/sparse.cpp:704-783
bool sparse_scaled_dot_product_attention(const SparseTensorF32 & query,
                                         const SparseTensorF32 & key,
                                         const SparseTensorF32 & value, int num_heads,
                                         int head_dim, float scale, SparseTensorF32 & output,
                                         std::string * error) {
    DevSparse dq, dk, dv;
    if (!upload_valid_sparse(query, kInCoords, kInFeats, dq, error) ||
        !upload_valid_sparse(key, kAuxCoords, kAuxFeats, dk, error) ||
        !upload_valid_sparse(value, kOutCoords, kAux2Feats, dv, error)) {
        return false;
    }
    if (num_heads <= 0 || head_dim <= 0 || query.channels != num_heads * head_dim ||
        key.channels != num_heads * head_dim || value.channels <= 0 ||
        value.channels % num_heads != 0) {
        set_error(error, "sparse attention channel/head dimensions are invalid");
        return false;
    }
    if (query.batch_size != key.batch_size || query.batch_size != value.batch_size) {
        set_error(error, "sparse attention batch sizes do not match");
        return false;
    }
    if (!(scale > 0.0f) || !std::isfinite(scale)) {
        set_error(error, "sparse attention scale must be finite and positive");
        return false;
    }
    const std::vector<int64_t> cu_q = batch_bounds(query);
    const std::vector<int64_t> cu_k = batch_bounds(key);
    const std::vector<int64_t> cu_v = batch_bounds(value);
    for (int b = 0; b < query.batch_size; ++b) {
        const int64_t keys = cu_k[b + 1] - cu_k[b];
        if (keys == 0 || cu_v[b + 1] - cu_v[b] != keys) {
            set_error(error, "sparse attention has no keys or mismatched key/value rows");
            return false;
        }
    }
    SparseTensorF32 result;
    copy_shape(query, value.channels, result);
    if (!device_attention(dq.feats, dq.n, dk.feats, dv.feats, key.channels, value.channels, cu_q,
                          cu_k, num_heads, head_dim, scale, result.feats, error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// src/sparse.cpp:785-859
bool sparse_cross_attention(const SparseTensorF32 & query, const VarLenTensorF32 & key,
                            const VarLenTensorF32 & value, int num_heads, int head_dim,
                            float scale, SparseTensorF32 & output, std::string * error) {
    DevSparse dq;
    DevVarLen dk, dv;
    if (!upload_valid_sparse(query, kInCoords, kInFeats, dq, error) ||
        !upload_valid_varlen(key, kAuxFeats, dk, error) ||
        !upload_valid_varlen(value, kAux2Feats, dv, error)) {
        return false;
    }
    if (key.batch_size != value.batch_size || key.offsets != value.offsets || num_heads <= 0 ||
        head_dim <= 0 || query.channels != num_heads * head_dim ||
        key.channels != num_heads * head_dim || value.channels <= 0 ||
        value.channels % num_heads != 0) {
        set_error(error, "sparse cross-attention dimensions or offsets are invalid");
        return false;
    }
    if (query.batch_size != key.batch_size) {
        set_error(error, "sparse cross-attention batch sizes do not match");
        return false;
    }
    if (!(scale > 0.0f) || !std::isfinite(scale)) {
        set_error(error, "sparse cross-attention scale must be finite and positive");
        return false;
    }
    const std::vector<int64_t> cu_q = batch_bounds(query);
    const std::vector<int64_t> cu_k = to_i64(key.offsets);
    for (int b = 0; b < query.batch_size; ++b) {
        if (cu_k[b] == cu_k[b + 1]) {
            set_error(error, "sparse cross-attention has an empty key sequence");
            return false;
        }
    }
    SparseTensorF32 result;
    copy_shape(query, value.channels, result);
    if (!device_attention(dq.feats, dq.n, dk.feats, dv.feats, key.channels, value.channels, cu_q,
                          cu_k, num_heads, head_dim, scale, result.feats, error)) {
        return false;
    }
    output = std::move(result);
    return true;
}

// ---- a10, a11: RoPE and multi-head RMS norm ----------------------------------------------

// src/sparse.cpp:861-917
bool sparse_rotary_position_embedding(const SparseTensorF32 & input, int num_heads,
                                      int head_dim, float frequency_min, float frequency_base,
                                      SparseTensorF32 & output, std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (num_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 ||
        input.channels != num_heads * head_dim) {
        set_error(error, "sparse RoPE head dimensions are invalid");
        return false;
    }
    if (!(frequency_min > 0.0f) || !std::isfinite(frequency_min) || !(frequency_base > 0.0f) ||
        !std::isfinite(frequency_base)) {
        set_error(error, "sparse RoPE frequencies must be finite and positive");
        return false;
    }
    Device & d = device();
    float * y = scratch<float>(kOut, input.feats.size(), error);
    if (!y) return false;
    if (!pxs_ok(pxs_rope(PXS_F32, in.coords, in.feats, input.channels, in.n, num_heads, head_dim,
                         frequency_min, frequency_base, y, input.channels, d.stream()),
                error)) {
        return false;
    }
    SparseTensorF32 result;
    copy_shape(input, input.channels, result);
    result.feats.resize(input.feats.size());
    if (!download(result.feats.data(), y, result.feats.size(), error)) return false;
    output = std::move(result);
    return true;
}

// src/sparse.cpp:919-954
bool sparse_multihead_rms_norm(const SparseTensorF32 & input, int num_heads, int head_dim,
                               const float * gamma, SparseTensorF32 & output,
                               std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error)) return false;
    if (num_heads <= 0 || head_dim <= 0 || input.channels != num_heads * head_dim) {
        set_error(error, "sparse RMS norm head dimensions are invalid");
        return false;
    }
    if (!gamma) {
        set_error(error, "sparse RMS norm gamma pointer is null");
        return false;
    }
    Device & d = device();
    const float * g = upload(kGamma, gamma, static_cast<std::size_t>(input.channels), error);
    float * y = g ? scratch<float>(kOut, input.feats.size(), error) : nullptr;
    if (!y) return false;
    if (!pxs_ok(pxs_mh_rms_norm(PXS_F32, in.feats, input.channels, in.n, num_heads, head_dim, g, y,
                                input.channels, d.stream()),
                error)) {
        return false;
    }
    SparseTensorF32 result;
    copy_shape(input, input.channels, result);
    result.feats.resize(input.feats.size());
    if (!download(result.feats.data(), y, result.feats.size(), error)) return false;
    output = std::move(result);
    return true;
}

// src/sparse.cpp:956-997
bool varlen_multihead_rms_norm(const VarLenTensorF32 & input, int num_heads, int head_dim,
                               const float * gamma, VarLenTensorF32 & output,
                               std::string * error) {
    DevVarLen in;
    if (!upload_valid_varlen(input, kInFeats, in, error)) return false;
    if (num_heads <= 0 || head_dim <= 0 || input.channels != num_heads * head_dim) {
        set_error(error, "variable-length RMS norm head dimensions are invalid");
        return false;
    }
    if (!gamma) {
        set_error(error, "variable-length RMS norm gamma pointer is null");
        return false;
    }
    Device & d = device();
    const float * g = upload(kGamma, gamma, static_cast<std::size_t>(input.channels), error);
    float * y = g ? scratch<float>(kOut, input.feats.size(), error) : nullptr;
    if (!y) return false;
    if (!pxs_ok(pxs_mh_rms_norm(PXS_F32, in.feats, input.channels, in.tokens, num_heads, head_dim,
                                g, y, input.channels, d.stream()),
                error)) {
        return false;
    }
    VarLenTensorF32 result;
    result.batch_size = input.batch_size;
    result.channels = input.channels;
    result.offsets = input.offsets;
    result.feats.resize(input.feats.size());
    if (!download(result.feats.data(), y, result.feats.size(), error)) return false;
    output = std::move(result);
    return true;
}

// ---- a2, a3: submanifold convolution ------------------------------------------------------

// src/sparse.cpp:999-1055: neighbor map from the device voxel hash, then the
// output-stationary gather-GEMM (bias added after the offsets).
bool sparse_submanifold_conv3d(const SparseTensorF32 & input, const float * weight,
                               const float * bias, int out_channels, SparseTensorF32 & output,
                               std::string * error) {
    DevSparse in;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error) ||
        !check_output_channels(out_channels, error)) {
        return false;
    }
    if (!weight) {
        set_error(error, "sparse weight pointer is null");
        return false;
    }
    if (!bias) {
        set_error(error, "sparse bias pointer is null");
        return false;
    }
    std::size_t count = 0;
    if (!checked_product(input.points(), static_cast<std::size_t>(out_channels), count)) {
        set_error(error, "sparse convolution output size overflows size_t");
        return false;
    }
    Device & d = device();
    const int64_t n = in.n;
    SparseTensorF32 result;
    copy_shape(input, out_channels, result);
    result.feats.assign(count, 0.0f);
    if (n == 0) {
        output = std::move(result);
        return true;
    }
    // The validation call left the hash of these coordinates in kTable.
    void * table = device().buffer(kTable, pxs_voxel_hash_bytes(n), error);
    int32_t * nbr = scratch<int32_t>(kNbr, static_cast<std::size_t>(n) * 27, error);
    uint32_t * masks = scratch<uint32_t>(kMasks, static_cast<std::size_t>(n), error);
    const float * w = upload(kWeight, weight,
                             static_cast<std::size_t>(27) * out_channels * input.channels, error);
    const float * b = w ? upload(kBias, bias, static_cast<std::size_t>(out_channels), error) : nullptr;
    float * y = b ? scratch<float>(kOut, count, error) : nullptr;
    if (!table || !nbr || !masks || !y) return false;
    if (!pxs_ok(pxs_neighbor_map_k3(in.coords, n, table, nbr, masks, d.stream()), error) ||
        !pxs_ok(pxs_subm_conv3d(PXS_F32, in.feats, n, input.channels, w, b, out_channels, nbr,
                                masks, y, d.stream()),
                error)) {
        return false;
    }
    if (!download(result.feats.data(), y, count, error)) return false;
    output = std::move(result);
    return true;
}

// ---- a13: the transformer block -------------------------------------------------------------

namespace {

bool require_pointer(const float * p, const char * name, std::string * error) {
    if (p) return true;
    set_error(error, std::string("missing sparse transformer tensor: ") + name);
    return false;
}

bool same_coords(const SparseTensorF32 & a, const SparseTensorF32 & b) {
    return a.batch_size == b.batch_size && a.coords == b.coords;
}

// Block weight slots start after the primitive slots.
constexpr std::size_t kBlockSlot = kSlotCount;

} // namespace

// src/sparse_transformer.cpp:138-292, with every intermediate kept in HBM.
bool sparse_transformer_cross_block_f32(const SparseTensorF32 & input,
                                        const float * timestep_modulation,
                                        const VarLenTensorF32 & global_context,
                                        const SparseTensorF32 * projected_context,
                                        const SparseTransformerBlockConfig & config,
                                        const SparseTransformerBlockWeightsF32 & weights,
                                        SparseTensorF32 & output, std::string * error) {
    DevSparse in;
    DevVarLen ctx;
    if (!upload_valid_sparse(input, kInCoords, kInFeats, in, error) ||
        !upload_valid_varlen(global_context, kAuxFeats, ctx, error)) {
        return false;
    }
    if (!timestep_modulation || config.channels <= 0 || config.num_heads <= 0 ||
        config.mlp_hidden <= 0 || config.context_channels <= 0 ||
        config.channels % config.num_heads != 0 || input.channels != config.channels ||
        global_context.channels != config.context_channels ||
        global_context.batch_size != input.batch_size || !(config.norm_eps > 0.0f) ||
        !std::isfinite(config.norm_eps)) {
        set_error(error, "invalid sparse transformer block configuration");
        return false;
    }
    if (config.use_projection) {
        if (config.proj_in_channels <= 0 || !projected_context ||
            projected_context->channels != config.proj_in_channels ||
            !same_coords(input, *projected_context)) {
            set_error(error, "sparse transformer projection shape does not match query");
            return false;
        }
    }
    const SparseTransformerBlockWeightsF32 & w = weights;
    if (!require_pointer(w.modulation, "modulation", error) ||
        !require_pointer(w.self_to_qkv_weight, "self_attn.to_qkv.weight", error) ||
        !require_pointer(w.self_to_qkv_bias, "self_attn.to_qkv.bias", error) ||
        !require_pointer(w.self_to_out_weight, "self_attn.to_out.weight", error) ||
        !require_pointer(w.self_to_out_bias, "self_attn.to_out.bias", error) ||
        !require_pointer(w.norm2_weight, "norm2.weight", error) ||
        !require_pointer(w.norm2_bias, "norm2.bias", error) ||
        !require_pointer(w.cross_to_q_weight, "cross_attn.to_q.weight", error) ||
        !require_pointer(w.cross_to_q_bias, "cross_attn.to_q.bias", error) ||
        !require_pointer(w.cross_to_kv_weight, "cross_attn.to_kv.weight", error) ||
        !require_pointer(w.cross_to_kv_bias, "cross_attn.to_kv.bias", error) ||
        !require_pointer(w.cross_to_out_weight, "cross_attn.to_out.weight", error) ||
        !require_pointer(w.cross_to_out_bias, "cross_attn.to_out.bias", error) ||
        !require_pointer(w.mlp0_weight, "mlp.mlp.0.weight", error) ||
        !require_pointer(w.mlp0_bias, "mlp.mlp.0.bias", error) ||
        !require_pointer(w.mlp2_weight, "mlp.mlp.2.weight", error) ||
        !require_pointer(w.mlp2_bias, "mlp.mlp.2.bias", error)) {
        return false;
    }
    if (config.qk_rms_norm &&
        (!require_pointer(w.self_q_gamma, "self_attn.q_rms_norm.gamma", error) ||
         !require_pointer(w.self_k_gamma, "self_attn.k_rms_norm.gamma", error))) {
        return false;
    }
    if (config.qk_rms_norm_cross &&
        (!require_pointer(w.cross_q_gamma, "cross_attn.q_rms_norm.gamma", error) ||
         !require_pointer(w.cross_k_gamma, "cross_attn.k_rms_norm.gamma", error))) {
        return false;
    }
    if (config.use_projection &&
        (!require_pointer(w.proj_weight, "cross_attn.proj_linear.weight", error) ||
         !require_pointer(w.proj_bias, "cross_attn.proj_linear.bias", error))) {
        return false;
    }
    const int C = config.channels, H = config.num_heads;
    if (C / H > 64) {
        set_error(error, "sparse transformer head_dim above 64 is not supported on this device path");
        return false;
    }
    // The reference's attention calls reject batches without keys.
    const std::vector<int64_t> cu = batch_bounds(input);
    for (int b = 0; b < input.batch_size; ++b) {
        if (cu[b] == cu[b + 1]) {
            set_error(error, "sparse attention has no keys or mismatched key/value rows");
            return false;
        }
    }
    for (int b = 0; b < input.batch_size; ++b) {
        if (global_context.offsets[b] == global_context.offsets[b + 1]) {
            set_error(error, "sparse cross-attention has an empty key sequence");
            return false;
        }
    }
    DevSparse proj;
    if (config.use_projection &&
        !upload_valid_sparse(*projected_context, kAuxCoords, kAux2Feats, proj, error)) {
        return false;
    }

    Device & d = device();
    std::size_t slot = kBlockSlot;
    bool ok = true;
    auto put = [&](const float * host, std::size_t count) -> const float * {
        if (!ok || !host) return nullptr;
        const float * p = upload(slot++, host, count, error);
        if (!p) ok = false;
        return p;
    };
    const std::size_t Cs = static_cast<std::size_t>(C);
    const std::size_t M = static_cast<std::size_t>(config.mlp_hidden);
    const std::size_t X = static_cast<std::size_t>(config.context_channels);
    const std::size_t P = static_cast<std::size_t>(std::max(config.proj_in_channels, 0));
    pxs_block_weights dw{};
    dw.modulation = put(w.modulation, 6 * Cs);
    dw.self_to_qkv_weight = put(w.self_to_qkv_weight, 3 * Cs * Cs);
    dw.self_to_qkv_bias = put(w.self_to_qkv_bias, 3 * Cs);
    dw.self_q_gamma = config.qk_rms_norm ? put(w.self_q_gamma, Cs) : nullptr;
    dw.self_k_gamma = config.qk_rms_norm ? put(w.self_k_gamma, Cs) : nullptr;
    dw.self_to_out_weight = put(w.self_to_out_weight, Cs * Cs);
    dw.self_to_out_bias = put(w.self_to_out_bias, Cs);
    dw.norm2_weight = put(w.norm2_weight, Cs);
    dw.norm2_bias = put(w.norm2_bias, Cs);
    dw.cross_to_q_weight = put(w.cross_to_q_weight, Cs * Cs);
    dw.cross_to_q_bias = put(w.cross_to_q_bias, Cs);
    dw.cross_to_kv_weight = put(w.cross_to_kv_weight, 2 * Cs * X);
    dw.cross_to_kv_bias = put(w.cross_to_kv_bias, 2 * Cs);
    dw.cross_q_gamma = config.qk_rms_norm_cross ? put(w.cross_q_gamma, Cs) : nullptr;
    dw.cross_k_gamma = config.qk_rms_norm_cross ? put(w.cross_k_gamma, Cs) : nullptr;
    dw.cross_to_out_weight = put(w.cross_to_out_weight, Cs * Cs);
    dw.cross_to_out_bias = put(w.cross_to_out_bias, Cs);
    dw.proj_weight = config.use_projection ? put(w.proj_weight, Cs * P) : nullptr;
    dw.proj_bias = config.use_projection ? put(w.proj_bias, Cs) : nullptr;
    dw.mlp0_weight = put(w.mlp0_weight, M * Cs);
    dw.mlp0_bias = put(w.mlp0_bias, M);
    dw.mlp2_weight = put(w.mlp2_weight, Cs * M);
    dw.mlp2_bias = put(w.mlp2_bias, Cs);
    const float * tmod = put(timestep_modulation, static_cast<std::size_t>(input.batch_size) * 6 * Cs);
    if (!ok) return false;
    const int64_t * dcu = upload(slot++, cu.data(), cu.size(), error);
    const std::vector<int64_t> ctx_off = to_i64(global_context.offsets);
    const int64_t * dctx = dcu ? upload(slot++, ctx_off.data(), ctx_off.size(), error) : nullptr;
    // The residual stream starts as a copy of the input features.
    float * hidden = dctx ? scratch<float>(kOut, input.feats.size(), error) : nullptr;
    if (!hidden) return false;
    if (!hip_ok(hipMemcpyAsync(hidden, in.feats, input.feats.size() * sizeof(float),
                               hipMemcpyDeviceToDevice, d.stream()),
                "device copy", error)) {
        return false;
    }
    pxs_block_config cfg{};
    cfg.channels = C;
    cfg.num_heads = H;
    cfg.mlp_hidden = config.mlp_hidden;
    cfg.context_channels = config.context_channels;
    cfg.proj_in_channels = config.proj_in_channels;
    cfg.norm_eps = config.norm_eps;
    cfg.rope_freq_min = config.rope_freq_min;
    cfg.rope_freq_base = config.rope_freq_base;
    cfg.use_rope = config.use_rope ? 1 : 0;
    cfg.qk_rms_norm = config.qk_rms_norm ? 1 : 0;
    cfg.qk_rms_norm_cross = config.qk_rms_norm_cross ? 1 : 0;
    cfg.use_projection = config.use_projection ? 1 : 0;
    void * ws = device().buffer(kWork,
                                pxs_transformer_block_workspace_bytes(PXS_F32, &cfg, in.n,
                                                                      ctx.tokens, input.batch_size),
                                error);
    int64_t * status = scratch<int64_t>(kStatus, 1, error);
    if (!ws || !status) return false;
    if (!pxs_ok(pxs_transformer_block(PXS_F32, &cfg, &dw, in.coords, in.n, input.batch_size, dcu,
                                      hidden, tmod, ctx.feats, dctx, ctx.tokens,
                                      config.use_projection ? proj.feats : nullptr, ws,
                                      d.stream()),
                error) ||
        !pxs_ok(pxs_status_reset(status, d.stream()), error) ||
        !pxs_ok(pxs_check_finite(PXS_F32, hidden, in.n, C, C, status, d.stream()), error)) {
        return false;
    }
    int64_t host_status = 0;
    if (!download(&host_status, status, 1, error)) return false;
    if (host_status != std::numeric_limits<int64_t>::max()) {
        // The reference reports a non-finite intermediate when the next
        // primitive validates it; the fused block reports it on its output.
        set_error(error, "sparse features contain a non-finite value");
        return false;
    }
    SparseTensorF32 result;
    copy_shape(input, C, result);
    result.feats.resize(input.feats.size());
    if (!download(result.feats.data(), hidden, result.feats.size(), error)) return false;
    output = std::move(result);
    return true;
}

// ---- flow Euler sampler (src/flow_sampler.cpp) ------------------------------
//
// The reference control flow, error checks and messages, with the model as a
// host callback; the blend, CFG rescale, x0 and Euler update run on the
// device (pxs_flow_guidance and friends), so the state is uploaded once,
// updated in HBM, and copied back each step for the next callback.

namespace {

// PIXAL3D_FLOW_NONFINITE_TRACE (src/flow_sampler.cpp:20-83).  Every tensor
// the reference traces is in HBM here when it is traced, so the figures come
// from one device reduction over that copy (pxs_value_stats_f32) and only a
// 48-byte summary crosses to the host.  The printed line and the error text
// are the reference's; its mean is a serial long-double sum divided by the
// value count, the device's a double tree sum, which the six printed digits
// do not tell apart.
bool trace_requested() {
    const char * v = std::getenv("PIXAL3D_FLOW_NONFINITE_TRACE");
    if (v == nullptr || v[0] == '\0') return false;
    return std::strcmp(v, "0") != 0;
}

struct TracePoint {
    int step;
    float timestep;
    const char * branch;
};

bool trace_on_device(const float * values, int64_t points, int channels, const char * tensor,
                     const TracePoint & at, std::string * error) {
    Device & d = device();
    const int64_t count = points * channels;
    auto * summary = static_cast<pxs_value_stats *>(
        d.buffer(kTraceStats, sizeof(pxs_value_stats), error));
    void * work = d.buffer(kTraceWork, pxs_value_stats_workspace_bytes(count), error);
    if (!summary || !work ||
        !pxs_ok(pxs_value_stats_f32(values, count, summary, work, d.stream()), error)) {
        return false;
    }
    pxs_value_stats st{};
    if (!download(&st, summary, 1, error)) return false;
    const bool has_values = count > 0;
    std::ostringstream line;
    line << "pixal3d: flow trace step=" << at.step << " timestep=" << at.timestep
         << " branch=" << at.branch << " tensor=" << tensor << " points=" << points
         << " values=" << count << " min=" << (has_values ? st.min : 0.0f)
         << " max=" << (has_values ? st.max : 0.0f) << " max_abs=" << st.max_abs
         << " mean=" << (has_values ? st.sum / static_cast<double>(count) : 0.0)
         << " nonfinite=" << st.nonfinite;
    if (st.nonfinite > 0) {
        line << " first_bad_index=" << st.first_bad << " first_bad_value=" << st.first_bad_value;
    }
    std::cerr << line.str() << std::endl;
    if (st.nonfinite == 0) return true;
    std::ostringstream msg;
    msg << "flow " << tensor << " contains non-finite values at step " << at.step
        << " (branch=" << at.branch << ", first index=" << st.first_bad << ")";
    set_error(error, msg.str());
    return false;
}

// check_model_output (src/flow_sampler.cpp:126-136): a velocity must be a
// valid tensor over exactly the state's voxels, shape and channel count.
bool accept_velocity(const SparseTensorF32 & state, const SparseTensorF32 & velocity,
                     std::string * error) {
    if (!velocity.valid(error)) return false;
    const int want[5] = {state.batch_size, state.channels, state.spatial_x, state.spatial_y,
                         state.spatial_z};
    const int got[5] = {velocity.batch_size, velocity.channels, velocity.spatial_x,
                        velocity.spatial_y, velocity.spatial_z};
    if (std::equal(want, want + 5, got) && velocity.feats.size() == state.feats.size() &&
        velocity.coords == state.coords) {
        return true;
    }
    set_error(error, "flow model velocity shape or coordinates changed during sampling");
    return false;
}

pxs_flow_sampler_config sampler_config(const FlowEulerSamplerConfig & c) {
    pxs_flow_sampler_config s{};
    s.steps = c.steps;
    s.sigma_min = c.sigma_min;
    s.rescale_t = c.rescale_t;
    s.guidance_strength = c.guidance_strength;
    s.guidance_rescale = c.guidance_rescale;
    s.guidance_interval_min = c.guidance_interval_min;
    s.guidance_interval_max = c.guidance_interval_max;
    return s;
}

// The first failing check of sparse_batch_std's input on an x0 computed in
// HBM (src/flow_sampler.cpp:162-182): finiteness (SparseTensorF32::valid;
// the coordinates are the state's, already valid), then a point per item.
bool x0_checks(const float * state, const float * pred, int64_t count, float t, float sigma_min,
               int64_t rows, int channels, bool empty_item, std::string * error) {
    Device & d = device();
    float * x0 = scratch<float>(kFlowX0, static_cast<std::size_t>(count), error);
    int64_t * status = scratch<int64_t>(kStatus, 1, error);
    if (!x0 || !status) return false;
    if (!pxs_ok(pxs_flow_pred_to_xstart(state, pred, count, t, sigma_min, x0, d.stream()), error) ||
        !pxs_ok(pxs_status_reset(status, d.stream()), error) ||
        !pxs_ok(pxs_check_finite(PXS_F32, x0, rows, channels, channels, status, d.stream()), error)) {
        return false;
    }
    int64_t host_status = 0;
    if (!download(&host_status, status, 1, error)) return false;
    if (host_status != std::numeric_limits<int64_t>::max()) {
        set_error(error, "sparse features contain a non-finite value");
        return false;
    }
    if (empty_item) {
        set_error(error, "flow CFG rescale requires at least one point per batch");
        return false;
    }
    return true;
}

} // namespace

bool flow_euler_sample_f32(const SparseTensorF32 & noise, const FlowEulerSamplerConfig & config,
                           const FlowVelocityFn & model, FlowEulerSampleF32 & output,
                           std::string * error) {
    output = FlowEulerSampleF32{};
    if (!noise.valid(error)) return false;
    const pxs_flow_sampler_config scfg = sampler_config(config);
    {
        float t0 = 0.0f, t1 = 0.0f, g = 0.0f;
        // Configuration checks of valid_config (src/flow_sampler.cpp:111-124).
        if (pxs_flow_sampler_schedule(&scfg, 0, &t0, &t1, &g) != PXS_OK &&
            std::string(pxs_last_error()) == "invalid flow Euler sampler configuration") {
            set_error(error, "invalid flow Euler sampler configuration");
            return false;
        }
    }
    if (!model) {
        set_error(error, "flow Euler sampler model callback is empty");
        return false;
    }
    SparseTensorF32 state = noise;
    const bool diagnostics = trace_requested();
    if (config.record_trajectory) {
        output.pred_x_t.reserve(static_cast<std::size_t>(config.steps));
        output.pred_x_0.reserve(static_cast<std::size_t>(config.steps));
    }
    Device & d = device();
    if (!d.ready(error)) return false;
    const int64_t rows = static_cast<int64_t>(state.points());
    const int channels = state.channels;
    const int64_t count = rows * channels;
    const std::size_t ucount = static_cast<std::size_t>(count);
    float * dstate = upload(kFlowState, state.feats.data(), ucount, error);
    if (!dstate) return false;
    // A traced tensor: trace_on_device over its HBM copy, when requested.
    auto traced = [&](const float * values, const char * tensor, int step, float t,
                      const char * branch) {
        return !diagnostics ||
               trace_on_device(values, rows, channels, tensor, TracePoint{step, t, branch}, error);
    };
    if (!traced(dstate, "state_before", -1, 1.0f, "initial")) return false;
    const std::vector<int64_t> cu = batch_bounds(state);
    bool empty_item = false;
    for (int b = 0; b < state.batch_size; ++b) empty_item |= cu[b + 1] == cu[b];
    // One model call: the velocity lands in a fresh host tensor (as the
    // reference clears its workspace tensor before each callback), is checked,
    // then copied to the device slot and traced there.
    SparseTensorF32 velocity;
    auto evaluate = [&](bool conditional, float t, int step, std::size_t slot) -> const float * {
        velocity = SparseTensorF32{};
        if (!model(state, 1000.0f * t, conditional, velocity, error) ||
            !accept_velocity(state, velocity, error)) {
            return nullptr;
        }
        const float * dv = upload(slot, velocity.feats.data(), ucount, error);
        if (!dv || !traced(dv, "prediction", step, t, conditional ? "conditional" : "unconditional"))
            return nullptr;
        return dv;
    };
    for (int step = 0; step < config.steps; ++step) {
        float t = 0.0f, t_next = 0.0f, guidance = 1.0f;
        if (pxs_flow_sampler_schedule(&scfg, step, &t, &t_next, &guidance) != PXS_OK) {
            set_error(error, pxs_last_error());
            return false;
        }
        const float * dpred = nullptr;
        if (guidance == 1.0f || guidance == 0.0f) {
            dpred = evaluate(guidance == 1.0f, t, step, kFlowPred);
            if (!dpred) return false;
        } else {
            const float * dpos = evaluate(true, t, step, kFlowPos);
            if (!dpos) return false;
            const float * dneg = evaluate(false, t, step, kFlowNeg);
            if (!dneg) return false;
            float * blend = scratch<float>(kFlowPred, ucount, error);
            if (!blend ||
                !pxs_ok(pxs_flow_guidance(dstate, dpos, dneg, nullptr, nullptr, rows, channels,
                                          state.batch_size, t, config.sigma_min, guidance, 0.0f,
                                          blend, nullptr, d.stream()),
                        error) ||
                !traced(blend, "cfg_blend", step, t, "guided")) {
                return false;
            }
            if (config.guidance_rescale > 0.0f) {
                if (!x0_checks(dstate, dpos, count, t, config.sigma_min, rows, channels, empty_item,
                               error) ||
                    !x0_checks(dstate, blend, count, t, config.sigma_min, rows, channels,
                               empty_item, error)) {
                    return false;
                }
                const int64_t * dcu = upload(kFlowCu, cu.data(), cu.size(), error);
                void * ws = d.buffer(kFlowWork, pxs_flow_guidance_workspace_bytes(state.batch_size),
                                     error);
                const int32_t * dcoords =
                    dcu && ws ? upload(kInCoords, state.coords.data(), state.coords.size(), error)
                              : nullptr;
                if (!dcoords ||
                    !pxs_ok(pxs_flow_guidance(dstate, dpos, dneg, dcoords, dcu, rows, channels,
                                              state.batch_size, t, config.sigma_min, guidance,
                                              config.guidance_rescale, blend, ws, d.stream()),
                            error) ||
                    !traced(blend, "guidance_rescale", step, t, "guided")) {
                    return false;
                }
            }
            dpred = blend;
        }
        SparseTensorF32 x0;
        if (config.record_trajectory) {
            float * dx0 = scratch<float>(kFlowX0, ucount, error);
            if (!dx0 ||
                !pxs_ok(pxs_flow_pred_to_xstart(dstate, dpred, count, t, config.sigma_min, dx0,
                                                d.stream()),
                        error) ||
                !traced(dx0, "x0", step, t, "guided")) {
                return false;
            }
            copy_shape(state, channels, x0);
            x0.feats.resize(ucount);
            if (!download(x0.feats.data(), dx0, ucount, error)) return false;
        }
        if (!pxs_ok(pxs_flow_euler_update(dstate, dpred, count, t - t_next, d.stream()), error) ||
            !traced(dstate, "state_after", step, t_next, "euler") ||
            !download(state.feats.data(), dstate, ucount, error)) {
            return false;
        }
        if (config.record_trajectory) {
            output.pred_x_t.push_back(state);
            output.pred_x_0.push_back(std::move(x0));
        }
    }
    output.samples = std::move(state);
    return true;
}

} // namespace pixal3d
