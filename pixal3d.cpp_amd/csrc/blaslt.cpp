// Plain linears (sparse_linear / varlen_linear, src/sparse.cpp:337-488, with
// the block's residual adds), bf16 or fp32, through hipBLASLt: these are dense
// GEMMs over rows, with no gather, where the library's kernels run 1.7-2x the
// gather-GEMM kernels of gemm.hip (fp32 ones in full fp32: compute type 32F,
// v_mfma_f32_*_f32).  Column-major view of the row-major
// operands: D (cout x rows, ld cout) = op(A) B with A = the weight
// [cout, cin] row-major read as cin x cout and transposed, B = x (cin x rows).
// The fp32 bias is the epilogue's bias vector (one per D row, i.e. per output
// channel); GELU (tanh form) and SiLU are the epilogue's GELU and Swish(x, 1)
// (x * sigmoid(x)); a residual add is
// C = D = the fp32 residual with beta = 1.
//
// One handle per device; matrix layouts and the heuristic's algorithm are
// cached per shape and workspace cap (at most 4096 shapes), the matmul
// descriptor (which holds the bias pointer) is made per call.  The library's workspace is the caller's
// (compositions carve kLibWorkspaceBytes from their own workspace; the plain
// entry points have none, and then only algorithms that need no workspace
// qualify): nothing is allocated per call.  Tall products over few channels
// run 2-5x faster with one (2.5M x 64 -> 256 bf16: 377 against 866 us).  A
// shape for which the heuristic offers no algorithm is left to the caller, and
// so are the ones the gemm.hip kernels run faster: bf16 with at most 64 input
// and output channels, fp32 under 2^26 multiply-adds.

#include "pxs_common.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <mutex>
#include <tuple>

namespace pxs {
namespace {

// Layouts and algorithm of one shape.  Held by shared pointer: a call keeps
// its shape alive while it runs, even if another thread's miss evicts it.
struct Shape {
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
    bool ok = false;
    Shape() = default;
    Shape(const Shape &) = delete;
    Shape & operator=(const Shape &) = delete;
    ~Shape() {
        if (a) hipblasLtMatrixLayoutDestroy(a);
        if (b) hipblasLtMatrixLayoutDestroy(b);
        if (c) hipblasLtMatrixLayoutDestroy(c);
    }
};

// (device, rows, cin, cout, epilogue, A/B type, D type, accumulate, workspace cap)
using ShapeKey = std::tuple<int, int64_t, int, int, int, int, int, int, size_t>;

std::mutex g_mutex;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<ShapeKey, std::shared_ptr<const Shape>> g_shapes;

// Row counts vary from call to call (each input has its own voxel count), so
// the cache is bounded: past this many entries it starts over.
constexpr size_t kMaxShapes = 4096;

bool set_desc(hipblasLtMatmulDesc_t desc, hipblasLtMatmulDescAttributes_t attr, const void * v,
              size_t bytes) {
    return hipblasLtMatmulDescSetAttribute(desc, attr, v, bytes) == HIPBLAS_STATUS_SUCCESS;
}

// The descriptor of one call: transposes, epilogue and its bias.
hipblasLtMatmulDesc_t make_desc(hipblasLtEpilogue_t epi, const float * bias) {
    hipblasLtMatmulDesc_t desc = nullptr;
    if (hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return nullptr;
    const hipblasOperation_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
    const uint32_t e = static_cast<uint32_t>(epi);
    bool ok = set_desc(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof(op_t)) &&
              set_desc(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof(op_n)) &&
              set_desc(desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &e, sizeof(e));
    if (ok && bias) {
        const hipDataType bt = HIP_R_32F;
        ok = set_desc(desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) &&
             set_desc(desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
    }
    if (!ok) {
        hipblasLtMatmulDescDestroy(desc);
        return nullptr;
    }
    return desc;
}

// The cached layouts and algorithm of a shape, or nullptr (no algorithm).
// Called with g_mutex held.
std::shared_ptr<const Shape> shape_for(int device, hipblasLtHandle_t handle, int64_t rows, int cin, int cout,
                        hipblasLtEpilogue_t epi, hipDataType dtype_in, hipDataType dtype_d,
                        bool accumulate, size_t ws_cap) {
    const ShapeKey key{device, rows, cin, cout, static_cast<int>(epi), static_cast<int>(dtype_in),
                       static_cast<int>(dtype_d), accumulate ? 1 : 0, ws_cap};
    auto it = g_shapes.find(key);
    if (it != g_shapes.end()) return it->second->ok ? it->second : nullptr;
    if (g_shapes.size() >= kMaxShapes) g_shapes.clear();  // shapes in use stay alive
    auto made = std::make_shared<Shape>();
    Shape & sh = *made;
    bool ok = hipblasLtMatrixLayoutCreate(&sh.a, dtype_in, cin, cout, cin) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&sh.b, dtype_in, cin, rows, cin) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&sh.c, dtype_d, cout, rows, cout) == HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulDesc_t desc = ok ? make_desc(epi, nullptr) : nullptr;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (desc && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
        const uint64_t ws = ws_cap;
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                              sizeof(ws));
        hipblasLtMatmulHeuristicResult_t result{};
        int found = 0;
        if (hipblasLtMatmulAlgoGetHeuristic(handle, desc, sh.a, sh.b, sh.c, sh.c, pref, 1, &result,
                                            &found) == HIPBLAS_STATUS_SUCCESS &&
            found > 0 && result.state == HIPBLAS_STATUS_SUCCESS && result.workspaceSize <= ws_cap) {
            sh.algo = result.algo;
            sh.workspace = result.workspaceSize;
            sh.ok = true;
        }
        hipblasLtMatmulPreferenceDestroy(pref);
    }
    if (desc) hipblasLtMatmulDescDestroy(desc);
    g_shapes[key] = made;
    return sh.ok ? made : nullptr;
}

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

} // namespace

// y (rows x cout, y_dtype) = x W^T + bias, then act (PXS_ACT_NONE,
// PXS_ACT_GELU_TANH or PXS_ACT_SILU), x and w of type dtype; with accumulate,
// y (fp32) += x W^T + bias.  ws (256-byte aligned, ws_bytes; may be null) is
// the library's workspace for this call.  Returns PXS_OK and sets *done when
// hipBLASLt ran it; leaves *done false when the shape is not one it takes
// (the caller runs its own kernel).
int blaslt_linear(int dtype, const void * x, int64_t rows, int cin, const void * w,
                  const float * bias, int cout, int act, int y_dtype, void * y, bool accumulate,
                  void * ws, size_t ws_bytes, hipStream_t s, bool * done) {
    *done = false;
#ifndef PXS_BLASLT
#define PXS_BLASLT 1
#endif
    if (!PXS_BLASLT) return PXS_OK;
    if (act != PXS_ACT_NONE && act != PXS_ACT_GELU_TANH && act != PXS_ACT_SILU) return PXS_OK;
    if (accumulate && (y_dtype != PXS_F32 || act != PXS_ACT_NONE)) return PXS_OK;
    if (dtype != PXS_BF16 && dtype != PXS_F32) return PXS_OK;
    if (dtype == PXS_F32 && y_dtype != PXS_F32) return PXS_OK;
    const int vec = dtype == PXS_BF16 ? 8 : 4;  // elements per 16 bytes
    if (rows < 256 || cin % vec != 0 || cout % 8 != 0 || !aligned16(x) || !aligned16(w) ||
        !aligned16(y) || (bias && !aligned16(bias)))
        return PXS_OK;
    // Shapes the gemm.hip kernels run faster (measured: bf16 64 -> 64 over
    // 2.5M rows 228 against 258 us, fp32 16k x 64 -> 64 13 against 17 us).
    if (dtype == PXS_BF16 && cin <= 64 && cout <= 64) return PXS_OK;
    if (dtype == PXS_F32 && static_cast<double>(rows) * cin * cout < 67108864.0) return PXS_OK;
    const size_t ws_cap = ws ? ws_bytes : 0;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return PXS_OK;
    const hipblasLtEpilogue_t epi =
        act == PXS_ACT_GELU_TANH ? (bias ? HIPBLASLT_EPILOGUE_GELU_BIAS : HIPBLASLT_EPILOGUE_GELU)
        : act == PXS_ACT_SILU
            ? (bias ? HIPBLASLT_EPILOGUE_SWISH_BIAS_EXT : HIPBLASLT_EPILOGUE_SWISH_EXT)
                                 : (bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT);
    const hipDataType dtype_in = dtype == PXS_F32 ? HIP_R_32F : HIP_R_16BF;
    const hipDataType dtype_d = y_dtype == PXS_F32 ? HIP_R_32F : HIP_R_16BF;
    hipblasLtHandle_t handle = nullptr;
    std::shared_ptr<const Shape> sh;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        auto hit = g_handles.find(device);
        if (hit == g_handles.end()) {
            hipblasLtHandle_t h = nullptr;
            if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
            hit = g_handles.emplace(device, h).first;
        }
        handle = hit->second;
        if (!handle) return PXS_OK;
        sh = shape_for(device, handle, rows, cin, cout, epi, dtype_in, dtype_d, accumulate, ws_cap);
    }
    if (!sh) return PXS_OK;
    hipblasLtMatmulDesc_t desc = make_desc(epi, bias);
    if (!desc) return PXS_OK;
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    const hipblasStatus_t st = hipblasLtMatmul(handle, desc, &alpha, w, sh->a, x, sh->b, &beta, y,
                                               sh->c, y, sh->c, &sh->algo,
                                               sh->workspace ? ws : nullptr, sh->workspace, s);
    hipblasLtMatmulDescDestroy(desc);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail(PXS_ERR_HIP, "hipblasLtMatmul failed");
    *done = true;
    return check_launch("hipblasLtMatmul");
}

} // namespace pxs
