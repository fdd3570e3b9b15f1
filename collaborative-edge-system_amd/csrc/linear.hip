// Fused column-parallel projection on hipBLASLt: out = x . W^T (+ bias).
//
// FusedColumnParallelLinear.forward (collab_infer/parallel/tensor_parallel.py:294-295) runs
// the Q/K/V projections (and the gate/up projections of gated MLPs) of one input as a single
// F.linear over the concatenated weight and returns column slices of its output.  That is a
// plain GEMM, so it goes to the library: bf16/f16 (or f32) operands, f32 accumulation, the
// bias added before the single rounding to the output dtype, as torch's addmm does.  The
// column slices that feed the rotary / KV-cache append / SiLU-gate kernels are strided
// views of the output; nothing is copied.
//
// The first call for a shape times the library heuristic's first candidates and keeps the
// fastest (a small per-process table keyed by device, dtype and shape); that call waits for
// the stream.  Under stream capture the heuristic's first choice is kept without timing.
//
// torch's row-major [N, K] x [M, K]^T is the column-major product W^T(KxM, transposed) x
// x^T(KxN) = out^T (MxN) with the row strides as leading dimensions.
#include <hipblaslt/hipblaslt.h>

#include <mutex>

#include "cea_kernels.hpp"

namespace cea {
namespace {

constexpr int kMaxDevices = 64;
constexpr int kAlgoCache = 32;
constexpr int kTuneCandidates = 8;  // heuristic candidates timed on a shape's first call
constexpr int kTuneReps = 3;

struct AlgoKey {
  int dev, dtype, bias;
  int64_t M, N, K, ldw, ldx, ldo;
  size_t ws;
  bool operator==(const AlgoKey& o) const {
    return dev == o.dev && dtype == o.dtype && bias == o.bias && M == o.M && N == o.N &&
           K == o.K && ldw == o.ldw && ldx == o.ldx && ldo == o.ldo && ws == o.ws;
  }
};

struct AlgoEntry {
  AlgoKey key;
  hipblasLtMatmulAlgo_t algo;
  bool valid;
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
AlgoEntry g_algos[kAlgoCache] = {};
int g_next_algo = 0;

hipDataType lt_type(int dt) {
  switch (dt) {
    case CEA_BF16: return HIP_R_16BF;
    case CEA_F16: return HIP_R_16F;
    default: return HIP_R_32F;
  }
}

// RAII holders of the per-call descriptors
struct Desc {
  hipblasLtMatmulDesc_t d = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  ~Desc() {
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (c) hipblasLtMatrixLayoutDestroy(c);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (d) hipblasLtMatmulDescDestroy(d);
  }
};

#define CEA_LT(call, what)                                                              \
  do {                                                                                  \
    hipblasStatus_t _s = (call);                                                        \
    if (_s != HIPBLAS_STATUS_SUCCESS) {                                                 \
      ::cea::set_error("linear: %s failed (hipBLASLt status %d)", (what), (int)_s);     \
      return CEA_ELAUNCH;                                                               \
    }                                                                                   \
  } while (0)

}  // namespace

int launch_linear(const cea_tensor* x, const cea_tensor* w, const cea_tensor* bias,
                  cea_tensor* out, void* workspace, size_t ws_bytes, hipStream_t st) {
  const int dt = x->dtype;
  const int64_t N = x->size[0], K = x->size[1], M = w->size[0];
  if (N == 0 || M == 0) return CEA_OK;
  int dev = 0;
  hipError_t he = hipGetDevice(&dev);
  CEA_REQUIRE(he == hipSuccess && dev >= 0 && dev < kMaxDevices, CEA_ELAUNCH,
              "linear: no current device (%s)", hipGetErrorString(he));
  hipblasLtHandle_t handle;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_handle[dev]) CEA_LT(hipblasLtCreate(&g_handle[dev]), "hipblasLtCreate");
    handle = g_handle[dev];
  }
  const hipDataType t = lt_type(dt);
  Desc ds;
  CEA_LT(hipblasLtMatmulDescCreate(&ds.d, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul descriptor");
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  CEA_LT(hipblasLtMatmulDescSetAttribute(ds.d, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)),
         "transA");
  CEA_LT(hipblasLtMatmulDescSetAttribute(ds.d, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)),
         "transB");
  if (bias) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const void* bp = bias->data;
    const int32_t bt = (int32_t)t;
    CEA_LT(hipblasLtMatmulDescSetAttribute(ds.d, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)),
           "bias epilogue");
    CEA_LT(hipblasLtMatmulDescSetAttribute(ds.d, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)),
           "bias pointer");
    CEA_LT(hipblasLtMatmulDescSetAttribute(ds.d, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)),
           "bias type");
  }
  const int64_t ldw = w->stride[0], ldx = x->stride[0], ldo = out->stride[0];
  CEA_LT(hipblasLtMatrixLayoutCreate(&ds.a, t, (uint64_t)K, (uint64_t)M, ldw), "layout of W");
  CEA_LT(hipblasLtMatrixLayoutCreate(&ds.b, t, (uint64_t)K, (uint64_t)N, ldx), "layout of x");
  CEA_LT(hipblasLtMatrixLayoutCreate(&ds.c, t, (uint64_t)M, (uint64_t)N, ldo), "layout of out");

  const AlgoKey key{dev, dt, bias ? 1 : 0, M, N, K, ldw, ldx, ldo, ws_bytes};
  hipblasLtMatmulAlgo_t algo;
  bool found = false;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    for (int i = 0; i < kAlgoCache; ++i)
      if (g_algos[i].valid && g_algos[i].key == key) {
        algo = g_algos[i].algo;
        found = true;
        break;
      }
  }
  if (!found) {
    CEA_LT(hipblasLtMatmulPreferenceCreate(&ds.pref), "preference");
    const uint64_t maxws = ws_bytes;
    CEA_LT(hipblasLtMatmulPreferenceSetAttribute(ds.pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                 &maxws, sizeof(maxws)),
           "workspace preference");
    hipblasLtMatmulHeuristicResult_t res[kTuneCandidates];
    int n = 0;
    CEA_LT(hipblasLtMatmulAlgoGetHeuristic(handle, ds.d, ds.a, ds.b, ds.c, ds.c, ds.pref,
                                           kTuneCandidates, res, &n),
           "algorithm heuristic");
    CEA_REQUIRE(n > 0, CEA_EUNSUPPORTED, "linear: hipBLASLt has no algorithm for %lldx%lldx%lld %s",
                (long long)M, (long long)N, (long long)K, dtype_name(dt));
    algo = res[0].algo;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone;
    if (n > 1 && !capturing) {
      // first call for this shape: time the heuristic's candidates on the caller's stream
      // (their results land in out and are overwritten by the final product below)
      hipEvent_t e0, e1;
      if (hipEventCreate(&e0) == hipSuccess) {
        if (hipEventCreate(&e1) == hipSuccess) {
          const float one = 1.f, zero = 0.f;
          float best = 3.4e38f;
          for (int i = 0; i < n; ++i) {
            if (res[i].state != HIPBLAS_STATUS_SUCCESS) continue;
            bool ok = true;
            hipEventRecord(e0, st);
            for (int r = 0; r < kTuneReps && ok; ++r)
              ok = hipblasLtMatmul(handle, ds.d, &one, w->data, ds.a, x->data, ds.b, &zero,
                                   out->data, ds.c, out->data, ds.c, &res[i].algo, workspace,
                                   ws_bytes, st) == HIPBLAS_STATUS_SUCCESS;
            hipEventRecord(e1, st);
            float ms = 0.f;
            if (ok && hipEventSynchronize(e1) == hipSuccess &&
                hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms < best) {
              best = ms;
              algo = res[i].algo;
            }
          }
          hipEventDestroy(e1);
        }
        hipEventDestroy(e0);
      }
    }
    std::lock_guard<std::mutex> lock(g_mu);
    g_algos[g_next_algo] = AlgoEntry{key, algo, true};
    g_next_algo = (g_next_algo + 1) % kAlgoCache;
  }
  const float alpha = 1.f, beta = 0.f;
  CEA_LT(hipblasLtMatmul(handle, ds.d, &alpha, w->data, ds.a, x->data, ds.b, &beta, out->data, ds.c,
                         out->data, ds.c, &algo, workspace, ws_bytes, st),
         "matmul");
  return CEA_OK;
}

}  // namespace cea
