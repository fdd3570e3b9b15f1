// Shared helpers of the gfx950 kernels: element types, rounding, wavefront reductions,
// error reporting and tensor-argument validation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <atomic>
#include <string>

#include "collab_edge_attn.h"

namespace cea {

typedef __bf16 bf16;
typedef _Float16 f16;

// ---------------------------------------------------------------------------------------
// error reporting (one message per host thread)
// ---------------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
const char* last_error();

#define CEA_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      ::cea::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)

#define CEA_CHECK_LAUNCH(what)                                                    \
  do {                                                                            \
    hipError_t _e = hipGetLastError();                                            \
    if (_e != hipSuccess) {                                                       \
      ::cea::set_error("%s: launch failed: %s", (what), hipGetErrorString(_e));   \
      return CEA_ELAUNCH;                                                         \
    }                                                                             \
  } while (0)

// Raises a kernel's dynamic LDS limit to 'bytes' on the current device, once per device
// (kernel attributes are per device; the first call on a device does the work, concurrent
// first calls may both set it, which is harmless).
template <auto Kernel>
hipError_t reserve_lds(int bytes) {
  static std::atomic<uint64_t> done{0};  // bit d: device d configured (devices 0..63)
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute((const void*)Kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// Compute units of the current device (queried once per device; 0 on error).
inline int device_cus() {
  static std::atomic<int> cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) {
    const int c = cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

inline size_t dtype_size(int32_t dt) {
  switch (dt) {
    case CEA_F32: return 4;
    case CEA_BF16: return 2;
    case CEA_F16: return 2;
    case CEA_F64: return 8;
    case CEA_I64: return 8;
    default: return 0;
  }
}

inline const char* dtype_name(int32_t dt) {
  switch (dt) {
    case CEA_F32: return "float32";
    case CEA_BF16: return "bfloat16";
    case CEA_F16: return "float16";
    case CEA_F64: return "float64";
    case CEA_I64: return "int64";
    default: return "unknown";
  }
}

// Checks rank, dtype and (optionally) a unit innermost stride.  Returns 0 or an error code.
int check_tensor(const cea_tensor* t, const char* name, int ndim, int dtype_or_minus1,
                 bool inner_contiguous);

// ---------------------------------------------------------------------------------------
// device-side element conversion
// ---------------------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
template <> __device__ __forceinline__ float to_f32<bf16>(bf16 x) {
  return __uint_as_float(((uint32_t)__builtin_bit_cast(uint16_t, x)) << 16);
}

// Round-to-nearest-even conversions (hardware v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }
template <typename T> __device__ __forceinline__ T from_f64(double x) { return (T)x; }

// x rounded to the storage type T and widened back to float: the value a torch op
// producing a T tensor would hand to the next op.
template <typename T> __device__ __forceinline__ float round_to(float x) {
  return to_f32<T>(from_f32<T>(x));
}
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }

// Accumulation type: f64 for f64 inputs, f32 otherwise (attention.py:56-57).
template <typename T> struct acc_of { typedef float type; };
template <> struct acc_of<double> { typedef double type; };

template <typename A> __device__ __forceinline__ A neg_inf();
template <> __device__ __forceinline__ float neg_inf<float>() { return -__builtin_inff(); }
template <> __device__ __forceinline__ double neg_inf<double>() { return -__builtin_inf(); }

// Element load widened to the accumulation type.
template <typename T, typename A> __device__ __forceinline__ A load_acc(const T* p) {
  return (A)to_f32<T>(*p);
}
template <> __device__ __forceinline__ double load_acc<double, double>(const double* p) {
  return *p;
}
template <> __device__ __forceinline__ float load_acc<float, float>(const float* p) { return *p; }

template <typename T, typename A> __device__ __forceinline__ T store_cast(A x) { return (T)x; }
template <> __device__ __forceinline__ bf16 store_cast<bf16, float>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ bf16 store_cast<bf16, double>(double x) {
  return (bf16)(float)x;  // f64 results are only stored as f64; kept for completeness
}

// Exact-rounding arithmetic without contraction into FMA, to follow the reference's
// separately rounded tensor ops.
// (written out with contraction switched off in their own bodies: hip's __fmul_rn / __fadd_rn
// are plain operators, which a file compiled with contraction on may fuse into an FMA with a
// neighbouring product after inlining; these never carry the permission)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ double mul_rn(double a, double b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ double add_rn(double a, double b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }
__device__ __forceinline__ double div_rn(double a, double b) { return __ddiv_rn(a, b); }

__device__ __forceinline__ float exp_acc(float x) { return expf(x); }
__device__ __forceinline__ double exp_acc(double x) { return exp(x); }
__device__ __forceinline__ float log_acc(float x) { return logf(x); }
__device__ __forceinline__ double log_acc(double x) { return log(x); }
__device__ __forceinline__ float log1p_acc(float x) { return log1pf(x); }
__device__ __forceinline__ double log1p_acc(double x) { return log1p(x); }
__device__ __forceinline__ bool is_finite(float x) { return __builtin_isfinite(x); }
__device__ __forceinline__ bool is_finite(double x) { return __builtin_isfinite(x); }
__device__ __forceinline__ bool is_inf(float x) { return __builtin_isinf(x); }
__device__ __forceinline__ bool is_inf(double x) { return __builtin_isinf(x); }

// Activations of the gated MLP (the reference's _ACTIVATIONS, llama.py:44-49), in f32 for
// bf16 / f16 / f32 tensors and in f64 for f64, the way torch's elementwise kernels compute
// them (silu in f32 with the exp and quotient of exp_act / silu_f32 below, within a few ulp):
//   silu              g / (1 + exp(-g))
//   gelu              (g * 0.5) * (1 + erf(g * (1/sqrt 2)))
//   gelu_pytorch_tanh (0.5 * g) * (1 + tanh(sqrt(2/pi) * (g + 0.044715 * g^3)))
//   relu              g when g > 0 or g is NaN, else 0
template <typename M> __device__ __forceinline__ M erf_acc(M x);
template <> __device__ __forceinline__ float erf_acc<float>(float x) { return erff(x); }
template <> __device__ __forceinline__ double erf_acc<double>(double x) { return erf(x); }
template <typename M> __device__ __forceinline__ M tanh_acc(M x);
template <> __device__ __forceinline__ float tanh_acc<float>(float x) { return tanhf(x); }
template <> __device__ __forceinline__ double tanh_acc<double>(double x) { return tanh(x); }

// e^x in f32 for the activations: 2^(x log2 e), with the rounding error of the product
// x * log2(e) kept as an exact FMA remainder and applied as 2^t (1 + lo ln 2), so the result
// stays within about 2 ulp for every x (v_exp_f32 is good to 1 ulp) instead of losing
// accuracy as |x| grows.  x is clamped below at -104 (the result is 0 there either way), so
// -inf gives 0; +inf gives NaN and finite x above 88.72 gives +inf.
__device__ __forceinline__ float exp_act(float x) {
  constexpr float kL2e = 1.44269502162933349609375f;   // log2(e) rounded to f32
  constexpr float kL2eLo = 1.925963033500e-8f;          // log2(e) - kL2e
  x = __builtin_fmaxf(x, -104.0f);
  const float t = x * kL2e;
  float lo = __builtin_fmaf(x, kL2e, -t);   // x * kL2e - t, exactly
  lo = __builtin_fmaf(x, kL2eLo, lo);
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p, lo * 0.693147180559945309417f, p);
}

// tanh(u) for the tanh form of GELU, whose value only enters as 1 + tanh(u): 1 - 2 / (e^(2u)
// + 1), with e^(2u) from exp_act (within 2 ulp; 2u is exact) and the quotient from the
// reciprocal with one FMA correction.  Its absolute error stays within a few units of 2^-24,
// which the sum with 1 rounds away.  |u| is clamped to 10 first (tanh(10) and tanh(-10) round
// to +-1 in f32, and e^(2u) stays finite); NaN passes the clamp and gives NaN.
__device__ __forceinline__ float tanh_gelu_f32(float u) {
  const float uc = u > 10.0f ? 10.0f : (u < -10.0f ? -10.0f : u);
  const float d = exp_act(2.0f * uc) + 1.0f;
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = 2.0f * r;
  const float q2 = __builtin_fmaf(__builtin_fmaf(-d, q, 2.0f), r, q);  // q + (2 - d q) / d
  return 1.0f - q2;
}

// silu(g) = g / (1 + e^-g) in f32: the quotient from the reciprocal with one FMA correction
// (the correctly rounded quotient but in rare cases), and g / inf = -0 as in IEEE division.
__device__ __forceinline__ float silu_f32(float g) {
  const float d = 1.0f + exp_act(-g);
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = g * r;
  const float q2 = __builtin_fmaf(__builtin_fmaf(-q, d, g), r, q);
  return __builtin_isinf(d) ? q : q2;
}

template <int ACT, typename M> __device__ __forceinline__ M gate_act(M a) {
  if constexpr (ACT == CEA_ACT_SILU && sizeof(M) == 4) {
    return silu_f32(a);
  } else if constexpr (ACT == CEA_ACT_SILU) {
    return div_rn(a, add_rn((M)1, exp_acc(-a)));
  } else if constexpr (ACT == CEA_ACT_GELU) {
    const M alpha = (M)0.70710678118654752440;  // 1/sqrt(2)
    return mul_rn(mul_rn(a, (M)0.5), add_rn((M)1, erf_acc<M>(mul_rn(a, alpha))));
  } else if constexpr (ACT == CEA_ACT_GELU_TANH) {
    const M beta = (M)0.79788456080286535588;   // sqrt(2/pi)
    const M kappa = (M)0.044715;
    const M cube = mul_rn(mul_rn(a, a), a);
    const M inner = mul_rn(beta, add_rn(a, mul_rn(kappa, cube)));
    if constexpr (sizeof(M) == 4)
      return mul_rn(mul_rn((M)0.5, a), add_rn((M)1, tanh_gelu_f32(inner)));
    else
      return mul_rn(mul_rn((M)0.5, a), add_rn((M)1, tanh_acc<M>(inner)));
  } else {
    return a <= (M)0 ? (M)0 : a;
  }
}

// torch.logaddexp semantics: equal infinities return that infinity, otherwise
// max + log1p(exp(-|a-b|)).
template <typename A> __device__ __forceinline__ A logaddexp(A a, A b) {
  if (is_inf(a) && a == b) return a;
  A m = a > b ? a : b;
  A d = a > b ? a - b : b - a;
  return m + log1p_acc(exp_acc(-d));
}

// ---------------------------------------------------------------------------------------
// wavefront (64-lane) reductions
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ int64_t wave_min_i64(int64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    int64_t o = __shfl_xor(v, off, 64);
    v = o < v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int64_t wave_max_i64(int64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    int64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Uniform (scalar) copy of a wave-uniform value.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------------------------------
// key-tile position summary used to skip or classify KV tiles without host syncs
// ---------------------------------------------------------------------------------------
struct TileInfo {
  int64_t min_valid;  // smallest k_pos >= 0 in the tile (INT64_MAX if none)
  int64_t max_valid;  // largest  k_pos >= 0 in the tile (INT64_MIN if none)
  int32_t n_valid;    // number of keys with k_pos >= 0 (keys past Sk count as invalid)
  int32_t pad[3];
};
static_assert(sizeof(TileInfo) == 32, "TileInfo must stay 32 bytes");

// Query-head -> KV-head mapping passed by value to the kernels.
struct HeadMap {
  int32_t group;  // > 0: kv = h / group; 0: explicit table
  int16_t kv[CEA_MAX_MAPPED_HEADS];
  __device__ __forceinline__ int kv_of(int h) const { return group > 0 ? h / group : kv[h]; }
};

int make_head_map(HeadMap* m, int64_t Hq, int64_t Hkv, const int32_t* kv_map, int32_t len);

}  // namespace cea
