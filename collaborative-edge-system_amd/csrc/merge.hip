// Exact LSE merges of partial attention results.
//
// merge_attention      (collab_infer/parallel/attention.py:242-250)
// merge_attention_list (collab_infer/parallel/attention.py:253-264)
//
// Both are HBM-bound: one pass reads every partial output once and writes the merged row.
// A thread owns VEC consecutive features of one (b, s, h) row and recomputes the row's
// weights (all lanes of a wave execute them together, so the redundancy costs no issue
// slots).  The arithmetic follows the reference's rounding order: each weighted partial
// is rounded before it is added, in the order of the partial list.
#include <type_traits>

#include "cea_kernels.hpp"

namespace cea {

// NMAX >= p.n: the partials a launch can hold (registers for all of them are held at once)
template <typename A, typename O, int VEC, int NMAX>
__global__ __launch_bounds__(256) void merge_kernel(const MergeParams p) {
  const int64_t nvec = p.D / VEC;
  const int64_t total = (int64_t)p.B * p.Sq * p.H * nvec;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= total) return;
  const int dv = (int)(tid % nvec);
  int64_t row = tid / nvec;
  const int h = (int)(row % p.H);
  row /= p.H;
  const int s = (int)(row % p.Sq);
  const int b = (int)(row / p.Sq);

  // every partial's features and lse are loaded before any of the weights is computed: one
  // memory round trip per thread, not one for the lses and another for the features
  A x[NMAX][VEC];
  A l[NMAX];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    if (i < p.n) {
      const A* op = (const A*)p.outs[i] + b * p.os[i][0] + s * p.os[i][1] + h * p.os[i][2] +
                    (int64_t)dv * VEC;
      if constexpr (VEC == 4 && sizeof(A) == 4) {
        const float4 t = *(const float4*)op;
        x[i][0] = t.x; x[i][1] = t.y; x[i][2] = t.z; x[i][3] = t.w;
      } else if constexpr (VEC == 2 && sizeof(A) == 8) {
        const double2 t = *(const double2*)op;
        x[i][0] = t.x; x[i][1] = t.y;
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[i][e] = op[e];
      }
      const A* lp = (const A*)p.lses[i];
      l[i] = lp[b * p.ls[i][0] + h * p.ls[i][1] + s * p.ls[i][2]];
    }
  }
  // lse = logsumexp over the partials (n == 2 uses logaddexp, as merge_attention does)
  A m = neg_inf<A>();
#pragma unroll
  for (int i = 0; i < NMAX; ++i)
    if (i < p.n) m = l[i] > m ? l[i] : m;
  A lse;
  if (p.pairwise) {
    lse = logaddexp<A>(l[0], l[1]);
  } else {
    const A shift = is_inf(m) ? (A)0 : m;  // logsumexp's infinite-max guard
    A sum = 0;
#pragma unroll
    for (int i = 0; i < NMAX; ++i)
      if (i < p.n) sum = add_rn(sum, exp_acc(l[i] - shift));
    lse = log_acc(sum) + shift;
  }
  const A safe = is_finite(lse) ? lse : (A)0;

  A acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0;
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    if (i < p.n) {
      const A w = exp_acc(l[i] - safe);
      if (i == 0) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = mul_rn(x[i][e], w);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = add_rn(acc[e], mul_rn(x[i][e], w));
      }
    }
  }
  if constexpr (sizeof(O) == sizeof(A)) {
    A* dst = (A*)p.out + b * p.dos[0] + s * p.dos[1] + h * p.dos[2] + (int64_t)dv * VEC;
    if constexpr (VEC == 4 && sizeof(A) == 4) {
      *(float4*)dst = make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else if constexpr (VEC == 2 && sizeof(A) == 8) {
      *(double2*)dst = make_double2(acc[0], acc[1]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e] = acc[e];
    }
  } else {
    // final result in the query dtype (out.to(q.dtype))
    O* dst = (O*)p.out + b * p.dos[0] + s * p.dos[1] + h * p.dos[2] + (int64_t)dv * VEC;
#pragma unroll
    for (int e = 0; e < VEC; ++e) dst[e] = (O)acc[e];
  }
  if (dv == 0 && p.lse) {
    A* lp = (A*)p.lse;
    lp[b * p.dls[0] + h * p.dls[1] + s * p.dls[2]] = lse;
  }
}

static bool aligned(const void* ptr, size_t a) { return ((uintptr_t)ptr % a) == 0; }

int launch_merge(const MergeParams& p, hipStream_t st) {
  const size_t esz = p.dtype == CEA_F64 ? 8 : 4;
  const size_t osz = dtype_size(p.out_dtype);
  const int vec_bytes = 16;
  const size_t ovb = vec_bytes / esz * osz;  // bytes of one output vector
  bool vec_ok = (p.D * esz) % vec_bytes == 0 && aligned(p.out, ovb) &&
                (p.dos[0] * osz) % ovb == 0 && (p.dos[1] * osz) % ovb == 0 &&
                (p.dos[2] * osz) % ovb == 0;
  for (int i = 0; i < p.n && vec_ok; ++i) {
    vec_ok = aligned(p.outs[i], vec_bytes) && (p.os[i][0] * esz) % vec_bytes == 0 &&
             (p.os[i][1] * esz) % vec_bytes == 0 && (p.os[i][2] * esz) % vec_bytes == 0;
  }
  const int vec = vec_ok ? (int)(vec_bytes / esz) : 1;
  const int64_t total = (int64_t)p.B * p.Sq * p.H * (p.D / vec);
  if (total == 0) return CEA_OK;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  CEA_REQUIRE(blocks < (int64_t)1 << 31, CEA_EUNSUPPORTED, "merge: tensor too large");
  const dim3 grid((unsigned)blocks), block(threads);
  auto go = [&](auto nmax) {
    constexpr int NM = decltype(nmax)::value;
    if (p.dtype == CEA_F64) {
      if (vec == 2) hipLaunchKernelGGL((merge_kernel<double, double, 2, NM>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((merge_kernel<double, double, 1, NM>), grid, block, 0, st, p);
    } else if (p.out_dtype == CEA_BF16) {
      if (vec == 4) hipLaunchKernelGGL((merge_kernel<float, bf16, 4, NM>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((merge_kernel<float, bf16, 1, NM>), grid, block, 0, st, p);
    } else if (p.out_dtype == CEA_F16) {
      if (vec == 4) hipLaunchKernelGGL((merge_kernel<float, f16, 4, NM>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((merge_kernel<float, f16, 1, NM>), grid, block, 0, st, p);
    } else {
      if (vec == 4) hipLaunchKernelGGL((merge_kernel<float, float, 4, NM>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((merge_kernel<float, float, 1, NM>), grid, block, 0, st, p);
    }
  };
  // registers for the partials a launch holds: few partials keep the kernel small (more
  // waves in flight for the large two-way merges of ring steps)
  if (p.n <= 2) go(std::integral_constant<int, 2>());
  else if (p.n <= 4) go(std::integral_constant<int, 4>());
  else go(std::integral_constant<int, CEA_MAX_PARTS>());
  CEA_CHECK_LAUNCH("merge");
  return CEA_OK;
}

}  // namespace cea
