// LLaMA-family layer ops, HBM-bound, with the reference's rounding points.
//
//   RMSNorm        collab_infer/models/llama.py:52-61
//   rotary tables  collab_infer/models/llama.py:64-77 (inv_freq: models/config.py:165-189)
//   apply_rotary   collab_infer/models/llama.py:80-88 (half-split, NeoX/HF convention)
//   gated act      collab_infer/models/llama.py:44-49, 305, 316 (silu, gelu, gelu_pytorch_tanh,
//                  relu)
//
// Rounding: the reference runs separate tensor ops, each rounding to the tensor dtype.  The
// kernels keep every such rounding point (x*r -> T, w*that -> out dtype; x*cos -> T,
// rot*sin -> T, sum -> T; silu -> T, silu*up -> T) and compute between them in f32
// (f64 for f64 tensors), so a fused kernel returns what the op sequence returns.
#include "cea_kernels.hpp"

namespace cea {

// ---------------------------------------------------------------------------------------
// vector I/O: VEC elements of T as one 16-byte access when VEC * sizeof(T) == 16
// ---------------------------------------------------------------------------------------
template <typename T, int VEC> struct Vec {
  T v[VEC];
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, T (&out)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) {
    const uint4 raw = *(const uint4*)p;
    __builtin_memcpy(out, &raw, 16);
  } else if constexpr (VEC * sizeof(T) == 8) {
    const uint2 raw = *(const uint2*)p;
    __builtin_memcpy(out, &raw, 8);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = p[e];
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const T (&in)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) {
    uint4 raw;
    __builtin_memcpy(&raw, in, 16);
    *(uint4*)p = raw;
  } else if constexpr (VEC * sizeof(T) == 8) {
    uint2 raw;
    __builtin_memcpy(&raw, in, 8);
    *(uint2*)p = raw;
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) p[e] = in[e];
  }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Non-temporal store for output written exactly once (streamed past the caches; measured
// faster than plain stores for the row and elementwise passes here, while their loads are
// fastest as plain loads); 16-byte vectors only, plain stores otherwise.
template <typename T, int VEC>
__device__ __forceinline__ void store_vec_stream(T* p, const T (&in)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) {
    u32x4_t raw;
    __builtin_memcpy(&raw, in, 16);
    __builtin_nontemporal_store(raw, (u32x4_t*)p);
  } else {
    store_vec<T, VEC>(p, in);
  }
}

template <typename T> struct math_of { typedef float type; };
template <> struct math_of<double> { typedef double type; };

template <typename T, typename M> __device__ __forceinline__ M widen(T x) {
  return (M)to_f32<T>(x);
}
template <> __device__ __forceinline__ double widen<double, double>(double x) { return x; }

template <typename T, typename M> __device__ __forceinline__ T narrow(M x) { return (T)x; }

// x rounded to bf16 (nearest even) and read back as f32 by one v_cvt_pk_bf16_f32 that puts
// the rounded value in the high half and a zero in the low half: the word is then exactly
// the f32 of that bf16, with no widening instruction (the compiler's own form of this
// conversion adds a v_perm_b32)
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(u) : "v"(x));
  return __uint_as_float(u);
}

// value after a round trip through T (identity when T is the math type)
template <typename T, typename M> __device__ __forceinline__ M rnd(M x) {
  if constexpr (sizeof(T) == sizeof(M)) return x;
  else if constexpr (__is_same(T, bf16) && __is_same(M, float)) return round_bf16(x);
  else return widen<T, M>(narrow<T, M>(x));
}

__device__ __forceinline__ float rsqrt_rn(float v) { return __fdiv_rn(1.0f, __fsqrt_rn(v)); }
__device__ __forceinline__ double rsqrt_rn(double v) { return __ddiv_rn(1.0, __dsqrt_rn(v)); }

template <typename M> __device__ __forceinline__ M block_sum_256(M v, M* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  M t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------------------
// RMSNorm: one 256-thread block per row; NV vectors per thread stay in registers between
// the reduction and the scaling pass (rows of up to 256*VEC*NV elements).
// ---------------------------------------------------------------------------------------
template <typename T, typename W, typename O, int VEC, int NV>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x, int64_t xs,
                                                      const W* __restrict__ w,
                                                      O* __restrict__ y, int64_t ys, int C,
                                                      double eps_d) {
  typedef typename math_of<T>::type M;
  __shared__ M red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * xs;
  O* yr = y + row * ys;
  T cache[NV][VEC];
  M ss = 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 256 + threadIdx.x) * VEC;
    if (c < C) {
      load_vec<T, VEC>(xr + c, cache[i]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const M h = widen<T, M>(cache[i][e]);
        ss += h * h;
      }
    }
  }
  for (int c = (NV * 256 + threadIdx.x) * VEC; c < C; c += 256 * VEC) {
    T tmp[VEC];
    load_vec<T, VEC>(xr + c, tmp);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const M h = widen<T, M>(tmp[e]);
      ss += h * h;
    }
  }
  ss = block_sum_256<M>(ss, red);
  const M eps = (M)eps_d;
  const M r = rsqrt_rn(add_rn(div_rn(ss, (M)C), eps));

  auto emit = [&](int c, const T (&xv)[VEC]) {
    W wv[VEC];
    load_vec<W, VEC>(w + c, wv);
    O ov[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const M yn = rnd<T, M>(mul_rn(widen<T, M>(xv[e]), r));  // (x * r).to(x.dtype)
      ov[e] = narrow<O, M>(mul_rn(widen<W, M>(wv[e]), yn));  // weight * that
    }
    store_vec<O, VEC>(yr + c, ov);
  };
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * 256 + threadIdx.x) * VEC;
    if (c < C) emit(c, cache[i]);
  }
  for (int c = (NV * 256 + threadIdx.x) * VEC; c < C; c += 256 * VEC) {
    T tmp[VEC];
    load_vec<T, VEC>(xr + c, tmp);
    emit(c, tmp);
  }
}

// ---------------------------------------------------------------------------------------
// rotary tables
// ---------------------------------------------------------------------------------------
template <typename M> __device__ __forceinline__ M pos_to(int64_t p) {
  return (M)(p < 0 ? 0 : p);  // positions.clamp(min=0).to(inv_freq.dtype)
}
__device__ __forceinline__ void sincos_acc(float a, float* s, float* c) {
  *s = sinf(a);
  *c = cosf(a);
}
__device__ __forceinline__ void sincos_acc(double a, double* s, double* c) {
  *s = sin(a);
  *c = cos(a);
}

template <typename T>
__global__ __launch_bounds__(256) void rope_tables_kernel(
    const int64_t* __restrict__ pos, int64_t ps_b, int64_t ps_s,
    const typename math_of<T>::type* __restrict__ inv_freq, T* __restrict__ cosb,
    T* __restrict__ sinb, int64_t cs_b, int64_t cs_s, int64_t ss_b, int64_t ss_s, int B, int S,
    int half) {
  typedef typename math_of<T>::type M;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * S * half;
  if (t >= total) return;
  const int j = (int)(t % half);
  const int64_t bs = t / half;
  const int s = (int)(bs % S);
  const int b = (int)(bs / S);
  const M f = mul_rn(pos_to<M>(pos[b * ps_b + s * ps_s]), inv_freq[j]);
  M sv, cv;
  sincos_acc(f, &sv, &cv);
  const T c = narrow<T, M>(cv), sn = narrow<T, M>(sv);
  T* cp = cosb + b * cs_b + s * cs_s;
  T* sp = sinb + b * ss_b + s * ss_s;
  cp[j] = c;
  cp[j + half] = c;
  sp[j] = sn;
  sp[j + half] = sn;
}

// ---------------------------------------------------------------------------------------
// apply_rotary: out = x*cos + rotate_half(x)*sin; one thread owns VEC features of the first
// half and the matching VEC features of the second half of one (b, s, h) row.
// ---------------------------------------------------------------------------------------
template <typename T, typename M, int VEC>
__device__ __forceinline__ void rotate_pair(const T (&x1)[VEC], const T (&x2)[VEC],
                                            const T (&c1)[VEC], const T (&c2)[VEC],
                                            const T (&s1)[VEC], const T (&s2)[VEC],
                                            T (&o1)[VEC], T (&o2)[VEC]) {
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const M a1 = widen<T, M>(x1[e]), a2 = widen<T, M>(x2[e]);
    // first half: x1*cos + (-x2)*sin ; second half: x2*cos + x1*sin
    const M p1 = rnd<T, M>(mul_rn(a1, widen<T, M>(c1[e])));
    // (-x2)*sin rounds to the negation of x2*sin (round-to-nearest-even is symmetric)
    const M q1 = -rnd<T, M>(mul_rn(a2, widen<T, M>(s1[e])));
    const M p2 = rnd<T, M>(mul_rn(a2, widen<T, M>(c2[e])));
    const M q2 = rnd<T, M>(mul_rn(a1, widen<T, M>(s2[e])));
    o1[e] = narrow<T, M>(add_rn(p1, q1));
    o2[e] = narrow<T, M>(add_rn(p2, q2));
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void apply_rotary_kernel(
    const T* __restrict__ x, int64_t xs_b, int64_t xs_s, int64_t xs_h,
    const T* __restrict__ cosb, int64_t cs_b, int64_t cs_s, const T* __restrict__ sinb,
    int64_t ss_b, int64_t ss_s, T* __restrict__ out, int64_t os_b, int64_t os_s, int64_t os_h,
    int B, int S, int H, int D) {
  typedef typename math_of<T>::type M;
  const int half = D / 2;
  const int nch = half / VEC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * S * H * nch;
  if (t >= total) return;
  const int j = (int)(t % nch) * VEC;
  int64_t r = t / nch;
  const int h = (int)(r % H);
  r /= H;
  const int s = (int)(r % S);
  const int b = (int)(r / S);
  const T* xr = x + b * xs_b + s * xs_s + h * xs_h;
  const T* cr = cosb + b * cs_b + s * cs_s;
  const T* sr = sinb + b * ss_b + s * ss_s;
  T x1[VEC], x2[VEC], c1[VEC], c2[VEC], s1[VEC], s2[VEC], o1[VEC], o2[VEC];
  load_vec<T, VEC>(xr + j, x1);
  load_vec<T, VEC>(xr + j + half, x2);
  load_vec<T, VEC>(cr + j, c1);
  load_vec<T, VEC>(cr + j + half, c2);
  load_vec<T, VEC>(sr + j, s1);
  load_vec<T, VEC>(sr + j + half, s2);
  rotate_pair<T, M, VEC>(x1, x2, c1, c2, s1, s2, o1, o2);
  T* orow = out + b * os_b + s * os_s + h * os_h;
  store_vec<T, VEC>(orow + j, o1);
  store_vec<T, VEC>(orow + j + half, o2);
}

// ---------------------------------------------------------------------------------------
// KV-cache append: token-major k, v [B,n,H,D] (k optionally rotated first, exactly as
// apply_rotary) written into head-major caches [B,H,cap,D] at slots offset..offset+n, and
// the positions into [B,cap].  One thread owns VEC features of the first half and the
// matching VEC of the second half of one (b, token, head) row, for k and for v.
// ---------------------------------------------------------------------------------------
template <typename T, int VEC, bool ROT>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const T* __restrict__ k, int64_t ks_b, int64_t ks_s, int64_t ks_h,
    const T* __restrict__ v, int64_t vs_b, int64_t vs_s, int64_t vs_h,
    const T* __restrict__ cosb, int64_t cs_b, int64_t cs_s, const T* __restrict__ sinb,
    int64_t ss_b, int64_t ss_s, const int64_t* __restrict__ pos, int64_t ps_b, int64_t ps_s,
    T* __restrict__ ck, int64_t cks_b, int64_t cks_h, int64_t cks_s,
    T* __restrict__ cv, int64_t cvs_b, int64_t cvs_h, int64_t cvs_s,
    int64_t* __restrict__ cpos, int64_t cps_b, int64_t cps_s, int64_t offset, int B, int n,
    int H, int D) {
  typedef typename math_of<T>::type M;
  const int half = D / 2;
  const int nch = half / VEC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * n * H * nch;
  if (t >= total) return;
  const int j = (int)(t % nch) * VEC;
  int64_t r = t / nch;
  const int h = (int)(r % H);
  r /= H;
  const int s = (int)(r % n);
  const int b = (int)(r / n);
  const int64_t slot = offset + s;
  const T* kr = k + b * ks_b + s * ks_s + h * ks_h;
  const T* vr = v + b * vs_b + s * vs_s + h * vs_h;
  T* ckr = ck + b * cks_b + h * cks_h + slot * cks_s;
  T* cvr = cv + b * cvs_b + h * cvs_h + slot * cvs_s;
  T k1[VEC], k2[VEC], v1[VEC], v2[VEC];
  load_vec<T, VEC>(kr + j, k1);
  load_vec<T, VEC>(kr + j + half, k2);
  load_vec<T, VEC>(vr + j, v1);
  load_vec<T, VEC>(vr + j + half, v2);
  if constexpr (ROT) {
    const T* cr = cosb + b * cs_b + s * cs_s;
    const T* sr = sinb + b * ss_b + s * ss_s;
    T c1[VEC], c2[VEC], s1[VEC], s2[VEC], o1[VEC], o2[VEC];
    load_vec<T, VEC>(cr + j, c1);
    load_vec<T, VEC>(cr + j + half, c2);
    load_vec<T, VEC>(sr + j, s1);
    load_vec<T, VEC>(sr + j + half, s2);
    rotate_pair<T, M, VEC>(k1, k2, c1, c2, s1, s2, o1, o2);
    store_vec<T, VEC>(ckr + j, o1);
    store_vec<T, VEC>(ckr + j + half, o2);
  } else {
    store_vec<T, VEC>(ckr + j, k1);
    store_vec<T, VEC>(ckr + j + half, k2);
  }
  store_vec<T, VEC>(cvr + j, v1);
  store_vec<T, VEC>(cvr + j + half, v2);
  if (h == 0 && j == 0) cpos[b * cps_b + slot * cps_s] = pos[b * ps_b + s * ps_s];
}

// ---------------------------------------------------------------------------------------
// fused RMSNorm + rotary: one 256-thread block per token row of H*D features.  The row's
// rotary tables (D/2 angles) are evaluated once into LDS; every feature pair (j, j+D/2) of
// every head is normalised, weighted and rotated in registers.
// ---------------------------------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(
    const T* __restrict__ x, int64_t xs, const T* __restrict__ w, const int64_t* __restrict__ pos,
    int64_t ps, const typename math_of<T>::type* __restrict__ inv_freq, T* __restrict__ out,
    int64_t os, int H, int D, double eps_d) {
  typedef typename math_of<T>::type M;
  __shared__ M red[4];
  __shared__ T tab_c[512];
  __shared__ T tab_s[512];
  const int64_t row = blockIdx.x;
  const int C = H * D;
  const int half = D / 2;
  const T* xr = x + row * xs;
  T* orow = out + row * os;

  M ss = 0;
  for (int c = threadIdx.x * VEC; c < C; c += 256 * VEC) {
    T v[VEC];
    load_vec<T, VEC>(xr + c, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const M h = widen<T, M>(v[e]);
      ss += h * h;
    }
  }
  const M pf = pos_to<M>(pos[row * ps]);
  for (int j = threadIdx.x; j < half; j += 256) {
    M sv, cv;
    sincos_acc(mul_rn(pf, inv_freq[j]), &sv, &cv);
    tab_c[j] = narrow<T, M>(cv);
    tab_s[j] = narrow<T, M>(sv);
  }
  ss = block_sum_256<M>(ss, red);  // contains the barrier that publishes the tables
  const M r = rsqrt_rn(add_rn(div_rn(ss, (M)C), (M)eps_d));

  const int nch = half / VEC;
  for (int it = threadIdx.x; it < H * nch; it += 256) {
    const int h = it / nch;
    const int j = (it % nch) * VEC;
    const int c1 = h * D + j, c2 = c1 + half;
    T x1[VEC], x2[VEC], w1[VEC], w2[VEC], y1[VEC], y2[VEC], cs[VEC], sn[VEC], o1[VEC], o2[VEC];
    load_vec<T, VEC>(xr + c1, x1);
    load_vec<T, VEC>(xr + c2, x2);
    load_vec<T, VEC>(w + c1, w1);
    load_vec<T, VEC>(w + c2, w2);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      y1[e] = narrow<T, M>(mul_rn(widen<T, M>(w1[e]),
                                  rnd<T, M>(mul_rn(widen<T, M>(x1[e]), r))));
      y2[e] = narrow<T, M>(mul_rn(widen<T, M>(w2[e]),
                                  rnd<T, M>(mul_rn(widen<T, M>(x2[e]), r))));
      cs[e] = tab_c[j + e];
      sn[e] = tab_s[j + e];
    }
    rotate_pair<T, M, VEC>(y1, y2, cs, cs, sn, sn, o1, o2);
    store_vec<T, VEC>(orow + c1, o1);
    store_vec<T, VEC>(orow + c2, o2);
  }
}

// Single-pass variant for rows of at most 256 feature-pair chunks (e.g. 32 heads x 128) and
// D <= 512: a block takes R consecutive rows and every thread owns the same VEC-wide pair
// chunk (j, j + D/2 of one head) of each of them, in the sum of squares and in the output.
// x is read from memory once and kept in registers, the weight chunk is loaded once for the
// R rows, and the output is written non-temporally (measured: plain loads with streaming
// stores beat every other combination for this read-once, write-once row pass).  The position and frequency loads of the
// rotary table entries are issued ahead of the row loads (loads complete in order), so
// the table evaluation overlaps the row loads instead of waiting behind them.
// ---- bf16 pairs for the fused row kernel: one v_cvt_pk_bf16_f32 rounds two f32 values to
// bf16 (nearest even); the low half widens back with a shift, the high half with a mask
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

template <typename T, int VEC, int R>
__global__ __launch_bounds__(256) void rmsnorm_rope_rows_kernel(
    const T* __restrict__ x, int64_t xs, const T* __restrict__ w, const int64_t* __restrict__ pos,
    int64_t ps, const typename math_of<T>::type* __restrict__ inv_freq, T* __restrict__ out,
    int64_t os, int64_t S, int H, int D, double eps_d) {
  typedef typename math_of<T>::type M;
  static_assert(VEC * sizeof(T) == 16, "16-byte chunks");
  constexpr int TE = (R * 256 + 255) / 256;  // table entries per thread (half <= 256)
  __shared__ M red[R][4];
  // the tables hold the T-rounded cos / sin widened back to M, ready for the products
  __shared__ __attribute__((aligned(16))) M tab_c[R][256];
  __shared__ __attribute__((aligned(16))) M tab_s[R][256];
  const int64_t row0 = (int64_t)blockIdx.x * R;
  const int C = H * D;
  const int half = D / 2;
  const int nch = half / VEC;
  const int it = threadIdx.x;
  const bool active = it < H * nch;
  const int h = active ? it / nch : 0;
  const int j = active ? (it % nch) * VEC : 0;
  const int c1 = h * D + j, c2 = c1 + half;

  M ang[TE];
#pragma unroll
  for (int k = 0; k < TE; ++k) {
    const int t = threadIdx.x + 256 * k;
    const int r = t / half, jj = t - r * half;
    ang[k] = (t < R * half && row0 + r < S) ? mul_rn(pos_to<M>(pos[(row0 + r) * ps]), inv_freq[jj])
                                           : (M)0;
  }
  __builtin_amdgcn_sched_barrier(0);
  T x1[R][VEC], x2[R][VEC], w1[VEC], w2[VEC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (active && row0 + r < S) {
      const T* xr = x + (row0 + r) * xs;
      load_vec<T, VEC>(xr + c1, x1[r]);
      load_vec<T, VEC>(xr + c2, x2[r]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x1[r][e] = x2[r][e] = T(0);
    }
  }
  if (active) {
    load_vec<T, VEC>(w + c1, w1);
    load_vec<T, VEC>(w + c2, w2);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < TE; ++k) {
    const int t = threadIdx.x + 256 * k;
    const int r = t / half, jj = t - r * half;
    if (t < R * half) {
      M sv, cv;
      sincos_acc(ang[k], &sv, &cv);
      tab_c[r][jj] = rnd<T, M>(cv);
      tab_s[r][jj] = rnd<T, M>(sv);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    M acc = 0;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const M a = widen<T, M>(x1[r][e]), b = widen<T, M>(x2[r][e]);
      if constexpr (__is_same(T, bf16) || __is_same(T, f16)) {
        // the square of an f16 value, or of a bf16 value of magnitude at least 2^-63, is
        // exact in f32, so one fma is the reference's h.pow(2) followed by the add
        acc = __builtin_fmaf(a, a, acc);
        acc = __builtin_fmaf(b, b, acc);
      } else {
        acc += a * a;
        acc += b * b;
      }
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[r][threadIdx.x >> 6] = acc;
  }
  __syncthreads();  // publishes the partial sums and the tables
  if (!active) return;
  if constexpr (__is_same(T, bf16)) {
    // the same rounding points, each one conversion that leaves the rounded value in f32;
    // x and the weight stay packed between uses (widened where read), which keeps the kernel
    // at 64 VGPRs: 8 waves per SIMD, the whole grid of a 4096-row call resident at once
    constexpr int NP = VEC / 2;
    uint32_t wp1[NP], wp2[NP];
    __builtin_memcpy(wp1, w1, 16);
    __builtin_memcpy(wp2, w2, 16);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r >= S) break;
      const M ss = red[r][0] + red[r][1] + red[r][2] + red[r][3];
      const float rs = rsqrt_rn(add_rn(div_rn(ss, (M)C), (M)eps_d));
      uint32_t xp1[NP], xp2[NP], o1[NP], o2[NP];
      __builtin_memcpy(xp1, x1[r], 16);
      __builtin_memcpy(xp2, x2[r], 16);
      float cf[VEC], sf[VEC];
#pragma unroll
      for (int e = 0; e < VEC; e += 4) {
        *(float4*)&cf[e] = *(const float4*)&tab_c[r][j + e];
        *(float4*)&sf[e] = *(const float4*)&tab_s[r][j + e];
      }
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        const float xa1[2] = {bf16_lo(xp1[q]), bf16_hi(xp1[q])}, xa2[2] = {bf16_lo(xp2[q]), bf16_hi(xp2[q])};
        const float wa1[2] = {bf16_lo(wp1[q]), bf16_hi(wp1[q])}, wa2[2] = {bf16_lo(wp2[q]), bf16_hi(wp2[q])};
        float r1[2], r2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          // RMSNorm: yn = (x * rs).to(bf16); y = (w * yn).to(bf16)
          const float y1 = round_bf16(mul_rn(wa1[u], round_bf16(mul_rn(xa1[u], rs))));
          const float y2 = round_bf16(mul_rn(wa2[u], round_bf16(mul_rn(xa2[u], rs))));
          const float cv = cf[2 * q + u], sv = sf[2 * q + u];
          // first half: (y1*cos).to(bf16) + (-y2*sin).to(bf16); second: y2*cos + y1*sin
          r1[u] = add_rn(round_bf16(mul_rn(y1, cv)), -round_bf16(mul_rn(y2, sv)));
          r2[u] = add_rn(round_bf16(mul_rn(y2, cv)), round_bf16(mul_rn(y1, sv)));
        }
        o1[q] = pack_bf16(r1[0], r1[1]);
        o2[q] = pack_bf16(r2[0], r2[1]);
      }
      T v1[VEC], v2[VEC];
      __builtin_memcpy(v1, o1, 16);
      __builtin_memcpy(v2, o2, 16);
      T* orow = out + (row0 + r) * os;
      store_vec_stream<T, VEC>(orow + c1, v1);
      store_vec_stream<T, VEC>(orow + c2, v2);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (row0 + r >= S) break;
    const M ss = red[r][0] + red[r][1] + red[r][2] + red[r][3];
    const M rs = rsqrt_rn(add_rn(div_rn(ss, (M)C), (M)eps_d));
    T y1[VEC], y2[VEC], cs[VEC], sn[VEC], o1[VEC], o2[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      y1[e] = narrow<T, M>(mul_rn(widen<T, M>(w1[e]), rnd<T, M>(mul_rn(widen<T, M>(x1[r][e]), rs))));
      y2[e] = narrow<T, M>(mul_rn(widen<T, M>(w2[e]), rnd<T, M>(mul_rn(widen<T, M>(x2[r][e]), rs))));
      cs[e] = narrow<T, M>(tab_c[r][j + e]);
      sn[e] = narrow<T, M>(tab_s[r][j + e]);
    }
    rotate_pair<T, M, VEC>(y1, y2, cs, cs, sn, sn, o1, o2);
    T* orow = out + (row0 + r) * os;
    store_vec_stream<T, VEC>(orow + c1, o1);
    store_vec_stream<T, VEC>(orow + c2, o2);
  }
}

// ---------------------------------------------------------------------------------------
// Gated activations: out = act(gate) * up, act(gate) rounded to T first (the reference's
// self.act(gate) * up, llama.py:44-49, 305: two separately rounded tensor ops; gate_act in
// cea_common.hpp computes the activation as torch's elementwise kernels do)
template <typename T, int VEC, int ACT>
__global__ __launch_bounds__(256) void gated_mul_kernel(const T* __restrict__ g, int64_t gs,
                                                        const T* __restrict__ u, int64_t us,
                                                        T* __restrict__ out, int64_t os,
                                                        int64_t N, int I) {
  // grid: x over VEC-wide chunks of a row, y over rows (strided when N exceeds the grid)
  typedef typename math_of<T>::type M;
  const int c = (int)(blockIdx.x * 256 + threadIdx.x) * VEC;
  if (c >= I) return;
  for (int64_t row = blockIdx.y; row < N; row += gridDim.y) {
    T gv[VEC], uv[VEC], ov[VEC];
    load_vec<T, VEC>(g + row * gs + c, gv);
    load_vec<T, VEC>(u + row * us + c, uv);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const M act = rnd<T, M>(gate_act<ACT, M>(widen<T, M>(gv[e])));
      ov[e] = narrow<T, M>(mul_rn(act, widen<T, M>(uv[e])));
    }
    store_vec_stream<T, VEC>(out + row * os + c, ov);
  }
}

// ---------------------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------------------
static bool al(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
static bool strides_ok(std::initializer_list<int64_t> s, size_t esz, size_t a) {
  for (int64_t v : s)
    if (((uint64_t)v * esz) % a) return false;
  return true;
}

template <typename T, typename W, typename O>
static int rmsnorm_typed(const cea_tensor* x, const cea_tensor* w, double eps, cea_tensor* y,
                         hipStream_t st) {
  const int64_t N = x->size[0];
  const int C = (int)x->size[1];
  if (N == 0 || C == 0) return CEA_OK;
  constexpr int VEC = 16 / sizeof(T) < 16 / sizeof(W) ? 16 / sizeof(T) : 16 / sizeof(W);
  const bool vec = C % VEC == 0 && al(x->data, 16) && al(w->data, 16) &&
                   al(y->data, VEC * sizeof(O)) && strides_ok({x->stride[0]}, sizeof(T), 16) &&
                   strides_ok({y->stride[0]}, sizeof(O), VEC * sizeof(O));
  CEA_REQUIRE(N < (int64_t)1 << 31, CEA_EUNSUPPORTED, "rmsnorm: too many rows");
  if (vec)
    hipLaunchKernelGGL((rmsnorm_kernel<T, W, O, VEC, 4>), dim3(N), dim3(256), 0, st,
                       (const T*)x->data, x->stride[0], (const W*)w->data, (O*)y->data,
                       y->stride[0], C, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<T, W, O, 1, 8>), dim3(N), dim3(256), 0, st,
                       (const T*)x->data, x->stride[0], (const W*)w->data, (O*)y->data,
                       y->stride[0], C, eps);
  CEA_CHECK_LAUNCH("rmsnorm");
  return CEA_OK;
}

int launch_rmsnorm(const cea_tensor* x, const cea_tensor* w, double eps, cea_tensor* y,
                   hipStream_t st) {
  const int xt = x->dtype, wt = w->dtype, yt = y->dtype;
  if (xt == CEA_BF16 && wt == CEA_BF16 && yt == CEA_BF16) return rmsnorm_typed<bf16, bf16, bf16>(x, w, eps, y, st);
  if (xt == CEA_F16 && wt == CEA_F16 && yt == CEA_F16) return rmsnorm_typed<f16, f16, f16>(x, w, eps, y, st);
  if (xt == CEA_F32 && wt == CEA_F32 && yt == CEA_F32) return rmsnorm_typed<float, float, float>(x, w, eps, y, st);
  if (xt == CEA_F64 && wt == CEA_F64 && yt == CEA_F64) return rmsnorm_typed<double, double, double>(x, w, eps, y, st);
  if (xt == CEA_BF16 && wt == CEA_F32 && yt == CEA_F32) return rmsnorm_typed<bf16, float, float>(x, w, eps, y, st);
  if (xt == CEA_F16 && wt == CEA_F32 && yt == CEA_F32) return rmsnorm_typed<f16, float, float>(x, w, eps, y, st);
  set_error("rmsnorm: unsupported dtype combination x=%s weight=%s y=%s", dtype_name(xt),
            dtype_name(wt), dtype_name(yt));
  return CEA_EUNSUPPORTED;
}

template <typename T>
static int rope_tables_typed(const cea_tensor* pos, const cea_tensor* inv, cea_tensor* c,
                             cea_tensor* s, hipStream_t st) {
  const int B = (int)pos->size[0], S = (int)pos->size[1];
  const int half = (int)inv->size[0];
  const int64_t total = (int64_t)B * S * half;
  if (total == 0) return CEA_OK;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((rope_tables_kernel<T>), dim3(blocks), dim3(256), 0, st,
                     (const int64_t*)pos->data, pos->stride[0], pos->stride[1],
                     (const typename math_of<T>::type*)inv->data, (T*)c->data, (T*)s->data,
                     c->stride[0], c->stride[1], s->stride[0], s->stride[1], B, S, half);
  CEA_CHECK_LAUNCH("rope_tables");
  return CEA_OK;
}

int launch_rope_tables(const cea_tensor* pos, const cea_tensor* inv, cea_tensor* c,
                       cea_tensor* s, hipStream_t st) {
  switch (c->dtype) {
    case CEA_BF16: return rope_tables_typed<bf16>(pos, inv, c, s, st);
    case CEA_F16: return rope_tables_typed<f16>(pos, inv, c, s, st);
    case CEA_F32: return rope_tables_typed<float>(pos, inv, c, s, st);
    case CEA_F64: return rope_tables_typed<double>(pos, inv, c, s, st);
  }
  set_error("rope_tables: unsupported table dtype %s", dtype_name(c->dtype));
  return CEA_EUNSUPPORTED;
}

template <typename T>
static int apply_rotary_typed(const cea_tensor* x, const cea_tensor* c, const cea_tensor* s,
                              cea_tensor* o, hipStream_t st) {
  const int B = (int)x->size[0], S = (int)x->size[1], H = (int)x->size[2], D = (int)x->size[3];
  const int half = D / 2;
  constexpr int V = 16 / sizeof(T);
  const bool vec = half % V == 0 && al(x->data, 16) && al(c->data, 16) && al(s->data, 16) &&
                   al(o->data, 16) &&
                   strides_ok({x->stride[0], x->stride[1], x->stride[2], c->stride[0],
                               c->stride[1], s->stride[0], s->stride[1], o->stride[0],
                               o->stride[1], o->stride[2], (int64_t)half},
                              sizeof(T), 16);
  const int vecw = vec ? V : 1;
  const int64_t total = (int64_t)B * S * H * (half / vecw);
  if (total == 0) return CEA_OK;
  const int64_t blocks = (total + 255) / 256;
#define CEA_ROT_ARGS                                                                      \
  (const T*)x->data, x->stride[0], x->stride[1], x->stride[2], (const T*)c->data,         \
      c->stride[0], c->stride[1], (const T*)s->data, s->stride[0], s->stride[1],         \
      (T*)o->data, o->stride[0], o->stride[1], o->stride[2], B, S, H, D
  if (vec)
    hipLaunchKernelGGL((apply_rotary_kernel<T, V>), dim3(blocks), dim3(256), 0, st, CEA_ROT_ARGS);
  else
    hipLaunchKernelGGL((apply_rotary_kernel<T, 1>), dim3(blocks), dim3(256), 0, st, CEA_ROT_ARGS);
#undef CEA_ROT_ARGS
  CEA_CHECK_LAUNCH("apply_rotary");
  return CEA_OK;
}

int launch_apply_rotary(const cea_tensor* x, const cea_tensor* c, const cea_tensor* s,
                        cea_tensor* o, hipStream_t st) {
  switch (x->dtype) {
    case CEA_BF16: return apply_rotary_typed<bf16>(x, c, s, o, st);
    case CEA_F16: return apply_rotary_typed<f16>(x, c, s, o, st);
    case CEA_F32: return apply_rotary_typed<float>(x, c, s, o, st);
    case CEA_F64: return apply_rotary_typed<double>(x, c, s, o, st);
  }
  set_error("apply_rotary: unsupported dtype %s", dtype_name(x->dtype));
  return CEA_EUNSUPPORTED;
}

template <typename T>
static int kv_append_typed(const cea_tensor* k, const cea_tensor* v, const cea_tensor* pos,
                           const cea_tensor* c, const cea_tensor* sn, cea_tensor* ck,
                           cea_tensor* cv, cea_tensor* cp, int64_t offset, hipStream_t st) {
  const int B = (int)k->size[0], n = (int)k->size[1], H = (int)k->size[2], D = (int)k->size[3];
  const int half = D / 2;
  const bool rot = c != nullptr;
  constexpr int V = 16 / sizeof(T);
  bool vec = half % V == 0 && al(k->data, 16) && al(v->data, 16) && al(ck->data, 16) &&
             al(cv->data, 16) &&
             strides_ok({k->stride[0], k->stride[1], k->stride[2], v->stride[0], v->stride[1],
                         v->stride[2], ck->stride[0], ck->stride[1], ck->stride[2],
                         cv->stride[0], cv->stride[1], cv->stride[2], (int64_t)half},
                        sizeof(T), 16);
  if (rot)
    vec = vec && al(c->data, 16) && al(sn->data, 16) &&
          strides_ok({c->stride[0], c->stride[1], sn->stride[0], sn->stride[1]}, sizeof(T), 16);
  const int vecw = vec ? V : 1;
  const int64_t total = (int64_t)B * n * H * (half / vecw);
  if (total == 0) return CEA_OK;
  const int64_t blocks = (total + 255) / 256;
  const T* cd = rot ? (const T*)c->data : nullptr;
  const T* sd = rot ? (const T*)sn->data : nullptr;
  const int64_t c0 = rot ? c->stride[0] : 0, c1 = rot ? c->stride[1] : 0;
  const int64_t s0 = rot ? sn->stride[0] : 0, s1 = rot ? sn->stride[1] : 0;
#define CEA_KV_ARGS                                                                          \
  (const T*)k->data, k->stride[0], k->stride[1], k->stride[2], (const T*)v->data,             \
      v->stride[0], v->stride[1], v->stride[2], cd, c0, c1, sd, s0, s1,                      \
      (const int64_t*)pos->data, pos->stride[0], pos->stride[1], (T*)ck->data, ck->stride[0], \
      ck->stride[1], ck->stride[2], (T*)cv->data, cv->stride[0], cv->stride[1],              \
      cv->stride[2], (int64_t*)cp->data, cp->stride[0], cp->stride[1], offset, B, n, H, D
  if (vec && rot)
    hipLaunchKernelGGL((kv_append_kernel<T, V, true>), dim3(blocks), dim3(256), 0, st, CEA_KV_ARGS);
  else if (vec)
    hipLaunchKernelGGL((kv_append_kernel<T, V, false>), dim3(blocks), dim3(256), 0, st, CEA_KV_ARGS);
  else if (rot)
    hipLaunchKernelGGL((kv_append_kernel<T, 1, true>), dim3(blocks), dim3(256), 0, st, CEA_KV_ARGS);
  else
    hipLaunchKernelGGL((kv_append_kernel<T, 1, false>), dim3(blocks), dim3(256), 0, st, CEA_KV_ARGS);
#undef CEA_KV_ARGS
  CEA_CHECK_LAUNCH("kv_append");
  return CEA_OK;
}

int launch_kv_append(const cea_tensor* k, const cea_tensor* v, const cea_tensor* pos,
                     const cea_tensor* c, const cea_tensor* sn, cea_tensor* ck, cea_tensor* cv,
                     cea_tensor* cp, int64_t offset, hipStream_t st) {
  switch (k->dtype) {
    case CEA_BF16: return kv_append_typed<bf16>(k, v, pos, c, sn, ck, cv, cp, offset, st);
    case CEA_F16: return kv_append_typed<f16>(k, v, pos, c, sn, ck, cv, cp, offset, st);
    case CEA_F32: return kv_append_typed<float>(k, v, pos, c, sn, ck, cv, cp, offset, st);
    case CEA_F64: return kv_append_typed<double>(k, v, pos, c, sn, ck, cv, cp, offset, st);
  }
  set_error("kv_append: unsupported dtype %s", dtype_name(k->dtype));
  return CEA_EUNSUPPORTED;
}

#ifndef CEA_RR_ROWS
#define CEA_RR_ROWS 2  // rows per block of the single-pass RMSNorm + rotary kernel
#endif

template <typename T>
static int rmsnorm_rope_typed(const cea_tensor* x, const cea_tensor* w, double eps,
                              const cea_tensor* pos, const cea_tensor* inv, int H,
                              cea_tensor* o, hipStream_t st) {
  const int64_t S = x->size[0];
  const int C = (int)x->size[1];
  const int D = C / H, half = D / 2;
  if (S == 0) return CEA_OK;
  constexpr int V = 16 / sizeof(T);
  const bool vec = half % V == 0 && al(x->data, 16) && al(w->data, 16) && al(o->data, 16) &&
                   strides_ok({x->stride[0], o->stride[0], (int64_t)half}, sizeof(T), 16);
  const int64_t ps = pos->ndim == 2 ? pos->stride[1] : pos->stride[0];
#define CEA_RR_ARGS                                                                    \
  (const T*)x->data, x->stride[0], (const T*)w->data, (const int64_t*)pos->data, ps,   \
      (const typename math_of<T>::type*)inv->data, (T*)o->data, o->stride[0], H, D, eps
  if (vec && H * (half / V) <= 256 && half <= 256) {
    constexpr int R = CEA_RR_ROWS;
    hipLaunchKernelGGL((rmsnorm_rope_rows_kernel<T, V, R>), dim3((unsigned)((S + R - 1) / R)),
                       dim3(256), 0, st, (const T*)x->data, x->stride[0], (const T*)w->data,
                       (const int64_t*)pos->data, ps, (const typename math_of<T>::type*)inv->data,
                       (T*)o->data, o->stride[0], S, H, D, eps);
  } else if (vec)
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, V>), dim3(S), dim3(256), 0, st, CEA_RR_ARGS);
  else
    hipLaunchKernelGGL((rmsnorm_rope_kernel<T, 1>), dim3(S), dim3(256), 0, st, CEA_RR_ARGS);
#undef CEA_RR_ARGS
  CEA_CHECK_LAUNCH("rmsnorm_rope");
  return CEA_OK;
}

int launch_rmsnorm_rope(const cea_tensor* x, const cea_tensor* w, double eps,
                        const cea_tensor* pos, const cea_tensor* inv, int H, cea_tensor* o,
                        hipStream_t st) {
  switch (x->dtype) {
    case CEA_BF16: return rmsnorm_rope_typed<bf16>(x, w, eps, pos, inv, H, o, st);
    case CEA_F16: return rmsnorm_rope_typed<f16>(x, w, eps, pos, inv, H, o, st);
    case CEA_F32: return rmsnorm_rope_typed<float>(x, w, eps, pos, inv, H, o, st);
    case CEA_F64: return rmsnorm_rope_typed<double>(x, w, eps, pos, inv, H, o, st);
  }
  set_error("rmsnorm_rope: unsupported dtype %s", dtype_name(x->dtype));
  return CEA_EUNSUPPORTED;
}

template <typename T, int ACT>
static int gated_mul_typed(const cea_tensor* g, const cea_tensor* u, cea_tensor* o,
                           hipStream_t st) {
  const int64_t N = g->size[0];
  const int I = (int)g->size[1];
  constexpr int V = 16 / sizeof(T);
  const bool vec = I % V == 0 && al(g->data, 16) && al(u->data, 16) && al(o->data, 16) &&
                   strides_ok({g->stride[0], u->stride[0], o->stride[0]}, sizeof(T), 16);
  const int vw = vec ? V : 1;
  if (N == 0 || I / vw == 0) return CEA_OK;
  const dim3 grid((unsigned)((I / vw + 255) / 256), (unsigned)(N < 65535 ? N : 65535));
  if (vec)
    hipLaunchKernelGGL((gated_mul_kernel<T, V, ACT>), grid, dim3(256), 0, st,
                       (const T*)g->data, g->stride[0], (const T*)u->data, u->stride[0],
                       (T*)o->data, o->stride[0], N, I);
  else
    hipLaunchKernelGGL((gated_mul_kernel<T, 1, ACT>), grid, dim3(256), 0, st,
                       (const T*)g->data, g->stride[0], (const T*)u->data, u->stride[0],
                       (T*)o->data, o->stride[0], N, I);
  CEA_CHECK_LAUNCH("gated_mul");
  return CEA_OK;
}

template <typename T>
static int gated_mul_act(const cea_tensor* g, const cea_tensor* u, cea_tensor* o, int act,
                         hipStream_t st) {
  switch (act) {
    case CEA_ACT_SILU: return gated_mul_typed<T, CEA_ACT_SILU>(g, u, o, st);
    case CEA_ACT_GELU: return gated_mul_typed<T, CEA_ACT_GELU>(g, u, o, st);
    case CEA_ACT_GELU_TANH: return gated_mul_typed<T, CEA_ACT_GELU_TANH>(g, u, o, st);
    case CEA_ACT_RELU: return gated_mul_typed<T, CEA_ACT_RELU>(g, u, o, st);
  }
  set_error("gated_mul: unknown activation %d", act);
  return CEA_EUNSUPPORTED;
}

int launch_gated_mul(const cea_tensor* g, const cea_tensor* u, cea_tensor* o, int act,
                     hipStream_t st) {
  switch (g->dtype) {
    case CEA_BF16: return gated_mul_act<bf16>(g, u, o, act, st);
    case CEA_F16: return gated_mul_act<f16>(g, u, o, act, st);
    case CEA_F32: return gated_mul_act<float>(g, u, o, act, st);
    case CEA_F64: return gated_mul_act<double>(g, u, o, act, st);
  }
  set_error("gated_mul: unsupported dtype %s", dtype_name(g->dtype));
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
