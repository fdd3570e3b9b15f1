// Attention with LSE for any element type (f32 / f64 / bf16 / f16) and head size up to 256.
//
// This is the kernel behind the f32 and f64 modes of attention_with_lse
// (collab_infer/parallel/attention.py:201-239, the CPU flash path _flash_lse :163-181 and
// the math path _math_lse :184-198) and behind shapes the MFMA kernel does not tile
// (head sizes other than 64/128).  One thread owns one query row; key/value tiles are
// staged through LDS in the accumulation type and every visible key updates the row's
// online softmax in natural-log units, so the LSE it returns is log(sum(exp(scale*q.k))).
//
// It also hosts the key-tile summary pre-pass used by the MFMA prefill kernel.
#include "cea_kernels.hpp"

namespace cea {

// ---------------------------------------------------------------------------------------
// tile summaries: for every 64-key tile, the range of valid positions and their count
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void tile_info_kernel(const int64_t* __restrict__ k_pos,
                                                       int64_t kps_b, int64_t kps_s, int Sk,
                                                       int ntiles, TileInfo* __restrict__ out) {
  const int t = blockIdx.x, b = blockIdx.y;
  const int key = t * kTileKeys + threadIdx.x;
  int64_t p = -1;
  if (key < Sk) p = k_pos[b * kps_b + (int64_t)key * kps_s];
  const bool valid = p >= 0;
  const int64_t mn = wave_min_i64(valid ? p : INT64_MAX);
  const int64_t mx = wave_max_i64(valid ? p : INT64_MIN);
  const int cnt = wave_sum_i32(valid ? 1 : 0);
  if (threadIdx.x == 0) {
    TileInfo ti;
    ti.min_valid = mn;
    ti.max_valid = mx;
    ti.n_valid = cnt;
    ti.pad[0] = ti.pad[1] = ti.pad[2] = 0;
    out[(int64_t)b * ntiles + t] = ti;
  }
}

int launch_tile_info(const int64_t* k_pos, int64_t kps_b, int64_t kps_s, int32_t B, int32_t Sk,
                     TileInfo* tiles, int32_t ntiles, hipStream_t st) {
  if (B == 0 || ntiles == 0) return CEA_OK;
  CEA_REQUIRE(B < 65536, CEA_EUNSUPPORTED, "attention: batch %d too large", B);
  hipLaunchKernelGGL(tile_info_kernel, dim3(ntiles, B), dim3(64), 0, st, k_pos, kps_b, kps_s, Sk,
                     ntiles, tiles);
  CEA_CHECK_LAUNCH("tile_info");
  return CEA_OK;
}

// The same summaries for every block of a segment table: tile t of the launch's numbering
// belongs to the last block whose first tile is <= t.
__global__ __launch_bounds__(64) void tile_info_segs_kernel(const KvSegs segs, int ntiles,
                                                            TileInfo* __restrict__ out) {
  const int t = blockIdx.x, b = blockIdx.y;
  int s = 0;
  while (s + 1 < segs.n && t >= segs.seg[s + 1].tile0) ++s;
  const KvSeg& g = segs.seg[s];
  const int key = (t - g.tile0) * kTileKeys + threadIdx.x;
  int64_t p = -1;
  if (key < g.Sk) p = g.k_pos[b * g.kps_b + (int64_t)key * g.kps_s];
  const bool valid = p >= 0;
  const int64_t mn = wave_min_i64(valid ? p : INT64_MAX);
  const int64_t mx = wave_max_i64(valid ? p : INT64_MIN);
  const int cnt = wave_sum_i32(valid ? 1 : 0);
  if (threadIdx.x == 0) {
    TileInfo ti;
    ti.min_valid = mn;
    ti.max_valid = mx;
    ti.n_valid = cnt;
    ti.pad[0] = ti.pad[1] = ti.pad[2] = 0;
    out[(int64_t)b * ntiles + t] = ti;
  }
}

int launch_tile_info_segs(const KvSegs& segs, int32_t B, TileInfo* tiles, int32_t ntiles,
                          hipStream_t st) {
  if (B == 0 || ntiles == 0) return CEA_OK;
  CEA_REQUIRE(B < 65536, CEA_EUNSUPPORTED, "attention: batch %d too large", B);
  hipLaunchKernelGGL(tile_info_segs_kernel, dim3(ntiles, B), dim3(64), 0, st, segs, ntiles, tiles);
  CEA_CHECK_LAUNCH("tile_info");
  return CEA_OK;
}

// ---------------------------------------------------------------------------------------
// generic attention
// ---------------------------------------------------------------------------------------
template <typename T, typename A, typename O, int DMAX, int KT>
__global__ __launch_bounds__(64) void attn_generic_kernel(const AttnParams p) {
  __shared__ A ks[KT][DMAX];
  __shared__ A vs[KT][DMAX];
  __shared__ int64_t kp[KT];

  const int b = blockIdx.z, h = blockIdx.y;
  const int row = blockIdx.x * 64 + threadIdx.x;
  const bool active = row < p.Sq;
  const int kvh = p.map.kv_of(h);
  const int D = p.D;
  const A scale = (A)p.scale;

  const T* qp = (const T*)p.q + b * p.qs_b + (int64_t)row * p.qs_s + h * p.qs_h;
  const T* kbase = (const T*)p.k + b * p.ks_b + kvh * p.ks_h;
  const T* vbase = (const T*)p.v + b * p.vs_b + kvh * p.vs_h;
  const int64_t* kpos = p.k_pos + b * p.kps_b;

  A q[DMAX], o[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    q[d] = (active && d < D) ? load_acc<T, A>(qp + d) : (A)0;
    o[d] = 0;
  }
  const int64_t qpos = active ? p.q_pos[b * p.qps_b + (int64_t)row * p.qps_s] : 0;
  A m = neg_inf<A>(), l = 0;

  for (int k0 = 0; k0 < p.Sk; k0 += KT) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < KT * D; idx += 64) {
      const int j = idx / D, d = idx % D;
      const int key = k0 + j;
      A kv = 0, vv = 0;
      if (key < p.Sk) {
        kv = load_acc<T, A>(kbase + (int64_t)key * p.ks_s + d);
        vv = load_acc<T, A>(vbase + (int64_t)key * p.vs_s + d);
      }
      ks[j][d] = kv;
      vs[j][d] = vv;
    }
    for (int j = threadIdx.x; j < KT; j += 64) {
      const int key = k0 + j;
      kp[j] = key < p.Sk ? kpos[(int64_t)key * p.kps_s] : -1;
    }
    __syncthreads();
    if (!active) continue;
    const int nk = p.Sk - k0 < KT ? p.Sk - k0 : KT;
    for (int j = 0; j < nk; ++j) {
      const int64_t kpj = kp[j];
      if (kpj < 0 || (p.causal && kpj > qpos)) continue;
      A s = 0;
#pragma unroll
      for (int d = 0; d < DMAX; ++d)
        if (d < D) s += q[d] * ks[j][d];
      s *= scale;
      if (s > m) {
        const A c = exp_acc(m - s);  // m == -inf gives 0
        l *= c;
#pragma unroll
        for (int d = 0; d < DMAX; ++d) o[d] *= c;
        m = s;
      }
      const A e = exp_acc(s - m);
      l += e;
#pragma unroll
      for (int d = 0; d < DMAX; ++d)
        if (d < D) o[d] += e * vs[j][d];
    }
  }
  if (!active) return;

  // finalise: rows without a visible key are (0, -inf)
  const bool empty = !(l > (A)0);
  const A lse_new = empty ? neg_inf<A>() : m + log_acc(l);
  const A inv = empty ? (A)0 : (A)1 / l;
  O* op = (O*)p.out + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
  A* lp = p.lse ? (A*)p.lse + b * p.ls_b + h * p.ls_h + (int64_t)row * p.ls_s : nullptr;
  if (p.accumulate) {
    // exact merge with the running result, as merge_attention does
    const A lse_old = *lp;
    const A lse = logaddexp<A>(lse_old, lse_new);
    const A safe = is_finite(lse) ? lse : (A)0;
    const A w_old = exp_acc(lse_old - safe), w_new = exp_acc(lse_new - safe);
#pragma unroll
    for (int d = 0; d < DMAX; ++d) {
      if (d < D) {
        const A on = empty ? (A)0 : o[d] * inv;
        const A prev = (A)op[d];
        op[d] = (O)add_rn(mul_rn(prev, w_old), mul_rn(on, w_new));
      }
    }
    *lp = lse;
  } else {
#pragma unroll
    for (int d = 0; d < DMAX; ++d)
      if (d < D) op[d] = (O)(empty ? (A)0 : o[d] * inv);
    if (lp) *lp = lse_new;
  }
}

template <typename T, typename A, typename O, int DMAX>
static void launch_generic_d(const AttnParams& p, hipStream_t st) {
  constexpr int KT = (DMAX * sizeof(A) * 2 * 32 <= 48 * 1024) ? 32 : 16;
  dim3 grid((p.Sq + 63) / 64, p.Hq, p.B);
  hipLaunchKernelGGL((attn_generic_kernel<T, A, O, DMAX, KT>), grid, dim3(64), 0, st, p);
}

template <typename T, typename A, typename O>
static int launch_generic_typed(const AttnParams& p, hipStream_t st) {
  if (p.D <= 16) launch_generic_d<T, A, O, 16>(p, st);
  else if (p.D <= 32) launch_generic_d<T, A, O, 32>(p, st);
  else if (p.D <= 64) launch_generic_d<T, A, O, 64>(p, st);
  else if (p.D <= 128) launch_generic_d<T, A, O, 128>(p, st);
  else if (p.D <= 256) launch_generic_d<T, A, O, 256>(p, st);
  else {
    set_error("attention: head size %d > 256 is not supported", p.D);
    return CEA_EUNSUPPORTED;
  }
  CEA_CHECK_LAUNCH("attention_generic");
  return CEA_OK;
}

int launch_attn_generic(const AttnParams& p, hipStream_t st) {
  if (p.B == 0 || p.Sq == 0 || p.Hq == 0) return CEA_OK;
  CEA_REQUIRE(p.Hq < 65536 && p.B < 65536, CEA_EUNSUPPORTED, "attention: grid too large");
  const int it = p.in_dtype, ot = p.out_dtype;
  if (it == CEA_F32) return launch_generic_typed<float, float, float>(p, st);
  if (it == CEA_F64) return launch_generic_typed<double, double, double>(p, st);
  if (it == CEA_BF16 && ot == CEA_F32) return launch_generic_typed<bf16, float, float>(p, st);
  if (it == CEA_BF16 && ot == CEA_BF16) return launch_generic_typed<bf16, float, bf16>(p, st);
  if (it == CEA_F16 && ot == CEA_F32) return launch_generic_typed<f16, float, float>(p, st);
  if (it == CEA_F16 && ot == CEA_F16) return launch_generic_typed<f16, float, f16>(p, st);
  set_error("attention: unsupported dtypes in=%s out=%s", dtype_name(it), dtype_name(ot));
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
