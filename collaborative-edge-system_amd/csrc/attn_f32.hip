// f32 attention with LSE on gfx950 matrix cores (v_mfma_f32_16x16x4_f32, IEEE f32 products
// and sums).
//
// Computes what attention_with_lse (collab_infer/parallel/attention.py:201-239) returns for f32
// inputs - the reference's fp32 mode, whose CPU route runs torch's flash kernel in f32
// (attention.py:163-181): out[B,Sq,Hq,D] and the natural-log lse[B,Hq,Sq] over the keys visible
// under the position rule (attention.py:96-101), GQA head mapping, empty rows as (0, -inf), and
// the optional exact merge into a running (out, lse) (attention.py:242-250).
//
// Structure (one workgroup = 4 waves = 16 query rows of one head):
//   * the 16 rows are the columns of 16x16 matrix-core tiles; each wave walks every 4th 16-key
//     tile of the block (the key range split four ways), so a short sequence still spreads over
//     many waves, and the four partial (max, sum, output) results are merged exactly in LDS;
//   * S^T = K.Q^T per tile: D/4 products of 16x16x4, A = 16 keys x 4 features, B = 4 features x
//     16 queries.  The reduction over features may run in any order, so each lane loads its
//     row's features as 16-byte vectors (features 16j + 4g .. +3 for lane group g) and step
//     (j, t) reduces over feature 16j + 4g + t in both operands;
//   * the keys of the tile are placed on the accumulator rows in the order 4*(r%4) + r/4, which
//     puts key 4i + g in register i of lane group g: exactly the layout the value product's B
//     operand (4 keys x 16 queries, key 4i + g in lane group g) needs, so P goes from the score
//     registers into O^T += V^T.P^T without any lane exchange;
//   * V^T's rows (features) are placed likewise: lane c of a tile loads the D/16 consecutive
//     features c*D/16 .., output block m holds feature c*D/16 + m, so each lane ends up with
//     runs of D/16 consecutive output features and writes them as whole vectors;
//   * online softmax in natural-log units per query column: row statistics are combined over
//     the four lane groups with two lane exchanges; K, V and key positions of the next tile are
//     fetched while the current one is computed.
#include "cea_kernels.hpp"

namespace cea {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int QB = 16;        // query rows per workgroup
constexpr int KT = 16;        // keys per tile
constexpr int NW = 4;         // waves per workgroup, each taking every 4th tile
constexpr int NT = NW * 64;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 load4(const float* p) { return *(const f32x4*)p; }

template <int D>
struct F32Tile {
  f32x4 k[D / 16];        // lane (r, g): features 16j + 4g .. of key 4*(r%4) + r/4
  f32x4 v[4][D / 64];     // lane (c, g), k-block i: features c*D/16 .. of key 4i + g
  int64_t kp[4];          // positions of keys 4i + g (-1: padding or past the block)
};

template <int D>
__device__ __forceinline__ void load_tile(F32Tile<D>& t, const float* kb, const float* vb,
                                          const int64_t* kpb, int64_t ks, int64_t vs,
                                          int64_t kps, int key0, int Sk, int c16, int g) {
  const int kr = key0 + 4 * (c16 & 3) + (c16 >> 2);
#pragma unroll
  for (int j = 0; j < D / 16; ++j)
    t.k[j] = kr < Sk ? load4(kb + (int64_t)kr * ks + 16 * j + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = key0 + 4 * i + g;
#pragma unroll
    for (int u = 0; u < D / 64; ++u)
      t.v[i][u] = key < Sk ? load4(vb + (int64_t)key * vs + c16 * (D / 16) + 4 * u)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
    t.kp[i] = key < Sk ? kpb[(int64_t)key * kps] : -1;
  }
}

// max / sum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the 16-lane rows of one query column)
// by the gfx950 permlane swaps (no LDS round trip): each step combines the same two values
// in both lanes of a pair, so every lane holds the bitwise same result
__device__ __forceinline__ float xor_max(float x) {
  uint32_t u = __float_as_uint(x);
  auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  u = __float_as_uint(fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
  sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float xor_sum(float x) {
  uint32_t u = __float_as_uint(x);
  auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  u = __float_as_uint(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
  sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

template <int D>
__global__ __launch_bounds__(NT) void attn_f32_kernel(const AttnParams p) {
  constexpr int NB = D / 16;    // output feature blocks (value products per k-block)
  constexpr int RUN = D / 16;   // consecutive output features per lane and register
  __shared__ float red_m[NW][QB], red_l[NW][QB];
  __shared__ float red_o[NW][QB][D + 4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c16 = lane & 15;   // query column of the tiles / feature row block of V^T
  const int g = lane >> 4;     // k-group of the matrix instructions
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int kvh = p.map.kv_of(h);

  const int row = qb * QB + c16;
  const bool row_ok = row < p.Sq;
  const int64_t qpos = row_ok ? p.q_pos[b * p.qps_b + (int64_t)row * p.qps_s] : 0;
  const bool row_sees = row_ok && (!p.causal || qpos >= 0);
  const uint64_t qlim = p.causal ? (uint64_t)qpos : (uint64_t)INT64_MAX;
  const float scale = (float)p.scale;

  f32x4 qf[D / 16];
  {
    const float* qrow = (const float*)p.q + b * p.qs_b + (int64_t)row * p.qs_s + h * p.qs_h;
#pragma unroll
    for (int j = 0; j < D / 16; ++j)
      qf[j] = row_ok ? load4(qrow + 16 * j + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float* kb = (const float*)p.k + b * p.ks_b + kvh * p.ks_h;
  const float* vb = (const float*)p.v + b * p.vs_b + kvh * p.vs_h;
  const int64_t* kpb = p.k_pos + b * p.kps_b;

  f32x4 o[NB];
#pragma unroll
  for (int m = 0; m < NB; ++m) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff(), l_run = 0.f;

  const int ntiles = (p.Sk + KT - 1) / KT;
  F32Tile<D> cur, nxt;
  int t = wave;
  if (t < ntiles) load_tile<D>(cur, kb, vb, kpb, p.ks_s, p.vs_s, p.kps_s, t * KT, p.Sk, c16, g);
  for (; t < ntiles; t += NW) {
    const bool more = t + NW < ntiles;
    if (more) load_tile<D>(nxt, kb, vb, kpb, p.ks_s, p.vs_s, p.kps_s, (t + NW) * KT, p.Sk, c16, g);
    // visibility of keys 4i + g to this lane's query; padding keys (and keys past the block)
    // have position -1, which read as unsigned exceeds any causal limit
    bool vis[4];
    bool any = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vis[i] = row_sees && cur.kp[i] >= 0 && (uint64_t)cur.kp[i] <= qlim;
      any = any || vis[i];
    }
    if (__ballot(any) != 0) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < D / 16; ++j) {
        s = mfma4(cur.k[j][0], qf[j][0], s);
        s = mfma4(cur.k[j][1], qf[j][1], s);
        s = mfma4(cur.k[j][2], qf[j][2], s);
        s = mfma4(cur.k[j][3], qf[j][3], s);
      }
      float sc[4];
      float mx = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = vis[i] ? s[i] * scale : -__builtin_inff();
        mx = fmaxf(mx, sc[i]);
      }
      mx = xor_max(mx);
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
      const float alpha = expf(m_run - m_use);  // 0 while the row has seen nothing
      float pr[4];
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = expf(sc[i] - m_use);  // exactly 0 for hidden keys
        ls += pr[i];
      }
      l_run = l_run * alpha + xor_sum(ls);
      m_run = m_new;
#pragma unroll
      for (int m = 0; m < NB; ++m) o[m] *= alpha;
      // O^T += V^T . P^T over the four 4-key blocks of the tile
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < NB; ++m) o[m] = mfma4(cur.v[i][m / 4][m % 4], pr[i], o[m]);
    }
    if (more) cur = nxt;
  }

  // ---- merge the four waves' partial results (exact: common reference max)
  if (g == 0) {
    red_m[wave][c16] = m_run;
    red_l[wave][c16] = l_run;
  }
  // lane (c16, g), block m, register r holds feature (4g + r) * RUN + m of query c16
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < NB; ++m) red_o[wave][c16][(4 * g + r) * RUN + m] = o[m][r];
  __syncthreads();

  const int qq = tid >> 4;           // query of the block this thread finishes
  const int f0 = (tid & 15) * RUN;   // its RUN consecutive features
  const int orow = qb * QB + qq;
  if (orow >= p.Sq) return;
  float M = -__builtin_inff();
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][qq]);
  const float Mu = M == -__builtin_inff() ? 0.f : M;
  float wgt[NW];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    wgt[w] = expf(red_m[w][qq] - Mu);  // 0 for a wave that saw nothing
    L += red_l[w][qq] * wgt[w];
  }
  const bool empty = !(L > 0.f);
  const float inv = empty ? 0.f : 1.f / L;
  const float lse_new = empty ? -__builtin_inff() : M + logf(L);
  float on[RUN];
#pragma unroll
  for (int e = 0; e < RUN; ++e) {
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a += red_o[w][qq][f0 + e] * wgt[w];
    on[e] = empty ? 0.f : a * inv;
  }
  float* op = (float*)p.out + b * p.os_b + (int64_t)orow * p.os_s + h * p.os_h + f0;
  float* lp = p.lse ? (float*)p.lse + b * p.ls_b + h * p.ls_h + (int64_t)orow * p.ls_s : nullptr;
  if (p.accumulate) {
    const float lse_old = *lp;
    const float lse = logaddexp<float>(lse_old, lse_new);
    const float safe = is_finite(lse) ? lse : 0.f;
    const float w_old = expf(lse_old - safe), w_new = expf(lse_new - safe);
#pragma unroll
    for (int e = 0; e < RUN; e += 4) {
      f32x4 prev = load4(op + e);
#pragma unroll
      for (int c = 0; c < 4; ++c) prev[c] = add_rn(mul_rn(prev[c], w_old), mul_rn(on[e + c], w_new));
      *(f32x4*)(op + e) = prev;
    }
    // the 16 threads of a row are lanes of one wave and read lse_old in the same instruction,
    // before the value this store writes is computed from it
    __builtin_amdgcn_wave_barrier();
    if ((tid & 15) == 0) *lp = lse;
  } else {
#pragma unroll
    for (int e = 0; e < RUN; e += 4)
      *(f32x4*)(op + e) = f32x4{on[e], on[e + 1], on[e + 2], on[e + 3]};
    if (lp && (tid & 15) == 0) *lp = lse_new;
  }
}

template <int D>
int launch_f32(const AttnParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.Sq + QB - 1) / QB), (unsigned)p.Hq, (unsigned)p.B);
  hipLaunchKernelGGL((attn_f32_kernel<D>), grid, dim3(NT), 0, st, p);
  CEA_CHECK_LAUNCH("attention_f32");
  return CEA_OK;
}

}  // namespace

static bool al16f(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

bool f32_mfma_supported(const AttnParams& p) {
  if (p.in_dtype != CEA_F32 || p.out_dtype != CEA_F32) return false;
  if (!(p.D == 64 || p.D == 128)) return false;
  if (p.final_out) return false;
  if (p.B >= 65536 || p.Hq >= 65536) return false;
  if (!std::isfinite(p.scale)) return false;
  // 16-byte vector loads of q, k, v rows and stores of out rows
  const int64_t s4[] = {p.qs_b, p.qs_s, p.qs_h, p.ks_b, p.ks_s, p.ks_h,
                        p.vs_b, p.vs_s, p.vs_h, p.os_b, p.os_s, p.os_h};
  for (int64_t s : s4)
    if (s % 4) return false;
  return al16f(p.q) && al16f(p.k) && al16f(p.v) && al16f(p.out);
}

int launch_attn_f32_mfma(const AttnParams& p, hipStream_t st) {
  if (p.B == 0 || p.Sq == 0 || p.Hq == 0) return CEA_OK;
  if (p.D == 64) return launch_f32<64>(p, st);
  if (p.D == 128) return launch_f32<128>(p, st);
  set_error("attention: f32 matrix-core path does not cover head size %d", p.D);
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
