// Split-KV decode attention with LSE for short query blocks (decoding against a KV cache).
//
// Covers attention_with_lse (collab_infer/parallel/attention.py:201-239) when the query block
// is a few tokens, and the per-device compute of distributed_kv_attention
// (collab_infer/parallel/sequence_parallel.py:250-280): every KV partition's partial
// (out, lse) and their exact merge (merge_attention_list, attention.py:253-264), all on one
// device and in two launches.
//
// HBM-bound design:
//   * work item = (batch, kv head, key chunk of one partition); the NR = Sq*G query rows that
//     share the kv head (G query heads per kv head) are the columns of 16 x 16 matrix-core
//     tiles, so each K/V row is read from HBM once for all of them and the arithmetic stays
//     off the vector ALU: S = K.Q^T with v_mfma_f32_16x16x32 (a lane holds 4 keys of one
//     query row) and O^T += V^T.P^T with v_mfma_f32_16x16x16 (P is the score tile as is);
//   * every wave streams its own 16-key tiles of K and V straight into a private pair of LDS
//     buffers (buffer_load ... lds, one tile ahead, explicit vmcnt waits, no barriers); V is
//     read back transposed with ds_read_b64_tr_b16; both tiles are XOR-swizzled so the
//     fragment and transpose reads are free of LDS bank conflicts;
//   * key positions of the chunk are staged in LDS; 16-key tiles that no query row can see
//     are never loaded, and chunks past every valid key return after the position scan;
//   * the waves of a workgroup merge their online-softmax partials in LDS and write one
//     (o unnormalised, m, l) partial per chunk; the reduction kernel then merges the chunks
//     of each partition exactly (optionally emitting each partition's (out, lse)), merges the
//     partitions with the reference's logsumexp, and writes out (f32 or the query dtype) and
//     lse.
#include "cea_kernels.hpp"
#include "cea_lds_dma.hpp"

namespace cea {
namespace {

constexpr int DTHREADS = 256;
constexpr int NW = DTHREADS / 64;     // waves per workgroup
constexpr int TK = 16;                // keys per tile
constexpr int CHMAX = 1024;           // keys per chunk at most
constexpr int NTILE_MAX = CHMAX / TK;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold, log2 units

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

template <typename T> struct Mfma16;
template <> struct Mfma16<bf16> {
  typedef bf16x8 frag8;
  static __device__ __forceinline__ f32x4 qk(frag8 a, frag8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(s16x4 a, s16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ s16x4 pack(float a, float b, float c, float d) {
    bf16x4 v = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
    s16x4 r;
    __builtin_memcpy(&r, &v, 8);
    return r;
  }
};
template <> struct Mfma16<f16> {
  typedef f16x8 frag8;
  static __device__ __forceinline__ f32x4 qk(frag8 a, frag8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(s16x4 a, s16x4 b, f32x4 c) {
    f16x4 x, y;
    __builtin_memcpy(&x, &a, 8);
    __builtin_memcpy(&y, &b, 8);
    return __builtin_amdgcn_mfma_f32_16x16x16f16(x, y, c, 0, 0, 0);
  }
  static __device__ __forceinline__ s16x4 pack(float a, float b, float c, float d) {
    f16x4 v = {(f16)a, (f16)b, (f16)c, (f16)d};
    s16x4 r;
    __builtin_memcpy(&r, &v, 8);
    return r;
  }
};

template <int D> struct DLayout {
  static constexpr int ROW = D * 2;                 // bytes per key row
  static constexpr int TILE_BYTES = TK * ROW;       // one K or V tile
  static constexpr int BUF_BYTES = 2 * TILE_BYTES;  // K + V
  static constexpr int WAVE_BYTES = 2 * BUF_BYTES;  // double-buffered per wave
  static constexpr int LDS_BYTES = NW * WAVE_BYTES;
  static constexpr int LOADS = TILE_BYTES / 1024;   // direct loads per tensor per tile
};

__device__ __forceinline__ float max_halves(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

__device__ __forceinline__ int part_of(const DecodeParams& p, int chunk) {
  int part = 0;
  while (part + 1 < p.nparts && chunk >= p.chunk_begin[part + 1]) ++part;
  return part;
}

// Partial layout: [B][Hkv][total_chunks][NR][D + 2] floats: o (relative to m), m, l, where
// m is in natural-log units (max of scale*q.k) and l = sum exp(scale*q.k - m).
template <typename T, int D, int NR>
__global__ __launch_bounds__(DTHREADS, 2) void decode_split_kernel(const DecodeParams p) {
  typedef DLayout<D> L;
  typedef typename Mfma16<T>::frag8 frag8;
  extern __shared__ __attribute__((aligned(16))) char dsmem[];
  __shared__ int64_t kpos_s[CHMAX];
  __shared__ uint32_t tile_any[NTILE_MAX];
  __shared__ float red_m[NW][NR];
  __shared__ float red_l[NW][NR];

  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int part = part_of(p, chunk);
  const int lchunk = chunk - p.chunk_begin[part];
  const int Sk = p.Sk[part];
  const int key0 = lchunk * p.chunk;
  const int nkeys = min(p.chunk, Sk - key0);
  const int ntile = (nkeys + TK - 1) / TK;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int row = lane & 15;   // query row (MFMA column) of this lane
  const int grp = lane >> 4;   // 4-key group of the 16-key tile
  const int G = p.G;
  const int nreal = p.Sq * G;
  const int total_chunks = p.chunk_begin[p.nparts];
  float* part_out = p.partial + (((int64_t)b * p.Hkv + kvh) * total_chunks + chunk) * NR * (D + 2);

  // ---- query rows of this kv head: row r = (s, gi) -> head kvh*G + gi, position q_pos[b, s]
  const bool row_real = row < nreal;
  const int64_t qpos = row_real ? p.q_pos[b * p.qps_b + (int64_t)(row / G) * p.qps_s] : INT64_MIN;
  int64_t qmax = INT64_MIN;
  for (int r = 0; r < nreal; ++r) {
    const int64_t v = p.q_pos[b * p.qps_b + (int64_t)(r / G) * p.qps_s];
    qmax = v > qmax ? v : qmax;
  }

  // ---- positions of the chunk into LDS; which 16-key tiles have a visible key
  const int64_t* kp = p.k_pos[part] + b * p.kps[part][0];
  const int64_t kps = p.kps[part][1];
  for (int i = tid; i < nkeys; i += DTHREADS) kpos_s[i] = kp[(int64_t)(key0 + i) * kps];
  __syncthreads();
  for (int t0 = wave * 4; t0 < ntile; t0 += NW * 4) {
    const int k = t0 * TK + lane;
    bool vis = false;
    if (k < nkeys) {
      const int64_t pk = kpos_s[k];
      vis = pk >= 0 && (!p.causal || pk <= qmax);
    }
    const uint64_t bal = __ballot(vis);
    if (lane < 4 && t0 + lane < ntile) tile_any[t0 + lane] = (uint32_t)((bal >> (16 * lane)) & 0xffffu);
  }
  __syncthreads();
  bool any = false;
  for (int t = 0; t < ntile; ++t) any |= tile_any[t] != 0;
  if (!any) {
    if (tid < NR) {
      part_out[tid * (D + 2) + D] = -__builtin_inff();
      part_out[tid * (D + 2) + D + 1] = 0.f;
    }
    return;
  }

  // ---- this lane's Q fragments (B operand of S = K.Q^T), sign folded for a negative scale
  const float scale = (float)p.scale;
  const float c = fabsf(scale) * 1.4426950408889634f;  // exp2 units
  const float grow_thr = kRescaleLog2 / c;
  const uint32_t flip = scale < 0.f ? 0x80008000u : 0u;
  frag8 qf[D / 32];
  {
    const T* qrow = (const T*)p.q + b * p.qs_b + (int64_t)(row / G) * p.qs_s + (kvh * G + row % G) * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      u32x4 raw = {0, 0, 0, 0};
      if (row_real) raw = *(const u32x4*)(qrow + ks * 32 + grp * 8);
#pragma unroll
      for (int w = 0; w < 4; ++w) raw[w] ^= flip;
      __builtin_memcpy(&qf[ks], &raw, 16);
    }
  }

  // ---- per-lane constant offsets
  const char* kbase = (const char*)((const T*)p.k[part] + b * p.ks[part][0] + kvh * p.ks[part][2]);
  const char* vbase = (const char*)((const T*)p.v[part] + b * p.vs[part][0] + kvh * p.vs[part][2]);
  const uint32_t krow = (uint32_t)(p.ks[part][1] * sizeof(T)), vrow = (uint32_t)(p.vs[part][1] * sizeof(T));
  uint32_t k_voff[L::LOADS], v_voff[L::LOADS];
#pragma unroll
  for (int i = 0; i < L::LOADS; ++i) {
    const int r = i * (1024 / L::ROW) + lane / (L::ROW / 16);
    const int pg = lane % (L::ROW / 16);                   // physical 16-byte group
    k_voff[i] = r * krow + ((pg ^ (r & 15)) << 4);          // K: 16-byte groups ^ row
    const int lgv = ((((pg >> 1) ^ (r & 7)) << 1) | (pg & 1));  // V: 32-byte blocks ^ row
    v_voff[i] = r * vrow + (lgv << 4);
  }
  uint32_t k_raddr[D / 32];  // A operand of S: key 'row', features grp*8 + 32*ks
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) k_raddr[ks] = row * L::ROW + (((grp + 4 * ks) ^ (row & 15)) << 4);
  uint32_t v_raddr[D / 16];  // transposing reads: source lane s of group grp -> key grp*4 + s/4
  {
    const int vr = grp * 4 + (row >> 2);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      v_raddr[dt] = L::TILE_BYTES + vr * L::ROW + ((dt ^ (vr & 7)) << 5) + 8 * (row & 3);
  }

  char* wb = dsmem + wave * L::WAVE_BYTES;
  auto next_tile = [&](int t) -> int {
    for (t += NW; t < ntile; t += NW)
      if (tile_any[t]) return t;
    return -1;
  };
  auto load_tile = [&](int t, int buf) {
    const int k0 = key0 + t * TK;
    const uint32_t rows = (uint32_t)min(Sk - k0, TK);  // rows past the end of the keys read 0
    const i32x4 krs = make_rsrc(kbase + (int64_t)k0 * krow, (rows - 1) * krow + L::ROW);
    const i32x4 vrs = make_rsrc(vbase + (int64_t)k0 * vrow, (rows - 1) * vrow + L::ROW);
    char* kb = wb + buf * L::BUF_BYTES;
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) buffer_load_lds16(krs, kb + i * 1024, k_voff[i]);
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) buffer_load_lds16(vrs, kb + L::TILE_BYTES + i * 1024, v_voff[i]);
  };

  f32x4 o[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff(), m_use = 0.f, l_run = 0.f;

  auto compute = [&](int t, int buf) {
    const char* kb = wb + buf * L::BUF_BYTES;
    frag8 kf[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) kf[ks] = *(const frag8*)(kb + k_raddr[ks]);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) s = Mfma16<T>::qk(kf[ks], qf[ks], s);
    // lane holds keys t*16 + grp*4 + i of query row 'row'
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = t * TK + grp * 4 + i;
      const int64_t pk = k < nkeys ? kpos_s[k] : -1;
      const bool vis = row_real && pk >= 0 && (!p.causal || pk <= qpos);
      if (!vis) s[i] = -__builtin_inff();
    }
    float mx = __builtin_fmaxf(__builtin_fmaxf(s[0], s[1]), __builtin_fmaxf(s[2], s[3]));
    mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = max_halves(mx);
    const bool grow = mx > m_run + grow_thr;
    if (__ballot(grow) != 0) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? __builtin_amdgcn_exp2f((m_run - m_new) * c) : 1.f;
      m_run = m_new;
      m_use = m_run == -__builtin_inff() ? 0.f : m_run * c;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) o[dt] *= alpha;
    }
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c, -m_use));
    l_run += (pv[0] + pv[1]) + (pv[2] + pv[3]);
    const s16x4 pf = Mfma16<T>::pack(pv[0], pv[1], pv[2], pv[3]);
    s16x4 vf[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      vf[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(kb + v_raddr[dt]));
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) o[dt] = Mfma16<T>::pv(vf[dt], pf, o[dt]);
  };

  // ---- per-wave stream over its tiles (wave w: tiles w, w+NW, ...), one tile ahead
  {
    int t = next_tile(wave - NW);
    int buf = 0;
    if (t >= 0) load_tile(t, 0);
    while (t >= 0) {
      const int tn = next_tile(t);
      if (tn >= 0) {
        wait_lgkmcnt0();  // the previous tile's LDS reads of buffer buf^1 have completed
        load_tile(tn, buf ^ 1);
        wait_vmcnt<2 * L::LOADS>();  // tile t landed; tile tn may still be in flight
      } else {
        wait_vmcnt<0>();
      }
      compute(t, buf);
      t = tn;
      buf ^= 1;
    }
  }

  // ---- merge the waves of the workgroup and write the chunk partial
  float l_row = l_run + __shfl_xor(l_run, 16, 64);
  l_row = sum_halves(l_row);
  if (grp == 0 && row < NR) {
    red_m[wave][row] = m_run == -__builtin_inff() ? m_run : m_run * fabsf(scale);
    red_l[wave][row] = l_row;
  }
  float* red_o = (float*)wb;  // this wave's own buffer, no longer read by the tile loop
  if (row < NR) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red_o[row * D + dt * 16 + grp * 4 + i] = o[dt][i];
  }
  __syncthreads();
  for (int i = tid; i < NR * D; i += DTHREADS) {
    const int r = i / D, d = i % D;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][r]);
    float acc = 0.f, Lsum = 0.f;
    if (M != -__builtin_inff()) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        if (red_m[w][r] == -__builtin_inff()) continue;
        const float wt = expf(red_m[w][r] - M);
        acc = __builtin_fmaf(((const float*)(dsmem + w * L::WAVE_BYTES))[r * D + d], wt, acc);
        Lsum = __builtin_fmaf(red_l[w][r], wt, Lsum);
      }
    }
    part_out[r * (D + 2) + d] = acc;
    if (d == 0) {
      part_out[r * (D + 2) + D] = M;
      part_out[r * (D + 2) + D + 1] = Lsum;
    }
  }
}

// One workgroup of D threads per (b, s, h) output row: merge the chunks of each partition,
// then the partitions.
template <typename O, int D, int NR>
__global__ __launch_bounds__(D) void decode_reduce_kernel(const DecodeParams p) {
  const int row = blockIdx.x;  // (b, s, h)
  const int h = row % p.Hq;
  const int s = (row / p.Hq) % p.Sq;
  const int b = row / (p.Hq * p.Sq);
  const int d = threadIdx.x;
  const int kvh = p.map.kv_of(h);
  const int r = s * p.G + (h - kvh * p.G);
  const int total_chunks = p.chunk_begin[p.nparts];
  const float* base = p.partial + ((int64_t)b * p.Hkv + kvh) * total_chunks * NR * (D + 2) + r * (D + 2);

  constexpr int WCH = 4 * D;  // chunk weights staged per round
  __shared__ float w_s[WCH];
  __shared__ float l_s[WCH];
  __shared__ float red[D / 64];
  const int64_t cstride = (int64_t)NR * (D + 2);

  float lse_p[CEA_MAX_PARTS], out_p[CEA_MAX_PARTS];
  for (int part = 0; part < p.nparts; ++part) {
    const int c0 = p.chunk_begin[part], c1 = p.chunk_begin[part + 1];
    // reference maximum over the partition's chunks (all threads, then the workgroup)
    float mx = -__builtin_inff();
    for (int ch = c0 + d; ch < c1; ch += D) mx = fmaxf(mx, base[ch * cstride + D]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if ((d & 63) == 0) red[d >> 6] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int i = 1; i < D / 64; ++i) M = fmaxf(M, red[i]);
    __syncthreads();
    float acc = 0.f, L = 0.f;
    if (M != -__builtin_inff()) {
      for (int cb = c0; cb < c1; cb += WCH) {
        const int n = min(WCH, c1 - cb);
        for (int j = d; j < n; j += D) {
          const float mc = base[(cb + j) * cstride + D];
          const float w = mc == -__builtin_inff() ? 0.f : expf(mc - M);
          w_s[j] = w;
          l_s[j] = w == 0.f ? 0.f : base[(cb + j) * cstride + D + 1];
        }
        __syncthreads();
        // independent loads across chunks; chunks without visible keys hold no output
#pragma unroll 8
        for (int j = 0; j < n; ++j) {
          const float w = w_s[j];
          if (w != 0.f) {
            acc = __builtin_fmaf(base[(cb + j) * cstride + d], w, acc);
            L = __builtin_fmaf(l_s[j], w, L);
          }
        }
        __syncthreads();
      }
    }
    const bool empty = !(L > 0.f);
    lse_p[part] = empty ? -__builtin_inff() : M + logf(L);
    out_p[part] = empty ? 0.f : acc / L;
    if (p.part_out[part]) {
      float* po = (float*)p.part_out[part] + b * p.pos_[part][0] + s * p.pos_[part][1] + h * p.pos_[part][2];
      po[d] = out_p[part];
      if (d == 0) {
        float* pl = (float*)p.part_lse[part] + b * p.pls_[part][0] + h * p.pls_[part][1] + s * p.pls_[part][2];
        *pl = lse_p[part];
      }
    }
  }
  // merge of the partitions: logsumexp and weighted sum in partition order
  float lse, res;
  if (p.nparts == 1) {
    lse = lse_p[0];
    res = out_p[0];
  } else {
    float mx = -__builtin_inff();
    for (int part = 0; part < p.nparts; ++part) mx = fmaxf(mx, lse_p[part]);
    const float shift = is_inf(mx) ? 0.f : mx;
    float sum = 0.f;
    for (int part = 0; part < p.nparts; ++part) sum = add_rn(sum, expf(lse_p[part] - shift));
    lse = logf(sum) + shift;
    const float safe = is_finite(lse) ? lse : 0.f;
    res = 0.f;
    for (int part = 0; part < p.nparts; ++part)
      res = add_rn(res, mul_rn(out_p[part], expf(lse_p[part] - safe)));
  }
  float* lptr = p.lse ? (float*)p.lse + b * p.ls_b + h * p.ls_h + s * p.ls_s : nullptr;
  O* optr = (O*)p.out + b * p.os_b + s * p.os_s + h * p.os_h;
  if (p.accumulate) {  // merge_attention(running, new)
    const float lse_old = *lptr;
    const float lm = logaddexp<float>(lse_old, lse);
    const float safe = is_finite(lm) ? lm : 0.f;
    const float v = add_rn(mul_rn((float)optr[d], expf(lse_old - safe)), mul_rn(res, expf(lse - safe)));
    optr[d] = (O)v;
    __syncthreads();  // every thread has read lse_old
    if (d == 0) *lptr = lm;
  } else {
    optr[d] = (O)res;
    if (lptr && d == 0) *lptr = lse;
  }
}

template <typename T, int D, int NR>
int launch_nr(const DecodeParams& p, hipStream_t st) {
  const int total = p.chunk_begin[p.nparts];
  if (total > 0) {
    static bool configured = false;
    if (!configured) {
      hipError_t e = hipFuncSetAttribute((const void*)decode_split_kernel<T, D, NR>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         DLayout<D>::LDS_BYTES);
      CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "decode: cannot reserve %d bytes of LDS: %s",
                  DLayout<D>::LDS_BYTES, hipGetErrorString(e));
      configured = true;
    }
    hipLaunchKernelGGL((decode_split_kernel<T, D, NR>), dim3(total, p.Hkv, p.B), dim3(DTHREADS),
                       DLayout<D>::LDS_BYTES, st, p);
    CEA_CHECK_LAUNCH("decode_split");
  }
  const int rows = p.B * p.Sq * p.Hq;
  if (rows == 0) return CEA_OK;
  if (p.out_dtype == CEA_F32)
    hipLaunchKernelGGL((decode_reduce_kernel<float, D, NR>), dim3(rows), dim3(D), 0, st, p);
  else if (p.out_dtype == CEA_BF16)
    hipLaunchKernelGGL((decode_reduce_kernel<bf16, D, NR>), dim3(rows), dim3(D), 0, st, p);
  else
    hipLaunchKernelGGL((decode_reduce_kernel<f16, D, NR>), dim3(rows), dim3(D), 0, st, p);
  CEA_CHECK_LAUNCH("decode_reduce");
  return CEA_OK;
}

template <typename T, int D>
int launch_d(const DecodeParams& p, int nr, hipStream_t st) {
  switch (nr) {
    case 1: return launch_nr<T, D, 1>(p, st);
    case 2: return launch_nr<T, D, 2>(p, st);
    case 4: return launch_nr<T, D, 4>(p, st);
    case 8: return launch_nr<T, D, 8>(p, st);
    case 16: return launch_nr<T, D, 16>(p, st);
  }
  set_error("decode: %d query rows per kv head not supported", nr);
  return CEA_EUNSUPPORTED;
}

}  // namespace

int decode_rows(int32_t Sq, int32_t G) {
  const int r = Sq * G;
  return r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : r <= 8 ? 8 : r <= 16 ? 16 : 0;
}

bool decode_supported(int32_t Sq, int32_t Hq, int32_t Hkv, int32_t D, int32_t dtype,
                      const HeadMap& map) {
  if (!(dtype == CEA_BF16 || dtype == CEA_F16)) return false;
  if (D != 128) return false;
  if (map.group <= 0) return false;  // regular GQA grouping only
  return decode_rows(Sq, Hq / Hkv) != 0;
}

int decode_plan_chunk(int64_t keys_per_head, int32_t B, int32_t Hkv) {
  // enough work items to fill 256 CUs several times, chunks of 256..1024 keys
  const int64_t heads = (int64_t)B * Hkv;
  int ch = 256;
  while (ch < CHMAX && heads * ((keys_per_head + ch - 1) / ch) > 16384) ch *= 2;
  return ch;
}

int launch_attn_decode(const DecodeParams& p, hipStream_t st) {
  const int nr = decode_rows(p.Sq, p.G);
  CEA_REQUIRE(p.chunk <= CHMAX && p.chunk % TK == 0, CEA_EINVAL, "decode: bad chunk %d", p.chunk);
  if (p.D == 128 && p.in_dtype == CEA_BF16) return launch_d<bf16, 128>(p, nr, st);
  if (p.D == 128 && p.in_dtype == CEA_F16) return launch_d<f16, 128>(p, nr, st);
  set_error("decode: unsupported dtype %s / head size %d", dtype_name(p.in_dtype), p.D);
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
