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
//     share the kv head (G query heads per kv head) are processed together, so each K/V row
//     is read from HBM once for all of them;
//   * a 16-lane group owns one key row at a time: lane j loads features 8j..8j+7 of K and V
//     with 16-byte loads (a wave reads 4 consecutive 256-byte rows per instruction);
//     q.k is 4 v_dot2_f32_bf16 per row plus a 4-step DPP butterfly across the group;
//   * key positions of the chunk are staged in LDS; keys that no row can see are never
//     loaded, and chunks past every valid key return after the position scan;
//   * the 16 groups of a workgroup merge their online-softmax partials in LDS and write one
//     (o unnormalised, m, l) partial per chunk; the reduction kernel then merges the chunks of
//     each partition exactly (optionally emitting each partition's (out, lse)), merges the
//     partitions with the reference's logsumexp, and writes out (f32 or the query dtype) and
//     lse.
#include "cea_kernels.hpp"

namespace cea {
namespace {

constexpr int DTHREADS = 256;
constexpr int NGROUPS = DTHREADS / 16;  // 16-lane groups per workgroup
constexpr int NB = 4;                   // keys per group per batch
constexpr int BATCH = NGROUPS * NB;     // keys per workgroup batch

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <typename T> __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);
template <> __device__ __forceinline__ float dot2<bf16>(uint32_t a, uint32_t b, float c) {
  bf16x2 x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
}
template <> __device__ __forceinline__ float dot2<f16>(uint32_t a, uint32_t b, float c) {
  f16x2 x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  return __builtin_amdgcn_fdot2(x, y, c, false);
}

template <typename T> __device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi);
template <> __device__ __forceinline__ void unpack2<bf16>(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}
template <> __device__ __forceinline__ void unpack2<f16>(uint32_t w, float& lo, float& hi) {
  f16x2 v;
  __builtin_memcpy(&v, &w, 4);
  lo = (float)v[0];
  hi = (float)v[1];
}

// sum over the 16 lanes of a DPP row, result in every lane (xor 1, xor 2, mirror 8, mirror 16)
__device__ __forceinline__ float row16_sum(float x) {
  int v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false)); // row_half_mirror
  v = __float_as_int(x);
  x += __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false)); // row_mirror
  return x;
}

__device__ __forceinline__ int part_of(const DecodeParams& p, int chunk) {
  int part = 0;
  while (part + 1 < p.nparts && chunk >= p.chunk_begin[part + 1]) ++part;
  return part;
}

// Partial layout: [B][Hkv][total_chunks][NR][D + 2] floats: o (relative to m), m, l, where
// m is in natural-log units (max of scale*q.k) and l = sum exp(scale*q.k - m).
template <typename T, int D, int NR>
__global__ __launch_bounds__(DTHREADS) void decode_split_kernel(const DecodeParams p) {
  constexpr int CHMAX = 2048;
  __shared__ int64_t kpos_s[CHMAX];
  __shared__ uint32_t batch_any[CHMAX / BATCH];
  __shared__ float red_m[NGROUPS][NR];
  __shared__ float red_l[NGROUPS][NR];
  __shared__ float red_o[NGROUPS][NR][D];

  const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int part = part_of(p, chunk);
  const int lchunk = chunk - p.chunk_begin[part];
  const int Sk = p.Sk[part];
  const int key0 = lchunk * p.chunk;
  const int nkeys = min(p.chunk, Sk - key0);
  const int tid = threadIdx.x, lane = tid & 63, grp = tid >> 4, li = tid & 15;
  const int G = p.G;
  const int total_chunks = p.chunk_begin[p.nparts];
  float* part_out = p.partial + (((int64_t)b * p.Hkv + kvh) * total_chunks + chunk) * NR * (D + 2);

  // ---- query rows of this kv head: row r = (s, gi) -> head kvh*G + gi, position q_pos[b, s]
  int64_t qp[NR];
  int64_t qmax = INT64_MIN;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int s = r / G;
    qp[r] = (r < p.Sq * G) ? p.q_pos[b * p.qps_b + (int64_t)s * p.qps_s] : INT64_MIN;
    qmax = qp[r] > qmax ? qp[r] : qmax;
  }

  // ---- positions of the chunk into LDS; which 64-key batches have any visible key
  const int64_t* kp = p.k_pos[part] + b * p.kps[part][0];
  const int64_t kps = p.kps[part][1];
  for (int i = tid; i < nkeys; i += DTHREADS) kpos_s[i] = kp[(int64_t)(key0 + i) * kps];
  const int nbatch = (nkeys + BATCH - 1) / BATCH;
  __syncthreads();
  for (int bi = tid >> 6; bi < nbatch; bi += DTHREADS / 64) {
    const int k = bi * BATCH + lane;
    bool vis = false;
    if (k < nkeys) {
      const int64_t pk = kpos_s[k];
      vis = pk >= 0 && (!p.causal || pk <= qmax);
    }
    const uint64_t bal = __ballot(vis);
    if (lane == 0) batch_any[bi] = bal != 0;
  }
  __syncthreads();
  bool any = false;
  for (int bi = 0; bi < nbatch; ++bi) any |= batch_any[bi] != 0;
  if (!any) {
    if (tid < NR) {
      part_out[tid * (D + 2) + D] = -__builtin_inff();
      part_out[tid * (D + 2) + D + 1] = 0.f;
    }
    return;
  }

  // ---- this lane's 8 features of every query row (bf16/f16 pairs), sign folded for scale<0
  const float scale = (float)p.scale;
  const float c = fabsf(scale) * 1.4426950408889634f;  // exp2 units
  const uint32_t flip = scale < 0.f ? 0x80008000u : 0u;
  uint32_t q[NR][4];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    u32x4 raw = {0, 0, 0, 0};
    if (r < p.Sq * G) {
      const int s = r / G, h = kvh * G + r % G;
      raw = *(const u32x4*)((const T*)p.q + b * p.qs_b + (int64_t)s * p.qs_s + h * p.qs_h + li * 8);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) q[r][w] = raw[w] ^ flip;
  }

  const char* kb = (const char*)((const T*)p.k[part] + b * p.ks[part][0] + kvh * p.ks[part][2]) + li * 16;
  const char* vb = (const char*)((const T*)p.v[part] + b * p.vs[part][0] + kvh * p.vs[part][2]) + li * 16;
  const int64_t krow = p.ks[part][1] * (int64_t)sizeof(T), vrow = p.vs[part][1] * (int64_t)sizeof(T);

  float m[NR], l[NR], o[NR][8];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    m[r] = -__builtin_inff();
    l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[r][e] = 0.f;
  }

  for (int bi = 0; bi < nbatch; ++bi) {
    if (!batch_any[bi]) continue;
    u32x4 kr[NB], vr[NB];
    bool kv[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int k = bi * BATCH + u * NGROUPS + grp;
      bool vis = false;
      if (k < nkeys) {
        const int64_t pk = kpos_s[k];
        vis = pk >= 0 && (!p.causal || pk <= qmax);
      }
      kv[u] = vis;
      kr[u] = {0, 0, 0, 0};
      vr[u] = {0, 0, 0, 0};
      if (vis) {
        kr[u] = *(const u32x4*)(kb + (int64_t)(key0 + k) * krow);
        vr[u] = *(const u32x4*)(vb + (int64_t)(key0 + k) * vrow);
      }
    }
    float s[NB][NR];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int k = bi * BATCH + u * NGROUPS + grp;
      const int64_t pk = kv[u] ? kpos_s[k] : -1;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float a = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) a = dot2<T>(q[r][w], kr[u][w], a);
        a = row16_sum(a);
        const bool ok = kv[u] && (!p.causal || pk <= qp[r]) && qp[r] != INT64_MIN;
        s[u][r] = ok ? a : -__builtin_inff();
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float mb = s[0][r];
#pragma unroll
      for (int u = 1; u < NB; ++u) mb = fmaxf(mb, s[u][r]);
      const float mn = fmaxf(m[r], mb);
      if (mn == -__builtin_inff()) continue;  // nothing visible to this row so far
      const float alpha = __builtin_amdgcn_exp2f((m[r] - mn) * c);
      m[r] = mn;
      l[r] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[r][e] *= alpha;
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const float pv = __builtin_amdgcn_exp2f((s[u][r] - mn) * c);
        l[r] += pv;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float lo, hi;
          unpack2<T>(vr[u][w], lo, hi);
          o[r][2 * w] = __builtin_fmaf(pv, lo, o[r][2 * w]);
          o[r][2 * w + 1] = __builtin_fmaf(pv, hi, o[r][2 * w + 1]);
        }
      }
    }
  }

  // ---- merge the 16 group partials of the workgroup and write the chunk partial
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      red_m[grp][r] = m[r];
      red_l[grp][r] = l[r];
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) red_o[grp][r][li * 8 + e] = o[r][e];
  __syncthreads();
  for (int i = tid; i < NR * D; i += DTHREADS) {
    const int r = i / D, d = i % D;
    float M = -__builtin_inff();
#pragma unroll
    for (int gi = 0; gi < NGROUPS; ++gi) M = fmaxf(M, red_m[gi][r]);
    float acc = 0.f, L = 0.f;
    if (M != -__builtin_inff()) {
#pragma unroll
      for (int gi = 0; gi < NGROUPS; ++gi) {
        const float w = __builtin_amdgcn_exp2f((red_m[gi][r] - M) * c);  // -inf -> 0
        acc = __builtin_fmaf(red_o[gi][r][d], w, acc);
        L = __builtin_fmaf(red_l[gi][r], w, L);
      }
    }
    part_out[r * (D + 2) + d] = acc;
    if (d == 0) {
      part_out[r * (D + 2) + D] = M == -__builtin_inff() ? M : M * fabsf(scale);
      part_out[r * (D + 2) + D + 1] = L;
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

  float lse_p[CEA_MAX_PARTS], out_p[CEA_MAX_PARTS];
  for (int part = 0; part < p.nparts; ++part) {
    float M = -__builtin_inff();
    for (int ch = p.chunk_begin[part]; ch < p.chunk_begin[part + 1]; ++ch)
      M = fmaxf(M, base[(int64_t)ch * NR * (D + 2) + D]);
    float acc = 0.f, L = 0.f;
    if (M != -__builtin_inff()) {
      for (int ch = p.chunk_begin[part]; ch < p.chunk_begin[part + 1]; ++ch) {
        const float* pc = base + (int64_t)ch * NR * (D + 2);
        const float mc = pc[D];
        if (mc == -__builtin_inff()) continue;
        const float w = expf(mc - M);
        acc = __builtin_fmaf(pc[d], w, acc);
        L = __builtin_fmaf(pc[D + 1], w, L);
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
    hipLaunchKernelGGL((decode_split_kernel<T, D, NR>), dim3(total, p.Hkv, p.B), dim3(DTHREADS), 0,
                       st, p);
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
  }
  set_error("decode: %d query rows per kv head not supported", nr);
  return CEA_EUNSUPPORTED;
}

}  // namespace

int decode_rows(int32_t Sq, int32_t G) {
  const int r = Sq * G;
  return r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : 0;
}

bool decode_supported(int32_t Sq, int32_t Hq, int32_t Hkv, int32_t D, int32_t dtype,
                      const HeadMap& map) {
  if (!(dtype == CEA_BF16 || dtype == CEA_F16)) return false;
  if (D != 128) return false;  // a 16-lane group covers one 256-byte row
  if (map.group <= 0) return false;  // regular GQA grouping only
  return decode_rows(Sq, Hq / Hkv) != 0;
}

int decode_plan_chunk(int64_t keys_per_head, int32_t B, int32_t Hkv) {
  // enough work items to fill 256 CUs several times, chunks of 256..2048 keys
  const int64_t heads = (int64_t)B * Hkv;
  int ch = 256;
  while (ch < 2048 && heads * ((keys_per_head + ch - 1) / ch) > 16384) ch *= 2;
  return ch;
}

int launch_attn_decode(const DecodeParams& p, hipStream_t st) {
  const int nr = decode_rows(p.Sq, p.G);
  CEA_REQUIRE(p.chunk <= 2048 && p.chunk % BATCH == 0, CEA_EINVAL, "decode: bad chunk %d", p.chunk);
  if (p.D == 128 && p.in_dtype == CEA_BF16) return launch_d<bf16, 128>(p, nr, st);
  if (p.D == 128 && p.in_dtype == CEA_F16) return launch_d<f16, 128>(p, nr, st);
  set_error("decode: unsupported dtype %s / head size %d", dtype_name(p.in_dtype), p.D);
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
