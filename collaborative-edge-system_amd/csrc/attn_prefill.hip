// Prefill attention with LSE on gfx950 matrix cores (bf16 / f16 inputs, f32 accumulation).
//
// Computes what attention_with_lse (collab_infer/parallel/attention.py:201-239) returns for
// one KV block: out[B,Sq,Hq,D] and the natural-log lse[B,Hq,Sq] of scale*q.k over the keys
// visible under the position rule of visibility_mask (attention.py:96-101), with GQA head
// mapping (attention.py:68-93), empty rows as (0, -inf) (attention.py:152-157, 173-176), and
// optionally the exact online merge of merge_attention (attention.py:242-250) into a running
// (out, lse) pair, as ring_attention does per step (sequence_parallel.py:117-121).
//
// Tiling (one workgroup = 4 waves = 128 query rows of one query head):
//   * every wave owns 32 query rows; its Q fragment stays in VGPRs for the whole kernel;
//   * S^T = K.Q^T per 64-key tile with v_mfma_f32_32x32x16 (A = K from LDS, B = Q):
//     lane (r, g) of the accumulator holds query row r and 16 of the 32 keys of a sub-tile,
//     so the row statistics of the online softmax are per-lane scalars;
//   * O^T += V^T.P^T with the same instruction (A = V^T from LDS, B = P from registers):
//     the score accumulator is already in B-operand order once V^T is stored with the
//     key-slot permutation below, so P never leaves the registers;
//   * K and V^T tiles are double-buffered in LDS (global -> VGPR -> LDS; V is transposed on
//     the way), XOR-swizzled so both the 16-byte fragment reads and the tile writes are
//     free of bank conflicts;
//   * softmax runs in the exp2 domain with log2(e)*scale folded into one FMA per score;
//   * a 64-key tile is skipped, computed unmasked, or computed with an element mask,
//     decided per wave from the tile's position summary (min/max valid position, count)
//     and the wave's query-position range, so causal, zigzag and padding masks cost nothing
//     on tiles that are entirely visible or entirely hidden.
#include "cea_kernels.hpp"

namespace cea {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int BM = 128;       // query rows per workgroup
constexpr int BN = kTileKeys; // keys per tile
constexpr int NTHREADS = 256;

template <int D> struct Layout {
  static constexpr int KROW = D * 2;                 // bytes per K row
  static constexpr int NCG = D / 8;                  // 16-byte groups per K row
  static constexpr int K_BYTES = BN * KROW;
  static constexpr int VT_BYTES = D * BN * 2;        // V^T rows of 64 slots (128 bytes)
  static constexpr int POS_BYTES = BN * 8;
  static constexpr int BUF_BYTES = K_BYTES + VT_BYTES + POS_BYTES;
  static constexpr int LDS_BYTES = 2 * BUF_BYTES;
  static constexpr int K_CHUNKS = BN * NCG / NTHREADS;  // 16-byte K chunks per thread
};

// K row swizzle: 16-byte group g of key row 'key' lives at group (g ^ swz(key)).
template <int D> __device__ __forceinline__ int k_swz(int key) {
  if constexpr (D / 8 >= 16) return key & 15;
  else return (key >> 1) & 7;
}
__device__ __forceinline__ int vt_swz(int d) { return (d >> 1) & 7; }

// Slot of key 'key' (0..63) in a V^T row: within each 16-key step, keys
// a*8 + g*4 + b go to slot g*8 + a*4 + b, which makes the 8 keys a lane of half g needs
// for one MFMA step contiguous (one 16-byte read).
__device__ __forceinline__ int vt_slot(int key) {
  return (key & ~15) | (((key >> 2) & 1) << 3) | (((key >> 3) & 1) << 2) | (key & 3);
}

__device__ __forceinline__ int64_t lds_i64(const char* base, int idx) {
  return *(const int64_t*)(base + idx * 8);
}

template <typename T, int D>
__global__ __launch_bounds__(NTHREADS, 2) void attn_prefill_kernel(const AttnParams p) {
  typedef Layout<D> L;
  typedef typename Mfma<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ int64_t red_q[2][4];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 31;   // query row inside the wave / MFMA column
  const int g = lane >> 5;   // half of the wave

  // ---- XCD-aware work mapping: consecutive logical blocks share (b, kv head) and land on
  // the same XCD (blocks are dispatched round-robin over 8 XCDs).
  const int nqb = (p.Sq + BM - 1) / BM;
  const int total = nqb * p.Hq * p.B;
  int blk = blockIdx.x;
  if ((total & 7) == 0) blk = (blk & 7) * (total >> 3) + (blk >> 3);
  const int qb = nqb - 1 - (blk % nqb);  // later (heavier causal) query blocks first
  const int bh = blk / nqb;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int kvh = p.map.kv_of(h);

  const int row = qb * BM + wave * 32 + r;
  const bool row_ok = row < p.Sq;
  const int64_t qpos = row_ok ? p.q_pos[b * p.qps_b + (int64_t)row * p.qps_s] : 0;

  // ---- query position ranges of the wave and of the workgroup
  int64_t qmin_w = wave_min_i64(row_ok ? qpos : INT64_MAX);
  int64_t qmax_w = wave_max_i64(row_ok ? qpos : INT64_MIN);
  const bool wave_active = __builtin_amdgcn_readfirstlane(qb * BM + wave * 32 < p.Sq ? 1 : 0);
  if (lane == 0) {
    red_q[0][wave] = qmin_w;
    red_q[1][wave] = qmax_w;
  }
  __syncthreads();
  const int64_t qmax_wg = max(max(red_q[1][0], red_q[1][1]), max(red_q[1][2], red_q[1][3]));

  // ---- scale folded into exp2: p = exp2(s*c - m*c), c = |scale|*log2(e) > 0.  A negative
  // scale is absorbed by negating Q (exact in bf16/f16).
  const float scale = (float)p.scale;
  const float c = fabsf(scale) * 1.4426950408889634f;
  const uint32_t qflip = scale < 0.f ? 0x80008000u : 0u;

  frag qf[D / 16];
  {
    const T* qrow = (const T*)p.q + b * p.qs_b + (int64_t)row * p.qs_s + h * p.qs_h;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (row_ok) raw = *(const uint4*)(qrow + ks * 16 + g * 8);
      raw.x ^= qflip; raw.y ^= qflip; raw.z ^= qflip; raw.w ^= qflip;
      __builtin_memcpy(&qf[ks], &raw, 16);
    }
  }

  const T* kbase = (const T*)p.k + b * p.ks_b + kvh * p.ks_h;
  const T* vbase = (const T*)p.v + b * p.vs_b + kvh * p.vs_h;
  const int64_t* kpos_b = p.k_pos + b * p.kps_b;
  const TileInfo* tinfo = p.tiles + (int64_t)b * p.ntiles;

  // ---- list of tiles the workgroup visits: 64 summaries per ballot
  int chunk_base = -64;
  uint64_t chunk_mask = 0;
  auto next_tile = [&]() -> int {
    while (chunk_mask == 0) {
      chunk_base += 64;
      if (chunk_base >= p.ntiles) return -1;
      const int t = chunk_base + lane;
      bool need = false;
      if (t < p.ntiles) {
        const TileInfo ti = tinfo[t];
        need = ti.n_valid > 0 && !(p.causal && qmax_wg < ti.min_valid);
      }
      chunk_mask = __ballot(need);
    }
    const int t = chunk_base + __builtin_ctzll(chunk_mask);
    chunk_mask &= chunk_mask - 1;
    return __builtin_amdgcn_readfirstlane(t);
  };

  // ---- tile staging: K as 16-byte chunks, V as 4-key x 8-feature blocks (transposed)
  uint4 kreg[L::K_CHUNKS];
  uint4 vreg[4];
  int64_t preg = -1;
  const int v_kq = (lane >> 1) & 15;
  const int v_c = (lane & 1) + 2 * (lane >> 5) + 4 * wave;  // 8-feature chunk of V
  const bool v_on = v_c < D / 8;

  auto load_tile = [&](int t) {
    const int key0 = t * BN;
#pragma unroll
    for (int i = 0; i < L::K_CHUNKS; ++i) {
      const int q = tid + i * NTHREADS;
      const int key = q / L::NCG, cg = q % L::NCG;
      kreg[i] = make_uint4(0, 0, 0, 0);
      if (key0 + key < p.Sk)
        kreg[i] = *(const uint4*)(kbase + (int64_t)(key0 + key) * p.ks_s + cg * 8);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = key0 + v_kq * 4 + j;
      vreg[j] = make_uint4(0, 0, 0, 0);
      if (v_on && key < p.Sk) vreg[j] = *(const uint4*)(vbase + (int64_t)key * p.vs_s + v_c * 8);
    }
    if (tid < BN) {
      const int key = key0 + tid;
      preg = key < p.Sk ? kpos_b[(int64_t)key * p.kps_s] : -1;
    }
  };

  auto store_tile = [&](int buf) {
    char* kl = smem + buf * L::BUF_BYTES;
    char* vl = kl + L::K_BYTES;
    char* pl = vl + L::VT_BYTES;
#pragma unroll
    for (int i = 0; i < L::K_CHUNKS; ++i) {
      const int q = tid + i * NTHREADS;
      const int key = q / L::NCG, cg = q % L::NCG;
      *(uint4*)(kl + key * L::KROW + ((cg ^ k_swz<D>(key)) << 4)) = kreg[i];
    }
    if (v_on) {
      const int slot = vt_slot(v_kq * 4);
      const int cgv = slot >> 3, within = (slot & 7) * 2;
      const uint32_t* w0 = (const uint32_t*)&vreg[0];
      const uint32_t* w1 = (const uint32_t*)&vreg[1];
      const uint32_t* w2 = (const uint32_t*)&vreg[2];
      const uint32_t* w3 = (const uint32_t*)&vreg[3];
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        const int e = dd ^ (v_c & 1);     // row order alternates between lane pairs
        const int d = v_c * 8 + e;
        const int sh = (e & 1) * 16;
        const uint32_t lo = ((w0[e >> 1] >> sh) & 0xffffu) | (((w1[e >> 1] >> sh) & 0xffffu) << 16);
        const uint32_t hi = ((w2[e >> 1] >> sh) & 0xffffu) | (((w3[e >> 1] >> sh) & 0xffffu) << 16);
        *(uint2*)(vl + d * 128 + ((cgv ^ vt_swz(d)) << 4) + within) = make_uint2(lo, hi);
      }
    }
    if (tid < BN) *(int64_t*)(pl + tid * 8) = preg;
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
  float m_run = -__builtin_inff();  // running max of raw scores (q.k)
  float l_run = 0.f;                // this lane's partial row sum

  int t_cur = next_tile();
  if (t_cur >= 0) {
    load_tile(t_cur);
    store_tile(0);
  }
  __syncthreads();
  int buf = 0;
  while (t_cur >= 0) {
    const int t_next = next_tile();
    if (t_next >= 0) load_tile(t_next);

    // per-wave mode of this tile: 0 skip, 1 full, 2 element-masked
    const TileInfo ti = tinfo[t_cur];
    int mode;
    if (!wave_active || ti.n_valid == 0 || (p.causal && qmax_w < ti.min_valid)) mode = 0;
    else if (ti.n_valid == BN && (!p.causal || ti.max_valid <= qmin_w)) mode = 1;
    else mode = 2;
    mode = __builtin_amdgcn_readfirstlane(mode);

    if (mode != 0) {
      const char* kl = smem + buf * L::BUF_BYTES;
      const char* vl = kl + L::K_BYTES;
      const char* pl = vl + L::VT_BYTES;
      f32x16 sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.f;
        const int key = kb * 32 + r;
        const char* krow = kl + key * L::KROW;
        const int sw = k_swz<D>(key);
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
          const frag kf = *(const frag*)(krow + (((2 * ks + g) ^ sw) << 4));
          sacc[kb] = Mfma<T>::run(kf, qf[ks], sacc[kb]);
        }
      }
      if (mode == 2) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const int key = kb * 32 + i4 * 8 + g * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int64_t kp = lds_i64(pl, key + j);
              const bool vis = row_ok && kp >= 0 && (!p.causal || kp <= qpos);
              if (!vis) sacc[kb][i4 * 4 + j] = -__builtin_inff();
            }
          }
      }
      // online softmax (exp2 domain)
      float mx = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -__builtin_inff() ? 0.f : m_new * c;
      const float alpha = __builtin_amdgcn_exp2f(m_run * c - m_use);
      m_run = m_new;
      float psum = 0.f;
      frag pf[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][e], c, -m_use));
          psum += pv;
          pf[kb * 2 + (e >> 3)][e & 7] = (T)pv;
        }
      l_run = l_run * alpha + psum;
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[dt][e] *= alpha;
      }
      // O^T += V^T . P^T
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int d = dt * 32 + r;
        const char* vrow = vl + d * 128;
        const int sw = vt_swz(d);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const frag vf = *(const frag*)(vrow + (((2 * s + g) ^ sw) << 4));
          oacc[dt] = Mfma<T>::run(vf, pf[s], oacc[dt]);
        }
      }
    }
    if (t_next < 0) break;
    store_tile(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    t_cur = t_next;
  }

  // ---- epilogue: normalise, emit (out, lse) or merge them into the running pair
  if (!row_ok) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const bool empty = !(l_tot > 0.f);
  const float inv = empty ? 0.f : 1.f / l_tot;
  const float lse_new = empty ? -__builtin_inff() : m_run * fabsf(scale) + logf(l_tot);
  float* lse_ptr = p.lse ? (float*)p.lse + b * p.ls_b + h * p.ls_h + (int64_t)row * p.ls_s
                         : nullptr;
  if (p.accumulate) {
    const float lse_old = *lse_ptr;
    const float lse = logaddexp<float>(lse_old, lse_new);
    const float safe = is_finite(lse) ? lse : 0.f;
    const float w_old = expf(lse_old - safe), w_new = expf(lse_new - safe);
    float* orow = (float*)p.out + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        float4* dst = (float4*)(orow + dt * 32 + i4 * 8 + g * 4);
        float4 prev = *dst;
        float o0 = oacc[dt][i4 * 4 + 0] * inv, o1 = oacc[dt][i4 * 4 + 1] * inv;
        float o2 = oacc[dt][i4 * 4 + 2] * inv, o3 = oacc[dt][i4 * 4 + 3] * inv;
        prev.x = add_rn(mul_rn(prev.x, w_old), mul_rn(o0, w_new));
        prev.y = add_rn(mul_rn(prev.y, w_old), mul_rn(o1, w_new));
        prev.z = add_rn(mul_rn(prev.z, w_old), mul_rn(o2, w_new));
        prev.w = add_rn(mul_rn(prev.w, w_old), mul_rn(o3, w_new));
        *dst = prev;
      }
    // both halves have read lse_old before either writes it
    __builtin_amdgcn_wave_barrier();
    if (g == 0) *lse_ptr = lse;
  } else {
    if (p.out_dtype == CEA_F32) {
      float* orow = (float*)p.out + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          *(float4*)(orow + dt * 32 + i4 * 8 + g * 4) =
              make_float4(oacc[dt][i4 * 4 + 0] * inv, oacc[dt][i4 * 4 + 1] * inv,
                          oacc[dt][i4 * 4 + 2] * inv, oacc[dt][i4 * 4 + 3] * inv);
    } else {
      T* orow = (T*)p.out + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          T v4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v4[j] = (T)(oacc[dt][i4 * 4 + j] * inv);
          uint2 raw;
          __builtin_memcpy(&raw, v4, 8);
          *(uint2*)(orow + dt * 32 + i4 * 8 + g * 4) = raw;
        }
    }
    if (lse_ptr && g == 0) *lse_ptr = lse_new;
  }
}

template <typename T, int D>
int launch_typed(const AttnParams& p, hipStream_t st) {
  const int nqb = (p.Sq + BM - 1) / BM;
  const int64_t total = (int64_t)nqb * p.Hq * p.B;
  if (total == 0) return CEA_OK;
  CEA_REQUIRE(total < (int64_t)1 << 31, CEA_EUNSUPPORTED, "attention: grid too large");
  static bool configured = false;
  if (!configured) {
    hipError_t e = hipFuncSetAttribute((const void*)attn_prefill_kernel<T, D>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       Layout<D>::LDS_BYTES);
    CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "attention: cannot reserve %d bytes of LDS: %s",
                Layout<D>::LDS_BYTES, hipGetErrorString(e));
    configured = true;
  }
  hipLaunchKernelGGL((attn_prefill_kernel<T, D>), dim3((unsigned)total), dim3(NTHREADS),
                     Layout<D>::LDS_BYTES, st, p);
  CEA_CHECK_LAUNCH("attention_prefill");
  return CEA_OK;
}

}  // namespace

static bool al16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

bool prefill_mfma_supported(const AttnParams& p) {
  if (!(p.in_dtype == CEA_BF16 || p.in_dtype == CEA_F16)) return false;
  if (!(p.D == 64 || p.D == 128)) return false;
  if (!(p.out_dtype == CEA_F32 || p.out_dtype == p.in_dtype)) return false;
  if (p.accumulate && p.out_dtype != CEA_F32) return false;
  // the exp2 fold needs c = |scale|*log2(e) to be a normal f32 (a zero c would turn the
  // -inf of masked scores into NaN); degenerate scales use the generic kernel
  if (!(fabs(p.scale) >= 1e-30 && fabs(p.scale) <= 1e30)) return false;
  // 16-byte fragments: 8-element aligned strides and bases
  const int64_t s8[] = {p.qs_b, p.qs_s, p.qs_h, p.ks_b, p.ks_s, p.ks_h, p.vs_b, p.vs_s, p.vs_h};
  for (int64_t s : s8)
    if (s % 8) return false;
  if (!al16(p.q) || !al16(p.k) || !al16(p.v) || !al16(p.out)) return false;
  const int64_t so[] = {p.os_b, p.os_s, p.os_h};
  for (int64_t s : so)
    if (s % (p.out_dtype == CEA_F32 ? 4 : 4)) return false;
  return true;
}

int launch_attn_prefill_mfma(const AttnParams& p, hipStream_t st) {
  if (p.in_dtype == CEA_BF16) {
    if (p.D == 128) return launch_typed<bf16, 128>(p, st);
    if (p.D == 64) return launch_typed<bf16, 64>(p, st);
  } else if (p.in_dtype == CEA_F16) {
    if (p.D == 128) return launch_typed<f16, 128>(p, st);
    if (p.D == 64) return launch_typed<f16, 64>(p, st);
  }
  set_error("attention: MFMA path does not cover dtype %s, head size %d",
            dtype_name(p.in_dtype), p.D);
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
