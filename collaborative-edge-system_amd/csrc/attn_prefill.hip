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
//   * K tiles go global -> LDS directly (buffer_load ... lds, no VGPR staging); V tiles go
//     through VGPRs and are transposed into V^T on the LDS write; both are double-buffered
//     and XOR-swizzled so 16-byte fragment reads and tile writes are bank-conflict free;
//   * buffer resources clamp reads past the last key to zero, so partial tiles need no
//     branches; the tile base lives in the resource (scalar), lane offsets are constants;
//   * softmax runs in the exp2 domain with log2(e)*scale folded into one FMA per score, and
//     the running maximum is only moved (and O rescaled) when a row's maximum grows by more
//     than 2^8 - the result is exact either way because l and O share the reference max;
//   * a 64-key tile is skipped, computed unmasked, or computed with an element mask,
//     decided per wave from the tile's position summary (min/max valid position, count)
//     and the wave's query-position range, so causal, zigzag and padding masks cost nothing
//     on tiles that are entirely visible or entirely hidden.
#include <type_traits>

#include "cea_kernels.hpp"

namespace cea {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

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

constexpr int BM = 128;        // query rows per workgroup
constexpr int BN = kTileKeys;  // keys per tile
constexpr int NTHREADS = 256;
constexpr float kRescaleLog2 = 8.0f;        // lazy-rescale threshold, log2 units
constexpr int kRsrcFlags = 0x00020000;      // raw buffer resource word 3 (gfx9 family)

template <int D> struct Layout {
  static constexpr int KROW = D * 2;                 // bytes per K row
  static constexpr int NCG = D / 8;                  // 16-byte groups per K row
  static constexpr int K_BYTES = BN * KROW;
  static constexpr int VT_BYTES = D * BN * 2;        // V^T rows of 64 slots (128 bytes)
  static constexpr int POS_BYTES = BN * 8;
  static constexpr int BUF_BYTES = K_BYTES + VT_BYTES + POS_BYTES;
  static constexpr int LDS_BYTES = 2 * BUF_BYTES;
  static constexpr int K_LOADS = K_BYTES / (NTHREADS * 16);  // direct loads per wave
  static constexpr int KEYS_PER_LOAD = 1024 / KROW;          // keys per wave load
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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcFlags);
}

// 16 bytes per lane from a buffer straight into LDS at lds_base + lane*16.  Kept out of
// lambdas: used inside one, the builtin makes the host pass drop the kernel's launch stub.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rs, char* lds_base,
                                                  uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_ptr)lds_base, 16, voffset, 0, 0, 0);
}

__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
}

// max of x over the two 32-lane halves of the wave (v_permlane32_swap)
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
  const int64_t qmin_w = wave_min_i64(row_ok ? qpos : INT64_MAX);
  const int64_t qmax_w = wave_max_i64(row_ok ? qpos : INT64_MIN);
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
  const float grow_thr = kRescaleLog2 / c;  // raw-score growth that triggers a rescale
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

  const char* kbase = (const char*)((const T*)p.k + b * p.ks_b + kvh * p.ks_h);
  const char* vbase = (const char*)((const T*)p.v + b * p.vs_b + kvh * p.vs_h);
  const int64_t* kpos_b = p.k_pos + b * p.kps_b;
  const TileInfo* tinfo = p.tiles + (int64_t)b * p.ntiles;
  const uint32_t krow_bytes = (uint32_t)(p.ks_s * 2), vrow_bytes = (uint32_t)(p.vs_s * 2);

  // ---- per-lane constant offsets
  // direct K loads: wave load i covers keys (wave*K_LOADS+i)*KEYS_PER_LOAD ...; lane l writes
  // LDS bytes l*16 of that 1 KB and so must fetch logical group (l % NCG) ^ swz(key)
  uint32_t k_voff[L::K_LOADS];
#pragma unroll
  for (int i = 0; i < L::K_LOADS; ++i) {
    const int key = (wave * L::K_LOADS + i) * L::KEYS_PER_LOAD + lane / L::NCG;
    const int cg = (lane % L::NCG) ^ k_swz<D>(key);
    k_voff[i] = key * krow_bytes + cg * 16;
  }
  // V: lane owns 4 consecutive keys x 8 features; transposed LDS writes
  const int v_kq = (lane >> 1) & 15;
  const int v_c = (lane & 1) + 2 * (lane >> 5) + 4 * wave;  // 8-feature chunk of V
  const bool v_on = v_c < D / 8;
  uint32_t v_voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v_voff[j] = (v_kq * 4 + j) * vrow_bytes + v_c * 16;
  uint32_t v_waddr[8];
  {
    const int slot = vt_slot(v_kq * 4);
    const int cgv = slot >> 3, within = (slot & 7) * 2;
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const int d = v_c * 8 + (dd ^ (v_c & 1));  // alternate row order between lane pairs
      v_waddr[dd] = L::K_BYTES + d * 128 + ((cgv ^ vt_swz(d)) << 4) + within;
    }
  }
  // fragment reads
  uint32_t k_raddr[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) k_raddr[ks] = r * L::KROW + (((2 * ks + g) ^ k_swz<D>(r)) << 4);
  uint32_t v_raddr[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) v_raddr[s] = L::K_BYTES + r * 128 + (((2 * s + g) ^ vt_swz(r)) << 4);

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

  u32x4 vreg[4];
  int64_t preg = -1;
  // issue the global reads of tile t: K straight into LDS buffer 'bo', V and positions to VGPRs
  auto load_tile = [&](int t, int bo) {
    const int key0 = t * BN;
    const int left = p.Sk - key0;  // > 0 for every visited tile
    const uint32_t kbytes = (uint32_t)(left - 1) * krow_bytes + L::KROW;
    const uint32_t vbytes = (uint32_t)(left - 1) * vrow_bytes + L::KROW;
    const auto krs = make_rsrc(kbase + (int64_t)key0 * krow_bytes, kbytes);
    const auto vrs = make_rsrc(vbase + (int64_t)key0 * vrow_bytes, vbytes);
#pragma unroll
    for (int i = 0; i < L::K_LOADS; ++i)
      buffer_load_lds16(krs, smem + bo + (wave * L::K_LOADS + i) * 1024, k_voff[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      vreg[j] = v_on ? __builtin_amdgcn_raw_buffer_load_b128(vrs, v_voff[j], 0, 0) : u32x4{0, 0, 0, 0};
    if (tid < BN) preg = tid < left ? kpos_b[(int64_t)(key0 + tid) * p.kps_s] : -1;
  };
  // write the register-staged part of a tile (V^T, positions) into LDS buffer 'bo'
  auto store_tile = [&](int bo) {
    if (v_on) {
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        const int e = dd ^ (v_c & 1);
        const int wi = e >> 1;
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(vreg[1][wi], vreg[0][wi], sel);
        const uint32_t hi = __builtin_amdgcn_perm(vreg[3][wi], vreg[2][wi], sel);
        *(u32x2*)(smem + bo + v_waddr[dd]) = u32x2{lo, hi};
      }
    }
    if (tid < BN) *(int64_t*)(smem + bo + L::K_BYTES + L::VT_BYTES + tid * 8) = preg;
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
  float m_run = -__builtin_inff();  // reference max of raw scores (q.k)
  float m_use = 0.f;                // m_run * c, or 0 while the row has seen nothing
  float l_run = 0.f;                // this lane's partial row sum

  auto compute = [&](auto bufc, int t) {
    constexpr int BO = decltype(bufc)::value * L::BUF_BYTES;
    const TileInfo ti = tinfo[t];
    int mode;  // 0 skip, 1 full, 2 element-masked
    if (!wave_active || ti.n_valid == 0 || (p.causal && qmax_w < ti.min_valid)) mode = 0;
    else if (ti.n_valid == BN && (!p.causal || ti.max_valid <= qmin_w)) mode = 1;
    else mode = 2;
    mode = __builtin_amdgcn_readfirstlane(mode);
    if (mode == 0) return;

    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      frag kf[D / 16];
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        kf[ks] = *(const frag*)(smem + BO + kb * 32 * L::KROW + k_raddr[ks]);
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) acc = Mfma<T>::run(kf[ks], qf[ks], acc);
      sacc[kb] = acc;
    }
    if (mode == 2) {
      const char* pl = smem + BO + L::K_BYTES + L::VT_BYTES + g * 32;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t kp = *(const int64_t*)(pl + (kb * 32 + i4 * 8 + j) * 8);
            const bool vis = row_ok && kp >= 0 && (!p.causal || kp <= qpos);
            if (!vis) sacc[kb][i4 * 4 + j] = -__builtin_inff();
          }
        }
    }
    // online softmax (exp2 domain) with a lazily moved reference maximum
    float mx = max3f(sacc[0][0], sacc[0][1], sacc[0][2]);
#pragma unroll
    for (int e = 3; e < 15; e += 2) mx = max3f(mx, sacc[0][e], sacc[0][e + 1]);
    mx = max3f(mx, sacc[0][15], sacc[1][0]);
#pragma unroll
    for (int e = 1; e < 15; e += 2) mx = max3f(mx, sacc[1][e], sacc[1][e + 1]);
    mx = __builtin_fmaxf(mx, sacc[1][15]);
    mx = max_halves(mx);
    const bool grow = mx > m_run + grow_thr;
    if (__ballot(grow) != 0) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? __builtin_amdgcn_exp2f((m_run - m_new) * c) : 1.f;
      m_run = m_new;
      m_use = m_run == -__builtin_inff() ? 0.f : m_run * c;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[dt][e] *= alpha;
    }
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
    l_run += psum;
    // O^T += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      frag vf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) vf[s] = *(const frag*)(smem + BO + dt * 32 * 128 + v_raddr[s]);
#pragma unroll
      for (int s = 0; s < 4; ++s) oacc[dt] = Mfma<T>::run(vf[s], pf[s], oacc[dt]);
    }
  };

  auto sync_tile = [&]() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  int t_cur = next_tile();
  if (t_cur >= 0) {
    load_tile(t_cur, 0);
    store_tile(0);
  }
  sync_tile();
  // two-stage software pipeline, unrolled so each stage reads one LDS buffer with
  // immediate offsets: buffer 0 holds t_cur on entry of the first stage
  while (t_cur >= 0) {
    int t_next = next_tile();
    if (t_next >= 0) load_tile(t_next, L::BUF_BYTES);
    compute(std::integral_constant<int, 0>(), t_cur);
    if (t_next < 0) break;
    store_tile(L::BUF_BYTES);
    sync_tile();
    t_cur = t_next;

    t_next = next_tile();
    if (t_next >= 0) load_tile(t_next, 0);
    compute(std::integral_constant<int, 1>(), t_cur);
    if (t_next < 0) break;
    store_tile(0);
    sync_tile();
    t_cur = t_next;
  }

  // ---- epilogue: normalise, emit (out, lse) or merge them into the running pair
  if (!row_ok) return;
  const float l_tot = sum_halves(l_run);
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
        const float o0 = oacc[dt][i4 * 4 + 0] * inv, o1 = oacc[dt][i4 * 4 + 1] * inv;
        const float o2 = oacc[dt][i4 * 4 + 2] * inv, o3 = oacc[dt][i4 * 4 + 3] * inv;
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
    if (s % 4) return false;
  // buffer resources address one (batch, kv head) block with 32-bit offsets: rows must not
  // overlap and the block must stay below 2 GiB
  if (p.ks_s < p.D || p.vs_s < p.D) return false;
  const int64_t kspan = ((int64_t)p.Sk - 1) * p.ks_s * 2 + p.D * 2;
  const int64_t vspan = ((int64_t)p.Sk - 1) * p.vs_s * 2 + p.D * 2;
  if (kspan >= ((int64_t)1 << 31) || vspan >= ((int64_t)1 << 31)) return false;
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
