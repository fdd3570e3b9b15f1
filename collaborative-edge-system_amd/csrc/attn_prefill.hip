// Prefill attention with LSE on gfx950 matrix cores (bf16 / f16 inputs, f32 accumulation).
//
// Computes what attention_with_lse (collab_infer/parallel/attention.py:201-239) returns for
// one KV block: out[B,Sq,Hq,D] and the natural-log lse[B,Hq,Sq] of scale*q.k over the keys
// visible under the position rule of visibility_mask (attention.py:96-101), with GQA head
// mapping (attention.py:68-93), empty rows as (0, -inf) (attention.py:152-157, 173-176), and
// optionally the exact online merge of merge_attention (attention.py:242-250) into a running
// (out, lse) pair, as ring_attention does per step (sequence_parallel.py:117-121).
//
// Structure (one workgroup = 8 waves = 256 query rows, one per CU; the rows of one query
// head, or, for short query blocks, of 2, 4 or 8 query heads that read the same KV head):
//   * every wave owns 32 query rows; its Q fragment stays in VGPRs for the whole kernel;
//   * S^T = K.Q^T per 64-key tile with v_mfma_f32_32x32x16 (A = K from LDS, B = Q):
//     lane (r, g) of the accumulator holds query row r and 16 of the 32 keys of a sub-tile,
//     so the row statistics of the online softmax are per-lane scalars;
//   * O^T += V^T.P^T with the same instruction (A = V^T, B = P straight from the score
//     registers): V stays row-major in LDS and ds_read_b64_tr_b16 transposes it on the way
//     to the registers (each 16-lane group turns 16 x 4 elements into 4 keys of 16 columns);
//   * K, V and the key positions of a tile go global -> LDS directly (buffer_load ... lds),
//     through a 4-stage ring of LDS buffers with 3 tiles in flight, so HBM/L2 latency is
//     hidden behind two tiles of matrix work; buffer resources return zero past the last
//     key, so partial tiles need no branches;
//   * K rows are XOR-swizzled in 16-byte groups and V rows in 64-byte blocks, which keeps
//     both the fragment reads and the transposing reads free of LDS bank conflicts;
//   * softmax runs in the exp2 domain with log2(e)*scale folded into one FMA per score, and
//     the running maximum only moves (and O is only rescaled) when a row's maximum grows
//     by more than 2^8; l and O share that reference maximum, so the result is exact;
//   * the tiles a workgroup visits are listed up front from per-tile position summaries;
//     each wave then computes a tile unmasked, element-masked or not at all from its own
//     query-position range, so causal, zigzag and padding masks cost nothing on tiles that
//     are entirely visible or entirely hidden;
//   * a launch whose query blocks are too few to fill the device repeats its grid for up to
//     16 key splits, each listing its own run of the block's tiles and writing a partial
//     (out, lse) that the list merge combines.
#include <string.h>

#include <algorithm>

#include "cea_kernels.hpp"
#include "cea_lds_dma.hpp"

namespace cea {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

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

constexpr int NWAVES = 8;
constexpr int NTHREADS = NWAVES * 64;
constexpr int BM = NWAVES * 32;   // query rows per workgroup
constexpr int BN = kTileKeys;     // keys per tile
constexpr int NSTAGE = 4;         // LDS ring depth (NSTAGE - 1 tiles in flight)
constexpr int LIST_CAP = 2048;    // tiles listed per pass over the key block
constexpr float kRescaleLog2 = 8.0f;    // lazy-rescale threshold, log2 units

template <int D> struct Layout {
  static constexpr int KROW = D * 2;                 // bytes per K / V row
  static constexpr int NCG = D / 8;                  // 16-byte groups per row
  static constexpr int K_BYTES = BN * KROW;
  static constexpr int V_BYTES = BN * KROW;
  static constexpr int POS_BYTES = BN * 8;
  static constexpr int STAGE_BYTES = K_BYTES + V_BYTES + POS_BYTES;
  static constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;
  static constexpr int KV_LOADS = K_BYTES / (NTHREADS * 16);  // per wave, for K and for V
  static constexpr int ROWS_PER_LOAD = 1024 / KROW;           // rows one wave load covers
  static constexpr int LOADS_PER_TILE = 2 * KV_LOADS;         // K and V loads of one wave
  // wave 0 also loads the tile's 64 key positions (512 B, 32 lanes x 16 B) in one load
  static_assert(KV_LOADS >= 1, "tile too small for one load per wave");
};

// K row swizzle: 16-byte group c of row 'key' lives at group (c ^ k_swz(key)).
template <int D> __device__ __forceinline__ int k_swz(int key) {
  if constexpr (D / 8 >= 16) return key & 15;
  else return (key >> 1) & 7;
}
// V row swizzle: 64-byte block b of row 'key' lives at block (b ^ v_swz(key)).
template <int D> __device__ __forceinline__ int v_swz(int key) {
  if constexpr (D == 128) return key & 3;
  else return (key >> 1) & 1;
}

template <typename F>
__device__ __forceinline__ F read_tr_frag(const char* a0, const char* a1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)a0);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)a1);
  F f;
  __builtin_memcpy(&f, &lo, 8);
  __builtin_memcpy((char*)&f + 8, &hi, 8);
  return f;
}

__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
}

// max / sum of x over the two 32-lane halves of the wave (v_permlane32_swap)
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

// Waits until at most 'ahead' tiles' worth of this wave's buffer loads are outstanding.
template <int LPT> __device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  static_assert(NSTAGE == 4, "wait ladder written for 2 tiles ahead at most");
  if (ahead >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPT) : "memory");
  else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPT) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// MULTI: the launch streams several KV blocks (segs.n > 1); otherwise block 0 only, whose
// addresses the compiler keeps in registers for the whole kernel.
template <typename T, int D, bool MULTI>
__global__ __launch_bounds__(NTHREADS, 2) void attn_prefill_kernel(const AttnParams p,
                                                                   const KvSegs segs) {
  typedef Layout<D> L;
  typedef typename Mfma<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // listed tiles: (block << 24 | tile of the block, 2-bit mode of every wave: 0 skip, 1 full,
  // 2 element-masked)
  __shared__ int2 tile_list[LIST_CAP];
  __shared__ int64_t red_q[NWAVES], red_qmin[NWAVES];
  __shared__ int red_act[NWAVES];
  __shared__ int wave_cnt[NWAVES];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane & 31;   // query row inside the wave / MFMA column
  const int g = lane >> 5;   // half of the wave

  // ---- XCD-aware work mapping: consecutive logical blocks share (b, kv head) and land on
  // the same XCD (blocks are dispatched round-robin over 8 XCDs).
  // A key-split launch repeats the grid once per split, split slowest, so the workgroups of
  // one split and KV head (which read the same tiles) stay together as well.  A workgroup
  // holds hp query heads of one KV head's group (NWAVES / hp waves and BM / hp rows each), so
  // short query blocks do not leave most of its rows empty.
  const int hp = MULTI ? 1 : max(p.heads_per_wg, 1);
  const int rows_pb = BM / hp;  // query rows of one head in a workgroup
  const int nqb = (p.Sq + rows_pb - 1) / rows_pb;
  const int ngroups = p.Hq / hp;
  const int total = nqb * ngroups * p.B;
  const int nsplit = MULTI ? 1 : max(p.splits, 1);
  const int all = total * nsplit;
  int blk = blockIdx.x;
  if ((all & 7) == 0) blk = (blk & 7) * (all >> 3) + (blk >> 3);
  const int split = MULTI ? 0 : blk / total;
  blk -= split * total;
  const int qb = nqb - 1 - (blk % nqb);  // later (heavier causal) query blocks first
  const int bh = blk / nqb;
  const int hg = bh % ngroups;
  const int b = bh / ngroups;
  const int waves_ph = NWAVES / hp;
  const int h = hg * hp + wave / waves_ph;   // this wave's query head
  const int kvh = p.map.kv_of(hg * hp);      // one KV head for the whole workgroup
  const int qrow0 = qb * rows_pb + (wave % waves_ph) * 32;  // this wave's first query row

  const int row = qrow0 + r;
  const bool row_ok = row < p.Sq;
  const int64_t qpos = row_ok ? p.q_pos[b * p.qps_b + (int64_t)row * p.qps_s] : 0;

  // ---- query position ranges of the wave and of the workgroup
  const int64_t qmin_w = wave_min_i64(row_ok ? qpos : INT64_MAX);
  const int64_t qmax_w = wave_max_i64(row_ok ? qpos : INT64_MIN);
  const bool wave_active = __builtin_amdgcn_readfirstlane(qrow0 < p.Sq ? 1 : 0);
  if (lane == 0) {
    red_q[wave] = qmax_w;
    red_qmin[wave] = qmin_w;
    red_act[wave] = wave_active ? 1 : 0;
  }
  __syncthreads();
  int64_t qmax_wg = red_q[0];
#pragma unroll
  for (int w = 1; w < NWAVES; ++w) qmax_wg = max(qmax_wg, red_q[w]);

  // ---- scale folded into exp2: p = exp2(s*c - m*c), c = |scale|*log2(e) > 0.  A negative
  // scale is absorbed by negating Q (exact in bf16/f16).
  const float scale = (float)p.scale;
  const float c = fabsf(scale) * 1.4426950408889634f;
  const float grow_thr = kRescaleLog2 / c;  // raw-score growth that triggers a rescale
  const uint32_t qflip = scale < 0.f ? 0x80008000u : 0u;

  // Under the causal rule a row with position < 0 (padding) sees no key and its scores are
  // always masked, so its query features are not read (a workgroup of padding rows only
  // writes its empty result).
  frag qf[D / 16];
  {
    const T* qrow = (const T*)p.q + b * p.qs_b + (int64_t)row * p.qs_s + h * p.qs_h;
    const bool load_q = row_ok && !(p.causal && qpos < 0);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (load_q) raw = *(const uint4*)(qrow + ks * 16 + g * 8);
      raw.x ^= qflip; raw.y ^= qflip; raw.z ^= qflip; raw.w ^= qflip;
      __builtin_memcpy(&qf[ks], &raw, 16);
    }
  }

  // tile summaries of all blocks, numbered block after block
  const TileInfo* tinfo = p.tiles + (int64_t)b * p.ntiles;
  const uint32_t krow_bytes = (uint32_t)(p.ks_s * 2), vrow_bytes = (uint32_t)(p.vs_s * 2);

  // ---- per-lane constant offsets of the direct loads: wave load i covers rows
  // (wave*KV_LOADS + i)*ROWS_PER_LOAD ...; lane l lands on LDS bytes l*16 of that 1 KB and
  // fetches the logical 16-byte group the swizzle puts there
  uint32_t k_voff[L::KV_LOADS], v_voff[L::KV_LOADS];
#pragma unroll
  for (int i = 0; i < L::KV_LOADS; ++i) {
    const int key = (wave * L::KV_LOADS + i) * L::ROWS_PER_LOAD + lane / L::NCG;
    const int pg = lane % L::NCG;  // physical 16-byte group in the row
    k_voff[i] = key * krow_bytes + ((pg ^ k_swz<D>(key)) << 4);
    const int lgv = (((pg >> 2) ^ v_swz<D>(key)) << 2) | (pg & 3);
    v_voff[i] = key * vrow_bytes + (lgv << 4);
  }
  const uint32_t p_voff = (lane & 31) * 16;  // wave 0: 2 positions per lane, lanes 0-31

  // fragment reads: K rows for S^T, transposing reads for V^T
  uint32_t k_raddr[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) k_raddr[ks] = r * L::KROW + (((2 * ks + g) ^ k_swz<D>(r)) << 4);
  uint32_t v_raddr[D / 32];
  {
    const int src = lane & 15, grp = lane >> 4;
    const int vrow = g * 4 + (src >> 2);  // + s*16 + half*8 (immediates), multiple-of-4 base
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
      v_raddr[dt] = L::K_BYTES + vrow * L::KROW + ((dt ^ v_swz<D>(vrow)) << 6) +
                    (16 * (grp & 1) + 4 * (src & 3)) * 2;
  }

  // LDS byte address of the dynamic LDS block and of this wave's 1 KB load windows in a
  // stage (wave-uniform: scalar registers)
  const uint32_t smem_lds = lds_addr(smem);
  const uint32_t wave_kv = __builtin_amdgcn_readfirstlane(wave) * (L::KV_LOADS * 1024);
  const bool pos_loader = __builtin_amdgcn_readfirstlane(wave) == 0;
  // block of a list entry (block << 24 | tile): a compile-time 0 for single-block launches
  auto seg_of = [&](int x) -> const KvSeg& { return segs.seg[MULTI ? (x >> 24) : 0]; };
  // buffer sources of one tile (the block's pointers come from kernel arguments)
  struct TileSrc {
    i32x4 krs, vrs, prs;
  };
  // With several blocks the list runs block by block, so the bases of the block whose tiles
  // are being loaded are kept and recomputed only when the block changes.
  int src_seg = -1, src_sk = 0;
  const char *src_k = nullptr, *src_v = nullptr, *src_p = nullptr;
  int cur_seg = -1, cur_sk = 0;  // the same for the block of the tile being computed
  auto tile_src = [&](int x) {
    const int si = MULTI ? (x >> 24) : 0;
    if (!MULTI || si != src_seg) {
      const KvSeg& sg = segs.seg[si];
      src_k = (const char*)((const T*)sg.k + b * sg.ks_b + kvh * sg.ks_h);
      src_v = (const char*)((const T*)sg.v + b * sg.vs_b + kvh * sg.vs_h);
      src_p = (const char*)(sg.k_pos + b * sg.kps_b);
      src_sk = sg.Sk;
      src_seg = si;
    }
    const int key0 = (x & 0xffffff) * BN;
    // keys of the tile that exist (> 0 for every listed tile); the resources span those rows
    // only, so their ranges stay 32-bit however large the block is
    const int rows = min(src_sk - key0, BN);
    const char* kbase = src_k;
    const char* vbase = src_v;
    const char* pbase = src_p;
    TileSrc ts;
    ts.krs = make_rsrc(kbase + (int64_t)key0 * krow_bytes, (uint32_t)(rows - 1) * krow_bytes + L::KROW);
    ts.vrs = make_rsrc(vbase + (int64_t)key0 * vrow_bytes, (uint32_t)(rows - 1) * vrow_bytes + L::KROW);
    ts.prs = make_rsrc(pbase + (int64_t)key0 * 8, (uint32_t)rows * 8);
    return ts;
  };
  // this wave's share of a tile's loads: K rows, V rows and (16 lanes) key positions
  auto load_tile = [&](const TileSrc& ts, int stage) {
    const uint32_t st = smem_lds + stage * L::STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < L::KV_LOADS; ++i) buffer_load_lds16_m0(ts.krs, st + wave_kv + i * 1024, k_voff[i]);
#pragma unroll
    for (int i = 0; i < L::KV_LOADS; ++i)
      buffer_load_lds16_m0(ts.vrs, st + L::K_BYTES + wave_kv + i * 1024, v_voff[i]);
    if (pos_loader && lane < 32) buffer_load_lds16_m0(ts.prs, st + L::K_BYTES + L::V_BYTES, p_voff);
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[i][e] = 0.f;
  float m_run = -__builtin_inff();  // reference max of raw scores (q.k)
  float m_use = 0.f;                // m_run * c, or 0 while the row has seen nothing
  float l_run = 0.f;                // this lane's partial row sum

  // mode: 1 every key of the tile visible to every row of the wave, 2 element-masked;
  // left: keys of the tile's block from the tile's first key on
  auto compute = [&](int stage, int left, int mode) {
    const char* sb = smem + stage * L::STAGE_BYTES;

    f32x16 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      frag kf[D / 16];
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        kf[ks] = *(const frag*)(sb + kb * 32 * L::KROW + k_raddr[ks]);
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) acc = Mfma<T>::run(kf[ks], qf[ks], acc);
      sacc[kb] = acc;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, D / 16, 0);
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, D / 16, 0);
    if (mode == 2) {
      // key visible: it exists (key < left) and, read as unsigned, k_pos <= q_pos (causal;
      // -1 wraps to the maximum) or k_pos >= 0 (not causal); a padded query row sees
      // nothing when causal
      const char* pl = sb + L::K_BYTES + L::V_BYTES;
      const bool row_sees = p.causal ? (row_ok && qpos >= 0) : row_ok;
      const uint64_t qlim = p.causal ? (uint64_t)qpos : (uint64_t)INT64_MAX;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int key0 = kb * 32 + i4 * 8 + g * 4;
          const uint4 a = *(const uint4*)(pl + key0 * 8);        // keys key0, key0 + 1
          const uint4 a2 = *(const uint4*)(pl + key0 * 8 + 16);  // keys key0 + 2, key0 + 3
          const uint64_t kp[4] = {((uint64_t)a.y << 32) | a.x, ((uint64_t)a.w << 32) | a.z,
                                  ((uint64_t)a2.y << 32) | a2.x, ((uint64_t)a2.w << 32) | a2.z};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool vis = row_sees && key0 + j < left && kp[j] <= qlim;
            if (!vis) sacc[kb][i4 * 4 + j] = -__builtin_inff();
          }
        }
    }
    // online softmax (exp2 domain) with a lazily moved reference maximum
    // row maximum as a tree of independent max3 (short dependency chains)
    float t1[11];
#pragma unroll
    for (int i = 0; i < 10; ++i) {
      const int e = 3 * i;
      t1[i] = max3f(sacc[e >> 4][e & 15], sacc[(e + 1) >> 4][(e + 1) & 15], sacc[(e + 2) >> 4][(e + 2) & 15]);
    }
    t1[10] = __builtin_fmaxf(sacc[1][14], sacc[1][15]);
    const float t2a = max3f(t1[0], t1[1], t1[2]), t2b = max3f(t1[3], t1[4], t1[5]);
    const float t2c = max3f(t1[6], t1[7], t1[8]), t2d = __builtin_fmaxf(t1[9], t1[10]);
    float mx = __builtin_fmaxf(max3f(t2a, t2b, t2c), t2d);
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
    frag pf[4];
    float pr[32];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        pr[kb * 16 + e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][e], c, -m_use));
        pf[kb * 2 + (e >> 3)][e & 7] = (T)pr[kb * 16 + e];
      }
    // f32 row sum as a tree of independent adds
#pragma unroll
    for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
      for (int e = 0; e < w; ++e) pr[e] += pr[e + w];
    l_run += pr[0];
    // O^T += V^T . P^T: fragment of step s holds keys s*16 + {g*4..+3, 8+g*4..+3}
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      frag vf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        vf[s] = read_tr_frag<frag>(sb + s * 16 * L::KROW + v_raddr[dt],
                                   sb + (s * 16 + 8) * L::KROW + v_raddr[dt]);
#pragma unroll
      for (int s = 0; s < 4; ++s) oacc[dt] = Mfma<T>::run(vf[s], pf[s], oacc[dt]);
    }
    // the transposing reads of the next 16 columns overlap the products of these
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
#pragma unroll
    for (int j = 0; j < D / 32 - 1; ++j) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
  };

  // ---- passes over the key block: list the tiles this workgroup needs, then stream them.
  // Under the causal rule a workgroup whose rows all have position < 0 (padding) sees no key
  // (a visible key needs 0 <= k_pos <= q_pos), so it goes straight to the epilogue.
  // tiles [t_first, t_last) of the block, all of them unless the launch splits the keys
  const int per_split = (p.ntiles + nsplit - 1) / nsplit;
  const int t_first = min(p.ntiles, split * per_split);
  const int t_last = min(p.ntiles, t_first + per_split);
  const int passes_end = p.causal && qmax_wg < 0 ? t_first : t_last;
  for (int base = t_first; base < passes_end; base += LIST_CAP) {
    const int span = min(LIST_CAP, t_last - base);
    int n = 0;
    for (int r0 = 0; r0 < span; r0 += NTHREADS) {
      const int t = base + r0 + tid;
      bool need = false;
      int modes = 0, x = 0;
      if (r0 + tid < span) {
        const TileInfo ti = tinfo[t];
        int sgi = 0;
        if constexpr (MULTI)
          while (sgi + 1 < segs.n && t >= segs.seg[sgi + 1].tile0) ++sgi;
        x = (sgi << 24) | (t - segs.seg[sgi].tile0);
        need = ti.n_valid > 0 && !(p.causal && qmax_wg < ti.min_valid);
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
          int m;
          if (!red_act[w] || ti.n_valid == 0 || (p.causal && red_q[w] < ti.min_valid)) m = 0;
          else if (ti.n_valid == BN && (!p.causal || ti.max_valid <= red_qmin[w])) m = 1;
          else m = 2;
          modes |= m << (2 * w);
        }
      }
      const uint64_t bal = __ballot(need);
      if (lane == 0) wave_cnt[wave] = __builtin_popcountll(bal);
      __syncthreads();
      int off = n;
      for (int w = 0; w < wave; ++w) off += wave_cnt[w];
      int tot = n;
      for (int w = 0; w < NWAVES; ++w) tot += wave_cnt[w];
      if (need) tile_list[off + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0))] =
          make_int2(x, modes);
      __syncthreads();
      n = tot;
    }
    if (n == 0) continue;
    int issued = 0;
    for (; issued < n && issued < NSTAGE - 1; ++issued)
      load_tile(tile_src(__builtin_amdgcn_readfirstlane(tile_list[issued].x)), (int)((unsigned)issued % NSTAGE));
    // The list entries of the next step (its tile and this wave's mode, and the tile to load
    // after it) are read from LDS right after the barrier and only used after this step's
    // work, so their latency hides under it; so does the kernel-argument read of the tile's
    // block size that masked tiles use.
    const int mshift = 2 * wave;
    int x_cur = __builtin_amdgcn_readfirstlane(tile_list[0].x);
    int m_cur = __builtin_amdgcn_readfirstlane((tile_list[0].y >> mshift) & 3);
    int x_load = issued < n ? __builtin_amdgcn_readfirstlane(tile_list[issued].x) : 0;
    for (int i = 0; i < n; ++i) {
      if (pos_loader) wait_tiles_ahead<L::LOADS_PER_TILE + 1>(issued - i - 1);
      else wait_tiles_ahead<L::LOADS_PER_TILE>(issued - i - 1);
      barrier_no_fence();  // tile i landed for every wave; the stage of tile i-1 is free
      if (issued < n) {
        load_tile(tile_src(x_load), (int)((unsigned)issued % NSTAGE));
        ++issued;
      }
      if (MULTI && (x_cur >> 24) != cur_seg) {
        cur_seg = x_cur >> 24;
        cur_sk = segs.seg[cur_seg].Sk;
      }
      const int left_cur = (MULTI ? cur_sk : segs.seg[0].Sk) - (x_cur & 0xffffff) * BN;
      const int2 e_nxt = tile_list[i + 1 < n ? i + 1 : i];
      const int xl_nxt = tile_list[issued < n ? issued : 0].x;
      if (m_cur != 0) compute((int)((unsigned)i % NSTAGE), left_cur, m_cur);
      x_cur = __builtin_amdgcn_readfirstlane(e_nxt.x);
      m_cur = __builtin_amdgcn_readfirstlane((e_nxt.y >> mshift) & 3);
      x_load = __builtin_amdgcn_readfirstlane(xl_nxt);
    }
    __syncthreads();  // the next pass rewrites the list and the stages
  }

  // ---- epilogue: normalise, emit (out, lse) or merge them into the running pair
  if (!row_ok) return;
  const float l_tot = sum_halves(l_run);
  const bool empty = !(l_tot > 0.f);
  const float inv = empty ? 0.f : 1.f / l_tot;
  const float lse_new = empty ? -__builtin_inff() : m_run * fabsf(scale) + logf(l_tot);
  // a key split's partial pair (offsets 0 without splits)
  const int64_t o_split = (int64_t)split * p.split_out;
  float* lse_ptr = p.lse ? (float*)p.lse + (int64_t)split * p.split_lse + b * p.ls_b + h * p.ls_h +
                               (int64_t)row * p.ls_s
                         : nullptr;
  if (p.accumulate) {
    const float lse_old = *lse_ptr;
    // a row that sees no key of this block merges to exactly its running pair (weights 1
    // and 0); only a final output still has to be written
    if (empty && !p.final_out && lse_old > -__builtin_inff()) return;
    const float lse = logaddexp<float>(lse_old, lse_new);
    const float safe = is_finite(lse) ? lse : 0.f;
    const float w_old = expf(lse_old - safe), w_new = expf(lse_new - safe);
    float* orow = (float*)p.out + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
    // the last merge of a ring can write the result in the query dtype straight away (the
    // reference's final out.to(q.dtype)); the running output is then only read
    T* frow = p.final_out && p.final_dtype != CEA_F32
                  ? (T*)p.final_out + b * p.fs_b + (int64_t)row * p.fs_s + h * p.fs_h
                  : nullptr;
    float* ffrow = p.final_out && p.final_dtype == CEA_F32
                       ? (float*)p.final_out + b * p.fs_b + (int64_t)row * p.fs_s + h * p.fs_h
                       : orow;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int col = dt * 32 + i4 * 8 + g * 4;
        float4 prev = *(const float4*)(orow + col);
        const float o0 = oacc[dt][i4 * 4 + 0] * inv, o1 = oacc[dt][i4 * 4 + 1] * inv;
        const float o2 = oacc[dt][i4 * 4 + 2] * inv, o3 = oacc[dt][i4 * 4 + 3] * inv;
        prev.x = add_rn(mul_rn(prev.x, w_old), mul_rn(o0, w_new));
        prev.y = add_rn(mul_rn(prev.y, w_old), mul_rn(o1, w_new));
        prev.z = add_rn(mul_rn(prev.z, w_old), mul_rn(o2, w_new));
        prev.w = add_rn(mul_rn(prev.w, w_old), mul_rn(o3, w_new));
        if (frow) {
          const T v4[4] = {(T)prev.x, (T)prev.y, (T)prev.z, (T)prev.w};
          uint2 raw;
          __builtin_memcpy(&raw, v4, 8);
          *(uint2*)(frow + col) = raw;
        } else {
          *(float4*)(ffrow + col) = prev;
        }
      }
    // both halves have read lse_old before either writes it
    __builtin_amdgcn_wave_barrier();
    if (g == 0) *lse_ptr = lse;
  } else {
    if (p.out_dtype == CEA_F32) {
      float* orow = (float*)p.out + o_split + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
          *(float4*)(orow + dt * 32 + i4 * 8 + g * 4) =
              make_float4(oacc[dt][i4 * 4 + 0] * inv, oacc[dt][i4 * 4 + 1] * inv,
                          oacc[dt][i4 * 4 + 2] * inv, oacc[dt][i4 * 4 + 3] * inv);
    } else {
      T* orow = (T*)p.out + o_split + b * p.os_b + (int64_t)row * p.os_s + h * p.os_h;
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

template <typename T, int D, bool MULTI>
int launch_typed(const AttnParams& p, const KvSegs& segs, hipStream_t st) {
  const int hp = MULTI ? 1 : std::max(p.heads_per_wg, 1);
  const int nqb = (p.Sq + BM / hp - 1) / (BM / hp);
  const int64_t total = (int64_t)nqb * (p.Hq / hp) * p.B * (MULTI ? 1 : std::max(p.splits, 1));
  if (total == 0) return CEA_OK;
  CEA_REQUIRE(total < (int64_t)1 << 31, CEA_EUNSUPPORTED, "attention: grid too large");
  const hipError_t e = reserve_lds<attn_prefill_kernel<T, D, MULTI>>(Layout<D>::LDS_BYTES);
  CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "attention: cannot reserve %d bytes of LDS: %s",
              Layout<D>::LDS_BYTES, hipGetErrorString(e));
  hipLaunchKernelGGL((attn_prefill_kernel<T, D, MULTI>), dim3((unsigned)total), dim3(NTHREADS),
                     Layout<D>::LDS_BYTES, st, p, segs);
  CEA_CHECK_LAUNCH("attention_prefill");
  return CEA_OK;
}

}  // namespace

static bool al16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

KvSegs single_segment(const AttnParams& p) {
  KvSegs s;
  memset(&s, 0, sizeof(s));
  s.n = 1;
  KvSeg& g = s.seg[0];
  g.k = p.k; g.v = p.v; g.k_pos = p.k_pos;
  g.ks_b = p.ks_b; g.ks_h = p.ks_h; g.vs_b = p.vs_b; g.vs_h = p.vs_h;
  g.kps_b = p.kps_b; g.kps_s = p.kps_s;
  g.Sk = p.Sk;
  g.tile0 = 0;
  return s;
}

// everything but the KV blocks: dtypes, head size, scale, q / out / final_out layout
static bool prefill_common_ok(const AttnParams& p) {
  if (!(p.in_dtype == CEA_BF16 || p.in_dtype == CEA_F16)) return false;
  if (!(p.D == 64 || p.D == 128)) return false;
  if (!(p.out_dtype == CEA_F32 || p.out_dtype == p.in_dtype)) return false;
  if (p.accumulate && p.out_dtype != CEA_F32) return false;
  if (p.final_out) {
    if (!(p.final_dtype == CEA_F32 || p.final_dtype == p.in_dtype)) return false;
    if (p.fs_b % 4 || p.fs_s % 4 || p.fs_h % 4) return false;
    if (((uintptr_t)p.final_out & 15) != 0) return false;
  }
  // the exp2 fold needs c = |scale|*log2(e) to be a normal f32 (a zero c would turn the
  // -inf of masked scores into NaN); degenerate scales use the generic kernel
  if (!(fabs(p.scale) >= 1e-30 && fabs(p.scale) <= 1e30)) return false;
  // 16-byte fragments: 8-element aligned strides and bases
  const int64_t s8[] = {p.qs_b, p.qs_s, p.qs_h, p.ks_s, p.vs_s};
  for (int64_t s : s8)
    if (s % 8) return false;
  if (!al16(p.q) || !al16(p.out)) return false;
  const int64_t so[] = {p.os_b, p.os_s, p.os_h};
  for (int64_t s : so)
    if (s % 4) return false;
  // buffer resources address one (batch, kv head) block with 32-bit offsets: rows must not
  // overlap, and the per-lane row offsets of a tile (up to 63 rows past its first key) must
  // not wrap 32 bits
  if (p.ks_s < p.D || p.vs_s < p.D) return false;
  if ((int64_t)kTileKeys * p.ks_s * 2 >= ((int64_t)1 << 31) ||
      (int64_t)kTileKeys * p.vs_s * 2 >= ((int64_t)1 << 31))
    return false;
  return true;
}

// one KV block of a launch (row strides p.ks_s / p.vs_s)
static bool prefill_block_ok(const AttnParams& p, const KvSeg& g) {
  const int64_t s8[] = {g.ks_b, g.ks_h, g.vs_b, g.vs_h};
  for (int64_t s : s8)
    if (s % 8) return false;
  if (!al16(g.k) || !al16(g.v)) return false;
  // key positions are fetched 16 bytes at a time: contiguous, 16-byte aligned per batch
  if (g.kps_s != 1 || g.kps_b % 2 || !al16(g.k_pos)) return false;
  // tiles are addressed from 64-bit bases with 32-bit offsets inside one tile, so a block may
  // span any number of bytes; list entries hold a tile of the block in 24 bits
  return ((int64_t)g.Sk + kTileKeys - 1) / kTileKeys < ((int64_t)1 << 24);
}

int prefill_heads_per_wg(int64_t Sq, int64_t G) {
  // fewest padded query rows per head (ceil(Sq / rows) * rows - Sq with BM / hp rows of a
  // head per workgroup); the smallest count on ties, so query blocks that are multiples of
  // BM keep one head per workgroup
  int best = 1;
  int64_t best_pad = (Sq + BM - 1) / BM * BM - Sq;
  for (int hp = 2; hp <= NWAVES && G > 0 && G % hp == 0; hp *= 2) {
    const int64_t rows = BM / hp;
    const int64_t pad = (Sq + rows - 1) / rows * rows - Sq;
    if (pad < best_pad) best = hp, best_pad = pad;
  }
  return best;
}

int prefill_key_splits(int64_t B, int64_t Sq, int64_t Hq, int64_t Sk, int hp) {
  // One 8-wave workgroup per compute unit at a time: below 256 workgroups part of the device
  // idles for the whole launch (a 128-token prefill chunk at batch 1 and 32 heads has 32).
  // Splits bring the grid to about 512 workgroups, each with at least 8 tiles of keys; their
  // partials are merged afterwards.
  const int64_t rows = BM / hp;
  const int64_t grid = (Sq + rows - 1) / rows * (Hq / hp) * B;
  const int64_t tiles = (Sk + kTileKeys - 1) / kTileKeys;
  if (grid <= 0 || grid >= 256) return 1;
  int64_t s = std::min<int64_t>({(int64_t)kMaxKeySplits, (512 + grid - 1) / grid, tiles / 8});
  return s >= 2 ? (int)s : 1;
}

bool prefill_mfma_supported(const AttnParams& p) {
  return prefill_common_ok(p) && prefill_block_ok(p, single_segment(p).seg[0]);
}

bool prefill_segs_supported(const AttnParams& p, const KvSegs& segs) {
  if (p.accumulate || p.final_out || !prefill_common_ok(p)) return false;
  if (segs.n < 1 || segs.n > kMaxKvSegs) return false;
  int64_t tiles = 0;
  for (int i = 0; i < segs.n; ++i) {
    const KvSeg& g = segs.seg[i];
    if (g.Sk < 1 || g.tile0 != tiles || !prefill_block_ok(p, g)) return false;
    tiles += (g.Sk + kTileKeys - 1) / kTileKeys;
  }
  // list entries hold the block in bits 24.. and its tile in bits 0..23
  return tiles == p.ntiles && tiles < ((int64_t)1 << 24);
}

template <bool MULTI>
static int launch_dispatch(const AttnParams& p, const KvSegs& segs, hipStream_t st) {
  if (p.in_dtype == CEA_BF16) {
    if (p.D == 128) return launch_typed<bf16, 128, MULTI>(p, segs, st);
    if (p.D == 64) return launch_typed<bf16, 64, MULTI>(p, segs, st);
  } else if (p.in_dtype == CEA_F16) {
    if (p.D == 128) return launch_typed<f16, 128, MULTI>(p, segs, st);
    if (p.D == 64) return launch_typed<f16, 64, MULTI>(p, segs, st);
  }
  set_error("attention: MFMA path does not cover dtype %s, head size %d",
            dtype_name(p.in_dtype), p.D);
  return CEA_EUNSUPPORTED;
}

int launch_attn_prefill_mfma(const AttnParams& p, hipStream_t st) {
  return launch_dispatch<false>(p, single_segment(p), st);
}

int launch_attn_prefill_segs(const AttnParams& p, const KvSegs& segs, hipStream_t st) {
  if (segs.n == 1) return launch_dispatch<false>(p, segs, st);
  return launch_dispatch<true>(p, segs, st);
}

}  // namespace cea
