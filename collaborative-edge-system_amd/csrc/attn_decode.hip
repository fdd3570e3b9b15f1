// Split-KV decode attention with LSE for short query blocks (decoding against a KV cache).
//
// Covers attention_with_lse (collab_infer/parallel/attention.py:201-239) when the query block
// is a few tokens, and the per-device compute of distributed_kv_attention
// (collab_infer/parallel/sequence_parallel.py:250-280): every KV partition's partial
// (out, lse) and their exact merge (merge_attention_list, attention.py:253-264), all on one
// device and in three launches.
//
// HBM-bound design:
//   * work item = (batch, kv head, one or two consecutive key chunks of one partition); the
//     NR = Sq*G query rows that share the kv head (G query heads per kv head) are the columns
//     of 16 x 16 matrix-core tiles, so each K/V row is read from HBM once for all of them and
//     the arithmetic stays off the vector ALU: S = K.Q^T with v_mfma_f32_16x16x32 (a lane
//     holds 4 keys of one query row) and O^T += V^T.P^T with v_mfma_f32_16x16x16 (P is the
//     score tile as is);
//   * every wave streams its own 16-key tiles of K and V straight into a private pair of LDS
//     buffers (non-temporal buffer_load ... lds, explicit vmcnt waits, no barriers); a buffer
//     is refilled as soon as its fragments are in registers, so two tiles stay in flight; V is
//     read back transposed with ds_read_b64_tr_b16; both tiles are XOR-swizzled so the
//     fragment and transpose reads are free of LDS bank conflicts; the query rows come in by
//     LDS-DMA as well, together with the item's tile masks;
//   * a prepass reads the key positions once per batch row (not once per kv head) and turns
//     them into a 16-bit visibility word per key (bit s: query s sees it) and a mask of the
//     16-key tiles of each chunk that hold a visible key; the split kernel loads each tile's
//     words with its K and V, never loads an invisible tile, and an item with empty masks
//     writes nothing;
//   * the waves of a workgroup merge their online-softmax partials in LDS and write one
//     (o unnormalised, m, l) partial per item with non-temporal stores (stores during the
//     K/V stream cost its read rate far more than their size, so there are as few partial
//     bytes as the tail allows: pairs of chunks per item except in the last batch rows);
//   * the reduction kernel merges the items of a row (optionally emitting each partition's
//     (out, lse)), computes lse with the reference's logsumexp over partitions, and writes
//     out (f32 or the query dtype) and lse.
#include "cea_kernels.hpp"
#include "cea_lds_dma.hpp"

namespace cea {
namespace {

constexpr int DTHREADS = 256;
constexpr int NW = DTHREADS / 64;     // waves per workgroup
constexpr int TK = 16;                // keys per tile
#ifndef CEA_DECODE_CHMAX
#define CEA_DECODE_CHMAX 1024
#endif
#ifndef CEA_DECODE_ITEMS
#define CEA_DECODE_ITEMS 8192
#endif
constexpr int CHMAX = CEA_DECODE_CHMAX;  // keys per chunk at most
static_assert(CHMAX % DTHREADS == 0 && CHMAX <= 4 * DTHREADS, "one 64-bit tile mask per chunk");
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
  static constexpr int VIS_OFF = 2 * TILE_BYTES;    // 16 visibility words after K and V
  static constexpr int BUF_BYTES = VIS_OFF + 64;
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
// the same over the lane pairs l, l ^ 16 (v_permlane16_swap: rows 0 and 1, rows 2 and 3)
__device__ __forceinline__ float max_rows16(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float sum_rows16(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto sw = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}
// max / sum over the 64 lanes, the result in every lane, without LDS round trips: each step
// pairs every lane with one partner (xor 1 and xor 2 by DPP quad permutes, the quads of a
// half-row by DPP row_half_mirror, the half-rows by row_mirror, then l ^ 16 and l ^ 32 by
// the permlane swaps), so both lanes of a pair combine the same two values and all lanes
// end with the bitwise same result
#define CEA_DPP_F32(x, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), (ctrl), 0xf, 0xf, false))
__device__ __forceinline__ float wave_max_lanes(float v) {
  v = __builtin_fmaxf(v, CEA_DPP_F32(v, 0xB1));   // quad_perm [1,0,3,2]
  v = __builtin_fmaxf(v, CEA_DPP_F32(v, 0x4E));   // quad_perm [2,3,0,1]
  v = __builtin_fmaxf(v, CEA_DPP_F32(v, 0x141));  // row_half_mirror
  v = __builtin_fmaxf(v, CEA_DPP_F32(v, 0x140));  // row_mirror
  return max_halves(max_rows16(v));
}
__device__ __forceinline__ float wave_sum_lanes(float v) {
  v = v + CEA_DPP_F32(v, 0xB1);
  v = v + CEA_DPP_F32(v, 0x4E);
  v = v + CEA_DPP_F32(v, 0x141);
  v = v + CEA_DPP_F32(v, 0x140);
  return sum_halves(sum_rows16(v));
}
#undef CEA_DPP_F32

__device__ __forceinline__ int part_of(const DecodeParams& p, int chunk) {
  int part = 0;
  while (part + 1 < p.nparts && chunk >= p.chunk_begin[part + 1]) ++part;
  return part;
}

// Work items of the split kernel.  Batch rows b < p.pair_rows take pairs of consecutive chunks
// of a partition (item_begin: prefix of pair items per partition), the remaining rows single
// chunks (chunk_begin), so the last workgroups of the launch, which set its tail, are short.
// Item i of row b: its partition, first chunk and chunk count.
struct DecodeItem {
  int part, chunk, nch;
};
__device__ __forceinline__ DecodeItem item_of(const DecodeParams& p, int b, int item) {
  DecodeItem it;
  if (b < p.pair_rows) {
    int part = 0;
    while (part + 1 < p.nparts && item >= p.item_begin[part + 1]) ++part;
    it.part = part;
    it.chunk = p.chunk_begin[part] + 2 * (item - p.item_begin[part]);
    it.nch = min(2, p.chunk_begin[part + 1] - it.chunk);
  } else {
    it.part = part_of(p, item);
    it.chunk = item;
    it.nch = 1;
  }
  return it;
}
__device__ __forceinline__ int items_of_row(const DecodeParams& p, int b) {
  return b < p.pair_rows ? p.item_begin[p.nparts] : p.chunk_begin[p.nparts];
}

// Visibility prepass, one workgroup per (chunk, batch): for every key of the chunk a word whose
// bit s says whether query s of the batch sees it (k_pos >= 0 and, when causal,
// k_pos <= q_pos[s]), and for the chunk a mask of the 16-key tiles holding a visible key.
// The split kernel then never reads positions, and skips invisible tiles without loading them.
__global__ __launch_bounds__(DTHREADS) void decode_vis_kernel(const DecodeParams p) {
  const int chunk = blockIdx.x, b = blockIdx.y;
  const int part = part_of(p, chunk);
  const int key0 = (chunk - p.chunk_begin[part]) * p.chunk;
  const int nkeys = min(p.chunk, p.Sk[part] - key0);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int total_chunks = p.chunk_begin[p.nparts];
  __shared__ uint32_t wmask[NW];
  // every load is issued before the first wait (key indices clamped into the chunk)
  const int64_t* kp = p.k_pos[part] + b * p.kps[part][0];
  const int64_t kps = p.kps[part][1];
  int64_t pk[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) pk[u] = kp[(int64_t)(key0 + min(tid * 4 + u, nkeys - 1)) * kps];
  uint32_t words[4] = {0u, 0u, 0u, 0u};
  for (int q = 0; q < p.Sq; ++q) {
    const int64_t qs = p.q_pos[b * p.qps_b + (int64_t)q * p.qps_s];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (tid * 4 + u < nkeys && pk[u] >= 0 && (!p.causal || pk[u] <= qs)) words[u] |= 1u << q;
  }
  if (tid * 4 < p.chunk) {
    uint2 packed = {words[0] | (words[1] << 16), words[2] | (words[3] << 16)};
    *(uint2*)(p.vis + ((int64_t)b * total_chunks + chunk) * p.chunk + tid * 4) = packed;
  }
  // lanes 4j..4j+3 of wave w hold tile w*16 + j
  const uint64_t bal = __ballot((words[0] | words[1] | words[2] | words[3]) != 0);
  if (lane == 0) {
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) m |= (((bal >> (4 * j)) & 0xfu) != 0 ? 1u : 0u) << j;
    wmask[wave] = m;
  }
  __syncthreads();
  if (tid == 0) {
    uint64_t m = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) m |= (uint64_t)wmask[w] << (16 * w);
    p.tile_mask[(int64_t)b * total_chunks + chunk] = m;
  }
}

// Partial layout: [B][Hkv][total_chunks][NR][D + 2] floats: o (relative to m), m, l, where
// m is in natural-log units (max of scale*q.k) and l = sum exp(scale*q.k - m).
template <typename T, int D, int NR>
__global__ __launch_bounds__(DTHREADS, 2) void decode_split_kernel(const DecodeParams p) {
  typedef DLayout<D> L;
  typedef typename Mfma16<T>::frag8 frag8;
  extern __shared__ __attribute__((aligned(16))) char dsmem[];
  __shared__ float red_m[NW][NR];
  __shared__ float red_l[NW][NR];

  // 1-D grid: pair items of rows [0, pair_rows), then single-chunk items of the other rows;
  // item fastest, then unit, then batch row - except when several units read one KV head
  // (per_head): units go fastest then, so those reading one KV head's chunk run side by side
  // and share its reads in the caches
  const int total_chunks = p.chunk_begin[p.nparts];
  int b, unit, item;
  {
    const int n2 = p.item_begin[p.nparts];
    const int first = p.pair_rows * p.units * n2;
    const int id = blockIdx.x;
    const int r = id < first ? id : id - first;
    const int ni = id < first ? n2 : total_chunks;  // items per (row, unit)
    b = (id < first ? 0 : p.pair_rows) + r / (p.units * ni);
    if (p.per_head) {
      unit = r % p.units;
      item = (r / p.units) % ni;
    } else {
      unit = (r / ni) % p.units;
      item = r % ni;
    }
  }
  const int kvh = p.map.kv_of(unit * p.G);  // KV head the unit's query heads read
  const DecodeItem it = item_of(p, b, item);
  const int part = it.part, chunk = it.chunk, nch = it.nch;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float* part_out = p.partial + (((int64_t)b * p.units + unit) * total_chunks + item) * NR * (D + 2);
  const int row = lane & 15;   // query row (MFMA column) of this lane
  const int grp = lane >> 4;   // 4-key group of the 16-key tile
  const int G = p.G;
  const bool row_real = row < p.Sq * G;
  const int qbit = row / G;    // query index s of this row
  char* wb = dsmem + wave * L::WAVE_BYTES;

  // ---- the query rows r = s * G + g of this kv head come straight into the wave's first tile
  // buffer (free until the first tile load), in flight together with the chunk's tile mask, so
  // the workgroup starts streaming after one memory round trip
  {
    constexpr int QROWS = 1024 / L::ROW;  // query rows one 1 KB load covers
    constexpr int QLOADS = NR <= QROWS ? 1 : NR / QROWS;
    const i32x4 qrs = make_rsrc((const T*)p.q + b * p.qs_b,
                                (uint32_t)((((int64_t)p.Sq - 1) * p.qs_s + ((int64_t)p.Hq - 1) * p.qs_h + D) * sizeof(T)));
#pragma unroll
    for (int i = 0; i < QLOADS; ++i) {
      const int r = i * QROWS + lane / (L::ROW / 16);
      const int rr = r < p.Sq * G ? r : 0;  // padding rows read row 0 (zeroed below)
      const uint32_t off = (uint32_t)(((int64_t)(rr / G) * p.qs_s + (int64_t)(unit * G + rr % G) * p.qs_h) * sizeof(T)) +
                           (lane % (L::ROW / 16)) * 16;
      buffer_load_lds16(qrs, wb + i * 1024, off);
    }
  }
  const uint64_t mask = p.tile_mask[(int64_t)b * total_chunks + chunk];
  const uint64_t mask1 = nch > 1 ? p.tile_mask[(int64_t)b * total_chunks + chunk + 1] : 0ull;
  wait_vmcnt<0>();  // query rows in LDS (also before an early exit frees the LDS)
  // no key of the item is visible to any query row: no partial (the reduction reads the masks)
  if ((mask | mask1) == 0) return;
  const int Sk = p.Sk[part];
  const int key0 = (chunk - p.chunk_begin[part]) * p.chunk;

  // ---- this lane's Q fragments (B operand of S = K.Q^T), sign folded for a negative scale
  const float scale = (float)p.scale;
  const float c = fabsf(scale) * 1.4426950408889634f;  // exp2 units
  const float grow_thr = kRescaleLog2 / c;
  const uint32_t flip = scale < 0.f ? 0x80008000u : 0u;
  frag8 qf[D / 32];
  {
    const char* qs = wb + (row_real ? row : 0) * (D * 2);
    const uint32_t keep = row_real ? 0xffffffffu : 0u;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      u32x4 raw = *(const u32x4*)(qs + ks * 64 + grp * 16);
#pragma unroll
      for (int w = 0; w < 4; ++w) raw[w] = (raw[w] ^ flip) & keep;
      __builtin_memcpy(&qf[ks], &raw, 16);
    }
  }
  wait_lgkmcnt0();  // Q in registers before the first tile load overwrites the buffer

  // ---- per-lane constant offsets
  const char* kbase = (const char*)((const T*)p.k[part] + b * p.ks[part][0] + kvh * p.ks[part][2]);
  const char* vbase = (const char*)((const T*)p.v[part] + b * p.vs[part][0] + kvh * p.vs[part][2]);
  const char* visbase = (const char*)(p.vis + ((int64_t)b * total_chunks + chunk) * p.chunk);
  const uint32_t krow = (uint32_t)(p.ks[part][1] * sizeof(T)), vrow = (uint32_t)(p.vs[part][1] * sizeof(T));
  uint32_t k_voff[L::LOADS], v_voff[L::LOADS];
#pragma unroll
  for (int i = 0; i < L::LOADS; ++i) {
    const int r = i * (1024 / L::ROW) + lane / (L::ROW / 16);
    const int pg = lane % (L::ROW / 16);                   // physical 16-byte group
    k_voff[i] = r * krow + ((pg ^ (r & (L::ROW / 16 - 1))) << 4);          // K: 16-byte groups ^ row
    const int lgv = ((((pg >> 1) ^ (r & (L::ROW / 32 - 1))) << 1) | (pg & 1));  // V: 32-byte blocks ^ row
    v_voff[i] = r * vrow + (lgv << 4);
  }
  uint32_t k_raddr[D / 32];  // A operand of S: key 'row', features grp*8 + 32*ks
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks)
    k_raddr[ks] = row * L::ROW + (((grp + 4 * ks) ^ (row & (L::ROW / 16 - 1))) << 4);
  uint32_t v_raddr[D / 16];  // transposing reads: source lane s of group grp -> key grp*4 + s/4
  {
    const int vr = grp * 4 + (row >> 2);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      v_raddr[dt] = L::TILE_BYTES + vr * L::ROW + ((dt ^ (vr & (L::ROW / 32 - 1))) << 5) + 8 * (row & 3);
  }

  // this wave's tiles: wave, wave + NW, ... that hold a visible key (tile t of the item is
  // tile t % tpc of its chunk t / tpc; tpc is a multiple of NW, so the lane pattern is the same
  // in both chunks of a pair)
  const int tpc = p.chunk / TK;
  uint64_t todo = mask & (0x1111111111111111ull << wave);
  uint64_t todo1 = mask1 & (0x1111111111111111ull << wave);
  auto pop_tile = [&]() -> int {
    if (todo != 0) {
      const int t = (int)__builtin_ctzll(todo);
      todo &= todo - 1;
      return t;
    }
    if (todo1 == 0) return -1;
    const int t = (int)__builtin_ctzll(todo1);
    todo1 &= todo1 - 1;
    return tpc + t;
  };
  auto load_tile = [&](int t, int buf) {
    const int k0 = key0 + t * TK;
    const uint32_t rows = (uint32_t)min(Sk - k0, TK);  // rows past the end of the keys read 0
    const i32x4 krs = make_rsrc(kbase + (int64_t)k0 * krow, (rows - 1) * krow + L::ROW);
    const i32x4 vrs = make_rsrc(vbase + (int64_t)k0 * vrow, (rows - 1) * vrow + L::ROW);
    char* kb = wb + buf * L::BUF_BYTES;
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) buffer_load_lds16_nt(krs, kb + i * 1024, k_voff[i]);
#pragma unroll
    for (int i = 0; i < L::LOADS; ++i) buffer_load_lds16_nt(vrs, kb + L::TILE_BYTES + i * 1024, v_voff[i]);
    if (lane < TK * 2 / 4) {  // 16 visibility words, 4 bytes per lane
      const i32x4 wrs = make_rsrc(visbase + t * TK * 2, TK * 2);
      buffer_load_lds4(wrs, kb + L::VIS_OFF, lane * 4);
    }
  };
  constexpr int LOADS_PER_TILE = 2 * L::LOADS + 1;

  f32x4 o[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff(), m_use = 0.f, l_run = 0.f;

  // Fragments of one tile, read from LDS before the math so the buffer can be refilled.
  struct Frags {
    frag8 k[D / 32];
    s16x4 v[D / 16];
    uint2 vis;
  };
  auto read_frags = [&](int buf, Frags& f) {
    const char* kb = wb + buf * L::BUF_BYTES;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) f.k[ks] = *(const frag8*)(kb + k_raddr[ks]);
    f.vis = *(const uint2*)(kb + L::VIS_OFF + grp * 8);  // keys grp*4 .. grp*4+3
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      f.v[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(kb + v_raddr[dt]));
  };
  auto compute = [&](const Frags& f) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) s = Mfma16<T>::qk(f.k[ks], qf[ks], s);
    // lane holds keys grp*4 + i of the tile for query row 'row'
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = ((i < 2 ? f.vis.x : f.vis.y) >> (16 * (i & 1))) & 0xffffu;
      const bool vis = row_real && ((word >> qbit) & 1u);
      if (!vis) s[i] = -__builtin_inff();
    }
    float mx = __builtin_fmaxf(__builtin_fmaxf(s[0], s[1]), __builtin_fmaxf(s[2], s[3]));
    mx = max_halves(max_rows16(mx));
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
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) o[dt] = Mfma16<T>::pv(f.v[dt], pf, o[dt]);
  };

  // ---- per-wave stream over its tiles: two buffers, refilled as soon as their fragments are
  // in registers, so two tiles are in flight during the math of a third
  {
    int t = pop_tile();
    int t1 = pop_tile();
    int buf = 0;
    if (t >= 0) load_tile(t, 0);
    if (t1 >= 0) load_tile(t1, 1);
    while (t >= 0) {
      if (t1 >= 0)
        wait_vmcnt<LOADS_PER_TILE>();  // tile t landed; tile t1 may still be in flight
      else
        wait_vmcnt<0>();
      Frags f;
      read_frags(buf, f);
      const int t2 = pop_tile();
      if (t2 >= 0) {
        wait_lgkmcnt0();  // fragments in registers before the buffer is refilled
        load_tile(t2, buf);
      }
      compute(f);
      t = t1;
      t1 = t2;
      buf ^= 1;
    }
  }

  // ---- merge the waves of the workgroup and write the chunk partial
  const float l_row = sum_halves(sum_rows16(l_run));
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
    // non-temporal stores: written back past the caches' keep-set, they disturb the K/V read
    // stream of the other workgroups far less than ordinary write-backs do
    __builtin_nontemporal_store(acc, part_out + r * (D + 2) + d);
    if (d == 0) {
      __builtin_nontemporal_store(M, part_out + r * (D + 2) + D);
      __builtin_nontemporal_store(Lsum, part_out + r * (D + 2) + D + 1);
    }
  }
}

// Reduction of the chunk partials, one workgroup of RTHREADS per (b, s, h) output row.
//   1. the (m, l) of every chunk into LDS, the first chunk outputs into registers;
//   2. in one wave: per partition M_p = max m, L_p = sum l * exp(m - M_p), lse_p = M_p +
//      log L_p; then lse = logsumexp over partitions (the reference merge's formula) and
//      per-chunk weights W = exp(m - lse), which fold a chunk's partition normalisation and
//      its merge weight;
//   3. out = sum over chunks of o * W, the waves taking interleaved chunks (all loads of a
//      row independent), combined in a fixed order.  Partition outputs, when requested, are
//      the same sums restricted to a partition, times exp(lse - lse_p).
constexpr int RTHREADS = 256;
constexpr int RWAVES = RTHREADS / 64;
constexpr int RCH = kDecodeMaxChunks;  // work items of a row at most (m and weight in LDS)
constexpr int RPF = 12;                // chunk outputs per wave read ahead of their weights

// Output features per lane: D / 64 consecutive floats (a float2 for D = 128, one float for 64).
template <int D> struct RVec;
template <> struct RVec<128> {
  typedef float2 V;
  static __device__ __forceinline__ V load(const float* q) { return *(const float2*)q; }
  static __device__ __forceinline__ V fma(V a, float w, V c) {
    return V{__builtin_fmaf(a.x, w, c.x), __builtin_fmaf(a.y, w, c.y)};
  }
  static __device__ __forceinline__ V add(V a, V b) { return V{a.x + b.x, a.y + b.y}; }
  static __device__ __forceinline__ float get(V a, int i) { return i ? a.y : a.x; }
};
template <> struct RVec<64> {
  typedef float V;
  static __device__ __forceinline__ V load(const float* q) { return *q; }
  static __device__ __forceinline__ V fma(V a, float w, V c) { return __builtin_fmaf(a, w, c); }
  static __device__ __forceinline__ V add(V a, V b) { return a + b; }
  static __device__ __forceinline__ float get(V a, int) { return a; }
};

template <typename O, int D, int NR>
__global__ __launch_bounds__(RTHREADS) void decode_reduce_kernel(const DecodeParams p) {
  typedef RVec<D> RV;
  typedef typename RV::V V;
  constexpr int FPL = D / 64;  // output features per lane
  const int row = blockIdx.x;  // (b, s, h)
  const int h = row % p.Hq;
  const int s = (row / p.Hq) % p.Sq;
  const int b = row / (p.Hq * p.Sq);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int unit = h / p.G;  // the work unit that computed this head
  const int r = s * p.G + (h - unit * p.G);
  const int total_chunks = p.chunk_begin[p.nparts];
  const int total = items_of_row(p, b);  // work items (partials) of this batch row
  const int* ibegin = b < p.pair_rows ? p.item_begin : p.chunk_begin;
  const int64_t cstride = (int64_t)NR * (D + 2);
  const float* base = p.partial + ((int64_t)b * p.units + unit) * total_chunks * cstride + r * (D + 2);

  // m of every item of the row, then its weight: 2 x total_chunks floats of dynamic LDS
  extern __shared__ float stage_s[];
  float* m_s = stage_s;
  float* w_s = stage_s + total_chunks;
  __shared__ V acc_s[RWAVES][64];

  // the first chunk outputs of this wave, read now so their latency overlaps the statistics
  // (chunks past the end read chunk 0; unused)
  V pre[RPF];
#pragma unroll
  for (int k = 0; k < RPF; ++k) {
    const int j = wave + RWAVES * k;
    pre[k] = total > 0 ? RV::load(base + (j < total ? j : 0) * cstride + FPL * lane) : V{};
  }
  // items without a visible key wrote no partial: their weight is 0
  const uint64_t* cmask = p.tile_mask + (int64_t)b * total_chunks;
  auto item_ml = [&](int j) -> float2 {  // (m, l) of item j, (-inf, 0) for an empty item
    const DecodeItem it = item_of(p, b, j);
    const bool live = (cmask[it.chunk] | (it.nch > 1 ? cmask[it.chunk + 1] : 0ull)) != 0;
    const float2 ml = *(const float2*)(base + j * cstride + D);
    return live ? ml : make_float2(-__builtin_inff(), 0.f);
  };
  // lse = logsumexp over the partitions' lse_p (the reference merge's formula)
  auto combine = [&](const float (&lp)[CEA_MAX_PARTS]) -> float {
    if (p.nparts == 1) return lp[0];
    float mx = -__builtin_inff();
    for (int part = 0; part < p.nparts; ++part) mx = fmaxf(mx, lp[part]);
    const float shift = is_inf(mx) ? 0.f : mx;
    float sum = 0.f;
    for (int part = 0; part < p.nparts; ++part) sum = add_rn(sum, expf(lp[part] - shift));
    return logf(sum) + shift;
  };
  // statistics in wave 0 alone (lane reductions, no workgroup barriers): per partition
  // M_p = max m, L_p = sum l * exp(m - M_p), lse_p = M_p + log L_p; then lse and the item
  // weights exp(m - lse)
  __shared__ float s_lse[CEA_MAX_PARTS + 1];
  float lp[CEA_MAX_PARTS];
  if (total <= 64) {
    // one item per lane: its (m, l) stays in registers from the load to the weight, and the
    // workgroup waits at one barrier (the weights) instead of two
    if (wave == 0) {
      const float2 ml = lane < total ? item_ml(lane) : make_float2(-__builtin_inff(), 0.f);
      for (int part = 0; part < p.nparts; ++part) {
        const bool in = lane >= ibegin[part] && lane < ibegin[part + 1];
        const float mx = wave_max_lanes(in ? ml.x : -__builtin_inff());
        const bool use = in && mx != -__builtin_inff() && ml.x != -__builtin_inff();
        const float l = wave_sum_lanes(use ? ml.y * expf(ml.x - mx) : 0.f);
        lp[part] = l > 0.f ? mx + logf(l) : -__builtin_inff();
      }
      const float lse = combine(lp);
      const bool empty = lse == -__builtin_inff();
      if (lane < total) w_s[lane] = (empty || ml.x == -__builtin_inff()) ? 0.f : expf(ml.x - lse);
      if (lane == 0) {
        for (int part = 0; part < p.nparts; ++part) s_lse[part] = lp[part];
        s_lse[p.nparts] = lse;
      }
    }
  } else {
    for (int j = tid; j < total; j += RTHREADS) {
      const float2 ml = item_ml(j);
      m_s[j] = ml.x;
      w_s[j] = ml.y;  // l, replaced by the weight below
    }
    __syncthreads();
    if (wave == 0) {
      for (int part = 0; part < p.nparts; ++part) {
        const int c0 = ibegin[part], c1 = ibegin[part + 1];
        float mx = -__builtin_inff();
        for (int j = c0 + lane; j < c1; j += 64) mx = fmaxf(mx, m_s[j]);
        mx = wave_max_lanes(mx);
        float l = 0.f;
        if (mx != -__builtin_inff())
          for (int j = c0 + lane; j < c1; j += 64)
            if (m_s[j] != -__builtin_inff()) l = __builtin_fmaf(w_s[j], expf(m_s[j] - mx), l);
        l = wave_sum_lanes(l);
        lp[part] = l > 0.f ? mx + logf(l) : -__builtin_inff();
      }
      const float lse = combine(lp);
      const bool empty = lse == -__builtin_inff();
      for (int j = lane; j < total; j += 64)
        w_s[j] = (empty || m_s[j] == -__builtin_inff()) ? 0.f : expf(m_s[j] - lse);
      if (lane == 0) {
        for (int part = 0; part < p.nparts; ++part) s_lse[part] = lp[part];
        s_lse[p.nparts] = lse;
      }
    }
  }
  __syncthreads();
  float lse_p[CEA_MAX_PARTS];
  for (int part = 0; part < p.nparts; ++part) lse_p[part] = s_lse[part];
  const float lse = s_lse[p.nparts];

  // weighted sum of the chunk outputs over [c0, c1): wave w takes chunks w, w + 4, ...; the
  // first RPF of them came in with the statistics (pre), later ones are read when their weight
  // is known (a chunk of weight 0 is never read or used: it may hold no partial)
  auto chunk_sum = [&](int c0, int c1) -> V {
    V a{};
#pragma unroll
    for (int k = 0; k < RPF; ++k) {
      const int j = wave + RWAVES * k;
      if (j >= c0 && j < c1) {
        const float w = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(w_s[j])));
        a = w != 0.f ? RV::fma(pre[k], w, a) : a;
      }
    }
    const int j0 = wave + RWAVES * RPF;
    for (int j = j0 + ((c0 > j0 ? c0 - j0 + RWAVES - 1 : 0) / RWAVES) * RWAVES; j < c1; j += RWAVES) {
      const float w = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(w_s[j])));
      if (w != 0.f) a = RV::fma(RV::load(base + j * cstride + FPL * lane), w, a);
    }
    acc_s[wave][lane] = a;
    __syncthreads();
    V t = acc_s[0][lane];
#pragma unroll
    for (int i = 1; i < RWAVES; ++i) t = RV::add(t, acc_s[i][lane]);
    __syncthreads();
    return t;
  };

  V res;
  if (p.part_out[0]) {
    res = V{};
    for (int part = 0; part < p.nparts; ++part) {
      const V t = chunk_sum(ibegin[part], ibegin[part + 1]);
      res = RV::add(res, t);
      if (wave == 0) {
        const bool pe = lse_p[part] == -__builtin_inff();
        const float f = pe ? 0.f : expf(lse - lse_p[part]);
        float* po = (float*)p.part_out[part] + b * p.pos_[part][0] + s * p.pos_[part][1] + h * p.pos_[part][2];
#pragma unroll
        for (int i = 0; i < FPL; ++i) po[FPL * lane + i] = RV::get(t, i) * f;
        if (lane == 0) {
          float* pl = (float*)p.part_lse[part] + b * p.pls_[part][0] + h * p.pls_[part][1] + s * p.pls_[part][2];
          *pl = lse_p[part];
        }
      }
    }
  } else {
    res = chunk_sum(0, total);
  }
  if (wave != 0) return;
  float* lptr = p.lse ? (float*)p.lse + b * p.ls_b + h * p.ls_h + s * p.ls_s : nullptr;
  O* optr = (O*)p.out + b * p.os_b + s * p.os_s + h * p.os_h + FPL * lane;
  if (p.accumulate) {  // merge_attention(running, new)
    const float lse_old = *lptr;
    const float lm = logaddexp<float>(lse_old, lse);
    const float safe = is_finite(lm) ? lm : 0.f;
    const float fo = expf(lse_old - safe), fn = expf(lse - safe);
    float v[FPL];
#pragma unroll
    for (int i = 0; i < FPL; ++i) v[i] = add_rn(mul_rn((float)optr[i], fo), mul_rn(RV::get(res, i), fn));
#pragma unroll
    for (int i = 0; i < FPL; ++i) optr[i] = (O)v[i];
    if (lane == 0) *lptr = lm;  // the wave's loads of lse_old precede this store
  } else {
#pragma unroll
    for (int i = 0; i < FPL; ++i) optr[i] = (O)RV::get(res, i);
    if (lptr && lane == 0) *lptr = lse;
  }
}

template <typename T, int D, int NR>
int launch_nr(const DecodeParams& p, hipStream_t st) {
  const int total = p.chunk_begin[p.nparts];
  if (total > 0) {
    hipLaunchKernelGGL(decode_vis_kernel, dim3(total, p.B), dim3(DTHREADS), 0, st, p);
    CEA_CHECK_LAUNCH("decode_vis");
    const hipError_t e = reserve_lds<decode_split_kernel<T, D, NR>>(DLayout<D>::LDS_BYTES);
    CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "decode: cannot reserve %d bytes of LDS: %s",
                DLayout<D>::LDS_BYTES, hipGetErrorString(e));
    const int64_t grid = ((int64_t)p.pair_rows * p.item_begin[p.nparts] + (int64_t)(p.B - p.pair_rows) * total) * p.units;
    hipLaunchKernelGGL((decode_split_kernel<T, D, NR>), dim3((unsigned)grid), dim3(DTHREADS),
                       DLayout<D>::LDS_BYTES, st, p);
    CEA_CHECK_LAUNCH("decode_split");
  }
  const int rows = p.B * p.Sq * p.Hq;
  if (rows == 0) return CEA_OK;
  const int stage = 2 * total * (int)sizeof(float);
  hipError_t e;
  if (p.out_dtype == CEA_F32) {
    e = reserve_lds<decode_reduce_kernel<float, D, NR>>(2 * RCH * (int)sizeof(float));
    if (e == hipSuccess)
      hipLaunchKernelGGL((decode_reduce_kernel<float, D, NR>), dim3(rows), dim3(RTHREADS), stage, st, p);
  } else if (p.out_dtype == CEA_BF16) {
    e = reserve_lds<decode_reduce_kernel<bf16, D, NR>>(2 * RCH * (int)sizeof(float));
    if (e == hipSuccess)
      hipLaunchKernelGGL((decode_reduce_kernel<bf16, D, NR>), dim3(rows), dim3(RTHREADS), stage, st, p);
  } else {
    e = reserve_lds<decode_reduce_kernel<f16, D, NR>>(2 * RCH * (int)sizeof(float));
    if (e == hipSuccess)
      hipLaunchKernelGGL((decode_reduce_kernel<f16, D, NR>), dim3(rows), dim3(RTHREADS), stage, st, p);
  }
  CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "decode: cannot reserve %d bytes of LDS: %s",
              2 * RCH * (int)sizeof(float), hipGetErrorString(e));
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
  if (!(D == 64 || D == 128)) return false;
  // the regular grouping shares each K/V row among the query heads of a KV head (all of
  // them, or a divisor of the group whose rows fit one unit); any other map runs one unit per
  // query head
  if (map.group > 0) return decode_rows(Sq, 1) != 0;
  return Hq <= CEA_MAX_MAPPED_HEADS && decode_rows(Sq, 1) != 0;
}

// Work items wanted per launch: enough to fill 256 CUs several times.  An item's bytes per key
// scale with the head size, so the count scales with it too (a head size of 64 takes half as
// many, twice the keys each: the same bytes per item as at 128).
static int64_t decode_item_target(int32_t D) { return (int64_t)CEA_DECODE_ITEMS * D / 128; }

int decode_plan_chunk(int64_t keys_per_head, int32_t B, int32_t units, int32_t D) {
  // chunks of 256..1024 keys
  const int64_t heads = (int64_t)B * units;
  int ch = 256;
  while (ch < CHMAX && heads * ((keys_per_head + ch - 1) / ch) > decode_item_target(D)) ch *= 2;
  return ch;
}

int launch_attn_decode(const DecodeParams& params, hipStream_t st) {
  DecodeParams p = params;
  const int nr = decode_rows(p.Sq, p.G);
  CEA_REQUIRE(p.chunk <= CHMAX && p.chunk % TK == 0, CEA_EINVAL, "decode: bad chunk %d", p.chunk);
  CEA_REQUIRE(p.chunk_begin[p.nparts] <= kDecodeMaxChunks, CEA_EUNSUPPORTED,
              "decode: %d chunks exceed %d", p.chunk_begin[p.nparts], kDecodeMaxChunks);
  // Pair items (half the partials written while K/V stream: those writes cost the read stream
  // far more than their size) once chunks are at their largest and plentiful.  The last batch
  // rows keep single chunks: enough of them for about two rounds of resident workgroups (two
  // per compute unit), so the launch ends on short workgroups.
  p.item_begin[0] = 0;
  for (int i = 0; i < p.nparts; ++i)
    p.item_begin[i + 1] = p.item_begin[i] + (p.chunk_begin[i + 1] - p.chunk_begin[i] + 1) / 2;
  const int64_t row_items = (int64_t)p.units * p.chunk_begin[p.nparts];
  const bool pairs = p.chunk == CHMAX && p.B * row_items >= decode_item_target(p.D);
  const int cus = device_cus();
  const int64_t tail_rows = row_items > 0 ? (4 * (int64_t)(cus > 0 ? cus : 256) + row_items - 1) / row_items : 1;
  p.pair_rows = pairs ? (int)max((int64_t)0, (int64_t)p.B - tail_rows) : 0;
  if (p.D == 128 && p.in_dtype == CEA_BF16) return launch_d<bf16, 128>(p, nr, st);
  if (p.D == 128 && p.in_dtype == CEA_F16) return launch_d<f16, 128>(p, nr, st);
  if (p.D == 64 && p.in_dtype == CEA_BF16) return launch_d<bf16, 64>(p, nr, st);
  if (p.D == 64 && p.in_dtype == CEA_F16) return launch_d<f16, 64>(p, nr, st);
  set_error("decode: unsupported dtype %s / head size %d", dtype_name(p.in_dtype), p.D);
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
