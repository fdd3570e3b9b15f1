// Column-parallel projection GEMMs on gfx950 matrix cores.
//
//   plain  y[M, N] = x[M, K] . w[N, K]^T (+ bias[N]), f32 accumulation rounded once to the
//          input dtype: F.linear(x, self.weight, self.bias) of FusedColumnParallelLinear
//          (collab_infer/parallel/tensor_parallel.py:294-295); the per-projection outputs of
//          .split(local_sizes, dim=-1) are column views of y.
//   gated  the gated MLP's gate/up projection and activation in one pass
//          (collab_infer/models/llama.py:298-305, and its replicated-token branch :309-316):
//          gate = T(x . w_g^T + b_g), up = T(x . w_u^T + b_u), y = T(T(act(gate)) * up), with
//          w_g / w_u any two row ranges of one weight (the fused [gate; up] parameter); the
//          [M, 2I] gate/up intermediate never reaches memory.
//
// Matrix-core kernel (bf16 / f16, 16-byte aligned rows, K a multiple of 8):
//   * one workgroup = 8 waves, two per SIMD (256 registers each), computes 256 tokens x 256
//     weight rows; each wave owns 128 tokens x 64 weight rows, 32 accumulators of
//     v_mfma_f32_16x16x32 (128 registers); with two waves per SIMD one wave's stalls (load
//     issue, barrier, the activation epilogue's transcendental latencies) leave the matrix
//     core to the other;
//   * the MFMA's A operand is the weight (16 rows) and B the tokens (16 columns), so the 4
//     accumulator values of a lane are 4 consecutive output features of one token;
//   * 64-wide K slices of both operands go global -> LDS directly (buffer_load ... lds) into
//     two stages; a slice row is one 128-byte cache line, so each load instruction touches 8
//     lines (the address unit's cost is per line touched); rows are XOR-swizzled in 16-byte
//     groups so that the fragment reads (ds_read_b128) hit distinct banks;
//   * one barrier per slice, between its two 32-wide steps; a step's 32 matrix instructions
//     run token-block major and each carries a share of the rest: every token fragment is
//     reloaded for the next step right after its last use (so only one token set is held),
//     the next weight fragments go into a second set, and in the second step the 8 loads
//     refilling the buffer just freed go out one per 4 instructions, so neither the LDS nor
//     the address unit sees a burst;
//   * rows past M / N and columns past K read as zero through the buffer resources' range
//     check, so ragged tiles take no branches in the loop; slices past K load as zeros, so the
//     loop runs uniformly;
//   * the output block goes through LDS and leaves as whole 16-byte row chunks, so each
//     cache line of y is written by one store instruction;
//   * workgroups are dealt to the 8 XCDs round robin; tiles are renumbered so that each XCD
//     works through a compact group of tiles that share operand rows in its L2.
// Generic kernel (any dtype, stride or alignment): LDS-tiled FMA loop with f32 accumulation
// (f64 for f64 tensors).
#include <type_traits>

#include "cea_kernels.hpp"
#include "cea_lds_dma.hpp"

namespace cea {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct GMfma;
template <> struct GMfma<bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct GMfma<f16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x4 run(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

enum { kPlain = 0, kGated = 1 };

constexpr int G_THREADS = 512;                       // 8 waves, two per SIMD
constexpr int G_BM = 256;                            // tokens per tile
constexpr int G_BW = 256;                            // weight rows per tile
constexpr int G_BK = 64;                             // K per LDS slice
constexpr int G_ROW = G_BK * 2;                      // bytes of one row of a slice: a cache line
constexpr int G_NST = 2;                             // LDS stages
constexpr int G_OPER = G_BM * G_ROW;                 // 32 KB per operand per slice
constexpr int G_STAGE = 2 * G_OPER;                  // weight slice, then token slice
constexpr int G_LDS = G_NST * G_STAGE;               // 128 KB
constexpr int G_LOADS = G_OPER / (G_THREADS * 16);   // 16-byte loads per lane per operand
constexpr uint32_t kOutOfRange = 0x80000000u;        // above every resource's range
constexpr int kLgkm0 = 0xC07F;   // s_waitcnt lgkmcnt(0), vmcnt / expcnt left at their maximum
static_assert(G_LOADS == 4 && G_BM == G_BW, "the load pattern assumes 4 x 8 rows per wave");

struct GemmParams {
  const void* x;    // [M, K], row stride ldx
  const void* wg;   // [N, K], row stride ldw (gated: the gate rows)
  const void* wu;   // gated: the up rows, same row stride
  const void* bg;   // [N] or null (gated: gate bias)
  const void* bu;   // gated: up bias or null
  void* y;          // [M, N], row stride ldy
  int64_t ldx, ldw, ldy;
  int32_t M, N, K;  // N = output columns
  int32_t tiles_m, tiles_n, group_m;
  int32_t vec_out;  // 2: 16-byte row chunks, 1: 4-element stores, 0: element stores
};

// 16-byte group swizzle of a slice row (8 groups of 16 bytes): group c of row r sits at group
// c ^ g_swz(r).  A fragment read has 16 rows per 16-lane quarter and the quarters read groups
// c, c+1, c+2, c+3.  Measured on gfx950 (LDS bank-conflict counter), the reads behave as if 32
// lanes share a 512-byte bank window; this swizzle gives distinct 16-byte slots for any 32
// lanes (rows of equal r & 3 in one window), for any 16 lanes within 256 bytes and for any 8
// within 128 bytes.  Depends on r & 15 only.
__device__ __forceinline__ int g_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// Tile (token block, weight block) of this workgroup.
__device__ __forceinline__ void tile_of(const GemmParams& p, int& tm, int& tn) {
  const int nwg = p.tiles_m * p.tiles_n;
  int b = blockIdx.x;
  if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);   // one contiguous run per XCD
  const int per_group = p.group_m * p.tiles_n;                // group_m token blocks wide
  const int grp = b / per_group;
  const int first = grp * p.group_m;
  const int gm = min(p.tiles_m - first, p.group_m);
  const int r = b - grp * per_group;
  tm = first + r % gm;
  tn = r / gm;
}

template <typename T, typename A> __device__ __forceinline__ A rnd_acc(A v) {
  if constexpr (sizeof(T) >= sizeof(A)) return v;
  else return (A)round_to<T>((float)v);
}

// Bias of 4 consecutive columns (zero without a bias, or past n).
template <typename T, typename A>
__device__ __forceinline__ void bias4(const void* b, int col, int n, bool vec, A (&v)[4]) {
  const T* bp = (const T*)b;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = A(0);
  if (bp == nullptr) return;
  if (vec && col + 3 < n) {
    T t[4];
    __builtin_memcpy(t, bp + col, sizeof(t));
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (A)to_f32<T>(t[j]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (col + j < n) v[j] = load_acc<T, A>(bp + col + j);
  }
}

// Stores 4 consecutive columns of one output row.
template <typename T, typename A>
__device__ __forceinline__ void store4(T* row, int col, int n, bool vec, const A (&v)[4]) {
  T t[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) t[j] = store_cast<T, A>(v[j]);
  if (vec && col + 3 < n) {
    if constexpr (sizeof(T) == 2) {
      uint2 raw;
      __builtin_memcpy(&raw, t, 8);
      *(uint2*)(row + col) = raw;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) row[col + j] = t[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (col + j < n) row[col + j] = t[j];
  }
}

// The epilogue of 4 consecutive columns: plain y = acc + bias; gated
// y = T(act(T(gate + b_g))) * T(up + b_u).
template <typename T, int MODE, int ACT, bool BIAS, typename A>
__device__ __forceinline__ void finish4(const A (&g)[4], const A (&u)[4], const A (&bg)[4],
                                        const A (&bu)[4], A (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (MODE == kPlain) {
      v[j] = BIAS ? add_rn(g[j], bg[j]) : g[j];
    } else {
      const A gate = rnd_acc<T, A>(BIAS ? add_rn(g[j], bg[j]) : g[j]);
      const A up = rnd_acc<T, A>(BIAS ? add_rn(u[j], bu[j]) : u[j]);
      v[j] = mul_rn(rnd_acc<T, A>(gate_act<ACT, A>(gate)), up);
    }
  }
}

template <typename T, int MODE, int ACT>
__global__ __launch_bounds__(G_THREADS, 1) void gemm_mfma_kernel(const GemmParams p) {
  typedef typename GMfma<T>::frag frag;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int ESZ = sizeof(T);
  constexpr int OUT_N = MODE == kGated ? G_BW / 2 : G_BW;   // output columns per tile

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int wm = wave & 1;    // token half of the tile
  const int wn = wave >> 1;   // weight quarter (gated: output-column quarter)
  int tm, tn;
  tile_of(p, tm, tn);
  const int m0 = tm * G_BM;
  const int n0 = tn * OUT_N;
  const int K = p.K;
  const int KT = (K + G_BK - 1) / G_BK;

  const int rows_x = min(G_BM, p.M - m0);
  const i32x4 rx = make_rsrc((const char*)p.x + (int64_t)m0 * p.ldx * ESZ,
                             (uint32_t)((int64_t)(rows_x - 1) * p.ldx * ESZ + (int64_t)K * ESZ));
  i32x4 rw;
  if constexpr (MODE == kGated) {   // waves 0-3 load the 128 gate rows, 4-7 the 128 up rows
    const int rows = min(OUT_N, p.N - n0);
    const char* base = (const char*)(wave < 4 ? p.wg : p.wu) + (int64_t)n0 * p.ldw * ESZ;
    rw = make_rsrc(base, (uint32_t)((int64_t)(rows - 1) * p.ldw * ESZ + (int64_t)K * ESZ));
  } else {
    const int rows = min(G_BW, p.N - n0);
    rw = make_rsrc((const char*)p.wg + (int64_t)n0 * p.ldw * ESZ,
                   (uint32_t)((int64_t)(rows - 1) * p.ldw * ESZ + (int64_t)K * ESZ));
  }

  // slice loads: wave w fills rows [32w, 32w + 32) of both operands, 8 rows x 128 bytes per
  // instruction (same lane pattern and swizzle as the 4-wave kernel)
  int kcol[2];
  uint32_t off_w[G_LOADS], off_x[G_LOADS];
#pragma unroll
  for (int i = 0; i < G_LOADS; ++i) {
    const int row = 32 * wave + 8 * i + (lane >> 3);
    const int grp = (lane & 7) ^ g_swz(row);
    if (i < 2) kcol[i] = grp * 8;
    const int wrow = MODE == kGated ? (row & 127) : row;
    off_w[i] = (uint32_t)((int64_t)wrow * p.ldw * ESZ) + grp * 16;
    off_x[i] = (uint32_t)((int64_t)row * p.ldx * ESZ) + grp * 16;
  }
  const uint32_t lds_wave = lds_addr(smem) + wave * G_LOADS * 1024;
  auto issue_one = [&](int s, int i) {   // i < G_LOADS: weight rows, else token rows
    const uint32_t sb = lds_wave + (uint32_t)(s & (G_NST - 1)) * G_STAGE;
    const uint32_t kb = (uint32_t)s * G_ROW;
    const int li = i < G_LOADS ? i : i - G_LOADS;
    const bool kin = s * G_BK + kcol[li & 1] < K;
    if (i < G_LOADS)
      buffer_load_lds16_m0_so(rw, sb + li * 1024, kin ? off_w[li] : kOutOfRange, kb);
    else
      buffer_load_lds16_m0_so(rx, sb + G_OPER + li * 1024, kin ? off_x[li] : kOutOfRange, kb);
  };

  // fragments: 4 weight blocks (j < 4) and 8 token blocks (j >= 4) of 16 rows per step
  uint32_t rd[2];
#pragma unroll
  for (int q = 0; q < 2; ++q)
    rd[q] = (lane & 15) * G_ROW + (((4 * q + (lane >> 4)) ^ g_swz(lane & 15)) << 4);
  auto frag_row = [&](int j) {
    if (j < 4)
      return MODE == kGated ? (j >> 1) * 128 + wn * 32 + (j & 1) * 16 : wn * 64 + j * 16;
    return G_BM + wm * 128 + (j - 4) * 16;
  };
  auto read_a = [&](int s, int q, int j, frag (&fa)[4]) {
    fa[j] = *(const frag*)(smem + (s & (G_NST - 1)) * G_STAGE + rd[q] + frag_row(j) * G_ROW);
  };
  auto read_b = [&](int s, int q, int t, frag (&fb)[8]) {
    fb[t] = *(const frag*)(smem + (s & (G_NST - 1)) * G_STAGE + rd[q] + frag_row(4 + t) * G_ROW);
  };

  f32x4 acc[4][8];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[f][t][e] = 0.0f;

  // One 32-wide step: 32 matrix instructions token-block major; each token fragment is
  // reloaded for the next step (slice rs, step rq) right after its last use, the next
  // weight fragments go into the other set early, and with DMA the 8 refill loads of slice
  // s + 2 are spread one per 4 instructions.
  frag fa0[4], fa1[4], fb[8];
  auto step = [&](int s, const frag (&fa)[4], int rs, int rq, frag (&na)[4], auto dma) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int i = t * 4 + f;
        acc[f][t] = GMfma<T>::run(fa[f], fb[t], acc[f][t]);
        if (f == 3) read_b(rs, rq, t, fb);
        if ((i & 3) == 1 && i < 16) read_a(rs, rq, i >> 2, na);
        if constexpr (decltype(dma)::value) {
          if ((i & 3) == 2) issue_one(s + G_NST, i >> 2);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  };

#pragma unroll
  for (int s = 0; s < G_NST; ++s)
#pragma unroll
    for (int i = 0; i < 2 * G_LOADS; ++i) issue_one(s, i);
  wait_vmcnt<2 * G_LOADS>();
  barrier_no_fence();
#pragma unroll
  for (int j = 0; j < 4; ++j) read_a(0, 0, j, fa0);
#pragma unroll
  for (int t = 0; t < 8; ++t) read_b(0, 0, t, fb);
  __builtin_amdgcn_sched_barrier(0);
  for (int s = 0; s < KT; ++s) {
    step(s, fa0, s, 1, fa1, std::integral_constant<bool, false>());
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    barrier_no_fence();
    __builtin_amdgcn_sched_barrier(0);
    step(s, fa1, s + 1, 0, fa0, std::integral_constant<bool, true>());
  }
  wait_vmcnt<0>();

  // epilogue: block (f, t) holds token t * 16 + (l & 15) and weight rows f * 16 + 4 (l >> 4) ..
  const int q4 = lane >> 4;
  const bool vec = p.vec_out != 0;
  T* y = (T*)p.y;
  constexpr int NF = MODE == kGated ? 2 : 4;   // output column blocks of 16 per wave
  constexpr int NCOL = NF * 16;
  const int col0 = n0 + wn * NCOL;
  auto values = [&](int f, int t, const float (&bgv)[4], const float (&buv)[4], float (&v)[4],
                    auto bias) {
    float gv[4], uv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gv[j] = acc[f][t][j];
      uv[j] = MODE == kGated ? acc[f + 2][t][j] : 0.0f;
    }
    finish4<T, MODE, ACT, decltype(bias)::value, float>(gv, uv, bgv, buv, v);
  };
  if (p.vec_out == 2) {
    constexpr int RB = NCOL * 2;
    constexpr int CPR = RB / 16;
    constexpr int RPI = 64 / CPR;
    auto row_swz = [](int r) { return CPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3); };
    __builtin_amdgcn_s_waitcnt(kLgkm0);
    barrier_no_fence();
    char* stage = smem + wave * (128 * RB);
    auto to_lds = [&](auto bias) {
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int c4 = f * 16 + 4 * q4;
        float bgv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, buv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (decltype(bias)::value) {
          bias4<T, float>(p.bg, col0 + c4, p.N, true, bgv);
          if constexpr (MODE == kGated) bias4<T, float>(p.bu, col0 + c4, p.N, true, buv);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          float v[4];
          values(f, t, bgv, buv, v, bias);
          T o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = store_cast<T, float>(v[j]);
          uint2 raw;
          __builtin_memcpy(&raw, o, 8);
          const int row = t * 16 + (lane & 15);
          const int chunk = (c4 >> 3) ^ row_swz(row);
          *(uint2*)(stage + row * RB + chunk * 16 + (q4 & 1) * 8) = raw;
        }
      }
    };
    if (p.bg != nullptr) to_lds(std::integral_constant<bool, true>());
    else to_lds(std::integral_constant<bool, false>());
#pragma unroll
    for (int k = 0; k < 128 / RPI; ++k) {
      const int row = k * RPI + lane / CPR;
      const int c = lane % CPR;
      const uint4 raw = *(const uint4*)(stage + row * RB + ((c ^ row_swz(row)) * 16));
      const int tok = m0 + wm * 128 + row;
      const int col = col0 + c * 8;
      if (tok < p.M && col < p.N) *(uint4*)(y + (int64_t)tok * p.ldy + col) = raw;
    }
    return;
  }
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int col = col0 + f * 16 + 4 * q4;
    if (col >= p.N) continue;
    float bgv[4], buv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    bias4<T, float>(p.bg, col, p.N, vec, bgv);
    if constexpr (MODE == kGated) bias4<T, float>(p.bu, col, p.N, vec, buv);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int tok = m0 + wm * 128 + t * 16 + (lane & 15);
      if (tok >= p.M) continue;
      float v[4];
      values(f, t, bgv, buv, v, std::integral_constant<bool, true>());
      store4<T, float>(y + (int64_t)tok * p.ldy, col, p.N, vec, v);
    }
  }
}

// ---------------------------------------------------------------------------------------
// generic kernel: 64 tokens x 64 output columns per 256-thread block, 4 x 4 per thread
// ---------------------------------------------------------------------------------------
constexpr int GG_T = 64;
constexpr int GG_N = 64;
constexpr int GG_K = 16;

template <typename A> __device__ __forceinline__ A fma_acc(A a, A b, A c);
template <> __device__ __forceinline__ float fma_acc<float>(float a, float b, float c) {
  return __builtin_fmaf(a, b, c);
}
template <> __device__ __forceinline__ double fma_acc<double>(double a, double b, double c) {
  return __builtin_fma(a, b, c);
}

template <typename T, int MODE, int ACT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const GemmParams p) {
  typedef typename acc_of<T>::type A;
  constexpr int NW = MODE == kGated ? 2 : 1;   // weight operands
  __shared__ A xs[GG_K][GG_T + 1];
  __shared__ A ws[NW][GG_K][GG_N + 1];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int n0 = blockIdx.x * GG_N;
  const int m0 = blockIdx.y * GG_T;
  const T* x = (const T*)p.x;
  A acc[NW][4][4];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[w][i][j] = A(0);

  for (int k0 = 0; k0 < p.K; k0 += GG_K) {
    for (int e = tid; e < GG_T * GG_K; e += 256) {
      const int r = e / GG_K, c = e % GG_K;
      const int k = k0 + c;
      const int tok = m0 + r, col = n0 + r;
      xs[c][r] = (tok < p.M && k < p.K) ? load_acc<T, A>(x + (int64_t)tok * p.ldx + k) : A(0);
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const T* wp = (const T*)(w == 0 ? p.wg : p.wu);
        ws[w][c][r] = (col < p.N && k < p.K) ? load_acc<T, A>(wp + (int64_t)col * p.ldw + k) : A(0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < GG_K; ++c) {
      A xv[4], wv[NW][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = xs[c][ty * 4 + i];
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[w][j] = ws[w][c][tx * 4 + j];
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[w][i][j] = fma_acc<A>(xv[i], wv[w][j], acc[w][i][j]);
    }
    __syncthreads();
  }

  const int col = n0 + tx * 4;
  if (col >= p.N) return;
  A bgv[4], buv[4] = {A(0), A(0), A(0), A(0)};
  bias4<T, A>(p.bg, col, p.N, false, bgv);
  if constexpr (MODE == kGated) bias4<T, A>(p.bu, col, p.N, false, buv);
  T* y = (T*)p.y;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tok = m0 + ty * 4 + i;
    if (tok >= p.M) continue;
    A gv[4], uv[4], v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      gv[j] = acc[0][i][j];
      uv[j] = MODE == kGated ? acc[NW - 1][i][j] : A(0);
    }
    finish4<T, MODE, ACT, true, A>(gv, uv, bgv, buv, v);
    store4<T, A>(y + (int64_t)tok * p.ldy, col, p.N, false, v);
  }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
int g_group_m = 8;   // token blocks per tile group

bool mfma_path(const GemmParams& p, int dtype, int mode) {
  if (dtype != CEA_BF16 && dtype != CEA_F16) return false;
  if (p.K % 8 || p.ldx % 8 || p.ldw % 8) return false;
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  if (!al16(p.x) || !al16(p.wg) || (mode == kGated && !al16(p.wu))) return false;
  // every byte offset of a tile's rows must stay below the out-of-range marker
  const int64_t lim = (int64_t)kOutOfRange;
  const int wrows = mode == kGated ? G_BW / 2 : G_BW;
  if ((int64_t)(G_BM - 1) * p.ldx * 2 + (int64_t)p.K * 2 >= lim) return false;
  if ((int64_t)(wrows - 1) * p.ldw * 2 + (int64_t)p.K * 2 >= lim) return false;
  return true;
}

template <typename T, int MODE, int ACT>
int launch_one(GemmParams p, bool mfma, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (mfma) {
      const int out_n = MODE == kGated ? G_BW / 2 : G_BW;
      p.tiles_m = (p.M + G_BM - 1) / G_BM;
      p.tiles_n = (p.N + out_n - 1) / out_n;
      p.group_m = g_group_m;
      const int64_t total = (int64_t)p.tiles_m * p.tiles_n;
      CEA_REQUIRE(total <= INT32_MAX, CEA_EUNSUPPORTED, "linear: problem too large");
      const hipError_t e = reserve_lds<gemm_mfma_kernel<T, MODE, ACT>>(G_LDS);
      CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "linear: cannot reserve %d bytes of LDS: %s",
                  G_LDS, hipGetErrorString(e));
      hipLaunchKernelGGL((gemm_mfma_kernel<T, MODE, ACT>), dim3((unsigned)total),
                         dim3(G_THREADS), G_LDS, st, p);
      CEA_CHECK_LAUNCH(MODE == kGated ? "linear_gated" : "linear");
      return CEA_OK;
    }
  }
  const int64_t gy = (p.M + GG_T - 1) / GG_T;
  CEA_REQUIRE(gy <= 65535, CEA_EUNSUPPORTED, "linear: %d rows exceed the generic kernel's grid",
              p.M);
  hipLaunchKernelGGL((gemm_generic_kernel<T, MODE, ACT>),
                     dim3((unsigned)((p.N + GG_N - 1) / GG_N), (unsigned)gy), dim3(256), 0, st, p);
  CEA_CHECK_LAUNCH(MODE == kGated ? "linear_gated" : "linear");
  return CEA_OK;
}

template <typename T>
int launch_typed(const GemmParams& p, int mode, int act, bool mfma, hipStream_t st) {
  if (mode == kPlain) return launch_one<T, kPlain, 0>(p, mfma, st);
  switch (act) {
    case CEA_ACT_SILU: return launch_one<T, kGated, CEA_ACT_SILU>(p, mfma, st);
    case CEA_ACT_GELU: return launch_one<T, kGated, CEA_ACT_GELU>(p, mfma, st);
    case CEA_ACT_GELU_TANH: return launch_one<T, kGated, CEA_ACT_GELU_TANH>(p, mfma, st);
    case CEA_ACT_RELU: return launch_one<T, kGated, CEA_ACT_RELU>(p, mfma, st);
  }
  set_error("linear_gated: unknown activation %d", act);
  return CEA_EUNSUPPORTED;
}

}  // namespace

// x [M, K], w_gate / w_up [N, K] (one row stride), biases [N] or null, y [M, N]; shapes and
// dtypes validated by the caller.  mode: 0 plain (w_up / b_up unused), 1 gated.
int launch_linear(const cea_tensor* x, const cea_tensor* wg, const cea_tensor* wu,
                  const cea_tensor* bg, const cea_tensor* bu, cea_tensor* y, int mode, int act,
                  hipStream_t st) {
  GemmParams p{};
  p.x = x->data;
  p.wg = wg->data;
  p.wu = wu ? wu->data : nullptr;
  p.bg = bg ? bg->data : nullptr;
  p.bu = bu ? bu->data : nullptr;
  p.y = y->data;
  p.M = (int32_t)x->size[0];
  p.K = (int32_t)x->size[1];
  p.N = (int32_t)wg->size[0];
  p.ldx = x->size[0] > 1 ? x->stride[0] : p.K;
  p.ldw = wg->size[0] > 1 ? wg->stride[0] : p.K;
  p.ldy = y->size[0] > 1 ? y->stride[0] : p.N;
  // output stores: 2 = whole 16-byte chunks staged through LDS, 1 = 8-byte stores,
  // 0 = element stores
  const bool v8 = p.N % 4 == 0 && p.ldy % 4 == 0 && ((uintptr_t)p.y & 7) == 0 &&
                  (p.bg == nullptr || ((uintptr_t)p.bg & 7) == 0) &&
                  (p.bu == nullptr || ((uintptr_t)p.bu & 7) == 0);
  const bool v16 = v8 && p.N % 8 == 0 && p.ldy % 8 == 0 && ((uintptr_t)p.y & 15) == 0;
  p.vec_out = v16 ? 2 : v8 ? 1 : 0;
  if (p.M == 0 || p.N == 0) return CEA_OK;
  const bool mfma = mfma_path(p, x->dtype, mode);
  switch (x->dtype) {
    case CEA_BF16: return launch_typed<bf16>(p, mode, act, mfma, st);
    case CEA_F16: return launch_typed<f16>(p, mode, act, mfma, st);
    case CEA_F32: return launch_typed<float>(p, mode, act, false, st);
    case CEA_F64: return launch_typed<double>(p, mode, act, false, st);
  }
  set_error("linear: unsupported dtype %s", dtype_name(x->dtype));
  return CEA_EUNSUPPORTED;
}

}  // namespace cea
