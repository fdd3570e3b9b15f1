// Wire formats of the sequence-parallel collectives, built and consumed on the device.
//
// * pack_partial_kernel: one rank's partial attention result (out [B,Sq,H,D], lse [B,H,Sq])
//   packed into the all-gather message [B,Sq,H,D+1] (out | lse), as
//   distributed_kv_attention does before its all-gather
//   (collab_infer/parallel/sequence_parallel.py:275).  The gathered [n,B,Sq,H,D+1] buffer is
//   merged in place by the merge kernel (merge.hip) through strided views.
// * ulysses_scatter_kernel: the first Ulysses all-to-all seen from one rank
//   (sequence_parallel.py:163-178): every rank's sequence shard contributes this rank's
//   query / KV heads, concatenated per token as [q heads | k heads | v heads] and over tokens
//   in rank order, plus the all-gathered positions.
// * ulysses_gather_kernel: the second all-to-all (sequence_parallel.py:182-194): this rank's
//   tokens with the head outputs of every rank concatenated in rank order.
//
// All three are HBM-bound copies.  One wave moves one row (a token, or a (b,s,h) row of the
// packed message): its segments are contiguous runs of bytes that the lanes stream with
// 16-byte loads and non-temporal 16-byte stores when every base, stride and length is a
// multiple of 16 bytes, element by element otherwise.
#include "cea_kernels.hpp"

namespace cea {
namespace {

typedef uint32_t wire_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWireThreads = 256;
constexpr int kWireRowsPerBlock = kWireThreads / 64;

// Copies 'bytes' bytes from src to dst with the 64 lanes of a wave (VEC = 16: 16-byte
// vectors, both pointers and the length multiples of 16; VEC = 2, 4 or 8: elements).
template <int VEC>
__device__ __forceinline__ void wave_copy(char* dst, const char* src, int bytes, int lane) {
  if constexpr (VEC == 16) {
    for (int o = lane * 16; o < bytes; o += 64 * 16) {
      const wire_u32x4 x = *(const wire_u32x4*)(src + o);
      __builtin_nontemporal_store(x, (wire_u32x4*)(dst + o));
    }
  } else if constexpr (VEC == 8) {
    for (int o = lane * 8; o < bytes; o += 64 * 8) *(uint64_t*)(dst + o) = *(const uint64_t*)(src + o);
  } else if constexpr (VEC == 4) {
    for (int o = lane * 4; o < bytes; o += 64 * 4) *(uint32_t*)(dst + o) = *(const uint32_t*)(src + o);
  } else {
    for (int o = lane * 2; o < bytes; o += 64 * 2) *(uint16_t*)(dst + o) = *(const uint16_t*)(src + o);
  }
}

template <int VEC>
__global__ __launch_bounds__(kWireThreads) void ulysses_scatter_kernel(const UlyssesScatterParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWireRowsPerBlock + (threadIdx.x >> 6);
  if (row >= (int64_t)p.B * p.S) return;
  const int b = (int)(row / p.S);
  const int t = (int)(row - (int64_t)b * p.S);
  // source rank of token t (tokens are concatenated in rank order)
  int j = 0;
#pragma unroll
  for (int i = 1; i < CEA_MAX_PARTS; ++i)
    if (i < p.n && t >= p.tok_off[i]) j = i;
  const int tl = t - p.tok_off[j];
  char* dst = p.out + b * p.os_b + (int64_t)t * p.os_s;
  wave_copy<VEC>(dst, p.q[j] + b * p.qs[j][0] + (int64_t)tl * p.qs[j][1], p.q_bytes, lane);
  wave_copy<VEC>(dst + p.q_bytes, p.k[j] + b * p.ks[j][0] + (int64_t)tl * p.ks[j][1], p.kv_bytes, lane);
  wave_copy<VEC>(dst + p.q_bytes + p.kv_bytes, p.v[j] + b * p.vs[j][0] + (int64_t)tl * p.vs[j][1],
                 p.kv_bytes, lane);
  if (p.pos_out && lane == 0)
    p.pos_out[b * p.pos_b + (int64_t)t * p.pos_s] = p.pos[j][b * p.ps[j][0] + (int64_t)tl * p.ps[j][1]];
}

template <int VEC>
__global__ __launch_bounds__(kWireThreads) void ulysses_gather_kernel(const UlyssesGatherParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWireRowsPerBlock + (threadIdx.x >> 6);
  if (row >= (int64_t)p.B * p.S) return;
  const int b = (int)(row / p.S);
  const int s = (int)(row - (int64_t)b * p.S);
  char* dst = p.out + b * p.os_b + (int64_t)s * p.os_s;
  for (int j = 0; j < p.n; ++j)
    wave_copy<VEC>(dst + p.dst_off[j], p.src[j] + b * p.ss[j][0] + (int64_t)s * p.ss[j][1], p.bytes[j],
                   lane);
}

// out | lse -> [.., D+1]; A = float or double
template <typename A>
__global__ __launch_bounds__(kWireThreads) void pack_partial_kernel(const PackParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWireRowsPerBlock + (threadIdx.x >> 6);
  const int64_t rows = (int64_t)p.B * p.Sq * p.H;
  if (row >= rows) return;
  const int h = (int)(row % p.H);
  const int64_t bs = row / p.H;
  const int s = (int)(bs % p.Sq);
  const int b = (int)(bs / p.Sq);
  const A* src = (const A*)p.out + b * p.os[0] + (int64_t)s * p.os[1] + (int64_t)h * p.os[2];
  A* dst = (A*)p.packed + b * p.ps[0] + (int64_t)s * p.ps[1] + (int64_t)h * p.ps[2];
  for (int d = lane; d < p.D; d += 64) dst[d] = src[d];
  if (lane == 0) dst[p.D] = ((const A*)p.lse)[b * p.ls[0] + (int64_t)h * p.ls[1] + (int64_t)s * p.ls[2]];
}

unsigned grid_rows(int64_t rows) { return (unsigned)((rows + kWireRowsPerBlock - 1) / kWireRowsPerBlock); }

}  // namespace

int launch_ulysses_scatter(const UlyssesScatterParams& p, int vec, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.S;
  if (rows == 0) return CEA_OK;
  CEA_REQUIRE(rows / kWireRowsPerBlock < ((int64_t)1 << 31), CEA_EUNSUPPORTED, "ulysses_scatter: too many rows");
  const dim3 grid(grid_rows(rows)), block(kWireThreads);
  switch (vec) {
    case 16: hipLaunchKernelGGL(ulysses_scatter_kernel<16>, grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL(ulysses_scatter_kernel<8>, grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL(ulysses_scatter_kernel<4>, grid, block, 0, st, p); break;
    default: hipLaunchKernelGGL(ulysses_scatter_kernel<2>, grid, block, 0, st, p); break;
  }
  CEA_CHECK_LAUNCH("ulysses_scatter");
  return CEA_OK;
}

int launch_ulysses_gather(const UlyssesGatherParams& p, int vec, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.S;
  if (rows == 0) return CEA_OK;
  CEA_REQUIRE(rows / kWireRowsPerBlock < ((int64_t)1 << 31), CEA_EUNSUPPORTED, "ulysses_gather: too many rows");
  const dim3 grid(grid_rows(rows)), block(kWireThreads);
  switch (vec) {
    case 16: hipLaunchKernelGGL(ulysses_gather_kernel<16>, grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL(ulysses_gather_kernel<8>, grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL(ulysses_gather_kernel<4>, grid, block, 0, st, p); break;
    default: hipLaunchKernelGGL(ulysses_gather_kernel<2>, grid, block, 0, st, p); break;
  }
  CEA_CHECK_LAUNCH("ulysses_gather");
  return CEA_OK;
}

int launch_pack_partial(const PackParams& p, hipStream_t st) {
  const int64_t rows = (int64_t)p.B * p.Sq * p.H;
  if (rows == 0) return CEA_OK;
  CEA_REQUIRE(rows / kWireRowsPerBlock < ((int64_t)1 << 31), CEA_EUNSUPPORTED, "pack_partial: too many rows");
  const dim3 grid(grid_rows(rows)), block(kWireThreads);
  if (p.dtype == CEA_F64) hipLaunchKernelGGL(pack_partial_kernel<double>, grid, block, 0, st, p);
  else hipLaunchKernelGGL(pack_partial_kernel<float>, grid, block, 0, st, p);
  CEA_CHECK_LAUNCH("pack_partial");
  return CEA_OK;
}

}  // namespace cea
