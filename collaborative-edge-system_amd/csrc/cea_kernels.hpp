// Parameter blocks and launcher declarations shared between the C ABI (capi.hip) and the
// kernel translation units.  Sizes are validated on the host before any launch.
#pragma once

#include "cea_common.hpp"

namespace cea {

// One attention call: query block [B,Sq,Hq,D] against one KV block [B,Sk,Hkv,D].
struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  const int64_t* q_pos;
  const int64_t* k_pos;
  void* out;
  void* lse;                 // may be null (plain attention)
  const TileInfo* tiles;     // [B, ntiles] summaries of k_pos (prefill kernels)
  int32_t B, Sq, Hq, Sk, Hkv, D;
  int64_t qs_b, qs_s, qs_h;  // element strides
  int64_t ks_b, ks_s, ks_h;
  int64_t vs_b, vs_s, vs_h;
  int64_t qps_b, qps_s;
  int64_t kps_b, kps_s;
  int64_t os_b, os_s, os_h;
  int64_t ls_b, ls_h, ls_s;
  double scale;
  int32_t causal;
  int32_t accumulate;        // merge into existing (out, lse)
  int32_t in_dtype;
  int32_t out_dtype;
  int32_t ntiles;
  HeadMap map;
  // accumulate only: the merged output goes here (in final_dtype) instead of into out
  void* final_out;
  int64_t fs_b, fs_s, fs_h;
  int32_t final_dtype;
  // key-split prefill launches (0 or 1: none): the block's tiles are dealt in equal runs to
  // `splits` groups of workgroups; group i writes its partial (out, lse) at
  // out + i * split_out and lse + i * split_lse (elements)
  int32_t splits;
  int64_t split_out, split_lse;
  // prefill workgroups hold this many query heads of one KV head's group (0 or 1: one), each
  // with 1 / heads_per_wg of the workgroup's query rows
  int32_t heads_per_wg;
};

// KV blocks of one prefill launch, in the order their tiles are visited (a ring share's
// blocks in ring order; one block for an ordinary call).  Row strides (ks_s / vs_s) are the
// launch's AttnParams ones, shared by every block; tile0 is the block's first tile in the
// launch's tile numbering (and in its tile-summary array).
constexpr int kMaxKvSegs = CEA_MAX_PARTS;
struct KvSeg {
  const void* k;
  const void* v;
  const int64_t* k_pos;
  int64_t ks_b, ks_h, vs_b, vs_h, kps_b, kps_s;
  int32_t Sk;
  int32_t tile0;
};
struct KvSegs {
  int32_t n;
  KvSeg seg[kMaxKvSegs];
};

// n-way merge of partial results (n <= CEA_MAX_PARTS).
struct MergeParams {
  int32_t n;
  int32_t pairwise;          // 1: logaddexp of two partials (merge_attention), 0: logsumexp
  int32_t B, Sq, H, D;
  int32_t dtype;             // partial dtype: CEA_F32 or CEA_F64
  int32_t out_dtype;         // merged output: the partial dtype, or bf16/f16 from f32
  const void* outs[CEA_MAX_PARTS];
  const void* lses[CEA_MAX_PARTS];
  int64_t os[CEA_MAX_PARTS][3];   // b, s, h strides
  int64_t ls[CEA_MAX_PARTS][3];   // b, h, s strides
  void* out;
  void* lse;
  int64_t dos[3];
  int64_t dls[3];
};

// Split-KV decode over one or more KV partitions (short query blocks).
struct DecodeParams {
  int32_t nparts;
  const void* q;
  const int64_t* q_pos;
  int32_t B, Sq, Hq, Hkv, D;
  int64_t qs_b, qs_s, qs_h;
  int64_t qps_b, qps_s;
  const void* k[CEA_MAX_PARTS];
  const void* v[CEA_MAX_PARTS];
  const int64_t* k_pos[CEA_MAX_PARTS];
  int32_t Sk[CEA_MAX_PARTS];
  int64_t ks[CEA_MAX_PARTS][3];
  int64_t vs[CEA_MAX_PARTS][3];
  int64_t kps[CEA_MAX_PARTS][2];
  int32_t chunk_begin[CEA_MAX_PARTS + 1];  // prefix sum of key chunks per partition
  int32_t chunk;                            // keys per chunk
  // set by the launcher: rows b < pair_rows take pairs of chunks as work items, item_begin is
  // the prefix sum of those pair items per partition
  int32_t pair_rows;
  int32_t item_begin[CEA_MAX_PARTS + 1];
  double scale;
  int32_t causal;
  int32_t in_dtype;
  HeadMap map;
  // partial results [B, units, total_chunks, NR rows (s, g)] x {D + 2} floats (o unnormalised,
  // m, l); per-key visibility words [B, total_chunks, chunk] (bit s: query s sees the key);
  // per-chunk masks [B, total_chunks] of 16-key tiles with a visible key
  float* partial;
  uint16_t* vis;
  uint64_t* tile_mask;
  int32_t G;                 // query heads of one work unit (all read one KV head)
  // work units per batch row: unit u holds query heads u*G .. u*G+G-1 and reads KV head
  // map.kv_of(u*G) - a KV head's whole group, part of it, or (G = 1) one query head of an
  // explicit map
  int32_t units;
  int32_t per_head;          // 1: units fastest in the grid (several units per KV head)
  // outputs of the reduction
  void* part_out[CEA_MAX_PARTS];   // optional per-partition (out, lse), f32
  void* part_lse[CEA_MAX_PARTS];
  int64_t pos_[CEA_MAX_PARTS][3];  // per-partition out strides (b, s, h)
  int64_t pls_[CEA_MAX_PARTS][3];  // per-partition lse strides (b, h, s)
  void* out;
  void* lse;
  int64_t os_b, os_s, os_h;
  int64_t ls_b, ls_h, ls_s;
  int32_t out_dtype;
  int32_t accumulate;
};

// Packing of one partial result into the all-gather message [B,Sq,H,D+1] (out | lse).
struct PackParams {
  int32_t B, Sq, H, D;
  int32_t dtype;             // CEA_F32 or CEA_F64
  const void* out;
  int64_t os[3];             // b, s, h element strides
  const void* lse;
  int64_t ls[3];             // b, h, s
  void* packed;
  int64_t ps[3];             // b, s, h
};

// First Ulysses all-to-all seen from one rank: n source shards -> [B, S, width, D].  Pointers
// are bytes, already offset to the first head of the slice; strides are bytes (b, s).
struct UlyssesScatterParams {
  int32_t n, B, S;
  int32_t tok_off[CEA_MAX_PARTS + 1];  // first token of each source in the output
  const char* q[CEA_MAX_PARTS];
  const char* k[CEA_MAX_PARTS];
  const char* v[CEA_MAX_PARTS];
  int64_t qs[CEA_MAX_PARTS][2], ks[CEA_MAX_PARTS][2], vs[CEA_MAX_PARTS][2];
  const int64_t* pos[CEA_MAX_PARTS];   // element strides (b, s); may be null with pos_out
  int64_t ps[CEA_MAX_PARTS][2];
  int32_t q_bytes, kv_bytes;            // bytes of the q slice / of each kv slice per token
  char* out;
  int64_t os_b, os_s;
  int64_t* pos_out;
  int64_t pos_b, pos_s;
};

// Second Ulysses all-to-all seen from one rank: n head outputs -> [B, S_r, H, D].
struct UlyssesGatherParams {
  int32_t n, B, S;
  const char* src[CEA_MAX_PARTS];      // offset to the rank's first token
  int64_t ss[CEA_MAX_PARTS][2];        // bytes (b, s)
  int32_t bytes[CEA_MAX_PARTS];        // bytes per token of source j
  int32_t dst_off[CEA_MAX_PARTS];      // their offset in an output token row
  char* out;
  int64_t os_b, os_s;
};

int launch_merge(const MergeParams& p, hipStream_t s);
int launch_pack_partial(const PackParams& p, hipStream_t s);
int launch_ulysses_scatter(const UlyssesScatterParams& p, int vec, hipStream_t s);
int launch_ulysses_gather(const UlyssesGatherParams& p, int vec, hipStream_t s);
int launch_rmsnorm(const cea_tensor* x, const cea_tensor* w, double eps, cea_tensor* y,
                   hipStream_t s);
int launch_rope_tables(const cea_tensor* pos, const cea_tensor* inv, cea_tensor* c,
                       cea_tensor* sn, hipStream_t s);
int launch_apply_rotary(const cea_tensor* x, const cea_tensor* c, const cea_tensor* sn,
                        cea_tensor* o, hipStream_t s);
int launch_kv_append(const cea_tensor* k, const cea_tensor* v, const cea_tensor* pos,
                     const cea_tensor* c, const cea_tensor* sn, cea_tensor* ck, cea_tensor* cv,
                     cea_tensor* cp, int64_t offset, hipStream_t st);
int launch_rmsnorm_rope(const cea_tensor* x, const cea_tensor* w, double eps,
                        const cea_tensor* pos, const cea_tensor* inv, int H, cea_tensor* o,
                        hipStream_t s);
int launch_gated_mul(const cea_tensor* g, const cea_tensor* u, cea_tensor* o, int act,
                     hipStream_t s);
// x [M, K], w_gate / w_up [N, K] (one row stride), biases [N] or null, y [M, N]; mode 0 is
// the plain projection (w_up / b_up unused), 1 the gated one with activation act
int launch_linear(const cea_tensor* x, const cea_tensor* wg, const cea_tensor* wu,
                  const cea_tensor* bg, const cea_tensor* bu, cea_tensor* y, int mode, int act,
                  hipStream_t s);
int launch_attn_generic(const AttnParams& p, hipStream_t s);
int launch_tile_info(const int64_t* k_pos, int64_t kps_b, int64_t kps_s, int32_t B, int32_t Sk,
                     TileInfo* tiles, int32_t ntiles, hipStream_t s);
// summaries of every block of 'segs' into one [B, ntiles] array (ntiles = all blocks' tiles)
int launch_tile_info_segs(const KvSegs& segs, int32_t B, TileInfo* tiles, int32_t ntiles,
                          hipStream_t s);
// the KV block of p as a one-entry segment table
KvSegs single_segment(const AttnParams& p);
bool prefill_mfma_supported(const AttnParams& p);
// p carries q / out / lse / head map / row strides; the blocks come from segs (p.k, p.v,
// p.k_pos and p.Sk are not read); p.ntiles and p.tiles cover all blocks
bool prefill_segs_supported(const AttnParams& p, const KvSegs& segs);
// Key splits worth a prefill launch of these shapes (1: none): enough workgroups to fill the
// device when the query blocks alone would not.  At most kMaxKeySplits (one n-way merge).
constexpr int kMaxKeySplits = CEA_MAX_PARTS;
int prefill_key_splits(int64_t B, int64_t Sq, int64_t Hq, int64_t Sk, int heads_per_wg);
// Query heads per prefill workgroup for Sq query rows and G query heads per KV head (G = 0:
// an explicit head map, one head per workgroup): 1, 2, 4 or 8.
int prefill_heads_per_wg(int64_t Sq, int64_t G);
int launch_attn_prefill_mfma(const AttnParams& p, hipStream_t s);
int launch_attn_prefill_segs(const AttnParams& p, const KvSegs& segs, hipStream_t s);
bool f32_mfma_supported(const AttnParams& p);
int launch_attn_f32_mfma(const AttnParams& p, hipStream_t s);
bool decode_supported(int32_t Sq, int32_t Hq, int32_t Hkv, int32_t D, int32_t dtype,
                      const HeadMap& map);
constexpr int kDecodeMaxChunks = 16384;  // key chunks per (batch, kv head), all partitions
int decode_plan_chunk(int64_t total_keys, int32_t B, int32_t units, int32_t D);
int decode_rows(int32_t Sq, int32_t G);  // padded query rows per kv head, 0 = unsupported
int launch_attn_decode(const DecodeParams& p, hipStream_t s);

constexpr int kTileKeys = 64;  // keys per KV tile of the prefill kernels / tile summaries

}  // namespace cea
