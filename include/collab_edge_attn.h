/*
 * collab_edge_attn.h - C ABI of the MI355X (gfx950) attention / LSE / layer-op kernels.
 *
 * Every entry point replaces one operator of collab_infer's per-device hot path.  The
 * reference interface each one stands in for is cited (paths relative to the
 * collab_infer checkout).  Conventions:
 *   - all tensors are device pointers described by a cea_tensor (sizes and strides in
 *     elements, innermost stride must be 1 unless stated otherwise);
 *   - outputs are allocated by the caller; nothing here allocates device memory;
 *   - every call is asynchronous on the given stream (a hipStream_t passed as void*,
 *     NULL = the default stream);
 *   - the return value is CEA_OK (0) or a negative CEA_E* status; cea_last_error()
 *     returns the message of the last failure on the calling thread.  Nothing throws.
 *
 * Masking is position based: key j is visible to query i iff k_pos[j] >= 0 and
 * (!causal || k_pos[j] <= q_pos[i]).  Rows without a visible key give out = 0 and
 * lse = -inf, the neutral element of the merges.
 */
#ifndef COLLAB_EDGE_ATTN_H
#define COLLAB_EDGE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define CEA_F32 0
#define CEA_BF16 1
#define CEA_F16 2
#define CEA_F64 3
#define CEA_I64 4

/* status codes */
#define CEA_OK 0
#define CEA_EINVAL (-1)       /* shape / stride / dtype inconsistency (Python: ValueError)   */
#define CEA_EUNSUPPORTED (-2) /* valid request the kernels do not cover (NotImplementedError) */
#define CEA_ELAUNCH (-3)      /* HIP launch or runtime failure (RuntimeError)                 */
#define CEA_ENOSPACE (-4)     /* workspace smaller than cea_*_workspace_bytes() reported      */

#define CEA_MAX_DIMS 4
#define CEA_MAX_PARTS 16      /* maximum number of partial results one merge call combines   */
#define CEA_MAX_MAPPED_HEADS 512 /* maximum query heads when an explicit kv_map is given     */

#define CEA_NOALLOC_SCRATCH_BYTES (32 << 20) /* per-GPU scratch of cea_attention_with_lse_noalloc */

/* gated activations of cea_gated_mul: the reference's _ACTIVATIONS table (llama.py:44-49) */
#define CEA_ACT_SILU 0        /* F.silu                              */
#define CEA_ACT_GELU 1        /* F.gelu (erf form)                   */
#define CEA_ACT_GELU_TANH 2   /* F.gelu(x, approximate="tanh")       */
#define CEA_ACT_RELU 3        /* F.relu                              */

typedef struct cea_tensor {
  void* data;                    /* device pointer to element [0, ..., 0]       */
  int32_t dtype;                 /* CEA_F32 / CEA_BF16 / CEA_F16 / CEA_F64 / CEA_I64 */
  int32_t ndim;                  /* number of used entries of size / stride    */
  int64_t size[CEA_MAX_DIMS];
  int64_t stride[CEA_MAX_DIMS];  /* in elements                                 */
} cea_tensor;

/* Message of the last failed call on this thread ("" if none). */
const char* cea_last_error(void);

/* Library version as major*10000 + minor*100 + patch. */
int cea_version(void);

/*
 * Bytes of device workspace cea_attention_with_lse needs for these shapes (q: [B,Sq,Hq,D],
 * k: [B,Sk,Hkv,D]).  The workspace holds per-key-tile position summaries and, for short
 * query blocks, split-KV partial results; for query blocks too few to fill the device
 * against long key blocks, the partial (out, lse) pairs of a key-split launch.  A smaller
 * workspace that still holds the summaries runs such a call without key splits.
 */
size_t cea_attention_workspace_bytes(int64_t B, int64_t Sq, int64_t Hq, int64_t Sk, int64_t Hkv,
                                     int64_t D, int32_t in_dtype);

/*
 * Masked softmax attention over one KV block returning (out, lse).
 * Replaces attention_with_lse (collab_infer/parallel/attention.py:201-239) for one KV block:
 * _flash_lse / _math_lse (attention.py:163-198) with the visibility rule of
 * visibility_mask (attention.py:96-101) and the GQA mapping of expand_kv / gqa_group
 * (attention.py:68-93).
 *   q      [B,Sq,Hq,D]   bf16 / f16 / f32 / f64
 *   k, v   [B,Sk,Hkv,D]  same dtype as q, any strides with innermost stride 1
 *   q_pos  [B,Sq] i64,  k_pos [B,Sk] i64
 *   kv_map host array of Hq entries (query head -> KV head) or NULL for h // (Hq/Hkv)
 *   out    [B,Sq,Hq,D]   f32 (f64 for f64 inputs), or q's dtype when lse is NULL
 *                        (the plain attention of attention.py:270-301)
 *   lse    [B,Hq,Sq]     f32 (f64 for f64 inputs) natural-log log-sum-exp, or NULL
 *   accumulate  0: write (out, lse);  1: merge this block's result exactly into the
 *               existing (out, lse) like merge_attention (attention.py:242-250), the
 *               online merge of ring_attention (sequence_parallel.py:117-121)
 *   workspace   device buffer of at least cea_attention_workspace_bytes() bytes
 */
int cea_attention_with_lse(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                           const cea_tensor* q_pos, const cea_tensor* k_pos, int32_t causal,
                           double scale, const int32_t* kv_map, int32_t kv_map_len,
                           cea_tensor* out, cea_tensor* lse, int32_t accumulate,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * cea_attention_with_lse without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference: it computes exactly what cea_attention_with_lse computes,
 * with the same kernels, but its scratch (tile summaries or split-KV chunk partials) is a
 * static device array of CEA_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  It
 * calls no allocating routine; a call whose scratch need (cea_attention_workspace_bytes)
 * exceeds the array returns CEA_ENOSPACE.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race and must be serialised
 * by the caller.
 */
int cea_attention_with_lse_noalloc(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                                   const cea_tensor* q_pos, const cea_tensor* k_pos,
                                   int32_t causal, double scale, const int32_t* kv_map,
                                   int32_t kv_map_len, cea_tensor* out, cea_tensor* lse,
                                   int32_t accumulate, void* stream);

/*
 * The last step of a ring: merges attention over one more KV block into the running
 * (out, lse) exactly as cea_attention_with_lse with accumulate = 1, and writes the merged
 * output to final_out (q's dtype or the accumulation dtype) instead of back into out.
 * Replaces the last online merge of ring_attention together with its final
 * `out.to(q.dtype)` (collab_infer/parallel/sequence_parallel.py:121, 128).
 *   out, lse  the running pair (f32 / f64); lse receives the merged lse; out is read, and
 *             its content after the call is unspecified
 *   final_out [B,Sq,Hq,D]
 */
int cea_attention_merge_final(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                              const cea_tensor* q_pos, const cea_tensor* k_pos, int32_t causal,
                              double scale, const int32_t* kv_map, int32_t kv_map_len,
                              cea_tensor* out, cea_tensor* lse, cea_tensor* final_out,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * One rank's share of ring attention when every rank's KV block is resident on this device:
 * attention of q over n KV blocks given in ring order, merged exactly - what the per-rank
 * loop of ring_attention returns (collab_infer/parallel/sequence_parallel.py:68-130: the
 * attention_with_lse of each block :118-120, the online merge_attention :121, the skip of
 * fully masked blocks :117 and the final out.to(q.dtype) :128).  For bf16 / f16 with head
 * size 64 or 128 and one row stride shared by the blocks, all blocks run in one launch that
 * keeps each query row's softmax state across them (one output write, no intermediate
 * merges); other calls run block after block into a running (out, lse) pair in the
 * accumulation dtype.  Rows that see no key of any block get out = 0, lse = -inf.
 *   ks, vs    n tensors [B,Sk_i,Hkv,D], q's dtype, innermost stride 1 (Sk_i may be 0)
 *   k_pos_s   n tensors [B,Sk_i] i64
 *   out       [B,Sq,Hq,D] in q's dtype (the reference's return value) or the accumulation
 *             dtype; with lse it must be the accumulation dtype
 *   lse       [B,Hq,Sq] accumulation dtype, or NULL
 *   workspace at least cea_ring_attention_workspace_bytes() of these same arguments
 */
size_t cea_ring_attention_workspace_bytes(const cea_tensor* q, int32_t n, const cea_tensor* ks,
                                          const cea_tensor* vs, const cea_tensor* q_pos,
                                          const cea_tensor* k_pos_s, int32_t causal,
                                          const int32_t* kv_map, int32_t kv_map_len,
                                          const cea_tensor* out, const cea_tensor* lse);
int cea_ring_attention(const cea_tensor* q, int32_t n, const cea_tensor* ks, const cea_tensor* vs,
                       const cea_tensor* q_pos, const cea_tensor* k_pos_s, int32_t causal,
                       double scale, const int32_t* kv_map, int32_t kv_map_len, cea_tensor* out,
                       cea_tensor* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Pairwise exact merge: lse = logaddexp(lse_a, lse_b); out = out_a*w_a + out_b*w_b.
 * Replaces merge_attention (collab_infer/parallel/attention.py:242-250).
 *   out_*  [B,Sq,H,D] f32/f64,  lse_* [B,H,Sq] same dtype.  out may alias out_a (each
 *   element is read before it is written); lse must not alias an input lse.
 */
int cea_merge_attention(const cea_tensor* out_a, const cea_tensor* lse_a, const cea_tensor* out_b,
                        const cea_tensor* lse_b, cea_tensor* out, cea_tensor* lse, void* stream);

/*
 * n-way exact merge (n <= CEA_MAX_PARTS): lse = logsumexp_i lse_i; out = sum_i out_i*w_i.
 * Replaces merge_attention_list (collab_infer/parallel/attention.py:253-264).
 */
int cea_merge_attention_list(int32_t n, const cea_tensor* outs, const cea_tensor* lses,
                             cea_tensor* out, cea_tensor* lse, void* stream);

/*
 * Packs one partial result into the all-gather message of distributed-KV decoding:
 * packed[..., :D] = out, packed[..., D] = lse transposed to [B,Sq,H].
 * Replaces torch.cat([o, l.transpose(1, 2).unsqueeze(-1)], dim=-1)
 * (collab_infer/parallel/sequence_parallel.py:275).
 *   out [B,Sq,H,D] f32/f64 (innermost stride 1), lse [B,H,Sq] same dtype,
 *   packed [B,Sq,H,D+1] same dtype (innermost stride 1), e.g. one rank's slot of the
 *   gathered [n,B,Sq,H,D+1] buffer.
 */
int cea_pack_partial(const cea_tensor* out, const cea_tensor* lse, cea_tensor* packed,
                     void* stream);

/*
 * Exact merge of n packed partial results read in place from the all-gathered buffer:
 * out_i = part_i[..., :D], lse_i = part_i[..., D] transposed to [B,H,Sq], merged like
 * cea_merge_attention_list and written in out's dtype.
 * Replaces the unpacking and merge after the all-gather of distributed_kv_attention,
 * `outs = [p[..., :D]]; lses = [p[..., D].transpose(1, 2)]; merge_attention_list(outs, lses)`
 * and the final `.to(q.dtype)` (collab_infer/parallel/sequence_parallel.py:277-280).
 *   parts  n tensors [B,Sq,H,D+1] f32/f64 (innermost stride 1), e.g. views of the gathered
 *          [n,B,Sq,H,D+1] buffer;  out [B,Sq,H,D] the parts' dtype, or bf16/f16 from f32;
 *   lse    [B,H,Sq] the parts' dtype, or NULL.
 */
int cea_merge_packed(int32_t n, const cea_tensor* parts, cea_tensor* out, cea_tensor* lse,
                     void* stream);

/*
 * First Ulysses all-to-all as seen by one rank, on one device: the n ranks' sequence shards
 * q_j [B,s_j,Hq,D], k_j / v_j [B,s_j,Hkv,D] contribute this rank's heads
 * q[:, :, q_start:q_start+q_count], k/v[:, :, kv_start:kv_start+kv_count], packed per token
 * as [q heads | k heads | v heads] and concatenated over the ranks' tokens in rank order;
 * positions_j [B,s_j] are all-gathered the same way.
 * Replaces the send-side slicing, concatenation and .contiguous(), the all_to_all plus
 * torch.cat(received, dim=1), and the positions all_gather of ulysses_scatter
 * (collab_infer/parallel/sequence_parallel.py:163-178); q_f, k_f, v_f are the head slices
 * [0,q_count), [q_count, q_count+kv_count), [q_count+kv_count, width) of out.
 *   out [B,S,q_count+2*kv_count,D] (S = sum s_j, heads of a token contiguous), all shards in
 *   out's dtype with the heads of a token contiguous;  positions / pos_out [B,S] i64 both
 *   given or both NULL.
 */
int cea_ulysses_scatter(int32_t n, const cea_tensor* qs, const cea_tensor* ks, const cea_tensor* vs,
                        const cea_tensor* positions, int32_t q_start, int32_t q_count,
                        int32_t kv_start, int32_t kv_count, cea_tensor* out, cea_tensor* pos_out,
                        void* stream);

/*
 * Second Ulysses all-to-all as seen by one rank, on one device: tokens
 * [token_start, token_start + S_r) of every rank's head output outs_j [B,S,h_j,D],
 * concatenated over heads in rank order into out [B,S_r,sum h_j,D].
 * Replaces the per-destination slicing, the all_to_all and torch.cat(back, dim=2) of
 * ulysses_gather (collab_infer/parallel/sequence_parallel.py:182-194).
 */
int cea_ulysses_gather(int32_t n, const cea_tensor* outs, int64_t token_start, cea_tensor* out,
                       void* stream);

/*
 * Attention of one query block against n KV partitions plus the exact merge, in one pass:
 * the per-device compute of distributed_kv_attention
 * (collab_infer/parallel/sequence_parallel.py:250-280) for n simulated ranks, with the
 * all-gather replaced by reading every partition on this device.
 *   ks, vs, k_pos_s  n tensors, partition p is [B,Sk_p,Hkv,D] with positions [B,Sk_p]
 *   part_out, part_lse  optional (NULL) arrays of n per-partition results
 *                       ([B,Sq,Hq,D] / [B,Hq,Sq] f32), i.e. each rank's attention_with_lse
 *   out    [B,Sq,Hq,D]  q's dtype or f32;  lse [B,Hq,Sq] f32 or NULL
 */
size_t cea_partitioned_attention_workspace_bytes(int32_t n, const int64_t* Sk, int64_t B,
                                                 int64_t Sq, int64_t Hq, int64_t Hkv, int64_t D,
                                                 int32_t in_dtype);
int cea_partitioned_attention(const cea_tensor* q, int32_t n, const cea_tensor* ks,
                              const cea_tensor* vs, const cea_tensor* q_pos,
                              const cea_tensor* k_pos_s, int32_t causal, double scale,
                              const int32_t* kv_map, int32_t kv_map_len, cea_tensor* part_out,
                              cea_tensor* part_lse, cea_tensor* out, cea_tensor* lse,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMSNorm over the last dimension with the reference's rounding points:
 * y = weight * (x * rsqrt(mean(x^2) + eps)).to(x.dtype), computed in f32 (f64 for f64).
 * Replaces RMSNorm.forward (collab_infer/models/llama.py:52-61).
 *   x [N,C] (row stride free), weight [C], y [N,C] in promote(weight, x) dtype.
 */
int cea_rmsnorm(const cea_tensor* x, const cea_tensor* weight, double eps, cea_tensor* y,
                void* stream);

/*
 * Rotary tables at explicit positions: freqs = clamp(pos,0) * inv_freq,
 * emb = cat(freqs, freqs), cos/sin rounded to the table dtype.
 * Replaces RotaryEmbedding.forward (collab_infer/models/llama.py:64-77); inv_freq comes
 * from rope_inv_freq (collab_infer/models/config.py:165-189).
 *   positions [B,S] i64, inv_freq [D/2] f32 (f64 tables use an f64 inv_freq),
 *   cos, sin [B,S,D].
 */
int cea_rope_tables(const cea_tensor* positions, const cea_tensor* inv_freq, cea_tensor* cos,
                    cea_tensor* sin, void* stream);

/*
 * Half-split rotary embedding: out = x*cos + rotate_half(x)*sin with each product and the
 * sum rounded to x's dtype, as the reference's three tensor ops do.
 * Replaces apply_rotary / _rotate_half (collab_infer/models/llama.py:80-88).
 *   x [B,S,H,D], cos/sin [B,S,D] (batch stride may be 0), out [B,S,H,D].
 */
int cea_apply_rotary(const cea_tensor* x, const cea_tensor* cos, const cea_tensor* sin,
                     cea_tensor* out, void* stream);

/*
 * KV-cache append with the rotary of K fused in: writes k (rotated with cos/sin exactly as
 * cea_apply_rotary would, when the tables are given) and v, token-major [B,n,H,D], into
 * head-major caches [B,H,capacity,D] at slots offset..offset+n-1, and the positions [B,n]
 * into cache_pos [B,capacity].  One launch instead of apply_rotary plus two transposing
 * copies.  Growth (reallocation) stays with the caller.
 * Replaces `k = apply_rotary(k, cos, sin)` (collab_infer/models/llama.py:161, 196, 205, 208)
 * followed by LayerKVCache.append (collab_infer/models/cache.py:51-62).
 *   k, v [B,n,H,D] (any outer strides), positions [B,n] i64, cos/sin [B,n,D] or both NULL
 *   (plain append; D must still be even), cache_k/cache_v [B,H,cap,D], cache_pos [B,cap].
 */
int cea_kv_append(const cea_tensor* k, const cea_tensor* v, const cea_tensor* pos,
                  const cea_tensor* cos, const cea_tensor* sin, cea_tensor* cache_k,
                  cea_tensor* cache_v, cea_tensor* cache_pos, int64_t offset, void* stream);

/*
 * Fused RMSNorm + rotary: the RMSNorm output of x [S, H*D] viewed as [1,S,H,D] and rotated
 * at positions [S] with tables generated in-kernel (same rounding points as
 * cea_rmsnorm followed by cea_rope_tables + cea_apply_rotary).
 * Replaces the RMSNorm (llama.py:58-61) -> RotaryEmbedding (llama.py:74-77) ->
 * apply_rotary (llama.py:85-88) sequence.
 */
int cea_rmsnorm_rope(const cea_tensor* x, const cea_tensor* weight, double eps,
                     const cea_tensor* positions, const cea_tensor* inv_freq, int32_t num_heads,
                     cea_tensor* out, void* stream);

/*
 * SiLU-gate: out = silu(gate) * up with silu rounded to the tensor dtype before the product.
 * Replaces act(gate) * up with act = F.silu (collab_infer/models/llama.py:45, 305, 316).
 *   gate, up [N,I] (row strides free, e.g. column halves of a fused gate/up GEMM output),
 *   out [N,I].
 */
int cea_silu_mul(const cea_tensor* gate, const cea_tensor* up, cea_tensor* out, void* stream);

/*
 * Gated activation: out = act(gate) * up with act(gate) rounded to the tensor dtype before
 * the product, act one of CEA_ACT_* (silu, gelu, gelu_pytorch_tanh, relu).
 * Replaces act(gate) * up for every entry of _ACTIVATIONS (collab_infer/models/llama.py:44-49,
 * 298-305, 316).  Shapes as cea_silu_mul; an unknown act returns CEA_EUNSUPPORTED.
 */
int cea_gated_mul(const cea_tensor* gate, const cea_tensor* up, cea_tensor* out, int32_t act,
                  void* stream);

/*
 * Fused column-parallel projection: y = x . weight^T (+ bias), one GEMM for all the
 * projections that share the input (Q/K/V, gate/up), f32 accumulation (f64 for f64) rounded
 * once to the input dtype.  Replaces F.linear(x, self.weight, self.bias) of
 * FusedColumnParallelLinear (collab_infer/parallel/tensor_parallel.py:294-295); the
 * per-projection outputs of .split(local_sizes, dim=-1) are column views of y.
 *   x [M, K], weight [N, K], bias [N] or NULL, y [M, N]: one dtype (bf16 / f16 / f32 / f64),
 *   innermost stride 1, any row strides (rows must not overlap); y must not overlap x, weight
 *   or bias.  bf16 / f16 with K, both row strides a multiple of 8 and 16-byte aligned x and
 *   weight run on the matrix cores; everything else on a generic kernel.
 */
int cea_linear(const cea_tensor* x, const cea_tensor* weight, const cea_tensor* bias,
               cea_tensor* y, void* stream);

/*
 * The gated MLP's gate/up projection and its activation in one pass:
 *   gate = x . w_gate^T + b_gate,  up = x . w_up^T + b_up  (each rounded to the input dtype),
 *   y = act(gate) * up  with act(gate) rounded first,
 * without the [M, 2I] gate/up intermediate.  Replaces `gate, up = self.gate_up_proj(x);
 * h = self.act(gate) * up` of the gated MLP (collab_infer/models/llama.py:302-305, the fused
 * GEMM of tensor_parallel.py:294-295) and the two F.linear calls and activation of its
 * replicated-token branch (llama.py:309-316).
 *   x [M, K]; w_gate, w_up [I, K] with one row stride (e.g. the two halves, or any two row
 *   ranges, of the fused [2I, K] parameter); b_gate, b_up [I] (both or neither); y [M, I];
 *   act one of CEA_ACT_*.  Dtypes and paths as cea_linear.
 */
int cea_linear_gated(const cea_tensor* x, const cea_tensor* w_gate, const cea_tensor* w_up,
                     const cea_tensor* b_gate, const cea_tensor* b_up, cea_tensor* y,
                     int32_t act, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COLLAB_EDGE_ATTN_H */
