// C ABI: argument validation, dtype/shape dispatch and workspace layout.  Every entry point
// returns a status code; messages go to a per-thread buffer read by cea_last_error().
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "cea_kernels.hpp"

namespace cea {

static thread_local char g_error[1024] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_error; }

int check_tensor(const cea_tensor* t, const char* name, int ndim, int dtype, bool inner) {
  CEA_REQUIRE(t != nullptr, CEA_EINVAL, "%s: missing tensor", name);
  CEA_REQUIRE(t->ndim == ndim, CEA_EINVAL, "%s: expected %d dimensions, got %d", name, ndim,
              t->ndim);
  CEA_REQUIRE(dtype < 0 || t->dtype == dtype, CEA_EINVAL, "%s: expected dtype %s, got %s", name,
              dtype_name(dtype), dtype_name(t->dtype));
  CEA_REQUIRE(dtype_size(t->dtype) != 0, CEA_EINVAL, "%s: unknown dtype code %d", name,
              t->dtype);
  int64_t numel = 1;
  for (int i = 0; i < ndim; ++i) {
    CEA_REQUIRE(t->size[i] >= 0, CEA_EINVAL, "%s: negative size", name);
    CEA_REQUIRE(t->size[i] <= INT32_MAX, CEA_EUNSUPPORTED, "%s: dimension %d too large", name, i);
    numel *= t->size[i];
  }
  CEA_REQUIRE(numel == 0 || t->data != nullptr, CEA_EINVAL, "%s: null data pointer", name);
  if (inner && ndim > 0 && t->size[ndim - 1] > 1)
    CEA_REQUIRE(t->stride[ndim - 1] == 1, CEA_EINVAL, "%s: innermost stride must be 1", name);
  return CEA_OK;
}

int make_head_map(HeadMap* m, int64_t Hq, int64_t Hkv, const int32_t* kv_map, int32_t len) {
  memset(m, 0, sizeof(*m));
  if (kv_map == nullptr) {
    CEA_REQUIRE(Hkv >= 1 && Hq % Hkv == 0, CEA_EINVAL,
                "%lld query heads cannot share %lld KV heads evenly", (long long)Hq,
                (long long)Hkv);
    m->group = (int32_t)(Hq / Hkv);
    return CEA_OK;
  }
  CEA_REQUIRE(len == Hq, CEA_EINVAL, "kv_map must have one entry per query head");
  bool regular = Hkv >= 1 && Hq % Hkv == 0;
  const int64_t grp = regular ? Hq / Hkv : 0;
  for (int64_t h = 0; h < Hq; ++h) {
    CEA_REQUIRE(kv_map[h] >= 0 && kv_map[h] < Hkv, CEA_EINVAL,
                "kv_map[%lld] = %d out of range for %lld KV heads", (long long)h, kv_map[h],
                (long long)Hkv);
    if (regular && kv_map[h] != h / grp) regular = false;
  }
  if (regular) {
    m->group = (int32_t)grp;
    return CEA_OK;
  }
  CEA_REQUIRE(Hq <= CEA_MAX_MAPPED_HEADS, CEA_EUNSUPPORTED,
              "explicit kv_map supports at most %d query heads", CEA_MAX_MAPPED_HEADS);
  m->group = 0;
  for (int64_t h = 0; h < Hq; ++h) m->kv[h] = (int16_t)kv_map[h];
  return CEA_OK;
}

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static int64_t ntiles_of(int64_t Sk) { return (Sk + kTileKeys - 1) / kTileKeys; }

static size_t tile_bytes(int64_t B, int64_t Sk) {
  return align_up((size_t)(B * ntiles_of(Sk)) * sizeof(TileInfo), 256);
}

// Workspace of a key-split prefill call after its tile summaries: one f32 (out, lse) pair per
// split, [B, Sq, Hq, D] and [B, Hq, Sq] each.
static size_t split_bytes(int S, int64_t B, int64_t Sq, int64_t Hq, int64_t D) {
  if (S <= 1) return 0;
  return (size_t)S * ((size_t)B * Sq * Hq * D + (size_t)B * Hq * Sq) * sizeof(float);
}

// Builds the attention parameter block for one KV block; validates shapes and dtypes.
static int make_attn_params(AttnParams* p, const cea_tensor* q, const cea_tensor* k,
                            const cea_tensor* v, const cea_tensor* q_pos,
                            const cea_tensor* k_pos, int32_t causal, double scale,
                            const int32_t* kv_map, int32_t kv_map_len, cea_tensor* out,
                            cea_tensor* lse, int32_t accumulate) {
  int rc;
  if ((rc = check_tensor(q, "q", 4, -1, true))) return rc;
  const int dt = q->dtype;
  CEA_REQUIRE(dt == CEA_F32 || dt == CEA_BF16 || dt == CEA_F16 || dt == CEA_F64,
              CEA_EUNSUPPORTED, "attention: unsupported dtype %s", dtype_name(dt));
  if ((rc = check_tensor(k, "k", 4, dt, true))) return rc;
  if ((rc = check_tensor(v, "v", 4, dt, true))) return rc;
  if ((rc = check_tensor(q_pos, "q_pos", 2, CEA_I64, false))) return rc;
  if ((rc = check_tensor(k_pos, "k_pos", 2, CEA_I64, false))) return rc;
  const int64_t B = q->size[0], Sq = q->size[1], Hq = q->size[2], D = q->size[3];
  const int64_t Sk = k->size[1], Hkv = k->size[2];
  CEA_REQUIRE(k->size[0] == B && v->size[0] == B && v->size[1] == Sk && v->size[2] == Hkv &&
                  k->size[3] == D && v->size[3] == D,
              CEA_EINVAL, "attention: k/v shapes do not match q");
  CEA_REQUIRE(q_pos->size[0] == B && q_pos->size[1] == Sq, CEA_EINVAL,
              "attention: q_pos must be [B, Sq]");
  CEA_REQUIRE(k_pos->size[0] == B && k_pos->size[1] == Sk, CEA_EINVAL,
              "attention: k_pos must be [B, Sk]");
  const int acc = dt == CEA_F64 ? CEA_F64 : CEA_F32;
  if ((rc = check_tensor(out, "out", 4, -1, true))) return rc;
  CEA_REQUIRE(out->size[0] == B && out->size[1] == Sq && out->size[2] == Hq && out->size[3] == D,
              CEA_EINVAL, "attention: out must be [B, Sq, Hq, D]");
  if (lse) {
    CEA_REQUIRE(out->dtype == acc, CEA_EINVAL, "attention: out must be %s when lse is returned",
                dtype_name(acc));
    if ((rc = check_tensor(lse, "lse", 3, acc, false))) return rc;
    CEA_REQUIRE(lse->size[0] == B && lse->size[1] == Hq && lse->size[2] == Sq, CEA_EINVAL,
                "attention: lse must be [B, Hq, Sq]");
  } else {
    CEA_REQUIRE(out->dtype == acc || out->dtype == dt, CEA_EINVAL,
                "attention: out must be %s or %s", dtype_name(acc), dtype_name(dt));
    CEA_REQUIRE(!accumulate, CEA_EINVAL, "attention: accumulate needs lse");
  }
  CEA_REQUIRE(D >= 1, CEA_EINVAL, "attention: empty head dimension");
  memset(p, 0, sizeof(*p));
  if ((rc = make_head_map(&p->map, Hq, Hkv, kv_map, kv_map_len))) return rc;
  p->q = q->data; p->k = k->data; p->v = v->data;
  p->q_pos = (const int64_t*)q_pos->data;
  p->k_pos = (const int64_t*)k_pos->data;
  p->out = out->data;
  p->lse = lse ? lse->data : nullptr;
  p->B = (int32_t)B; p->Sq = (int32_t)Sq; p->Hq = (int32_t)Hq;
  p->Sk = (int32_t)Sk; p->Hkv = (int32_t)Hkv; p->D = (int32_t)D;
  p->qs_b = q->stride[0]; p->qs_s = q->stride[1]; p->qs_h = q->stride[2];
  p->ks_b = k->stride[0]; p->ks_s = k->stride[1]; p->ks_h = k->stride[2];
  p->vs_b = v->stride[0]; p->vs_s = v->stride[1]; p->vs_h = v->stride[2];
  p->qps_b = q_pos->stride[0]; p->qps_s = q_pos->stride[1];
  p->kps_b = k_pos->stride[0]; p->kps_s = k_pos->stride[1];
  p->os_b = out->stride[0]; p->os_s = out->stride[1]; p->os_h = out->stride[2];
  if (lse) { p->ls_b = lse->stride[0]; p->ls_h = lse->stride[1]; p->ls_s = lse->stride[2]; }
  p->scale = scale;
  p->causal = causal ? 1 : 0;
  p->accumulate = accumulate ? 1 : 0;
  p->in_dtype = dt;
  p->out_dtype = out->dtype;
  p->ntiles = (int32_t)ntiles_of(Sk);
  return CEA_OK;
}

// Split-KV decode over n KV blocks that share q / q_pos / out (n = 1: one attention call).
struct DecodePlan {
  int chunk;
  int total_chunks;
  int nr;
  size_t partial_bytes;  // partials + visibility words + tile masks
  size_t vis_offset, mask_offset;
};

// Work units of the decode kernels: G consecutive query heads that read one KV head, whose
// Sq * G rows share every K/V tile.  The regular grouping takes a KV head's whole group
// (G = Hq / Hkv) when its rows fit one unit, else the largest divisor of the group whose rows
// do (two units of 16 heads for 32 heads on one KV head); any other map takes one query head
// per unit (G = 1).  Units that split a KV head's group, and query-head units, go fastest in
// the grid (per_head), so the units reading one KV head's tiles run side by side.
struct DecodeUnits {
  int32_t units, G, per_head;
};
static DecodeUnits decode_units(int64_t Hq, int64_t Hkv, int64_t Sq, const HeadMap& map) {
  if (map.group > 0) {
    const int64_t G = Hq / Hkv;
    if (decode_rows((int32_t)Sq, (int32_t)G) != 0) return {(int32_t)Hkv, (int32_t)G, 0};
    for (int64_t gs = G - 1; gs > 1; --gs)
      if (G % gs == 0 && decode_rows((int32_t)Sq, (int32_t)gs) != 0)
        return {(int32_t)(Hq / gs), (int32_t)gs, 1};
  }
  return {(int32_t)Hq, 1, 1};
}

// A plan the decode launches can take: at most kDecodeMaxChunks chunks per batch row, batch
// rows within the visibility pass's second grid dimension, and every grid within 31 bits
// (the split kernel's: one work item per unit and chunk at most, before chunk pairs halve
// it; the reduction's: one workgroup per output row).
static bool decode_plan_fits(int64_t B, int64_t Sq, int64_t Hq, int64_t units,
                             int64_t total_chunks) {
  return total_chunks <= kDecodeMaxChunks && B < 65536 && B * units * total_chunks < INT32_MAX &&
         B * Sq * Hq < INT32_MAX;
}

static DecodePlan plan_decode(const int64_t* Sk, int n, int64_t B, int64_t Sq, int64_t units,
                              int64_t G, int64_t D) {
  DecodePlan pl;
  int64_t keys = 0;
  for (int i = 0; i < n; ++i) keys += Sk[i];
  pl.chunk = decode_plan_chunk(keys, (int32_t)B, (int32_t)units, (int32_t)D);
  pl.total_chunks = 0;
  for (int i = 0; i < n; ++i) pl.total_chunks += (int)((Sk[i] + pl.chunk - 1) / pl.chunk);
  pl.nr = decode_rows((int32_t)Sq, (int32_t)G);
  pl.vis_offset = align_up((size_t)(B * units) * pl.total_chunks * (pl.nr > 0 ? pl.nr : 1) *
                               (D + 2) * sizeof(float), 256);
  pl.mask_offset = pl.vis_offset + align_up((size_t)B * pl.total_chunks * pl.chunk * sizeof(uint16_t), 256);
  pl.partial_bytes = pl.mask_offset + align_up((size_t)B * pl.total_chunks * sizeof(uint64_t), 256);
  return pl;
}

// Decode scratch of the largest plan a call of these shapes can take, for callers that do not
// pass the head map: the regular grouping's plan and the per-query-head plan of any other map,
// and none for dtypes or head sizes the decode kernels do not take.
static size_t decode_ws_bytes(const int64_t* Sk, int n, int64_t B, int64_t Sq, int64_t Hq,
                              int64_t Hkv, int64_t D, int32_t dtype) {
  HeadMap regular;
  regular.group = 1;
  size_t need = 0;
  if (Hkv > 0 && Hq % Hkv == 0 &&
      decode_supported((int32_t)Sq, (int32_t)Hq, (int32_t)Hkv, (int32_t)D, dtype, regular)) {
    const DecodeUnits du = decode_units(Hq, Hkv, Sq, regular);
    need = plan_decode(Sk, n, B, Sq, du.units, du.G, D).partial_bytes;
  }
  HeadMap table;
  table.group = 0;
  if (Hkv > 0 && decode_supported((int32_t)Sq, (int32_t)Hq, (int32_t)Hkv, (int32_t)D, dtype, table)) {
    const size_t ph = plan_decode(Sk, n, B, Sq, Hq, 1, D).partial_bytes;
    need = ph > need ? ph : need;
  }
  return need;
}

// Fills a DecodeParams from n per-block parameter blocks (same q, q_pos, out, lse).
static int run_decode(const AttnParams* blocks, int n, cea_tensor* part_out, cea_tensor* part_lse,
                      char* ws, size_t ws_bytes, hipStream_t st) {
  const AttnParams& a = blocks[0];
  int64_t sks[CEA_MAX_PARTS];
  for (int i = 0; i < n; ++i) sks[i] = blocks[i].Sk;
  const DecodeUnits du = decode_units(a.Hq, a.Hkv, a.Sq, a.map);
  const DecodePlan pl = plan_decode(sks, n, a.B, a.Sq, du.units, du.G, a.D);
  CEA_REQUIRE(ws != nullptr && ws_bytes >= pl.partial_bytes, CEA_ENOSPACE,
              "decode: workspace of %zu bytes needed, %zu given", pl.partial_bytes, ws_bytes);
  DecodeParams d;
  memset(&d, 0, sizeof(d));
  d.nparts = n;
  d.q = a.q; d.q_pos = a.q_pos;
  d.B = a.B; d.Sq = a.Sq; d.Hq = a.Hq; d.Hkv = a.Hkv; d.D = a.D;
  d.qs_b = a.qs_b; d.qs_s = a.qs_s; d.qs_h = a.qs_h;
  d.qps_b = a.qps_b; d.qps_s = a.qps_s;
  d.chunk = pl.chunk;
  d.chunk_begin[0] = 0;
  for (int i = 0; i < n; ++i) {
    const AttnParams& bi = blocks[i];
    d.k[i] = bi.k; d.v[i] = bi.v; d.k_pos[i] = bi.k_pos;
    d.Sk[i] = bi.Sk;
    d.ks[i][0] = bi.ks_b; d.ks[i][1] = bi.ks_s; d.ks[i][2] = bi.ks_h;
    d.vs[i][0] = bi.vs_b; d.vs[i][1] = bi.vs_s; d.vs[i][2] = bi.vs_h;
    d.kps[i][0] = bi.kps_b; d.kps[i][1] = bi.kps_s;
    d.chunk_begin[i + 1] = d.chunk_begin[i] + (bi.Sk + pl.chunk - 1) / pl.chunk;
    if (part_out) {
      d.part_out[i] = part_out[i].data;
      d.part_lse[i] = part_lse[i].data;
      for (int j = 0; j < 3; ++j) {
        d.pos_[i][j] = part_out[i].stride[j];
        d.pls_[i][j] = part_lse[i].stride[j];
      }
    }
  }
  d.scale = a.scale;
  d.causal = a.causal;
  d.in_dtype = a.in_dtype;
  d.map = a.map;
  d.partial = (float*)ws;
  d.vis = (uint16_t*)(ws + pl.vis_offset);
  d.tile_mask = (uint64_t*)(ws + pl.mask_offset);
  d.G = du.G;
  d.units = du.units;
  d.per_head = du.per_head;
  d.out = a.out; d.lse = a.lse;
  d.os_b = a.os_b; d.os_s = a.os_s; d.os_h = a.os_h;
  d.ls_b = a.ls_b; d.ls_h = a.ls_h; d.ls_s = a.ls_s;
  d.out_dtype = a.out_dtype;
  d.accumulate = a.accumulate;
  return launch_attn_decode(d, st);
}

static bool use_decode(const AttnParams& p) {
  if (!decode_supported(p.Sq, p.Hq, p.Hkv, p.D, p.in_dtype, p.map)) return false;
  const int64_t sk = p.Sk;
  const DecodeUnits du = decode_units(p.Hq, p.Hkv, p.Sq, p.map);
  if (!decode_plan_fits(p.B, p.Sq, p.Hq, du.units,
                        plan_decode(&sk, 1, p.B, p.Sq, du.units, du.G, p.D).total_chunks))
    return false;
  if (!(p.out_dtype == CEA_F32 || p.out_dtype == p.in_dtype)) return false;
  if (p.accumulate && p.out_dtype != CEA_F32) return false;
  if (!(fabs(p.scale) >= 1e-30 && fabs(p.scale) <= 1e30)) return false;
  const int64_t s8[] = {p.qs_b, p.qs_s, p.qs_h, p.ks_b, p.ks_s, p.ks_h, p.vs_b, p.vs_s, p.vs_h};
  for (int64_t s : s8)
    if (s % 8) return false;
  if (p.ks_s > (1 << 24) || p.vs_s > (1 << 24)) return false;  // 16-row tile spans stay 32-bit
  return ((uintptr_t)p.q & 15) == 0 && ((uintptr_t)p.k & 15) == 0 && ((uintptr_t)p.v & 15) == 0;
}

// A prefill call whose query blocks alone give too few workgroups to fill the device (short
// query blocks against long key blocks: prefill chunks, decode shapes the split-KV kernels do
// not take): the block's tiles are dealt to S groups of workgroups, each writing a partial
// (out, lse) into the workspace, and the partials are merged with merge_attention_list's
// formula into the caller's out (f32 or the query dtype) and lse.
static int run_prefill_split(const AttnParams& p, int S, char* ws, hipStream_t st) {
  const int64_t n_out = (int64_t)p.B * p.Sq * p.Hq * p.D, n_lse = (int64_t)p.B * p.Hq * p.Sq;
  float* po = (float*)ws;
  float* pl = po + S * n_out;
  AttnParams sp = p;
  sp.splits = S;
  sp.split_out = n_out;
  sp.split_lse = n_lse;
  sp.out = po;
  sp.lse = pl;
  sp.out_dtype = CEA_F32;
  sp.os_b = (int64_t)p.Sq * p.Hq * p.D; sp.os_s = (int64_t)p.Hq * p.D; sp.os_h = p.D;
  sp.ls_b = (int64_t)p.Hq * p.Sq; sp.ls_h = p.Sq; sp.ls_s = 1;
  int rc = launch_attn_prefill_mfma(sp, st);
  if (rc) return rc;
  MergeParams m;
  memset(&m, 0, sizeof(m));
  m.n = S;
  m.pairwise = 0;
  m.B = p.B; m.Sq = p.Sq; m.H = p.Hq; m.D = p.D;
  m.dtype = CEA_F32;
  m.out_dtype = p.out_dtype;
  for (int i = 0; i < S; ++i) {
    m.outs[i] = po + i * n_out;
    m.lses[i] = pl + i * n_lse;
    m.os[i][0] = sp.os_b; m.os[i][1] = sp.os_s; m.os[i][2] = sp.os_h;
    m.ls[i][0] = sp.ls_b; m.ls[i][1] = sp.ls_h; m.ls[i][2] = sp.ls_s;
  }
  m.out = p.out;
  m.dos[0] = p.os_b; m.dos[1] = p.os_s; m.dos[2] = p.os_h;
  if (p.lse) {
    m.lse = p.lse;
    m.dls[0] = p.ls_b; m.dls[1] = p.ls_h; m.dls[2] = p.ls_s;
  }
  return launch_merge(m, st);
}

// Runs one attention call with a prepared parameter block.  allow_decode = false keeps the
// call off the split-KV decode kernels, whose workspace (chunk partials) is larger than the
// tile summaries the other kernels need.
static int run_attention(AttnParams& p, char* ws, size_t ws_bytes, hipStream_t st,
                         bool allow_decode = true) {
  if (allow_decode && p.Sk > 0 && use_decode(p))
    return run_decode(&p, 1, nullptr, nullptr, ws, ws_bytes, st);
  if (p.Sk > 0 && f32_mfma_supported(p)) return launch_attn_f32_mfma(p, st);
  if (p.Sk > 0 && prefill_mfma_supported(p)) {
    const size_t need = tile_bytes(p.B, p.Sk);
    CEA_REQUIRE(ws != nullptr && ws_bytes >= need, CEA_ENOSPACE,
                "attention: workspace of %zu bytes needed, %zu given", need, ws_bytes);
    p.tiles = (const TileInfo*)ws;
    int rc = launch_tile_info(p.k_pos, p.kps_b, p.kps_s, p.B, p.Sk, (TileInfo*)ws, p.ntiles, st);
    if (rc) return rc;
    p.heads_per_wg = prefill_heads_per_wg(p.Sq, p.map.group > 0 ? p.map.group : 0);
    // key splits when they help and the workspace holds their partials (a smaller workspace,
    // such as the slice a partitioned call leaves, runs the unsplit launch)
    if (!p.accumulate && !p.final_out) {
      const int S = prefill_key_splits(p.B, p.Sq, p.Hq, p.Sk, p.heads_per_wg);
      if (S > 1 && ws_bytes >= need + split_bytes(S, p.B, p.Sq, p.Hq, p.D))
        return run_prefill_split(p, S, ws + need, st);
    }
    return launch_attn_prefill_mfma(p, st);
  }
  return launch_attn_generic(p, st);
}

// ---- scratch of the no-allocation entry point -------------------------------------------
// A file-scope device array replaces the caller's workspace for callers that cannot allocate
// (code under graph capture, tight serving loops).  Every GPU holds its own copy at its own
// address until the process ends; host code never uses the array's name as a device address,
// only the per-device pointer that hipGetSymbolAddress returns.  Calls that overlap on one GPU
// share (and race on) this memory.
static __device__ __align__(256) char scratch[CEA_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::atomic<char*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The device address of this GPU's scratch, looked up once per device (with that device
// current) on its first use.
static int device_scratch(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  CEA_REQUIRE(e == hipSuccess, CEA_ELAUNCH, "no-alloc scratch: hipGetDevice failed: %s",
              hipGetErrorString(e));
  CEA_REQUIRE(dev >= 0 && dev < kMaxDevices, CEA_EUNSUPPORTED,
              "no-alloc scratch: device %d beyond the %d supported", dev, kMaxDevices);
  char* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      CEA_REQUIRE(e == hipSuccess && addr != nullptr, CEA_ELAUNCH,
                  "no-alloc scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(e));
      ptr = (char*)addr;
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return CEA_OK;
}

}  // namespace cea

using namespace cea;

extern "C" {

const char* cea_last_error(void) { return cea::last_error(); }

int cea_version(void) { return 100; }

// with_splits: room for the partials of a key-split prefill launch as well (the no-allocation
// entry point refuses only calls whose other scratch does not fit, and runs key splits when
// their partials fit too)
static size_t attention_ws_bytes(int64_t B, int64_t Sq, int64_t Hq, int64_t Sk, int64_t Hkv,
                                 int64_t D, int32_t in_dtype, bool with_splits) {
  if (B <= 0 || Sk <= 0) return 256;
  size_t need = tile_bytes(B, Sk);
  // (the regular grouping's plan: an explicit map has one head per workgroup, so more
  // workgroups and no more splits)
  if (with_splits && (in_dtype == CEA_BF16 || in_dtype == CEA_F16) && (D == 64 || D == 128)) {
    const int hp = prefill_heads_per_wg(Sq, Hkv > 0 && Hq % Hkv == 0 ? Hq / Hkv : 0);
    need += split_bytes(prefill_key_splits(B, Sq, Hq, Sk, hp), B, Sq, Hq, D);
  }
  const size_t dec = decode_ws_bytes(&Sk, 1, B, Sq, Hq, Hkv, D, in_dtype);
  return dec > need ? dec : need;
}

size_t cea_attention_workspace_bytes(int64_t B, int64_t Sq, int64_t Hq, int64_t Sk, int64_t Hkv,
                                     int64_t D, int32_t in_dtype) {
  return attention_ws_bytes(B, Sq, Hq, Sk, Hkv, D, in_dtype, true);
}

int cea_attention_with_lse(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                           const cea_tensor* q_pos, const cea_tensor* k_pos, int32_t causal,
                           double scale, const int32_t* kv_map, int32_t kv_map_len,
                           cea_tensor* out, cea_tensor* lse, int32_t accumulate,
                           void* workspace, size_t workspace_bytes, void* stream) {
  AttnParams p;
  int rc = make_attn_params(&p, q, k, v, q_pos, k_pos, causal, scale, kv_map, kv_map_len, out,
                            lse, accumulate);
  if (rc) return rc;
  return run_attention(p, (char*)workspace, workspace_bytes, (hipStream_t)stream);
}

int cea_attention_with_lse_noalloc(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                                   const cea_tensor* q_pos, const cea_tensor* k_pos,
                                   int32_t causal, double scale, const int32_t* kv_map,
                                   int32_t kv_map_len, cea_tensor* out, cea_tensor* lse,
                                   int32_t accumulate, void* stream) {
  AttnParams p;
  int rc = make_attn_params(&p, q, k, v, q_pos, k_pos, causal, scale, kv_map, kv_map_len, out,
                            lse, accumulate);
  if (rc) return rc;
  const size_t need = attention_ws_bytes(p.B, p.Sq, p.Hq, p.Sk, p.Hkv, p.D, p.in_dtype, false);
  CEA_REQUIRE(need <= (size_t)CEA_NOALLOC_SCRATCH_BYTES, CEA_ENOSPACE,
              "attention_with_lse_noalloc: this call needs %zu bytes of scratch, the static "
              "scratch holds %zu (use cea_attention_with_lse with a workspace)",
              need, (size_t)CEA_NOALLOC_SCRATCH_BYTES);
  char* ws = nullptr;
  if ((rc = device_scratch(&ws))) return rc;
  return run_attention(p, ws, (size_t)CEA_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

static int merge_impl(int32_t n, const cea_tensor* outs, const cea_tensor* lses, cea_tensor* out,
                      cea_tensor* lse, int pairwise, hipStream_t st);

int cea_attention_merge_final(const cea_tensor* q, const cea_tensor* k, const cea_tensor* v,
                              const cea_tensor* q_pos, const cea_tensor* k_pos, int32_t causal,
                              double scale, const int32_t* kv_map, int32_t kv_map_len,
                              cea_tensor* out, cea_tensor* lse, cea_tensor* final_out,
                              void* workspace, size_t workspace_bytes, void* stream) {
  CEA_REQUIRE(out && lse && final_out, CEA_EINVAL, "attention_merge_final: missing tensor");
  AttnParams p;
  int rc = make_attn_params(&p, q, k, v, q_pos, k_pos, causal, scale, kv_map, kv_map_len, out,
                            lse, 1);
  if (rc) return rc;
  if ((rc = check_tensor(final_out, "final_out", 4, -1, true))) return rc;
  CEA_REQUIRE(final_out->dtype == out->dtype || final_out->dtype == q->dtype, CEA_EINVAL,
              "attention_merge_final: final_out must be %s or %s", dtype_name(out->dtype),
              dtype_name(q->dtype));
  for (int j = 0; j < 4; ++j)
    CEA_REQUIRE(final_out->size[j] == out->size[j], CEA_EINVAL,
                "attention_merge_final: final_out must be [B, Sq, Hq, D]");
  hipStream_t st = (hipStream_t)stream;
  p.final_out = final_out->data;
  p.fs_b = final_out->stride[0];
  p.fs_s = final_out->stride[1];
  p.fs_h = final_out->stride[2];
  p.final_dtype = final_out->dtype;
  if (p.Sk > 0 && !use_decode(p) && prefill_mfma_supported(p))
    return run_attention(p, (char*)workspace, workspace_bytes, st);
  // other kernels: merge into the running pair, then cast it (a one-partial merge)
  p.final_out = nullptr;
  if (p.Sk > 0 && (rc = run_attention(p, (char*)workspace, workspace_bytes, st))) return rc;
  return merge_impl(1, out, lse, final_out, nullptr, 0, st);
}

// ---- one rank's share of ring attention with every block resident -----------------------
// The non-empty blocks, in ring order, become the segment table of one prefill launch when
// the MFMA kernel covers them (one row stride shared by all blocks); otherwise the blocks run
// one launch each, merged into running f32/f64 (out, lse) buffers exactly as the reference's
// per-step merge does.
struct RingPlan {
  AttnParams p;   // q / out / lse / head map, row strides of the first non-empty block
  KvSegs segs;    // non-empty blocks in ring order
  int first;      // index of the first non-empty block, -1 if every block is empty
  bool fused;
  size_t bytes;   // workspace this call needs
};

static int ring_plan(RingPlan* rp, const cea_tensor* q, int32_t n, const cea_tensor* ks,
                     const cea_tensor* vs, const cea_tensor* q_pos, const cea_tensor* k_pos_s,
                     int32_t causal, double scale, const int32_t* kv_map, int32_t kv_map_len,
                     cea_tensor* out, cea_tensor* lse) {
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "ring_attention: between 1 and %d KV blocks per call supported, got %d",
              CEA_MAX_PARTS, n);
  CEA_REQUIRE(q && ks && vs && q_pos && k_pos_s && out, CEA_EINVAL, "ring_attention: missing tensor");
  memset(rp, 0, sizeof(*rp));
  rp->first = -1;
  bool same_rows = true;
  int64_t tiles = 0;
  size_t block_ws = 0;
  for (int i = 0; i < n; ++i) {
    AttnParams bp;
    int rc = make_attn_params(&bp, q, &ks[i], &vs[i], q_pos, &k_pos_s[i], causal, scale, kv_map,
                              kv_map_len, out, lse, 0);
    if (rc) return rc;
    if (i == 0) rp->p = bp;
    CEA_REQUIRE(bp.Hkv == rp->p.Hkv, CEA_EINVAL,
                "ring_attention: block %d has %d KV heads, block 0 has %d", i, bp.Hkv, rp->p.Hkv);
    const size_t w = cea_attention_workspace_bytes(bp.B, bp.Sq, bp.Hq, bp.Sk, bp.Hkv, bp.D,
                                                   bp.in_dtype);
    block_ws = w > block_ws ? w : block_ws;
    if (bp.Sk == 0) continue;
    if (rp->first < 0) {
      rp->first = i;
      rp->p = bp;
    } else {
      same_rows = same_rows && bp.ks_s == rp->p.ks_s && bp.vs_s == rp->p.vs_s;
    }
    KvSeg& g = rp->segs.seg[rp->segs.n++];
    g.k = bp.k; g.v = bp.v; g.k_pos = bp.k_pos;
    g.ks_b = bp.ks_b; g.ks_h = bp.ks_h; g.vs_b = bp.vs_b; g.vs_h = bp.vs_h;
    g.kps_b = bp.kps_b; g.kps_s = bp.kps_s;
    g.Sk = bp.Sk;
    g.tile0 = (int32_t)tiles;
    tiles += ntiles_of(bp.Sk);
  }
  rp->p.ntiles = (int32_t)tiles;
  rp->fused = rp->first >= 0 && same_rows && tiles < ((int64_t)1 << 24) &&
              prefill_segs_supported(rp->p, rp->segs);
  if (rp->fused) {
    // one summary per tile of every block and batch row (tile_bytes takes a key count)
    rp->bytes = align_up((size_t)rp->p.B * (size_t)tiles * sizeof(TileInfo), 256);
  } else {
    // running (out, lse) in the accumulation dtype unless the caller's pair is that already
    const size_t esz = rp->p.in_dtype == CEA_F64 ? 8 : 4;
    const size_t run = lse ? 0
                           : align_up((size_t)rp->p.B * rp->p.Sq * rp->p.Hq * rp->p.D * esz, 256) +
                                 align_up((size_t)rp->p.B * rp->p.Hq * rp->p.Sq * esz, 256);
    rp->bytes = run + block_ws;
  }
  return CEA_OK;
}

extern "C" size_t cea_ring_attention_workspace_bytes(const cea_tensor* q, int32_t n,
                                                     const cea_tensor* ks, const cea_tensor* vs,
                                                     const cea_tensor* q_pos,
                                                     const cea_tensor* k_pos_s, int32_t causal,
                                                     const int32_t* kv_map, int32_t kv_map_len,
                                                     const cea_tensor* out, const cea_tensor* lse) {
  RingPlan rp;
  // scale does not change the route; an invalid call needs no workspace (it fails anyway)
  if (ring_plan(&rp, q, n, ks, vs, q_pos, k_pos_s, causal, 1.0, kv_map, kv_map_len,
                (cea_tensor*)out, (cea_tensor*)lse))
    return 256;
  return rp.bytes > 256 ? rp.bytes : 256;
}

extern "C" int cea_ring_attention(const cea_tensor* q, int32_t n, const cea_tensor* ks,
                                  const cea_tensor* vs, const cea_tensor* q_pos,
                                  const cea_tensor* k_pos_s, int32_t causal, double scale,
                                  const int32_t* kv_map, int32_t kv_map_len, cea_tensor* out,
                                  cea_tensor* lse, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  RingPlan rp;
  int rc = ring_plan(&rp, q, n, ks, vs, q_pos, k_pos_s, causal, scale, kv_map, kv_map_len, out,
                     lse);
  if (rc) return rc;
  CEA_REQUIRE(workspace != nullptr && workspace_bytes >= rp.bytes, CEA_ENOSPACE,
              "ring_attention: workspace of %zu bytes needed, %zu given", rp.bytes,
              workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  if (rp.fused) {
    rp.p.tiles = (const TileInfo*)workspace;
    if ((rc = launch_tile_info_segs(rp.segs, rp.p.B, (TileInfo*)workspace, rp.p.ntiles, st)))
      return rc;
    return launch_attn_prefill_segs(rp.p, rp.segs, st);
  }
  // block after block into the running pair, then the one-partial merge casts it into out
  char* ws = (char*)workspace;
  size_t left = workspace_bytes;
  cea_tensor run_out = *out, run_lse;
  if (lse) {
    run_lse = *lse;
  } else {
    const int acc = rp.p.in_dtype == CEA_F64 ? CEA_F64 : CEA_F32;
    const int64_t esz = acc == CEA_F64 ? 8 : 4;
    const int64_t B = rp.p.B, Sq = rp.p.Sq, Hq = rp.p.Hq, D = rp.p.D;
    memset(&run_out, 0, sizeof(run_out));
    run_out.data = ws;
    run_out.dtype = acc;
    run_out.ndim = 4;
    const int64_t osz[4] = {B, Sq, Hq, D}, ost[4] = {Sq * Hq * D, Hq * D, D, 1};
    for (int j = 0; j < 4; ++j) { run_out.size[j] = osz[j]; run_out.stride[j] = ost[j]; }
    const size_t ob = align_up((size_t)(B * Sq * Hq * D * esz), 256);
    memset(&run_lse, 0, sizeof(run_lse));
    run_lse.data = ws + ob;
    run_lse.dtype = acc;
    run_lse.ndim = 3;
    const int64_t lsz[3] = {B, Hq, Sq}, lst[3] = {Hq * Sq, Sq, 1};
    for (int j = 0; j < 3; ++j) { run_lse.size[j] = lsz[j]; run_lse.stride[j] = lst[j]; }
    const size_t used = ob + align_up((size_t)(B * Hq * Sq * esz), 256);
    ws += used;
    left -= used;
  }
  int done = 0;
  for (int i = 0; i < n; ++i) {
    // every block empty: the first one writes the merge's neutral element (0, -inf)
    if (ks[i].size[1] == 0 && !(rp.first < 0 && i == 0)) continue;
    AttnParams bp;
    if ((rc = make_attn_params(&bp, q, &ks[i], &vs[i], q_pos, &k_pos_s[i], causal, scale, kv_map,
                               kv_map_len, &run_out, &run_lse, done > 0 ? 1 : 0)))
      return rc;
    if ((rc = run_attention(bp, ws, left, st))) return rc;
    ++done;
  }
  if (lse) return CEA_OK;
  return merge_impl(1, &run_out, &run_lse, out, nullptr, 0, st);
}

static int fill_merge_part(MergeParams* m, int i, const cea_tensor* o, const cea_tensor* l,
                           int64_t B, int64_t Sq, int64_t H, int64_t D, int dt) {
  int rc;
  if ((rc = check_tensor(o, "out_i", 4, dt, true))) return rc;
  if ((rc = check_tensor(l, "lse_i", 3, dt, false))) return rc;
  CEA_REQUIRE(o->size[0] == B && o->size[1] == Sq && o->size[2] == H && o->size[3] == D,
              CEA_EINVAL, "merge: partial %d has a different output shape", i);
  CEA_REQUIRE(l->size[0] == B && l->size[1] == H && l->size[2] == Sq, CEA_EINVAL,
              "merge: partial %d lse must be [B, H, Sq]", i);
  m->outs[i] = o->data;
  m->lses[i] = l->data;
  for (int j = 0; j < 3; ++j) {
    m->os[i][j] = o->stride[j];
    m->ls[i][j] = l->stride[j];
  }
  return CEA_OK;
}

static int merge_impl(int32_t n, const cea_tensor* outs, const cea_tensor* lses, cea_tensor* out,
                      cea_tensor* lse, int pairwise, hipStream_t st) {
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "merge: between 1 and %d partial results supported, got %d", CEA_MAX_PARTS, n);
  int rc;
  if ((rc = check_tensor(&outs[0], "out_0", 4, -1, true))) return rc;
  const int dt = outs[0].dtype;
  CEA_REQUIRE(dt == CEA_F32 || dt == CEA_F64, CEA_EUNSUPPORTED,
              "merge: partial results must be float32 or float64, got %s", dtype_name(dt));
  const int64_t B = outs[0].size[0], Sq = outs[0].size[1], H = outs[0].size[2],
                D = outs[0].size[3];
  MergeParams m;
  memset(&m, 0, sizeof(m));
  m.n = n;
  m.pairwise = pairwise;
  m.B = (int32_t)B; m.Sq = (int32_t)Sq; m.H = (int32_t)H; m.D = (int32_t)D;
  m.dtype = dt;
  for (int i = 0; i < n; ++i)
    if ((rc = fill_merge_part(&m, i, &outs[i], &lses[i], B, Sq, H, D, dt))) return rc;
  if ((rc = check_tensor(out, "out", 4, -1, true))) return rc;
  CEA_REQUIRE(out->dtype == dt || (dt == CEA_F32 && (out->dtype == CEA_BF16 ||
                                                     out->dtype == CEA_F16)),
              CEA_EINVAL, "merge: output dtype %s not allowed for %s partials",
              dtype_name(out->dtype), dtype_name(dt));
  CEA_REQUIRE(out->size[0] == B && out->size[1] == Sq && out->size[2] == H && out->size[3] == D,
              CEA_EINVAL, "merge: out must be [B, Sq, H, D]");
  m.out_dtype = out->dtype;
  m.out = out->data;
  for (int j = 0; j < 3; ++j) m.dos[j] = out->stride[j];
  if (lse) {
    if ((rc = check_tensor(lse, "lse", 3, dt, false))) return rc;
    CEA_REQUIRE(lse->size[0] == B && lse->size[1] == H && lse->size[2] == Sq, CEA_EINVAL,
                "merge: lse must be [B, H, Sq]");
    m.lse = lse->data;
    for (int j = 0; j < 3; ++j) m.dls[j] = lse->stride[j];
  }
  return launch_merge(m, st);
}

int cea_merge_attention(const cea_tensor* out_a, const cea_tensor* lse_a, const cea_tensor* out_b,
                        const cea_tensor* lse_b, cea_tensor* out, cea_tensor* lse, void* stream) {
  CEA_REQUIRE(out_a && lse_a && out_b && lse_b && lse, CEA_EINVAL, "merge: missing tensor");
  cea_tensor outs[2] = {*out_a, *out_b};
  cea_tensor lses[2] = {*lse_a, *lse_b};
  return merge_impl(2, outs, lses, out, lse, 1, (hipStream_t)stream);
}

int cea_merge_attention_list(int32_t n, const cea_tensor* outs, const cea_tensor* lses,
                             cea_tensor* out, cea_tensor* lse, void* stream) {
  CEA_REQUIRE(outs && lses && lse, CEA_EINVAL, "merge: missing tensor");
  return merge_impl(n, outs, lses, out, lse, 0, (hipStream_t)stream);
}

int cea_merge_packed(int32_t n, const cea_tensor* parts, cea_tensor* out, cea_tensor* lse,
                     void* stream) {
  CEA_REQUIRE(parts && out, CEA_EINVAL, "merge_packed: missing tensor");
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "merge_packed: between 1 and %d partial results supported, got %d", CEA_MAX_PARTS, n);
  int rc;
  if ((rc = check_tensor(&parts[0], "part_0", 4, -1, true))) return rc;
  const int dt = parts[0].dtype;
  CEA_REQUIRE(dt == CEA_F32 || dt == CEA_F64, CEA_EUNSUPPORTED,
              "merge_packed: packed partials must be float32 or float64, got %s", dtype_name(dt));
  CEA_REQUIRE(parts[0].size[3] >= 2, CEA_EINVAL, "merge_packed: rows must hold D values and the lse");
  const int64_t D = parts[0].size[3] - 1;
  const size_t esz = dtype_size(dt);
  cea_tensor outs[CEA_MAX_PARTS], lses[CEA_MAX_PARTS];
  for (int i = 0; i < n; ++i) {
    const cea_tensor& t = parts[i];
    if ((rc = check_tensor(&t, "part_i", 4, dt, true))) return rc;
    for (int j = 0; j < 4; ++j)
      CEA_REQUIRE(t.size[j] == parts[0].size[j], CEA_EINVAL,
                  "merge_packed: partial %d has a different shape", i);
    // out_i = part[..., :D];  lse_i = part[..., D].transpose(1, 2)
    outs[i] = t;
    outs[i].size[3] = D;
    lses[i].data = (char*)t.data + D * esz;
    lses[i].dtype = dt;
    lses[i].ndim = 3;
    lses[i].size[0] = t.size[0]; lses[i].size[1] = t.size[2]; lses[i].size[2] = t.size[1];
    lses[i].stride[0] = t.stride[0]; lses[i].stride[1] = t.stride[2]; lses[i].stride[2] = t.stride[1];
    lses[i].size[3] = 0; lses[i].stride[3] = 0;
  }
  return merge_impl(n, outs, lses, out, lse, 0, (hipStream_t)stream);
}

int cea_pack_partial(const cea_tensor* out, const cea_tensor* lse, cea_tensor* packed,
                     void* stream) {
  int rc;
  if ((rc = check_tensor(out, "out", 4, -1, false))) return rc;
  const int dt = out->dtype;
  CEA_REQUIRE(dt == CEA_F32 || dt == CEA_F64, CEA_EUNSUPPORTED,
              "pack_partial: partial results must be float32 or float64, got %s", dtype_name(dt));
  if ((rc = check_tensor(lse, "lse", 3, dt, false))) return rc;
  if ((rc = check_tensor(packed, "packed", 4, dt, true))) return rc;
  const int64_t B = out->size[0], Sq = out->size[1], H = out->size[2], D = out->size[3];
  CEA_REQUIRE(lse->size[0] == B && lse->size[1] == H && lse->size[2] == Sq, CEA_EINVAL,
              "pack_partial: lse must be [B, H, Sq]");
  CEA_REQUIRE(packed->size[0] == B && packed->size[1] == Sq && packed->size[2] == H &&
                  packed->size[3] == D + 1,
              CEA_EINVAL, "pack_partial: packed must be [B, Sq, H, D + 1]");
  CEA_REQUIRE(D == 0 || out->stride[3] == 1, CEA_EINVAL, "pack_partial: innermost stride must be 1");
  PackParams p;
  memset(&p, 0, sizeof(p));
  p.B = (int32_t)B; p.Sq = (int32_t)Sq; p.H = (int32_t)H; p.D = (int32_t)D;
  p.dtype = dt;
  p.out = out->data;
  p.lse = lse->data;
  p.packed = packed->data;
  for (int j = 0; j < 3; ++j) {
    p.os[j] = out->stride[j];
    p.ls[j] = lse->stride[j];
    p.ps[j] = packed->stride[j];
  }
  return launch_pack_partial(p, (hipStream_t)stream);
}

// 16 when every pointer, stride and length (bytes) is a multiple of 16, else the element size
static int copy_vec(const int64_t* vals, int count, int esz) {
  for (int i = 0; i < count; ++i)
    if (vals[i] % 16) return esz;
  return 16;
}

int cea_ulysses_scatter(int32_t n, const cea_tensor* qs, const cea_tensor* ks, const cea_tensor* vs,
                        const cea_tensor* positions, int32_t q_start, int32_t q_count,
                        int32_t kv_start, int32_t kv_count, cea_tensor* out, cea_tensor* pos_out,
                        void* stream) {
  CEA_REQUIRE(qs && ks && vs && out, CEA_EINVAL, "ulysses_scatter: missing tensor");
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "ulysses_scatter: between 1 and %d ranks supported, got %d", CEA_MAX_PARTS, n);
  CEA_REQUIRE((positions == nullptr) == (pos_out == nullptr), CEA_EINVAL,
              "ulysses_scatter: positions and pos_out go together");
  int rc;
  if ((rc = check_tensor(out, "out", 4, -1, true))) return rc;
  const int dt = out->dtype;
  const int esz = (int)dtype_size(dt);
  const int64_t B = out->size[0], S = out->size[1], W = out->size[2], D = out->size[3];
  CEA_REQUIRE(q_count >= 0 && kv_count >= 0 && W == q_count + 2 * (int64_t)kv_count, CEA_EINVAL,
              "ulysses_scatter: out must hold q_count + 2 * kv_count heads");
  CEA_REQUIRE(W <= 1 || out->stride[2] == D, CEA_EINVAL,
              "ulysses_scatter: the heads of an output token must be contiguous");
  if (pos_out) {
    if ((rc = check_tensor(pos_out, "pos_out", 2, CEA_I64, false))) return rc;
    CEA_REQUIRE(pos_out->size[0] == B && pos_out->size[1] == S, CEA_EINVAL,
                "ulysses_scatter: pos_out must be [B, S]");
  }
  UlyssesScatterParams p;
  memset(&p, 0, sizeof(p));
  p.n = n; p.B = (int32_t)B; p.S = (int32_t)S;
  p.q_bytes = (int32_t)(q_count * D * esz);
  p.kv_bytes = (int32_t)(kv_count * D * esz);
  int64_t align[8 * CEA_MAX_PARTS + 6];
  int na = 0;
  int64_t tok = 0;
  for (int j = 0; j < n; ++j) {
    const cea_tensor* src[3] = {&qs[j], &ks[j], &vs[j]};
    const int64_t start[3] = {q_start, kv_start, kv_start};
    const int64_t count[3] = {q_count, kv_count, kv_count};
    for (int c = 0; c < 3; ++c) {
      if ((rc = check_tensor(src[c], c == 0 ? "q_j" : c == 1 ? "k_j" : "v_j", 4, dt, true))) return rc;
      const cea_tensor* t = src[c];
      CEA_REQUIRE(t->size[0] == B && t->size[1] == qs[j].size[1] && t->size[3] == D, CEA_EINVAL,
                  "ulysses_scatter: shard %d shapes do not match the output", j);
      CEA_REQUIRE(start[c] >= 0 && start[c] + count[c] <= t->size[2], CEA_EINVAL,
                  "ulysses_scatter: head slice out of range for shard %d", j);
      CEA_REQUIRE(count[c] <= 1 || t->stride[2] == D, CEA_EINVAL,
                  "ulysses_scatter: the heads of a shard token must be contiguous");
      const char* base = (const char*)t->data + start[c] * t->stride[2] * esz;
      int64_t* st = c == 0 ? p.qs[j] : c == 1 ? p.ks[j] : p.vs[j];
      st[0] = t->stride[0] * esz;
      st[1] = t->stride[1] * esz;
      if (c == 0) p.q[j] = base; else if (c == 1) p.k[j] = base; else p.v[j] = base;
      align[na++] = (int64_t)(uintptr_t)base;
      align[na++] = st[0];
      align[na++] = st[1];
    }
    if (positions) {
      if ((rc = check_tensor(&positions[j], "positions_j", 2, CEA_I64, false))) return rc;
      CEA_REQUIRE(positions[j].size[0] == B && positions[j].size[1] == qs[j].size[1], CEA_EINVAL,
                  "ulysses_scatter: positions of shard %d must be [B, s_j]", j);
      p.pos[j] = (const int64_t*)positions[j].data;
      p.ps[j][0] = positions[j].stride[0];
      p.ps[j][1] = positions[j].stride[1];
    }
    p.tok_off[j] = (int32_t)tok;
    tok += qs[j].size[1];
  }
  p.tok_off[n] = (int32_t)tok;
  CEA_REQUIRE(tok == S, CEA_EINVAL, "ulysses_scatter: the shards hold %lld tokens, out has %lld",
              (long long)tok, (long long)S);
  p.out = (char*)out->data;
  p.os_b = out->stride[0] * esz;
  p.os_s = out->stride[1] * esz;
  if (pos_out) {
    p.pos_out = (int64_t*)pos_out->data;
    p.pos_b = pos_out->stride[0];
    p.pos_s = pos_out->stride[1];
  }
  align[na++] = (int64_t)(uintptr_t)p.out;
  align[na++] = p.os_b;
  align[na++] = p.os_s;
  align[na++] = p.q_bytes;
  align[na++] = p.kv_bytes;
  return launch_ulysses_scatter(p, copy_vec(align, na, esz), (hipStream_t)stream);
}

int cea_ulysses_gather(int32_t n, const cea_tensor* outs, int64_t token_start, cea_tensor* out,
                       void* stream) {
  CEA_REQUIRE(outs && out, CEA_EINVAL, "ulysses_gather: missing tensor");
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "ulysses_gather: between 1 and %d ranks supported, got %d", CEA_MAX_PARTS, n);
  int rc;
  if ((rc = check_tensor(out, "out", 4, -1, true))) return rc;
  const int dt = out->dtype;
  const int esz = (int)dtype_size(dt);
  const int64_t B = out->size[0], S = out->size[1], H = out->size[2], D = out->size[3];
  CEA_REQUIRE(H <= 1 || out->stride[2] == D, CEA_EINVAL,
              "ulysses_gather: the heads of an output token must be contiguous");
  UlyssesGatherParams p;
  memset(&p, 0, sizeof(p));
  p.n = n; p.B = (int32_t)B; p.S = (int32_t)S;
  int64_t align[4 * CEA_MAX_PARTS + 3];
  int na = 0;
  int64_t heads = 0;
  for (int j = 0; j < n; ++j) {
    const cea_tensor* t = &outs[j];
    if ((rc = check_tensor(t, "outs_j", 4, dt, true))) return rc;
    CEA_REQUIRE(t->size[0] == B && t->size[3] == D, CEA_EINVAL,
                "ulysses_gather: head output %d does not match the output", j);
    CEA_REQUIRE(token_start >= 0 && token_start + S <= t->size[1], CEA_EINVAL,
                "ulysses_gather: tokens [%lld, %lld) outside head output %d", (long long)token_start,
                (long long)(token_start + S), j);
    CEA_REQUIRE(t->size[2] <= 1 || t->stride[2] == D, CEA_EINVAL,
                "ulysses_gather: the heads of a source token must be contiguous");
    p.src[j] = (const char*)t->data + token_start * t->stride[1] * esz;
    p.ss[j][0] = t->stride[0] * esz;
    p.ss[j][1] = t->stride[1] * esz;
    p.bytes[j] = (int32_t)(t->size[2] * D * esz);
    p.dst_off[j] = (int32_t)(heads * D * esz);
    heads += t->size[2];
    align[na++] = (int64_t)(uintptr_t)p.src[j];
    align[na++] = p.ss[j][0];
    align[na++] = p.ss[j][1];
    align[na++] = p.bytes[j];
  }
  CEA_REQUIRE(heads == H, CEA_EINVAL, "ulysses_gather: head outputs hold %lld heads, out has %lld",
              (long long)heads, (long long)H);
  p.out = (char*)out->data;
  p.os_b = out->stride[0] * esz;
  p.os_s = out->stride[1] * esz;
  align[na++] = (int64_t)(uintptr_t)p.out;
  align[na++] = p.os_b;
  align[na++] = p.os_s;
  return launch_ulysses_gather(p, copy_vec(align, na, esz), (hipStream_t)stream);
}

size_t cea_partitioned_attention_workspace_bytes(int32_t n, const int64_t* Sk, int64_t B,
                                                 int64_t Sq, int64_t Hq, int64_t Hkv, int64_t D,
                                                 int32_t in_dtype) {
  if (n <= 0 || n > CEA_MAX_PARTS || B <= 0) return 256;
  const size_t esz = in_dtype == CEA_F64 ? 8 : 4;
  size_t need = 0;
  int64_t maxsk = 0;
  for (int i = 0; i < n; ++i) maxsk = Sk[i] > maxsk ? Sk[i] : maxsk;
  need += tile_bytes(B, maxsk);
  // per-partition partials (out, lse) in the accumulation dtype
  need += (size_t)n * align_up((size_t)(B * Sq * Hq * D) * esz, 256);
  need += (size_t)n * align_up((size_t)(B * Hq * Sq) * esz, 256);
  const size_t dec = decode_ws_bytes(Sk, n, B, Sq, Hq, Hkv, D, in_dtype);
  return dec > need ? dec : need;
}

int cea_partitioned_attention(const cea_tensor* q, int32_t n, const cea_tensor* ks,
                              const cea_tensor* vs, const cea_tensor* q_pos,
                              const cea_tensor* k_pos_s, int32_t causal, double scale,
                              const int32_t* kv_map, int32_t kv_map_len, cea_tensor* part_out,
                              cea_tensor* part_lse, cea_tensor* out, cea_tensor* lse,
                              void* workspace, size_t workspace_bytes, void* stream) {
  CEA_REQUIRE(n >= 1 && n <= CEA_MAX_PARTS, CEA_EUNSUPPORTED,
              "partitioned attention: between 1 and %d partitions supported, got %d",
              CEA_MAX_PARTS, n);
  CEA_REQUIRE(q && ks && vs && q_pos && k_pos_s && out, CEA_EINVAL,
              "partitioned attention: missing tensor");
  CEA_REQUIRE((part_out == nullptr) == (part_lse == nullptr), CEA_EINVAL,
              "partitioned attention: part_out and part_lse go together");
  hipStream_t st = (hipStream_t)stream;
  int rc = check_tensor(q, "q", 4, -1, true);
  if (rc) return rc;
  CEA_REQUIRE(q->dtype != CEA_F64 || out->dtype == CEA_F64, CEA_EINVAL,
              "partitioned attention: float64 inputs need a float64 output");
  const int64_t B = q->size[0], Sq = q->size[1], Hq = q->size[2], D = q->size[3];
  const int acc = q->dtype == CEA_F64 ? CEA_F64 : CEA_F32;
  const size_t esz = acc == CEA_F64 ? 8 : 4;
  int64_t sks[CEA_MAX_PARTS];
  for (int i = 0; i < n; ++i) sks[i] = ks[i].size[1];
  const size_t need = cea_partitioned_attention_workspace_bytes(n, sks, B, Sq, Hq, ks[0].size[2],
                                                                D, q->dtype);
  CEA_REQUIRE(workspace != nullptr && workspace_bytes >= need, CEA_ENOSPACE,
              "partitioned attention: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
  char* ws = (char*)workspace;
  // fast path: every partition through the split-KV decode kernels, merged in one reduction
  {
    AttnParams blocks[CEA_MAX_PARTS];
    bool dec = true;
    for (int i = 0; i < n; ++i) {
      rc = make_attn_params(&blocks[i], q, &ks[i], &vs[i], q_pos, &k_pos_s[i], causal, scale,
                            kv_map, kv_map_len, out, lse, 0);
      if (rc) return rc;
      dec = dec && use_decode(blocks[i]);
    }
    if (dec) {
      const DecodeUnits du = decode_units(Hq, blocks[0].Hkv, Sq, blocks[0].map);
      dec = decode_plan_fits(B, Sq, Hq, du.units,
                             plan_decode(sks, n, B, Sq, du.units, du.G, D).total_chunks);
    }
    if (dec && part_out) {
      for (int i = 0; i < n && rc == 0; ++i) {
        rc = check_tensor(&part_out[i], "part_out", 4, acc, true);
        if (!rc) rc = check_tensor(&part_lse[i], "part_lse", 3, acc, false);
        if (!rc)
          CEA_REQUIRE(part_out[i].size[0] == B && part_out[i].size[1] == Sq &&
                          part_out[i].size[2] == Hq && part_out[i].size[3] == D &&
                          part_lse[i].size[0] == B && part_lse[i].size[1] == Hq &&
                          part_lse[i].size[2] == Sq,
                      CEA_EINVAL, "partitioned attention: per-partition outputs have wrong shapes");
      }
      if (rc) return rc;
    }
    if (dec) return run_decode(blocks, n, part_out, part_lse, ws, workspace_bytes, st);
  }
  int64_t maxsk = 0;
  for (int i = 0; i < n; ++i) maxsk = sks[i] > maxsk ? sks[i] : maxsk;
  char* tiles = ws;
  char* parts = ws + tile_bytes(B, maxsk);
  const size_t obytes = align_up((size_t)(B * Sq * Hq * D) * esz, 256);
  const size_t lbytes = align_up((size_t)(B * Hq * Sq) * esz, 256);

  cea_tensor po[CEA_MAX_PARTS], pl[CEA_MAX_PARTS];
  for (int i = 0; i < n; ++i) {
    if (part_out) {
      po[i] = part_out[i];
      pl[i] = part_lse[i];
    } else {
      cea_tensor& o = po[i];
      cea_tensor& l = pl[i];
      o.data = parts + i * obytes;
      o.dtype = acc; o.ndim = 4;
      o.size[0] = B; o.size[1] = Sq; o.size[2] = Hq; o.size[3] = D;
      o.stride[3] = 1; o.stride[2] = D; o.stride[1] = Hq * D; o.stride[0] = Sq * Hq * D;
      l.data = parts + n * obytes + i * lbytes;
      l.dtype = acc; l.ndim = 3;
      l.size[0] = B; l.size[1] = Hq; l.size[2] = Sq;
      l.stride[2] = 1; l.stride[1] = Sq; l.stride[0] = Hq * Sq;
    }
    AttnParams p;
    rc = make_attn_params(&p, q, &ks[i], &vs[i], q_pos, &k_pos_s[i], causal, scale, kv_map,
                          kv_map_len, &po[i], &pl[i], 0);
    if (rc) return rc;
    // the workspace past the tile summaries holds the partials: this partition must not
    // take the decode route (its chunk partials would not fit in the tile slice)
    rc = run_attention(p, tiles, tile_bytes(B, maxsk), st, false);
    if (rc) return rc;
  }
  if (n == 1 && out->data == po[0].data) return CEA_OK;
  return merge_impl(n, po, pl, out, lse, 0, st);
}

int cea_rmsnorm(const cea_tensor* x, const cea_tensor* weight, double eps, cea_tensor* y,
                void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2, -1, true))) return rc;
  if ((rc = check_tensor(weight, "weight", 1, -1, true))) return rc;
  if ((rc = check_tensor(y, "y", 2, -1, true))) return rc;
  CEA_REQUIRE(weight->size[0] == x->size[1], CEA_EINVAL, "rmsnorm: weight must be [C]");
  CEA_REQUIRE(y->size[0] == x->size[0] && y->size[1] == x->size[1], CEA_EINVAL,
              "rmsnorm: y must match x");
  return launch_rmsnorm(x, weight, eps, y, (hipStream_t)stream);
}

int cea_rope_tables(const cea_tensor* positions, const cea_tensor* inv_freq, cea_tensor* cos,
                    cea_tensor* sin, void* stream) {
  int rc;
  if ((rc = check_tensor(positions, "positions", 2, CEA_I64, false))) return rc;
  if ((rc = check_tensor(inv_freq, "inv_freq", 1, -1, true))) return rc;
  if ((rc = check_tensor(cos, "cos", 3, -1, true))) return rc;
  if ((rc = check_tensor(sin, "sin", 3, cos->dtype, true))) return rc;
  const int want = cos->dtype == CEA_F64 ? CEA_F64 : CEA_F32;
  CEA_REQUIRE(inv_freq->dtype == want, CEA_EINVAL, "rope_tables: inv_freq must be %s",
              dtype_name(want));
  const int64_t half = inv_freq->size[0];
  for (const cea_tensor* t : {(const cea_tensor*)cos, (const cea_tensor*)sin})
    CEA_REQUIRE(t->size[0] == positions->size[0] && t->size[1] == positions->size[1] &&
                    t->size[2] == 2 * half,
                CEA_EINVAL, "rope_tables: tables must be [B, S, 2*len(inv_freq)]");
  return launch_rope_tables(positions, inv_freq, cos, sin, (hipStream_t)stream);
}

int cea_apply_rotary(const cea_tensor* x, const cea_tensor* cos, const cea_tensor* sin,
                     cea_tensor* out, void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 4, -1, true))) return rc;
  if ((rc = check_tensor(cos, "cos", 3, x->dtype, true))) return rc;
  if ((rc = check_tensor(sin, "sin", 3, x->dtype, true))) return rc;
  if ((rc = check_tensor(out, "out", 4, x->dtype, true))) return rc;
  const int64_t D = x->size[3];
  CEA_REQUIRE(D % 2 == 0, CEA_EINVAL, "apply_rotary: head size must be even");
  for (const cea_tensor* t : {cos, sin})
    CEA_REQUIRE((t->size[0] == x->size[0] || (t->size[0] == 1 && t->stride[0] == 0) ||
                 t->size[0] == 1) &&
                    t->size[1] == x->size[1] && t->size[2] == D,
                CEA_EINVAL, "apply_rotary: cos/sin must be [B, S, D]");
  for (int i = 0; i < 4; ++i)
    CEA_REQUIRE(out->size[i] == x->size[i], CEA_EINVAL, "apply_rotary: out must match x");
  cea_tensor c = *cos, s = *sin;
  if (c.size[0] == 1) c.stride[0] = 0;  // broadcast over the batch
  if (s.size[0] == 1) s.stride[0] = 0;
  return launch_apply_rotary(x, &c, &s, out, (hipStream_t)stream);
}

int cea_kv_append(const cea_tensor* k, const cea_tensor* v, const cea_tensor* pos,
                  const cea_tensor* cos, const cea_tensor* sin, cea_tensor* cache_k,
                  cea_tensor* cache_v, cea_tensor* cache_pos, int64_t offset, void* stream) {
  int rc;
  if ((rc = check_tensor(k, "k", 4, -1, true))) return rc;
  const int dt = k->dtype;
  if ((rc = check_tensor(v, "v", 4, dt, true))) return rc;
  if ((rc = check_tensor(pos, "positions", 2, CEA_I64, false))) return rc;
  if ((rc = check_tensor(cache_k, "cache_k", 4, dt, true))) return rc;
  if ((rc = check_tensor(cache_v, "cache_v", 4, dt, true))) return rc;
  if ((rc = check_tensor(cache_pos, "cache_pos", 2, CEA_I64, false))) return rc;
  const int64_t B = k->size[0], n = k->size[1], H = k->size[2], D = k->size[3];
  for (int i = 0; i < 4; ++i)
    CEA_REQUIRE(v->size[i] == k->size[i], CEA_EINVAL, "kv_append: v must match k [B,n,H,D]");
  CEA_REQUIRE(pos->size[0] == B && pos->size[1] == n, CEA_EINVAL,
              "kv_append: positions must be [B, n]");
  const int64_t cap = cache_k->size[2];
  for (const cea_tensor* c : {(const cea_tensor*)cache_k, (const cea_tensor*)cache_v})
    CEA_REQUIRE(c->size[0] == B && c->size[1] == H && c->size[2] == cap && c->size[3] == D,
                CEA_EINVAL, "kv_append: caches must be [B, H, capacity, D]");
  CEA_REQUIRE(cache_pos->size[0] == B && cache_pos->size[1] == cap, CEA_EINVAL,
              "kv_append: cache positions must be [B, capacity]");
  CEA_REQUIRE(offset >= 0 && offset + n <= cap, CEA_EINVAL,
              "kv_append: slots %lld..%lld exceed the capacity %lld", (long long)offset,
              (long long)(offset + n), (long long)cap);
  CEA_REQUIRE((cos == nullptr) == (sin == nullptr), CEA_EINVAL,
              "kv_append: give both rotary tables or neither");
  cea_tensor c, sn;
  if (cos) {
    if ((rc = check_tensor(cos, "cos", 3, dt, true))) return rc;
    if ((rc = check_tensor(sin, "sin", 3, dt, true))) return rc;
    CEA_REQUIRE(D % 2 == 0, CEA_EINVAL, "kv_append: head size must be even to rotate");
    for (const cea_tensor* t : {cos, sin})
      CEA_REQUIRE((t->size[0] == B || t->size[0] == 1) && t->size[1] == n && t->size[2] == D,
                  CEA_EINVAL, "kv_append: cos/sin must be [B, n, D]");
    c = *cos;
    sn = *sin;
    if (c.size[0] == 1) c.stride[0] = 0;  // broadcast over the batch
    if (sn.size[0] == 1) sn.stride[0] = 0;
  } else {
    CEA_REQUIRE(D % 2 == 0, CEA_EINVAL, "kv_append: head size must be even");
  }
  return launch_kv_append(k, v, pos, cos ? &c : nullptr, cos ? &sn : nullptr, cache_k, cache_v,
                          cache_pos, offset, (hipStream_t)stream);
}

int cea_rmsnorm_rope(const cea_tensor* x, const cea_tensor* weight, double eps,
                     const cea_tensor* positions, const cea_tensor* inv_freq, int32_t num_heads,
                     cea_tensor* out, void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2, -1, true))) return rc;
  if ((rc = check_tensor(weight, "weight", 1, x->dtype, true))) return rc;
  if ((rc = check_tensor(out, "out", 2, x->dtype, true))) return rc;
  CEA_REQUIRE(positions && (positions->ndim == 1 || positions->ndim == 2) &&
                  positions->dtype == CEA_I64,
              CEA_EINVAL, "rmsnorm_rope: positions must be int64 [S] or [1, S]");
  const int64_t S = x->size[0], C = x->size[1];
  const int64_t npos = positions->ndim == 2 ? positions->size[1] : positions->size[0];
  CEA_REQUIRE(positions->ndim == 1 || positions->size[0] == 1, CEA_EINVAL,
              "rmsnorm_rope: positions must have batch 1");
  CEA_REQUIRE(npos == S, CEA_EINVAL, "rmsnorm_rope: one position per row needed");
  CEA_REQUIRE(num_heads >= 1 && C % num_heads == 0, CEA_EINVAL,
              "rmsnorm_rope: %lld features do not split into %d heads", (long long)C, num_heads);
  const int64_t D = C / num_heads;
  CEA_REQUIRE(D % 2 == 0 && D <= 1024, CEA_EUNSUPPORTED,
              "rmsnorm_rope: head size %lld must be even and <= 1024", (long long)D);
  CEA_REQUIRE(weight->size[0] == C, CEA_EINVAL, "rmsnorm_rope: weight must be [C]");
  CEA_REQUIRE(out->size[0] == S && out->size[1] == C, CEA_EINVAL, "rmsnorm_rope: out must match x");
  if ((rc = check_tensor(inv_freq, "inv_freq", 1, x->dtype == CEA_F64 ? CEA_F64 : CEA_F32, true)))
    return rc;
  CEA_REQUIRE(inv_freq->size[0] == D / 2, CEA_EINVAL, "rmsnorm_rope: inv_freq must be [D/2]");
  return launch_rmsnorm_rope(x, weight, eps, positions, inv_freq, num_heads, out,
                             (hipStream_t)stream);
}

int cea_gated_mul(const cea_tensor* gate, const cea_tensor* up, cea_tensor* out, int32_t act,
                  void* stream) {
  int rc;
  if ((rc = check_tensor(gate, "gate", 2, -1, true))) return rc;
  if ((rc = check_tensor(up, "up", 2, gate->dtype, true))) return rc;
  if ((rc = check_tensor(out, "out", 2, gate->dtype, true))) return rc;
  for (int i = 0; i < 2; ++i)
    CEA_REQUIRE(up->size[i] == gate->size[i] && out->size[i] == gate->size[i], CEA_EINVAL,
                "gated_mul: gate, up and out must have the same shape");
  CEA_REQUIRE(act >= CEA_ACT_SILU && act <= CEA_ACT_RELU, CEA_EUNSUPPORTED,
              "gated_mul: unknown activation %d", (int)act);
  return launch_gated_mul(gate, up, out, act, (hipStream_t)stream);
}

int cea_silu_mul(const cea_tensor* gate, const cea_tensor* up, cea_tensor* out, void* stream) {
  return cea_gated_mul(gate, up, out, CEA_ACT_SILU, stream);
}

// x [M, K]; weight rows [N, K] (innermost stride 1, any row stride); bias [N] or NULL
static int check_projection(const char* what, const cea_tensor* x, const cea_tensor* w,
                            const cea_tensor* b, const char* wname, const char* bname) {
  int rc;
  if ((rc = check_tensor(w, wname, 2, x->dtype, true))) return rc;
  CEA_REQUIRE(w->size[1] == x->size[1], CEA_EINVAL,
              "%s: %s has %lld input features, x has %lld", what, wname, (long long)w->size[1],
              (long long)x->size[1]);
  CEA_REQUIRE(w->size[0] <= 1 || w->stride[0] >= w->size[1], CEA_EINVAL,
              "%s: %s rows overlap", what, wname);
  if (b != nullptr) {
    if ((rc = check_tensor(b, bname, 1, x->dtype, true))) return rc;
    CEA_REQUIRE(b->size[0] == w->size[0], CEA_EINVAL, "%s: %s must be [%lld]", what, bname,
                (long long)w->size[0]);
  }
  return CEA_OK;
}

static int check_linear_io(const char* what, const cea_tensor* x, const cea_tensor* y,
                           int64_t n) {
  int rc;
  if ((rc = check_tensor(x, "x", 2, -1, true))) return rc;
  CEA_REQUIRE(x->dtype == CEA_BF16 || x->dtype == CEA_F16 || x->dtype == CEA_F32 ||
                  x->dtype == CEA_F64,
              CEA_EUNSUPPORTED, "%s: unsupported dtype %s", what, dtype_name(x->dtype));
  CEA_REQUIRE(x->size[0] <= 1 || x->stride[0] >= x->size[1], CEA_EINVAL, "%s: x rows overlap",
              what);
  if ((rc = check_tensor(y, "y", 2, x->dtype, true))) return rc;
  CEA_REQUIRE(y->size[0] == x->size[0] && y->size[1] == n, CEA_EINVAL,
              "%s: y must be [%lld, %lld]", what, (long long)x->size[0], (long long)n);
  CEA_REQUIRE(y->size[0] <= 1 || y->stride[0] >= y->size[1], CEA_EINVAL, "%s: y rows overlap",
              what);
  return CEA_OK;
}

int cea_linear(const cea_tensor* x, const cea_tensor* weight, const cea_tensor* bias,
               cea_tensor* y, void* stream) {
  int rc;
  CEA_REQUIRE(x != nullptr && weight != nullptr, CEA_EINVAL, "linear: missing tensor");
  if ((rc = check_tensor(weight, "weight", 2, -1, true))) return rc;
  if ((rc = check_linear_io("linear", x, y, weight->size[0]))) return rc;
  if ((rc = check_projection("linear", x, weight, bias, "weight", "bias"))) return rc;
  return launch_linear(x, weight, nullptr, bias, nullptr, y, 0, 0, (hipStream_t)stream);
}

int cea_linear_gated(const cea_tensor* x, const cea_tensor* w_gate, const cea_tensor* w_up,
                     const cea_tensor* b_gate, const cea_tensor* b_up, cea_tensor* y,
                     int32_t act, void* stream) {
  int rc;
  CEA_REQUIRE(x != nullptr && w_gate != nullptr && w_up != nullptr, CEA_EINVAL,
              "linear_gated: missing tensor");
  if ((rc = check_tensor(w_gate, "w_gate", 2, -1, true))) return rc;
  if ((rc = check_linear_io("linear_gated", x, y, w_gate->size[0]))) return rc;
  if ((rc = check_projection("linear_gated", x, w_gate, b_gate, "w_gate", "b_gate"))) return rc;
  if ((rc = check_projection("linear_gated", x, w_up, b_up, "w_up", "b_up"))) return rc;
  CEA_REQUIRE(w_up->size[0] == w_gate->size[0], CEA_EINVAL,
              "linear_gated: w_gate and w_up must have the same number of rows");
  CEA_REQUIRE(w_gate->size[0] <= 1 || w_up->stride[0] == w_gate->stride[0], CEA_EINVAL,
              "linear_gated: w_gate and w_up must share a row stride");
  CEA_REQUIRE((b_gate == nullptr) == (b_up == nullptr), CEA_EINVAL,
              "linear_gated: give both biases or neither");
  CEA_REQUIRE(act >= CEA_ACT_SILU && act <= CEA_ACT_RELU, CEA_EUNSUPPORTED,
              "linear_gated: unknown activation %d", (int)act);
  return launch_linear(x, w_gate, w_up, b_gate, b_up, y, 1, act, (hipStream_t)stream);
}

}  // extern "C"
