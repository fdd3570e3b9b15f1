// PyTorch operators of the collab_edge library: the thin PyTorch-ROCm layer between the
// package's Python functions and the C ABI of include/collab_edge_attn.h.
//
// Each operator checks that its tensors live on one ROCm device, allocates its outputs (and
// the kernels' workspace) through PyTorch's caching allocator on that device, makes the
// device current, and calls the C ABI on PyTorch's current stream of that device.  C ABI
// status codes become the exceptions the reference raises for the same conditions:
// CEA_EINVAL -> ValueError, CEA_EUNSUPPORTED -> NotImplementedError, others -> RuntimeError.
// Host (CPU) tensors are refused with RuntimeError: there is no host path.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "collab_edge_attn.h"

namespace {

using at::Tensor;

int32_t code_of(c10::ScalarType t) {
  switch (t) {
    case at::kFloat: return CEA_F32;
    case at::kBFloat16: return CEA_BF16;
    case at::kHalf: return CEA_F16;
    case at::kDouble: return CEA_F64;
    case at::kLong: return CEA_I64;
    default: return -1;
  }
}

cea_tensor arg(const Tensor& t) {
  cea_tensor a;
  const int32_t code = code_of(t.scalar_type());
  TORCH_CHECK_NOT_IMPLEMENTED(code >= 0, "dtype ", t.scalar_type(), " is not supported by the kernels");
  TORCH_CHECK_VALUE(t.dim() <= CEA_MAX_DIMS, "at most ", CEA_MAX_DIMS, " dimensions supported, got ",
                    t.dim());
  a.data = t.numel() > 0 ? t.data_ptr() : nullptr;
  a.dtype = code;
  a.ndim = (int32_t)t.dim();
  for (int i = 0; i < CEA_MAX_DIMS; ++i) {
    a.size[i] = i < t.dim() ? t.size(i) : 0;
    a.stride[i] = i < t.dim() ? t.stride(i) : 0;
  }
  return a;
}

std::vector<cea_tensor> args(at::TensorList ts) {
  std::vector<cea_tensor> v;
  v.reserve(ts.size());
  for (const Tensor& t : ts) v.push_back(arg(t));
  return v;
}

void check_rc(int rc, const char* what) {
  if (rc == CEA_OK) return;
  const std::string msg = std::string(what) + ": " + cea_last_error();
  TORCH_CHECK_VALUE(rc != CEA_EINVAL, msg);
  TORCH_CHECK_NOT_IMPLEMENTED(rc != CEA_EUNSUPPORTED, msg);
  TORCH_CHECK(false, msg);
}

// The device all tensors share (every defined tensor must be on one ROCm device).
at::Device device_of(std::initializer_list<const Tensor*> ts, at::TensorList more = {}) {
  c10::optional<at::Device> dev;
  auto visit = [&](const Tensor& t) {
    if (!t.defined()) return;
    TORCH_CHECK(t.is_cuda(), "collaborative-edge-system_amd runs its kernels on a ROCm GPU; got a tensor on ",
                t.device());
    if (!dev) dev = t.device();
    TORCH_CHECK(t.device() == *dev, "tensors on different devices: ", *dev, " and ", t.device());
  };
  for (const Tensor* t : ts) visit(*t);
  for (const Tensor& t : more) visit(t);
  TORCH_CHECK(dev.has_value(), "no tensor given");
  return *dev;
}

// Every tensor of a further list on the device `dev` found for the call's other tensors.
void on_device(const at::Device& dev, at::TensorList more) {
  if (more.empty()) return;
  const at::Device d = device_of({}, more);
  TORCH_CHECK(d == dev, "tensors on different devices: ", dev, " and ", d);
}

void* stream_of(const at::Device& d) {
  return (void*)c10::hip::getCurrentHIPStream(d.index()).stream();
}

// The kernels' workspace: one buffer per (device, stream), grown to the largest request seen
// and then reused by every call on that stream (calls on one stream run in order, so a call
// never overwrites scratch a queued call still reads).  A grown-out buffer returns to
// PyTorch's caching allocator, which hands its memory out again only in stream order - unless
// a HIP graph capture may have recorded it: graph replays keep writing to the captured
// address whatever the allocator has since handed it to, so such a buffer is kept alive
// (retired, never freed) when a larger one replaces it.
struct WsEntry {
  Tensor t;
  bool captured = false;  // used while its stream was capturing a graph
};
std::mutex g_ws_mu;
std::map<std::pair<int, void*>, WsEntry> g_ws;
std::vector<Tensor> g_ws_retired;

Tensor workspace(size_t bytes, const at::Device& d) {
  void* st = stream_of(d);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing((hipStream_t)st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
  const int64_t want = (int64_t)std::max<size_t>((bytes + 4095) & ~(size_t)4095, 4096);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  WsEntry& e = g_ws[{(int)d.index(), st}];
  if (!e.t.defined() || e.t.numel() < want) {
    if (e.t.defined() && (e.captured || capturing)) g_ws_retired.push_back(e.t);
    e.t = at::empty({want}, at::TensorOptions().dtype(at::kByte).device(d));
    e.captured = false;
  }
  e.captured = e.captured || capturing;
  return e.t;
}

// q / k / v style operands need a unit innermost stride
Tensor inner(const Tensor& t) {
  return (t.dim() == 0 || t.size(-1) <= 1 || t.stride(-1) == 1) ? t : t.contiguous();
}

Tensor as_i64(const Tensor& t) { return t.scalar_type() == at::kLong ? t : t.to(at::kLong); }

at::ScalarType acc_of(at::ScalarType t) { return t == at::kDouble ? at::kDouble : at::kFloat; }

std::vector<int32_t> map_of(const c10::optional<at::IntArrayRef>& kv_map) {
  std::vector<int32_t> m;
  if (kv_map) for (int64_t x : *kv_map) m.push_back((int32_t)x);
  return m;
}

// ---------------------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------------------
std::vector<Tensor> attention(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in,
                              const Tensor& q_pos_in, const Tensor& k_pos_in, bool causal, double scale,
                              c10::optional<at::IntArrayRef> kv_map, bool with_lse) {
  const at::Device dev = device_of({&q_in, &k_in, &v_in, &q_pos_in, &k_pos_in});
  const Tensor q = inner(q_in), k = inner(k_in), v = inner(v_in);
  const Tensor qp = as_i64(q_pos_in), kp = as_i64(k_pos_in);
  TORCH_CHECK_VALUE(q.dim() == 4 && k.dim() == 4, "q and k must be [B, S, H, D]");
  const int64_t B = q.size(0), Sq = q.size(1), Hq = q.size(2), D = q.size(3);
  const int64_t Sk = k.size(1), Hkv = k.size(2);
  const at::ScalarType acc = acc_of(q.scalar_type());
  const auto o_opts = at::TensorOptions().device(dev).dtype(with_lse ? acc : q.scalar_type());
  Tensor out = at::empty({B, Sq, Hq, D}, o_opts);
  Tensor lse = with_lse ? at::empty({B, Hq, Sq}, o_opts.dtype(acc)) : Tensor();
  c10::DeviceGuard guard(dev);
  const std::vector<int32_t> m = map_of(kv_map);
  Tensor ws = workspace(cea_attention_workspace_bytes(B, Sq, Hq, Sk, Hkv, D, code_of(q.scalar_type())), dev);
  cea_tensor a[5] = {arg(q), arg(k), arg(v), arg(qp), arg(kp)};
  cea_tensor o = arg(out), l = with_lse ? arg(lse) : cea_tensor{};
  check_rc(cea_attention_with_lse(&a[0], &a[1], &a[2], &a[3], &a[4], causal ? 1 : 0, scale,
                                  m.empty() ? nullptr : m.data(), (int32_t)m.size(), &o,
                                  with_lse ? &l : nullptr, 0, ws.data_ptr(), (size_t)ws.numel(),
                                  stream_of(dev)),
           "attention_with_lse");
  if (with_lse) return {out, lse};
  return {out};
}

void attention_into(Tensor out, Tensor lse, const Tensor& q_in, const Tensor& k_in, const Tensor& v_in,
                    const Tensor& q_pos_in, const Tensor& k_pos_in, bool causal, double scale,
                    c10::optional<at::IntArrayRef> kv_map, bool accumulate,
                    c10::optional<Tensor> final_out) {
  const Tensor fin = final_out ? *final_out : Tensor();
  const at::Device dev = device_of({&out, &lse, &q_in, &k_in, &v_in, &q_pos_in, &k_pos_in, &fin});
  const Tensor q = inner(q_in), k = inner(k_in), v = inner(v_in);
  const Tensor qp = as_i64(q_pos_in), kp = as_i64(k_pos_in);
  TORCH_CHECK_VALUE(q.dim() == 4 && k.dim() == 4, "q and k must be [B, S, H, D]");
  c10::DeviceGuard guard(dev);
  const std::vector<int32_t> m = map_of(kv_map);
  Tensor ws = workspace(cea_attention_workspace_bytes(q.size(0), q.size(1), q.size(2), k.size(1), k.size(2),
                                                      q.size(3), code_of(q.scalar_type())),
                        dev);
  cea_tensor a[5] = {arg(q), arg(k), arg(v), arg(qp), arg(kp)};
  cea_tensor o = arg(out), l = arg(lse);
  if (fin.defined()) {
    cea_tensor f = arg(fin);
    check_rc(cea_attention_merge_final(&a[0], &a[1], &a[2], &a[3], &a[4], causal ? 1 : 0, scale,
                                       m.empty() ? nullptr : m.data(), (int32_t)m.size(), &o, &l, &f,
                                       ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
             "attention_merge_final");
    return;
  }
  check_rc(cea_attention_with_lse(&a[0], &a[1], &a[2], &a[3], &a[4], causal ? 1 : 0, scale,
                                  m.empty() ? nullptr : m.data(), (int32_t)m.size(), &o, &l,
                                  accumulate ? 1 : 0, ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
           "attention_with_lse");
}

std::vector<Tensor> merge(at::TensorList outs_in, at::TensorList lses, bool pairwise,
                          c10::optional<at::ScalarType> out_dtype) {
  TORCH_CHECK_VALUE(!outs_in.empty() && outs_in.size() == lses.size(),
                    "need the same positive number of outputs and lses");
  const at::Device dev = device_of({}, outs_in);
  on_device(dev, lses);
  std::vector<Tensor> outs;
  for (const Tensor& o : outs_in) outs.push_back(inner(o));
  const Tensor& o0 = outs[0];
  Tensor out = at::empty(o0.sizes(), o0.options().dtype(out_dtype ? *out_dtype : o0.scalar_type()));
  Tensor lse = at::empty(lses[0].sizes(), lses[0].options());
  c10::DeviceGuard guard(dev);
  std::vector<cea_tensor> oa = args(outs), la = args(lses);
  cea_tensor o = arg(out), l = arg(lse);
  if (pairwise && outs.size() == 2)
    check_rc(cea_merge_attention(&oa[0], &la[0], &oa[1], &la[1], &o, &l, stream_of(dev)), "merge_attention");
  else
    check_rc(cea_merge_attention_list((int32_t)outs.size(), oa.data(), la.data(), &o, &l, stream_of(dev)),
             "merge_attention_list");
  return {out, lse};
}

std::vector<Tensor> partitioned(const Tensor& q_in, const Tensor& q_pos_in, at::TensorList ks_in,
                                at::TensorList vs_in, at::TensorList ps_in, bool causal, double scale,
                                c10::optional<at::IntArrayRef> kv_map, at::ScalarType out_dtype,
                                bool with_lse, bool with_parts) {
  const int64_t n = (int64_t)ks_in.size();
  TORCH_CHECK_VALUE(n >= 1 && (int64_t)vs_in.size() == n && (int64_t)ps_in.size() == n,
                    "need one k, v and position tensor per partition");
  const at::Device dev = device_of({&q_in, &q_pos_in}, ks_in);
  on_device(dev, vs_in);
  on_device(dev, ps_in);
  const Tensor q = inner(q_in), qp = as_i64(q_pos_in);
  std::vector<Tensor> ks, vs, ps;
  for (int64_t i = 0; i < n; ++i) {
    ks.push_back(inner(ks_in[i]));
    vs.push_back(inner(vs_in[i]));
    ps.push_back(as_i64(ps_in[i]));
  }
  const int64_t B = q.size(0), Sq = q.size(1), Hq = q.size(2), D = q.size(3);
  const at::ScalarType acc = acc_of(q.scalar_type());
  const auto opts = q.options();
  Tensor out = at::empty({B, Sq, Hq, D}, opts.dtype(out_dtype));
  Tensor lse = with_lse ? at::empty({B, Hq, Sq}, opts.dtype(acc)) : Tensor();
  std::vector<Tensor> pouts, plses;
  if (with_parts)
    for (int64_t i = 0; i < n; ++i) {
      pouts.push_back(at::empty({B, Sq, Hq, D}, opts.dtype(acc)));
      plses.push_back(at::empty({B, Hq, Sq}, opts.dtype(acc)));
    }
  c10::DeviceGuard guard(dev);
  std::vector<int64_t> sks;
  for (const Tensor& k : ks) sks.push_back(k.size(1));
  const size_t ws_bytes = cea_partitioned_attention_workspace_bytes(
      (int32_t)n, sks.data(), B, Sq, Hq, ks[0].size(2), D, code_of(q.scalar_type()));
  Tensor ws = workspace(ws_bytes, dev);
  const std::vector<int32_t> m = map_of(kv_map);
  cea_tensor qa = arg(q), qpa = arg(qp), o = arg(out);
  cea_tensor l = with_lse ? arg(lse) : cea_tensor{};
  std::vector<cea_tensor> ka = args(ks), va = args(vs), pa = args(ps);
  std::vector<cea_tensor> poa = args(pouts), pla = args(plses);
  check_rc(cea_partitioned_attention(&qa, (int32_t)n, ka.data(), va.data(), &qpa, pa.data(), causal ? 1 : 0,
                                     scale, m.empty() ? nullptr : m.data(), (int32_t)m.size(),
                                     with_parts ? poa.data() : nullptr, with_parts ? pla.data() : nullptr, &o,
                                     with_lse ? &l : nullptr, ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
           "partitioned_attention");
  std::vector<Tensor> res{out};
  if (with_lse) res.push_back(lse);
  for (int64_t i = 0; i < (int64_t)pouts.size(); ++i) {
    res.push_back(pouts[i]);
    res.push_back(plses[i]);
  }
  return res;
}

// One rank's share of ring attention over KV blocks in ring order (cea_ring_attention).
std::vector<Tensor> ring(const Tensor& q_in, const Tensor& q_pos_in, at::TensorList ks_in,
                         at::TensorList vs_in, at::TensorList ps_in, bool causal, double scale,
                         c10::optional<at::IntArrayRef> kv_map, bool with_lse) {
  const int64_t n = (int64_t)ks_in.size();
  TORCH_CHECK_VALUE(n >= 1 && (int64_t)vs_in.size() == n && (int64_t)ps_in.size() == n,
                    "need one k, v and position tensor per KV block");
  const at::Device dev = device_of({&q_in, &q_pos_in}, ks_in);
  on_device(dev, vs_in);
  on_device(dev, ps_in);
  const Tensor q = inner(q_in), qp = as_i64(q_pos_in);
  TORCH_CHECK_VALUE(q.dim() == 4, "q must be [B, S, H, D]");
  std::vector<Tensor> ks, vs, ps;
  for (int64_t i = 0; i < n; ++i) {
    ks.push_back(inner(ks_in[i]));
    vs.push_back(inner(vs_in[i]));
    ps.push_back(as_i64(ps_in[i]));
  }
  const int64_t B = q.size(0), Sq = q.size(1), Hq = q.size(2), D = q.size(3);
  const at::ScalarType acc = acc_of(q.scalar_type());
  const auto opts = q.options();
  Tensor out = at::empty({B, Sq, Hq, D}, opts.dtype(with_lse ? acc : q.scalar_type()));
  Tensor lse = with_lse ? at::empty({B, Hq, Sq}, opts.dtype(acc)) : Tensor();
  c10::DeviceGuard guard(dev);
  const std::vector<int32_t> m = map_of(kv_map);
  cea_tensor qa = arg(q), qpa = arg(qp), o = arg(out);
  cea_tensor l = with_lse ? arg(lse) : cea_tensor{};
  std::vector<cea_tensor> ka = args(ks), va = args(vs), pa = args(ps);
  const size_t ws_bytes = cea_ring_attention_workspace_bytes(
      &qa, (int32_t)n, ka.data(), va.data(), &qpa, pa.data(), causal ? 1 : 0,
      m.empty() ? nullptr : m.data(), (int32_t)m.size(), &o, with_lse ? &l : nullptr);
  Tensor ws = workspace(ws_bytes, dev);
  check_rc(cea_ring_attention(&qa, (int32_t)n, ka.data(), va.data(), &qpa, pa.data(), causal ? 1 : 0, scale,
                              m.empty() ? nullptr : m.data(), (int32_t)m.size(), &o,
                              with_lse ? &l : nullptr, ws.data_ptr(), (size_t)ws.numel(), stream_of(dev)),
           "ring_attention");
  if (with_lse) return {out, lse};
  return {out};
}

// ---------------------------------------------------------------------------------------
// wire formats
// ---------------------------------------------------------------------------------------
void pack_partial(const Tensor& out_in, const Tensor& lse, Tensor packed) {
  const at::Device dev = device_of({&out_in, &lse, &packed});
  const Tensor out = inner(out_in);
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(out), l = arg(lse), p = arg(packed);
  check_rc(cea_pack_partial(&a, &l, &p, stream_of(dev)), "pack_partial");
}

std::vector<Tensor> merge_packed(at::TensorList parts_in, at::ScalarType out_dtype, bool with_lse) {
  TORCH_CHECK_VALUE(!parts_in.empty(), "need at least one packed partial");
  const at::Device dev = device_of({}, parts_in);
  std::vector<Tensor> parts;
  for (const Tensor& p : parts_in) parts.push_back(inner(p));
  const Tensor& p0 = parts[0];
  TORCH_CHECK_VALUE(p0.dim() == 4, "packed partials must be [B, Sq, H, D+1]");
  const int64_t B = p0.size(0), Sq = p0.size(1), H = p0.size(2), D1 = p0.size(3);
  Tensor out = at::empty({B, Sq, H, D1 - 1}, p0.options().dtype(out_dtype));
  Tensor lse = with_lse ? at::empty({B, H, Sq}, p0.options()) : Tensor();
  c10::DeviceGuard guard(dev);
  std::vector<cea_tensor> pa = args(parts);
  cea_tensor o = arg(out), l = with_lse ? arg(lse) : cea_tensor{};
  check_rc(cea_merge_packed((int32_t)parts.size(), pa.data(), &o, with_lse ? &l : nullptr, stream_of(dev)),
           "merge_packed");
  if (with_lse) return {out, lse};
  return {out};
}

std::vector<Tensor> ulysses_scatter(at::TensorList qs, at::TensorList ks, at::TensorList vs,
                                    at::TensorList ps, int64_t q_start, int64_t q_count, int64_t kv_start,
                                    int64_t kv_count) {
  const int64_t n = (int64_t)qs.size();
  TORCH_CHECK_VALUE(n >= 1 && (int64_t)ks.size() == n && (int64_t)vs.size() == n && (int64_t)ps.size() == n,
                    "need one q, k, v and position shard per rank");
  const at::Device dev = device_of({}, qs);
  on_device(dev, ks);
  on_device(dev, vs);
  on_device(dev, ps);
  std::vector<Tensor> pl;
  for (const Tensor& p : ps) pl.push_back(as_i64(p));
  int64_t S = 0;
  for (const Tensor& q : qs) S += q.size(1);
  const Tensor& q0 = qs[0];
  Tensor full = at::empty({q0.size(0), S, q_count + 2 * kv_count, q0.size(3)}, q0.options());
  Tensor pos_f = at::empty({q0.size(0), S}, q0.options().dtype(at::kLong));
  c10::DeviceGuard guard(dev);
  std::vector<cea_tensor> qa = args(qs), ka = args(ks), va = args(vs), pa = args(pl);
  cea_tensor f = arg(full), pf = arg(pos_f);
  check_rc(cea_ulysses_scatter((int32_t)n, qa.data(), ka.data(), va.data(), pa.data(), (int32_t)q_start,
                               (int32_t)q_count, (int32_t)kv_start, (int32_t)kv_count, &f, &pf, stream_of(dev)),
           "ulysses_scatter");
  return {full, pos_f};
}

Tensor ulysses_gather(at::TensorList outs, int64_t start, int64_t length) {
  TORCH_CHECK_VALUE(!outs.empty(), "need one head output per rank");
  const at::Device dev = device_of({}, outs);
  const Tensor& o0 = outs[0];
  int64_t H = 0;
  for (const Tensor& o : outs) H += o.size(2);
  Tensor res = at::empty({o0.size(0), length, H, o0.size(3)}, o0.options());
  c10::DeviceGuard guard(dev);
  std::vector<cea_tensor> oa = args(outs);
  cea_tensor r = arg(res);
  check_rc(cea_ulysses_gather((int32_t)outs.size(), oa.data(), start, &r, stream_of(dev)), "ulysses_gather");
  return res;
}

// ---------------------------------------------------------------------------------------
// layer ops
// ---------------------------------------------------------------------------------------
Tensor rmsnorm(const Tensor& x, const Tensor& weight_in, double eps) {
  const at::Device dev = device_of({&x, &weight_in});
  const Tensor w = inner(weight_in);
  Tensor y = at::empty(x.sizes(), x.options().dtype(at::promote_types(w.scalar_type(), x.scalar_type())));
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(x), b = arg(w), c = arg(y);
  check_rc(cea_rmsnorm(&a, &b, eps, &c, stream_of(dev)), "rmsnorm");
  return y;
}

std::vector<Tensor> rope_tables(const Tensor& pos_in, const Tensor& inv, at::ScalarType dtype) {
  const at::Device dev = device_of({&pos_in, &inv});
  const Tensor pos = as_i64(pos_in);
  TORCH_CHECK_VALUE(pos.dim() == 2 && inv.dim() == 1, "positions must be [B, S] and inv_freq [D/2]");
  const auto opts = inv.options().dtype(dtype);
  Tensor cos = at::empty({pos.size(0), pos.size(1), 2 * inv.size(0)}, opts);
  Tensor sin = at::empty({pos.size(0), pos.size(1), 2 * inv.size(0)}, opts);
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(pos), b = arg(inv), c = arg(cos), d = arg(sin);
  check_rc(cea_rope_tables(&a, &b, &c, &d, stream_of(dev)), "rope_tables");
  return {cos, sin};
}

Tensor apply_rotary(const Tensor& x_in, const Tensor& cos_in, const Tensor& sin_in) {
  const at::Device dev = device_of({&x_in, &cos_in, &sin_in});
  const Tensor x = inner(x_in), cos = inner(cos_in), sin = inner(sin_in);
  Tensor out = at::empty(x.sizes(), x.options());
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(x), b = arg(cos), c = arg(sin), d = arg(out);
  check_rc(cea_apply_rotary(&a, &b, &c, &d, stream_of(dev)), "apply_rotary");
  return out;
}

Tensor rmsnorm_rope(const Tensor& x, const Tensor& weight, double eps, const Tensor& pos_in, const Tensor& inv,
                    int64_t num_heads) {
  const at::Device dev = device_of({&x, &weight, &pos_in, &inv});
  const Tensor pos = as_i64(pos_in);
  Tensor out = at::empty(x.sizes(), x.options());
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(x), b = arg(weight), c = arg(pos), d = arg(inv), e = arg(out);
  check_rc(cea_rmsnorm_rope(&a, &b, eps, &c, &d, (int32_t)num_heads, &e, stream_of(dev)), "rmsnorm_rope");
  return out;
}

Tensor gated_mul(const Tensor& gate, const Tensor& up, int64_t act) {
  const at::Device dev = device_of({&gate, &up});
  Tensor out = at::empty(gate.sizes(), gate.options());
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(gate), b = arg(up), c = arg(out);
  check_rc(cea_gated_mul(&a, &b, &c, (int32_t)act, stream_of(dev)), "gated_mul");
  return out;
}

// x [..., K] as a 2-D [M, K] view (a copy only when the leading dimensions do not collapse)
Tensor rows_of(const Tensor& x) {
  TORCH_CHECK_VALUE(x.dim() >= 1, "x must have at least one dimension");
  int64_t rows = 1;
  for (int64_t i = 0; i + 1 < x.dim(); ++i) rows *= x.size(i);
  return inner(x.reshape({rows, x.size(-1)}));
}

std::vector<int64_t> out_shape(const Tensor& x, int64_t n) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end());
  s.back() = n;
  return s;
}

void linear_call(const Tensor& x2, const Tensor& weight, const c10::optional<Tensor>& bias,
                 const Tensor& y2, const at::Device& dev) {
  const Tensor w = inner(weight);
  const Tensor b = bias ? inner(*bias) : Tensor();
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(x2), c = arg(w), e = arg(y2);
  if (b.defined()) {
    cea_tensor d = arg(b);
    check_rc(cea_linear(&a, &c, &d, &e, stream_of(dev)), "linear");
  } else {
    check_rc(cea_linear(&a, &c, nullptr, &e, stream_of(dev)), "linear");
  }
}

Tensor linear(const Tensor& x, const Tensor& weight, const c10::optional<Tensor>& bias) {
  const Tensor bd = bias ? *bias : Tensor();
  const at::Device dev = device_of({&x, &weight, &bd});
  TORCH_CHECK_VALUE(weight.dim() == 2, "weight must be [out_features, in_features]");
  const Tensor x2 = rows_of(x);
  Tensor y = at::empty(out_shape(x, weight.size(0)), x.options());
  linear_call(x2, weight, bias, y.view({x2.size(0), weight.size(0)}), dev);
  return y;
}

// y: a preallocated [M, N] buffer (any row stride, innermost stride 1)
void linear_into(Tensor y, const Tensor& x, const Tensor& weight, const c10::optional<Tensor>& bias) {
  const Tensor bd = bias ? *bias : Tensor();
  const at::Device dev = device_of({&y, &x, &weight, &bd});
  TORCH_CHECK_VALUE(weight.dim() == 2, "weight must be [out_features, in_features]");
  TORCH_CHECK_VALUE(y.dim() == 2, "out must be 2-D [rows, out_features]");
  TORCH_CHECK_VALUE(y.size(-1) <= 1 || y.stride(-1) == 1, "out must have innermost stride 1");
  linear_call(rows_of(x), weight, bias, y, dev);
}

Tensor linear_gated(const Tensor& x, const Tensor& w_gate, const Tensor& w_up,
                    const c10::optional<Tensor>& b_gate, const c10::optional<Tensor>& b_up, int64_t act) {
  const Tensor bg = b_gate ? inner(*b_gate) : Tensor(), bu = b_up ? inner(*b_up) : Tensor();
  const at::Device dev = device_of({&x, &w_gate, &w_up, &bg, &bu});
  TORCH_CHECK_VALUE(w_gate.dim() == 2 && w_up.dim() == 2, "weights must be [units, in_features]");
  const Tensor x2 = rows_of(x);
  Tensor wg = inner(w_gate), wu = inner(w_up);
  if (wg.size(0) > 1 && wu.stride(0) != wg.stride(0)) {
    wg = wg.contiguous();
    wu = wu.contiguous();
  }
  Tensor y = at::empty(out_shape(x, w_gate.size(0)), x.options());
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(x2), c = arg(wg), d = arg(wu), e = arg(y.view({x2.size(0), w_gate.size(0)}));
  cea_tensor f, g;
  if (bg.defined()) f = arg(bg);
  if (bu.defined()) g = arg(bu);
  check_rc(cea_linear_gated(&a, &c, &d, bg.defined() ? &f : nullptr, bu.defined() ? &g : nullptr, &e,
                            (int32_t)act, stream_of(dev)),
           "linear_gated");
  return y;
}

void kv_append(Tensor cache_k, Tensor cache_v, Tensor cache_pos, int64_t offset, const Tensor& k_in,
               const Tensor& v_in, const Tensor& pos_in, c10::optional<Tensor> cos_in,
               c10::optional<Tensor> sin_in) {
  TORCH_CHECK_VALUE(cos_in.has_value() == sin_in.has_value(), "give both rotary tables or neither");
  const Tensor cosd = cos_in ? *cos_in : Tensor(), sind = sin_in ? *sin_in : Tensor();
  const at::Device dev = device_of({&cache_k, &cache_v, &cache_pos, &k_in, &v_in, &pos_in, &cosd, &sind});
  const Tensor k = inner(k_in), v = inner(v_in), pos = as_i64(pos_in);
  c10::DeviceGuard guard(dev);
  cea_tensor a = arg(k), b = arg(v), c = arg(pos), ck = arg(cache_k), cv = arg(cache_v), cp = arg(cache_pos);
  if (cosd.defined()) {
    const Tensor cs = inner(cosd.to(k.scalar_type())), sn = inner(sind.to(k.scalar_type()));
    cea_tensor tc = arg(cs), ts = arg(sn);
    check_rc(cea_kv_append(&a, &b, &c, &tc, &ts, &ck, &cv, &cp, offset, stream_of(dev)), "kv_append");
  } else {
    check_rc(cea_kv_append(&a, &b, &c, nullptr, nullptr, &ck, &cv, &cp, offset, stream_of(dev)), "kv_append");
  }
}

}  // namespace

TORCH_LIBRARY(collab_edge, m) {
  m.def("attention(Tensor q, Tensor k, Tensor v, Tensor q_pos, Tensor k_pos, bool causal, float scale, "
        "int[]? kv_map, bool with_lse) -> Tensor[]");
  m.def("attention_into(Tensor(a!) out, Tensor(b!) lse, Tensor q, Tensor k, Tensor v, Tensor q_pos, "
        "Tensor k_pos, bool causal, float scale, int[]? kv_map, bool accumulate, Tensor(c!)? final) -> ()");
  m.def("merge(Tensor[] outs, Tensor[] lses, bool pairwise, ScalarType? out_dtype) -> Tensor[]");
  m.def("partitioned(Tensor q, Tensor q_pos, Tensor[] ks, Tensor[] vs, Tensor[] ps, bool causal, "
        "float scale, int[]? kv_map, ScalarType out_dtype, bool with_lse, bool with_parts) -> Tensor[]");
  m.def("ring(Tensor q, Tensor q_pos, Tensor[] ks, Tensor[] vs, Tensor[] ps, bool causal, float scale, "
        "int[]? kv_map, bool with_lse) -> Tensor[]");
  m.def("pack_partial(Tensor out, Tensor lse, Tensor(a!) packed) -> ()");
  m.def("merge_packed(Tensor[] parts, ScalarType out_dtype, bool with_lse) -> Tensor[]");
  m.def("ulysses_scatter(Tensor[] qs, Tensor[] ks, Tensor[] vs, Tensor[] ps, int q_start, int q_count, "
        "int kv_start, int kv_count) -> Tensor[]");
  m.def("ulysses_gather(Tensor[] outs, int start, int length) -> Tensor");
  m.def("rmsnorm(Tensor x, Tensor weight, float eps) -> Tensor");
  m.def("rope_tables(Tensor positions, Tensor inv_freq, ScalarType dtype) -> Tensor[]");
  m.def("apply_rotary(Tensor x, Tensor cos, Tensor sin) -> Tensor");
  m.def("rmsnorm_rope(Tensor x, Tensor weight, float eps, Tensor positions, Tensor inv_freq, int num_heads) "
        "-> Tensor");
  m.def("gated_mul(Tensor gate, Tensor up, int act) -> Tensor");
  m.def("linear(Tensor x, Tensor weight, Tensor? bias) -> Tensor");
  m.def("linear_into(Tensor(a!) out, Tensor x, Tensor weight, Tensor? bias) -> ()");
  m.def("linear_gated(Tensor x, Tensor w_gate, Tensor w_up, Tensor? b_gate, Tensor? b_up, int act) -> Tensor");
  m.def("kv_append(Tensor(a!) cache_k, Tensor(b!) cache_v, Tensor(c!) cache_pos, int offset, Tensor k, "
        "Tensor v, Tensor pos, Tensor? cos, Tensor? sin) -> ()");
}

TORCH_LIBRARY_IMPL(collab_edge, CompositeExplicitAutograd, m) {
  m.impl("attention", attention);
  m.impl("attention_into", attention_into);
  m.impl("merge", merge);
  m.impl("partitioned", partitioned);
  m.impl("ring", ring);
  m.impl("pack_partial", pack_partial);
  m.impl("merge_packed", merge_packed);
  m.impl("ulysses_scatter", ulysses_scatter);
  m.impl("ulysses_gather", ulysses_gather);
  m.impl("rmsnorm", rmsnorm);
  m.impl("rope_tables", rope_tables);
  m.impl("apply_rotary", apply_rotary);
  m.impl("rmsnorm_rope", rmsnorm_rope);
  m.impl("gated_mul", gated_mul);
  m.impl("linear", linear);
  m.impl("linear_into", linear_into);
  m.impl("linear_gated", linear_gated);
  m.impl("kv_append", kv_append);
}
