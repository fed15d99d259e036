// torch.ops.nsg.*: the verify-step kernels of libnsg_spec.so as PyTorch
// operators, registered from C++ (TORCH_LIBRARY) over the library's C ABI.
//
// The reference reaches this path through Python: FlashInfer's
// BatchPrefillWithPagedKVCacheWrapper.plan / .run
// (nano_sglang/engine/engine.py:451-462, nano_sglang/model/causal_lm.py:340),
// the KV index_put (causal_lm.py:335-338), and the per-position loop of
// SpeculativeDecoder.speculative_step (nano_sglang/decode/speculative.py:130-196)
// with sample_token (nano_sglang/engine/sampling.py:25-50).  Each operator here
// checks its arguments, allocates its outputs through PyTorch's caching
// allocator, and enqueues the HIP kernels on the current HIP stream of the
// inputs' device; nothing synchronises the host except the host-side planner.
//
//   nsg::verify_attention       plan + run in one call (plans on the host)
//   nsg::verify_attention_plan  the host planner: plan record + work list
//   nsg::verify_attention_run   one layer from a plan; allocates nothing
//   nsg::spec_accept            acceptance / residual / bonus / rollback slots
//   nsg::spec_accept_check_flags  its device error flags for the current stream
//   nsg::sample                 temperature / top-k / top-p, one token per row
//   nsg::kv_write, nsg::rope_kv_write
//                               K / V rows (after RoPE) into flat KV slots
//
// Host (CPU) tensors given to a device operator are rejected with an error;
// there is no CPU implementation.  Shape-only (fake) implementations are
// registered from Python (nanosglang_amd/ops.py).
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "../../include/nsg_spec.h"

namespace {

using at::Tensor;
using c10::optional;

constexpr int64_t kPlanInts = sizeof(nsg_attn_plan_t) / 4;
constexpr int64_t kRecordInts = kPlanInts + 3;   // + query rows, page ids, batch
constexpr int64_t kMi355xCus = 256;

void check_status(int32_t rc, const char* what) {
  TORCH_CHECK(rc == NSG_OK, what, " failed (status ", rc, "): ", nsg_last_error());
}

void require_gpu(const Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor (no CPU path exists)");
}

void require(const Tensor& t, const char* name, at::ScalarType dtype) {
  require_gpu(t, name);
  TORCH_CHECK_VALUE(t.scalar_type() == dtype && t.is_contiguous(), name, " must be contiguous ",
                    c10::toString(dtype));
}

// PyTorch-ROCm presents HIP devices and streams as "cuda" ones.
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

void* stream_of(const Tensor& t) {
  return static_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

template <typename T>
const T* ptr_or_null(const optional<Tensor>& t) {
  return t.has_value() ? static_cast<const T*>(t->data_ptr()) : nullptr;
}

// Host int32 copy of an index tensor (any device).
Tensor host_i32(const Tensor& t) { return t.to(at::kCPU, at::kInt).contiguous(); }

// ---- plan records ----

Tensor make_record(const nsg_attn_plan_t& pl, int64_t total_q, int64_t nnz, int64_t batch) {
  Tensor r = at::empty({kRecordInts}, at::TensorOptions().dtype(at::kInt));
  int32_t* p = r.data_ptr<int32_t>();
  std::memcpy(p, &pl, sizeof(pl));
  p[kPlanInts] = static_cast<int32_t>(total_q);
  p[kPlanInts + 1] = static_cast<int32_t>(nnz);
  p[kPlanInts + 2] = static_cast<int32_t>(batch);
  return r;
}

void read_record(const Tensor& rec, nsg_attn_plan_t* pl, int64_t* total_q, int64_t* nnz,
                 int64_t* batch) {
  TORCH_CHECK_VALUE(!rec.is_cuda() && rec.scalar_type() == at::kInt && rec.numel() == kRecordInts,
                    "plan record must be a host int32 tensor of ", kRecordInts);
  const Tensor r = rec.contiguous();
  const int32_t* p = r.data_ptr<int32_t>();
  std::memcpy(pl, p, sizeof(*pl));
  *total_q = p[kPlanInts];
  *nnz = p[kPlanInts + 1];
  *batch = p[kPlanInts + 2];
}

// Upper bound on the work (plus merge) items of a dynamic plan: every query
// tile split into every 32-token KV step, plus one merge item (tiles of the
// smallest size a plan takes: 16 rows when the GQA group is 16 or less).
int64_t work_bound(const int32_t* qo, const int32_t* kvp, const int32_t* last, int64_t B,
                   int64_t Hq, int64_t Hkv, int64_t P) {
  const int64_t G = std::max<int64_t>(1, Hq / std::max<int64_t>(1, Hkv));
  int64_t maxq = 1;
  for (int64_t b = 0; b < B; ++b) maxq = std::max<int64_t>(maxq, qo[b + 1] - qo[b]);
  const int64_t T = std::max<int64_t>(1, std::min<int64_t>((G <= 16 ? 16 : 64) / G, maxq));
  int64_t bound = 0;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t ql = qo[b + 1] - qo[b], npg = kvp[b + 1] - kvp[b];
    const int64_t L = npg ? (npg - 1) * P + last[b] : 0;
    bound += (ql + T - 1) / T * (1 + std::max<int64_t>(1, (L + 31) / 32));
  }
  return std::max<int64_t>(1, bound);
}

std::tuple<Tensor, Tensor> verify_attention_plan(const Tensor& qo_indptr,
                                                 const Tensor& paged_kv_indptr,
                                                 const Tensor& paged_kv_last_page_len,
                                                 int64_t num_qo_heads, int64_t num_kv_heads,
                                                 int64_t head_dim, int64_t page_size,
                                                 bool causal, int64_t num_cus) {
  const Tensor qo = host_i32(qo_indptr), kvp = host_i32(paged_kv_indptr),
               last = host_i32(paged_kv_last_page_len);
  const int64_t B = qo.numel() - 1;
  TORCH_CHECK_VALUE(B >= 0 && kvp.numel() == B + 1 && last.numel() == B,
                    "qo_indptr, paged_kv_indptr and last_page_len disagree on batch");
  const int64_t cap = work_bound(qo.data_ptr<int32_t>(), kvp.data_ptr<int32_t>(),
                                 last.data_ptr<int32_t>(), B, num_qo_heads, num_kv_heads,
                                 page_size);
  Tensor work = at::zeros({cap * NSG_ATTN_WORK_INTS}, at::TensorOptions().dtype(at::kInt));
  nsg_attn_plan_t pl{};
  check_status(nsg_attn_plan(qo.data_ptr<int32_t>(), kvp.data_ptr<int32_t>(),
                             last.data_ptr<int32_t>(), static_cast<int32_t>(B),
                             static_cast<int32_t>(num_qo_heads),
                             static_cast<int32_t>(num_kv_heads), static_cast<int32_t>(head_dim),
                             static_cast<int32_t>(page_size), causal ? 1 : 0,
                             static_cast<int32_t>(num_cus), work.data_ptr<int32_t>(),
                             static_cast<int32_t>(cap), &pl),
               "nsg_attn_plan");
  const int64_t n = static_cast<int64_t>(pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS;
  return {make_record(pl, qo.data_ptr<int32_t>()[B], kvp.data_ptr<int32_t>()[B], B),
          work.narrow(0, 0, n).clone()};
}

void verify_attention_run(const Tensor& plan, const Tensor& work, const Tensor& q,
                          const Tensor& k_cache, const Tensor& v_cache, const Tensor& qo_indptr,
                          const Tensor& paged_kv_indptr, const Tensor& paged_kv_indices,
                          const Tensor& paged_kv_last_page_len, double sm_scale, bool causal,
                          const Tensor& workspace, const Tensor& out) {
  for (const auto& [t, name] : {std::pair<const Tensor&, const char*>{q, "q"},
                                {k_cache, "k_cache"}, {v_cache, "v_cache"}, {out, "out"}})
    require(t, name, at::kBFloat16);
  for (const auto& [t, name] : {std::pair<const Tensor&, const char*>{work, "work"},
                                {qo_indptr, "qo_indptr"}, {paged_kv_indptr, "paged_kv_indptr"},
                                {paged_kv_indices, "paged_kv_indices"},
                                {paged_kv_last_page_len, "paged_kv_last_page_len"}})
    require(t, name, at::kInt);
  require_gpu(workspace, "workspace");
  nsg_attn_plan_t pl;
  int64_t total_q, nnz, B;
  read_record(plan, &pl, &total_q, &nnz, &B);
  TORCH_CHECK_VALUE(q.dim() == 3 && q.size(0) == total_q && q.size(1) == pl.num_qo_heads &&
                        q.size(2) == pl.head_dim && out.sizes() == q.sizes(),
                    "q / out must be (", total_q, ", ", pl.num_qo_heads, ", ", pl.head_dim,
                    ") as planned");
  TORCH_CHECK_VALUE(qo_indptr.numel() == B + 1 && paged_kv_indptr.numel() == B + 1 &&
                        paged_kv_last_page_len.numel() == B && paged_kv_indices.numel() >= nnz,
                    "CSR arrays do not match the planned batch ", B, " / ", nnz, " page ids");
  TORCH_CHECK_VALUE(k_cache.dim() == 4 && k_cache.size(2) == pl.num_kv_heads &&
                        k_cache.size(3) == pl.head_dim && v_cache.sizes() == k_cache.sizes(),
                    "caches must be (pages, P, ", pl.num_kv_heads, ", ", pl.head_dim, ")");
  TORCH_CHECK_VALUE(work.numel() >= static_cast<int64_t>(pl.num_work + pl.num_merge) *
                                         NSG_ATTN_WORK_INTS,
                    "work list shorter than the plan");
  const int64_t wsb = workspace.numel() * workspace.element_size();
  TORCH_CHECK_VALUE(wsb >= pl.workspace_bytes, "workspace has ", wsb,
                    " bytes, the plan needs ", pl.workspace_bytes);
  const DeviceGuard guard(q.device());
  check_status(nsg_attn_run(&pl, work.data_ptr<int32_t>(), q.data_ptr(), k_cache.data_ptr(),
                            v_cache.data_ptr(), out.data_ptr(), qo_indptr.data_ptr<int32_t>(),
                            paged_kv_indptr.data_ptr<int32_t>(),
                            paged_kv_indices.data_ptr<int32_t>(),
                            paged_kv_last_page_len.data_ptr<int32_t>(),
                            static_cast<int32_t>(k_cache.size(1)),
                            static_cast<int32_t>(k_cache.size(0)), static_cast<float>(sm_scale),
                            causal ? 1 : 0, workspace.data_ptr(), wsb, stream_of(q)),
               "nsg_attn_run");
}

// ---- per-(device, stream) workspaces ----
//
// The reference's 128 MiB attention workspace (engine.py:103-108) for the
// one-call attention operator, and the acceptance and sampling workspaces
// (one of each per stream: calls on one stream run in order, so they may
// share it; each kind keeps its own, the acceptance one being zero between
// calls).  All are zero-filled when created.
//
// A HIP graph captured while a workspace was current keeps its address, so
// a workspace replaced by a larger one stays allocated (in `retired`) for
// the life of the process, and none is created or grown while its stream is
// being captured (the caller makes one eager call of its largest shape on
// that stream first): an allocation there would come from the graph's
// private pool.

struct Workspace {
  Tensor cur;
  std::vector<Tensor> retired;
};

std::mutex g_ws_mu;
std::map<std::tuple<int, void*, int>, Workspace> g_ws;

const char* const kWsNames[] = {"attention", "acceptance", "sampling"};

Tensor workspace(const at::Device& dev, void* stream, int kind, int64_t bytes) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  Workspace& w = g_ws[{dev.index(), stream, kind}];
  if (!w.cur.defined() || w.cur.numel() < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs);
    TORCH_CHECK(e == hipSuccess, "hipStreamIsCapturing failed: ", hipGetErrorString(e));
    TORCH_CHECK(cs == hipStreamCaptureStatusNone, "the ", kWsNames[kind],
                " workspace of this stream needs ", bytes, " bytes (has ",
                w.cur.defined() ? w.cur.numel() : 0,
                ") while the stream is being captured; make one eager call of the largest "
                "shape on this stream before capturing");
    const int64_t n = w.cur.defined() ? std::max(bytes, 2 * w.cur.numel()) : bytes;
    if (w.cur.defined()) w.retired.push_back(w.cur);
    w.cur = at::zeros({n}, at::TensorOptions().dtype(at::kByte).device(dev));
  }
  return w.cur;
}

enum { kAttnWs = 0, kAcceptWs = 1, kSampleWs = 2 };

Tensor verify_attention(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache,
                        const Tensor& qo_indptr, const Tensor& paged_kv_indptr,
                        const Tensor& paged_kv_indices, const Tensor& paged_kv_last_page_len,
                        bool causal, optional<double> sm_scale) {
  require(q, "q", at::kBFloat16);
  require(k_cache, "k_cache", at::kBFloat16);
  require(v_cache, "v_cache", at::kBFloat16);
  TORCH_CHECK_VALUE(q.dim() == 3 && k_cache.dim() == 4, "q (T, Hq, D), caches (N, P, Hkv, D)");
  const int64_t D = q.size(2);
  auto [rec, work_h] = verify_attention_plan(qo_indptr, paged_kv_indptr, paged_kv_last_page_len,
                                             q.size(1), k_cache.size(2), D, k_cache.size(1),
                                             causal, kMi355xCus);
  nsg_attn_plan_t pl;
  int64_t total_q, nnz, B;
  read_record(rec, &pl, &total_q, &nnz, &B);
  const at::Device dev = q.device();
  const DeviceGuard guard(dev);
  void* s = stream_of(q);
  auto dev_i32 = [&](const Tensor& t) { return t.to(dev, at::kInt).contiguous(); };
  const Tensor work = work_h.to(dev), qo = dev_i32(qo_indptr), kvp = dev_i32(paged_kv_indptr),
               idx = dev_i32(paged_kv_indices), last = dev_i32(paged_kv_last_page_len);
  const Tensor ws = workspace(dev, s, kAttnWs, std::max<int64_t>(128 << 20, pl.workspace_bytes));
  Tensor out = at::empty_like(q);
  verify_attention_run(rec, work, q, k_cache, v_cache, qo, kvp, idx, last,
                       sm_scale.has_value() ? *sm_scale : 1.0 / std::sqrt(static_cast<double>(D)),
                       causal, ws, out);
  return out;
}

// ---- acceptance and sampling ----

std::tuple<Tensor, Tensor, Tensor> spec_accept(
    const Tensor& target_logits, const optional<Tensor>& draft_logits,
    const optional<Tensor>& draft_tokens, const optional<Tensor>& uniforms, double temperature,
    const optional<Tensor>& kv_indptr, const optional<Tensor>& kv_indices,
    const optional<Tensor>& start_pos, int64_t page_size, const optional<Tensor>& bonus_tokens) {
  require_gpu(target_logits, "target_logits");
  TORCH_CHECK_VALUE(target_logits.dim() == 3, "target_logits must be (B, k+1, V)");
  const at::ScalarType st = target_logits.scalar_type();
  TORCH_CHECK(st == at::kBFloat16 || st == at::kFloat, "logits dtype ", c10::toString(st),
              ": bf16 or fp32");
  TORCH_CHECK_VALUE(target_logits.stride(2) == 1,
                    "target_logits must be contiguous along the vocabulary");
  const int64_t B = target_logits.size(0), k = target_logits.size(1) - 1,
                V = target_logits.size(2);
  const bool greedy = temperature < 1e-6;
  const at::Device dev = target_logits.device();
  const DeviceGuard guard(dev);
  optional<Tensor> dl, dt, u, bonus, ip, ix, sp;
  int64_t d_req = 0, d_row = 0;
  if (!greedy && k > 0) {
    TORCH_CHECK_VALUE(draft_logits.has_value(), "draft_logits required when temperature > 0");
    require_gpu(*draft_logits, "draft_logits");
    TORCH_CHECK_VALUE(draft_logits->scalar_type() == st && draft_logits->dim() == 3 &&
                          draft_logits->size(0) == B && draft_logits->size(1) == k &&
                          draft_logits->size(2) == V && draft_logits->stride(2) == 1,
                      "draft_logits must match target_logits' dtype with shape (B, k, V)");
    dl = *draft_logits;
    d_req = dl->stride(0);
    d_row = dl->stride(1);
  }
  if (k > 0) {
    TORCH_CHECK_VALUE(draft_tokens.has_value() && draft_tokens->dim() == 2 &&
                          draft_tokens->size(0) == B && draft_tokens->size(1) == k,
                      "draft_tokens must be (B, k)");
    require_gpu(*draft_tokens, "draft_tokens");
    dt = draft_tokens->to(at::kLong).contiguous();
  }
  if (!greedy) {
    TORCH_CHECK_VALUE(uniforms.has_value() && uniforms->numel() == B * (k + 1),
                      "uniforms must be (B, k+1) float32");
    require_gpu(*uniforms, "uniforms");
    u = uniforms->to(at::kFloat).contiguous();
    if (bonus_tokens.has_value()) {
      require(*bonus_tokens, "bonus_tokens", at::kLong);
      TORCH_CHECK_VALUE(bonus_tokens->numel() == B, "bonus_tokens must be (B,)");
      bonus = *bonus_tokens;
    }
  }
  const bool rb = kv_indptr.has_value() && k > 0;
  if (rb) {
    TORCH_CHECK_VALUE(kv_indices.has_value() && start_pos.has_value(),
                      "kv_indices and start_pos required for rollback slots");
    require_gpu(*kv_indptr, "kv_indptr");
    require_gpu(*kv_indices, "kv_indices");
    require_gpu(*start_pos, "start_pos");
    ip = kv_indptr->to(at::kInt).contiguous();
    ix = kv_indices->to(at::kInt).contiguous();
    sp = start_pos->to(at::kInt).contiguous();
  }
  const auto opts = target_logits.options();
  Tensor n_out = at::empty({B}, opts.dtype(at::kInt));
  Tensor emitted = at::empty({B, k + 1}, opts.dtype(at::kLong));
  Tensor rollback = at::full({B, k}, -1, opts.dtype(at::kLong));
  void* s = stream_of(target_logits);
  const int64_t need = nsg_spec_accept_workspace_bytes(B, k, V);
  TORCH_CHECK(need >= 0, "nsg_spec_accept_workspace_bytes failed");
  const Tensor ws = workspace(dev, s, kAcceptWs, std::max<int64_t>(need, 1));
  check_status(
      nsg_spec_accept(target_logits.data_ptr(), target_logits.stride(0), target_logits.stride(1),
                      dl ? dl->data_ptr() : nullptr, d_req, d_row, st == at::kBFloat16 ? 0 : 1,
                      ptr_or_null<int64_t>(dt), ptr_or_null<float>(u),
                      ptr_or_null<int64_t>(bonus), static_cast<int32_t>(B),
                      static_cast<int32_t>(k), static_cast<int32_t>(V),
                      static_cast<float>(temperature), ptr_or_null<int32_t>(ip),
                      ptr_or_null<int32_t>(ix), ptr_or_null<int32_t>(sp),
                      static_cast<int32_t>(page_size), n_out.data_ptr<int32_t>(),
                      emitted.data_ptr<int64_t>(), rb ? rollback.data_ptr<int64_t>() : nullptr,
                      ws.data_ptr(), ws.numel(), s),
      "nsg_spec_accept");
  return {n_out, emitted, rollback};
}

// The error flags of nsg::spec_accept's workspace for the current stream of
// `device` (bits of nsg_spec_accept: 1 a rolled-back position past its pages,
// 2 a draft token outside the vocabulary, 3 a hand-off wait gave up), read
// and cleared; after bit 3 the whole workspace is zeroed again.  Synchronises
// the stream.  0 when the stream has no acceptance workspace yet.
int64_t spec_accept_check_flags(at::Device device) {
  TORCH_CHECK(device.is_cuda(), "spec_accept_check_flags: a GPU device is required");
  const at::Device dev(device.type(), device.has_index() ? device.index()
                                                          : c10::hip::current_device());
  const DeviceGuard guard(dev);
  void* s = static_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream());
  Tensor ws;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find({dev.index(), s, kAcceptWs});
    if (it == g_ws.end() || !it->second.cur.defined()) return 0;
    ws = it->second.cur;
  }
  int32_t flags = 0;
  check_status(nsg_spec_accept_check_flags(ws.data_ptr(), ws.numel(), &flags, s),
               "nsg_spec_accept_check_flags");
  return flags;
}

Tensor sample(const Tensor& logits, double temperature, int64_t top_k, double top_p,
              const optional<Tensor>& uniforms) {
  require_gpu(logits, "logits");
  TORCH_CHECK_VALUE(logits.dim() == 2, "logits must be (rows, V)");
  const at::ScalarType st = logits.scalar_type();
  TORCH_CHECK(st == at::kBFloat16 || st == at::kFloat, "logits dtype ", c10::toString(st),
              ": bf16 or fp32");
  const int64_t R = logits.size(0), V = logits.size(1);
  TORCH_CHECK_VALUE(R == 0 || logits.stride(1) == 1,
                    "logits must be contiguous along the vocabulary");
  const bool greedy = temperature < 1e-6;
  const at::Device dev = logits.device();
  const DeviceGuard guard(dev);
  optional<Tensor> u;
  if (!greedy) {
    TORCH_CHECK_VALUE(uniforms.has_value() && uniforms->numel() == R,
                      "uniforms (R,) float32 required when temperature > 0");
    require_gpu(*uniforms, "uniforms");
    u = uniforms->reshape({R}).to(at::kFloat).contiguous();
  }
  Tensor out = at::empty({R}, logits.options().dtype(at::kLong));
  void* s = stream_of(logits);
  const int64_t need = nsg_sample_workspace_bytes(R, V);
  TORCH_CHECK(need >= 0, "nsg_sample_workspace_bytes failed");
  const Tensor ws = workspace(dev, s, kSampleWs, std::max<int64_t>(need, 1));
  check_status(nsg_sample(logits.data_ptr(), R > 1 ? logits.stride(0) : V,
                          st == at::kBFloat16 ? 0 : 1, static_cast<int32_t>(R),
                          static_cast<int32_t>(V), static_cast<float>(temperature),
                          static_cast<int32_t>(top_k), static_cast<float>(top_p),
                          ptr_or_null<float>(u), 1, out.data_ptr<int64_t>(), ws.data_ptr(),
                          ws.numel(), s),
               "nsg_sample");
  return out;
}

// ---- KV writes ----

void kv_write(const Tensor& k, const Tensor& v, const Tensor& slots, const Tensor& k_cache,
              const Tensor& v_cache) {
  for (const auto& [t, name] : {std::pair<const Tensor&, const char*>{k, "k"}, {v, "v"},
                                {slots, "slots"}, {k_cache, "k_cache"}, {v_cache, "v_cache"}})
    require_gpu(t, name);
  TORCH_CHECK_VALUE(k.dim() == 3 && v.sizes() == k.sizes() && v.strides() == k.strides(),
                    "k and v must have the same (T, Hkv, D) shape and strides");
  const int64_t T = k.size(0), Hkv = k.size(1), D = k.size(2);
  TORCH_CHECK_VALUE(k.stride(2) == 1 && k.stride(1) == D,
                    "each K/V row must be a contiguous (Hkv, D) block");
  TORCH_CHECK(k.scalar_type() == at::kBFloat16 && k_cache.scalar_type() == at::kBFloat16,
              "K/V and caches must be bfloat16");
  TORCH_CHECK_VALUE(k_cache.is_contiguous() && v_cache.is_contiguous(), "caches must be contiguous");
  TORCH_CHECK_VALUE(k_cache.size(-2) == Hkv && k_cache.size(-1) == D,
                    "cache head layout does not match K/V");
  const DeviceGuard guard(k.device());
  const Tensor sl = slots.to(at::kLong).contiguous();
  check_status(nsg_kv_write(k.data_ptr(), v.data_ptr(), k.stride(0), sl.data_ptr<int64_t>(),
                            static_cast<int32_t>(T), k_cache.data_ptr(), v_cache.data_ptr(),
                            static_cast<int32_t>(Hkv), static_cast<int32_t>(D),
                            k_cache.numel() / (Hkv * D), stream_of(k)),
               "nsg_kv_write");
}

Tensor rope_kv_write(const Tensor& qkv, int64_t num_qo_heads, int64_t num_kv_heads,
                     int64_t head_dim, const Tensor& positions, const Tensor& cos_table,
                     const Tensor& sin_table, const Tensor& slots, const Tensor& k_cache,
                     const Tensor& v_cache) {
  for (const auto& [t, name] : {std::pair<const Tensor&, const char*>{qkv, "qkv"},
                                {positions, "positions"}, {cos_table, "cos_table"},
                                {sin_table, "sin_table"}, {slots, "slots"},
                                {k_cache, "k_cache"}, {v_cache, "v_cache"}})
    require_gpu(t, name);
  TORCH_CHECK_VALUE(qkv.scalar_type() == at::kBFloat16 && qkv.dim() == 2 && qkv.stride(1) == 1,
                    "qkv must be bfloat16 (T, (Hq + 2 Hkv) D) with unit inner stride");
  require(cos_table, "cos_table", at::kFloat);
  require(sin_table, "sin_table", at::kFloat);
  const int64_t T = qkv.size(0);
  const DeviceGuard guard(qkv.device());
  Tensor q_out = at::empty({T, num_qo_heads, head_dim}, qkv.options());
  const Tensor pos = positions.to(at::kLong).contiguous();
  const Tensor sl = slots.to(at::kLong).contiguous();
  check_status(nsg_rope_kv_write(qkv.data_ptr(), qkv.stride(0), pos.data_ptr<int64_t>(),
                                 cos_table.data_ptr<float>(), sin_table.data_ptr<float>(),
                                 static_cast<int32_t>(cos_table.size(0)),
                                 sl.data_ptr<int64_t>(), static_cast<int32_t>(T),
                                 static_cast<int32_t>(num_qo_heads),
                                 static_cast<int32_t>(num_kv_heads),
                                 static_cast<int32_t>(head_dim), q_out.data_ptr(),
                                 k_cache.data_ptr(), v_cache.data_ptr(),
                                 k_cache.numel() / (num_kv_heads * head_dim), nullptr,
                                 stream_of(qkv)),
               "nsg_rope_kv_write");
  return q_out;
}

// ---- host tensors given to the device operators ----

[[noreturn]] void host_tensors(const char* op) {
  TORCH_CHECK(false, "nsg::", op, ": inputs must be GPU tensors (no CPU path exists)");
}

}  // namespace

TORCH_LIBRARY(nsg, m) {
  m.def(
      "verify_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor qo_indptr, "
      "Tensor paged_kv_indptr, Tensor paged_kv_indices, Tensor paged_kv_last_page_len, "
      "bool causal=True, float? sm_scale=None) -> Tensor");
  m.def(
      "verify_attention_plan(Tensor qo_indptr, Tensor paged_kv_indptr, "
      "Tensor paged_kv_last_page_len, int num_qo_heads, int num_kv_heads, int head_dim, "
      "int page_size, bool causal=True, int num_cus=256) -> (Tensor, Tensor)");
  m.def(
      "verify_attention_run(Tensor plan, Tensor work, Tensor q, Tensor k_cache, "
      "Tensor v_cache, Tensor qo_indptr, Tensor paged_kv_indptr, Tensor paged_kv_indices, "
      "Tensor paged_kv_last_page_len, float sm_scale, bool causal, Tensor(a!) workspace, "
      "Tensor(b!) out) -> ()");
  m.def(
      "spec_accept(Tensor target_logits, Tensor? draft_logits, Tensor? draft_tokens, "
      "Tensor? uniforms, float temperature, Tensor? kv_indptr=None, Tensor? kv_indices=None, "
      "Tensor? start_pos=None, int page_size=16, Tensor? bonus_tokens=None) "
      "-> (Tensor, Tensor, Tensor)");
  m.def("spec_accept_check_flags(Device device) -> int", &spec_accept_check_flags);
  m.def(
      "sample(Tensor logits, float temperature, int top_k=0, float top_p=1.0, "
      "Tensor? uniforms=None) -> Tensor");
  m.def("kv_write(Tensor k, Tensor v, Tensor slots, Tensor(a!) k_cache, Tensor(b!) v_cache) -> ()");
  m.def(
      "rope_kv_write(Tensor qkv, int num_qo_heads, int num_kv_heads, int head_dim, "
      "Tensor positions, Tensor cos_table, Tensor sin_table, Tensor slots, "
      "Tensor(a!) k_cache, Tensor(b!) v_cache) -> Tensor");
}

TORCH_LIBRARY_IMPL(nsg, CUDA, m) {
  m.impl("verify_attention", &verify_attention);
  m.impl("verify_attention_plan", &verify_attention_plan);
  m.impl("verify_attention_run", &verify_attention_run);
  m.impl("spec_accept", &spec_accept);
  m.impl("sample", &sample);
  m.impl("kv_write", &kv_write);
  m.impl("rope_kv_write", &rope_kv_write);
}

TORCH_LIBRARY_IMPL(nsg, CPU, m) {
  m.impl("verify_attention_plan", &verify_attention_plan);   // the host planner
  m.impl("verify_attention", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                const Tensor&, const Tensor&, const Tensor&, bool,
                                optional<double>) -> Tensor { host_tensors("verify_attention"); });
  m.impl("verify_attention_run",
         [](const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const Tensor&, const Tensor&, double, bool,
            const Tensor&, const Tensor&) { host_tensors("verify_attention_run"); });
  m.impl("spec_accept",
         [](const Tensor&, const optional<Tensor>&, const optional<Tensor>&,
            const optional<Tensor>&, double, const optional<Tensor>&, const optional<Tensor>&,
            const optional<Tensor>&, int64_t,
            const optional<Tensor>&) -> std::tuple<Tensor, Tensor, Tensor> {
           host_tensors("spec_accept");
         });
  m.impl("sample", [](const Tensor&, double, int64_t, double, const optional<Tensor>&) -> Tensor {
    host_tensors("sample");
  });
  m.impl("kv_write", [](const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                        const Tensor&) { host_tensors("kv_write"); });
  m.impl("rope_kv_write",
         [](const Tensor&, int64_t, int64_t, int64_t, const Tensor&, const Tensor&, const Tensor&,
            const Tensor&, const Tensor&, const Tensor&) -> Tensor {
           host_tensors("rope_kv_write");
         });
}
