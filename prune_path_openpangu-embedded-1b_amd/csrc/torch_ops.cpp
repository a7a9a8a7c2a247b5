// torch.library registration of the PrunePath ops (namespace `prunepath`) over the C ABI
// of libprunepath_moe.so (include/prunepath_moe.h). Host code only: the kernels live
// in the HIP library; this file checks arguments, allocates outputs with the caching
// allocator, passes the current HIP stream and turns a failed call into a RuntimeError
// (TORCH_CHECK). Each op also has a Meta implementation (shapes only) for fake-tensor
// tracing. There is no CPU implementation: CPU tensors are refused.
//
// Ops and the reference interfaces they stand for (paths relative to the reference
// repository root):
//   route, route_logits   softmax_thresholding (src/MoEBlock_origin.py:50-97); the
//                         prefill router / sort / select / scatter
//                         (src/tl_kernel_optimized_Ultimate_PanGU.py:40-124, 550-564)
//   bucket                moe_local_scan / moe_global_scan / moe_dispatch (:133-266)
//   pack_experts,
//   pack_router           physical_reorder_for_inference (src/openpangu_moe.py:212-256)
//   moe_decode(_into)     TauSparseMoE.forward_decode (:494-530)
//   moe_decode_batch(_into)  TauSparseMoE.forward_prefill (:532-604) for 1 <= N <= 64
//                         tokens (the reference takes it for every N > 1, :606-615)
//   moe_prefill(_into)    TauSparseMoE.forward_prefill (:532-604)
//   masked_gate(_bwd)     MoELayer.forward's expert gating and its backward
//                         (src/MoEBlock_origin.py:205-212)
#include <ATen/ATen.h>
#include <algorithm>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/core/stack.h>
#include <torch/library.h>

#include "../../include/prunepath_moe.h"

namespace {

using at::Tensor;
using c10::optional;

void* stream_of(const Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == PP_OK, "prunepath.", what, " failed (code ", rc, "): ", pp_last_error());
}

void need_gpu(const char* name, const Tensor& ref, std::initializer_list<const Tensor*> ts) {
  for (const Tensor* t : ts) {
    if (t == nullptr || !t->defined()) continue;
    TORCH_CHECK(t->is_cuda(), "prunepath.", name, ": tensors must be on the GPU (got ", t->device(),
                "); there is no CPU implementation");
    TORCH_CHECK(t->is_contiguous(), "prunepath.", name, ": tensors must be contiguous");
    TORCH_CHECK(t->device() == ref.device(), "prunepath.", name, ": tensors on different devices (",
                ref.device(), ", ", t->device(), ")");
  }
}

const void* ptr(const optional<Tensor>& t) { return (t.has_value() && t->defined()) ? t->data_ptr() : nullptr; }

int x_code(const Tensor& x, const char* name) {
  if (x.scalar_type() == at::kBFloat16) return PP_DTYPE_BF16;
  TORCH_CHECK(x.scalar_type() == at::kFloat, "prunepath.", name, ": x must be float32 or bfloat16 (got ",
              x.scalar_type(), ")");
  return PP_DTYPE_F32;
}

int w_code(const Tensor& w, const char* name) {
  if (w.scalar_type() == at::kBFloat16) return PP_DTYPE_BF16;
  TORCH_CHECK(w.scalar_type() == at::kFloat, "prunepath.", name, ": weights must be float32 or bfloat16 (got ",
              w.scalar_type(), ")");
  return PP_DTYPE_F32;
}

void check_bias(const optional<Tensor>& bias, int64_t E, const char* name) {
  if (!bias.has_value()) return;
  TORCH_CHECK(bias->scalar_type() == at::kFloat && bias->numel() == E, "prunepath.", name,
              ": bias must be float32 [E]");
}

// ------------------------------------------------------------------ routing
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> route_gpu(const Tensor& x, const Tensor& router_packed,
                                                             const optional<Tensor>& bias, int64_t E,
                                                             double tau) {
  TORCH_CHECK(x.dim() == 2, "prunepath.route: x must be [N, H]");
  check_bias(bias, E, "route");
  need_gpu("route", x, {&x, &router_packed, bias.has_value() ? &*bias : nullptr});
  const c10::DeviceGuard g(x.device());
  const int64_t N = x.size(0), H = x.size(1);
  auto f = x.options().dtype(at::kFloat);
  Tensor logits = at::empty({N, E}, f), probs = at::empty({N, E}, f), gates = at::empty({N, E}, f);
  Tensor mask = at::empty({N, E}, x.options().dtype(at::kByte));
  Tensor count = at::empty({N}, x.options().dtype(at::kInt));
  check_rc(pp_route(x.data_ptr(), x_code(x, "route"), N, (int)H, router_packed.data_ptr<float>(),
                    (const float*)ptr(bias), (int)E, (float)tau, logits.data_ptr<float>(), probs.data_ptr<float>(),
                    gates.data_ptr<float>(), mask.data_ptr<uint8_t>(), count.data_ptr<int32_t>(), stream_of(x)),
           "route");
  return {logits, probs, gates, mask, count};
}

// Meta implementations use symbolic sizes (c10::SymInt), so the ops trace with dynamic shapes.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> route_meta(const Tensor& x, const Tensor&,
                                                              const optional<Tensor>&, int64_t E, double) {
  const c10::SymInt N = x.sym_size(0);
  auto f = x.options().dtype(at::kFloat);
  return {at::empty_symint({N, E}, f), at::empty_symint({N, E}, f), at::empty_symint({N, E}, f),
          at::empty_symint({N, E}, x.options().dtype(at::kByte)), at::empty_symint({N}, x.options().dtype(at::kInt))};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> route_logits_gpu(const Tensor& logits, double tau) {
  TORCH_CHECK(logits.scalar_type() == at::kFloat && logits.dim() == 2,
              "prunepath.route_logits: logits must be float32 [N, E]");
  need_gpu("route_logits", logits, {&logits});
  const c10::DeviceGuard g(logits.device());
  const int64_t N = logits.size(0), E = logits.size(1);
  Tensor probs = at::empty_like(logits), gates = at::empty_like(logits);
  Tensor mask = at::empty({N, E}, logits.options().dtype(at::kByte));
  Tensor count = at::empty({N}, logits.options().dtype(at::kInt));
  check_rc(pp_route_logits(logits.data_ptr<float>(), N, (int)E, (float)tau, probs.data_ptr<float>(),
                           gates.data_ptr<float>(), mask.data_ptr<uint8_t>(), count.data_ptr<int32_t>(),
                           stream_of(logits)),
           "route_logits");
  return {probs, gates, mask, count};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> route_logits_meta(const Tensor& logits, double) {
  const c10::SymInt N = logits.sym_size(0), E = logits.sym_size(1);
  return {at::empty_like(logits), at::empty_like(logits), at::empty_symint({N, E}, logits.options().dtype(at::kByte)),
          at::empty_symint({N}, logits.options().dtype(at::kInt))};
}

// ------------------------------------------------------------------ bucketing
// Output shapes of bucket: token_ids / pair_gates hold N*E + 1 entries (never empty),
// tiles the pp_max_tiles bound (N*E) / tile_m + E rows.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> bucket_shapes(const Tensor& mask, int64_t tile_m) {
  const c10::SymInt N = mask.sym_size(0), E = mask.sym_size(1);
  const int64_t tm = tile_m > 0 ? tile_m : pp_gemm_tile_m();
  const c10::SymInt cap = N * E + 1, mt = (N * E) / tm + E;
  auto i32 = mask.options().dtype(at::kInt);
  return {at::empty_symint({E + 1}, i32),
          at::empty_symint({cap}, i32),
          at::empty_symint({cap}, mask.options().dtype(at::kFloat)),
          at::empty_symint({N, E}, i32),
          at::empty_symint({mt, 4}, i32),
          at::empty({4}, i32)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> bucket_gpu(const Tensor& mask, const Tensor& gates,
                                                                      int64_t tile_m) {
  TORCH_CHECK(mask.scalar_type() == at::kByte && gates.scalar_type() == at::kFloat && mask.dim() == 2 &&
                  mask.sizes() == gates.sizes(),
              "prunepath.bucket: mask uint8 [N, E] and gates float32 [N, E] required");
  need_gpu("bucket", mask, {&mask, &gates});
  const c10::DeviceGuard g(mask.device());
  const int64_t N = mask.size(0), E = mask.size(1);
  const int tm = tile_m > 0 ? (int)tile_m : pp_gemm_tile_m();
  auto r = bucket_shapes(mask, tm);
  TORCH_CHECK(std::get<4>(r).size(0) == pp_max_tiles(N, (int)E, tm), "prunepath.bucket: tile bound mismatch");
  // capacity tails (token_ids / pair_gates past offsets[E], tiles past meta[0]) are zero,
  // so every output element is defined and the op's results are the same on every call
  std::get<1>(r).zero_();
  std::get<2>(r).zero_();
  std::get<4>(r).zero_();
  Tensor ws = at::empty({(int64_t)pp_bucket_workspace_bytes(N, (int)E)}, mask.options().dtype(at::kByte));
  check_rc(pp_bucket(mask.data_ptr<uint8_t>(), gates.data_ptr<float>(), N, (int)E, tm,
                     std::get<0>(r).data_ptr<int32_t>(), std::get<1>(r).data_ptr<int32_t>(),
                     std::get<2>(r).data_ptr<float>(), std::get<3>(r).data_ptr<int32_t>(),
                     std::get<4>(r).data_ptr<int32_t>(), std::get<5>(r).data_ptr<int32_t>(), ws.data_ptr(),
                     stream_of(mask)),
           "bucket");
  return r;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> bucket_meta(const Tensor& mask, const Tensor&,
                                                                       int64_t tile_m) {
  return bucket_shapes(mask, tile_m);
}

// ------------------------------------------------------------------ rearrangement
struct PackLayout {
  int64_t H, I, s_n, s_h, d_n, d_h;
};

PackLayout pack_layout(const Tensor& w_gate, const Tensor& w_down, c10::string_view layout) {
  TORCH_CHECK(w_gate.dim() == 2 && w_down.dim() == 2, "prunepath.pack_experts: 2-D weights required");
  if (layout == "linear") {  // gate/up [I, H], down [H, I]
    const int64_t I = w_gate.size(0), H = w_gate.size(1);
    TORCH_CHECK(w_down.size(0) == H && w_down.size(1) == I, "prunepath.pack_experts: down must be [H, I]");
    return {H, I, H, 1, 1, I};
  }
  TORCH_CHECK(layout == "tau", "prunepath.pack_experts: layout must be 'linear' or 'tau'");
  const int64_t H = w_gate.size(0), I = w_gate.size(1);  // W_gate/W_up [H, I], W_down [I, H]
  TORCH_CHECK(w_down.size(0) == I && w_down.size(1) == H, "prunepath.pack_experts: W_down must be [I, H]");
  return {H, I, 1, I, H, 1};
}

Tensor pack_experts_gpu(const Tensor& w_gate, const Tensor& w_up, const Tensor& w_down, int64_t E, int64_t G,
                        const optional<Tensor>& perm, c10::string_view layout) {
  const PackLayout L = pack_layout(w_gate, w_down, layout);
  TORCH_CHECK(w_up.sizes() == w_gate.sizes() && w_up.scalar_type() == w_gate.scalar_type() &&
                  w_down.scalar_type() == w_gate.scalar_type(),
              "prunepath.pack_experts: gate/up/down shapes or dtypes disagree");
  TORCH_CHECK(L.I == E * G, "prunepath.pack_experts: I=", L.I, " != E*G=", E * G);
  if (perm.has_value())
    TORCH_CHECK(perm->scalar_type() == at::kInt && perm->numel() == L.I, "prunepath.pack_experts: perm must be int32 [I]");
  need_gpu("pack_experts", w_gate, {&w_gate, &w_up, &w_down, perm.has_value() ? &*perm : nullptr});
  const c10::DeviceGuard g(w_gate.device());
  Tensor out = at::empty({(int64_t)(pp_packed_expert_bytes((int)L.H, (int)E, (int)G) / 2)},
                         w_gate.options().dtype(at::kBFloat16));
  check_rc(pp_pack_experts(w_gate.data_ptr(), w_up.data_ptr(), L.s_n, L.s_h, w_down.data_ptr(), L.d_n, L.d_h,
                           w_code(w_gate, "pack_experts"), (const int32_t*)ptr(perm), (int)L.H, (int)E, (int)G,
                           out.data_ptr(), stream_of(w_gate)),
           "pack_experts");
  return out;
}

Tensor pack_experts_meta(const Tensor& w_gate, const Tensor&, const Tensor&, int64_t E, int64_t G,
                         const optional<Tensor>&, c10::string_view layout) {
  // packed = rows [E*G][3][H] + down_t [E][H][G]: 4*E*G*H bf16 (pp_packed_expert_bytes / 2)
  const c10::SymInt H = layout == "linear" ? w_gate.sym_size(1) : w_gate.sym_size(0);
  return at::empty_symint({H * (4 * E * G)}, w_gate.options().dtype(at::kBFloat16));
}

std::pair<int64_t, int64_t> router_dims(const Tensor& w, c10::string_view layout, int64_t* s_e, int64_t* s_h) {
  TORCH_CHECK(w.dim() == 2, "prunepath.pack_router: 2-D router weights required");
  if (layout == "linear") {  // [E, H]
    *s_e = w.size(1);
    *s_h = 1;
    return {w.size(0), w.size(1)};
  }
  TORCH_CHECK(layout == "tau", "prunepath.pack_router: layout must be 'linear' or 'tau'");
  *s_e = 1;  // [H, E]
  *s_h = w.size(1);
  return {w.size(1), w.size(0)};
}

Tensor pack_router_gpu(const Tensor& w, c10::string_view layout) {
  int64_t s_e, s_h;
  const auto [E, H] = router_dims(w, layout, &s_e, &s_h);
  need_gpu("pack_router", w, {&w});
  const c10::DeviceGuard g(w.device());
  Tensor out = at::empty({(E + 15) / 16 * 16, H}, w.options().dtype(at::kFloat));
  check_rc(pp_pack_router(w.data_ptr(), s_e, s_h, w_code(w, "pack_router"), (int)H, (int)E, out.data_ptr<float>(),
                          stream_of(w)),
           "pack_router");
  return out;
}

Tensor pack_router_meta(const Tensor& w, c10::string_view layout) {
  const c10::SymInt E = layout == "linear" ? w.sym_size(0) : w.sym_size(1);
  const c10::SymInt H = layout == "linear" ? w.sym_size(1) : w.sym_size(0);
  return at::empty_symint({(E + 15) / 16 * 16, H}, w.options().dtype(at::kFloat));
}

// ------------------------------------------------------------------ decode
void decode_workspace_init_gpu(const Tensor& ws, int64_t H, int64_t E) {
  TORCH_CHECK(ws.scalar_type() == at::kByte && ws.numel() >= (int64_t)pp_decode_workspace_bytes((int)H, (int)E),
              "prunepath.decode_workspace_init: uint8 workspace of pp_decode_workspace_bytes(H, E) required");
  need_gpu("decode_workspace_init", ws, {&ws});
  const c10::DeviceGuard g(ws.device());
  check_rc(pp_decode_workspace_init(ws.data_ptr(), (int)H, (int)E, stream_of(ws)), "decode_workspace_init");
}

void decode_workspace_init_meta(const Tensor&, int64_t, int64_t) {}

void decode_into(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E, int64_t G,
                 double tau, const Tensor& packed, const Tensor& workspace, const Tensor& out, int64_t grid) {
  const int64_t H = x.numel();
  check_bias(bias, E, "moe_decode");
  TORCH_CHECK(workspace.scalar_type() == at::kByte &&
                  workspace.numel() >= (int64_t)pp_decode_workspace_bytes((int)H, (int)E),
              "prunepath.moe_decode: uint8 workspace of pp_decode_workspace_bytes(H, E) required");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.numel() == H, "prunepath.moe_decode: out must be bf16 [1, H]");
  need_gpu("moe_decode", x, {&x, &router_packed, bias.has_value() ? &*bias : nullptr, &packed, &workspace, &out});
  const c10::DeviceGuard g(x.device());
  check_rc(pp_moe_decode(x.data_ptr(), x_code(x, "moe_decode"), (int)H, router_packed.data_ptr<float>(),
                         (const float*)ptr(bias), (int)E, (int)G, (float)tau, packed.data_ptr(), out.data_ptr(),
                         workspace.data_ptr(), (int)grid, stream_of(x)),
           "moe_decode");
}

Tensor moe_decode_gpu(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E,
                      int64_t G, double tau, const Tensor& packed, const Tensor& workspace, int64_t grid) {
  Tensor out = at::empty({1, x.numel()}, x.options().dtype(at::kBFloat16));
  decode_into(x, router_packed, bias, E, G, tau, packed, workspace, out, grid);
  return out;
}

void moe_decode_into_meta(const Tensor&, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                          const Tensor&, const Tensor&, const Tensor&, int64_t) {}

Tensor moe_decode_meta(const Tensor& x, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                       const Tensor&, const Tensor&, int64_t) {
  return at::empty_symint({c10::SymInt(1), x.sym_numel()}, x.options().dtype(at::kBFloat16));
}

// ------------------------------------------------------------------ small-batch decode
void decode_batch_into(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E,
                       int64_t G, double tau, const Tensor& packed, const Tensor& workspace,
                       const Tensor& batch_workspace, const Tensor& out, const optional<Tensor>& logits_out,
                       const optional<Tensor>& mask_out, int64_t grid) {
  TORCH_CHECK(x.dim() == 2, "prunepath.moe_decode_batch: x must be [N, H]");
  const int64_t N = x.size(0), H = x.size(1);
  check_bias(bias, E, "moe_decode_batch");
  TORCH_CHECK(workspace.scalar_type() == at::kByte &&
                  workspace.numel() >= (int64_t)pp_decode_workspace_bytes((int)H, (int)E),
              "prunepath.moe_decode_batch: uint8 workspace of pp_decode_workspace_bytes(H, E) required");
  TORCH_CHECK(batch_workspace.scalar_type() == at::kByte &&
                  batch_workspace.numel() >= (int64_t)pp_decode_batch_workspace_bytes((int)H, (int)E, (int)G),
              "prunepath.moe_decode_batch: uint8 batch_workspace of pp_decode_batch_workspace_bytes(H, E, G) required");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.numel() == N * H && out.is_contiguous(),
              "prunepath.moe_decode_batch: out must be contiguous bf16 [N, H]");
  if (logits_out.has_value())
    TORCH_CHECK(logits_out->scalar_type() == at::kFloat && logits_out->numel() == N * E && logits_out->is_contiguous(),
                "prunepath.moe_decode_batch: logits_out must be contiguous fp32 [N, E]");
  if (mask_out.has_value())
    TORCH_CHECK(mask_out->scalar_type() == at::kByte && mask_out->numel() == N * E && mask_out->is_contiguous(),
                "prunepath.moe_decode_batch: mask_out must be contiguous uint8 [N, E]");
  need_gpu("moe_decode_batch", x,
           {&x, &router_packed, bias.has_value() ? &*bias : nullptr, &packed, &workspace, &batch_workspace, &out,
            logits_out.has_value() ? &*logits_out : nullptr, mask_out.has_value() ? &*mask_out : nullptr});
  const c10::DeviceGuard g(x.device());
  check_rc(pp_moe_decode_batch(x.data_ptr(), x_code(x, "moe_decode_batch"), N, (int)H,
                               router_packed.data_ptr<float>(), (const float*)ptr(bias), (int)E, (int)G, (float)tau,
                               packed.data_ptr(), out.data_ptr(),
                               logits_out.has_value() ? logits_out->data_ptr<float>() : nullptr,
                               mask_out.has_value() ? mask_out->data_ptr<uint8_t>() : nullptr, workspace.data_ptr(),
                               batch_workspace.data_ptr(), (int)grid, stream_of(x)),
           "moe_decode_batch");
}

Tensor moe_decode_batch_gpu(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E,
                            int64_t G, double tau, const Tensor& packed, const Tensor& workspace,
                            const Tensor& batch_workspace, int64_t grid) {
  TORCH_CHECK(x.dim() == 2, "prunepath.moe_decode_batch: x must be [N, H]");
  Tensor out = at::empty({x.size(0), x.size(1)}, x.options().dtype(at::kBFloat16));
  decode_batch_into(x, router_packed, bias, E, G, tau, packed, workspace, batch_workspace, out, c10::nullopt,
                    c10::nullopt, grid);
  return out;
}

Tensor moe_decode_batch_meta(const Tensor& x, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                             const Tensor&, const Tensor&, const Tensor&, int64_t) {
  return at::empty_symint(x.sym_sizes(), x.options().dtype(at::kBFloat16));
}

void moe_decode_batch_into_meta(const Tensor&, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                                const Tensor&, const Tensor&, const Tensor&, const Tensor&, const optional<Tensor>&,
                                const optional<Tensor>&, int64_t) {}

// ------------------------------------------------------------------ prefill
// One implementation behind both boundaries: pp_moe_prefill_routed (the grouped pipeline,
// or for G % 64 != 0 the dense form of csrc/dense.hip), hand-written kernels only.
void prefill_into(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E, int64_t G,
                  double tau, const Tensor& packed, const Tensor& workspace, const Tensor& out,
                  const optional<Tensor>& logits_out, const optional<Tensor>& mask_out) {
  TORCH_CHECK(x.dim() == 2, "prunepath.moe_prefill: x must be [N, H]");
  const int64_t N = x.size(0), H = x.size(1);
  check_bias(bias, E, "moe_prefill");
  TORCH_CHECK(x.is_contiguous() && packed.is_contiguous(), "prunepath.moe_prefill: x and packed must be contiguous");
  TORCH_CHECK(workspace.scalar_type() == at::kByte &&
                  workspace.numel() >= (int64_t)pp_prefill_workspace_bytes(N, (int)H, (int)E, (int)G),
              "prunepath.moe_prefill: uint8 workspace of pp_prefill_workspace_bytes(N, H, E, G) required");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.numel() == N * H && out.is_contiguous(),
              "prunepath.moe_prefill: out must be contiguous bf16 [N, H]");
  if (logits_out.has_value())
    TORCH_CHECK(logits_out->scalar_type() == at::kFloat && logits_out->numel() == N * E && logits_out->is_contiguous(),
                "prunepath.moe_prefill: logits_out must be contiguous fp32 [N, E]");
  if (mask_out.has_value())
    TORCH_CHECK(mask_out->scalar_type() == at::kByte && mask_out->numel() == N * E && mask_out->is_contiguous(),
                "prunepath.moe_prefill: mask_out must be contiguous uint8 [N, E]");
  need_gpu("moe_prefill", x,
           {&x, &router_packed, bias.has_value() ? &*bias : nullptr, &packed, &workspace, &out,
            logits_out.has_value() ? &*logits_out : nullptr, mask_out.has_value() ? &*mask_out : nullptr});
  const c10::DeviceGuard g(x.device());
  check_rc(pp_moe_prefill_routed(x.data_ptr(), x_code(x, "moe_prefill"), N, (int)H, router_packed.data_ptr<float>(),
                                 (const float*)ptr(bias), (int)E, (int)G, (float)tau, packed.data_ptr(),
                                 out.data_ptr(), workspace.data_ptr(),
                                 logits_out.has_value() ? logits_out->data_ptr<float>() : nullptr,
                                 mask_out.has_value() ? mask_out->data_ptr<uint8_t>() : nullptr, stream_of(x)),
           "moe_prefill");
}

Tensor moe_prefill_gpu(const Tensor& x, const Tensor& router_packed, const optional<Tensor>& bias, int64_t E,
                       int64_t G, double tau, const Tensor& packed) {
  TORCH_CHECK(x.dim() == 2, "prunepath.moe_prefill: x must be [N, H]");
  const int64_t N = x.size(0), H = x.size(1);
  Tensor out = at::empty({N, H}, x.options().dtype(at::kBFloat16));
  Tensor ws = at::empty({(int64_t)pp_prefill_workspace_bytes(N, (int)H, (int)E, (int)G)},
                        x.options().dtype(at::kByte));
  prefill_into(x, router_packed, bias, E, G, tau, packed, ws, out, c10::nullopt, c10::nullopt);
  return out;
}

Tensor moe_prefill_meta(const Tensor& x, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                        const Tensor&) {
  return at::empty_symint(x.sym_sizes(), x.options().dtype(at::kBFloat16));
}

void moe_prefill_into_meta(const Tensor&, const Tensor&, const optional<Tensor>&, int64_t, int64_t, double,
                           const Tensor&, const Tensor&, const Tensor&, const optional<Tensor>&,
                           const optional<Tensor>&) {}

// CPU tensors: refused with the op's name (there is no host implementation, on purpose).
// ------------------------------------------------------------------ masked gating (training)
// masked_gate / masked_gate_bwd: MoELayer.forward's mask matmul and multiply
// (src/MoEBlock_origin.py:205-212), out = inter * gates[:, expert_ids], and its backward
// (autograd of masked_gate is registered from Python: ops.py). inter / d_out [..., I]
// (fp32 or bf16, the rows flattened), gates [..., E] fp32, expert_ids / perm int32 [I],
// seg int32 [E + 1] (masked_gate_layout in ops.py); perm and seg are the backward's
// expert segments, carried by the forward for autograd.
void masked_gate_check(const char* name, const Tensor& inter, const Tensor& gates, const Tensor& eid) {
  TORCH_CHECK(inter.dim() >= 1 && gates.dim() >= 1, "prunepath.", name, ": inter [..., I] and gates [..., E]");
  TORCH_CHECK(gates.scalar_type() == at::kFloat, "prunepath.", name, ": gates must be float32");
  TORCH_CHECK(eid.scalar_type() == at::kInt && eid.numel() == inter.size(-1), "prunepath.", name,
              ": expert_ids must be int32 [I]");
  TORCH_CHECK(gates.numel() / std::max<int64_t>(1, gates.size(-1)) == inter.numel() / std::max<int64_t>(1, inter.size(-1)),
              "prunepath.", name, ": inter and gates have different row counts");
}

Tensor masked_gate_gpu(const Tensor& inter, const Tensor& gates, const Tensor& eid, const Tensor& perm,
                       const Tensor& seg) {
  masked_gate_check("masked_gate", inter, gates, eid);
  need_gpu("masked_gate", inter, {&inter, &gates, &eid, &perm, &seg});
  const c10::DeviceGuard g(inter.device());
  const int64_t I = inter.size(-1), E = gates.size(-1), n = inter.numel() / std::max<int64_t>(1, I);
  Tensor out = at::empty_like(inter);
  if (n == 0) return out;
  check_rc(pp_masked_gate_fwd(inter.data_ptr(), x_code(inter, "masked_gate"), gates.data_ptr<float>(),
                              eid.data_ptr<int32_t>(), n, (int)I, (int)E, out.data_ptr(), stream_of(inter)),
           "masked_gate");
  return out;
}

Tensor masked_gate_meta(const Tensor& inter, const Tensor&, const Tensor&, const Tensor&, const Tensor&) {
  return at::empty_like(inter);
}

std::tuple<Tensor, Tensor> masked_gate_bwd_gpu(const Tensor& d_out, const Tensor& inter, const Tensor& gates,
                                               const Tensor& eid, const Tensor& perm, const Tensor& seg,
                                               bool need_d_inter) {
  masked_gate_check("masked_gate_bwd", inter, gates, eid);
  TORCH_CHECK(d_out.sizes() == inter.sizes() && d_out.scalar_type() == inter.scalar_type(),
              "prunepath.masked_gate_bwd: d_out must match inter's shape and dtype");
  TORCH_CHECK(perm.scalar_type() == at::kInt && perm.numel() == inter.size(-1) && seg.scalar_type() == at::kInt &&
                  seg.numel() == gates.size(-1) + 1,
              "prunepath.masked_gate_bwd: perm int32 [I] and seg int32 [E + 1] required");
  need_gpu("masked_gate_bwd", inter, {&d_out, &inter, &gates, &eid, &perm, &seg});
  const c10::DeviceGuard g(inter.device());
  const int64_t I = inter.size(-1), E = gates.size(-1), n = inter.numel() / std::max<int64_t>(1, I);
  Tensor d_inter = need_d_inter ? at::empty_like(inter) : at::empty({0}, inter.options());
  Tensor d_gates = at::empty_like(gates);
  if (n == 0) return {d_inter, d_gates};
  check_rc(pp_masked_gate_bwd(d_out.data_ptr(), inter.data_ptr(), x_code(inter, "masked_gate_bwd"),
                              gates.data_ptr<float>(), eid.data_ptr<int32_t>(), perm.data_ptr<int32_t>(),
                              seg.data_ptr<int32_t>(), n, (int)I, (int)E, need_d_inter ? d_inter.data_ptr() : nullptr,
                              d_gates.data_ptr<float>(), stream_of(inter)),
           "masked_gate_bwd");
  return {d_inter, d_gates};
}

std::tuple<Tensor, Tensor> masked_gate_bwd_meta(const Tensor&, const Tensor& inter, const Tensor& gates,
                                                const Tensor&, const Tensor&, const Tensor&, bool need_d_inter) {
  return {need_d_inter ? at::empty_like(inter) : at::empty({0}, inter.options()), at::empty_like(gates)};
}

void refuse_cpu(const c10::OperatorHandle& op, torch::jit::Stack*) {
  TORCH_CHECK(false, op.schema().name(), ": tensors must be on the GPU (got cpu); there is no CPU implementation");
}

}  // namespace

TORCH_LIBRARY(prunepath, m) {
  m.def("route(Tensor x, Tensor router_packed, Tensor? bias, int E, float tau) -> "
        "(Tensor logits, Tensor probs, Tensor gates, Tensor mask, Tensor count)");
  m.def("route_logits(Tensor logits, float tau) -> (Tensor probs, Tensor gates, Tensor mask, Tensor count)");
  m.def("bucket(Tensor mask, Tensor gates, int tile_m=0) -> (Tensor offsets, Tensor token_ids, Tensor pair_gates, "
        "Tensor token_pairs, Tensor tiles, Tensor meta)");
  m.def("pack_experts(Tensor w_gate, Tensor w_up, Tensor w_down, int E, int G, Tensor? perm=None, "
        "str layout='linear') -> Tensor");
  m.def("pack_router(Tensor w_router, str layout='linear') -> Tensor");
  m.def("decode_workspace_init(Tensor(a!) workspace, int H, int E) -> ()");
  m.def("moe_decode(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed, "
        "Tensor(a!) workspace, int grid=0) -> Tensor");
  m.def("moe_decode_into(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed, "
        "Tensor(a!) workspace, Tensor(b!) out, int grid=0) -> ()");
  m.def("moe_decode_batch(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed, "
        "Tensor(a!) workspace, Tensor(b!) batch_workspace, int grid=0) -> Tensor");
  m.def("moe_decode_batch_into(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed, "
        "Tensor(a!) workspace, Tensor(b!) batch_workspace, Tensor(c!) out, Tensor(d!)? logits_out=None, "
        "Tensor(e!)? mask_out=None, int grid=0) -> ()");
  m.def("moe_prefill(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed) -> Tensor");
  m.def("moe_prefill_into(Tensor x, Tensor router_packed, Tensor? bias, int E, int G, float tau, Tensor packed, "
        "Tensor(a!) workspace, Tensor(b!) out, Tensor(c!)? logits_out=None, Tensor(d!)? mask_out=None) -> ()");
  m.def("masked_gate(Tensor inter, Tensor gates, Tensor expert_ids, Tensor perm, Tensor seg) -> Tensor");
  m.def("masked_gate_bwd(Tensor d_out, Tensor inter, Tensor gates, Tensor expert_ids, Tensor perm, Tensor seg, "
        "bool need_d_inter=True) -> (Tensor d_inter, Tensor d_gates)");
}

TORCH_LIBRARY_IMPL(prunepath, CUDA, m) {
  m.impl("route", &route_gpu);
  m.impl("route_logits", &route_logits_gpu);
  m.impl("bucket", &bucket_gpu);
  m.impl("pack_experts", &pack_experts_gpu);
  m.impl("pack_router", &pack_router_gpu);
  m.impl("decode_workspace_init", &decode_workspace_init_gpu);
  m.impl("moe_decode", &moe_decode_gpu);
  m.impl("moe_decode_into", &decode_into);
  m.impl("moe_decode_batch", &moe_decode_batch_gpu);
  m.impl("moe_decode_batch_into", &decode_batch_into);
  m.impl("moe_prefill", &moe_prefill_gpu);
  m.impl("moe_prefill_into", &prefill_into);
  m.impl("masked_gate", &masked_gate_gpu);
  m.impl("masked_gate_bwd", &masked_gate_bwd_gpu);
}

TORCH_LIBRARY_IMPL(prunepath, Meta, m) {
  m.impl("route", &route_meta);
  m.impl("route_logits", &route_logits_meta);
  m.impl("bucket", &bucket_meta);
  m.impl("pack_experts", &pack_experts_meta);
  m.impl("pack_router", &pack_router_meta);
  m.impl("decode_workspace_init", &decode_workspace_init_meta);
  m.impl("moe_decode", &moe_decode_meta);
  m.impl("moe_decode_into", &moe_decode_into_meta);
  m.impl("moe_decode_batch", &moe_decode_batch_meta);
  m.impl("moe_decode_batch_into", &moe_decode_batch_into_meta);
  m.impl("moe_prefill", &moe_prefill_meta);
  m.impl("moe_prefill_into", &moe_prefill_into_meta);
  m.impl("masked_gate", &masked_gate_meta);
  m.impl("masked_gate_bwd", &masked_gate_bwd_meta);
}

TORCH_LIBRARY_IMPL(prunepath, CPU, m) {
  for (const char* name : {"route", "route_logits", "bucket", "pack_experts", "pack_router", "decode_workspace_init",
                           "moe_decode", "moe_decode_into", "moe_decode_batch", "moe_decode_batch_into",
                           "moe_prefill", "moe_prefill_into", "masked_gate", "masked_gate_bwd"})
    m.impl(name, torch::CppFunction::makeFromBoxedFunction<&refuse_cpu>());
}
