// One-time rearrangement of the expert weights (replaces physical_reorder_for_inference,
// src/openpangu_moe.py:212-256: argsort neuron->expert ids, permute gate/up rows and
// down columns, transpose, cast to bf16).
//
// Output layout (bf16):
//   rows   [E*G][3][H]: per rearranged neuron j a 6*H-byte record
//                       {gate row, up row, down column} -- what the decode GEMV streams
//                       (one contiguous record per neuron, 16-byte loads per lane);
//   down_t [E][H][G]:   per expert, the down projection with its G neurons contiguous --
//                       the K-contiguous B operand of the prefill down GEMM.
#include "pp_common.h"

template <typename ST>
__global__ __launch_bounds__(256) void pack_rows_kernel(const ST* __restrict__ w_gate,
                                                        const ST* __restrict__ w_up, int64_t s_n,
                                                        int64_t s_h, const ST* __restrict__ w_down,
                                                        int64_t d_n, int64_t d_h,
                                                        const int32_t* __restrict__ perm, int H,
                                                        int64_t n_rec, bf16_t* __restrict__ rows) {
  for (int64_t rec = blockIdx.x; rec < n_rec; rec += gridDim.x) {  // rearranged neuron j * 3 + part
    const int64_t j = rec / 3;
    const int part = (int)(rec % 3);
    const int64_t src = perm ? (int64_t)perm[j] : j;
    bf16_t* dst = rows + rec * H;
    for (int h = threadIdx.x; h < H; h += 256) {
      float v;
      if (part == 0) v = load_as_f32<ST>(w_gate, src * s_n + (int64_t)h * s_h);
      else if (part == 1) v = load_as_f32<ST>(w_up, src * s_n + (int64_t)h * s_h);
      else v = load_as_f32<ST>(w_down, src * d_n + (int64_t)h * d_h);
      dst[h] = f32_to_bf16(v);
    }
  }
}

// down_t[e][h][g] = down(neuron perm[e*G+g], h); g fastest.
template <typename ST>
__global__ __launch_bounds__(256) void pack_down_t_kernel(const ST* __restrict__ w_down, int64_t d_n,
                                                          int64_t d_h, const int32_t* __restrict__ perm,
                                                          int H, int G, int64_t total,
                                                          bf16_t* __restrict__ down_t) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t g = i % G;
    int64_t h = (i / G) % H;
    int64_t e = i / ((int64_t)G * H);
    int64_t j = e * G + g;
    int64_t src = perm ? (int64_t)perm[j] : j;
    down_t[i] = f32_to_bf16(load_as_f32<ST>(w_down, src * d_n + h * d_h));
  }
}

template <typename ST>
__global__ __launch_bounds__(256) void pack_router_kernel(const ST* __restrict__ w, int64_t s_e,
                                                          int64_t s_h, int H, int E, int Epad,
                                                          float* __restrict__ out) {
  int64_t total = (int64_t)Epad * H;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t e = i / H, h = i % H;
    out[i] = e < E ? load_as_f32<ST>(w, e * s_e + h * s_h) : 0.0f;
  }
}

extern "C" size_t pp_packed_expert_bytes(int H, int E, int G) {
  return (size_t)E * G * H * 4 * sizeof(bf16_t);
}

extern "C" int pp_pack_experts(const void* w_gate, const void* w_up, int64_t s_n, int64_t s_h,
                               const void* w_down, int64_t d_n, int64_t d_h, int src_dtype,
                               const int32_t* perm, int H, int E, int G, void* packed,
                               void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(w_gate && w_up && w_down && packed, PP_ERR_INVALID, "pp_pack_experts: null pointer");
  PP_REQUIRE(src_dtype == PP_DTYPE_F32 || src_dtype == PP_DTYPE_BF16, PP_ERR_INVALID,
             "pp_pack_experts: src_dtype %d", src_dtype);
  hipStream_t st = (hipStream_t)stream;
  const int64_t I = (int64_t)E * G;
  bf16_t* rows = (bf16_t*)packed;
  bf16_t* down_t = rows + I * 3 * H;
  const int64_t n_rec = I * 3;
  int grid1 = (int)(n_rec < 65536 ? n_rec : 65536);
  int64_t total = I * H;
  int grid2 = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
  if (src_dtype == PP_DTYPE_F32) {
    pack_rows_kernel<float><<<grid1, 256, 0, st>>>((const float*)w_gate, (const float*)w_up, s_n, s_h,
                                                   (const float*)w_down, d_n, d_h, perm, H, n_rec, rows);
    pack_down_t_kernel<float><<<grid2, 256, 0, st>>>((const float*)w_down, d_n, d_h, perm, H, G, total, down_t);
  } else {
    pack_rows_kernel<bf16_t><<<grid1, 256, 0, st>>>((const bf16_t*)w_gate, (const bf16_t*)w_up, s_n, s_h,
                                                    (const bf16_t*)w_down, d_n, d_h, perm, H, n_rec, rows);
    pack_down_t_kernel<bf16_t><<<grid2, 256, 0, st>>>((const bf16_t*)w_down, d_n, d_h, perm, H, G, total, down_t);
  }
  return pp_check_launch("pp_pack_experts");
}

extern "C" size_t pp_packed_router_bytes(int H, int E) {
  return (size_t)((E + 15) / 16 * 16) * H * sizeof(float);
}

extern "C" int pp_pack_router(const void* w_router, int64_t s_e, int64_t s_h, int src_dtype, int H,
                              int E, float* router_packed, void* stream) {
  int rc = pp_check_shape(H, E, 32);
  if (rc) return rc;
  PP_REQUIRE(w_router && router_packed, PP_ERR_INVALID, "pp_pack_router: null pointer");
  PP_REQUIRE(src_dtype == PP_DTYPE_F32 || src_dtype == PP_DTYPE_BF16, PP_ERR_INVALID,
             "pp_pack_router: src_dtype %d", src_dtype);
  const int Epad = (E + 15) / 16 * 16;
  int64_t total = (int64_t)Epad * H;
  int grid = (int)((total + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
  if (src_dtype == PP_DTYPE_F32)
    pack_router_kernel<float><<<grid, 256, 0, st>>>((const float*)w_router, s_e, s_h, H, E, Epad, router_packed);
  else
    pack_router_kernel<bf16_t><<<grid, 256, 0, st>>>((const bf16_t*)w_router, s_e, s_h, H, E, Epad, router_packed);
  return pp_check_launch("pp_pack_router");
}
