// Routing and bucketing for N tokens.
//
// route_kernel: fp32 router logits x @ Wr^T (+bias) on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32, one wave per 16 tokens, all experts), then tau selection
// per token (select_one_token, bit-exact with torch CPU given the logits).
// Replaces moe_router_kernel + torch.sort + moe_select_expert_kernel + scatter_
// (src/tl_kernel_optimized_Ultimate_PanGU.py:40-124, 550-564) and softmax_thresholding
// (src/MoEBlock_origin.py:50-97).
//
// bucket_*: stable counting sort of (token, expert) pairs into a CSR layout with
// experts ascending and tokens ascending inside each expert, plus the row-tile map
// of the grouped GEMMs. Replaces moe_local_scan_kernel / moe_global_scan_kernel /
// moe_dispatch_kernel (src/tl_kernel_optimized_Ultimate_PanGU.py:133-266) without the
// 512-tile cap of the global scan (:176, 206-208) and without the host sync (:581).
#include "pp_common.h"

#define ROUTE_TOK 16   // tokens per workgroup (one 16-row MFMA tile)
#define ROUTE_WAVES 4  // K split across the waves, then 4 selections per wave
#define ROUTE_EGRP 64  // experts per pass (4 MFMA tiles of 16)

// Logits of 16 tokens x 16 experts per MFMA tile: lane l supplies x[row l%16][k0+4(l/16)+j]
// and W[expert l%16][k0+4(l/16)+j] for j = 0..3, one MFMA per j, so every k of the
// 16-wide block is used exactly once. Result lane l, element q: token 4(l/16)+q,
// expert l%16. Wave w covers the k-blocks kb = w, w+4, ...; the four partial tiles are
// summed in wave order through LDS (fixed order: deterministic logits).
template <typename XT>
__device__ __forceinline__ float4 load_x4(const XT* x, int64_t off);
template <>
__device__ __forceinline__ float4 load_x4<float>(const float* x, int64_t off) {
  return *(const float4*)(x + off);
}
template <>
__device__ __forceinline__ float4 load_x4<bf16_t>(const bf16_t* x, int64_t off) {
  uint2 u = *(const uint2*)(x + off);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

template <typename XT, bool FROM_LOGITS>
__global__ __launch_bounds__(256) void route_kernel(
    const XT* __restrict__ x, const float* __restrict__ logits_in, int64_t N, int H,
    const float* __restrict__ router, const float* __restrict__ bias, int E, float tau,
    float* __restrict__ logits_out, float* __restrict__ probs_out, float* __restrict__ gates_out,
    uint8_t* __restrict__ mask_out, int32_t* __restrict__ count_out, bf16_t* __restrict__ xbf_out) {
  __shared__ SelScratch ssw[ROUTE_WAVES];
  __shared__ float lg_s[ROUTE_TOK][PP_MAX_EXPERTS];
  __shared__ float part[ROUTE_WAVES][ROUTE_TOK][ROUTE_EGRP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t tok0 = (int64_t)blockIdx.x * ROUTE_TOK;

  if (FROM_LOGITS) {
    for (int i = tid; i < ROUTE_TOK * E; i += 256) {
      const int r = i / E, e = i % E;
      const int64_t t = tok0 + r;
      lg_s[r][e] = t < N ? logits_in[t * E + e] : 0.0f;
    }
  } else {
    const int r = lane & 15, g = lane >> 4;
    const int64_t t = tok0 + r;
    const bool valid = t < N;
    const int ntile = (E + 15) / 16;
    for (int tg = 0; tg < ntile; tg += 4) {
      f32x4_t acc[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
      for (int k0 = 16 * w; k0 < H; k0 += 16 * ROUTE_WAVES) {
        const int kk = k0 + 4 * g;
        const float4 xa = valid ? load_x4<XT>(x, t * H + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (xbf_out && tg == 0 && valid) {
          uint2 pk;
          pk.x = (uint32_t)f32_to_bf16(xa.x) | ((uint32_t)f32_to_bf16(xa.y) << 16);
          pk.y = (uint32_t)f32_to_bf16(xa.z) | ((uint32_t)f32_to_bf16(xa.w) << 16);
          *(uint2*)(xbf_out + t * H + kk) = pk;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (tg + u < ntile) {
            const float4 wb = *(const float4*)(router + (int64_t)((tg + u) * 16 + r) * H + kk);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, wb.x, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, wb.y, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, wb.z, acc[u], 0, 0, 0);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, wb.w, acc[u], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) part[w][4 * g + q][u * 16 + r] = acc[u][q];
      __syncthreads();
      for (int i = tid; i < ROUTE_TOK * ROUTE_EGRP; i += 256) {
        const int rr = i / ROUTE_EGRP, c = i % ROUTE_EGRP, e = tg * 16 + c;
        if (e < E) {
          float l = __fadd_rn(__fadd_rn(__fadd_rn(part[0][rr][c], part[1][rr][c]), part[2][rr][c]), part[3][rr][c]);
          if (bias) l = __fadd_rn(l, bias[e]);
          lg_s[rr][e] = l;
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();

  // selection: wave w takes tokens 4w .. 4w+3
  SelScratch* ss = ssw + w;
  for (int rr = 4 * w; rr < 4 * w + 4; ++rr) {
    const int64_t t = tok0 + rr;
    if (t >= N) break;  // wave-uniform
    const float* lrow = lg_s[rr];
    select_one_token([&](int j) { return lrow[j]; }, E, tau, ss, lane);
    const int k = ss->k;
    for (int j = lane; j < E; j += 64) ss->sel[j] = 0;
    wave_sync_lds();
    for (int q = lane; q < k; q += 64) ss->sel[ss->order[q]] = 1;
    wave_sync_lds();
    for (int j = lane; j < E; j += 64) {
      const int s = ss->sel[j];
      const float l = lrow[j];
      if (logits_out) logits_out[t * E + j] = l;
      if (probs_out) probs_out[t * E + j] = ss->e[j];
      if (gates_out) gates_out[t * E + j] = s ? pp_sigmoid(l) : 0.0f;
      if (mask_out) mask_out[t * E + j] = (uint8_t)s;
    }
    if (lane == 0 && count_out) count_out[t] = k;
    wave_sync_lds();
  }
}

int pp_route_impl(const void* x, int x_dtype, const float* logits_in, int64_t N, int H,
                  const float* router, const float* bias, int E, float tau, float* logits_out,
                  float* probs_out, float* gates_out, uint8_t* mask_out, int32_t* count_out,
                  bf16_t* xbf_out, hipStream_t st) {
  if (N == 0) return PP_OK;
  const int grid = (int)((N + ROUTE_TOK - 1) / ROUTE_TOK);
  const size_t smem = 0;
  const int threads = 256;
  if (logits_in) {
    route_kernel<float, true><<<grid, threads, smem, st>>>(nullptr, logits_in, N, H, router, bias, E, tau,
                                                       logits_out, probs_out, gates_out, mask_out,
                                                       count_out, nullptr);
  } else if (x_dtype == PP_DTYPE_F32) {
    route_kernel<float, false><<<grid, threads, smem, st>>>((const float*)x, nullptr, N, H, router, bias, E,
                                                        tau, logits_out, probs_out, gates_out, mask_out,
                                                        count_out, xbf_out);
  } else {
    route_kernel<bf16_t, false><<<grid, threads, smem, st>>>((const bf16_t*)x, nullptr, N, H, router, bias, E,
                                                         tau, logits_out, probs_out, gates_out, mask_out,
                                                         count_out, xbf_out);
  }
  return pp_check_launch("route_kernel");
}

extern "C" int pp_route(const void* x, int x_dtype, int64_t n_tokens, int H, const float* router_packed,
                        const float* bias, int E, float tau, float* logits_out, float* probs_out,
                        float* gates_out, uint8_t* mask_out, int32_t* count_out, void* stream) {
  int rc = pp_check_shape(H, E, 32);
  if (rc) return rc;
  PP_REQUIRE(n_tokens >= 0, PP_ERR_INVALID, "pp_route: n_tokens < 0");
  PP_REQUIRE(n_tokens == 0 || (x && router_packed), PP_ERR_INVALID, "pp_route: null x/router");
  PP_REQUIRE(x_dtype == PP_DTYPE_F32 || x_dtype == PP_DTYPE_BF16, PP_ERR_INVALID, "pp_route: x_dtype %d", x_dtype);
  return pp_route_impl(x, x_dtype, nullptr, n_tokens, H, router_packed, bias, E, tau, logits_out,
                       probs_out, gates_out, mask_out, count_out, nullptr, (hipStream_t)stream);
}

extern "C" int pp_route_logits(const float* logits, int64_t n_tokens, int E, float tau, float* probs_out,
                               float* gates_out, uint8_t* mask_out, int32_t* count_out, void* stream) {
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "num_experts E=%d unsupported (1..256)", E);
  PP_REQUIRE(n_tokens >= 0, PP_ERR_INVALID, "pp_route_logits: n_tokens < 0");
  PP_REQUIRE(n_tokens == 0 || logits, PP_ERR_INVALID, "pp_route_logits: null logits");
  return pp_route_impl(nullptr, PP_DTYPE_F32, logits, n_tokens, 128, nullptr, nullptr, E, tau, nullptr,
                       probs_out, gates_out, mask_out, count_out, nullptr, (hipStream_t)stream);
}

// ------------------------------------------------------------------ bucketing
#define BKT_TOK 256  // tokens per bucketing block

// Per 256-token block: count of selected tokens per expert.
__global__ __launch_bounds__(256) void bucket_count_kernel(const uint8_t* __restrict__ mask, int64_t N,
                                                           int E, int32_t* __restrict__ blkcnt) {
  __shared__ int wcnt[4][PP_MAX_EXPERTS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * BKT_TOK + threadIdx.x;
  const bool valid = t < N;
  for (int e = 0; e < E; ++e) {
    const bool m = valid && mask[t * E + e];
    const unsigned long long b = __ballot(m);
    if (lane == 0) wcnt[w][e] = __popcll(b);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256)
    blkcnt[(int64_t)blockIdx.x * E + e] = wcnt[0][e] + wcnt[1][e] + wcnt[2][e] + wcnt[3][e];
}

// One workgroup: expert totals, CSR offsets, per-block write offsets, GEMM tile map.
__global__ __launch_bounds__(256) void bucket_scan_kernel(const int32_t* __restrict__ blkcnt, int nblk,
                                                          int E, int tile_m, int32_t* __restrict__ blkoff,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ tiles,
                                                          int32_t* __restrict__ meta) {
  __shared__ int tot[PP_MAX_EXPERTS];
  __shared__ int ntl[PP_MAX_EXPERTS];
  __shared__ int off_s[PP_MAX_EXPERTS + 1];
  __shared__ int toff_s[PP_MAX_EXPERTS + 1];
  const int e = threadIdx.x;
  if (e < E) {
    int s = 0;
    for (int b = 0; b < nblk; ++b) s += blkcnt[(int64_t)b * E + e];
    tot[e] = s;
    ntl[e] = (s + tile_m - 1) / tile_m;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int o = 0, to = 0;
    for (int j = 0; j < E; ++j) {
      off_s[j] = o;
      toff_s[j] = to;
      o += tot[j];
      to += ntl[j];
    }
    off_s[E] = o;
    toff_s[E] = to;
    meta[0] = to;
    meta[1] = o;
    meta[2] = 0;
    meta[3] = 0;
  }
  __syncthreads();
  for (int j = threadIdx.x; j <= E; j += 256) offsets[j] = off_s[j];
  if (e < E) {
    int run = off_s[e];
    for (int b = 0; b < nblk; ++b) {
      blkoff[(int64_t)b * E + e] = run;
      run += blkcnt[(int64_t)b * E + e];
    }
    const int n = tot[e];
    for (int i = 0; i < ntl[e]; ++i) {
      int32_t* tp = tiles + (int64_t)(toff_s[e] + i) * 4;
      tp[0] = e;
      tp[1] = off_s[e] + i * tile_m;
      tp[2] = min(tile_m, n - i * tile_m);
      tp[3] = 0;
    }
  }
}

// Per 256-token block: write pairs in token order into each expert's segment.
__global__ __launch_bounds__(256) void bucket_scatter_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ gates, int64_t N, int E,
    const int32_t* __restrict__ blkoff, int32_t* __restrict__ token_ids, float* __restrict__ pair_gates,
    int32_t* __restrict__ token_pairs) {
  __shared__ unsigned long long bal[4][PP_MAX_EXPERTS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * BKT_TOK + threadIdx.x;
  const bool valid = t < N;
  for (int e = 0; e < E; ++e) {
    const bool m = valid && mask[t * E + e];
    const unsigned long long b = __ballot(m);
    if (lane == 0) bal[w][e] = b;
  }
  __syncthreads();
  if (!valid) return;
  const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int slot = 0;
  for (int e = 0; e < E; ++e) {
    const unsigned long long b = bal[w][e];
    if (!((b >> lane) & 1ull)) continue;
    int base = blkoff[(int64_t)blockIdx.x * E + e];
    for (int v = 0; v < w; ++v) base += __popcll(bal[v][e]);
    const int pos = base + __popcll(b & lt);
    token_ids[pos] = (int32_t)t;
    if (pair_gates) pair_gates[pos] = gates ? gates[t * E + e] : 0.0f;
    if (token_pairs) token_pairs[t * E + slot] = pos;
    ++slot;
  }
  if (token_pairs)
    for (int s = slot; s < E; ++s) token_pairs[t * E + s] = -1;
}

extern "C" size_t pp_bucket_workspace_bytes(int64_t n_tokens, int E) {
  int64_t nblk = (n_tokens + BKT_TOK - 1) / BKT_TOK;
  if (nblk < 1) nblk = 1;
  return (size_t)nblk * E * sizeof(int32_t) * 2;
}

extern "C" int pp_gemm_tile_m(void) { return 128; }

extern "C" int64_t pp_max_tiles(int64_t n_tokens, int E, int tile_m) {
  if (tile_m <= 0) return 0;
  // sum_e ceil(c_e / tile_m) <= (sum_e c_e) / tile_m + E, with sum_e c_e <= N*E
  return (n_tokens * E) / tile_m + E;
}

int pp_bucket_impl(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m,
                   int32_t* offsets, int32_t* token_ids, float* pair_gates, int32_t* token_pairs,
                   int32_t* tiles, int32_t* meta, void* workspace, hipStream_t st) {
  int64_t nblk = (N + BKT_TOK - 1) / BKT_TOK;
  int32_t* blkcnt = (int32_t*)workspace;
  int32_t* blkoff = blkcnt + (nblk < 1 ? 1 : nblk) * E;
  if (nblk > 0) bucket_count_kernel<<<(unsigned)nblk, 256, 0, st>>>(mask, N, E, blkcnt);
  bucket_scan_kernel<<<1, 256, 0, st>>>(blkcnt, (int)nblk, E, tile_m, blkoff, offsets, tiles, meta);
  if (nblk > 0)
    bucket_scatter_kernel<<<(unsigned)nblk, 256, 0, st>>>(mask, gates, N, E, blkoff, token_ids, pair_gates,
                                                          token_pairs);
  return pp_check_launch("pp_bucket");
}

extern "C" int pp_bucket(const uint8_t* mask, const float* gates, int64_t n_tokens, int E, int tile_m,
                         int32_t* offsets, int32_t* token_ids, float* pair_gates, int32_t* token_pairs,
                         int32_t* tiles, int32_t* meta, void* workspace, void* stream) {
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "num_experts E=%d unsupported (1..256)", E);
  PP_REQUIRE(n_tokens >= 0 && n_tokens <= (int64_t)0x7fffffff / PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED,
             "pp_bucket: n_tokens %lld out of range", (long long)n_tokens);
  PP_REQUIRE(tile_m >= 1, PP_ERR_INVALID, "pp_bucket: tile_m %d", tile_m);
  PP_REQUIRE(offsets && tiles && meta && workspace, PP_ERR_INVALID, "pp_bucket: null output/workspace");
  PP_REQUIRE(n_tokens == 0 || (mask && token_ids), PP_ERR_INVALID, "pp_bucket: null mask/token_ids");
  return pp_bucket_impl(mask, gates, n_tokens, E, tile_m, offsets, token_ids, pair_gates, token_pairs, tiles,
                        meta, workspace, (hipStream_t)stream);
}
