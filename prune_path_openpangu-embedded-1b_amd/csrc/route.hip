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

// ------------------------------------------------------------------ E = 16 fast path
// 16 tokens x 16 experts per workgroup of 8 waves. Wave w owns the contiguous K slice
// [w H/8, (w+1) H/8) and issues all of its x and router loads before the first MFMA
// (RT16_CHUNK 16-wide K blocks at a time, the next chunk in flight under the current
// one); the four float4 components feed four independent MFMA chains, added in
// component order, then the eight wave partials are added in wave order through LDS
// (fixed order: deterministic logits). Selection: four tokens per wave at once, one
// per 16-lane group, branch-free, same arithmetic as select_small<16> (torch's sort is
// stable for E <= 16, so rank = number of (greater, or equal with smaller index)).
#define RT16_WAVES 8
#define RT16_CHUNK 8

template <typename XT>
__device__ __forceinline__ void rt16_load(const XT* __restrict__ x, const float* __restrict__ router, int64_t t,
                                          bool valid, int H, int kb0, int nkb, int r, int g, float4 (&xa)[RT16_CHUNK],
                                          float4 (&wa)[RT16_CHUNK]) {
#pragma unroll
  for (int i = 0; i < RT16_CHUNK; ++i) {
    const int kk = (kb0 + i) * 16 + 4 * g;
    const bool in = i < nkb;
    xa[i] = (in && valid) ? load_x4<XT>(x, t * H + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
    wa[i] = in ? *(const float4*)(router + (int64_t)r * H + kk) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

template <typename XT>
__global__ __launch_bounds__(64 * RT16_WAVES) void route16_kernel(
    const XT* __restrict__ x, int64_t N, int H, const float* __restrict__ router, const float* __restrict__ bias,
    float tau, float* __restrict__ logits_out, float* __restrict__ probs_out, float* __restrict__ gates_out,
    uint8_t* __restrict__ mask_out, int32_t* __restrict__ count_out, bf16_t* __restrict__ xbf_out) {
  __shared__ __align__(16) float part[RT16_WAVES][16][16];
  __shared__ __align__(16) float lg_s[16][16];
  __shared__ __align__(16) float ev_s[16][16];
  __shared__ __align__(16) float srt_s[16][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t tok0 = (int64_t)blockIdx.x * 16;
  {
    const int r = lane & 15, g = lane >> 4;
    const int64_t t = tok0 + r;
    const bool valid = t < N;
    const int nkb_w = H / (16 * RT16_WAVES);  // 16-wide K blocks per wave
    const int kbase = w * nkb_w;
    f32x4_t acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    float4 xa[RT16_CHUNK], wa[RT16_CHUNK], xn[RT16_CHUNK], wn[RT16_CHUNK];
    rt16_load<XT>(x, router, t, valid, H, kbase, nkb_w, r, g, xa, wa);
    for (int c0 = 0; c0 < nkb_w; c0 += RT16_CHUNK) {
      const int left = nkb_w - c0 - RT16_CHUNK;
      if (left > 0) rt16_load<XT>(x, router, t, valid, H, kbase + c0 + RT16_CHUNK, left, r, g, xn, wn);
#pragma unroll
      for (int i = 0; i < RT16_CHUNK; ++i) {
        if (c0 + i < nkb_w) {
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i].x, wa[i].x, acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i].y, wa[i].y, acc[1], 0, 0, 0);
          acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i].z, wa[i].z, acc[2], 0, 0, 0);
          acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[i].w, wa[i].w, acc[3], 0, 0, 0);
          if (xbf_out && valid) {
            uint2 pk;
            pk.x = (uint32_t)f32_to_bf16(xa[i].x) | ((uint32_t)f32_to_bf16(xa[i].y) << 16);
            pk.y = (uint32_t)f32_to_bf16(xa[i].z) | ((uint32_t)f32_to_bf16(xa[i].w) << 16);
            *(uint2*)(xbf_out + t * H + (kbase + c0 + i) * 16 + 4 * g) = pk;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < RT16_CHUNK; ++i) { xa[i] = xn[i]; wa[i] = wn[i]; }
    }
    // lane l, element q: token 4 (l / 16) + q, expert l % 16
#pragma unroll
    for (int q = 0; q < 4; ++q)
      part[w][4 * g + q][r] = __fadd_rn(__fadd_rn(__fadd_rn(acc[0][q], acc[1][q]), acc[2][q]), acc[3][q]);
  }
  __syncthreads();
  if (tid < 256) {
    const int rr = tid >> 4, e = tid & 15;
    float l = part[0][rr][e];
#pragma unroll
    for (int ww = 1; ww < RT16_WAVES; ++ww) l = __fadd_rn(l, part[ww][rr][e]);
    if (bias) l = __fadd_rn(l, bias[e]);
    lg_s[rr][e] = l;
  }
  __syncthreads();
  if (w >= 4) return;
  // ---- selection: wave w, group q4 = lane / 16 -> token 4 w + q4, lane j = expert
  const int rr = 4 * w + (lane >> 4), j = lane & 15;
  const int64_t t = tok0 + rr;
  const float xl = lg_s[rr][j];
  float m = xl;
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, PP_WAVE));
  const float e = pp_expf_u10(__fsub_rn(xl, m));
  ev_s[rr][j] = e;
  wave_sync_lds();
  float ev[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = *(const float4*)&ev_s[rr][4 * i];
    ev[4 * i] = v.x; ev[4 * i + 1] = v.y; ev[4 * i + 2] = v.z; ev[4 * i + 3] = v.w;
  }
  float a8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a8[i] = __fadd_rn(ev[i], ev[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) a8[i] = __fadd_rn(a8[i], a8[i + 4]);
#pragma unroll
  for (int i = 0; i < 2; ++i) a8[i] = __fadd_rn(a8[i], a8[i + 2]);
  const float rs = __fdiv_rn(1.0f, __fadd_rn(a8[0], a8[1]));
  const float p = __fmul_rn(e, rs);
  int rank = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const float pq = __fmul_rn(ev[q], rs);
    rank += (kv_before(pq, p) || (pq == p && q < j)) ? 1 : 0;
  }
  srt_s[rr][rank] = p;
  wave_sync_lds();
  float sv[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = *(const float4*)&srt_s[rr][4 * i];
    sv[4 * i] = v.x; sv[4 * i + 1] = v.y; sv[4 * i + 2] = v.z; sv[4 * i + 3] = v.w;
  }
  // (float) of the fp64 running sum is non-decreasing: the ranks with cum < tau are a
  // prefix, so counting them gives k (NaN compares false from its rank on)
  const float tau32 = tau;
  double a = 0.0;
  int k = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    a += (double)sv[q];
    k += ((float)a < tau32) ? 1 : 0;
  }
  k = k > 0 ? k : 1;
  if (t < N) {
    const bool s = rank < k;
    if (logits_out) logits_out[t * 16 + j] = xl;
    if (probs_out) probs_out[t * 16 + j] = p;
    if (gates_out) gates_out[t * 16 + j] = s ? pp_sigmoid(xl) : 0.0f;
    if (mask_out) mask_out[t * 16 + j] = (uint8_t)s;
    if (count_out && j == 0) count_out[t] = k;
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
  if (!logits_in && E == 16) {
    const int g16 = (int)((N + 15) / 16);
    if (x_dtype == PP_DTYPE_F32)
      route16_kernel<float><<<g16, 64 * RT16_WAVES, 0, st>>>((const float*)x, N, H, router, bias, tau, logits_out,
                                                            probs_out, gates_out, mask_out, count_out, xbf_out);
    else
      route16_kernel<bf16_t><<<g16, 64 * RT16_WAVES, 0, st>>>((const bf16_t*)x, N, H, router, bias, tau,
                                                             logits_out, probs_out, gates_out, mask_out,
                                                             count_out, xbf_out);
    return pp_check_launch("route16_kernel");
  }
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
// Blocks of BKT_TOK = 64 tokens; every (token, expert) pair of a block is one work
// item (pair i -> token i / E, expert i % E, so the mask and gate loads are coalesced
// and independent). A block summarises its selections as bit words in LDS:
//   tokw[e]     bit l set when token l of the block selected expert e,
//   expw[l][q]  bit e' = e - 64 q set when token l selected expert e.
// count:   per (block, expert) totals = popcount(tokw[e]);
// scan:    one workgroup: expert offsets, per-block bases, GEMM tile map;
// scatter: pair (l, e) -> position base[b][e] + popcount(tokw[e] below l) inside
//          expert e's segment (tokens ascending), slot = number of the token's
//          selected experts below e; the token's unselected slots are set to -1.
#define BKT_TOK 64
#define BKT_THREADS 256
#define BKT_QW (PP_MAX_EXPERTS / 64)
#define BKT_SCAN_CHUNK 8192  // ints of block counts staged in LDS at a time

__device__ __forceinline__ void bucket_block_words(const uint8_t* __restrict__ mask, int64_t N, int E, int64_t t0,
                                                   unsigned long long* tokw, unsigned long long (*expw)[BKT_QW]) {
  for (int e = threadIdx.x; e < E; e += BKT_THREADS) tokw[e] = 0ull;
  for (int l = threadIdx.x; l < BKT_TOK * BKT_QW; l += BKT_THREADS) expw[l / BKT_QW][l % BKT_QW] = 0ull;
  __syncthreads();
  const int pairs = BKT_TOK * E;
  for (int i = threadIdx.x; i < pairs; i += BKT_THREADS) {
    const int l = i / E, e = i - l * E;
    const int64_t t = t0 + l;
    if (t < N && mask[t * E + e]) {
      atomicOr(&tokw[e], 1ull << l);
      atomicOr(&expw[l][e >> 6], 1ull << (e & 63));
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(BKT_THREADS) void bucket_count_kernel(const uint8_t* __restrict__ mask, int64_t N,
                                                                   int E, int32_t* __restrict__ blkcnt) {
  __shared__ unsigned long long tokw[PP_MAX_EXPERTS];
  __shared__ unsigned long long expw[BKT_TOK][BKT_QW];
  bucket_block_words(mask, N, E, (int64_t)blockIdx.x * BKT_TOK, tokw, expw);
  for (int e = threadIdx.x; e < E; e += BKT_THREADS) blkcnt[(int64_t)blockIdx.x * E + e] = __popcll(tokw[e]);
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
  __shared__ int cnt_s[BKT_SCAN_CHUNK];
  const int e = threadIdx.x;
  // block counts pass through LDS in coalesced chunks of whole blocks, so the
  // per-expert loops below read LDS instead of one dependent load per block
  const int cb = BKT_SCAN_CHUNK / E;  // blocks per chunk
  int s = 0;
  for (int b0 = 0; b0 < nblk; b0 += cb) {
    const int nb = min(cb, nblk - b0);
    __syncthreads();
    for (int i = threadIdx.x; i < nb * E; i += 256) cnt_s[i] = blkcnt[(int64_t)b0 * E + i];
    __syncthreads();
    if (e < E)
      for (int b = 0; b < nb; ++b) s += cnt_s[b * E + e];
  }
  if (e < E) {
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
  int run = e < E ? off_s[e] : 0;
  for (int b0 = 0; b0 < nblk; b0 += cb) {
    const int nb = min(cb, nblk - b0);
    __syncthreads();
    for (int i = threadIdx.x; i < nb * E; i += 256) cnt_s[i] = blkcnt[(int64_t)b0 * E + i];
    __syncthreads();
    if (e < E)
      for (int b = 0; b < nb; ++b) {
        const int c = cnt_s[b * E + e];
        cnt_s[b * E + e] = run;  // this expert's column only: no other thread touches it
        run += c;
      }
    __syncthreads();
    for (int i = threadIdx.x; i < nb * E; i += 256) blkoff[(int64_t)b0 * E + i] = cnt_s[i];
  }
  for (int j = 0; j < E; ++j) {  // tile i of expert j
    const int n = tot[j];
    for (int i = threadIdx.x; i < ntl[j]; i += 256) {
      int32_t* tp = tiles + (int64_t)(toff_s[j] + i) * 4;
      tp[0] = j;
      tp[1] = off_s[j] + i * tile_m;
      tp[2] = min(tile_m, n - i * tile_m);
      tp[3] = 0;
    }
  }
}

__device__ __forceinline__ int popc_below(const unsigned long long* w, int bit) {
  int c = 0;
  for (int q = 0; q < (bit >> 6); ++q) c += __popcll(w[q]);
  const int r = bit & 63;
  if (r) c += __popcll(w[bit >> 6] & (~0ull >> (64 - r)));
  return c;
}

__global__ __launch_bounds__(BKT_THREADS) void bucket_scatter_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ gates, int64_t N, int E,
    const int32_t* __restrict__ blkoff, int32_t* __restrict__ token_ids, float* __restrict__ pair_gates,
    int32_t* __restrict__ token_pairs) {
  __shared__ unsigned long long tokw[PP_MAX_EXPERTS];
  __shared__ unsigned long long expw[BKT_TOK][BKT_QW];
  __shared__ int base_s[PP_MAX_EXPERTS];
  const int64_t t0 = (int64_t)blockIdx.x * BKT_TOK;
  for (int e = threadIdx.x; e < E; e += BKT_THREADS) base_s[e] = blkoff[(int64_t)blockIdx.x * E + e];
  bucket_block_words(mask, N, E, t0, tokw, expw);
  const int pairs = BKT_TOK * E;
  for (int i = threadIdx.x; i < pairs; i += BKT_THREADS) {
    const int l = i / E, e = i - l * E;
    const int64_t t = t0 + l;
    if (t >= N) break;  // pairs of later tokens are later too
    const unsigned long long* ew = expw[l];
    const bool sel = (ew[e >> 6] >> (e & 63)) & 1ull;
    const int below = popc_below(ew, e);  // selected experts of this token below e
    if (sel) {
      const int pos = base_s[e] + (l ? __popcll(tokw[e] & (~0ull >> (64 - l))) : 0);
      token_ids[pos] = (int32_t)t;
      if (pair_gates) pair_gates[pos] = gates ? gates[t * E + e] : 0.0f;
      if (token_pairs) token_pairs[t * E + below] = pos;
    } else if (token_pairs) {
      int cnt = 0;
      for (int q = 0; q < BKT_QW; ++q) cnt += __popcll(ew[q]);
      token_pairs[t * E + cnt + (e - below)] = -1;  // unselected experts fill the tail in order
    }
  }
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
  if (nblk > 0) bucket_count_kernel<<<(unsigned)nblk, BKT_THREADS, 0, st>>>(mask, N, E, blkcnt);
  bucket_scan_kernel<<<1, 256, 0, st>>>(blkcnt, (int)nblk, E, tile_m, blkoff, offsets, tiles, meta);
  if (nblk > 0)
    bucket_scatter_kernel<<<(unsigned)nblk, BKT_THREADS, 0, st>>>(mask, gates, N, E, blkoff, token_ids, pair_gates,
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
