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
#include "gemm_lds.h"

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

template <typename XT, bool FROM_LOGITS, bool SELECT = true>
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
    // logits-only launches give each group of 64 experts its own workgroup (blockIdx.y)
    const int tg_lo = SELECT ? 0 : 4 * (int)blockIdx.y;
    const int tg_hi = SELECT ? ntile : min(ntile, tg_lo + 4);
    for (int tg = tg_lo; tg < tg_hi; tg += 4) {
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
  if (!SELECT) {  // logits only, of this workgroup's 64 experts (the selection runs elsewhere)
    for (int i = tid; i < ROUTE_TOK * ROUTE_EGRP; i += 256) {
      const int rr = i / ROUTE_EGRP, e = 64 * (int)blockIdx.y + i % ROUTE_EGRP;
      const int64_t t = tok0 + rr;
      if (t < N && e < E) logits_out[t * E + e] = lg_s[rr][e];
    }
    return;
  }

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

// Selection for E > 64, one token per workgroup of 256 threads: the workgroup selection
// of the E > 16 decode (select_one_token_wg: keys sorted per wave, ranks by merging,
// parallel exact cut; the same result as select_one_token, pinned on the same golden
// families), about 3 us per token where one wave ranking E = 192 experts alone takes
// tens of us. Reads the token's logits (bias already added), writes probs, gates, mask
// and count. A selection whose ranks are not a permutation (never, for a correct sort)
// writes NaN probs and gates and count 0 rather than a plausible wrong routing.
__global__ __launch_bounds__(256) void route_select_wg_kernel(const float* __restrict__ logits, int64_t N, int E,
                                                              float tau, float* __restrict__ logits_copy,
                                                              float* __restrict__ probs_out,
                                                              float* __restrict__ gates_out,
                                                              uint8_t* __restrict__ mask_out,
                                                              int32_t* __restrict__ count_out) {
  __shared__ SelScratch ss;
  __shared__ unsigned long long keys_s[PP_MAX_EXPERTS];
  __shared__ float lg_s[PP_MAX_EXPERTS];
  __shared__ float red_s[4];
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.x;
  if (t >= N) return;  // uniform
  if (tid < E) {
    lg_s[tid] = logits[t * E + tid];
    if (logits_copy) logits_copy[t * E + tid] = lg_s[tid];
  }
  __syncthreads();
  select_one_token_wg([&](int j) { return lg_s[j]; }, E, tau, &ss, keys_s, red_s, tid, 256);
  const bool bad = ss.bad != 0;
  const int k = bad ? 0 : ss.k;
  if (tid < E) ss.sel[tid] = 0;
  __syncthreads();
  if (tid < k) ss.sel[ss.order[tid]] = 1;
  __syncthreads();
  if (tid < E) {
    const bool s = ss.sel[tid] != 0;
    if (probs_out) probs_out[t * E + tid] = bad ? __builtin_nanf("") : ss.e[tid];
    if (gates_out) gates_out[t * E + tid] = bad ? __builtin_nanf("") : (s ? pp_sigmoid(lg_s[tid]) : 0.0f);
    if (mask_out) mask_out[t * E + tid] = (uint8_t)s;
  }
  if (tid == 0 && count_out) count_out[t] = k;
}

// ------------------------------------------------------------------ E = 16 fast path
// 16 tokens x 16 experts per workgroup of 8 waves. x and the router pass through LDS in
// K chunks of RT16_KC (four stages, DMA three chunks ahead), loaded as whole rows -- one
// 1 KB row (or two 512-byte bf16 rows) per instruction, so a load touches a few cache
// lines instead of sixteen: the per-CU address path, not bandwidth, bounded loads that
// took sixteen rows x 64 bytes per instruction. 16-byte chunk c of LDS row r sits at
// position c ^ r, so the sixteen rows of a fragment read land in distinct bank slots.
// Wave w takes the 32-wide K block w of every chunk; lane (t = l % 16, g = l / 16) holds
// x[t][k + 8g + j] and W[expert l % 16][k + 8g + j], j = 0..7, one fp32 MFMA per j
// (chain j % 4), then the four chains are added in order and the eight wave partials in
// wave order through LDS (fixed order: deterministic logits). Selection: four tokens per
// wave at once, one per 16-lane group, branch-free, same arithmetic as select_small<16>
// (torch's sort is stable for E <= 16, so rank = number of (greater, or equal with
// smaller index)).
#define RT16_WAVES 8
#define RT16_KC 256
#define RT16_STAGES 4
#define RT16_RROW (RT16_KC * 4)  // router row bytes in a stage
template <typename XT>
struct Rt16 {
  static constexpr int XROW = RT16_KC * (int)sizeof(XT);  // x row bytes in a stage
  static constexpr int STAGE = 16 * (XROW + RT16_RROW);
  static constexpr int DMA = sizeof(XT) == 4 ? 4 : 3;     // DMA instructions per wave per stage
};

__device__ __forceinline__ void rt16_dma(const void* src, unsigned char* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void rt16_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// DMA of K chunk k0 .. k0 + kw into stage st: x rows of the workgroup's 16 tokens (rows
// past N repeat row N - 1), then the 16 router rows. Chunks past kw load chunk 0 (in
// range, never read).
template <typename XT>
__device__ __forceinline__ void rt16_issue(const XT* __restrict__ x, const float* __restrict__ router, int64_t N,
                                           int H, int64_t tok0, int k0, int kw, unsigned char* st, int w, int lane) {
  if (sizeof(XT) == 4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // x rows 2w, 2w + 1: 64 chunks of 4 floats
      const int r = 2 * w + h;
      const int c = lane ^ r;
      const int64_t t = min(tok0 + r, N - 1);
      rt16_dma(x + t * H + k0 + 4 * (c < kw / 4 ? c : 0), st + r * Rt16<XT>::XROW);
    }
  } else {  // x rows 2w (lanes 0..31), 2w + 1 (lanes 32..63): 32 chunks of 8 bf16
    const int r = 2 * w + (lane >> 5);
    const int c = (lane & 31) ^ r;
    const int64_t t = min(tok0 + r, N - 1);
    rt16_dma(x + t * H + k0 + 8 * (c < kw / 8 ? c : 0), st + 2 * w * Rt16<XT>::XROW);
  }
  unsigned char* rs = st + 16 * Rt16<XT>::XROW;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // router rows 2w, 2w + 1
    const int e = 2 * w + h;
    const int c = lane ^ e;
    rt16_dma(router + (int64_t)e * H + k0 + 4 * (c < kw / 4 ? c : 0), rs + e * RT16_RROW);
  }
}

// ---- selection: wave w, group q4 = lane / 16 -> token 4 w + q4, lane j = expert
__device__ __forceinline__ void route16_select(const float (*lg_s)[16], float (*ev_s)[16], float (*srt_s)[16],
                                               int* cnt_s, int64_t tok0, int64_t N, float tau, int lane, int w,
                                               float* __restrict__ logits_out, float* __restrict__ probs_out,
                                               float* __restrict__ gates_out, uint8_t* __restrict__ mask_out,
                                               int32_t* __restrict__ count_out) {
  const int rr = 4 * w + (lane >> 4), j = lane & 15;
  const int64_t t = tok0 + rr;
  const float xl = lg_s[rr][j];
  const float m = row16_max(xl);  // order-free: the same value as the xor butterfly
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
    if (s) atomicAdd(&cnt_s[j], 1);
  }
}

template <typename XT>
__global__ __launch_bounds__(64 * RT16_WAVES) void route16_kernel(
    const XT* __restrict__ x, int64_t N, int H, const float* __restrict__ router, const float* __restrict__ bias,
    float tau, float* __restrict__ logits_out, float* __restrict__ probs_out, float* __restrict__ gates_out,
    uint8_t* __restrict__ mask_out, int32_t* __restrict__ count_out, bf16_t* __restrict__ xbf_out,
    int32_t* __restrict__ blkcnt_out) {
  __shared__ __align__(16) float part[RT16_WAVES][16][16];
  __shared__ __align__(16) float lg_s[16][16];
  __shared__ __align__(16) float ev_s[16][16];
  __shared__ __align__(16) float srt_s[16][16];
  __shared__ int cnt_s[16];  // selections per expert over this workgroup's 16 tokens
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t tok0 = (int64_t)blockIdx.x * 16;
  if (tid < 16) cnt_s[tid] = 0;
  {
    __shared__ __align__(16) unsigned char stg[RT16_STAGES * Rt16<XT>::STAGE];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)stg;
    const int t_l = lane & 15, g = lane >> 4;
    const int nst = (H + RT16_KC - 1) / RT16_KC;
    auto chunk_w = [&](int sidx) { return min(RT16_KC, H - sidx * RT16_KC); };
    f32x4_t acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sidx = 0; sidx < RT16_STAGES - 1; ++sidx)
      if (sidx < nst)
        rt16_issue<XT>(x, router, N, H, tok0, sidx * RT16_KC, chunk_w(sidx), stg + sidx * Rt16<XT>::STAGE, w, lane);
    for (int sidx = 0; sidx < nst; ++sidx) {
      // chunk sidx has landed when at most the DMA of the chunks issued after it is
      // outstanding (loads complete in order; the x stores in between only make it stricter)
      if (sidx + 2 < nst) rt16_wait_barrier<2 * Rt16<XT>::DMA>();
      else if (sidx + 1 < nst) rt16_wait_barrier<Rt16<XT>::DMA>();
      else rt16_wait_barrier<0>();
      // LDS reads through asm (lds_read16): ordered after this chunk's DMAs by the wait and
      // barrier above, and not made to wait for the later chunks' DMAs still in flight
      const uint32_t sb = lds0 + (uint32_t)((sidx % RT16_STAGES) * Rt16<XT>::STAGE);
      const int kw = chunk_w(sidx);
      // x as bf16 for the grouped GEMMs (fp32 x only): thread -> row tid / 32, 8 values
      if (sizeof(XT) == 4 && xbf_out) {
        const int r = tid >> 5, k8 = (tid & 31) * 8;
        const int64_t t = tok0 + r;
        if (t < N && k8 < kw) {
          u32x4 v0 = lds_read16(sb + r * Rt16<XT>::XROW + (((k8 >> 2) ^ r) << 4));
          u32x4 v1 = lds_read16(sb + r * Rt16<XT>::XROW + ((((k8 >> 2) + 1) ^ r) << 4));
          lds_wait_all(v0, v1);
          uint4 pk;
          pk.x = (uint32_t)f32_to_bf16(__uint_as_float(v0.x)) | ((uint32_t)f32_to_bf16(__uint_as_float(v0.y)) << 16);
          pk.y = (uint32_t)f32_to_bf16(__uint_as_float(v0.z)) | ((uint32_t)f32_to_bf16(__uint_as_float(v0.w)) << 16);
          pk.z = (uint32_t)f32_to_bf16(__uint_as_float(v1.x)) | ((uint32_t)f32_to_bf16(__uint_as_float(v1.y)) << 16);
          pk.w = (uint32_t)f32_to_bf16(__uint_as_float(v1.z)) | ((uint32_t)f32_to_bf16(__uint_as_float(v1.w)) << 16);
          *(uint4*)(xbf_out + t * H + sidx * RT16_KC + k8) = pk;
        }
      }
      if (sidx + RT16_STAGES - 1 < nst)
        rt16_issue<XT>(x, router, N, H, tok0, (sidx + RT16_STAGES - 1) * RT16_KC, chunk_w(sidx + RT16_STAGES - 1),
                       stg + ((sidx + RT16_STAGES - 1) % RT16_STAGES) * Rt16<XT>::STAGE, w, lane);
      if (32 * w < kw) {  // this wave's K block of the chunk
        float xv[8], wv8[8];
        const int c0 = 8 * w + 2 * g;
        u32x4 xq[2], wq[2];
        if (sizeof(XT) == 4) {
          xq[0] = lds_read16(sb + t_l * Rt16<XT>::XROW + ((c0 ^ t_l) << 4));
          xq[1] = lds_read16(sb + t_l * Rt16<XT>::XROW + (((c0 + 1) ^ t_l) << 4));
        } else {
          xq[0] = lds_read16(sb + t_l * Rt16<XT>::XROW + (((4 * w + g) ^ t_l) << 4));
        }
        const uint32_t rs = sb + 16 * Rt16<XT>::XROW + t_l * RT16_RROW;  // expert row l % 16
        wq[0] = lds_read16(rs + ((c0 ^ t_l) << 4));
        wq[1] = lds_read16(rs + (((c0 + 1) ^ t_l) << 4));
        if constexpr (sizeof(XT) == 4) lds_wait_all(xq[0], xq[1], wq[0], wq[1]);
        else lds_wait_all(xq[0], wq[0], wq[1]);
        if (sizeof(XT) == 4) {
#pragma unroll
          for (int i = 0; i < 8; ++i) xv[i] = __uint_as_float(xq[i >> 2][i & 3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xv[2 * i] = __uint_as_float(xq[0][i] << 16);
            xv[2 * i + 1] = __uint_as_float(xq[0][i] & 0xffff0000u);
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) wv8[i] = __uint_as_float(wq[i >> 2][i & 3]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j], wv8[j], acc[j & 3], 0, 0, 0);
      }
    }
    // lane l, element q: token 4 (l / 16) + q, expert l % 16
#pragma unroll
    for (int q = 0; q < 4; ++q)
      part[w][4 * g + q][t_l] = __fadd_rn(__fadd_rn(__fadd_rn(acc[0][q], acc[1][q]), acc[2][q]), acc[3][q]);
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
  if (w < 4) route16_select(lg_s, ev_s, srt_s, cnt_s, tok0, N, tau, lane, w, logits_out, probs_out, gates_out,
                            mask_out, count_out);
  if (blkcnt_out) {  // per-block expert counts for the bucketing (blocks of 16 tokens)
    __syncthreads();
    if (tid < 16) blkcnt_out[(int64_t)blockIdx.x * 16 + tid] = cnt_s[tid];
  }
}

// ---- few tokens (E = 16, N <= RT_FEW_MAX_N, H = 512 CPL with CPL <= 4). route16_kernel
// runs such batches on one or four workgroups, each walking the whole K loop at one
// CU's load rate (~10 us at 16 tokens). Here a workgroup takes RT_FEW_TOK tokens: it
// reads the router once and x of its tokens straight into registers (8 waves; wave w
// takes the K slice w of 8, lane (row, col) of 4 x 16 the experts row + 4 i and the
// float4 chunks col + 16 c of the slice), rows add by DPP, the eight wave partials add
// in wave order (fixed order: deterministic logits); wave 0 runs route16_select with
// group g = token g. The counts go out per RT_FEW_TOK-token block.
#define RT_FEW_TOK 4
#define RT_FEW_MAX_N 64
template <typename XT, int CPL>
__global__ __launch_bounds__(512) void route16_few_kernel(
    const XT* __restrict__ x, int64_t N, const float* __restrict__ router, const float* __restrict__ bias,
    float tau, float* __restrict__ logits_out, float* __restrict__ probs_out, float* __restrict__ gates_out,
    uint8_t* __restrict__ mask_out, int32_t* __restrict__ count_out, bf16_t* __restrict__ xbf_out,
    int32_t* __restrict__ blkcnt_out) {
  constexpr int H = 512 * CPL, NW = 8, T = RT_FEW_TOK;
  __shared__ __align__(16) float part_s[T][16][NW];
  __shared__ __align__(16) float lg_s[16][16];
  __shared__ __align__(16) float ev_s[16][16];
  __shared__ __align__(16) float srt_s[16][16];
  __shared__ int cnt_s[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t tok0 = (int64_t)blockIdx.x * T;
  const int64_t tok_end = min(N, tok0 + T);
  if (tid < 16) cnt_s[tid] = 0;
  const int rw = lane >> 4, cl = lane & 15;
  const int ch0 = 16 * CPL * wv + cl;  // float4 chunk of x / of a router row
  float4 xv[T][CPL], wr[4][CPL];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t row = min(tok0 + t, N - 1);  // rows past N repeat row N - 1, never stored
#pragma unroll
    for (int c = 0; c < CPL; ++c) xv[t][c] = load_x4<XT>(x, row * H + 4 * (ch0 + 16 * c));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < CPL; ++c) wr[i][c] = *(const float4*)(router + (rw + 4 * i) * H + 4 * (ch0 + 16 * c));
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.0f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        s = __builtin_fmaf(xv[t][c].x, wr[i][c].x, s);
        s = __builtin_fmaf(xv[t][c].y, wr[i][c].y, s);
        s = __builtin_fmaf(xv[t][c].z, wr[i][c].z, s);
        s = __builtin_fmaf(xv[t][c].w, wr[i][c].w, s);
      }
      s = row16_sum(s);
      if (cl == 0) part_s[t][rw + 4 * i][wv] = s;
    }
  // x as bf16 for the grouped GEMMs (fp32 x only): lanes of row rw store token rw
  // (static token index per store: a register array indexed by rw would go to scratch)
  if (sizeof(XT) == 4 && xbf_out && tok0 + rw < N) {
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (rw == t)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const float4 v = xv[t][c];
          uint2 pk;
          pk.x = (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
          pk.y = (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
          *(uint2*)(xbf_out + (tok0 + t) * H + 4 * (ch0 + 16 * c)) = pk;
        }
  }
  __syncthreads();
  if (tid < 16 * T) {
    const int t = tid >> 4, e = tid & 15;
    const float4 p0 = *(const float4*)&part_s[t][e][0];
    const float4 p1 = *(const float4*)&part_s[t][e][4];
    float l = p0.x;
    l = __fadd_rn(l, p0.y);
    l = __fadd_rn(l, p0.z);
    l = __fadd_rn(l, p0.w);
    l = __fadd_rn(l, p1.x);
    l = __fadd_rn(l, p1.y);
    l = __fadd_rn(l, p1.z);
    l = __fadd_rn(l, p1.w);
    if (bias) l = __fadd_rn(l, bias[e]);
    lg_s[t][e] = l;
  }
  __syncthreads();
  if (wv == 0)
    route16_select(lg_s, ev_s, srt_s, cnt_s, tok0, tok_end, tau, lane, 0, logits_out, probs_out, gates_out,
                   mask_out, count_out);
  if (blkcnt_out) {
    __syncthreads();
    if (tid < 16) blkcnt_out[(int64_t)blockIdx.x * 16 + tid] = cnt_s[tid];
  }
}

// Tokens per count block of the E = 16 router kernels (0: the kernel writes no counts).
static bool route_few_fits(int64_t N, int H) { return N <= RT_FEW_MAX_N && H % 512 == 0 && H <= 2048; }
int pp_route_count_block(int64_t N, int H, int E) {
  if (E != 16) return 0;
  return route_few_fits(N, H) ? RT_FEW_TOK : 16;
}

template <typename XT>
static void launch_route_few(const XT* x, int64_t N, int H, const float* router, const float* bias, float tau,
                             float* logits_out, float* probs_out, float* gates_out, uint8_t* mask_out,
                             int32_t* count_out, bf16_t* xbf_out, int32_t* blkcnt_out, hipStream_t st) {
  const unsigned g = (unsigned)((N + RT_FEW_TOK - 1) / RT_FEW_TOK);
#define PP_FEW(C)                                                                                               \
  route16_few_kernel<XT, C><<<g, 512, 0, st>>>(x, N, router, bias, tau, logits_out, probs_out, gates_out,      \
                                               mask_out, count_out, xbf_out, blkcnt_out)
  switch (H / 512) {
    case 1: PP_FEW(1); break;
    case 2: PP_FEW(2); break;
    case 3: PP_FEW(3); break;
    default: PP_FEW(4); break;
  }
#undef PP_FEW
}

// blkcnt_out (E = 16 path only, else untouched): per block of pp_route_count_block
// tokens, per expert, the number of selections -- the bucketing's block counts, so it
// needs no counting pass.
int pp_route_logits_dense(const void* x, int x_dtype, int64_t N, int H, const float* router, const float* bias,
                          int E, float* logits_out, bf16_t* xbf_out, uint32_t* zero, int nzero, hipStream_t st);

int pp_route_impl(const void* x, int x_dtype, const float* logits_in, int64_t N, int H,
                  const float* router, const float* bias, int E, float tau, float* logits_out,
                  float* probs_out, float* gates_out, uint8_t* mask_out, int32_t* count_out,
                  bf16_t* xbf_out, hipStream_t st, int32_t* blkcnt_out) {
  if (N == 0) return PP_OK;
  const int grid = (int)((N + ROUTE_TOK - 1) / ROUTE_TOK);
  const size_t smem = 0;
  const int threads = 256;
  if (!logits_in && E == 16 && route_few_fits(N, H)) {
    if (x_dtype == PP_DTYPE_F32)
      launch_route_few<float>((const float*)x, N, H, router, bias, tau, logits_out, probs_out, gates_out, mask_out,
                              count_out, xbf_out, blkcnt_out, st);
    else
      launch_route_few<bf16_t>((const bf16_t*)x, N, H, router, bias, tau, logits_out, probs_out, gates_out,
                               mask_out, count_out, xbf_out, blkcnt_out, st);
    return pp_check_launch("route16_few_kernel");
  }
  if (!logits_in && E == 16) {
    const int g16 = (int)((N + 15) / 16);
    if (x_dtype == PP_DTYPE_F32)
      route16_kernel<float><<<g16, 64 * RT16_WAVES, 0, st>>>((const float*)x, N, H, router, bias, tau, logits_out,
                                                            probs_out, gates_out, mask_out, count_out, xbf_out,
                                                            blkcnt_out);
    else
      route16_kernel<bf16_t><<<g16, 64 * RT16_WAVES, 0, st>>>((const bf16_t*)x, N, H, router, bias, tau,
                                                             logits_out, probs_out, gates_out, mask_out,
                                                             count_out, xbf_out, blkcnt_out);
    return pp_check_launch("route16_kernel");
  }
  if (!logits_in && logits_out) {
    // E != 16 with a logits buffer: the LDS-staged logits pass (one fixed summation order
    // per (token, expert), the prefill's own router), then the selection from those logits
    int rc = pp_route_logits_dense(x, x_dtype, N, H, router, bias, E, logits_out, xbf_out, nullptr, 0, st);
    if (rc) return rc;
    logits_in = logits_out;
    logits_out = nullptr;
  }
  if (E > 64 && logits_in) {  // one token per workgroup
    const float* lg = logits_in;
    float* lcopy = (logits_out && logits_out != logits_in) ? logits_out : nullptr;
    for (int64_t t0 = 0; t0 < N; t0 += 65535) {
      const int64_t n = N - t0 < 65535 ? N - t0 : 65535;
      route_select_wg_kernel<<<(unsigned)n, 256, 0, st>>>(lg + t0 * E, n, E, tau, lcopy ? lcopy + t0 * E : nullptr,
                                                          probs_out ? probs_out + t0 * E : nullptr,
                                                          gates_out ? gates_out + t0 * E : nullptr,
                                                          mask_out ? mask_out + t0 * E : nullptr,
                                                          count_out ? count_out + t0 : nullptr);
    }
    return pp_check_launch("route_select_wg_kernel");
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
                       probs_out, gates_out, mask_out, count_out, nullptr, (hipStream_t)stream, nullptr);
}

extern "C" int pp_route_logits(const float* logits, int64_t n_tokens, int E, float tau, float* probs_out,
                               float* gates_out, uint8_t* mask_out, int32_t* count_out, void* stream) {
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "num_experts E=%d unsupported (1..256)", E);
  PP_REQUIRE(n_tokens >= 0, PP_ERR_INVALID, "pp_route_logits: n_tokens < 0");
  PP_REQUIRE(n_tokens == 0 || logits, PP_ERR_INVALID, "pp_route_logits: null logits");
  return pp_route_impl(nullptr, PP_DTYPE_F32, logits, n_tokens, 128, nullptr, nullptr, E, tau, nullptr,
                       probs_out, gates_out, mask_out, count_out, nullptr, (hipStream_t)stream, nullptr);
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
  // the block's mask bytes as 32-bit words (the block starts at byte t0 * E, a multiple
  // of 64 E, so words are aligned); the first words are loaded before the LDS clearing
  // and its barrier, and every word of a batch before the first LDS update
  const int64_t nt = min((int64_t)BKT_TOK, N - t0);
  const int nb = (int)nt * E, nw = (nb + 3) >> 2;
  const uint32_t* mw = (const uint32_t*)(mask + t0 * E);
  uint32_t v[4];
  auto load4 = [&](int w0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int wi = w0 + q * BKT_THREADS + threadIdx.x;
      v[q] = wi < nw ? mw[wi] : 0u;
    }
  };
  load4(0);
  for (int e = threadIdx.x; e < E; e += BKT_THREADS) tokw[e] = 0ull;
  for (int l = threadIdx.x; l < BKT_TOK * BKT_QW; l += BKT_THREADS) expw[l / BKT_QW][l % BKT_QW] = 0ull;
  __syncthreads();
  for (int w0 = 0; w0 < nw; w0 += 4 * BKT_THREADS) {
    if (w0) load4(w0);
    // rolled on purpose: the instruction cache is cold at launch, code size is latency
#pragma unroll 1
    for (int k = 0; k < 16; ++k) {
      const int q = k >> 2, by = k & 3;
      const int i = 4 * (w0 + q * BKT_THREADS + threadIdx.x) + by;
      const uint32_t vq = q == 0 ? v[0] : q == 1 ? v[1] : q == 2 ? v[2] : v[3];
      if (i < nb && ((vq >> (8 * by)) & 0xffu)) {
        const int l = i / E, e = i - l * E;
        atomicOr(&tokw[e], 1ull << l);
        atomicOr(&expw[l][e >> 6], 1ull << (e & 63));
      }
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

// Exclusive prefixes over experts of the pair totals (CSR offsets) and of their
// row-tile counts (tile-map offsets); thread e < E holds expert e's total, the others
// pass 0. One shuffle scan per wave (only as many steps as E needs), earlier waves'
// sums through LDS. Fills off_s / toff_s [E + 1]; every thread of the block calls it;
// ends on a barrier. blockDim.x == BKT_THREADS, E <= BKT_THREADS.
__device__ __forceinline__ void bucket_expert_scan(int tot, int E, int tile_m, int* off_s, int* toff_s) {
  __shared__ int wsum_s[2][BKT_THREADS / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nt = (tot + tile_m - 1) / tile_m;
  int ip = tot, it = nt;
  const int span = min(E, 64);
  for (int d = 1; d < span; d <<= 1) {
    const int vp = __shfl_up(ip, d), vt = __shfl_up(it, d);
    if (lane >= d) {
      ip += vp;
      it += vt;
    }
  }
  if (E > 64) {  // several waves hold experts
    if (lane == 63) {
      wsum_s[0][w] = ip;
      wsum_s[1][w] = it;
    }
    __syncthreads();
    for (int v = 0; v < w; ++v) {
      ip += wsum_s[0][v];
      it += wsum_s[1][v];
    }
  }
  if (tid < E) {
    off_s[tid] = ip - tot;
    toff_s[tid] = it - nt;
  }
  if (tid == E - 1) {
    off_s[E] = ip;
    toff_s[E] = it;
  }
  __syncthreads();
}

// Row-tile map from the scanned offsets: tile i of expert e is {e, first pair, rows,
// 0}; BKT_THREADS / E threads per expert take its tiles in turn.
__device__ __forceinline__ void bucket_write_tiles(int E, int tile_m, const int* off_s, const int* toff_s,
                                                   int32_t* __restrict__ tiles) {
  const int G = BKT_THREADS / E;  // >= 1
  if ((int)threadIdx.x < G * E) {
    const int g = threadIdx.x / E, e = threadIdx.x - g * E;
    const int o = off_s[e], ne = off_s[e + 1] - o, t0 = toff_s[e], nt = toff_s[e + 1] - t0;
    for (int i = g; i < nt; i += G) {
      int32_t* tp = tiles + (int64_t)(t0 + i) * 4;
      tp[0] = e;
      tp[1] = o + i * tile_m;
      tp[2] = min(tile_m, ne - i * tile_m);
      tp[3] = 0;
    }
  }
}

// One workgroup: expert totals, CSR offsets, per-block write offsets, GEMM tile map.
__global__ __launch_bounds__(256) void bucket_scan_kernel(const int32_t* __restrict__ blkcnt, int nblk,
                                                          int E, int tile_m, int32_t* __restrict__ blkoff,
                                                          int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ tiles,
                                                          int32_t* __restrict__ meta,
                                                          uint32_t* __restrict__ zero, int nzero) {
  __shared__ int off_s[PP_MAX_EXPERTS + 1];
  for (int i = threadIdx.x; i < nzero; i += 256) zero[i] = 0u;
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
  bucket_expert_scan(e < E ? s : 0, E, tile_m, off_s, toff_s);
  if (threadIdx.x == 0) {
    meta[0] = toff_s[E];
    meta[1] = off_s[E];
    meta[2] = 0;
    meta[3] = 0;
  }
  for (int j = threadIdx.x; j <= E; j += 256) offsets[j] = off_s[j];
  bucket_write_tiles(E, tile_m, off_s, toff_s, tiles);
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
}

__device__ __forceinline__ int popc_below(const unsigned long long* w, int bit) {
  int c = 0;
  for (int q = 0; q < (bit >> 6); ++q) c += __popcll(w[q]);
  const int r = bit & 63;
  if (r) c += __popcll(w[bit >> 6] & (~0ull >> (64 - r)));
  return c;
}

// Placement of the pairs of block blockIdx.x once its selection words are in LDS: four
// consecutive pairs per thread step (their gates as one 16-byte load when aligned).
// The gates of pairs 4i .. 4i+3 of the block (zeros past the block's end).
__device__ __forceinline__ float4 bucket_gate4(const float* __restrict__ gates, int64_t t0, int E, int nb, int i0) {
  float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i0 + 4 <= nb) {
    g = *(const float4*)(gates + t0 * E + i0);
  } else {
    if (i0 + 0 < nb) g.x = gates[t0 * E + i0 + 0];
    if (i0 + 1 < nb) g.y = gates[t0 * E + i0 + 1];
    if (i0 + 2 < nb) g.z = gates[t0 * E + i0 + 2];
  }
  return g;
}

// g_first: this thread's first gate quad (pairs 4 tid ..), loaded by the caller early.
__device__ __forceinline__ void bucket_scatter_pairs(const float* __restrict__ gates, int64_t N, int E,
                                                     const int* base_s, int32_t* __restrict__ token_ids,
                                                     float* __restrict__ pair_gates,
                                                     int32_t* __restrict__ token_pairs,
                                                     const unsigned long long* tokw,
                                                     const unsigned long long (*expw)[BKT_QW], float4 g_first) {
  const int64_t t0 = (int64_t)blockIdx.x * BKT_TOK;
  const int64_t nt = min((int64_t)BKT_TOK, N - t0);
  const int nb = (int)nt * E;
  for (int i0 = 4 * threadIdx.x; i0 < nb; i0 += 4 * BKT_THREADS) {
    float4 g = g_first;
    if (i0 != 4 * (int)threadIdx.x && gates && pair_gates) g = bucket_gate4(gates, t0, E, nb, i0);
#pragma unroll 1
    for (int by = 0; by < 4; ++by) {
      const int i = i0 + by;
      if (i >= nb) break;
      const int l = i / E, e = i - l * E;
      const int64_t t = t0 + l;
      const unsigned long long* ew = expw[l];
      const bool sel = (ew[e >> 6] >> (e & 63)) & 1ull;
      const int below = popc_below(ew, e);  // selected experts of this token below e
      if (sel) {
        const int pos = base_s[e] + (l ? __popcll(tokw[e] & (~0ull >> (64 - l))) : 0);
        token_ids[pos] = (int32_t)t;
        if (pair_gates) pair_gates[pos] = by == 0 ? g.x : by == 1 ? g.y : by == 2 ? g.z : g.w;
        if (token_pairs) token_pairs[t * E + below] = pos;
      } else if (token_pairs) {
        int cnt = 0;
        for (int q = 0; q < BKT_QW; ++q) cnt += __popcll(ew[q]);
        token_pairs[t * E + cnt + (e - below)] = -1;  // unselected experts fill the tail in order
      }
    }
  }
}

// Block blockIdx.x of BKT_TOK tokens: pair (l, e) -> position base_s[e] + (tokens of
// the block below l that selected e); base_s is read after the barrier inside
// bucket_block_words.
__device__ __forceinline__ void bucket_scatter_block(const uint8_t* __restrict__ mask,
                                                     const float* __restrict__ gates, int64_t N, int E,
                                                     const int* base_s, int32_t* __restrict__ token_ids,
                                                     float* __restrict__ pair_gates,
                                                     int32_t* __restrict__ token_pairs, unsigned long long* tokw,
                                                     unsigned long long (*expw)[BKT_QW]) {
  const int64_t t0 = (int64_t)blockIdx.x * BKT_TOK;
  const int nb = (int)min((int64_t)BKT_TOK, N - t0) * E;
  const float4 g_first = (gates && pair_gates) ? bucket_gate4(gates, t0, E, nb, 4 * threadIdx.x)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
  bucket_block_words(mask, N, E, t0, tokw, expw);
  bucket_scatter_pairs(gates, N, E, base_s, token_ids, pair_gates, token_pairs, tokw, expw, g_first);
}

__global__ __launch_bounds__(BKT_THREADS) void bucket_scatter_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ gates, int64_t N, int E,
    const int32_t* __restrict__ blkoff, int32_t* __restrict__ token_ids, float* __restrict__ pair_gates,
    int32_t* __restrict__ token_pairs) {
  __shared__ unsigned long long tokw[PP_MAX_EXPERTS];
  __shared__ unsigned long long expw[BKT_TOK][BKT_QW];
  __shared__ int base_s[PP_MAX_EXPERTS];
  for (int e = threadIdx.x; e < E; e += BKT_THREADS) base_s[e] = blkoff[(int64_t)blockIdx.x * E + e];
  bucket_scatter_block(mask, gates, N, E, base_s, token_ids, pair_gates, token_pairs, tokw, expw);
}

// Scan and scatter in one kernel when the block-count table is small (nblk_c * E <=
// BKT_PLACE_INTS): every workgroup stages the whole table (counts per block of cb
// tokens, cb dividing BKT_TOK) in LDS and computes the expert totals, the CSR offsets
// and its own blocks' bases itself -- a few KB of L2 reads per workgroup instead of a
// serial scan kernel between counting and scattering. Workgroup 0 also writes the CSR
// offsets, the tile map and meta, as bucket_scan_kernel does. Same layout bit for bit.
#define BKT_PLACE_INTS 8192
__global__ __launch_bounds__(BKT_THREADS) void bucket_place_kernel(
    const uint8_t* __restrict__ mask, const float* __restrict__ gates, int64_t N, int E,
    const int32_t* __restrict__ blkcnt, int cb, int nblk_c, int tile_m, int32_t* __restrict__ offsets,
    int32_t* __restrict__ token_ids, float* __restrict__ pair_gates, int32_t* __restrict__ token_pairs,
    int32_t* __restrict__ tiles, int32_t* __restrict__ meta, uint32_t* __restrict__ zero, int nzero) {
  __shared__ int cnt_s[BKT_PLACE_INTS];
  __shared__ int part_tot[BKT_THREADS], part_pre[BKT_THREADS];
  __shared__ int base_s[PP_MAX_EXPERTS];
  __shared__ int off_s[PP_MAX_EXPERTS + 1], toff_s[PP_MAX_EXPERTS + 1];
  __shared__ unsigned long long tokw[PP_MAX_EXPERTS];
  __shared__ unsigned long long expw[BKT_TOK][BKT_QW];
  const int tid = threadIdx.x;
  const int n = nblk_c * E;
  // independent loads first: the start of the count table, this thread's first gate
  // quad; the mask words follow inside bucket_block_words, all in one round trip
  int cv[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = tid + q * BKT_THREADS;
    cv[q] = i < n ? blkcnt[i] : 0;
  }
  const int64_t t0 = (int64_t)blockIdx.x * BKT_TOK;
  const bool has_tokens = t0 < N;
  const int nb = has_tokens ? (int)min((int64_t)BKT_TOK, N - t0) * E : 0;
  const float4 g_first = (has_tokens && gates && pair_gates) ? bucket_gate4(gates, t0, E, nb, 4 * tid)
                                                             : make_float4(0.f, 0.f, 0.f, 0.f);
  if (has_tokens) bucket_block_words(mask, N, E, t0, tokw, expw);  // has barriers
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = tid + q * BKT_THREADS;
    if (i < n) cnt_s[i] = cv[q];
  }
  for (int i = tid + 8 * BKT_THREADS; i < n; i += BKT_THREADS) cnt_s[i] = blkcnt[i];
  __syncthreads();
  // thread (g, e): column e of blocks g, g + G, ...; totals and the prefix before this
  // workgroup's first count block
  const int G = BKT_THREADS / E;  // >= 1 (E <= 256)
  const int c_first = (int)(((int64_t)blockIdx.x * BKT_TOK) / cb);
  if (tid < G * E) {
    const int g = tid / E, e = tid - g * E;
    int tot = 0, pre = 0;
#pragma unroll 4
    for (int c = g; c < nblk_c; c += G) {
      const int v = cnt_s[c * E + e];
      tot += v;
      pre += c < c_first ? v : 0;
    }
    part_tot[tid] = tot;
    part_pre[tid] = pre;
  }
  __syncthreads();
  int tot = 0, pre = 0;  // expert tid's column total and prefix
  if (tid < E) {
#pragma unroll 4
    for (int g = 0; g < G; ++g) {
      tot += part_tot[g * E + tid];
      pre += part_pre[g * E + tid];
    }
  }
  bucket_expert_scan(tot, E, tile_m, off_s, toff_s);  // ends on a barrier
  if (tid < E) base_s[tid] = off_s[tid] + pre;
  if (blockIdx.x == 0) {
    for (int i = tid; i < nzero; i += BKT_THREADS) zero[i] = 0u;
    for (int e = tid; e <= E; e += BKT_THREADS) offsets[e] = off_s[e];
    if (tid == 0) {
      meta[0] = toff_s[E];
      meta[1] = off_s[E];
      meta[2] = 0;
      meta[3] = 0;
    }
    bucket_write_tiles(E, tile_m, off_s, toff_s, tiles);
  }
  if (!has_tokens) return;  // N == 0: only the offsets / tile map
  __syncthreads();         // base_s
  bucket_scatter_pairs(gates, N, E, base_s, token_ids, pair_gates, token_pairs, tokw, expw, g_first);
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

// zero[0 .. nzero) (may be null): words the caller needs cleared before its next kernel
// (the prefill GEMMs' split sync words); workgroup 0 of the place / scan kernel clears them.
// Bucketing from block counts already made (cb tokens per count block, cb | BKT_TOK):
// one place kernel when the count table is small, else the scan + scatter pair (the
// scatter needs BKT_TOK-token block bases, summed from the cb-token counts by the scan
// only when cb == BKT_TOK -- callers with finer counts use the place path only).
static bool bucket_place_fits(int64_t nblk_c, int E) { return nblk_c * E <= BKT_PLACE_INTS; }

int pp_bucket_from_counts(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m,
                          const int32_t* blkcnt, int cb, int32_t* offsets, int32_t* token_ids, float* pair_gates,
                          int32_t* token_pairs, int32_t* tiles, int32_t* meta, hipStream_t st, uint32_t* zero,
                          int nzero) {
  const int64_t nblk_c = (N + cb - 1) / cb;
  const int64_t nblk = (N + BKT_TOK - 1) / BKT_TOK;
  bucket_place_kernel<<<(unsigned)(nblk > 0 ? nblk : 1), BKT_THREADS, 0, st>>>(
      mask, gates, N, E, blkcnt, cb, (int)nblk_c, tile_m, offsets, token_ids, pair_gates, token_pairs, tiles, meta,
      zero, zero ? nzero : 0);
  return pp_check_launch("pp_bucket");
}

int pp_bucket_impl(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m,
                   int32_t* offsets, int32_t* token_ids, float* pair_gates, int32_t* token_pairs,
                   int32_t* tiles, int32_t* meta, void* workspace, hipStream_t st, uint32_t* zero, int nzero) {
  int64_t nblk = (N + BKT_TOK - 1) / BKT_TOK;
  int32_t* blkcnt = (int32_t*)workspace;
  int32_t* blkoff = blkcnt + (nblk < 1 ? 1 : nblk) * E;
  if (nblk > 0) bucket_count_kernel<<<(unsigned)nblk, BKT_THREADS, 0, st>>>(mask, N, E, blkcnt);
  if (bucket_place_fits(nblk, E))
    return pp_bucket_from_counts(mask, gates, N, E, tile_m, blkcnt, BKT_TOK, offsets, token_ids, pair_gates,
                                 token_pairs, tiles, meta, st, zero, nzero);
  bucket_scan_kernel<<<1, 256, 0, st>>>(blkcnt, (int)nblk, E, tile_m, blkoff, offsets, tiles, meta, zero,
                                        zero ? nzero : 0);
  if (nblk > 0)
    bucket_scatter_kernel<<<(unsigned)nblk, BKT_THREADS, 0, st>>>(mask, gates, N, E, blkoff, token_ids, pair_gates,
                                                          token_pairs);
  return pp_check_launch("pp_bucket");
}

// Whether pp_bucket_from_counts can take the router kernel's cb-token counts for N tokens.
bool pp_bucket_counts_fit(int64_t N, int E, int cb) { return cb > 0 && bucket_place_fits((N + cb - 1) / cb, E); }

extern "C" int pp_bucket(const uint8_t* mask, const float* gates, int64_t n_tokens, int E, int tile_m,
                         int32_t* offsets, int32_t* token_ids, float* pair_gates, int32_t* token_pairs,
                         int32_t* tiles, int32_t* meta, void* workspace, void* stream) {
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "num_experts E=%d unsupported (1..256)", E);
  PP_REQUIRE(n_tokens >= 0 && n_tokens <= (int64_t)0x7fffffff / PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED,
             "pp_bucket: n_tokens %lld out of range", (long long)n_tokens);
  PP_REQUIRE(tile_m >= 1, PP_ERR_INVALID, "pp_bucket: tile_m %d", tile_m);
  PP_REQUIRE(offsets && tiles && meta && workspace, PP_ERR_INVALID, "pp_bucket: null output/workspace");
  PP_REQUIRE(n_tokens == 0 || (mask && token_ids), PP_ERR_INVALID, "pp_bucket: null mask/token_ids");
  PP_REQUIRE(((uintptr_t)mask & 3) == 0 && ((uintptr_t)gates & 3) == 0, PP_ERR_INVALID,
             "pp_bucket: mask must be 4-byte aligned (read as 32-bit words)");
  return pp_bucket_impl(mask, gates, n_tokens, E, tile_m, offsets, token_ids, pair_gates, token_pairs, tiles,
                        meta, workspace, (hipStream_t)stream, nullptr, 0);
}
