// Prefill / N > 1: grouped expert GEMMs on the bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Replaces moe_fused_expert_kernel (src/tl_kernel_optimized_Ultimate_PanGU.py:271-328) and
// the TauSparseMoE.forward_prefill orchestration (:532-604). The reference runs one
// 16-token tile per program, computes gate/up/down per tile and scatters with bf16
// atomics; here the pairs of one expert are cut into 128-row tiles and:
//   gateup_kernel  act[p, n] = silu(x[tok(p)] . Wg[n]) * (x[tok(p)] . Wu[n]) * gate[p]
//                  (gathered A rows, gate and up neurons in one B tile so the SwiGLU
//                  epilogue has both in the same lane), bf16 act [P][G];
//   down_kernel    y[p, h] = act[p] . Wd[:, h] over the expert's G neurons, fp32 y [P][H]
//                  (a bf16 y would add up to ~2e-3 absolute error per output after the
//                  k-term combine -- enough to break atol 2e-3 on small outputs);
//   combine_kernel out[t] = sum of y over the pairs of token t in expert order, fp32 ->
//                  bf16 (deterministic, no atomics).
// Both GEMMs are persistent over a device-side tile map (no host sync, no padding FLOPs
// beyond the last partial tile of each expert), 256 threads = 4 waves, BK = 64, LDS
// tiles double-buffered with a 16-byte row pad (conflict-free 16-byte fragment reads).
#include "pp_common.h"

#define GM_THREADS 256
#define GM_BK 64
#define GM_LDK (GM_BK + 8)  // padded LDS row (bf16 elements)
#define GM_BM 128

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x16_t mfma32(const uint4 a, const uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// D layout of the 32x32 MFMA: lane l, element q -> row (q/4)*8 + (l/32)*4 + q%4, col l%32.
__device__ __forceinline__ int mfma32_row(int q, int lane) { return (q >> 2) * 8 + (lane >> 5) * 4 + (q & 3); }

typedef bf16_t lds_row_t[GM_LDK];

// Chunk i of a thread covers tile row (tid >> 3) + 32 * i, columns kcol .. kcol + 7.
template <int N>
__device__ __forceinline__ void lds_put(lds_row_t* tile, int row0, int kcol, const uint4 (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) *(uint4*)&tile[row0 + 32 * i][kcol] = v[i];
}

// Gathered rows: src row index per chunk (-1 = padding row, loads zeros).
template <int N>
__device__ __forceinline__ void gmem_rows(const bf16_t* __restrict__ base, const int (&row)[N], int ld, int k,
                                          uint4 (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] = row[i] >= 0 ? *(const uint4*)(base + (int64_t)row[i] * ld + k) : make_uint4(0, 0, 0, 0);
}

// ------------------------------------------------------------------ gate/up + SwiGLU
// Tile: 128 pair rows x NB neurons (gate block and up block of the same NB neurons).
// Waves: WM x WN; wave (wm, wn) owns rows wm*TM*32.. and neurons wn*32..+32.
template <int WM, int WN, int TM>
__global__ __launch_bounds__(GM_THREADS, 2) void gateup_kernel(
    const bf16_t* __restrict__ xb, int H, int G, const bf16_t* __restrict__ wrows,
    const int32_t* __restrict__ token_ids, const float* __restrict__ pair_gates,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, bf16_t* __restrict__ act) {
  static_assert(WM * WN == 4 && WM * TM * 32 == GM_BM, "tile shape");
  constexpr int NB = WN * 32;
  constexpr int BROWS = 2 * NB;
  constexpr int A_CH = GM_BM * (GM_BK / 8) / GM_THREADS;  // 16-byte chunks per thread
  constexpr int B_CH = BROWS * (GM_BK / 8) / GM_THREADS;
  __shared__ __align__(16) bf16_t As[2][GM_BM][GM_LDK];
  __shared__ __align__(16) bf16_t Bs[2][BROWS][GM_LDK];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w / WN, wn = w % WN;
  const int n_ntile = G / NB;
  const int n_items = meta[0] * n_ntile;
  const int nkb = H / GM_BK;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int t = item / n_ntile, nt = item % n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int nb0 = nt * NB;

    // per-thread source rows of the A and B chunks (32-bit indices; -1 = padding row)
    int arow[A_CH];
    int brec[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + GM_THREADS * i, r = c >> 3;
      arow[i] = r < rows ? token_ids[p0 + r] : -1;
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + GM_THREADS * i, r = c >> 3;
      const int part = r < NB ? 0 : 1;
      brec[i] = (e * G + nb0 + (r % NB)) * 3 + part;
    }
    const int kcol = (tid & 7) * 8;  // same for every chunk of this thread
    uint4 ra[A_CH], rb[B_CH];
    const int row0 = tid >> 3;
#define GU_GLOAD(kb)                                                \
  {                                                                 \
    gmem_rows<A_CH>(xb, arow, H, (kb) * GM_BK + kcol, ra);           \
    gmem_rows<B_CH>(wrows, brec, H, (kb) * GM_BK + kcol, rb);        \
  }
#define GU_SSTORE(buf)                                              \
  {                                                                 \
    lds_put<A_CH>(As[buf], row0, kcol, ra);                         \
    lds_put<B_CH>(Bs[buf], row0, kcol, rb);                         \
  }

    f32x16_t accg[TM], accu[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int q = 0; q < 16; ++q) { accg[i][q] = 0.0f; accu[i][q] = 0.0f; }
    }

    GU_GLOAD(0);
    GU_SSTORE(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
      const int cur = kb & 1;
      if (kb + 1 < nkb) GU_GLOAD(kb + 1);
#pragma unroll
      for (int ks = 0; ks < GM_BK / 16; ++ks) {
        const int kc = ks * 16 + (lane >> 5) * 8;
        const uint4 bg = *(const uint4*)&Bs[cur][wn * 32 + (lane & 31)][kc];
        const uint4 bu = *(const uint4*)&Bs[cur][NB + wn * 32 + (lane & 31)][kc];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const uint4 a = *(const uint4*)&As[cur][wm * TM * 32 + i * 32 + (lane & 31)][kc];
          accg[i] = mfma32(a, bg, accg[i]);
          accu[i] = mfma32(a, bu, accu[i]);
        }
      }
      if (kb + 1 < nkb) GU_SSTORE(cur ^ 1);
      __syncthreads();
    }
#undef GU_GLOAD
#undef GU_SSTORE

    // epilogue: SwiGLU with the pair's router gate, bf16 act
    const int neuron = nb0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = wm * TM * 32 + i * 32 + mfma32_row(q, lane);
        if (r < rows) {
          const int p = p0 + r;
          const float a = pp_silu(accg[i][q]) * accu[i][q] * pair_gates[p];
          act[(int64_t)p * G + neuron] = f32_to_bf16(a);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ down projection
// Tile: 128 pair rows x 128 hidden columns; waves 2 x 2, each 64 x 64 (2 x 2 MFMA blocks).
__global__ __launch_bounds__(GM_THREADS, 2) void down_kernel(
    const bf16_t* __restrict__ act, int H, int G, const bf16_t* __restrict__ down_t,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, float* __restrict__ y) {
  constexpr int BN = 128;
  constexpr int A_CH = GM_BM * (GM_BK / 8) / GM_THREADS;  // 4
  constexpr int B_CH = BN * (GM_BK / 8) / GM_THREADS;     // 4
  __shared__ __align__(16) bf16_t As[2][GM_BM][GM_LDK];
  __shared__ __align__(16) bf16_t Bs[2][BN][GM_LDK];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int n_ntile = H / BN;
  const int n_items = meta[0] * n_ntile;
  const int nkb = (G + GM_BK - 1) / GM_BK;

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int t = item / n_ntile, nt = item % n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int h0 = nt * BN;
    const int kcol = (tid & 7) * 8;  // same for every chunk of this thread
    const int rbase = tid >> 3;        // chunk i covers row rbase + 32*i
    uint4 ra[A_CH], rb[B_CH];
    int arow[A_CH], brow[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int r = rbase + 32 * i;
      arow[i] = r < rows ? p0 + r : -1;
      brow[i] = e * H + h0 + r;
    }
    // rows of the last partial k-block beyond G read zeros: with G % 32 == 0 a chunk is
    // either fully inside or fully outside
#define DN_GLOAD(kb)                                                                      \
  {                                                                                       \
    const int k_ = (kb) * GM_BK + kcol;                                                   \
    if (k_ < G) {                                                                         \
      gmem_rows<A_CH>(act, arow, G, k_, ra);                                              \
      gmem_rows<B_CH>(down_t, brow, G, k_, rb);                                           \
    } else {                                                                              \
      _Pragma("unroll") for (int i = 0; i < A_CH; ++i) ra[i] = rb[i] = make_uint4(0, 0, 0, 0); \
    }                                                                                     \
  }
#define DN_SSTORE(buf)                                                                    \
  {                                                                                       \
    lds_put<A_CH>(As[buf], rbase, kcol, ra);                                              \
    lds_put<B_CH>(Bs[buf], rbase, kcol, rb);                                              \
  }
    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    DN_GLOAD(0);
    DN_SSTORE(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
      const int cur = kb & 1;
      if (kb + 1 < nkb) DN_GLOAD(kb + 1);
#pragma unroll
      for (int ks = 0; ks < GM_BK / 16; ++ks) {
        const int kc = ks * 16 + (lane >> 5) * 8;
        uint4 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = *(const uint4*)&As[cur][wm * 64 + i * 32 + (lane & 31)][kc];
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = *(const uint4*)&Bs[cur][wn * 64 + j * 32 + (lane & 31)][kc];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
      }
      if (kb + 1 < nkb) DN_SSTORE(cur ^ 1);
      __syncthreads();
    }
#undef DN_GLOAD
#undef DN_SSTORE
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int h = h0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int r = wm * 64 + i * 32 + mfma32_row(q, lane);
          if (r < rows) y[(int64_t)(p0 + r) * H + h] = acc[i][j][q];
        }
      }
    }
  }
}

// ------------------------------------------------------------------ combine
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y,
                                                      const int32_t* __restrict__ token_pairs,
                                                      const int32_t* __restrict__ count, int64_t N, int H,
                                                      int E, bf16_t* __restrict__ out) {
  const int HC = H >> 3;
  const int64_t total = N * HC;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / HC;
    const int ch = (int)(i % HC);
    float4 s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0;
    const int k = min(count[t], E);
    for (int q = 0; q < k; ++q) {
      const int p = token_pairs[t * E + q];
      if (p < 0) break;  // fewer pairs than count: inconsistent caller data, never read out of range
      const float4* src = (const float4*)(y + (int64_t)p * H + ch * 8);
      const float4 a = src[0], b = src[1];
      s0.x += a.x; s0.y += a.y; s0.z += a.z; s0.w += a.w;
      s1.x += b.x; s1.y += b.y; s1.z += b.z; s1.w += b.w;
    }
    uint4 o;
    o.x = (uint32_t)f32_to_bf16(s0.x) | ((uint32_t)f32_to_bf16(s0.y) << 16);
    o.y = (uint32_t)f32_to_bf16(s0.z) | ((uint32_t)f32_to_bf16(s0.w) << 16);
    o.z = (uint32_t)f32_to_bf16(s1.x) | ((uint32_t)f32_to_bf16(s1.y) << 16);
    o.w = (uint32_t)f32_to_bf16(s1.z) | ((uint32_t)f32_to_bf16(s1.w) << 16);
    *(uint4*)(out + t * H + ch * 8) = o;
  }
}

// ------------------------------------------------------------------ host side
static int gemm_grid(int64_t items) {
  int64_t g = 2 * (int64_t)pp_device_cus();
  if (items < g) g = items;
  return (int)(g < 1 ? 1 : g);
}

static int gateup_launch(const bf16_t* xb, int H, int G, const bf16_t* wrows, int E, const int32_t* token_ids,
                         const float* pair_gates, const int32_t* tiles, const int32_t* meta, int64_t max_tiles,
                         bf16_t* act, hipStream_t st) {
  (void)E;
  if (G % 64 == 0) {
    int grid = gemm_grid(max_tiles * (G / 64));
    gateup_kernel<2, 2, 2><<<grid, GM_THREADS, 0, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles, meta, act);
  } else {
    int grid = gemm_grid(max_tiles * (G / 32));
    gateup_kernel<4, 1, 1><<<grid, GM_THREADS, 0, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles, meta, act);
  }
  return pp_check_launch("gateup_kernel");
}

static int down_launch(const bf16_t* act, int H, int G, const bf16_t* down_t, const int32_t* tiles,
                       const int32_t* meta, int64_t max_tiles, float* y, hipStream_t st) {
  int grid = gemm_grid(max_tiles * (H / 128));
  down_kernel<<<grid, GM_THREADS, 0, st>>>(act, H, G, down_t, tiles, meta, y);
  return pp_check_launch("down_kernel");
}

static int combine_launch(const float* y, const int32_t* token_pairs, const int32_t* count, int64_t N, int H,
                          int E, bf16_t* out, hipStream_t st) {
  if (N == 0) return PP_OK;
  int64_t total = N * (H / 8);
  int64_t grid = (total + 255) / 256;
  if (grid > 65536) grid = 65536;
  combine_kernel<<<(unsigned)grid, 256, 0, st>>>(y, token_pairs, count, N, H, E, out);
  return pp_check_launch("combine_kernel");
}

extern "C" int pp_expert_gateup(const void* x_bf16, int H, int G, const void* packed, int E,
                                const int32_t* token_ids, const float* pair_gates, const int32_t* tiles,
                                const int32_t* meta, int64_t max_tiles, void* act_bf16, void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(x_bf16 && packed && token_ids && pair_gates && tiles && meta && act_bf16, PP_ERR_INVALID,
             "pp_expert_gateup: null pointer");
  PP_REQUIRE(max_tiles >= 0, PP_ERR_INVALID, "pp_expert_gateup: max_tiles < 0");
  if (max_tiles == 0) return PP_OK;
  return gateup_launch((const bf16_t*)x_bf16, H, G, (const bf16_t*)packed, E, token_ids, pair_gates, tiles, meta,
                       max_tiles, (bf16_t*)act_bf16, (hipStream_t)stream);
}

extern "C" int pp_expert_down(const void* act_bf16, int H, int G, const void* packed, int E, const int32_t* tiles,
                              const int32_t* meta, int64_t max_tiles, float* y_f32, void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(act_bf16 && packed && tiles && meta && y_f32, PP_ERR_INVALID, "pp_expert_down: null pointer");
  PP_REQUIRE(max_tiles >= 0, PP_ERR_INVALID, "pp_expert_down: max_tiles < 0");
  if (max_tiles == 0) return PP_OK;
  const bf16_t* down_t = (const bf16_t*)packed + (int64_t)E * G * 3 * H;
  return down_launch((const bf16_t*)act_bf16, H, G, down_t, tiles, meta, max_tiles, (float*)y_f32,
                     (hipStream_t)stream);
}

extern "C" int pp_combine(const float* y_f32, const int32_t* token_pairs, const int32_t* count, int64_t n_tokens,
                          int H, int E, void* out_bf16, void* stream) {
  int rc = pp_check_shape(H, E, 32);
  if (rc) return rc;
  PP_REQUIRE(n_tokens >= 0, PP_ERR_INVALID, "pp_combine: n_tokens < 0");
  PP_REQUIRE(n_tokens == 0 || (y_f32 && token_pairs && count && out_bf16), PP_ERR_INVALID,
             "pp_combine: null pointer");
  return combine_launch(y_f32, token_pairs, count, n_tokens, H, E, (bf16_t*)out_bf16, (hipStream_t)stream);
}

// ------------------------------------------------------------------ whole prefill
int pp_route_impl(const void* x, int x_dtype, const float* logits_in, int64_t N, int H, const float* router,
                  const float* bias, int E, float tau, float* logits_out, float* probs_out, float* gates_out,
                  uint8_t* mask_out, int32_t* count_out, bf16_t* xbf_out, hipStream_t st);
int pp_bucket_impl(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m, int32_t* offsets,
                   int32_t* token_ids, float* pair_gates, int32_t* token_pairs, int32_t* tiles, int32_t* meta,
                   void* workspace, hipStream_t st);

struct PrefillWs {
  size_t gates, mask, count, offsets, token_ids, pair_gates, token_pairs, tiles, meta, bws, xbf, act, y, total;
};

static PrefillWs prefill_layout(int64_t N, int H, int E, int G) {
  PrefillWs L;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  const int64_t P = N * E;
  const int64_t mt = pp_max_tiles(N, E, GM_BM);
  L.gates = take((size_t)P * 4);
  L.mask = take((size_t)P);
  L.count = take((size_t)N * 4);
  L.offsets = take((size_t)(E + 1) * 4);
  L.token_ids = take((size_t)P * 4);
  L.pair_gates = take((size_t)P * 4);
  L.token_pairs = take((size_t)P * 4);
  L.tiles = take((size_t)mt * 16);
  L.meta = take(16);
  L.bws = take(pp_bucket_workspace_bytes(N, E));
  L.xbf = take((size_t)N * H * 2);
  L.act = take((size_t)P * G * 2);
  L.y = take((size_t)P * H * 4);
  L.total = o;
  return L;
}

extern "C" size_t pp_prefill_workspace_bytes(int64_t n_tokens, int H, int E, int G) {
  return prefill_layout(n_tokens, H, E, G).total;
}

extern "C" int pp_moe_prefill(const void* x, int x_dtype, int64_t n_tokens, int H, const float* router_packed,
                              const float* bias, int E, int G, float tau, const void* packed, void* out_bf16,
                              void* workspace, void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(n_tokens >= 0 && n_tokens <= (int64_t)0x7fffffff / PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED,
             "pp_moe_prefill: n_tokens %lld out of range", (long long)n_tokens);
  PP_REQUIRE(x_dtype == PP_DTYPE_F32 || x_dtype == PP_DTYPE_BF16, PP_ERR_INVALID, "pp_moe_prefill: x_dtype %d",
             x_dtype);
  if (n_tokens == 0) return PP_OK;
  PP_REQUIRE(x && router_packed && packed && out_bf16 && workspace, PP_ERR_INVALID, "pp_moe_prefill: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const PrefillWs L = prefill_layout(n_tokens, H, E, G);
  char* ws = (char*)workspace;
  float* gates = (float*)(ws + L.gates);
  uint8_t* mask = (uint8_t*)(ws + L.mask);
  int32_t* count = (int32_t*)(ws + L.count);
  int32_t* offsets = (int32_t*)(ws + L.offsets);
  int32_t* token_ids = (int32_t*)(ws + L.token_ids);
  float* pair_gates = (float*)(ws + L.pair_gates);
  int32_t* token_pairs = (int32_t*)(ws + L.token_pairs);
  int32_t* tiles = (int32_t*)(ws + L.tiles);
  int32_t* meta = (int32_t*)(ws + L.meta);
  bf16_t* xbf = x_dtype == PP_DTYPE_BF16 ? (bf16_t*)x : (bf16_t*)(ws + L.xbf);
  bf16_t* act = (bf16_t*)(ws + L.act);
  float* y = (float*)(ws + L.y);
  const int64_t mt = pp_max_tiles(n_tokens, E, GM_BM);
  if ((rc = pp_route_impl(x, x_dtype, nullptr, n_tokens, H, router_packed, bias, E, tau, nullptr, nullptr, gates,
                          mask, count, x_dtype == PP_DTYPE_BF16 ? nullptr : xbf, st)))
    return rc;
  if ((rc = pp_bucket_impl(mask, gates, n_tokens, E, GM_BM, offsets, token_ids, pair_gates, token_pairs, tiles, meta,
                           ws + L.bws, st)))
    return rc;
  if ((rc = gateup_launch(xbf, H, G, (const bf16_t*)packed, E, token_ids, pair_gates, tiles, meta, mt, act, st)))
    return rc;
  const bf16_t* down_t = (const bf16_t*)packed + (int64_t)E * G * 3 * H;
  if ((rc = down_launch(act, H, G, down_t, tiles, meta, mt, y, st))) return rc;
  return combine_launch(y, token_pairs, count, n_tokens, H, E, (bf16_t*)out_bf16, st);
}
