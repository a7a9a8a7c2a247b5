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
// beyond the last partial tile of each expert), 256 threads = 4 waves, BK = 64:
// gemm_v3_kernel for G % 64 == 0 (LDS-DMA pipeline, below), gateup_kernel /
// down_kernel (register-staged, row-padded LDS tiles) otherwise.
#include <algorithm>

#include "pp_common.h"

#define GM_THREADS 256
#define GM_BK 64
#define GM_LDK (GM_BK + 8)  // padded LDS row (bf16 elements)
#define GM_BM 128

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

// ------------------------------------------------------------------ pipelined grouped GEMM
// Tile 128 rows x 128 B-rows x BK 64 on v_mfma_f32_32x32x16_bf16, 4 waves as 2 x 2
// (wave tile 64 x 64), two workgroups per CU, persistent over (row tile, column tile)
// items. Operands go straight from global memory into LDS (global_load_lds_dwordx4:
// lane i of a wave writes bytes [16 i, 16 i + 16) of the wave's 1 KB block, no VGPR
// staging) through GP_STAGES LDS stages; the DMA runs GP_STAGES - 1 K blocks ahead and
// does not stop at item boundaries -- the blocks of a workgroup's items form one
// stream, so the next item's first blocks are in flight under the current item's last
// MFMAs. Per-item data never stalls the stream: tile metadata comes through scalar
// loads, and the gathered token ids and pair gates of item i+1 are DMA'd into an LDS
// slot together with item i's first block, so building item i+1's row offsets is an
// LDS read.
//
// A tile row holds BK bf16 = BK/8 chunks of 16 bytes; chunk c of row r is stored at
// position c ^ gp_swz(r). A fragment read (ds_read_b128) covers 32 consecutive rows; any
// 16 of them then land in 16 distinct 16-byte slots of a 256-byte bank window.
//
// Synchronisation is explicit: the compiler cannot tell that an LDS read does not
// alias a DMA still in flight and would drain every prefetch before each read, and
// __syncthreads() adds a release fence that does the same. So fragment reads are
// inline ds_read_b128 whose results are fenced by s_waitcnt lgkmcnt tied to the
// fragment registers, and the per-K-block barrier waits only for this wave's DMA of
// the block about to be read: every wave issues at least GP_DMA DMA instructions per
// block (past the last block it re-fetches that block into the free stage, never
// read), so "at most GP_DMA * (GP_STAGES - 2) of this wave's vector memory ops
// outstanding" means its DMA of the block about to be read has landed (loads complete
// in order; extra ops -- slot DMA, epilogue stores -- only make the wait stricter); the
// barrier after it covers every wave and frees the stage written next.
//
// Where the time goes (2048-token prefill, timestamps per workgroup): a K block takes
// 1.07 us with two workgroups per CU -- 0.20 loop skeleton, 0.58 with only the MFMAs,
// 0.36 with only the fragment reads, 0.73 without the DMA -- and the same with every
// operand forced L2-resident, so the CU's own pipeline (DMA issue and landing, LDS,
// MFMA, barrier), not HBM or L2, sets the rate: about 1.85 128x128x64 blocks per us per
// CU. gate/up has ~630 items for 512 workgroups: the median workgroup is done at 34 us,
// the 118 with a second item at 52. down: 28 | 33 us, of which ~13 us is the 77 MB fp32
// y epilogue (HBM write rate).
// Measured alternatives (gate/up | down): the two-stage kernel without the cross-item
// stream 54 | 34 us; one workgroup per CU with four stages 81 | 50 (one wave per SIMD
// leaves the LDS and MFMA latencies exposed); BK 32 with four stages 59 | 37; BK 32,
// three stages, three workgroups per CU (every item in one round) 53 | 35 (the per-CU
// rate drops to ~1.5 blocks/us); stream-K -- equal (item, K block) ranges per
// workgroup, an item cut between two workgroups joined through an agent-scope ticket
// and fp32 partial sums -- 58 | 47 (a K block slows to 1.25-1.35 us once workgroups
// sharing a row tile or an expert's weights no longer walk K in step, and each join
// costs 2.6-3 us of memory-side round trips); 128 x 256 tiles, eight waves (2 x 4, the
// same 64 x 64 wave tile), three stages, one workgroup per CU 61 | 32 (one barrier
// keeps all eight waves in step, so the two waves of a SIMD no longer overlap each
// other's waits, and 315 items leave 59 CUs with two); this kernel 49 | 32. Small batches (16 /
// 64 tokens, ~100 items): four stages with the CU to itself 26.9 | 10.3 us against 26.4
// | 9.5 -- the weights stream from HBM into LDS, so the bytes in flight per CU are capped
// by LDS, ~5 MB over the chip where HBM needs ~16 MB; register-streamed loads (as in
// decode) are what such batches need.
#include "gemm_lds.h"

#define GP_BK 64         // K block (bf16 elements)
#define GP_STAGES 2
#define GP_WG_PER_CU 2
#define GP_ROWB (GP_BK * 2)                     // bytes of one tile row in a stage
#define GP_CH (GP_BK / 8)                       // 16-byte chunks per row
#define GP_TILE (128 * GP_ROWB)                 // one operand tile of one stage
#define GP_STAGE (2 * GP_TILE)
#define GP_RPI (1024 / GP_ROWB)                 // rows per DMA instruction (a wave's 1 KB)
#define GP_NI (128 / (4 * GP_RPI))              // DMA instructions per tile per wave
#define GP_DMA (2 * GP_NI)                      // per wave per K block (A + B)
#define GP_KS (GP_BK / 16)                      // MFMA k-steps per K block
#define GP_SLOT_BYTES 1024                      // per item: 128 token ids + 128 pair gates
#define GP_NSLOT 4
#define GP_LDS_BYTES (GP_STAGES * GP_STAGE + GP_NSLOT * GP_SLOT_BYTES)
// chunk c of row r is stored at position c ^ gp_swz(r): any 16 consecutive rows of a
// fragment read land in 16 distinct 16-byte slots of a 256-byte bank window
__device__ __forceinline__ int gp_swz(int r) { return GP_BK == 64 ? (r >> 1) & 7 : (r >> 2) & 3; }

// Join of a tail item's parts; every thread calls it, at the part's last K block. Every
// part stores its partial sums (agent-scope stores), waits until they are performed,
// then takes an agent-scope ticket: the part drawing the last ticket knows every other
// part's sums are in memory -- nobody waits for anybody -- adds the parts in part order
// (a fixed order: the same bits whichever part draws the last ticket), returns true and
// clears the ticket; the others return false. A(i) / SET(i, v): float i of the thread's
// NF accumulators. (Flags polled by the last part instead cost ~20 us at 2048 tokens:
// ~150 pollers on a few cache lines slow the very stores they wait for.)
template <int NF, typename Get, typename Set>
__device__ __forceinline__ bool gp_join(Get&& A, Set&& SET, const GpSched& sc, float* part, uint32_t* sync,
                                        int* role_s) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int ti = sc.part_item - sc.tail0, p = sc.unit % sc.nparts, u0 = sc.unit - p;
  uint32_t* tick = sync + 1 + ti;
  {
    unsigned long long* mine = (unsigned long long*)(part + (size_t)sc.unit * NF * nt) + tid;
#pragma unroll
    for (int c = 0; c < NF / 2; ++c) {
      const unsigned long long v =
          (unsigned long long)__float_as_uint(A(2 * c)) | ((unsigned long long)__float_as_uint(A(2 * c + 1)) << 32);
      __hip_atomic_store(mine + c * nt, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // every thread's stores performed
  if (tid == 0) *role_s = (int)__hip_atomic_fetch_add(tick, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (*role_s != sc.nparts - 1) return false;
  float tot[NF];
  for (int q = 0; q < sc.nparts; ++q) {
    if (q == p) {
#pragma unroll
      for (int i = 0; i < NF; ++i) tot[i] = q == 0 ? A(i) : tot[i] + A(i);
    } else {
      const unsigned long long* src = (const unsigned long long*)(part + (size_t)(u0 + q) * NF * nt) + tid;
#pragma unroll
      for (int c = 0; c < NF / 2; ++c) {
        const unsigned long long v = __hip_atomic_load(src + c * nt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float lo = __uint_as_float((uint32_t)v), hi = __uint_as_float((uint32_t)(v >> 32));
        tot[2 * c] = q == 0 ? lo : tot[2 * c] + lo;
        tot[2 * c + 1] = q == 0 ? hi : tot[2 * c + 1] + hi;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NF; ++i) SET(i, tot[i]);
  if (tid == 0) gp_st(tick, 0u);
  return true;
}

// MODE 0: gate/up + SwiGLU (A = gathered x rows, B = gate/up rows of 64 neurons);
// MODE 1: down (A = act rows, B = down_t rows of 128 hidden columns).
template <int MODE>
__global__ __launch_bounds__(GM_THREADS, GP_WG_PER_CU) void gemm_v3_kernel(
    const bf16_t* __restrict__ abase, int H, int G, const bf16_t* __restrict__ bbase,
    const int32_t* __restrict__ token_ids, const float* __restrict__ pair_gates,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, bf16_t* __restrict__ act,
    float* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* slots = smem + GP_STAGES * GP_STAGE;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int n_ntile = MODE == 0 ? G / 64 : H / 128;
  const int K = MODE == 0 ? H : G;
  const int nkb = K / GP_BK;
  const int n_items = meta[0] * n_ntile;
  const GpSched sc(n_items, nkb, false);  // whole items (a split costs this loop more than it saves)
  const int n_local_items = sc.n_local();
  const int F = sc.units(nkb);
  if (F <= 0) return;
  auto locate = [&](int f, int& li, int& kb) { sc.locate(f, nkb, li, kb); };

  // slot DMA of item li (wave 0): token ids and gates of the tile rows, row r >= rows
  // reading row rows - 1 (in range; padding rows are never stored)
  auto slot_dma = [&](int li) {
    if (MODE != 0 || w != 0) return;
    const int item = sc.item(li);
    const int t = item / n_ntile;
    const int p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    unsigned char* sl = slots + (li & (GP_NSLOT - 1)) * GP_SLOT_BYTES;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = min(64 * h + lane, rows - 1);
      gl2lds4(token_ids + p0 + r, sl + 256 * h);
      gl2lds4(pair_gates + p0 + r, sl + 512 + 256 * h);
    }
  };

  // issue cursor: row offsets of the item whose blocks are being issued
  int64_t aoff[GP_NI], boff[GP_NI];
  auto setup_item = [&](int li) {
    const int item = sc.item(li);
    const int t = item / n_ntile, nt = item - t * n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int32_t* tok = (const int32_t*)(slots + (li & (GP_NSLOT - 1)) * GP_SLOT_BYTES);
#pragma unroll
    for (int i = 0; i < GP_NI; ++i) {
      const int r = (4 * i + w) * GP_RPI + lane / GP_CH;
      const int pchunk = ((lane % GP_CH) ^ gp_swz(r)) * 8;
      if (MODE == 0) {
        aoff[i] = (int64_t)tok[r] * H + pchunk;
        // B tile row r = wn_*64 + j*32 + q -> gate (j=0) / up (j=1) row of neuron nt*64 + wn_*32 + q
        const int wn_ = r >> 6, j = (r >> 5) & 1, q = r & 31;
        boff[i] = ((int64_t)(e * G + nt * 64 + wn_ * 32 + q) * 3 + j) * H + pchunk;
      } else {
        aoff[i] = (int64_t)(p0 + min(r, rows - 1)) * G + pchunk;
        boff[i] = ((int64_t)e * H + nt * 128 + r) * G + pchunk;
      }
    }
  };
  auto issue = [&](int f) {
    int li, kb;
    locate(f < F ? f : F - 1, li, kb);  // past the end: the last block again, never read
    if (f < F && (kb == 0 || f == sc.n_whole * nkb)) {  // an item's first block (a part's: kb_lo)
      setup_item(li);
      // item li+1's slot is read nkb blocks later; items 0 and 1 get theirs in the
      // prologue (the first item's blocks may all be in flight before its first wait)
      if (li >= 1 && li + 1 < n_local_items) slot_dma(li + 1);
    }
    unsigned char* sb = smem + (f % GP_STAGES) * GP_STAGE;
#pragma unroll
    for (int i = 0; i < GP_NI; ++i) {
      const int blk = (4 * i + w) * 1024;
      gl2lds(abase + aoff[i] + kb * GP_BK, sb + blk);
      gl2lds(bbase + boff[i] + kb * GP_BK, sb + GP_TILE + blk);
    }
  };

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  uint32_t offA[GP_KS], offB[GP_KS];
#pragma unroll
  for (int ks = 0; ks < GP_KS; ++ks) {
    const int r = lane & 31, c = ks * 2 + (lane >> 5);
    const uint32_t o = (uint32_t)(r * GP_CH + (c ^ gp_swz(r))) * 16;
    offA[ks] = lds0 + wm * 64 * GP_ROWB + o;
    offB[ks] = lds0 + GP_TILE + wn * 64 * GP_ROWB + o;
  }

  // prologue: the first two items' slots, then the first GP_STAGES - 1 blocks
  slot_dma(0);
  if (n_local_items > 1) slot_dma(1);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int f = 0; f < GP_STAGES - 1; ++f) issue(f);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

  for (int f = 0; f < F; ++f) {
    gp_wait_barrier<GP_DMA * (GP_STAGES - 2)>();
    issue(f + GP_STAGES - 1);
    const uint32_t sbase = (f % GP_STAGES) * GP_STAGE;
    u32x4 fa[2][2], fb[2][2];
    fa[0][0] = gv_read<0>(offA[0] + sbase);
    fa[0][1] = gv_read<32 * GP_ROWB>(offA[0] + sbase);
    fb[0][0] = gv_read<0>(offB[0] + sbase);
    fb[0][1] = gv_read<32 * GP_ROWB>(offB[0] + sbase);
#pragma unroll
    for (int ks = 0; ks < GP_KS; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      if (ks < GP_KS - 1) {
        fa[nxt][0] = gv_read<0>(offA[ks + 1] + sbase);
        fa[nxt][1] = gv_read<32 * GP_ROWB>(offA[ks + 1] + sbase);
        fb[nxt][0] = gv_read<0>(offB[ks + 1] + sbase);
        fb[nxt][1] = gv_read<32 * GP_ROWB>(offB[ks + 1] + sbase);
        gv_wait<4>(fa[cur][0], fa[cur][1], fb[cur][0], fb[cur][1]);
      } else {
        gv_wait<0>(fa[cur][0], fa[cur][1], fb[cur][0], fb[cur][1]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32v(fa[cur][i], fb[cur][j], acc[i][j]);
    }
    int li, kb;
    locate(f, li, kb);
    if (kb != nkb - 1) continue;
    const int item = sc.item(li);
    // ---- epilogue of item li (lane laundered: its row indices are not worth registers
    // across the main loop)
    {
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int t = item / n_ntile, nt = item - t * n_ntile;
      const int p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
      if (MODE == 0) {
        const float* gts = (const float*)(slots + (li & (GP_NSLOT - 1)) * GP_SLOT_BYTES + 512);
        const int neuron = nt * 64 + wn * 32 + (ln & 31);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const int r = wm * 64 + i * 32 + mfma32_row(q, ln);
            if (r < rows)
              act[(int64_t)(p0 + r) * G + neuron] = f32_to_bf16(pp_silu(acc[i][0][q]) * acc[i][1][q] * gts[r]);
          }
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int h = nt * 128 + wn * 64 + j * 32 + (ln & 31);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              const int r = wm * 64 + i * 32 + mfma32_row(q, ln);
              if (r < rows) y[(int64_t)(p0 + r) * H + h] = acc[i][j][q];
            }
          }
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  }
  // the redundant tail DMAs must land before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ------------------------------------------------------------------ short tiles
// Small batches (N <= GS_MAX_N tokens): 32-row tiles (bucketed with tile_m = GS_TM),
// items of 64 neurons (gate/up) or 128 hidden columns (down) as above. At such sizes
// the 128-row kernel streams the weights at the rate its LDS stages allow in flight (two
// 32 KB stages per workgroup, ~100 workgroups): a 20 KB stage (4 KB of A rows, 16 KB of
// B rows) lets GS_STAGES - 1 blocks -- 96 KB of weights -- be in flight per CU. Four
// waves split N: wave w computes B rows 32 w .. 32 w + 31 over the whole K, one 32x32x16
// MFMA per k-step. gate/up: the B blocks are gate and up of neurons 0..31, then of
// 32..63, so the up waves (1, 3) hand their accumulators to the gate waves (0, 2)
// through LDS for the SwiGLU epilogue. Same DMA / slot / wait scheme as gemm_v3_kernel.
#define GS_MAX_N 64
#define GS_TM 32
#define GS_STAGES 7
#define GS_TILE_A (GS_TM * GP_ROWB)
#define GS_TILE_B (128 * GP_ROWB)
#define GS_STAGE (GS_TILE_A + GS_TILE_B)
#define GS_SLOT_BYTES 256  // 32 token ids, then 32 pair gates
#define GS_XCHG_BYTES (2 * 16 * 64 * 4)
#define GS_LDS_BYTES (GS_STAGES * GS_STAGE + GP_NSLOT * GS_SLOT_BYTES + GS_XCHG_BYTES)
#define GS_DMA 5  // DMA instructions per wave per K block: one A, four B

template <int N>
__device__ __forceinline__ void gv_wait2(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}

template <int MODE>
__global__ __launch_bounds__(GM_THREADS, 1) void gemm_s_kernel(
    const bf16_t* __restrict__ abase, int H, int G, const bf16_t* __restrict__ bbase,
    const int32_t* __restrict__ token_ids, const float* __restrict__ pair_gates,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, bf16_t* __restrict__ act,
    float* __restrict__ y, float* __restrict__ part, uint32_t* __restrict__ sync) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int role_s;
  unsigned char* slots = smem + GS_STAGES * GS_STAGE;
  float* xchg = (float*)(slots + GP_NSLOT * GS_SLOT_BYTES);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n_ntile = MODE == 0 ? G / 64 : H / 128;
  const int K = MODE == 0 ? H : G;
  const int nkb = K / GP_BK;
  const int n_items = meta[0] * n_ntile;
  const GpSched sc(n_items, nkb, MODE == 0 && part != nullptr);  // down items are too short to split
  const int n_local_items = sc.n_local();
  const int F = sc.units(nkb);
  if (F <= 0) return;
  auto locate = [&](int f, int& li, int& kb) { sc.locate(f, nkb, li, kb); };
  // slot of item li (wave 0, one 4-byte DMA per lane): token ids, then pair gates of the
  // tile rows, row r >= rows reading row rows - 1
  auto slot_dma = [&](int li) {
    if (MODE != 0 || w != 0) return;
    const int item = sc.item(li);
    const int t = item / n_ntile;
    const int p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int r = min(lane & 31, rows - 1);
    gl2lds4(lane < 32 ? (const void*)(token_ids + p0 + r) : (const void*)(pair_gates + p0 + r),
            slots + (li & (GP_NSLOT - 1)) * GS_SLOT_BYTES);
  };
  int64_t aoff, boff[4];
  auto setup_item = [&](int li) {
    const int item = sc.item(li);
    const int t = item / n_ntile, nt = item - t * n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int32_t* tok = (const int32_t*)(slots + (li & (GP_NSLOT - 1)) * GS_SLOT_BYTES);
    {
      const int r = w * GP_RPI + lane / GP_CH;  // A row 0..31
      const int pchunk = ((lane % GP_CH) ^ gp_swz(r)) * 8;
      aoff = MODE == 0 ? (int64_t)tok[r] * H + pchunk : (int64_t)(p0 + min(r, rows - 1)) * G + pchunk;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (4 * i + w) * GP_RPI + lane / GP_CH;  // B row 0..127
      const int pchunk = ((lane % GP_CH) ^ gp_swz(r)) * 8;
      if (MODE == 0) {
        const int wn_ = r >> 6, j = (r >> 5) & 1, q = r & 31;
        boff[i] = ((int64_t)(e * G + nt * 64 + wn_ * 32 + q) * 3 + j) * H + pchunk;
      } else {
        boff[i] = ((int64_t)e * H + nt * 128 + r) * G + pchunk;
      }
    }
  };
  auto issue = [&](int f) {
    int li, kb;
    locate(f < F ? f : F - 1, li, kb);  // past the end: the last block again, never read
    if (f < F && (kb == 0 || f == sc.n_whole * nkb)) {  // an item's first block (a part's: kb_lo)
      setup_item(li);
      if (li >= 1 && li + 1 < n_local_items) slot_dma(li + 1);
    }
    unsigned char* sb = smem + (f % GS_STAGES) * GS_STAGE;
    gl2lds(abase + aoff + kb * GP_BK, sb + w * 1024);
#pragma unroll
    for (int i = 0; i < 4; ++i) gl2lds(bbase + boff[i] + kb * GP_BK, sb + GS_TILE_A + (4 * i + w) * 1024);
  };

  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  uint32_t offA[GP_KS], offB[GP_KS];
#pragma unroll
  for (int ks = 0; ks < GP_KS; ++ks) {
    const int r = lane & 31, c = ks * 2 + (lane >> 5);
    const uint32_t o = (uint32_t)(r * GP_CH + (c ^ gp_swz(r))) * 16;  // gp_swz(32 w + r) == gp_swz(r)
    offA[ks] = lds0 + o;
    offB[ks] = lds0 + GS_TILE_A + w * 32 * GP_ROWB + o;
  }

  slot_dma(0);
  if (n_local_items > 1) slot_dma(1);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int f = 0; f < GS_STAGES - 1; ++f) issue(f);

  f32x16_t acc;
#pragma unroll
  for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
  for (int f = 0; f < F; ++f) {
    gp_wait_barrier<GS_DMA * (GS_STAGES - 2)>();
    issue(f + GS_STAGES - 1);
    const uint32_t sbase = (f % GS_STAGES) * GS_STAGE;
    u32x4 fa[2], fb[2];
    fa[0] = gv_read<0>(offA[0] + sbase);
    fb[0] = gv_read<0>(offB[0] + sbase);
#pragma unroll
    for (int ks = 0; ks < GP_KS; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      if (ks < GP_KS - 1) {
        fa[nxt] = gv_read<0>(offA[ks + 1] + sbase);
        fb[nxt] = gv_read<0>(offB[ks + 1] + sbase);
        gv_wait2<2>(fa[cur], fb[cur]);
      } else {
        gv_wait2<0>(fa[cur], fb[cur]);
      }
      acc = mfma32v(fa[cur], fb[cur], acc);
    }
    int li, kb;
    locate(f, li, kb);
    if (kb != nkb - 1 && f != F - 1) continue;
    if (MODE == 0 && li == sc.n_whole && sc.nparts > 1 &&
        !gp_join<16>([&](int i) { return acc[i]; }, [&](int i, float v) { acc[i] = v; }, sc, part, sync, &role_s)) {
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
      continue;
    }
    {
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int item = sc.item(li);
      const int t = item / n_ntile, nt = item - t * n_ntile;
      const int p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
      if (MODE == 0) {
        float* xw = xchg + (w >> 1) * 16 * 64;
        if (w & 1) {
#pragma unroll
          for (int q = 0; q < 16; ++q) xw[q * 64 + ln] = acc[q];
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // LDS only: the DMA stays in flight
        if (!(w & 1)) {
          const float* gts = (const float*)(slots + (li & (GP_NSLOT - 1)) * GS_SLOT_BYTES + 128);
          const int neuron = nt * 64 + (w >> 1) * 32 + (ln & 31);
#pragma unroll
          for (int q = 0; q < 16; ++q) {
            const int r = mfma32_row(q, ln);
            if (r < rows)
              act[(int64_t)(p0 + r) * G + neuron] = f32_to_bf16(pp_silu(acc[q]) * xw[q * 64 + ln] * gts[r]);
          }
        }
      } else {
        const int h = nt * 128 + w * 32 + (ln & 31);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int r = mfma32_row(q, ln);
          if (r < rows) y[(int64_t)(p0 + r) * H + h] = acc[q];
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
  }
  // the redundant tail DMAs must land before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ------------------------------------------------------------------ combine
// Per (token, 8 columns): the token's pair ids are read first (one batch of independent
// loads), then up to CB_BATCH y rows at once, summed in expert order: two memory round
// trips per batch instead of two per pair.
#define CB_BATCH 8
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
    const int32_t* tp = token_pairs + t * E;
    bool stop = false;
    for (int q0 = 0; q0 < k && !stop; q0 += CB_BATCH) {
      int p[CB_BATCH];
#pragma unroll
      for (int i2 = 0; i2 < CB_BATCH; ++i2) p[i2] = q0 + i2 < k ? tp[q0 + i2] : -1;
      float4 a[CB_BATCH], b[CB_BATCH];
#pragma unroll
      for (int i2 = 0; i2 < CB_BATCH; ++i2) {
        // a negative id (fewer pairs than count: inconsistent caller data) ends the sum;
        // nothing is read out of range
        if (p[i2] >= 0) {
          const float4* src = (const float4*)(y + (int64_t)p[i2] * H + ch * 8);
          a[i2] = src[0];
          b[i2] = src[1];
        }
      }
#pragma unroll
      for (int i2 = 0; i2 < CB_BATCH; ++i2) {
        if (q0 + i2 >= k) break;
        if (p[i2] < 0) { stop = true; break; }
        s0.x += a[i2].x; s0.y += a[i2].y; s0.z += a[i2].z; s0.w += a[i2].w;
        s1.x += b[i2].x; s1.y += b[i2].y; s1.z += b[i2].z; s1.w += b[i2].w;
      }
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

static int gemm_grid_v3(int64_t items) {  // GP_WG_PER_CU workgroups per CU, a multiple of 8 (XCD order)
  int64_t g = (int64_t)GP_WG_PER_CU * pp_device_cus();
  if (items < g) g = items;
  g = (g + 7) / 8 * 8;
  return (int)(g < 8 ? 8 : g);
}

// Short tiles (gemm_s_kernel) for small batches inside pp_moe_prefill: the tile map is
// then built with tile_m = GS_TM. Needs six K blocks per gate/up item (the next item's
// slot lands GS_STAGES - 1 blocks ahead).
static bool prefill_short_tiles(int64_t N, int H, int G) {
  return N <= GS_MAX_N && G % 64 == 0 && H / GP_BK >= GS_STAGES - 1;
}
static int gemm_s_grid() {  // one workgroup per CU, a multiple of 8 (XCD order); spare ones take item parts
  const int g = (pp_device_cus() + 7) / 8 * 8;
  return g < 8 ? 8 : g;
}

// Split workspace of the short-tile GEMMs (layout at GpSched): sync words, then one
// slot of 16 floats per thread (a workgroup's accumulators) per workgroup of their grid.
static int64_t gemm_split_slots() { return gemm_s_grid(); }
static size_t gemm_sync_bytes() { return (size_t)((1 + gemm_split_slots()) * 4 + 255) / 256 * 256; }
static size_t gemm_split_bytes() {
  return gemm_sync_bytes() + (size_t)gemm_split_slots() * 16 * GM_THREADS * sizeof(float);
}
static void gemm_split_ptrs(void* gws, uint32_t** sync, float** part) {
  *sync = gws ? (uint32_t*)gws : nullptr;
  *part = gws ? (float*)((char*)gws + gemm_sync_bytes()) : nullptr;
}

static int gateup_launch(const bf16_t* xb, int H, int G, const bf16_t* wrows, int E, const int32_t* token_ids,
                         const float* pair_gates, const int32_t* tiles, const int32_t* meta, int64_t max_tiles,
                         bf16_t* act, void* gws, hipStream_t st, bool short_tiles = false) {
  (void)E;
  uint32_t* sync;
  float* part;
  gemm_split_ptrs(gws, &sync, &part);
  if (short_tiles) {
    gemm_s_kernel<0><<<gemm_s_grid(), GM_THREADS, GS_LDS_BYTES, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles,
                                                                      meta, act, nullptr, part, sync);
  } else if (G % 64 == 0) {
    int grid = gemm_grid_v3(max_tiles * (G / 64));
    gemm_v3_kernel<0><<<grid, GM_THREADS, GP_LDS_BYTES, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles, meta,
                                                              act, nullptr);
  } else {
    int grid = gemm_grid(max_tiles * (G / 32));
    gateup_kernel<4, 1, 1><<<grid, GM_THREADS, 0, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles, meta, act);
  }
  return pp_check_launch("gateup_kernel");
}

static int down_launch(const bf16_t* act, int H, int G, const bf16_t* down_t, const int32_t* tiles,
                       const int32_t* meta, int64_t max_tiles, float* y, void* gws, hipStream_t st,
                       bool short_tiles = false) {
  uint32_t* sync;
  float* part;
  gemm_split_ptrs(gws, &sync, &part);
  if (short_tiles) {
    gemm_s_kernel<1><<<gemm_s_grid(), GM_THREADS, GS_LDS_BYTES, st>>>(act, H, G, down_t, nullptr, nullptr, tiles,
                                                                      meta, nullptr, y, part, sync);
  } else if (G % 64 == 0) {
    int grid = gemm_grid_v3(max_tiles * (H / 128));
    gemm_v3_kernel<1><<<grid, GM_THREADS, GP_LDS_BYTES, st>>>(act, H, G, down_t, nullptr, nullptr, tiles, meta,
                                                              nullptr, y);
  } else {
    int grid = gemm_grid(max_tiles * (H / 128));
    down_kernel<<<grid, GM_THREADS, 0, st>>>(act, H, G, down_t, tiles, meta, y);
  }
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
                       max_tiles, (bf16_t*)act_bf16, nullptr, (hipStream_t)stream);
}

extern "C" int pp_expert_down(const void* act_bf16, int H, int G, const void* packed, int E, const int32_t* tiles,
                              const int32_t* meta, int64_t max_tiles, float* y_f32, void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(act_bf16 && packed && tiles && meta && y_f32, PP_ERR_INVALID, "pp_expert_down: null pointer");
  PP_REQUIRE(max_tiles >= 0, PP_ERR_INVALID, "pp_expert_down: max_tiles < 0");
  if (max_tiles == 0) return PP_OK;
  const bf16_t* down_t = (const bf16_t*)packed + (int64_t)E * G * 3 * H;
  return down_launch((const bf16_t*)act_bf16, H, G, down_t, tiles, meta, max_tiles, (float*)y_f32, nullptr,
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
                  uint8_t* mask_out, int32_t* count_out, bf16_t* xbf_out, hipStream_t st, int32_t* blkcnt_out);
int pp_bucket_from_counts(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m,
                          const int32_t* blkcnt, int cb, int32_t* offsets, int32_t* token_ids, float* pair_gates,
                          int32_t* token_pairs, int32_t* tiles, int32_t* meta, hipStream_t st, uint32_t* zero,
                          int nzero);
bool pp_bucket_counts_fit(int64_t N, int E, int cb);
int pp_route_count_block(int64_t N, int H, int E);
int pp_bucket_impl(const uint8_t* mask, const float* gates, int64_t N, int E, int tile_m, int32_t* offsets,
                   int32_t* token_ids, float* pair_gates, int32_t* token_pairs, int32_t* tiles, int32_t* meta,
                   void* workspace, hipStream_t st, uint32_t* zero, int nzero);

struct PrefillWs {
  size_t gates, mask, count, offsets, token_ids, pair_gates, token_pairs, tiles, meta, bws, blk16, xbf, act, y,
      gws, logits, total;
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
  const int64_t mt = pp_max_tiles(N, E, prefill_short_tiles(N, H, G) ? GS_TM : GM_BM);
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
  L.blk16 = take((size_t)((N + 3) / 4) * 16 * 4);  // the E = 16 router's per-block expert counts (>= 4 tokens a block)
  L.xbf = take((size_t)N * H * 2);
  L.act = take((size_t)P * G * 2);
  L.y = take((size_t)P * H * 4);
  L.gws = prefill_short_tiles(N, H, G) ? take(gemm_split_bytes()) : 0;
  L.logits = E != 16 ? take((size_t)P * 4) : 0;  // the logits pass of E != 16 (selection from its logits)
  L.total = o;
  return L;
}

// Tokens per pass. The pair buffers are sized for the worst case, every token selecting
// every expert (P = N * E pairs: fp32 y [P][H], bf16 act [P][G], the CSR), since the
// actual P is only known on the device; a pass covers at most as many tokens as keep
// that y within PF_PASS_Y_BYTES (2048 tokens at E = 16, H = 1536 in one pass; 455
// tokens a pass at the checkpoint's E = 192), so the workspace stays bounded for any
// N and E. Longer inputs run in consecutive passes on the same workspace.
#define PF_PASS_Y_BYTES ((int64_t)512 << 20)
static int64_t prefill_pass_tokens(int64_t N, int H, int E) {
  const int64_t per_token = (int64_t)E * H * 4;
  // a multiple of 4 tokens: every pass's mask rows start 4-byte aligned (the bucketing reads words)
  return min(N, max((int64_t)64, PF_PASS_Y_BYTES / per_token / 4 * 4));
}

size_t pp_dense_workspace_bytes(int64_t N, int H, int E, int G);
int pp_dense_prefill(const void* x, int x_dtype, int64_t N, int H, const float* router, const float* bias, int E,
                     int G, float tau, const void* packed, void* out, void* workspace, hipStream_t st,
                     float* logits_out, uint8_t* mask_out);

// The dense form (dense.hip) serves the shapes whose experts are narrower than a 64-neuron
// MFMA column tile; the grouped pipeline below the rest.
static bool prefill_dense_form(int G) { return G % 64 != 0; }

extern "C" size_t pp_prefill_workspace_bytes(int64_t n_tokens, int H, int E, int G) {
  if (prefill_dense_form(G)) return pp_dense_workspace_bytes(n_tokens, H, E, G);
  return prefill_layout(prefill_pass_tokens(n_tokens, H, E), H, E, G).total;
}

// One pass over n_tokens tokens (at most prefill_pass_tokens) on the workspace.
static int prefill_pass(const void* x, int x_dtype, int64_t n_tokens, int H, const float* router_packed,
                        const float* bias, int E, int G, float tau, const void* packed, void* out_bf16,
                        void* workspace, hipStream_t st, float* logits_out, uint8_t* mask_out) {
  int rc;
  const PrefillWs L = prefill_layout(n_tokens, H, E, G);
  char* ws = (char*)workspace;
  float* gates = (float*)(ws + L.gates);
  uint8_t* mask = mask_out ? mask_out : (uint8_t*)(ws + L.mask);
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
  const bool short_tiles = prefill_short_tiles(n_tokens, H, G);
  const int tile_m = short_tiles ? GS_TM : GM_BM;
  const int64_t mt = pp_max_tiles(n_tokens, E, tile_m);
  // the GEMMs' split workspace: its sync words are cleared by this call's bucketing kernel
  void* gws = short_tiles ? (void*)(ws + L.gws) : nullptr;
  const int nzero = gws ? (int)(1 + gemm_split_slots()) : 0;
  // E = 16: the router kernel also counts selections per 16-token block, and the
  // bucketing is one kernel from those counts (no counting or scan pass)
  const int cb = pp_route_count_block(n_tokens, H, E);
  int32_t* blk16 = pp_bucket_counts_fit(n_tokens, E, cb) ? (int32_t*)(ws + L.blk16) : nullptr;
  if ((rc = pp_route_impl(x, x_dtype, nullptr, n_tokens, H, router_packed, bias, E, tau,
                          logits_out ? logits_out : E != 16 ? (float*)(ws + L.logits) : nullptr, nullptr, gates,
                          mask, count, x_dtype == PP_DTYPE_BF16 ? nullptr : xbf, st, blk16)))
    return rc;
  if (blk16)
    rc = pp_bucket_from_counts(mask, gates, n_tokens, E, tile_m, blk16, cb, offsets, token_ids, pair_gates,
                               token_pairs, tiles, meta, st, (uint32_t*)gws, nzero);
  else
    rc = pp_bucket_impl(mask, gates, n_tokens, E, tile_m, offsets, token_ids, pair_gates, token_pairs, tiles, meta,
                        ws + L.bws, st, (uint32_t*)gws, nzero);
  if (rc) return rc;
  if ((rc = gateup_launch(xbf, H, G, (const bf16_t*)packed, E, token_ids, pair_gates, tiles, meta, mt, act, gws,
                          st, short_tiles)))
    return rc;
  const bf16_t* down_t = (const bf16_t*)packed + (int64_t)E * G * 3 * H;
  if ((rc = down_launch(act, H, G, down_t, tiles, meta, mt, y, gws, st, short_tiles))) return rc;
  return combine_launch(y, token_pairs, count, n_tokens, H, E, (bf16_t*)out_bf16, st);
}

extern "C" int pp_moe_prefill_routed(const void* x, int x_dtype, int64_t n_tokens, int H,
                                     const float* router_packed, const float* bias, int E, int G, float tau,
                                     const void* packed, void* out_bf16, void* workspace, float* logits_out,
                                     uint8_t* mask_out, void* stream) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(n_tokens >= 0 && n_tokens <= (int64_t)0x7fffffff / PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED,
             "pp_moe_prefill: n_tokens %lld out of range", (long long)n_tokens);
  PP_REQUIRE(x_dtype == PP_DTYPE_F32 || x_dtype == PP_DTYPE_BF16, PP_ERR_INVALID, "pp_moe_prefill: x_dtype %d",
             x_dtype);
  if (n_tokens == 0) return PP_OK;
  PP_REQUIRE(x && router_packed && packed && out_bf16 && workspace, PP_ERR_INVALID, "pp_moe_prefill: null pointer");
  PP_REQUIRE(((uintptr_t)mask_out & 3) == 0, PP_ERR_INVALID, "pp_moe_prefill: mask_out must be 4-byte aligned");
  if (prefill_dense_form(G))
    return pp_dense_prefill(x, x_dtype, n_tokens, H, router_packed, bias, E, G, tau, packed, out_bf16, workspace,
                            (hipStream_t)stream, logits_out, mask_out);
  const int64_t nc = prefill_pass_tokens(n_tokens, H, E);
  const size_t xs = x_dtype == PP_DTYPE_BF16 ? 2 : 4;
  for (int64_t n0 = 0; n0 < n_tokens; n0 += nc) {
    const int64_t nt = min(nc, n_tokens - n0);
    if ((rc = prefill_pass((const char*)x + (size_t)n0 * H * xs, x_dtype, nt, H, router_packed, bias, E, G, tau,
                           packed, (bf16_t*)out_bf16 + (size_t)n0 * H, workspace, (hipStream_t)stream,
                           logits_out ? logits_out + n0 * E : nullptr, mask_out ? mask_out + n0 * E : nullptr)))
      return rc;
  }
  return PP_OK;
}

extern "C" int pp_moe_prefill(const void* x, int x_dtype, int64_t n_tokens, int H, const float* router_packed,
                              const float* bias, int E, int G, float tau, const void* packed, void* out_bf16,
                              void* workspace, void* stream) {
  return pp_moe_prefill_routed(x, x_dtype, n_tokens, H, router_packed, bias, E, G, tau, packed, out_bf16, workspace,
                               nullptr, nullptr, stream);
}
