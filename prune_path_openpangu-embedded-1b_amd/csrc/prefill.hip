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

// ------------------------------------------------------------------ pipelined grouped GEMM
// Tile 128 rows x 128 B-rows x BK=64 on v_mfma_f32_32x32x16_bf16, 4 waves as 2 x 2
// (wave tile 64 x 64), two workgroups per CU, persistent over (row tile, column tile)
// items. Operands go straight from global memory into LDS (global_load_lds_dwordx4:
// lane i of a wave writes bytes [16 i, 16 i + 16) of the wave's 1 KB block, no VGPR
// staging), two 32 KB LDS stages: the DMA of K block kb+1 runs under the MFMAs of kb.
//
// A tile row holds 64 bf16 = 8 chunks of 16 bytes; chunk c of row r is stored at
// position c ^ ((r >> 1) & 7). A fragment read (ds_read_b128) covers 32 consecutive
// rows; any 16 of them then land in 16 distinct 16-byte slots of a 256-byte bank
// window, and any 8 in 8 distinct slots of a 128-byte window.
//
// Synchronisation is explicit: the compiler cannot tell that an LDS read does not
// alias a DMA still in flight and would drain every prefetch before each read, and
// __syncthreads() adds a release fence that does the same. So fragment reads are
// inline ds_read_b128 whose results are fenced by s_waitcnt lgkmcnt tied to the
// fragment registers, and the per-K-block barrier waits only for this wave's DMA of
// the block about to be read.
#define GV_STAGES 2
#define GV_TILE_BYTES (128 * 64 * 2)               // one operand tile of one stage
#define GV_STAGE_BYTES (2 * GV_TILE_BYTES)         // A + B
typedef __attribute__((address_space(3))) void lds_void_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void gl2lds(const void* src, unsigned char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, 0);
}

__device__ __forceinline__ int gv_swz(int r) { return (r >> 1) & 7; }

template <int IMM>
__device__ __forceinline__ u32x4 gv_read(uint32_t lds_addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(lds_addr), "i"(IMM));
  return v;
}

// Wait until at most N LDS reads are outstanding; ties the four fragments of the
// current k-step so that their MFMAs cannot be scheduled above the wait.
template <int N>
__device__ __forceinline__ void gv_wait(u32x4& a0, u32x4& a1, u32x4& b0, u32x4& b1) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1) : "n"(N));
}

__device__ __forceinline__ f32x16_t mfma32v(u32x4 a, u32x4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// Item order: workgroup b runs on XCD b % 8 (round-robin dispatch); XCD x takes the
// contiguous item range [x * chunk, (x + 1) * chunk), so the column tiles of one row
// tile, and the row tiles of one expert, share that XCD's L2. gridDim.x is a multiple
// of 8.
struct GvItems {
  int first, last, step;
  __device__ GvItems(int n_items) {
    const int xcd = blockIdx.x & 7, per = gridDim.x >> 3;
    const int chunk = (n_items + 7) >> 3;
    first = xcd * chunk + (blockIdx.x >> 3);
    last = min(n_items, (xcd + 1) * chunk);
    step = per;
  }
};

// One item = (tile t, column block nt). A rows: a_row(i) = element offset of the tile's
// row i (i < 128, already clamped to a valid row); B rows: b_row(j) likewise (j < 128).
// Accumulates the 128 x 128 product over K (multiple of 64) into acc[2][2] of each wave.
template <typename AROW, typename BROW>
__device__ __forceinline__ void gv_mainloop(unsigned char* smem, AROW a_row, BROW b_row, int K,
                                            f32x16_t (&acc)[2][2]) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  // DMA assignment: instruction i covers rows 32 i + 8 w + lane/8, chunk position lane%8
  int64_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 32 * i + 8 * w + (lane >> 3);
    const int pchunk = ((lane & 7) ^ gv_swz(r)) * 8;  // logical chunk stored at this lane's position
    aoff[i] = a_row(r) + pchunk;
    boff[i] = b_row(r) + pchunk;
  }
  // fragment read addresses per k-step: row (lane & 31) of the wave's 32-row blocks
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  uint32_t offA[4], offB[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int r = lane & 31, c = ks * 2 + (lane >> 5);
    const uint32_t o = (uint32_t)(r * 8 + (c ^ gv_swz(r))) * 16;
    offA[ks] = lds0 + wm * 64 * 128 + o;
    offB[ks] = lds0 + GV_TILE_BYTES + wn * 64 * 128 + o;
  }
  const int nkb = K / 64;
  auto issue = [&](int kb, int st) {
    unsigned char* sb = smem + st * GV_STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int blk = (32 * i + 8 * w) * 128;  // wave's 1 KB block
      gl2lds(a_row.base + aoff[i] + kb * 64, sb + blk);
      gl2lds(b_row.base + boff[i] + kb * 64, sb + GV_TILE_BYTES + blk);
    }
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  issue(0, 0);
  int st = 0;
  for (int kb = 0; kb < nkb; ++kb) {
    // this wave's DMA of block kb has landed, every wave's after the barrier; all
    // waves are also done reading the other stage (block kb-1)
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const uint32_t sbase = st * GV_STAGE_BYTES;
    u32x4 fa[2][2], fb[2][2];
    fa[0][0] = gv_read<0>(offA[0] + sbase);
    fa[0][1] = gv_read<4096>(offA[0] + sbase);
    fb[0][0] = gv_read<0>(offB[0] + sbase);
    fb[0][1] = gv_read<4096>(offB[0] + sbase);
    // unconditional: past the end the last block is fetched again into the stage
    // everyone finished before the barrier, and never read
    issue(kb + 1 < nkb ? kb + 1 : nkb - 1, st ^ 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int cur = ks & 1, nxt = cur ^ 1;
      if (ks < 3) {
        fa[nxt][0] = gv_read<0>(offA[ks + 1] + sbase);
        fa[nxt][1] = gv_read<4096>(offA[ks + 1] + sbase);
        fb[nxt][0] = gv_read<0>(offB[ks + 1] + sbase);
        fb[nxt][1] = gv_read<4096>(offB[ks + 1] + sbase);
        gv_wait<4>(fa[cur][0], fa[cur][1], fb[cur][0], fb[cur][1]);
      } else {
        gv_wait<0>(fa[cur][0], fa[cur][1], fb[cur][0], fb[cur][1]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32v(fa[cur][i], fb[cur][j], acc[i][j]);
    }
    st ^= 1;
  }
  // the next item reuses both stages: drain the redundant tail DMA first
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct GvRows {  // row source: base pointer + per-row element offset function
  const bf16_t* base;
};

// gate/up with SwiGLU epilogue. B rows 0..63 = gate rows of neurons nb0..nb0+63,
// rows 64..127 = up rows of the same neurons; wave (wm, wn) takes rows wm*64.. and
// gate/up columns wn*32.. of each half, so lane-wise accG and accU line up.
__global__ __launch_bounds__(GM_THREADS, 2) void gateup_v2_kernel(
    const bf16_t* __restrict__ xb, int H, int G, const bf16_t* __restrict__ wrows,
    const int32_t* __restrict__ token_ids, const float* __restrict__ pair_gates,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, bf16_t* __restrict__ act) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int n_ntile = G / 64;
  const GvItems it(meta[0] * n_ntile);
  for (int item = it.first; item < it.last; item += it.step) {
    const int t = item / n_ntile, nt = item % n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int nb0 = nt * 64;
    struct ARow { const bf16_t* base; const int32_t* tok; int p0, rows, H;
      __device__ int64_t operator()(int r) const { return (int64_t)tok[p0 + (r < rows ? r : 0)] * H; } };
    struct BRow { const bf16_t* base; int e, G, nb0, H;
      __device__ int64_t operator()(int r) const {
        const int part = r < 64 ? 0 : 1;
        return ((int64_t)(e * G + nb0 + (r & 63)) * 3 + part) * H; } };
    ARow ar{xb, token_ids, p0, rows, H};
    BRow br{wrows, e, G, nb0, H};
    f32x16_t acc[2][2];
    // wave columns: gate block j=0 -> B rows wn*32.., up block j=1 -> B rows 64 + wn*32..
    // gv_mainloop takes B rows wn*64 + j*32; remap so that j=0 is gate and j=1 is up
    struct BRowPerm { const bf16_t* base; BRow inner;
      __device__ int64_t operator()(int r) const {
        // tile row r = wn*64 + j*32 + q  ->  gate/up row (j*64) + wn*32 + q
        const int wn_ = r >> 6, j = (r >> 5) & 1, q = r & 31;
        return inner(j * 64 + wn_ * 32 + q); } };
    BRowPerm bp{wrows, br};
    gv_mainloop(smem, ar, bp, H, acc);
    const int neuron = nb0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int r = wm * 64 + i * 32 + mfma32_row(q, lane);
        if (r < rows) {
          const int p = p0 + r;
          act[(int64_t)p * G + neuron] = f32_to_bf16(pp_silu(acc[i][0][q]) * acc[i][1][q] * pair_gates[p]);
        }
      }
    }
  }
}

// down projection: A = act rows (pairs), B = down_t rows (hidden columns), K = G
__global__ __launch_bounds__(GM_THREADS, 2) void down_v2_kernel(
    const bf16_t* __restrict__ act, int H, int G, const bf16_t* __restrict__ down_t,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ meta, float* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int n_ntile = H / 128;
  const GvItems it(meta[0] * n_ntile);
  for (int item = it.first; item < it.last; item += it.step) {
    const int t = item / n_ntile, nt = item % n_ntile;
    const int e = tiles[t * 4 + 0], p0 = tiles[t * 4 + 1], rows = tiles[t * 4 + 2];
    const int h0 = nt * 128;
    struct ARow { const bf16_t* base; int p0, rows, G;
      __device__ int64_t operator()(int r) const { return (int64_t)(p0 + (r < rows ? r : 0)) * G; } };
    struct BRow { const bf16_t* base; int e, H, h0, G;
      __device__ int64_t operator()(int r) const { return ((int64_t)e * H + h0 + r) * G; } };
    ARow ar{act, p0, rows, G};
    BRow br{down_t, e, H, h0, G};
    f32x16_t acc[2][2];
    gv_mainloop(smem, ar, br, G, acc);
#pragma unroll
    for (int i = 0; i < 2; ++i)
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

static int gemm_grid_v2(int64_t items) {  // two workgroups per CU, a multiple of 8 (XCD order)
  int64_t g = 2 * (int64_t)pp_device_cus();
  if (items < g) g = items;
  g = (g + 7) / 8 * 8;
  return (int)(g < 8 ? 8 : g);
}

static int gateup_launch(const bf16_t* xb, int H, int G, const bf16_t* wrows, int E, const int32_t* token_ids,
                         const float* pair_gates, const int32_t* tiles, const int32_t* meta, int64_t max_tiles,
                         bf16_t* act, hipStream_t st) {
  (void)E;
  if (G % 64 == 0) {
    int grid = gemm_grid_v2(max_tiles * (G / 64));
    gateup_v2_kernel<<<grid, GM_THREADS, GV_STAGES * GV_STAGE_BYTES, st>>>(xb, H, G, wrows, token_ids, pair_gates,
                                                                          tiles, meta, act);
  } else {
    int grid = gemm_grid(max_tiles * (G / 32));
    gateup_kernel<4, 1, 1><<<grid, GM_THREADS, 0, st>>>(xb, H, G, wrows, token_ids, pair_gates, tiles, meta, act);
  }
  return pp_check_launch("gateup_kernel");
}

static int down_launch(const bf16_t* act, int H, int G, const bf16_t* down_t, const int32_t* tiles,
                       const int32_t* meta, int64_t max_tiles, float* y, hipStream_t st) {
  if (G % 64 == 0) {
    int grid = gemm_grid_v2(max_tiles * (H / 128));
    down_v2_kernel<<<grid, GM_THREADS, GV_STAGES * GV_STAGE_BYTES, st>>>(act, H, G, down_t, tiles, meta, y);
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
