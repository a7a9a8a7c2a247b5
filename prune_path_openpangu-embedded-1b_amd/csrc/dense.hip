// Dense prefill form: the shapes whose experts are narrower than one MFMA column tile
// (G % 64 != 0; the checkpoint's E = 192 experts of G = 32 neurons). There a grouped
// per-expert GEMM has no tiling (each selected pair's down projection is a K = 32 product
// writing a full fp32 row of H, ~1 GB of partial rows at 2048 tokens), so the layer runs
// over every (token, neuron) with the router's gate as a per-(token, expert) factor that
// is exactly 0 for the experts a token does not select:
//   route_logits_kernel    fp32 logits x . Wr (+ bias), LDS-staged fp32 MFMA
//                          (v_mfma_f32_16x16x4_f32); every logit is summed in one fixed
//                          order, whatever the batch: a token routes the same way in any
//                          batch and at any position
//   route_select_wg_kernel (route.hip) the tau selection, bit-exact given the logits
//   dense_gemm_kernel<0>   act[t, n] = bf16(silu(x_t . Wg_n) * (x_t . Wu_n) * gate[t, n / G]),
//                          0 where the expert is not selected (never evaluated: no
//                          inf * 0 from an unselected expert reaches the output)
//   dense_gemm_kernel<1>   out[t, h] = bf16(sum over all neurons n of act[t, n] * Wd[n, h]),
//                          fp32 accumulation, one rounding
// Replaces moe_fused_expert_kernel (src/tl_kernel_optimized_Ultimate_PanGU.py:271-328) and
// the TauSparseMoE.forward_prefill orchestration (:532-604) at these shapes, with the
// reference's rounding points: bf16 act (acc_gate.to(bfloat16), :318-321) and fp32 sums
// of the per-expert down products.
//
// GEMM tiles: BM token rows x BN columns (BN/2 neurons as gate and up, or BN hidden
// columns), K blocks of BK bf16, NW waves in WR wave rows, each owning a BM/WR x BN/(NW/WR)
// wave tile of v_mfma_f32_32x32x16_bf16 blocks (accumulators in AGPRs: one workgroup per
// CU). Operands go global -> LDS by DMA (global_load_lds_dwordx4, no VGPR staging)
// through STAGES stages; the stream of K blocks runs across a workgroup's items (GpSched:
// whole items in full rounds, then the tail items cut into K ranges whose fp32 partial
// sums are joined by the part drawing the last ticket, in part order).
#include <algorithm>

#include "gemm_lds.h"

#define DG_MAX_GRID 256  // workgroups of a GEMM launch; also the split workspace's part slots
#ifndef DG_GU_GR
#define DG_GU_GR (1 << 30)  // gate/up items: every row tile of a column tile, then the next
#endif
#ifndef DG_DN_GR
// down items: pairs of row tiles, taken column by column. Every part of a K-split item goes
// to the same XCD, so an XCD holds 2 row tiles x 4 column tiles of the 8 x 8 at 2048 tokens:
// act blocks are fetched by 4 XCDs instead of all 8 (TCC hit rate of the launch 0.29 -> 0.47,
// 63 -> 56 us)
#define DG_DN_GR 2
#endif
#define DG_NPMAX 8       // K parts of a split tile at most
#ifndef DG_SPIN
#define DG_SPIN 4000     // polls (s_sleep 2, ~50 ns each) for the sibling parts of a split tile
#endif

// silu(g) = g * sigmoid(g) with the hardware exp2 and reciprocal (~1 ulp each): the act is
// rounded to bf16 right after, 2^-9 relative.
__device__ __forceinline__ float dg_silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

template <int BM, int BN, int BK, int NW, int WR>
struct Dg {
  static constexpr int NT = NW * 64;           // threads
  static constexpr int WN = NW / WR;           // wave columns (WR wave rows)
  static constexpr int WM = BM / WR;           // rows of a wave tile
  static constexpr int WC = BN / WN;           // columns of a wave tile
  static constexpr int MI = WM / 32;           // 32-row MFMA blocks per wave
  static constexpr int NJ = WC / 32;           // 32-column MFMA blocks per wave
  static constexpr int NF = MI * NJ * 16;      // fp32 accumulators per thread
  static constexpr int ROWB = BK * 2;          // bytes of one tile row in a stage
  static constexpr int CH = BK / 8;            // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROWB;      // rows per DMA instruction (a wave's 1 KB)
  static constexpr int NIA = BM / (NW * RPI);  // DMA instructions per wave per block, A
  static constexpr int NIB = BN / (NW * RPI);  // ... B (BN columns)
  static constexpr int DMA = NIA + NIB;
  static constexpr int KS = BK / 16;           // MFMA k-steps per block
  static constexpr int TA = BM * ROWB;         // A tile bytes per stage
  static constexpr int STAGE = TA + BN * ROWB;
  static constexpr int EPW = STAGE / NW;       // epilogue staging bytes per wave (in a free stage)
  // chunk c of row r sits at c ^ swz(r): the 16 rows any 16 lanes of a fragment read
  // touch fall in 16 distinct 16-byte slots of a 256-byte bank window
  __host__ __device__ static int swz(int r) { return BK == 64 ? (r >> 1) & 7 : (r >> 2) & 3; }
};

struct DgArgs {
  const bf16_t* a;  // MODE 0: x bf16 [N][H]; MODE 1: act bf16 [N][Ipad]
  const bf16_t* b;  // MODE 0: packed neuron records [I][3][H]; MODE 1: down_t [E][H][G]
  const float* gates;  // MODE 0: [N][E], 0 where not selected
  bf16_t* out;         // MODE 0: act [N][Ipad]; MODE 1: out [N][H]
  float* part;         // split partial sums (null: no split)
  uint32_t* sync;      // split tickets, zero at launch and left zero
  int64_t N;
  int H, E, G, I, Ipad;
  int ct_lo, ct_hi;  // column tiles [ct_lo, ct_hi) of the launch's tile width
};

// Wait until at most N LDS reads are outstanding, then tie the fragments of the current
// k-step (an empty asm per fragment, after the wait in program order: volatile asm
// statements keep their order), so that their MFMAs cannot be scheduled above the wait.
template <int I, int M>
__device__ __forceinline__ void dg_tie(u32x4 (&v)[M]) {
  if constexpr (I < M) {
    asm volatile("" : "+v"(v[I]));
    dg_tie<I + 1, M>(v);
  }
}
template <int N, int MI, int NJ>
__device__ __forceinline__ void dg_wait(u32x4 (&a)[MI], u32x4 (&b)[NJ]) {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
  dg_tie<0, MI>(a);
  dg_tie<0, NJ>(b);
}

// fragments v[0 .. N) of 32-row blocks RB bytes apart from base (compile-time offsets)
template <int RB, int N, int I = 0>
__device__ __forceinline__ void dg_read(u32x4 (&v)[N], uint32_t base) {
  if constexpr (I < N) {
    v[I] = gv_read<I * RB>(base);
    dg_read<RB, N, I + 1>(v, base);
  }
}

// Epilogue rows per pass: the largest multiple of 32 that divides the wave tile's wm rows
// and is at most rp0 (what the wave's staging holds).
__host__ __device__ constexpr int dg_pass_rows(int wm, int rp0) {
  int r = wm;
  while (r > 32 && (r > rp0 || wm % r != 0)) r -= 32;
  return r;
}
static_assert(dg_pass_rows(128, 96) == 64 && dg_pass_rows(128, 128) == 128 && dg_pass_rows(64, 192) == 64 &&
                  dg_pass_rows(128, 64) == 64,
              "epilogue pass rows");

// Item -> (row tile rt, launch column tile ctl): row tiles in groups of gr, each group
// taken column by column (gr >= n_rt: every row tile of a column, then the next column).
// The workgroups of one XCD take consecutive items, so gr sets the block of row x column
// tiles that shares one L2.
__device__ __forceinline__ void dg_tile(int item, int n_rt, int n_ct, int gr, int& rt, int& ctl) {
  gr = min(gr, n_rt);
  const int q = item / (gr * n_ct);
  const int r = item - q * gr * n_ct;
  const int rows = min(gr, n_rt - q * gr);
  ctl = r / rows;
  rt = q * gr + (r - ctl * rows);
}

template <int MODE, int BM, int BN, int BK, int STAGES, int NW, int WR, int WPC>
__global__ __launch_bounds__(NW * 64, WPC) void dense_gemm_kernel(DgArgs p) {
  using C = Dg<BM, BN, BK, NW, WR>;
  constexpr int NB2 = BN / 2;  // MODE 0: neurons of a column tile (their gate and up rows)
  // MODE 0: experts a column tile can touch, rounded up to a power of two (G >= 32: a
  // 128-neuron tile touches at most 5, a 64-neuron tile 3)
  constexpr int GX = NB2 > 64 ? 8 : 4;
  static_assert(BM == 128 || BM == 256, "tile rows");
  static_assert(NW == 4 || NW == 8, "waves");
  static_assert(C::MI >= 1 && C::NJ >= 2 && (MODE == 1 || C::NJ % 2 == 0) && C::MI * 32 * WR == BM &&
                    C::NJ * 32 * C::WN == BN && C::NIA * NW * C::RPI == BM && C::NIB * NW * C::RPI == BN,
                "tile shape");
  static_assert(MODE == 1 || (NB2 + 31) / 32 + 1 <= GX, "experts a column tile can touch");
  static_assert(STAGES >= 2 && WPC * (STAGES * C::STAGE + (MODE == 0 ? BM * GX * 4 : 0) + 64) <= 160 * 1024,
                "LDS of WPC workgroups per CU");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int role_s;
  __shared__ float gate_s[MODE == 0 ? BM * GX : 1];  // MODE 0 epilogue: the tile's router gates
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int wm = w / C::WN, wn = w % C::WN;
  const int n_rt = (int)((p.N + BM - 1) / BM);
  const int n_ct = p.ct_hi - p.ct_lo;  // column tiles of this launch, from p.ct_lo
  const int nkb = (MODE == 0 ? p.H : p.Ipad) / BK;
  const int n_items = n_rt * n_ct;
  const GpSched sc(n_items, nkb, p.sync != nullptr, DG_NPMAX);
  const int F = sc.units(nkb);
  if (F <= 0) return;

  // ---- DMA issue cursor. Wave w, instruction i covers tile rows (NW i + w) * RPI .. + RPI;
  // lane l takes row (NW i + w) * RPI + l / CH and LDS chunk position l % CH, i.e. global
  // chunk (l % CH) ^ swz(row) -- the same chunk for every i of a wave (swz only sees row
  // bits the instruction index does not change). Item bases are uniform; lanes add 32-bit
  // byte offsets of their rows inside the item's tiles.
  const int gc8 = ((lane % C::CH) ^ C::swz(w * C::RPI + lane / C::CH)) * 8;
  const bool bk_whole = MODE == 1 && BK % p.G == 0;  // down: K blocks of whole experts (G = 32)
  // down, bk_whole: a lane's expert and offset inside every block
  const uint32_t lane_k = bk_whole ? (uint32_t)((gc8 / p.G) * p.H * p.G + gc8 % p.G) * 2u : 0u;
  const int arow = MODE == 0 ? p.H : p.Ipad;  // A row length (elements)
  const bf16_t* a_item = p.a;
  const bf16_t* b_item = p.b;
  uint32_t aoff[C::NIA], boff[C::NIB];
  auto setup_item = [&](int li) {
    const int item = sc.item(li);
    int ctl, rt;
    dg_tile(item, n_rt, n_ct, MODE == 0 ? DG_GU_GR : DG_DN_GR, rt, ctl);
    const int ct = p.ct_lo + ctl;
    const int64_t t0 = (int64_t)rt * BM;
    a_item = p.a + t0 * arow;
#pragma unroll
    for (int i = 0; i < C::NIA; ++i) {
      const int r = (NW * i + w) * C::RPI + lane / C::CH;
      const int tr = (int)(min(t0 + r, p.N - 1) - t0);  // rows past N repeat row N - 1, never stored
      aoff[i] = (uint32_t)(tr * arow + gc8) * 2u;
    }
    if (MODE == 0) {
      // B row r: wave column r / WC; 32-row block jb = (r % WC) / 32 is the gate (jb < NJ/2)
      // or up row of neuron ct * NB2 + (r / WC) * WC/2 + (jb % (NJ/2)) * 32 + (r & 31)
      b_item = p.b + (int64_t)ct * NB2 * 3 * p.H;
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) {
        const int r = (NW * i + w) * C::RPI + lane / C::CH;
        const int jb = (r % C::WC) >> 5;
        const int nl = min(ct * NB2 + (r / C::WC) * (C::WC / 2) + (jb % (C::NJ / 2)) * 32 + (r & 31), p.I - 1) -
                       ct * NB2;
        boff[i] = (uint32_t)((nl * 3 + jb / (C::NJ / 2)) * p.H + gc8) * 2u;
      }
    } else {
      b_item = p.b + (int64_t)ct * BN * p.G;
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) {
        const int r = (NW * i + w) * C::RPI + lane / C::CH;
        boff[i] = (uint32_t)((min(ct * BN + r, p.H - 1) - ct * BN) * p.G) * 2u + lane_k;
      }
    }
  };
  // MODE 1: this block's B lane offsets, held until the next issue: a DMA reads its address
  // registers after issue, and the compiler makes any earlier reuse of them wait for the DMA
  uint32_t bcur[C::NIB];
#pragma unroll
  for (int i = 0; i < C::NIB; ++i) bcur[i] = 0;
  auto issue = [&](int f) {
    int li, kb;
    sc.locate(f < F ? f : F - 1, nkb, li, kb);  // past the end: the last block again, never read
    if (f < F && (kb == 0 || f == sc.n_whole * nkb)) setup_item(li);
    const uint32_t sb = (uint32_t)(f % STAGES) * C::STAGE;
    const char* ab = (const char*)(a_item + (int64_t)kb * BK);
#pragma unroll
    for (int i = 0; i < C::NIA; ++i) gl2lds(ab + aoff[i], smem + sb + (NW * i + w) * 1024);
    if (MODE == 0) {
      const char* bb = (const char*)(b_item + (int64_t)kb * BK);
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) gl2lds(bb + boff[i], smem + sb + C::TA + (NW * i + w) * 1024);
    } else {
      // K index k = neuron: down_t[e][h][g] with e = k / G, g = k % G; block kb starts in
      // expert e0 at g0, and a lane's chunk (gc8 < 64, G >= 32) lies at most two experts on
      const int e0 = (kb * BK) / p.G;
      const char* bb = (const char*)(b_item + (int64_t)e0 * p.H * p.G);
      uint32_t lk = 0;
      if (!(bk_whole && (kb + 1) * BK <= p.I)) {
        int de = 0, g = kb * BK - e0 * p.G + gc8;
        if (g >= p.G) g -= p.G, ++de;
        if (g >= p.G) g -= p.G, ++de;
        if (kb * BK + gc8 >= p.I)  // the zero act columns of the pad: any in-range weight
          de = p.E - 1 - e0, g = p.G - 8;
        lk = (uint32_t)(de * p.H * p.G + g) * 2u - lane_k;
      }
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) {
        asm volatile("" ::"v"(bcur[i]));  // the previous block's offsets live up to here
        bcur[i] = boff[i] + lk;
        asm volatile("" : "+v"(bcur[i]));  // a register of its own, not shared with boff
        gl2lds(bb + bcur[i], smem + sb + C::TA + (NW * i + w) * 1024);
      }
    }
  };

  // ---- fragment addresses: A rows wm * BM/2 + 32 i + l % 32, B rows wn * WC + 32 j + l % 32,
  // chunk 2 ks + l / 32
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  uint32_t offA[C::KS], offB[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    const int r = lane & 31, c = ks * 2 + (lane >> 5);
    const uint32_t o = (uint32_t)(r * C::CH + (c ^ C::swz(r))) * 16;
    offA[ks] = lds0 + wm * C::WM * C::ROWB + o;
    offB[ks] = lds0 + C::TA + wn * C::WC * C::ROWB + o;
  }

#pragma unroll
  for (int f = 0; f < STAGES - 1; ++f) issue(f);

  constexpr int RB = 32 * C::ROWB;  // bytes between 32-row fragment blocks
  const int n_local = sc.n_local();
  int f = 0;  // unit (item, K block) being computed
  for (int li = 0; li < n_local; ++li) {
    const bool part = li >= sc.n_whole;
    const int kb_end = part ? sc.kb_hi : nkb;
    f32x16_t acc[C::MI][C::NJ];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NJ; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
    // MODE 0: the tile's router gates (rows x the experts its 128 neurons touch), loaded at
    // the item's first block and written to gate_s at its second: ready for the epilogue
    // without a memory round trip there (gate_s[r * GX + k]: row r, expert e_lo + k)
    constexpr int NGL = MODE == 0 ? BM * GX / C::NT : 1;
    float gl[NGL];
    const int kb_first = part ? sc.kb_lo : 0;
    auto gates_store = [&]() {
#pragma unroll
      for (int c = 0; c < NGL; ++c) gate_s[tid + c * C::NT] = gl[c];
    };
    for (int kb = kb_first; kb < kb_end; ++kb, ++f) {
      gp_wait_barrier<C::DMA * (STAGES - 2)>();
      issue(f + STAGES - 1);
      if (MODE == 0 && kb == kb_first) {
        const int item = sc.item(li);
        int ctl, rt;
    dg_tile(item, n_rt, n_ct, MODE == 0 ? DG_GU_GR : DG_DN_GR, rt, ctl);
    const int ct = p.ct_lo + ctl;
        const int e_lo = ct * NB2 / p.G;
        const int ne = min(p.E, (ct * NB2 + NB2 - 1) / p.G + 1) - e_lo;
        const int64_t tt0 = (int64_t)rt * BM;
#pragma unroll
        for (int c = 0; c < NGL; ++c) {
          const int idx = tid + c * C::NT, r = idx / GX, k = idx % GX;
          gl[c] = (k < ne && tt0 + r < p.N) ? p.gates[(tt0 + r) * p.E + e_lo + k] : 0.0f;
        }
      } else if (MODE == 0 && kb == kb_first + 1) {
        gates_store();
      }
      const uint32_t sbase = (f % STAGES) * C::STAGE;
      u32x4 fa[2][C::MI], fb[2][C::NJ];
      auto rd = [&](int ks, u32x4(&a)[C::MI], u32x4(&b)[C::NJ]) {
        dg_read<RB>(a, offA[ks] + sbase);
        dg_read<RB>(b, offB[ks] + sbase);
      };
      rd(0, fa[0], fb[0]);
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        const int cur = ks & 1, nxt = cur ^ 1;
        if (ks < C::KS - 1) {
          rd(ks + 1, fa[nxt], fb[nxt]);
          dg_wait<C::MI + C::NJ, C::MI, C::NJ>(fa[cur], fb[cur]);
        } else {
          dg_wait<0, C::MI, C::NJ>(fa[cur], fb[cur]);
        }
#pragma unroll
        for (int i = 0; i < C::MI; ++i)
#pragma unroll
          for (int j = 0; j < C::NJ; ++j) acc[i][j] = mfma32v(fa[cur][i], fb[cur][j], acc[i][j]);
      }
    }
    const int fl = f - 1;  // the unit just computed: its stage is free once every wave is done with it
    if (MODE == 0 && kb_end - kb_first == 1) gates_store();  // a one-block item

    // ---- the item's (or part's) last block: join the parts, then the epilogue. Memory is
    // addressed as a uniform base (laundered through an SGPR asm operand, so the compiler
    // cannot precompute every address ahead of the loop) plus a 32-bit lane offset.
    if (part) {
      // Split tile: every part stores its fp32 sums (agent-scope stores), then counts itself
      // in. The tile's output is cut into np slabs of accumulator words, handed out by a
      // counter to the parts that have seen all np arrive (the last to arrive sees it at
      // once; the others poll, bounded): each slab is reduced once, in part order -- the
      // same bits whoever reduces it -- and written out. A part that stops polling (a
      // sibling not yet scheduled) just leaves its slabs to the others. The counters are
      // zeroed by the call's routing kernel, one set per GEMM launch.
      const int pi = sc.unit % sc.nparts, u0 = sc.unit - pi, np = sc.nparts;
      uint32_t* sy = p.sync + 2 * (sc.part_item - sc.tail0);  // [0] arrivals, [1] next slab
      constexpr size_t SLOT = (size_t)C::NF * C::NT * 4;      // bytes of one part's sums
      constexpr int WS = C::NT * 8;                           // 64-bit word w of thread tid: w * WS + tid * 8
      const uint32_t lo = (uint32_t)tid * 8u;
#pragma unroll
      for (int b = 0; b < C::MI * C::NJ; ++b) {
        size_t o = (size_t)sc.unit * SLOT + (size_t)b * 8 * WS;
        asm volatile("" : "+s"(o));
        char* bp = (char*)p.part + o;
        f32x16_t blk = acc[b / C::NJ][b % C::NJ];
        asm volatile("" : "+v"(blk));  // one 16-float block in VGPRs at a time
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const unsigned long long v = (unsigned long long)__float_as_uint(blk[2 * c]) |
                                       ((unsigned long long)__float_as_uint(blk[2 * c + 1]) << 32);
          __hip_atomic_store((unsigned long long*)(bp + c * WS + lo), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // every thread's stores performed
      if (tid == 0) {
        int all = (int)__hip_atomic_fetch_add(sy, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
        for (int it = 0; !all && it < DG_SPIN; ++it) {
          __builtin_amdgcn_s_sleep(2);
          all = (int)__hip_atomic_load(sy, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= np;
        }
        role_s = all;
      }
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (!role_s) break;  // uniform; a part is a workgroup's last unit
      // this thread's words: those thread tid of every part stored (the same output
      // positions as its own accumulators); MODE 0 reduces gate words with their up words.
      // A slab's words of every part are DMA'd into the (now free) stages in chunks, all of a
      // chunk in flight at once (agent-coherent loads: sc1), then summed from LDS.
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int item = sc.item(li);
      int ctl, rt;
    dg_tile(item, n_rt, n_ct, MODE == 0 ? DG_GU_GR : DG_DN_GR, rt, ctl);
    const int ct = p.ct_lo + ctl;
      const int64_t t0 = (int64_t)rt * BM + wm * C::WM;
      const int rows_in = (int)min((int64_t)C::WM, max((int64_t)0, p.N - t0));
      constexpr int NG = MODE == 0 ? C::NF / 4 : C::NF / 2;  // words per thread to reduce
      constexpr int HW = MODE == 0 ? 2 : 1;                   // words per reduced unit
      const int upc = (STAGES * C::STAGE) / (np * HW * WS);   // units per LDS chunk
      for (;;) {
        asm volatile("s_barrier" ::: "memory");  // every thread has read role_s, every LDS read done
        if (tid == 0) role_s = (int)__hip_atomic_fetch_add(sy + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int slab = role_s;
        if (slab >= np) break;
        const int g_lo = slab * NG / np, g_hi = (slab + 1) * NG / np;
        for (int c0 = g_lo; c0 < g_hi; c0 += upc) {
          const int cn = min(upc, g_hi - c0);
          // DMA: 1 KB pieces m = ((q * cn + k) * HW + hh) * (WS / 1024) + quarter
          const int total = np * cn * HW * (WS / 1024);
          for (int m = w; m < total; m += NW) {
            const int quarter = m % (WS / 1024), r1 = m / (WS / 1024);
            const int hh = r1 % HW, r2 = r1 / HW, k = r2 % cn, q = r2 / cn;
            const int gw = c0 + k, b = gw / 8, c = gw % 8;
            const int wg = MODE == 0 ? ((b / (C::NJ / 2)) * C::NJ + b % (C::NJ / 2) + hh * (C::NJ / 2)) * 8 + c : gw;
            const char* src = (const char*)p.part + (size_t)(u0 + q) * SLOT + (size_t)wg * WS + quarter * 1024 + ln * 16;
            __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(smem + m * 1024), 16, 0, 16);
          }
          asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
          for (int k = 0; k < cn; ++k) {
            const int gw = c0 + k, b = gw / 8, c = gw % 8;
            float sv[2] = {0.f, 0.f}, tv[2] = {0.f, 0.f};
            for (int q = 0; q < np; ++q) {
              const uint2 a = *(const uint2*)(smem + (size_t)((q * cn + k) * HW) * WS + tid * 8);
              sv[0] = q == 0 ? __uint_as_float(a.x) : __fadd_rn(sv[0], __uint_as_float(a.x));
              sv[1] = q == 0 ? __uint_as_float(a.y) : __fadd_rn(sv[1], __uint_as_float(a.y));
              if (MODE == 0) {
                const uint2 u2 = *(const uint2*)(smem + (size_t)((q * cn + k) * HW + 1) * WS + tid * 8);
                tv[0] = q == 0 ? __uint_as_float(u2.x) : __fadd_rn(tv[0], __uint_as_float(u2.x));
                tv[1] = q == 0 ? __uint_as_float(u2.y) : __fadd_rn(tv[1], __uint_as_float(u2.y));
              }
            }
            const int i = MODE == 0 ? b / (C::NJ / 2) : b / C::NJ;
            const int col = (MODE == 0 ? b % (C::NJ / 2) : b % C::NJ) * 32 + (ln & 31);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int rl = i * 32 + mfma32_row(2 * c + h, ln);
              if (rl >= rows_in) continue;
              if (MODE == 0) {
                const int n = ct * NB2 + wn * (C::WC / 2) + col;
                if (n >= p.Ipad) continue;
                const float gt = n < p.I ? gate_s[(wm * C::WM + rl) * GX + n / p.G - ct * NB2 / p.G] : 0.0f;
                const float a = gt == 0.0f ? 0.0f : dg_silu(sv[h]) * tv[h] * gt;
                p.out[(t0 + rl) * p.Ipad + n] = f32_to_bf16(a);
              } else {
                const int hc = ct * BN + wn * C::WC + col;
                if (hc < p.H) p.out[(t0 + rl) * p.H + hc] = f32_to_bf16(sv[h]);
              }
            }
          }
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // LDS reads done before the next chunk
        }
      }
      break;
    }
    // ---- epilogue: the wave's results go through its share of the free stage (bf16, row
    // major), then out as 16-byte row chunks: coalesced stores, no 2-byte scatter. Passes of
    // RP rows x GB 32-column blocks (as many as the wave's EPW bytes hold).
    {
      int ln = lane;
      asm volatile("" : "+v"(ln));  // keep the epilogue's lane math out of the main loop's registers
      const int item = sc.item(li);
      int ctl, rt;
    dg_tile(item, n_rt, n_ct, MODE == 0 ? DG_GU_GR : DG_DN_GR, rt, ctl);
    const int ct = p.ct_lo + ctl;
      const int64_t t0 = (int64_t)rt * BM + wm * C::WM;  // this wave's first output row
      const int rows_in = (int)min((int64_t)C::WM, max((int64_t)0, p.N - t0));
      unsigned char* ep = smem + (fl % STAGES) * C::STAGE + w * C::EPW;
      constexpr int NB = MODE == 0 ? C::NJ / 2 : C::NJ;  // 32-column output blocks of the wave
      constexpr int GB0 = C::EPW / (32 * 64);            // blocks of 32 rows the staging holds
      constexpr int GB = GB0 < NB ? GB0 : NB;            // blocks per pass
      constexpr int RW = GB * 64;                        // bytes of an LDS row
      constexpr int RP0 = C::EPW / RW / 32 * 32;
      constexpr int RP = dg_pass_rows(C::WM, RP0);       // rows per pass
      static_assert(GB >= 1 && RP >= 32 && C::WM % RP == 0, "epilogue passes");
      const int c0 = MODE == 0 ? ct * NB2 + wn * (C::WC / 2) : ct * BN + wn * C::WC;  // first column
      const int ncol = MODE == 0 ? p.Ipad : p.H;
      const int cols_in = min(NB * 32, ncol - c0);
      int64_t oo = t0 * ncol + c0;
      asm volatile("" : "+s"(oo));
      bf16_t* ob = p.out + oo;
      const int e_lo = MODE == 0 ? ct * NB2 / p.G : 0;
      if (MODE == 0)
        __syncthreads();  // gates staged; every wave done reading the free stage
      else
        asm volatile("s_barrier" ::: "memory");  // every wave done reading the free stage
#pragma unroll
      for (int hf = 0; hf < C::WM / RP; ++hf) {
#pragma unroll
        for (int jg = 0; jg < NB; jg += GB) {
#pragma unroll
          for (int jj = jg; jj < (jg + GB < NB ? jg + GB : NB); ++jj) {
            const int nl = jj * 32 + (ln & 31);  // column inside the wave's NB * 32
            const int ek = MODE == 0 ? (c0 + nl) / p.G - e_lo : 0;
            const bool real = MODE == 0 && c0 + nl < p.I;  // neurons of the pad [I, Ipad) get act 0
#pragma unroll
            for (int i = hf * (RP / 32); i < (hf + 1) * (RP / 32); ++i) {
              if (MODE == 0) {
                f32x16_t gv = acc[i][jj], uv = acc[i][jj + NB];
                asm volatile("" : "+v"(gv), "+v"(uv));  // two 16-float blocks in VGPRs at a time
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                  const int rl = i * 32 + mfma32_row(q, ln);
                  const float gt = real ? gate_s[(wm * C::WM + rl) * GX + ek] : 0.0f;
                  const float a = gt == 0.0f ? 0.0f : dg_silu(gv[q]) * uv[q] * gt;
                  *(bf16_t*)(ep + (rl - hf * RP) * RW + (nl - jg * 32) * 2) = f32_to_bf16(a);
                }
              } else {
                f32x16_t v = acc[i][jj];
                asm volatile("" : "+v"(v));  // one 16-float block in VGPRs at a time
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                  const int rl = i * 32 + mfma32_row(q, ln);
                  *(bf16_t*)(ep + (rl - hf * RP) * RW + (nl - jg * 32) * 2) = f32_to_bf16(v[q]);
                }
              }
            }
          }
          // out: row rl of the pass, 16-byte chunk c of its GB * 64 bytes
          constexpr int CPR = RW / 16;
          static_assert((RP * CPR) % 64 == 0, "epilogue chunks");
#pragma unroll
          for (int k = 0; k < RP * CPR / 64; ++k) {
            const int idx = ln + 64 * k, rl = idx / CPR, c = idx % CPR;
            const uint4 v = *(const uint4*)(ep + rl * RW + c * 16);
            const int rg = hf * RP + rl, cg = jg * 32 + c * 8;
            if (rg < rows_in && cg < cols_in && cg < (jg + GB) * 32) *(uint4*)(ob + rg * ncol + cg) = v;
          }
        }
      }
    }
  }
  // the redundant tail DMAs must land before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ------------------------------------------------------------------ router logits (E > 16)
// Logits of 32 tokens x 16 TE experts per workgroup of eight waves on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32), two waves per SIMD. x and the router rows pass through LDS in K chunks of RL_KC
// (RL_STAGES stages, DMA RL_STAGES - 1 chunks ahead; every DMA instruction moves whole
// rows, two 512-byte fp32 rows or four 256-byte bf16 rows). 16-byte chunk c of LDS row r
// sits at c ^ (r & 15): the sixteen rows a fragment read touches fall in distinct bank
// slots. Wave w takes the 32-wide K block w % 4 of every chunk for the 16-token tile
// w / 4; lane (t = l % 16, g = l / 16)
// holds x[t][k + 8 g + j] and W[expert l % 16][k + 8 g + j], j = 0..7, one MFMA per j per
// 16 x 16 tile, so each k of the block is used exactly once. Each tile accumulates in
// chunk order, j order; the four K-block partials are added in block order, then the bias:
// one fixed order per (token, expert) whatever N or the token's position, so a token
// routes the same way in any batch. Result lane l, element q: token 4 (l / 16) + q,
// expert l % 16 of the tile.
#define RL_TT 2
#define RL_KC 128
#define RL_STAGES 3
template <typename XT, int TE>
struct Rl {
  static constexpr int XROW = RL_KC * (int)sizeof(XT);  // x row bytes in a stage
  static constexpr int WROW = RL_KC * 4;                // router row bytes in a stage
  static constexpr int XB = 16 * RL_TT * XROW;
  static constexpr int STAGE = XB + 16 * TE * WROW;
  static constexpr int XI = XB / 8192;               // DMA instructions per wave per chunk, x
  static constexpr int WI = 16 * TE * WROW / 8192;   // ... router
  static constexpr int DMA = XI + WI;
};

// One wave DMA instruction over rows of RB bytes (RB = 256 or 512) starting at LDS row
// row0: lane l takes row row0 + l / (RB / 16), LDS chunk position l % (RB / 16), global
// chunk (l % (RB / 16)) ^ (row & 15); src(row) is the row's first element of the chunk.
template <int RB, typename T, typename Src>
__device__ __forceinline__ void rl_dma(Src&& src, int row0, unsigned char* lds_region, int lane) {
  constexpr int CPR = RB / 16;
  const int row = row0 + lane / CPR;
  const int gc = (lane % CPR) ^ (row & 15);
  gl2lds(src(row) + gc * (16 / (int)sizeof(T)), lds_region + row0 * RB);
}

template <typename XT, int TE>
__global__ __launch_bounds__(512, 1) void route_logits_kernel(const XT* __restrict__ x, int64_t N, int H,
                                                              const float* __restrict__ router, int Epad,
                                                              const float* __restrict__ bias, int E,
                                                              float* __restrict__ logits_out,
                                                              bf16_t* __restrict__ xbf_out, uint32_t* __restrict__ zero,
                                                              int nzero) {
  using R = Rl<XT, TE>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int kq = w & 3, ta = w >> 2;  // this wave's K block of a chunk and token tile
  const int64_t tok0 = (int64_t)blockIdx.x * (16 * RL_TT);
  const int e0 = (int)blockIdx.y * (16 * TE);
  if (zero && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = tid; i < nzero; i += 512) zero[i] = 0u;
  const int nch = H / RL_KC;
  auto issue = [&](int c) {
    const int cc = c < nch ? c : nch - 1;  // past the end: the last chunk again, never read
    unsigned char* st = smem + (c % RL_STAGES) * R::STAGE;
    const int k0 = cc * RL_KC;
#pragma unroll
    for (int i = 0; i < R::XI; ++i) {
      const int row0 = (8 * i + w) * (1024 / R::XROW);
      rl_dma<R::XROW, XT>([&](int r) { return x + min(tok0 + r, N - 1) * H + k0; }, row0, st, lane);
    }
#pragma unroll
    for (int i = 0; i < R::WI; ++i) {
      const int row0 = (8 * i + w) * (1024 / R::WROW);
      rl_dma<R::WROW, float>([&](int r) { return router + (int64_t)min(e0 + r, Epad - 1) * H + k0; }, row0,
                             st + R::XB, lane);
    }
  };
#pragma unroll
  for (int c = 0; c < RL_STAGES - 1; ++c) issue(c);

  const int t_l = lane & 15, g = lane >> 4;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)smem;
  f32x4_t acc[TE];
#pragma unroll
  for (int b = 0; b < TE; ++b) acc[b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; ++c) {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(R::DMA * (RL_STAGES - 2)) : "memory");
    issue(c + RL_STAGES - 1);
    // LDS reads through asm (lds_read16): ordered after this chunk's DMAs by the wait and
    // barrier above; plain loads would make the compiler wait for every DMA in flight,
    // the next chunks' included, before the first read
    const uint32_t sb = lds0 + (uint32_t)((c % RL_STAGES) * R::STAGE);
    u32x4 xq[2], wq[TE][2];
    {
      const int r = 16 * ta + t_l;
      if (sizeof(XT) == 4) {
        const int c0 = 8 * kq + 2 * g;
        xq[0] = lds_read16(sb + r * R::XROW + ((c0 ^ (r & 15)) << 4));
        xq[1] = lds_read16(sb + r * R::XROW + (((c0 + 1) ^ (r & 15)) << 4));
      } else {
        xq[0] = lds_read16(sb + r * R::XROW + (((4 * kq + g) ^ (r & 15)) << 4));
      }
    }
#pragma unroll
    for (int b = 0; b < TE; ++b) {
      const int r = 16 * b + t_l;
      const int c0 = 8 * kq + 2 * g;
      const uint32_t ws = sb + R::XB + r * R::WROW;
      wq[b][0] = lds_read16(ws + ((c0 ^ (r & 15)) << 4));
      wq[b][1] = lds_read16(ws + (((c0 + 1) ^ (r & 15)) << 4));
    }
    // x as bf16 for the GEMMs (fp32 x, first expert group only): thread -> row tid / 8,
    // 16 values at (tid % 8) * 16
    if (sizeof(XT) == 4 && xbf_out && blockIdx.y == 0 && tid < 256) {
      const int r = tid >> 3, k16 = (tid & 7) * 16;
      const int64_t t = tok0 + r;
      if (t < N) {
        u32x4 v4[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) v4[h] = lds_read16(sb + r * R::XROW + ((((k16 >> 2) + h) ^ (r & 15)) << 4));
        lds_wait_all(v4[0], v4[1], v4[2], v4[3]);
        uint32_t pk[8];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          pk[2 * h] = (uint32_t)f32_to_bf16(__uint_as_float(v4[h].x)) |
                      ((uint32_t)f32_to_bf16(__uint_as_float(v4[h].y)) << 16);
          pk[2 * h + 1] = (uint32_t)f32_to_bf16(__uint_as_float(v4[h].z)) |
                          ((uint32_t)f32_to_bf16(__uint_as_float(v4[h].w)) << 16);
        }
        uint4* dst = (uint4*)(xbf_out + t * H + c * RL_KC + k16);
        dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
      }
    }
    // no copy of a fragment may exist before its wait (a copy made earlier would hold the
    // registers' old contents): bf16 x waits on its one fragment alone
    if constexpr (sizeof(XT) == 4) lds_wait_all(xq[0], xq[1]);
    else lds_wait_all(xq[0]);
#pragma unroll
    for (int b = 0; b < TE; ++b) lds_wait_all(wq[b][0], wq[b][1]);
    float xv[8], wv[TE][8];
    if (sizeof(XT) == 4) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        xv[4 * h] = __uint_as_float(xq[h].x);
        xv[4 * h + 1] = __uint_as_float(xq[h].y);
        xv[4 * h + 2] = __uint_as_float(xq[h].z);
        xv[4 * h + 3] = __uint_as_float(xq[h].w);
      }
    } else {
      const uint32_t uw[4] = {xq[0].x, xq[0].y, xq[0].z, xq[0].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[2 * i] = __uint_as_float(uw[i] << 16);
        xv[2 * i + 1] = __uint_as_float(uw[i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int b = 0; b < TE; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        wv[b][4 * h] = __uint_as_float(wq[b][h].x);
        wv[b][4 * h + 1] = __uint_as_float(wq[b][h].y);
        wv[b][4 * h + 2] = __uint_as_float(wq[b][h].z);
        wv[b][4 * h + 3] = __uint_as_float(wq[b][h].w);
      }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int b = 0; b < TE; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[j], wv[b][j], acc[b], 0, 0, 0);
  }
  // wave partials through LDS (stage memory is free once every wave has passed here)
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  float* part = (float*)smem;  // [4 K blocks][32 tokens][16 TE]
  constexpr int NE = 16 * TE, NT = 16 * RL_TT;
#pragma unroll
  for (int b = 0; b < TE; ++b)
#pragma unroll
    for (int q = 0; q < 4; ++q) part[(kq * NT + 16 * ta + 4 * g + q) * NE + 16 * b + t_l] = acc[b][q];
  __syncthreads();
  for (int i = tid; i < NT * NE; i += 512) {
    const int r = i / NE, ce = i - r * NE;
    const int64_t t = tok0 + r;
    const int e = e0 + ce;
    if (t < N && e < E) {
      float l = part[r * NE + ce];
#pragma unroll
      for (int ww = 1; ww < 4; ++ww) l = __fadd_rn(l, part[(ww * NT + r) * NE + ce]);
      if (bias) l = __fadd_rn(l, bias[e]);
      logits_out[t * E + e] = l;
    }
  }
}

// Logits [N][E] of any E (Epad = E rounded up to 16 rows of router_packed); xbf_out (fp32 x
// only, may be null) receives x as bf16; zero[0 .. nzero) is cleared (null: nothing).
int pp_route_logits_dense(const void* x, int x_dtype, int64_t N, int H, const float* router, const float* bias,
                          int E, float* logits_out, bf16_t* xbf_out, uint32_t* zero, int nzero, hipStream_t st) {
  if (N == 0) return PP_OK;
  const int Epad = (E + 15) / 16 * 16;
  const int te = E <= 16 ? 1 : E <= 32 ? 2 : 3;
  const dim3 grid((unsigned)((N + 16 * RL_TT - 1) / (16 * RL_TT)), (unsigned)((E + 16 * te - 1) / (16 * te)));
#define PP_RL(XT, TE)                                                                                           \
  route_logits_kernel<XT, TE><<<grid, 512, RL_STAGES * Rl<XT, TE>::STAGE, st>>>(                                \
      (const XT*)x, N, H, router, Epad, bias, E, logits_out, xbf_out, zero, nzero)
  if (x_dtype == PP_DTYPE_F32) {
    if (te == 1) PP_RL(float, 1);
    else if (te == 2) PP_RL(float, 2);
    else PP_RL(float, 3);
  } else {
    if (te == 1) PP_RL(bf16_t, 1);
    else if (te == 2) PP_RL(bf16_t, 2);
    else PP_RL(bf16_t, 3);
  }
#undef PP_RL
  return pp_check_launch("route_logits_kernel");
}

// ------------------------------------------------------------------ host side
int pp_route_impl(const void* x, int x_dtype, const float* logits_in, int64_t N, int H, const float* router,
                  const float* bias, int E, float tau, float* logits_out, float* probs_out, float* gates_out,
                  uint8_t* mask_out, int32_t* count_out, bf16_t* xbf_out, hipStream_t st, int32_t* blkcnt_out);

// GEMM configurations (tile rows, K block, stages) of the two launches.
// Tiles (rows BM x columns BN, K block BK, stages, wave rows WR of the DG_NW waves).
// gate/up: 256 x 256 (128 neurons' gate and up rows), K blocks of 64, two stages, waves
// 2 x 4, for as many column tiles as fill whole rounds of the grid with no K split; the
// remaining column tiles as 128 x 256 tiles (three stages; a tail of those is K-split),
// so that no 256-row tile is cut (at N = 2048, I = 6144: 256 + 256 tiles, one round each).
// down: 256 x 192, K blocks of 64, two stages, waves 4 x 2 (wave tile 64 x 96), K-split
// (at N = 2048, H = 1536: 64 tiles in four K ranges).
#ifndef DG_GU_BM
#define DG_GU_BM 256
#endif
#ifndef DG_GU_BN
#define DG_GU_BN 256  // both gate/up launches: 128-neuron column tiles
#endif
#ifndef DG_GU_BK
#define DG_GU_BK 64
#endif
#ifndef DG_GU_ST
#define DG_GU_ST 2
#endif
#ifndef DG_GU_WR
#define DG_GU_WR 2
#endif
#ifndef DG_GT_BM
#define DG_GT_BM 128
#endif
#ifndef DG_GT_BK
#define DG_GT_BK 64
#endif
#ifndef DG_GT_ST
#define DG_GT_ST 3
#endif
#ifndef DG_GT_WR
#define DG_GT_WR 2
#endif
#ifndef DG_DN_BM
#define DG_DN_BM 256
#endif
#ifndef DG_DN_BN
#define DG_DN_BN 192
#endif
#ifndef DG_DN_BK
#define DG_DN_BK 64
#endif
#ifndef DG_DN_ST
#define DG_DN_ST 2
#endif
#ifndef DG_DN_WR
#define DG_DN_WR 4
#endif
#ifndef DG_SPLIT
#define DG_SPLIT 1  // tail items cut into K ranges joined in part order (0: whole items only)
#endif
#ifndef DG_NW
#define DG_NW 8  // waves per workgroup (two per SIMD)
#endif
#ifndef DG_GU_NW
#define DG_GU_NW DG_NW
#endif
#ifndef DG_GT_NW
#define DG_GT_NW DG_NW
#endif
#ifndef DG_DN_NW
#define DG_DN_NW DG_NW
#endif
#ifndef DG_GU_WPC
#define DG_GU_WPC 1  // workgroups per CU of each launch
#endif
#ifndef DG_GT_WPC
#define DG_GT_WPC 1
#endif
#ifndef DG_DN_WPC
#define DG_DN_WPC 1
#endif
#define DG_SYNC_WORDS (4 * DG_MAX_GRID)   // per GEMM launch: 2 counters per tail item
// one part's fp32 partial sums: a tile of either K-split launch (gate/up tail, down)
#define DG_SLOT_BYTES                                                                                  \
  ((size_t)std::max(Dg<DG_GT_BM, DG_GU_BN, DG_GT_BK, DG_GT_NW, DG_GT_WR>::NF * DG_GT_NW,                 \
                    Dg<DG_DN_BM, DG_DN_BN, DG_DN_BK, DG_DN_NW, DG_DN_WR>::NF * DG_DN_NW) * 64 * 4)

int pp_dense_ipad(int E, int G) { return (E * G + 63) / 64 * 64; }

__global__ void dg_zero_kernel(uint32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

struct DenseWs {
  size_t logits, gates, mask, xbf, act, sync, part, total;
};

static DenseWs dense_layout(int64_t n, int H, int E, int G) {
  DenseWs L;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  L.logits = take((size_t)n * E * 4);
  L.gates = take((size_t)n * E * 4);
  L.mask = take((size_t)n * E);
  L.xbf = take((size_t)n * H * 2);
  L.act = take((size_t)n * pp_dense_ipad(E, G) * 2);
  L.sync = take((size_t)DG_SYNC_WORDS * 4);
  L.part = take((size_t)DG_MAX_GRID * DG_SLOT_BYTES);
  L.total = o;
  return L;
}

// Tokens per pass: the per-token buffers (logits, gates, mask, bf16 x, act) of a pass stay
// within DG_PASS_BYTES (about 15000 tokens at H = 1536, E = 192, G = 32).
#define DG_PASS_BYTES ((int64_t)256 << 20)
static int64_t dense_pass_tokens(int64_t N, int H, int E, int G) {
  const int64_t per_token = (int64_t)E * 9 + (int64_t)H * 2 + (int64_t)pp_dense_ipad(E, G) * 2;
  return std::min<int64_t>(N, std::max<int64_t>(256, DG_PASS_BYTES / per_token));
}

size_t pp_dense_workspace_bytes(int64_t N, int H, int E, int G) {
  return dense_layout(dense_pass_tokens(N, H, E, G), H, E, G).total;
}

static int dense_grid() {
  const int g = (pp_device_cus() + 7) / 8 * 8;
  return std::max(8, std::min(DG_MAX_GRID, g));
}

template <int MODE, int BM, int BN, int BK, int ST, int NW, int WR, int WPC>
static int dense_gemm_launch(DgArgs a, hipStream_t st) {
  if (WPC > 1) a.part = nullptr, a.sync = nullptr;  // the split slots are sized for dense_grid() parts
  dense_gemm_kernel<MODE, BM, BN, BK, ST, NW, WR, WPC>
      <<<dense_grid() * WPC, NW * 64, ST * Dg<BM, BN, BK, NW, WR>::STAGE, st>>>(a);
  return pp_check_launch(MODE == 0 ? "dense_gemm_kernel (gate/up)" : "dense_gemm_kernel (down)");
}

// One pass over n tokens (at most dense_pass_tokens). logits_out / mask_out (may be null)
// receive the pass's routing.
static int dense_pass(const void* x, int x_dtype, int64_t n, int H, const float* router, const float* bias, int E,
                      int G, float tau, const void* packed, bf16_t* out, void* workspace, hipStream_t st,
                      float* logits_out, uint8_t* mask_out) {
  int rc;
  const DenseWs L = dense_layout(n, H, E, G);
  char* ws = (char*)workspace;
  float* logits = logits_out ? logits_out : (float*)(ws + L.logits);
  float* gates = (float*)(ws + L.gates);
  uint8_t* mask = mask_out ? mask_out : (uint8_t*)(ws + L.mask);
  const bf16_t* xbf = x_dtype == PP_DTYPE_BF16 ? (const bf16_t*)x : (const bf16_t*)(ws + L.xbf);
  bf16_t* xbf_w = x_dtype == PP_DTYPE_BF16 ? nullptr : (bf16_t*)(ws + L.xbf);
  uint32_t* sync = (uint32_t*)(ws + L.sync);
  float* part = (float*)(ws + L.part);
  if (E == 16) {  // the E = 16 router (the same logits as pp_route at E = 16)
    if ((rc = pp_route_impl(x, x_dtype, nullptr, n, H, router, bias, E, tau, logits, nullptr, gates, mask, nullptr,
                            xbf_w, st, nullptr)))
      return rc;
    // the split tickets (a fill kernel, not a memset node: callers capture this in graphs)
    dg_zero_kernel<<<1, 256, 0, st>>>(sync, DG_SYNC_WORDS);
    if ((rc = pp_check_launch("dg_zero_kernel"))) return rc;
  } else {
    if ((rc = pp_route_logits_dense(x, x_dtype, n, H, router, bias, E, logits, xbf_w, sync, DG_SYNC_WORDS, st)))
      return rc;
    if ((rc = pp_route_impl(nullptr, PP_DTYPE_F32, logits, n, H, nullptr, nullptr, E, tau, nullptr, nullptr, gates,
                            mask, nullptr, nullptr, st, nullptr)))
      return rc;
  }
  const int I = E * G, Ipad = pp_dense_ipad(E, G);
  bf16_t* act = (bf16_t*)(ws + L.act);
  DgArgs a;
  a.a = xbf;
  a.b = (const bf16_t*)packed;
  a.gates = gates;
  a.out = act;
  a.part = DG_SPLIT ? part : nullptr;
  a.sync = DG_SPLIT ? sync : nullptr;
  a.N = n;
  a.H = H;
  a.E = E;
  a.G = G;
  a.I = I;
  a.Ipad = Ipad;
  // gate/up: column tiles [0, ct_main) in whole rounds of 256-row tiles, no K split; the
  // rest as 128-row tiles
  const int grid = dense_grid() * DG_GU_WPC;
  const int ntc = (Ipad + DG_GU_BN / 2 - 1) / (DG_GU_BN / 2);
  const int64_t nrt = (n + DG_GU_BM - 1) / DG_GU_BM;
  const int ct_main = nrt * ntc >= grid ? (int)((nrt * ntc) / grid * grid / nrt) : 0;
  if (ct_main > 0) {
    DgArgs m = a;
    m.part = nullptr;
    m.sync = nullptr;
    m.ct_lo = 0;
    m.ct_hi = ct_main;
    if ((rc = dense_gemm_launch<0, DG_GU_BM, DG_GU_BN, DG_GU_BK, DG_GU_ST, DG_GU_NW, DG_GU_WR, DG_GU_WPC>(m, st))) return rc;
  }
  if (ct_main < ntc) {
    a.ct_lo = ct_main;
    a.ct_hi = ntc;
    if ((rc = dense_gemm_launch<0, DG_GT_BM, DG_GU_BN, DG_GT_BK, DG_GT_ST, DG_GT_NW, DG_GT_WR, DG_GT_WPC>(a, st))) return rc;
  }
  a.a = act;
  a.b = (const bf16_t*)packed + (int64_t)I * 3 * H;  // down_t
  if (a.sync) a.sync += DG_SYNC_WORDS / 2;            // the down GEMM's own split counters
  a.gates = nullptr;
  a.out = out;
  a.ct_lo = 0;
  a.ct_hi = (H + DG_DN_BN - 1) / DG_DN_BN;
  return dense_gemm_launch<1, DG_DN_BM, DG_DN_BN, DG_DN_BK, DG_DN_ST, DG_DN_NW, DG_DN_WR, DG_DN_WPC>(a, st);
}

// The whole dense-form prefill over N tokens in passes (inputs validated by the caller).
int pp_dense_prefill(const void* x, int x_dtype, int64_t N, int H, const float* router, const float* bias, int E,
                     int G, float tau, const void* packed, void* out, void* workspace, hipStream_t st,
                     float* logits_out, uint8_t* mask_out) {
  const int64_t nc = dense_pass_tokens(N, H, E, G);
  const size_t xs = x_dtype == PP_DTYPE_BF16 ? 2 : 4;
  for (int64_t n0 = 0; n0 < N; n0 += nc) {
    const int64_t nt = std::min(nc, N - n0);
    const int rc = dense_pass((const char*)x + (size_t)n0 * H * xs, x_dtype, nt, H, router, bias, E, G, tau, packed,
                              (bf16_t*)out + (size_t)n0 * H, workspace, st,
                              logits_out ? logits_out + n0 * E : nullptr, mask_out ? mask_out + n0 * E : nullptr);
    if (rc) return rc;
  }
  return PP_OK;
}
