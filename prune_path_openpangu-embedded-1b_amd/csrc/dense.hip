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
// GEMM tiles: 256 x 256 outputs (DG_BM token rows x 256 columns: 128 neurons as gate and
// up, or 256 hidden columns), K blocks of BK bf16, four waves each owning a BM/2 x 128
// wave tile of v_mfma_f32_32x32x16_bf16 blocks (accumulators in AGPRs: one workgroup per
// CU). Operands go global -> LDS by DMA (global_load_lds_dwordx4, no VGPR staging)
// through STAGES stages; the stream of K blocks runs across a workgroup's items (GpSched:
// whole items in full rounds, then the tail items cut into K ranges whose fp32 partial
// sums are joined by the part drawing the last ticket, in part order).
#include <algorithm>

#include "gemm_lds.h"

#define DG_MAX_GRID 256  // workgroups of a GEMM launch; also the split workspace's part slots
#define DG_GX 8          // experts a 128-neuron column tile can touch (G >= 32: at most 5)
#define DG_NPMAX 8       // K parts of a split tile at most
#ifndef DG_SPIN
#define DG_SPIN 4000     // polls (s_sleep 2, ~50 ns each) for the sibling parts of a split tile
#endif

// silu(g) = g * sigmoid(g) with the hardware exp2 and reciprocal (~1 ulp each): the act is
// rounded to bf16 right after, 2^-9 relative.
__device__ __forceinline__ float dg_silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

template <int BM, int BK, int NW>
struct Dg {
  static constexpr int NT = NW * 64;           // threads
  static constexpr int WN = NW / 2;            // wave columns (two wave rows)
  static constexpr int WC = 256 / WN;          // columns of a wave tile
  static constexpr int MI = BM / 64;           // 32-row MFMA blocks per wave (wave tile BM/2 rows)
  static constexpr int NJ = WC / 32;           // 32-column MFMA blocks per wave
  static constexpr int NF = MI * NJ * 16;      // fp32 accumulators per thread
  static constexpr int ROWB = BK * 2;          // bytes of one tile row in a stage
  static constexpr int CH = BK / 8;            // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROWB;      // rows per DMA instruction (a wave's 1 KB)
  static constexpr int NIA = BM / (NW * RPI);  // DMA instructions per wave per block, A
  static constexpr int NIB = 256 / (NW * RPI); // ... B (256 columns)
  static constexpr int DMA = NIA + NIB;
  static constexpr int KS = BK / 16;           // MFMA k-steps per block
  static constexpr int TA = BM * ROWB;         // A tile bytes per stage
  static constexpr int STAGE = TA + 256 * ROWB;
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
};

// Wait until at most N LDS reads are outstanding, tying the fragments of the current
// k-step so that their MFMAs cannot be scheduled above the wait.
template <int N, int MI, int NJ>
__device__ __forceinline__ void dg_wait(u32x4 (&a)[MI], u32x4 (&b)[NJ]) {
  static_assert(MI + NJ <= 8 && NJ >= 2, "fragments");
  if (MI == 4 && NJ == 4)
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(a[0]), "+v"(a[1 % MI]), "+v"(a[2 % MI]), "+v"(a[3 % MI]), "+v"(b[0]), "+v"(b[1]),
                   "+v"(b[2 % NJ]), "+v"(b[3 % NJ])
                 : "n"(N));
  else if (MI == 4)
    asm volatile("s_waitcnt lgkmcnt(%6)"
                 : "+v"(a[0]), "+v"(a[1 % MI]), "+v"(a[2 % MI]), "+v"(a[3 % MI]), "+v"(b[0]), "+v"(b[1])
                 : "n"(N));
  else if (NJ == 4)
    asm volatile("s_waitcnt lgkmcnt(%6)"
                 : "+v"(a[0]), "+v"(a[1 % MI]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2 % NJ]), "+v"(b[3 % NJ])
                 : "n"(N));
  else
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a[0]), "+v"(a[1 % MI]), "+v"(b[0]), "+v"(b[1]) : "n"(N));
}

template <int MODE, int BM, int BK, int STAGES, int NW>
__global__ __launch_bounds__(NW * 64, 1) void dense_gemm_kernel(DgArgs p) {
  using C = Dg<BM, BK, NW>;
  static_assert(BM == 128 || BM == 256, "tile rows");
  static_assert(NW == 4 || NW == 8, "waves");
  static_assert(STAGES >= 2 && STAGES * C::STAGE + (MODE == 0 ? BM * DG_GX * 4 : 0) <= 160 * 1024 - 64, "LDS");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int role_s;
  __shared__ float gate_s[MODE == 0 ? BM * DG_GX : 1];  // MODE 0 epilogue: the tile's router gates
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
  const int wm = w / C::WN, wn = w % C::WN;
  const int n_rt = (int)((p.N + BM - 1) / BM);
  const int n_ct = MODE == 0 ? (p.Ipad + 127) / 128 : (p.H + 255) / 256;
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
    const int ct = item / n_rt, rt = item - ct * n_rt;
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
      // or up row of neuron ct * 128 + (r / WC) * WC/2 + (jb % (NJ/2)) * 32 + (r & 31)
      b_item = p.b + (int64_t)ct * 128 * 3 * p.H;
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) {
        const int r = (NW * i + w) * C::RPI + lane / C::CH;
        const int jb = (r % C::WC) >> 5;
        const int nl = min(ct * 128 + (r / C::WC) * (C::WC / 2) + (jb % (C::NJ / 2)) * 32 + (r & 31), p.I - 1) -
                       ct * 128;
        boff[i] = (uint32_t)((nl * 3 + jb / (C::NJ / 2)) * p.H + gc8) * 2u;
      }
    } else {
      b_item = p.b + (int64_t)ct * 256 * p.G;
#pragma unroll
      for (int i = 0; i < C::NIB; ++i) {
        const int r = (NW * i + w) * C::RPI + lane / C::CH;
        boff[i] = (uint32_t)((min(ct * 256 + r, p.H - 1) - ct * 256) * p.G) * 2u + lane_k;
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
    offA[ks] = lds0 + wm * (BM / 2) * C::ROWB + o;
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
    // without a memory round trip there (gate_s[r * DG_GX + k]: row r, expert e_lo + k)
    constexpr int NGL = MODE == 0 ? BM * DG_GX / C::NT : 1;
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
        const int ct = item / n_rt, rt = item - ct * n_rt;
        const int e_lo = ct * 128 / p.G;
        const int ne = min(p.E, (ct * 128 + 127) / p.G + 1) - e_lo;
        const int64_t tt0 = (int64_t)rt * BM;
#pragma unroll
        for (int c = 0; c < NGL; ++c) {
          const int idx = tid + c * C::NT, r = idx / DG_GX, k = idx % DG_GX;
          gl[c] = (k < ne && tt0 + r < p.N) ? p.gates[(tt0 + r) * p.E + e_lo + k] : 0.0f;
        }
      } else if (MODE == 0 && kb == kb_first + 1) {
        gates_store();
      }
      const uint32_t sbase = (f % STAGES) * C::STAGE;
      u32x4 fa[2][C::MI], fb[2][C::NJ];
      auto rd = [&](int ks, u32x4(&a)[C::MI], u32x4(&b)[C::NJ]) {
        a[0] = gv_read<0>(offA[ks] + sbase);
        a[1] = gv_read<RB>(offA[ks] + sbase);
        if (C::MI > 2) {
          a[2 % C::MI] = gv_read<2 * RB>(offA[ks] + sbase);
          a[3 % C::MI] = gv_read<3 * RB>(offA[ks] + sbase);
        }
        b[0] = gv_read<0>(offB[ks] + sbase);
        b[1] = gv_read<RB>(offB[ks] + sbase);
        if (C::NJ > 2) {
          b[2 % C::NJ] = gv_read<2 * RB>(offB[ks] + sbase);
          b[3 % C::NJ] = gv_read<3 * RB>(offB[ks] + sbase);
        }
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
      const int ct = item / n_rt, rt = item - ct * n_rt;
      const int64_t t0 = (int64_t)rt * BM + wm * (BM / 2);
      const int rows_in = (int)min((int64_t)(BM / 2), max((int64_t)0, p.N - t0));
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
                const int n = ct * 128 + wn * (C::WC / 2) + col;
                if (n >= p.Ipad) continue;
                const float gt = n < p.I ? gate_s[(wm * (BM / 2) + rl) * DG_GX + n / p.G - ct * 128 / p.G] : 0.0f;
                const float a = gt == 0.0f ? 0.0f : dg_silu(sv[h]) * tv[h] * gt;
                p.out[(t0 + rl) * p.Ipad + n] = f32_to_bf16(a);
              } else {
                const int hc = ct * 256 + wn * C::WC + col;
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
    // major), then out as 16-byte row chunks: coalesced stores, no 2-byte scatter
    {
      int ln = lane;
      asm volatile("" : "+v"(ln));  // keep the epilogue's lane math out of the main loop's registers
      const int item = sc.item(li);
      const int ct = item / n_rt, rt = item - ct * n_rt;
      const int64_t t0 = (int64_t)rt * BM + wm * (BM / 2);  // this wave's first output row
      const int rows_in = (int)min((int64_t)(BM / 2), max((int64_t)0, p.N - t0));
      unsigned char* ep = smem + (fl % STAGES) * C::STAGE + w * C::EPW;
      if (MODE == 0) {
        const int e_lo = ct * 128 / p.G;
        __syncthreads();  // gates staged; every wave done reading the free stage
        // act of the wave's WC/2 neurons: LDS rows of WC/2 bf16, in passes of HR rows
        constexpr int RW = C::WC / 2 * 2;  // bytes of an LDS row
        constexpr int HR = C::EPW / RW < BM / 2 ? C::EPW / RW : BM / 2;  // rows per pass
        static_assert(HR % 32 == 0 && (BM / 2) % HR == 0, "epilogue passes");
        const int n0 = ct * 128 + wn * (C::WC / 2);
        const int cols_in = min(C::WC / 2, p.Ipad - n0);
        int64_t oo = t0 * p.Ipad + n0;
        asm volatile("" : "+s"(oo));
        bf16_t* ob = p.out + oo;
#pragma unroll
        for (int hf = 0; hf < (BM / 2) / HR; ++hf) {
#pragma unroll
          for (int jj = 0; jj < C::NJ / 2; ++jj) {
            const int nl = jj * 32 + (ln & 31);
            const int ek = (n0 + nl) / p.G - e_lo;
            const bool real = n0 + nl < p.I;  // neurons of the pad [I, Ipad) get act 0
#pragma unroll
            for (int i = hf * (HR / 32); i < (hf + 1) * (HR / 32); ++i) {
              f32x16_t gv = acc[i][jj], uv = acc[i][jj + C::NJ / 2];
              asm volatile("" : "+v"(gv), "+v"(uv));  // two 16-float blocks in VGPRs at a time
#pragma unroll
              for (int q = 0; q < 16; ++q) {
                const int rl = i * 32 + mfma32_row(q, ln);
                const float gt = real ? gate_s[(wm * (BM / 2) + rl) * DG_GX + ek] : 0.0f;
                const float a = gt == 0.0f ? 0.0f : dg_silu(gv[q]) * uv[q] * gt;
                *(bf16_t*)(ep + (rl - hf * HR) * RW + nl * 2) = f32_to_bf16(a);
              }
            }
          }
          // out: row rl, 16-byte chunk c of the row (WC/2 neurons = RW / 16 chunks)
          constexpr int CPR = RW / 16;
#pragma unroll
          for (int k = 0; k < HR * CPR / 64; ++k) {
            const int idx = ln + 64 * k, rl = idx / CPR, c = idx % CPR;
            const uint4 v = *(const uint4*)(ep + rl * RW + c * 16);
            const int rg = hf * HR + rl;
            if (rg < rows_in && c * 8 < cols_in) *(uint4*)(ob + rg * p.Ipad + c * 8) = v;
          }
        }
      } else {
        asm volatile("s_barrier" ::: "memory");  // every wave done reading the free stage
        // out rows of the wave's WC columns, in halves of BM/4 rows (EPW bytes each)
        constexpr int RW = C::WC * 2;  // bytes of an LDS row
        constexpr int HR = C::EPW / RW < BM / 2 ? C::EPW / RW : BM / 2;  // rows per pass
        static_assert(HR % 32 == 0 && (BM / 2) % HR == 0, "epilogue passes");
        const int h0 = ct * 256 + wn * C::WC;
        const int cols_in = min(C::WC, p.H - h0);
        int64_t oo = t0 * p.H + h0;
        asm volatile("" : "+s"(oo));
        bf16_t* ob = p.out + oo;
#pragma unroll
        for (int hf = 0; hf < (BM / 2) / HR; ++hf) {
#pragma unroll
          for (int i = hf * (HR / 32); i < (hf + 1) * (HR / 32); ++i)
#pragma unroll
            for (int j = 0; j < C::NJ; ++j) {
              f32x16_t v = acc[i][j];
              asm volatile("" : "+v"(v));  // one 16-float block in VGPRs at a time
#pragma unroll
              for (int q = 0; q < 16; ++q) {
                const int rl = (i - hf * (HR / 32)) * 32 + mfma32_row(q, ln);
                *(bf16_t*)(ep + rl * RW + (j * 32 + (ln & 31)) * 2) = f32_to_bf16(v[q]);
              }
            }
          constexpr int CPR = RW / 16;
#pragma unroll
          for (int k = 0; k < HR * CPR / 64; ++k) {
            const int idx = ln + 64 * k, rl = idx / CPR, c = idx % CPR;
            const uint4 v = *(const uint4*)(ep + rl * RW + c * 16);
            const int rg = hf * HR + rl;
            if (rg < rows_in && c * 8 < cols_in) *(uint4*)(ob + rg * p.H + c * 8) = v;
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
  f32x4_t acc[TE];
#pragma unroll
  for (int b = 0; b < TE; ++b) acc[b] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; ++c) {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(R::DMA * (RL_STAGES - 2)) : "memory");
    issue(c + RL_STAGES - 1);
    const unsigned char* st = smem + (c % RL_STAGES) * R::STAGE;
    // x as bf16 for the GEMMs (fp32 x, first expert group only): thread -> row tid / 8,
    // 16 values at (tid % 8) * 16
    if (sizeof(XT) == 4 && xbf_out && blockIdx.y == 0 && tid < 256) {
      const int r = tid >> 3, k16 = (tid & 7) * 16;
      const int64_t t = tok0 + r;
      if (t < N) {
        uint32_t pk[8];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float4 v = *(const float4*)(st + r * R::XROW + ((((k16 >> 2) + h) ^ (r & 15)) << 4));
          pk[2 * h] = (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
          pk[2 * h + 1] = (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
        }
        uint4* dst = (uint4*)(xbf_out + t * H + c * RL_KC + k16);
        dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
      }
    }
    float xv[8], wv[TE][8];
    {
      const int r = 16 * ta + t_l;
      if (sizeof(XT) == 4) {
        const int c0 = 8 * kq + 2 * g;
        const float4 v0 = *(const float4*)(st + r * R::XROW + ((c0 ^ (r & 15)) << 4));
        const float4 v1 = *(const float4*)(st + r * R::XROW + (((c0 + 1) ^ (r & 15)) << 4));
        xv[0] = v0.x; xv[1] = v0.y; xv[2] = v0.z; xv[3] = v0.w;
        xv[4] = v1.x; xv[5] = v1.y; xv[6] = v1.z; xv[7] = v1.w;
      } else {
        const uint4 u = *(const uint4*)(st + r * R::XROW + (((4 * kq + g) ^ (r & 15)) << 4));
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[2 * i] = __uint_as_float(uw[i] << 16);
          xv[2 * i + 1] = __uint_as_float(uw[i] & 0xffff0000u);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < TE; ++b) {
      const int r = 16 * b + t_l;
      const int c0 = 8 * kq + 2 * g;
      const unsigned char* ws = st + R::XB + r * R::WROW;
      const float4 v0 = *(const float4*)(ws + ((c0 ^ (r & 15)) << 4));
      const float4 v1 = *(const float4*)(ws + (((c0 + 1) ^ (r & 15)) << 4));
      wv[b][0] = v0.x; wv[b][1] = v0.y; wv[b][2] = v0.z; wv[b][3] = v0.w;
      wv[b][4] = v1.x; wv[b][5] = v1.y; wv[b][6] = v1.z; wv[b][7] = v1.w;
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
#ifndef DG_GU_BM
#define DG_GU_BM 256
#endif
#ifndef DG_GU_BK
#define DG_GU_BK 64
#endif
#ifndef DG_GU_ST
#define DG_GU_ST 2
#endif
#ifndef DG_DN_BM
#define DG_DN_BM 256
#endif
#ifndef DG_DN_BK
#define DG_DN_BK 64
#endif
#ifndef DG_DN_ST
#define DG_DN_ST 2
#endif
#ifndef DG_SPLIT
#define DG_SPLIT 1  // tail items cut into K ranges joined in part order (0: whole items only)
#endif
#ifndef DG_NW
#define DG_NW 8  // waves per workgroup (two per SIMD)
#endif
#define DG_SYNC_WORDS (4 * DG_MAX_GRID)   // per GEMM launch: 2 counters per tail item
#define DG_SLOT_BYTES ((size_t)256 * 256 * 4)  // one part's fp32 partial sums (a 256 x 256 tile or less)

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

template <int MODE, int BM, int BK, int ST>
static int dense_gemm_launch(const DgArgs& a, hipStream_t st) {
  dense_gemm_kernel<MODE, BM, BK, ST, DG_NW><<<dense_grid(), DG_NW * 64, ST * Dg<BM, BK, DG_NW>::STAGE, st>>>(a);
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
  if ((rc = dense_gemm_launch<0, DG_GU_BM, DG_GU_BK, DG_GU_ST>(a, st))) return rc;
  a.a = act;
  a.b = (const bf16_t*)packed + (int64_t)I * 3 * H;  // down_t
  if (a.sync) a.sync += DG_SYNC_WORDS / 2;            // the down GEMM's own split counters
  a.gates = nullptr;
  a.out = out;
  return dense_gemm_launch<1, DG_DN_BM, DG_DN_BK, DG_DN_ST>(a, st);
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
