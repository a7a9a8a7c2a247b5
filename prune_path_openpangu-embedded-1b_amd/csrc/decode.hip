// Decode (one token): a single fused kernel for the whole MoE-MLP layer.
//
// Replaces TauSparseMoE.forward_decode (src/tl_kernel_optimized_Ultimate_PanGU.py:494-530):
// decode_out.zero_() + moe_router_select_kernel_decode (:335-380) +
// moe_decode_swiglu_fused_kernel (:385-462). Differences by design: fp32 router, the
// torch-CPU selection rule (fp64-accumulated cumsum, torch sort order), every neuron of
// every selected expert computed (the reference's 1-D grid leaves pid_g at 0 and only
// covers 64 neurons per expert, :398-399, 515), and an fp32 reduction instead of bf16
// atomics.
//
// Routing. When the fp32 router is small (E <= 16 and 16*H*4 <= 128 KB, e.g. E=16 at
// H=1536) every workgroup computes all logits (fixed reduction order, so every workgroup
// gets the same bits) and runs the selection itself: no cross-workgroup wait at all.
// Otherwise workgroup e < E computes logit e and publishes it in a 64-bit slot tagged
// with the call epoch; every workgroup gathers the E slots (bounded spin on the tag) and
// runs the selection on its own copy. Workgroups are dispatched in index order, so the
// producers are resident before any waiter can take their slot; the bound only turns an
// impossible wait into an error flag instead of a hang.
//
// Work split. The layer's weight bytes are k * G neuron records of 6*H bytes each
// ({gate row, up row, down column}, see pack.hip). All workgroups share the k*G
// records evenly; each wave streams whole records with 16-byte loads per lane (the next
// record's loads are in flight while the current one is reduced), reduces the gate/up
// dot products across the wave, applies silu(g)*u*gate in registers and accumulates
// act * down into 8*CPL fp32 registers per lane. The workgroup's partial output goes to
// one of a few fp32 accumulator copies with float atomics; the last workgroup to finish
// (ticket) folds the copies, writes the bf16 output, advances the call epoch and resets
// the counters. Two accumulator sets alternate between calls, and each call clears the
// set of the previous call early, off its critical path, so no call needs a memset.
//
// Cross-workgroup data (logits, selection, counters, accumulators) is only accessed
// with agent-scope atomics, and ordering between them comes from waiting for
// completion (s_waitcnt vmcnt(0)) before the dependent atomic. Agent-scope fences are
// avoided on purpose: on gfx950 each one writes back and invalidates the L2, which
// hundreds of workgroups cannot afford inside a 5 us kernel.
#include <mutex>

#include "pp_common.h"

// Waves per workgroup of the general kernel: eight while the registers fit 256 per lane
// (CPL <= 5), else four. Eight waves keep twice the records per CU in flight
// (E = 192, G = 32: 25.6 -> 24.7 us per layer).
template <int CPL>
struct DecNW {
  static constexpr int NW = CPL <= 5 ? 8 : 4;
  static constexpr int NT = 64 * NW;
};
#define DEC_NCOPY 4   // accumulator copies per set (general kernel; the allocation): 4 beat 8 and 16 at E = 192
#define DEC16_NCOPY 4 // copies the E = 16 kernel uses (128 workgroups: 32 per address)
#define DEC16_SPEC(CPL) ((CPL) <= 4)  // speculative top-expert loads (register budget)
#ifndef DEC16_NW
#define DEC16_NW 8  // waves per workgroup in the E = 16 kernel
#endif
#define DEC_SPIN_LIMIT (1u << 22)
#define DEC_LOCAL_ROUTER_FLOATS 32768  // Epad*H at or below this: every workgroup routes

static constexpr size_t dec_acc_offset() { return (sizeof(pp_decode_state) + 255) / 256 * 256; }


__device__ __forceinline__ void vm_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <typename T>
__device__ __forceinline__ T ld_rlx(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_rlx(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_rlx(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Accumulators hold 64-bit fixed point (value * 2^32, two's complement). Integer
// addition is associative, so the sum of the workgroups' partials has the same bits
// whatever order their atomics land in: the decode output is bitwise reproducible.
// A partial must stay below 2^30 in magnitude (finite): the sum of up to 2^31 such
// partials cannot overflow, and the quantisation step 2^-32 per partial is far below the
// bf16 output's resolution. A partial outside that range sets error bit 4 and the call's
// output is NaN (never a wrapped value).
typedef unsigned long long dec_acc_t;
#define DEC_FIXED_SCALE 0x1p32
__device__ __forceinline__ float dec_from_fixed(dec_acc_t v) {
  return (float)((double)(long long)v * (1.0 / DEC_FIXED_SCALE));
}

// Accumulators: two sets of DEC_NCOPY x H fixed-point words, used by alternate calls (parity of the
// call epoch, st->router_ticket, which the last workgroup of every call advances).
// Call N adds into set N & 1 and its last workgroup only reads it; the workgroups of
// call N+1 clear set N & 1 early in the call, off the critical path, so call N+2
// finds it zero. 64-bit logit slots follow the two sets.
// hs: the stride of one accumulator copy (H for a caller's workspace; a fixed larger
// stride keeps one layout for a workspace shared by calls of different H).
__device__ __forceinline__ dec_acc_t* dec_acc_set(dec_acc_t* acc, int hs, uint32_t epoch) {
  return acc + (size_t)(epoch & 1u) * DEC_NCOPY * hs;
}
#define DEC_SLOT_REPS 16  // replicas of the logit slots (each written by its router workgroup)
__device__ __forceinline__ unsigned long long* dec_slots(dec_acc_t* acc, int hs) {
  return (unsigned long long*)(acc + (size_t)2 * DEC_NCOPY * hs);
}
// this workgroup's share of clearing the other set (the previous call's)
// (the first ncopy copies of it: the ones the kernel uses)
// (hclear values of each copy: the previous call's H, or the whole stride when the
// previous call's H is not known)
__device__ __forceinline__ void dec_clear_previous(dec_acc_t* acc, int hs, int hclear, uint32_t epoch, int b, int W,
                                                   int tid, int nthreads, int ncopy = DEC_NCOPY) {
  dec_acc_t* prev = dec_acc_set(acc, hs, epoch + 1u);
  int lo, hi;
  pp_split((uint32_t)(ncopy * hclear), (uint32_t)W, (uint32_t)b, lo, hi);
  for (int i = lo + tid; i < hi; i += nthreads) {
    const int c = (int)((uint32_t)i / (uint32_t)hclear);
    st_rlx(prev + (size_t)c * hs + (i - c * hclear), (dec_acc_t)0);
  }
}

// Completion ticket in two levels. One counter taken by every workgroup serialises at
// the memory side (~20 ns per atomic on one address). Here workgroup b counts in at its
// group's counter (DEC_TG workgroups per group, each counter on a 128-byte line of its
// own); the group's last arrival counts the group in at the top counter; the top's last
// arrival is the call's last workgroup. Every arrival has performed its accumulator
// atomics first, so the last workgroup sees them all; it zeroes the counters it used.
#define DEC_TG 16
#define DEC_TLINE 32                          // uint32 per 128-byte line
#define DEC_TMAX_GROUPS 64                    // larger grids use groups of ceil(W / 64)
#define DEC_TICKET_WORDS ((DEC_TMAX_GROUPS + 1) * DEC_TLINE)
__device__ __forceinline__ uint32_t* dec_tickets(dec_acc_t* acc, int hs) {
  return (uint32_t*)(dec_slots(acc, hs) + DEC_SLOT_REPS * PP_MAX_EXPERTS);
}
__device__ __forceinline__ int dec_tgroup_size(int W) {
  return max(DEC_TG, (W + DEC_TMAX_GROUPS - 1) / DEC_TMAX_GROUPS);
}
// thread 0 of each workgroup, after its accumulator atomics are performed: true in the last
__device__ __forceinline__ bool dec_ticket(uint32_t* tk, int b, int W) {
  const int tg = dec_tgroup_size(W), grp = b / tg, ngrp = (W + tg - 1) / tg;
  const uint32_t gsize = (uint32_t)min(tg, W - grp * tg);
  return add_rlx(tk + (size_t)(grp + 1) * DEC_TLINE, 1u) == gsize - 1u &&
         add_rlx(tk, 1u) == (uint32_t)ngrp - 1u;
}
// by the last workgroup, threads 0 .. ngrp
__device__ __forceinline__ void dec_ticket_reset(uint32_t* tk, int W, int tid) {
  const int tg = dec_tgroup_size(W), ngrp = (W + tg - 1) / tg;
  if (tid <= ngrp) st_rlx(tk + (size_t)tid * DEC_TLINE, 0u);
}

// Add one partial (fp32) to a fixed-point accumulator; out-of-range partials flag the call.
__device__ __forceinline__ void dec_acc_add(dec_acc_t* p, float v, pp_decode_state* st, uint32_t epoch) {
  if (!(fabsf(v) < 0x1p30f)) {  // also NaN
    __hip_atomic_fetch_or(&st->error, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    st_rlx(&st->error_call, epoch + 1u);
    v = 0.0f;
  }
  __hip_atomic_fetch_add(p, (dec_acc_t)__double2ll_rn((double)v * DEC_FIXED_SCALE), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}

// 8 bf16 packed in a uint4: dot with x[8], or acc += a * w
__device__ __forceinline__ float dot8(const uint4 w, const float* x) {
  float s = 0.0f;
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s = __builtin_fmaf(x[2 * i], __uint_as_float(u[i] << 16), s);
    s = __builtin_fmaf(x[2 * i + 1], __uint_as_float(u[i] & 0xffff0000u), s);
  }
  return s;
}
// 8 bf16 weights . 8 bf16 x values (both packed in pairs), fp32 accumulation with the
// bf16 dot-product instruction (products of bf16 values are exact in fp32)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot8_bf16(const uint4 w, const uint4 xb, float s) {
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, xb.x), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, xb.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, xb.z), s, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, xb.w), s, false);
}
__device__ __forceinline__ void axpy8(float a, const uint4 w, float* acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] = __builtin_fmaf(a, __uint_as_float(u[i] << 16), acc[2 * i]);
    acc[2 * i + 1] = __builtin_fmaf(a, __uint_as_float(u[i] & 0xffff0000u), acc[2 * i + 1]);
  }
}

// All logits of the token in this workgroup, for the local-routing mode. Wave w takes
// experts 4w..4w+3 of each group of 16; lane l the float4 chunks l, l+64, ... of x and of
// those router rows, all loaded up front (one memory round trip). Per-wave totals by a
// fixed butterfly (lane l ends with expert 4w + 2*b5 + b4), so the logits are
// deterministic and identical in every workgroup.
template <typename XT, int CPL>
__device__ void local_logits(const XT* __restrict__ x, int H, const float* __restrict__ router,
                             const float* __restrict__ bias, int E, float* lg_s, int tid) {
  constexpr int NC = 2 * CPL;  // float4 chunks per lane per row (H <= 512 * CPL)
  const int lane = tid & 63, wv = tid >> 6;
  const int HC4 = H >> 2;
  float4 xv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = lane + 64 * i;
    if (c < HC4) {
      xv[i].x = load_as_f32<XT>(x, 4 * c);
      xv[i].y = load_as_f32<XT>(x, 4 * c + 1);
      xv[i].z = load_as_f32<XT>(x, 4 * c + 2);
      xv[i].w = load_as_f32<XT>(x, 4 * c + 3);
    } else {
      xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  for (int e0 = 0; e0 < E; e0 += 4 * DecNW<CPL>::NW) {
    float4 wr[4][NC];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        const int er = e0 + 4 * wv + j;  // rows past E (the zero padding, or beyond) are not read
        wr[j][i] = (c < HC4 && er < E) ? *(const float4*)(router + (int64_t)er * H + 4 * c)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float sacc = 0.0f;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        sacc = __builtin_fmaf(xv[i].x, wr[j][i].x, sacc);
        sacc = __builtin_fmaf(xv[i].y, wr[j][i].y, sacc);
        sacc = __builtin_fmaf(xv[i].z, wr[j][i].z, sacc);
        sacc = __builtin_fmaf(xv[i].w, wr[j][i].w, sacc);
      }
      part[j] = sacc;
    }
    // butterfly: 4 values -> lane holds total of value 2*b5 + b4
    const int b5 = (lane >> 5) & 1, b4 = (lane >> 4) & 1;
    float a2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      a2[i] = __fadd_rn(b5 ? part[i + 2] : part[i], __shfl_xor(b5 ? part[i] : part[i + 2], 32, PP_WAVE));
    float t = __fadd_rn(b4 ? a2[1] : a2[0], __shfl_xor(b4 ? a2[0] : a2[1], 16, PP_WAVE));
    t = row16_sum(t);
    const int e = e0 + 4 * wv + 2 * b5 + b4;
    if ((lane & 15) == 0 && e < E) lg_s[e] = bias ? __fadd_rn(t, bias[e]) : t;
  }
  __syncthreads();
}

template <typename XT, int CPL, bool LOCAL>
__global__ __launch_bounds__(DecNW<CPL>::NT) void decode_kernel(
    const XT* __restrict__ x, int H, const float* __restrict__ router, const float* __restrict__ bias,
    int E, int G, float tau, const bf16_t* __restrict__ rows, bf16_t* __restrict__ out,
    pp_decode_state* __restrict__ st, dec_acc_t* __restrict__ acc, int hs, int hclear) {
  constexpr int NW = DecNW<CPL>::NW, NT = DecNW<CPL>::NT;
  extern __shared__ __align__(16) float red[];  // [NW][H] wave partials
  __shared__ SelScratch ss;
  __shared__ float red4[NW];
  __shared__ unsigned long long keys_s[PP_MAX_EXPERTS];
  __shared__ float lg_s[PP_MAX_EXPERTS];
  __shared__ int flag_s;
  __shared__ int k_s;
  __shared__ int sel_ids_s[PP_MAX_EXPERTS];
  __shared__ float sel_g_s[PP_MAX_EXPERTS];
  __shared__ __align__(16) unsigned char xs_raw[4096 * sizeof(XT)];  // x as given, for the stream

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = gridDim.x, b = blockIdx.x;
  const int HC = H >> 3;  // 16-byte chunks per row
  const uint32_t epoch = ld_rlx(&st->router_ticket);

  // x for the stream goes global -> LDS by DMA now (no registers held through the
  // routing); the stream reads it from LDS. Loaded at the stream's start, x cost ~3 us at
  // E = 192; loaded into registers here, +1.7 us (registers live through the selection).
  // 1 KB per instruction; lanes past the end re-read the last chunk (in bounds) into the
  // spare end of xs_raw.
  if (wv == NT / 64 - 1) {
    const int nbytes = H * (int)sizeof(XT), nch = nbytes >> 4;
    for (int c0 = 0; c0 < nch; c0 += 64)
      __builtin_amdgcn_global_load_lds((const unsigned char*)x + 16 * min(c0 + lane, nch - 1),
                                       (__attribute__((address_space(3))) void*)(xs_raw + 16 * c0), 16, 0, 0);
  }

  if (LOCAL) {
    // ---------------- every workgroup routes the token itself
    local_logits<XT, CPL>(x, H, router, bias, E, lg_s, tid);
    if (wv == 0) {
      select_small<16>([&](int j) { return lg_s[j]; }, E, tau, &ss, lane);
      const int k = ss.k;
      for (int q = lane; q < k; q += 64) {
        const int e = ss.order[q];
        sel_ids_s[q] = e;
        sel_g_s[q] = pp_sigmoid(lg_s[e]);
      }
      if (lane == 0) k_s = k;
    }
    __syncthreads();
    if (b == 0) {  // telemetry for the caller: logits and selection of this call
      for (int j = tid; j < E; j += NT) st_rlx(&st->logits[j], lg_s[j]);
      for (int q = tid; q < k_s; q += NT) {
        st_rlx(&st->sel_ids[q], sel_ids_s[q]);
        st_rlx(&st->sel_gates[q], sel_g_s[q]);
      }
      if (tid == 0) st_rlx(&st->k, k_s);
    }
  } else {
    // ---------------- router workgroups 0..E-1 (one expert each) publish their logit
    // as {tag, value} in one 64-bit store to their own slot; every workgroup gathers
    // the E slots (bounded spin) and selects for itself. The tag is this call's
    // epoch + 1; the last workgroup of the call stores it as the new epoch. No counter
    // is shared while routing (192 increments of one address serialise at the memory
    // side), and no second round trip for a published selection.
    unsigned long long* slots = dec_slots(acc, hs);
    const uint32_t tag = epoch + 1u;
    if (b < E) {
      // H <= 4096: at most 16 elements per thread, all loaded before the first FMA
      // (one memory round trip), then added in k order
      constexpr int KPT = 4096 / NT;
      float xv[KPT], wr[KPT];
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int kk = tid + i * NT;
        xv[i] = kk < H ? load_as_f32<XT>(x, kk) : 0.0f;
        wr[i] = kk < H ? router[(int64_t)b * H + kk] : 0.0f;
      }
      float sacc = 0.0f;
#pragma unroll
      for (int i = 0; i < KPT; ++i)
        if (tid + i * NT < H) sacc = __builtin_fmaf(xv[i], wr[i], sacc);
      sacc = wave_sum(sacc);
      if (lane == 0) red4[wv] = sacc;
      __syncthreads();
      if (tid < DEC_SLOT_REPS) {  // one copy of the slot per replica, thread r the r-th
        float l = red4[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) l = __fadd_rn(l, red4[w]);
        if (bias) l = __fadd_rn(l, bias[b]);
        st_rlx(&slots[tid * PP_MAX_EXPERTS + b], ((unsigned long long)tag << 32) | __float_as_uint(l));
      }
    }
    // this workgroup gathers from replica b % DEC_SLOT_REPS: a slot line is polled by
    // W / DEC_SLOT_REPS workgroups instead of all of them (reads of one line serialise at
    // the memory side; one copy for 256 workgroups made the gather ~2.8 us at E = 192)
    slots += (b % DEC_SLOT_REPS) * PP_MAX_EXPERTS;
    // router workgroup e publishes {tag, logit} in its own 64-bit slot; every workgroup
    // gathers the E slots (bounded spin). No counter is shared while routing (E
    // increments of one address serialise at the memory side).
    for (int j = tid; j < E; j += NT) {
      unsigned long long v = ld_rlx(&slots[j]);
      uint32_t n = 0;
      while ((uint32_t)(v >> 32) != tag) {
        __builtin_amdgcn_s_sleep(1);
        if (++n > DEC_SPIN_LIMIT) {
          __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          st_rlx(&st->error_call, epoch + 1u);
          break;
        }
        v = ld_rlx(&slots[j]);
      }
      lg_s[j] = __uint_as_float((uint32_t)v);
    }
    __syncthreads();
    if (E <= 16) {
      if (wv == 0) select_one_token([&](int j) { return lg_s[j]; }, E, tau, &ss, lane);
      __syncthreads();
    } else {
      select_one_token_wg([&](int j) { return lg_s[j]; }, E, tau, &ss, keys_s, red4, tid, NT);
    }
    // a selection that is not a permutation of the experts (a broken sort; never, for a
    // correct one) streams nothing and raises the error flag: the output is NaN, not a
    // wrong-but-plausible layer
    const bool bad = E > 16 && ss.bad;
    const int kq = bad ? 0 : ss.k;
    for (int q = tid; q < kq; q += NT) {
      const int e = ss.order[q];
      sel_ids_s[q] = e;
      sel_g_s[q] = pp_sigmoid(lg_s[e]);
    }
    if (tid == 0) {
      k_s = kq;
      if (bad) {
        __hip_atomic_fetch_or(&st->error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_rlx(&st->error_call, epoch + 1u);
      }
    }
    __syncthreads();
    if (b == 0) {  // telemetry for the caller: logits and selection of this call
      for (int j = tid; j < E; j += NT) st_rlx(&st->logits[j], lg_s[j]);
      for (int q = tid; q < k_s; q += NT) {
        st_rlx(&st->sel_ids[q], sel_ids_s[q]);
        st_rlx(&st->sel_gates[q], sel_g_s[q]);
      }
      if (tid == 0) st_rlx(&st->k, k_s);
    }
  }
  const int k = k_s;
  // x, rounded to bf16 like the reference's x.to(bfloat16), as fp32 in registers, from
  // the LDS copy (the DMA issued at the start has landed: the issuing wave waits for its
  // loads, then the barrier; the other waves' stores are not waited for)
  if (wv == NT / 64 - 1) vm_wait();
  __syncthreads();
  float xr[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float vx = ch < HC ? load_as_f32<XT>((const XT*)xs_raw, (int64_t)ch * 8 + i) : 0.0f;
      xr[c][i] = bf16_to_f32(f32_to_bf16(vx));
    }
  }
  dec_clear_previous(acc, hs, hclear, epoch, b, W, tid, NT);

  // ---------------- stream the selected neuron records
  // this workgroup: records [v0, v1) of the k*G selected ones; wave wv a contiguous
  // quarter of them, loaded DEC_RB records at a time (all loads in flight together)
  const int T = k * G;
  int v0, v1;
  pp_split((uint32_t)T, (uint32_t)W, (uint32_t)b, v0, v1);
  const int n = v1 - v0;
  int r = v0 + (n * wv) / NW;
  const int r_end = v0 + (n * (wv + 1)) / NW;

  float oacc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[c][i] = 0.0f;

  // one record per iteration (rolled loop: the code stays small, which matters because
  // the instruction cache is cold at every launch); the next record's loads are issued
  // before the current one is reduced
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  uint4 gq[CPL], uq[CPL], dq[CPL];
  int s_cur = 0, g_cur = 0;
  if (r < r_end) {
    s_cur = (int)((uint32_t)r / (uint32_t)G);
    g_cur = r - s_cur * G;
    const uint4* rec = (const uint4*)(rows + ((int64_t)sel_ids_s[s_cur] * G + g_cur) * 3 * H);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      const bool in = ch < HC;
      gq[c] = in ? rec[ch] : zero4;
      uq[c] = in ? rec[HC + ch] : zero4;
      dq[c] = in ? rec[2 * HC + ch] : zero4;
    }
  }
  for (; r < r_end; ++r) {
    uint4 g2[CPL], u2[CPL], d2[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) { g2[c] = gq[c]; u2[c] = uq[c]; d2[c] = dq[c]; }
    const float gwt = sel_g_s[s_cur];
    if (r + 1 < r_end) {
      if (++g_cur == G) { g_cur = 0; ++s_cur; }
      const uint4* rec = (const uint4*)(rows + ((int64_t)sel_ids_s[s_cur] * G + g_cur) * 3 * H);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + 64 * c;
        const bool in = ch < HC;
        gq[c] = in ? rec[ch] : zero4;
        uq[c] = in ? rec[HC + ch] : zero4;
        dq[c] = in ? rec[2 * HC + ch] : zero4;
      }
    }
    float gs = 0.0f, us = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      gs += dot8(g2[c], xr[c]);
      us += dot8(u2[c], xr[c]);
    }
    gs = wave_sum_dpp(gs);
    us = wave_sum_dpp(us);
    const float a = pp_silu(gs) * us * gwt;
#pragma unroll
    for (int c = 0; c < CPL; ++c) axpy8(a, d2[c], oacc[c]);
  }

  // ---------------- workgroup reduction -> fp32 accumulator copy
  // every wave parks its partials in its own LDS slot, one barrier, then all threads fold
  // the slots in wave order for contiguous h and add to the copy
  const bool has_work = n > 0;
  if (has_work) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + 64 * c;
      if (ch < HC) {
        float4* dst = (float4*)(red + (size_t)wv * H + ch * 8);
        dst[0] = make_float4(oacc[c][0], oacc[c][1], oacc[c][2], oacc[c][3]);
        dst[1] = make_float4(oacc[c][4], oacc[c][5], oacc[c][6], oacc[c][7]);
      }
    }
  }
  __syncthreads();
  if (has_work) {
    dec_acc_t* accc = dec_acc_set(acc, hs, epoch) + (size_t)(b % DEC_NCOPY) * hs;
    for (int h = tid; h < H; h += NT) {
      float sv = red[h];
#pragma unroll
      for (int w = 1; w < NW; ++w) sv += red[(size_t)w * H + h];
      dec_acc_add(accc + h, sv, st, epoch);
    }
  }
  vm_wait();  // every wave's accumulator atomics are performed before the ticket
  __syncthreads();
  if (tid == 0) flag_s = dec_ticket(dec_tickets(acc, hs), b, W);
  __syncthreads();
  if (flag_s) {  // last workgroup: fold copies, write bf16, advance the epoch, reset counters
    // DEC_FOLD_H values of h per thread per pass, every load of a pass issued before
    // the first add (one round trip per pass; one pass for H <= 2048)
    constexpr int DEC_FOLD_H = 8;
    const dec_acc_t* accs = dec_acc_set(acc, hs, epoch);
    const bool failed = ld_rlx(&st->error_call) == epoch + 1u || (ld_rlx(&st->error) & 1u) != 0u;
    for (int h0 = 0; h0 < H; h0 += NT * DEC_FOLD_H) {
      dec_acc_t sv[DEC_FOLD_H][DEC_NCOPY];
#pragma unroll
      for (int i = 0; i < DEC_FOLD_H; ++i) {
        const int h = h0 + tid + i * NT;
#pragma unroll
        for (int c = 0; c < DEC_NCOPY; ++c) sv[i][c] = h < H ? ld_rlx(accs + (size_t)c * hs + h) : (dec_acc_t)0;
      }
#pragma unroll
      for (int i = 0; i < DEC_FOLD_H; ++i) {
        const int h = h0 + tid + i * NT;
        if (h < H) {
          dec_acc_t tot = 0;
#pragma unroll
          for (int c = 0; c < DEC_NCOPY; ++c) tot += sv[i][c];
          out[h] = failed ? (bf16_t)0x7fc0 : f32_to_bf16(dec_from_fixed(tot));
        }
      }
    }
    dec_ticket_reset(dec_tickets(acc, hs), W, tid);
    if (tid == 0) st_rlx(&st->router_ticket, epoch + 1u);  // next call: other accumulator set, new slot tag
  }
}

// ------------------------------------------------------------------ E = 16 fast path
// Specialisation of decode_kernel for exactly 16 experts and H = 512 * CPL (the
// BASELINE shapes): every bound is a compile-time constant, so loads need no guards and
// the selection is branch-free. The instruction cache is cold at each launch and every
// workgroup executes the whole kernel, so the executed code size is latency.

// x chunk ch (8 values) as fp32, bf16-rounded when asked
template <typename XT>
__device__ __forceinline__ void load_x8(const XT* x, int ch, float* v, bool round_bf16);
template <>
__device__ __forceinline__ void load_x8<float>(const float* x, int ch, float* v, bool round_bf16) {
  const float4 a = *(const float4*)(x + ch * 8), b = *(const float4*)(x + ch * 8 + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  if (round_bf16)
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32(f32_to_bf16(v[i]));
}
template <>
__device__ __forceinline__ void load_x8<bf16_t>(const bf16_t* x, int ch, float* v, bool) {
  const uint4 u = *(const uint4*)(x + ch * 8);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// x chunk ch (4 values) as fp32
template <typename XT>
__device__ __forceinline__ float4 load_x4(const XT* x, int ch);
template <>
__device__ __forceinline__ float4 load_x4<float>(const float* x, int ch) {
  return *(const float4*)(x + ch * 4);
}
template <>
__device__ __forceinline__ float4 load_x4<bf16_t>(const bf16_t* x, int ch) {
  const uint2 u = *(const uint2*)(x + ch * 4);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xffff0000u));
}

// x chunk ch (8 values) as packed bf16 pairs, rounded to nearest even
template <typename XT>
__device__ __forceinline__ uint4 load_x8_bf16(const XT* x, int ch);
template <>
__device__ __forceinline__ uint4 load_x8_bf16<float>(const float* x, int ch) {
  const float4 a = *(const float4*)(x + ch * 8), b = *(const float4*)(x + ch * 8 + 4);
  const bf16x2_t p0 = {(__bf16)a.x, (__bf16)a.y}, p1 = {(__bf16)a.z, (__bf16)a.w};
  const bf16x2_t p2 = {(__bf16)b.x, (__bf16)b.y}, p3 = {(__bf16)b.z, (__bf16)b.w};
  return make_uint4(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                    __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3));
}
template <>
__device__ __forceinline__ uint4 load_x8_bf16<bf16_t>(const bf16_t* x, int ch) {
  return *(const uint4*)(x + ch * 8);
}

template <typename XT, int CPL, int NW>
__global__ __launch_bounds__(64 * NW) void decode16_kernel(
    const XT* __restrict__ x, const float* __restrict__ router, const float* __restrict__ bias, int G, float tau,
    const bf16_t* __restrict__ rows, bf16_t* __restrict__ out, pp_decode_state* __restrict__ st,
    dec_acc_t* __restrict__ acc, int hs, int hclear) {
  constexpr int H = 512 * CPL;
  constexpr int HC = H / 8;
  constexpr int NT = 64 * NW;
  extern __shared__ __align__(16) float red[];  // [NW][H]
  __shared__ __align__(16) float part_s[16 * NW];
  __shared__ __align__(16) float lg_s[16];
  __shared__ __align__(16) float pg_s[32];
  __shared__ __align__(16) float srt_s[16];
  __shared__ int flag_s;
  __shared__ int k_s;
  __shared__ int sel_ids_s[16];
  __shared__ float sel_g_s[16];
  __shared__ int main_ids_s[16];
  __shared__ float main_g_s[16];
  __shared__ int kmain_s, spec_s;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = gridDim.x, b = blockIdx.x;
  const uint32_t epoch = ld_rlx(&st->router_ticket);  // accumulator set parity

  // x for the stream as packed bf16 (round to nearest even), loaded now so the loads
  // overlap the routing
  uint4 xb[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) xb[c] = load_x8_bf16<XT>(x, lane + 64 * c);
  const float bias_j = bias != nullptr ? bias[lane & 15] : 0.0f;

  // ---- logits. Wave wv takes the slice [512 CPL wv / NW, 512 CPL (wv + 1) / NW) of
  // x, CPL float4 chunks per lane: lanes form rows of LR = 128 / NW lanes, row rw takes
  // experts rw, rw + NR, ... (NR = 64 / LR rows) and lane cl of the row the chunks
  // cl + LR i. Loads per workgroup: the router once and x once. Rows add by DPP; wave 0
  // adds the NW wave partials in wave order. Every workgroup uses the same order, so
  // every workgroup gets the same logits.
  static_assert(NW == 8 || NW == 16, "decode16_kernel: 8 or 16 waves");
  constexpr int LR = 128 / NW, NR = 64 / LR, EPL = 16 / NR;
  {
    const int rw = lane / LR, cl = lane % LR;
    const int ch0 = (16 * CPL * 8 / NW) * wv + cl;  // float4 chunk index into x / a router row
    float4 xv[CPL];
    float4 wr[EPL][CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) xv[i] = load_x4<XT>(x, ch0 + LR * i);
#pragma unroll
    for (int jj = 0; jj < EPL; ++jj)
#pragma unroll
      for (int i = 0; i < CPL; ++i)
        wr[jj][i] = *(const float4*)(router + (rw + NR * jj) * H + 4 * (ch0 + LR * i));
#pragma unroll
    for (int jj = 0; jj < EPL; ++jj) {
      float sacc = 0.0f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        sacc = __builtin_fmaf(xv[i].x, wr[jj][i].x, sacc);
        sacc = __builtin_fmaf(xv[i].y, wr[jj][i].y, sacc);
        sacc = __builtin_fmaf(xv[i].z, wr[jj][i].z, sacc);
        sacc = __builtin_fmaf(xv[i].w, wr[jj][i].w, sacc);
      }
      sacc = LR == 16 ? row16_sum(sacc) : row8_sum(sacc);
      if (cl == 0) part_s[(rw + NR * jj) * NW + wv] = sacc;
    }
  }
  __syncthreads();

  // ---- logit of expert j = lane & 15 in every wave: the NW wave partials in wave order
  const int j = lane & 15;
  float xl;
  {
    float4 pv[NW / 4];
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) pv[i] = *(const float4*)&part_s[j * NW + 4 * i];
    xl = pv[0].x;
    xl = __fadd_rn(xl, pv[0].y);
    xl = __fadd_rn(xl, pv[0].z);
    xl = __fadd_rn(xl, pv[0].w);
#pragma unroll
    for (int i = 1; i < NW / 4; ++i) {
      xl = __fadd_rn(xl, pv[i].x);
      xl = __fadd_rn(xl, pv[i].y);
      xl = __fadd_rn(xl, pv[i].z);
      xl = __fadd_rn(xl, pv[i].w);
    }
    if (bias != nullptr) xl = __fadd_rn(xl, bias_j);
  }
  const float m = row16_max(xl);

  // ---- speculative top experts. Rank 0 is always selected and is the expert with the
  // largest logit unless probabilities tie (then the lowest index among equal p); rank 1
  // usually is too. So while wave 0 runs the selection, waves 1..7 start loading this
  // workgroup's share of the records of e1 = the lowest index with the largest logit and,
  // when two shares fit (G <= 3 W), of e2 = the lowest index with the largest logit
  // among the rest -- one record per wave, e1's share on the first waves. After the
  // selection barrier a speculative record is used if its expert was selected (then the
  // main stream skips that expert) and dropped otherwise; either way every selected
  // record is used exactly once. No speculation for non-finite or NaN logits.
  // (wave 0 evaluates e1, e2 after its rank step, off its critical path)
  auto top_experts = [&](int& t1, int& t2) {
    t1 = t2 = -1;
    const bool finite = __all(xl == xl) && __fsub_rn(m, m) == 0.0f;
    if (!(DEC16_SPEC(CPL) && finite && G <= 7 * W)) return;
    t1 = __builtin_amdgcn_readfirstlane(row16_min_i(xl == m ? j : 16));
    if (G > 3 * W) return;
    const float m2 = row16_max(j != t1 ? xl : -__builtin_inff());
    t2 = __builtin_amdgcn_readfirstlane(row16_min_i((j != t1 && xl == m2) ? j : 16));
  };
  int e1 = -1, e2 = -1;
  // ---- selection (wave 0), same arithmetic as select_small. Lane (g, j) = 16 g + j
  // serves expert j; the critical path is short dependent chains, so the four 16-lane
  // groups split the work instead of repeating it:
  // * one exp / one division for both outputs: group 1 evaluates the gate
  //   1 / (exp(0 - x_j) + 1) while group 0 evaluates p_j = exp(x_j - max) * (1 / S);
  //   max and S are the xor butterfly i^8, i^4, i^2, i^1 (torch's reduce_all order);
  // * group g compares key_j with the keys of experts 4g .. 4g+3 (64-bit rank keys:
  //   NaN first, then descending p, equal p by index = torch's stable descending sort)
  //   and sums the p of those ranked before j; two xor steps combine the groups;
  // * when every p is 0 or >= 2^-29 each partial sum (< 2) is a multiple of 2^-52 and
  //   exact in double, so {p_q : rank_q <= rank_j} summed in any order equals the fp64
  //   running sum at rank_j; otherwise (or for NaN) the sequential running sum.
  if (wv == 0) {
    const int grp = lane >> 4;
    if (lane < 16) lg_s[j] = xl;  // telemetry
    const float e = pp_expf_u10(grp == 1 ? __fsub_rn(0.0f, xl) : __fsub_rn(xl, m));
    const float S = row16_sum(e);
    const float r = __fdiv_rn(1.0f, grp == 1 ? __fadd_rn(e, 1.0f) : S);
    if (lane < 32) pg_s[lane] = grp == 1 ? r : __fmul_rn(e, r);  // [p_0..15 | gate_0..15]
    wave_sync_lds();
    const float p = pg_s[j];
    const float4 p4 = *(const float4*)&pg_s[4 * grp];
    const float pq[4] = {p4.x, p4.y, p4.z, p4.w};
    const unsigned long long kj = sel_key(p, j);
    int rank = 0, exact = 1;
    double cum = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool before = sel_key(pq[i], 4 * grp + i) < kj;
      rank += before ? 1 : 0;
      cum += before ? (double)pq[i] : 0.0;
      exact &= (int)(pq[i] == 0.0f) | (int)(pq[i] >= 0x1p-29f);  // NaN fails both
    }
    rank += __shfl_xor(rank, 16, PP_WAVE);
    cum += __shfl_xor(cum, 16, PP_WAVE);
    rank += __shfl_xor(rank, 32, PP_WAVE);
    cum += __shfl_xor(cum, 32, PP_WAVE);
    const float tau32 = tau;
    int k;
    bool sel;
    if (__all(exact)) {
      sel = rank == 0 || (float)(cum + (double)p) < tau32;
      k = __popcll(__ballot(sel) & 0xffffull);
    } else {
      if (lane < 16) srt_s[rank] = p;
      wave_sync_lds();
      k = tau_cut([&](int q) { return srt_s[q]; }, 16, tau);
      sel = rank < k;
    }
    // full selection in rank order (telemetry), and the main stream's list: the same
    // without e1 / e2 when selected (their records come from the speculative loads)
    top_experts(e1, e2);
    const unsigned long long selm = __ballot(sel);
    const bool e1_sel = e1 >= 0 && ((selm >> e1) & 1ull);
    const bool e2_sel = e2 >= 0 && ((selm >> e2) & 1ull);
    const int rank_e1 = e1 >= 0 ? __builtin_amdgcn_readlane(rank, e1) : 0;
    const int rank_e2 = e2 >= 0 ? __builtin_amdgcn_readlane(rank, e2) : 0;
    if (lane < 16 && sel) {
      sel_ids_s[rank] = j;
      sel_g_s[rank] = pg_s[16 + j];
      if (!(e1_sel && j == e1) && !(e2_sel && j == e2)) {
        const int mi = rank - ((e1_sel && rank > rank_e1) ? 1 : 0) - ((e2_sel && rank > rank_e2) ? 1 : 0);
        main_ids_s[mi] = j;
        main_g_s[mi] = pg_s[16 + j];
      }
    }
    if (lane == 0) {
      k_s = k;
      kmain_s = k - (e1_sel ? 1 : 0) - (e2_sel ? 1 : 0);
      spec_s = (e1_sel ? 1 : 0) | (e2_sel ? 2 : 0);
    }
  }
  // wave wv >= 1 loads speculative record wv - 1 of this workgroup's shares: e1's share
  // [s0, s1) first, then e2's
  int s0 = 0, s1 = 0, es = -1, ebit = 0, rs = 0;
  if (wv != 0) {
    top_experts(e1, e2);
    if (e1 >= 0) {
      pp_split((uint32_t)G, (uint32_t)W, (uint32_t)b, s0, s1);
      const int q = wv - 1, nsh = s1 - s0;
      if (q < nsh) {
        es = e1, ebit = 1, rs = s0 + q;
      } else if (e2 >= 0 && q < 2 * nsh) {
        es = e2, ebit = 2, rs = s0 + q - nsh;
      }
    }
  }
  const bool have_spec = es >= 0;
  uint4 sg[CPL], su[CPL], sd[CPL];
  if (have_spec) {
    const uint4* rec = (const uint4*)(rows + ((int64_t)es * G + rs) * 3 * H);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      sg[c] = rec[lane + 64 * c];
      su[c] = rec[HC + lane + 64 * c];
      sd[c] = rec[2 * HC + lane + 64 * c];
    }
  }

  wg_lds_barrier();  // LDS only: the speculative loads stay in flight
  const int k = k_s;
  if (b == 0) {  // telemetry for the caller
    if (tid < 16) st_rlx(&st->logits[tid], lg_s[tid]);
    if (tid < k) {
      st_rlx(&st->sel_ids[tid], sel_ids_s[tid]);
      st_rlx(&st->sel_gates[tid], sel_g_s[tid]);
    }
    if (tid == 0) st_rlx(&st->k, k);
  }

  dec_clear_previous(acc, hs, hclear, epoch, b, W, tid, NT, DEC16_NCOPY);

  // ---- stream the selected neuron records (as decode_kernel)
  const bool spec_used = spec_s != 0;
  const int T = kmain_s * G;
  int v0, v1;
  pp_split((uint32_t)T, (uint32_t)W, (uint32_t)b, v0, v1);
  const int n = v1 - v0;
  int r = v0 + (n * wv) / NW;
  const int r_end = v0 + (n * (wv + 1)) / NW;
  float oacc[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[c][i] = 0.0f;
  // one record: gate/up dots over the wave, silu(g) * u * gate, acc += act * down
  auto process = [&](const uint4(&g2)[CPL], const uint4(&u2)[CPL], const uint4(&d2)[CPL], float gwt) {
    float gs = 0.0f, us = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      gs = dot8_bf16(g2[c], xb[c], gs);
      us = dot8_bf16(u2[c], xb[c], us);
    }
    gs = wave_sum_dpp(gs);
    us = wave_sum_dpp(us);
    const float av = pp_silu(gs) * us * gwt;
#pragma unroll
    for (int c = 0; c < CPL; ++c) axpy8(av, d2[c], oacc[c]);
  };
  uint4 gq[CPL], uq[CPL], dq[CPL];
  int s_cur = 0, g_cur = 0;
  if (r < r_end) {
    s_cur = (int)((uint32_t)r / (uint32_t)G);
    g_cur = r - s_cur * G;
    const uint4* rec = (const uint4*)(rows + ((int64_t)main_ids_s[s_cur] * G + g_cur) * 3 * H);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      gq[c] = rec[lane + 64 * c];
      uq[c] = rec[HC + lane + 64 * c];
      dq[c] = rec[2 * HC + lane + 64 * c];
    }
  }
  // the speculative record (loaded before the selection) with its expert's gate
  if (have_spec && (spec_s & ebit)) process(sg, su, sd, pg_s[16 + es]);
  for (; r < r_end; ++r) {
    uint4 g2[CPL], u2[CPL], d2[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) { g2[c] = gq[c]; u2[c] = uq[c]; d2[c] = dq[c]; }
    const float gwt = main_g_s[s_cur];
    if (r + 1 < r_end) {
      if (++g_cur == G) { g_cur = 0; ++s_cur; }
      const uint4* rec = (const uint4*)(rows + ((int64_t)main_ids_s[s_cur] * G + g_cur) * 3 * H);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        gq[c] = rec[lane + 64 * c];
        uq[c] = rec[HC + lane + 64 * c];
        dq[c] = rec[2 * HC + lane + 64 * c];
      }
    }
    process(g2, u2, d2, gwt);
  }

  // ---- workgroup reduction -> one of DEC16_NCOPY fp32 accumulators
  // every wave parks its partials in its LDS slot, then every thread folds the slots in
  // wave order for contiguous h and adds to the copy (uniform over the workgroup:
  // whether it has records of a speculated expert, from the same split)
  const bool spec_wg = spec_used && ((uint32_t)G / (uint32_t)W > 0u || (uint32_t)b < (uint32_t)G % (uint32_t)W);
  if (n > 0 || spec_wg) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      float4* dst = (float4*)(red + wv * H + (lane + 64 * c) * 8);
      dst[0] = make_float4(oacc[c][0], oacc[c][1], oacc[c][2], oacc[c][3]);
      dst[1] = make_float4(oacc[c][4], oacc[c][5], oacc[c][6], oacc[c][7]);
    }
    __syncthreads();
    dec_acc_t* accc = dec_acc_set(acc, hs, epoch) + (b % DEC16_NCOPY) * hs;
#pragma unroll
    for (int i = 0; i < (H + NT - 1) / NT; ++i) {
      const int h = tid + NT * i;
      if (h < H) {
        float v = red[h];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[w * H + h];
        dec_acc_add(accc + h, v, st, epoch);
      }
    }
  }
  vm_wait();  // every wave's accumulator atomics are performed before the ticket
  __syncthreads();
  if (tid == 0) flag_s = dec_ticket(dec_tickets(acc, hs), b, W);
  __syncthreads();
  if (flag_s) {  // last workgroup: fold copies, write bf16, advance the epoch, reset the counter
    // every load of the fold is issued before the first add (one round trip)
    constexpr int HPT = (H + NT - 1) / NT;
    const dec_acc_t* accs = dec_acc_set(acc, hs, epoch);
    const bool failed = ld_rlx(&st->error_call) == epoch + 1u || (ld_rlx(&st->error) & 1u) != 0u;
    dec_acc_t sv[HPT][DEC16_NCOPY];
#pragma unroll
    for (int i = 0; i < HPT; ++i)
#pragma unroll
      for (int c = 0; c < DEC16_NCOPY; ++c) {
        const int h = tid + NT * i;
        sv[i][c] = h < H ? ld_rlx(accs + c * hs + h) : (dec_acc_t)0;
      }
#pragma unroll
    for (int i = 0; i < HPT; ++i) {
      const int h = tid + NT * i;
      if (h < H) {
        dec_acc_t tot = 0;
#pragma unroll
        for (int c = 0; c < DEC16_NCOPY; ++c) tot += sv[i][c];
        out[h] = failed ? (bf16_t)0x7fc0 : f32_to_bf16(dec_from_fixed(tot));
      }
    }
    dec_ticket_reset(dec_tickets(acc, hs), W, tid);
    if (tid == 0) st_rlx(&st->router_ticket, epoch + 1u);
  }
}

__global__ void decode_ws_clear_kernel(uint32_t* p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// state | 2 x DEC_NCOPY x H fixed-point accumulators | DEC_SLOT_REPS x PP_MAX_EXPERTS 64-bit logit slots |
// completion-ticket counters
extern "C" size_t pp_decode_workspace_bytes(int H, int E) {
  (void)E;
  return dec_acc_offset() + (size_t)2 * DEC_NCOPY * H * sizeof(dec_acc_t) +
         (size_t)DEC_SLOT_REPS * PP_MAX_EXPERTS * sizeof(unsigned long long) + (size_t)DEC_TICKET_WORDS * sizeof(uint32_t);
}

extern "C" int pp_decode_workspace_init(void* workspace, int H, int E, void* stream) {
  int rc = pp_check_shape(H, E, 32);
  if (rc) return rc;
  PP_REQUIRE(workspace, PP_ERR_INVALID, "pp_decode_workspace_init: null workspace");
  size_t words = pp_decode_workspace_bytes(H, E) / 4;
  decode_ws_clear_kernel<<<64, 256, 0, (hipStream_t)stream>>>((uint32_t*)workspace, words);
  return pp_check_launch("pp_decode_workspace_init");
}

// The published-logit mode needs its E router workgroups resident together (each
// gathers every router workgroup's slot; the dispatcher starts workgroups in index
// order, so waiting workgroups beyond the first E cannot block them). Checked once per
// kernel variant and device from the occupancy calculator; PP_ERR_UNSUPPORTED when the
// device cannot hold E such workgroups at once.
static int dec_capacity(const void* kern, int nt, size_t smem);
static int dec_check_coresident(const void* kern, int nt, size_t smem, int E) {
  const int cap = dec_capacity(kern, nt, smem);
  PP_REQUIRE(cap >= E, PP_ERR_UNSUPPORTED,
             "pp_moe_decode: the device holds %d decode workgroups at once, fewer than the %d router "
             "workgroups that must be resident together", cap, E);
  return PP_OK;
}

// Workgroups of `kern` the current device holds at once (occupancy calculator), cached
// per kernel, dynamic LDS size and device.
static int dec_capacity(const void* kern, int nt, size_t smem) {
  static std::mutex mu;
  static struct { const void* k; int dev; size_t smem; int cap; } cache[64];
  static int n_cache = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  int cap = -1;
  {
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < n_cache; ++i)
      if (cache[i].k == kern && cache[i].dev == dev && cache[i].smem == smem) cap = cache[i].cap;
  }
  if (cap < 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nt, smem) != hipSuccess) {
      (void)hipGetLastError();
      per_cu = 0;
    }
    cap = per_cu * pp_device_cus();
    std::lock_guard<std::mutex> lk(mu);
    if (n_cache < 64) cache[n_cache++] = {kern, dev, smem, cap};
  }
  return cap;
}

template <typename XT, bool LOCAL>
static int launch_decode(int cpl, int grid, hipStream_t s, const XT* x, int H, const float* router,
                         const float* bias, int E, int G, float tau, const bf16_t* rows, bf16_t* out,
                         pp_decode_state* st, dec_acc_t* acc, int hs, int hclear) {
#define PP_DEC_CASE(C)                                                                                  \
  case C: {                                                                                             \
    const size_t sm = (size_t)DecNW<C>::NW * H * sizeof(float);                                         \
    if (!LOCAL) {                                                                                       \
      const int rc = dec_check_coresident((const void*)decode_kernel<XT, C, LOCAL>, DecNW<C>::NT, sm, E); \
      if (rc) return rc;                                                                                \
    }                                                                                                   \
    decode_kernel<XT, C, LOCAL><<<grid, DecNW<C>::NT, sm, s>>>(x, H, router, bias, E, G, tau, rows, out, st, acc, \
                                                               hs, hclear);                              \
  } break;
  switch (cpl) {
    PP_DEC_CASE(1)
    PP_DEC_CASE(2)
    PP_DEC_CASE(3)
    PP_DEC_CASE(4)
    PP_DEC_CASE(5)
    PP_DEC_CASE(6)
    PP_DEC_CASE(7)
    PP_DEC_CASE(8)
  }
#undef PP_DEC_CASE
  return PP_OK;
}

static int decode_check_args(const void* x, int x_dtype, int H, const float* router_packed, int E, int G,
                             const void* packed, void* out_bf16, int grid) {
  int rc = pp_check_shape(H, E, G);
  if (rc) return rc;
  PP_REQUIRE(x && router_packed && packed && out_bf16, PP_ERR_INVALID, "pp_moe_decode: null pointer");
  PP_REQUIRE(x_dtype == PP_DTYPE_F32 || x_dtype == PP_DTYPE_BF16, PP_ERR_INVALID, "pp_moe_decode: x_dtype %d",
             x_dtype);
  PP_REQUIRE(grid >= 0 && grid <= 65536, PP_ERR_INVALID, "pp_moe_decode: grid %d", grid);
  return PP_OK;
}

// The launch shared by both entry points: st / acc = the state and the accumulators of
// the workspace in use, hs = the stride of one accumulator copy, hclear = how much of
// each copy of the previous call's set to clear.
static int decode_dispatch(const void* x, int x_dtype, int H, const float* router_packed, const float* bias,
                           int E, int G, float tau, const void* packed, void* out_bf16, pp_decode_state* st,
                           dec_acc_t* acc, int hs, int hclear, int grid, hipStream_t s) {
  const int grid_in = grid;
  if (grid == 0) grid = pp_device_cus();
  if (grid < E) grid = E;  // every expert has its router workgroup
  const int cpl = (H / 8 + 63) / 64;  // 16-byte chunks per lane per row (H <= 4096 -> <= 8)
  if (E == 16 && H % 512 == 0) {
    const int c = H / 512;
    const size_t smem16 = (size_t)DEC16_NW * H * sizeof(float);
    if (grid_in == 0) grid = pp_device_cus() / 2;  // measured best: one 8-wave workgroup per two CUs
#define PP_DEC16_CASE(C)                                                                                     \
  case C:                                                                                                    \
    if (x_dtype == PP_DTYPE_F32)                                                                             \
      decode16_kernel<float, C, DEC16_NW><<<grid, 64 * DEC16_NW, smem16, s>>>((const float*)x, router_packed, bias, G, tau, \
                                                               (const bf16_t*)packed, (bf16_t*)out_bf16, st, acc, hs, hclear); \
    else                                                                                                     \
      decode16_kernel<bf16_t, C, DEC16_NW><<<grid, 64 * DEC16_NW, smem16, s>>>((const bf16_t*)x, router_packed, bias, G, tau, \
                                                                (const bf16_t*)packed, (bf16_t*)out_bf16, st, acc, hs, hclear); \
    break;
    switch (c) {
      PP_DEC16_CASE(1)
      PP_DEC16_CASE(2)
      PP_DEC16_CASE(3)
      PP_DEC16_CASE(4)
      PP_DEC16_CASE(5)
      PP_DEC16_CASE(6)
      PP_DEC16_CASE(7)
      PP_DEC16_CASE(8)
    }
#undef PP_DEC16_CASE
    return pp_check_launch("pp_moe_decode");
  }
  const bool local = E <= 16 && (int64_t)16 * H <= DEC_LOCAL_ROUTER_FLOATS;
  const bf16_t* rows = (const bf16_t*)packed;
  bf16_t* o = (bf16_t*)out_bf16;
  int rc;
  if (x_dtype == PP_DTYPE_F32) {
    if (local) rc = launch_decode<float, true>(cpl, grid, s, (const float*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear);
    else rc = launch_decode<float, false>(cpl, grid, s, (const float*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear);
  } else {
    if (local) rc = launch_decode<bf16_t, true>(cpl, grid, s, (const bf16_t*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear);
    else rc = launch_decode<bf16_t, false>(cpl, grid, s, (const bf16_t*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear);
  }
  if (rc) return rc;
  return pp_check_launch("pp_moe_decode");
}

extern "C" int pp_moe_decode(const void* x, int x_dtype, int H, const float* router_packed, const float* bias,
                             int E, int G, float tau, const void* packed, void* out_bf16, void* workspace,
                             int grid, void* stream) {
  int rc = decode_check_args(x, x_dtype, H, router_packed, E, G, packed, out_bf16, grid);
  if (rc) return rc;
  PP_REQUIRE(workspace, PP_ERR_INVALID, "pp_moe_decode: null workspace");
  pp_decode_state* st = (pp_decode_state*)workspace;
  dec_acc_t* acc = (dec_acc_t*)((char*)workspace + dec_acc_offset());
  return decode_dispatch(x, x_dtype, H, router_packed, bias, E, G, tau, packed, out_bf16, st, acc, H, H, grid,
                         (hipStream_t)stream);
}

// ------------------------------------------------------------------ allocation-free entry
// pp_moe_decode_noalloc: pp_moe_decode with the library's own workspace, for callers that
// cannot allocate (code under graph capture, serving loops that forbid hipMalloc). The
// workspace is `scratch`, a file-scope device array of fixed size, one copy per GPU, laid
// out for the largest supported H (accumulator stride 4096) so calls of any shape share
// it; each call clears the whole accumulator set of the previous call. Host code never
// passes `scratch` itself (in host code it names a host-side stand-in, not device
// memory): the device address comes from hipGetSymbolAddress, once per device.
#define PP_DECODE_SCRATCH_HS 4096
static constexpr size_t kDecScratchBytes =
    dec_acc_offset() + (size_t)2 * DEC_NCOPY * PP_DECODE_SCRATCH_HS * sizeof(dec_acc_t) +
    (size_t)DEC_SLOT_REPS * PP_MAX_EXPERTS * sizeof(unsigned long long) + (size_t)DEC_TICKET_WORDS * sizeof(uint32_t);
static_assert(kDecScratchBytes == 306560, "decode scratch: 299 KB per GPU (state, int64 accumulators at stride 4096, "
                                          "slot replicas, ticket counters)");
static __device__ __align__(256) unsigned char scratch[kDecScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// Device address of this device's scratch; the first call on a device also zeroes it
// (a fill kernel on the caller's stream, ordered before the caller's decode).
static int decode_scratch(hipStream_t s, void** out) {
  int dev = 0;
  PP_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, PP_ERR_HIP,
             "pp_moe_decode_noalloc: no current device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    PP_REQUIRE(e == hipSuccess && ptr != nullptr, PP_ERR_HIP, "pp_moe_decode_noalloc: hipGetSymbolAddress: %s",
               hipGetErrorString(e));
    decode_ws_clear_kernel<<<64, 256, 0, s>>>((uint32_t*)ptr, kDecScratchBytes / 4);
    const int rc = pp_check_launch("pp_moe_decode_noalloc (scratch init)");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PP_OK;
}

extern "C" int pp_moe_decode_noalloc(const void* x, int x_dtype, int H, const float* router_packed,
                                     const float* bias, int E, int G, float tau, const void* packed, void* out_bf16,
                                     int grid, void* stream) {
  int rc = decode_check_args(x, x_dtype, H, router_packed, E, G, packed, out_bf16, grid);
  if (rc) return rc;
  PP_REQUIRE(H <= PP_DECODE_SCRATCH_HS && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED,
             "pp_moe_decode_noalloc: H=%d E=%d beyond the scratch maximum (H <= %d, E <= %d)", H, E,
             PP_DECODE_SCRATCH_HS, PP_MAX_EXPERTS);
  hipStream_t s = (hipStream_t)stream;
  void* ptr = nullptr;
  rc = decode_scratch(s, &ptr);
  if (rc) return rc;
  pp_decode_state* st = (pp_decode_state*)ptr;
  dec_acc_t* acc = (dec_acc_t*)((char*)ptr + dec_acc_offset());
  return decode_dispatch(x, x_dtype, H, router_packed, bias, E, G, tau, packed, out_bf16, st, acc,
                         PP_DECODE_SCRATCH_HS, PP_DECODE_SCRATCH_HS, grid, s);
}
