// Decode (one token): a single fused kernel for the whole MoE-MLP layer.
//
// Replaces TauSparseMoE.forward_decode (src/tl_kernel_optimized_Ultimate_PanGU.py:494-530):
// decode_out.zero_() + moe_router_select_kernel_decode (:335-380) +
// moe_decode_swiglu_fused_kernel (:385-462). Differences by design: fp32 router, the
// torch-CPU selection rule (fp64-accumulated cumsum, torch sort order), every neuron of
// every selected expert computed (the reference's 1-D grid leaves pid_g at 0 and only
// covers 64 neurons per expert, :398-399, 515), and a reduction whose order does not
// depend on timing instead of bf16 atomics (the output is the same bits on every call).
//
// Two kernels, by shape.
//
// decode16_kernel (E = 16, H % 512 == 0, G <= 512; the configured shape): every
// workgroup computes all 16 logits (router 98 KB per workgroup, fixed reduction order,
// the same bits everywhere), wave 0 selects, and the layer runs in two phases inside
// the launch. Phase 1: the k*G selected gate/up records are dealt to the streaming
// waves of the whole grid; each publishes act = silu(g.x) * (u.x) * gate per record to
// the workspace. Phase 2: workgroup b owns output rows [h0, h1): their down rows
// (down_t, staged in LDS by DMA while phase 1 runs) times every act, summed in a fixed
// order, written as bf16. No partial output vectors cross workgroups, so no atomics, no
// completion ticket and no fold.
//
// decode_kernel (any other shape, e.g. the checkpoint's E = 192, G = 32): routing in every
// workgroup (small routers) or one logit per router workgroup published in tagged slots;
// every workgroup streams whole {gate, up, down} records, accumulates act * down into a
// partial output, the partials are added in 64-bit fixed point into a few accumulator
// copies, and the last workgroup (completion ticket) writes bf16.
//
// Cross-workgroup data (logits, selection, acts, counters, accumulators) is only accessed
// with agent-scope atomics, and ordering between them comes from waiting for
// completion (s_waitcnt vmcnt(0)) before the dependent atomic. Agent-scope fences are
// avoided on purpose: on gfx950 each one writes back and invalidates the L2, which
// hundreds of workgroups cannot afford inside a 10 us kernel.
#include <algorithm>
#include <cstddef>
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
#define DEC_SPIN_LIMIT (1u << 22)
#define DEC_LOCAL_ROUTER_FLOATS 32768  // Epad*H at or below this: every workgroup routes

static constexpr size_t dec_acc_offset() { return (sizeof(pp_decode_state) + 255) / 256 * 256; }

// Layout tag of a workspace (pp_decode_state::layout): the version of the workspace layout
// (the offsets and sizes below; raised whenever any of them changes) and the accumulator
// stride hs it was initialised for. Every kernel compares the workspace's tag with the one
// its launch expects before its first write into the workspace.
#define DEC_LAYOUT_VERSION 3u
static constexpr uint32_t dec_layout_tag(int hs) {
  return 0xD5000000u | ((DEC_LAYOUT_VERSION & 0x7ffu) << 13) | ((uint32_t)hs & 0x1fffu);
}
static_assert(offsetof(pp_decode_state, layout) == 24 && offsetof(pp_decode_state, error) == 12,
              "pp_decode_state: the header words every layout version keeps in place");


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

// The workspace's layout tag differs from the launch's: the workgroup ends without writing
// into the workspace; workgroup 0 writes NaN to the n outputs and sets error bit 8 (the
// state header sits at the start of every layout). DMAs into LDS issued so far are waited
// for before the workgroup ends. Every workgroup reads the same tag, so all of them end here.
__device__ __forceinline__ void dec_refuse(bf16_t* out, int n, pp_decode_state* st, int b, int tid, int nt) {
  vm_wait();
  if (b != 0) return;
  for (int i = tid; i < n; i += nt) out[i] = (bf16_t)0x7fc0;
  if (tid == 0) __hip_atomic_fetch_or(&st->error, 8u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
      a2[i] = __fadd_rn(b5 ? part[i + 2] : part[i], pl_xor32f(b5 ? part[i] : part[i + 2], lane));
    float t = __fadd_rn(b4 ? a2[1] : a2[0], pl_xor16f(b4 ? a2[0] : a2[1], lane));
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
    pp_decode_state* __restrict__ st, dec_acc_t* __restrict__ acc, int hs, int hclear, uint32_t layout) {
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
  const uint32_t lay = ld_rlx(&st->layout);  // compared before the first workspace write

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
    if (lay != layout) {
      dec_refuse(out, H, st, b, tid, NT);
      return;
    }
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
    }
    if (lay != layout) {
      dec_refuse(out, H, st, b, tid, NT);
      return;
    }
    if (b < E) {
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

// All 16 logits of the token, for the E = 16 kernels: every wave of the workgroup ends with
// the logit of expert lane & 15 (router and x read once per workgroup, a fixed reduction
// order, so every workgroup gets the same bits). Wave wv takes the slice
// [512 CPL wv / NW, 512 CPL (wv + 1) / NW) of x, CPL float4 chunks per lane: lanes form
// rows of LR = 128 / NW lanes, row rw takes experts rw, rw + NR, ... (NR = 64 / LR rows)
// and lane cl of the row the chunks cl + LR i. Rows add by DPP; the NW wave partials are
// added in wave order. part_s: LDS [16 * NW]. Contains a workgroup barrier; `issued` runs
// once this wave's loads are issued, before the barrier (work that waits on an earlier load
// goes there, so that its wait does not hold the router loads back).
struct DecNoHook {
  __device__ void operator()() const {}
};
template <typename XT, int CPL, int NW, typename Hook = DecNoHook>
__device__ __forceinline__ float dec16_logits(const XT* __restrict__ x, const float* __restrict__ router,
                                              const float* __restrict__ bias, float* part_s, int lane, int wv,
                                              Hook issued = Hook()) {
  constexpr int H = 512 * CPL;
  static_assert(NW == 8 || NW == 16, "dec16_logits: 8 or 16 waves");
  constexpr int LR = 128 / NW, NR = 64 / LR, EPL = 16 / NR;
  const float bias_j = bias != nullptr ? bias[lane & 15] : 0.0f;
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
    asm volatile("" ::: "memory");  // the loads above are issued before the hook's work
    issued();
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
  return xl;
}


// ------------------------------------------------------------------ two-phase decode (E = 16)
// Roles inside a workgroup of eight waves. Wave 0 runs the exact selection alone (the
// critical path to the first weight byte: 0.7 us after the logits) and publishes it to
// the other waves through an LDS flag, then DMAs its workgroup's down rows, clears its
// share of the next call's act bank and, in workgroup 0, advances the epoch. Waves 1..7
// stream the records.
// Phase 1 (gate/up): the k*G selected neuron records, in rank order, are dealt to the
// streaming waves of the grid: record t to wave 1 + t % (7W) / W of workgroup t % W, so
// consecutive records spread over workgroups and every workgroup gets the same share. A
// wave issues all its record loads at once, computes act = silu(g.x) * (u.x) * gate per
// record and publishes each act in its own 32-bit word (DEC2_REPS replicas) of this
// call's act bank.
// Phase 2 (down): workgroup b owns output rows [h0, h1) of H; the rows down_t[e][h0..h1)
// of every selected expert are in LDS (wave 0's DMAs). It waits for all k*G act words and
// writes out[h] = sum over ranks s of down_t[e_s][h][.] . act_s -- a fixed order: the bf16
// output is the same bits on every call, with no atomics and no cross-workgroup partial
// sums.
// Speculation: rank 0 is the expert with the largest logit unless probabilities tie, so
// its records and down rows are requested before the cut is known and replaced after it
// when the guess was wrong. Guessing further ranks does not pay: with the whole layer
// requested at once the memory pipeline is saturated, a wave stalls at issue, and
// whatever a guess misses is requested microseconds late.
// Act words: ~bits(act) with NaN canonical, so 0 never occurs and means "not yet
// written". Two banks alternate by call epoch; each call clears the other bank (the one
// the next call uses) early, off its critical path. Every workgroup also marks itself
// alive in the bank; workgroup 0 advances the epoch once every workgroup has (so no
// workgroup of the call can read the next epoch). All W workgroups must be resident
// together (the host clamps W to the device's capacity); waits are bounded: a timeout
// sets error bit 1 and the workgroup writes NaN.
#define DEC2_REPS 4            // replicas of the act words (a line is polled by W / DEC2_REPS workgroups)
// decode2p_kernel publishes and polls replica 0 only (the bank keeps DEC2_REPS replica
// slots for decode16_kernel): at E = 192, G = 32 its 2400 act words per call polled by 256
// workgroups take 16.77 us with one replica, 16.87 with two, 17.01 with four and 17.34
// with eight, where decode16 is fastest with two to four (10.60-10.65 us; one: 10.89)
#define DEC2P_REPS 1
#define DEC2_WMAX 1024         // workgroups per call at most (alive words per bank)
#define DEC2_GMAX 512          // neurons per expert at most (acts of one call fit LDS: 16 * 512 words)
#define DEC2_RS (16 * DEC2_GMAX)  // words per act replica: a fixed layout, whatever the call's G
#define DEC2_LREPS 16          // replicas of the published logit words (decode2p_kernel)
#define DEC2_LOGITS (DEC2_REPS * DEC2_RS)                    // bank offset of the logit words
#define DEC2_ALIVE (DEC2_LOGITS + DEC2_LREPS * PP_MAX_EXPERTS)  // bank offset of the alive marks
#define DEC2_BANK_WORDS (DEC2_ALIVE + DEC2_WMAX)
#define DEC2_DOWN_LDS (96 * 1024)  // LDS for the down rows of one pass (16 positions)

// LDS writes of this wave visible to its other lanes (LDS executes a wave's operations in
// order); unlike a wavefront fence it does not wait for the wave's global loads
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

// 16-byte load with the non-temporal hint (the weight stream is read once per call;
// keeping it out of the caches leaves room for the router and x)
typedef unsigned int dec_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const dec_u32x4 v = __builtin_nontemporal_load((const dec_u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t dec2_word(float a) {
  return ~(a == a ? __float_as_uint(a) : 0x7fc00000u);
}

// Exact tau selection of one token over 16 experts, on one wave: xl = logit of expert
// j = lane & 15 (every lane), m = the largest of the 16 logits. pg_s[0..15] receives the
// probabilities, pg_s[16..31] the gates (sigmoid of the logit). Returns, in every lane,
// whether expert j is selected, with its rank (descending probability, ties by index) and
// the number k of selected experts. When every probability is 0 or >= 2^-29 the fp64
// running sums are exact in any order, so each lane sums the probabilities ranked before
// its own; otherwise the sorted probabilities go through tau_cut's sequential sum.
// srt_s: LDS [16] of this wave. LDS traffic only (no barrier).
__device__ __forceinline__ bool sel16_wave(float xl, float m, float tau, float* pg_s, float* srt_s, int lane,
                                           int& rank_out, int& k_out) {
  const int j = lane & 15;
  const int grp = lane >> 4;
  const float e = pp_expf_u10(grp == 1 ? __fsub_rn(0.0f, xl) : __fsub_rn(xl, m));
  const float S = row16_sum(e);
  const float r = __fdiv_rn(1.0f, grp == 1 ? __fadd_rn(e, 1.0f) : S);
  if (lane < 32) pg_s[lane] = grp == 1 ? r : __fmul_rn(e, r);  // [p_0..15 | gate_0..15]
  wave_lds_sync();
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
    exact &= (int)(pq[i] == 0.0f) | (int)(pq[i] >= 0x1p-29f);
  }
  rank += (int)pl_xor16((uint32_t)rank, lane);
  cum += pl_xor16d(cum, lane);
  rank += (int)pl_xor32((uint32_t)rank, lane);
  cum += pl_xor32d(cum, lane);
  const float tau32 = tau;
  int k;
  bool sel;
  if (__all(exact)) {
    sel = rank == 0 || (float)(cum + (double)p) < tau32;
    k = __popcll(__ballot(sel) & 0xffffull);
  } else {
    if (lane < 16) srt_s[rank] = p;
    wave_lds_sync();
    k = tau_cut([&](int q) { return srt_s[q]; }, 16, tau);
    sel = rank < k;
  }
  rank_out = rank;
  k_out = k;
  return sel;
}

template <typename XT, int CPL>
__global__ __launch_bounds__(512) void decode16_kernel(
    const XT* __restrict__ x, const float* __restrict__ router, const float* __restrict__ bias, int G, float tau,
    const bf16_t* __restrict__ gu, int rec_h, const bf16_t* __restrict__ down_t, bf16_t* __restrict__ out,
    pp_decode_state* __restrict__ st, uint32_t* __restrict__ banks, int rp, int slot_bytes, uint32_t layout) {
  constexpr int NW = 8, NT = 512, H = 512 * CPL, HC = H / 8;
  extern __shared__ __align__(16) unsigned char dn_s[];  // [16][slot_bytes]: down rows of a pass
  __shared__ __align__(16) float part_s[16 * NW];
  __shared__ __align__(16) float pg_s[32];
  __shared__ __align__(16) float srt_s[16];
  __shared__ __align__(16) float act_s[16 * 512];
  __shared__ int k_s, fail_s, ready_s;
  __shared__ uint32_t epoch_s, lay_s;
  __shared__ int L_s[16];    // selected experts in rank order (the stream order)
  __shared__ float Lg_s[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = gridDim.x, b = blockIdx.x;
  // The call's state words are read by thread 0 alone, the load issued first and waited
  // for only once x and the router are requested (inside dec16_logits, before its
  // barrier); the other waves take them from LDS after the barrier.
  uint32_t ep0 = 0u, lay0 = 0u, err0 = 0u;
  if (tid == 0) {
    ep0 = ld_rlx(&st->epoch16);
    lay0 = ld_rlx(&st->layout);  // compared before the first workspace write
    err0 = ld_rlx(&st->error);
  }

  uint4 xb[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) xb[c] = load_x8_bf16<XT>(x, lane + 64 * c);

  const int j = lane & 15;
  const float xl = dec16_logits<XT, CPL, NW>(x, router, bias, part_s, lane, wv, [&]() {
    if (tid == 0) {
      epoch_s = ep0;
      lay_s = lay0;
      if (lay0 == layout)  // alive (has read the epoch)
        st_rlx(&banks[(size_t)(ep0 & 1u) * DEC2_BANK_WORDS + DEC2_ALIVE + b], 1u);
      // an earlier wait timed out: NaN until re-initialised (the AND in asm: computed here,
      // not next to the load, where it would wait for the load before x is requested)
      uint32_t sticky;
      asm volatile("v_and_b32 %0, 1, %1" : "=v"(sticky) : "v"(err0));
      fail_s = (int)sticky;
      ready_s = 0;
    }
  });
  const float m = row16_max(xl);
  if (lay_s != layout) {
    dec_refuse(out, H, st, b, tid, NT);
    return;
  }
  const uint32_t epoch = epoch_s;
  uint32_t* bank = banks + (size_t)(epoch & 1u) * DEC2_BANK_WORDS;

  int h0, h1;  // output rows of this workgroup
  pp_split((uint32_t)H, (uint32_t)W, (uint32_t)b, h0, h1);
  const int cpr = G >> 3;  // 16-byte chunks per down row
  auto dma_rows = [&](int s, int e, int r0, int r1) {  // down_t[e][r0..r1) -> slot s (one wave)
    const int nch = (r1 - r0) * cpr;
    const unsigned char* src = (const unsigned char*)(down_t + ((int64_t)e * H + r0) * G);
    unsigned char* dst = dn_s + s * slot_bytes;
    for (int c0 = 0; c0 < nch; c0 += 64)
      __builtin_amdgcn_global_load_lds(src + 16 * min(c0 + lane, nch - 1),
                                       (__attribute__((address_space(3))) void*)(dst + 16 * c0), 16, 0, 2 /* nt */);
  };
  const int p0_end = min(h1, h0 + rp);
  constexpr int NS = NW - 1;                          // streaming waves 1 .. NW-1

  if (wv == 0) {
    // ---- exact selection, alone on this wave; published to the other waves through an
    // LDS flag, no barrier
    int rank, k;
    const bool sel = sel16_wave(xl, m, tau, pg_s, srt_s, lane, rank, k);
    if (lane < 16 && sel) {
      L_s[rank] = j;
      Lg_s[rank] = pg_s[16 + j];
    }
    if (lane == 0) k_s = k;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_store(&ready_s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // the first pass's down rows of every selected position, DMA'd by this wave (the
    // streaming waves then wait on their own record loads only; a wave that issued DMAs
    // ahead of its records would hold each act until its down rows had landed) --
    // except position 0 when no logit is NaN: wave NW-1 requests it before the cut and
    // corrects it after
    if (h0 < h1)
      for (int s = __all(xl == xl) ? 1 : 0; s < k; ++s) dma_rows(s, L_s[s], h0, p0_end);
    if (b == 0) {  // telemetry for the caller
      if (lane < 16) st_rlx(&st->logits[lane], xl);
      if (lane < k) {
        st_rlx(&st->sel_ids[lane], L_s[lane]);
        st_rlx(&st->sel_gates[lane], Lg_s[lane]);
      }
      if (lane == 0) st_rlx(&st->k, k);
    }
    // the other bank (the next call's): this workgroup's share of clearing it
    uint32_t* nb = banks + (size_t)((epoch + 1u) & 1u) * DEC2_BANK_WORDS;
    int lo_w, hi_w;
    pp_split((uint32_t)DEC2_BANK_WORDS, (uint32_t)W, (uint32_t)b, lo_w, hi_w);
    for (int i = lo_w + lane; i < hi_w; i += 64) st_rlx(&nb[i], 0u);
    if (b == 0) {
      // once every workgroup of the call has marked itself alive (so has read the epoch),
      // advance the epoch: the next call uses the other bank
      bool ok = true;
      for (int i = lane; i < W; i += 64) {
        uint32_t n = 0;
        while (ld_rlx(&bank[DEC2_ALIVE + i]) == 0u) {
          __builtin_amdgcn_s_sleep(8);
          if (++n > DEC_SPIN_LIMIT) {
            ok = false;
            break;
          }
        }
      }
      if (!__all(ok) && lane == 0) {
        __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_rlx(&st->error_call, epoch + 1u);
      }
      if (lane == 0) st_rlx(&st->epoch16, epoch + 1u);
    }
  } else {
    // ---- waves 1 .. NW-1: once the selection is published, every load of the wave is
    // issued at once (its records and the first pass's down rows of its positions), then
    // the records are reduced and published as they arrive. (Loads issued before the cut
    // on a guess do not pay: with the whole layer requested at once the memory pipeline
    // is saturated and a wave stalls at issue, so whatever a guess misses is requested
    // microseconds late.)
    const int Q = W * NS;
    const int t0 = (wv - 1) * W + b, t1 = t0 + Q;
    uint4 ga[CPL], ua[CPL], gb[CPL], ub[CPL];
    auto load_rec = [&](uint4 (&gq)[CPL], uint4 (&uq)[CPL], int t) {
      const int s = t / G;
      const uint4* rec = (const uint4*)(gu + ((int64_t)L_s[s] * G + (t - s * G)) * rec_h * H);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        gq[c] = ld_nt(&rec[lane + 64 * c]);
        uq[c] = ld_nt(&rec[HC + lane + 64 * c]);
      }
    };
    auto dots_publish = [&](const uint4 (&gq)[CPL], const uint4 (&uq)[CPL], int t) {
      float gs = 0.0f, us = 0.0f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        gs = dot8_bf16(gq[c], xb[c], gs);
        us = dot8_bf16(uq[c], xb[c], us);
      }
      gs = wave_sum_dpp(gs);
      us = wave_sum_dpp(us);
      if (lane < DEC2_REPS) st_rlx(&bank[lane * DEC2_RS + t], dec2_word(pp_silu(gs) * us * Lg_s[t / G]));
    };
    // Position 0 (rank 0) is always selected and is the expert with the largest logit
    // unless probabilities tie: its records and down rows are requested before the cut is
    // known (one sixth of the layer's bytes at tau 0.70, in flight during the selection);
    // after the cut they are used if rank 0 is that expert, requested again otherwise.
    const bool spec_ok = __all(xl == xl);
    const int e_top = (int)__builtin_ctz((uint32_t)(__ballot(xl == m) & 0xffffull) | 0x8000u);
    const bool sp_rec = spec_ok && t0 < G, sp_dma = spec_ok && wv == NW - 1 && h0 < h1;
    if (sp_rec) {
      const uint4* rec = (const uint4*)(gu + ((int64_t)e_top * G + t0) * rec_h * H);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        ga[c] = ld_nt(&rec[lane + 64 * c]);
        ua[c] = ld_nt(&rec[HC + lane + 64 * c]);
      }
    }
    if (sp_dma) dma_rows(0, e_top, h0, p0_end);
    while (__hip_atomic_load(&ready_s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0) __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");
    const int k = k_s;
    const int T = k * G;
    const bool top_ok = L_s[0] == e_top;
    if ((sp_rec || sp_dma) && !top_ok) vm_wait();  // a wrong guess has landed before it is replaced
    if (sp_dma && !top_ok) dma_rows(0, L_s[0], h0, p0_end);
    if (t0 < T && !(sp_rec && top_ok)) load_rec(ga, ua, t0);
    if (t1 < T) load_rec(gb, ub, t1);
    for (int t = t0; t < T; t += 2 * Q) {
      dots_publish(ga, ua, t);
      const int ta = t + 2 * Q, tb = t + Q;
      if (ta < T) load_rec(ga, ua, ta);
      if (tb < T) {
        dots_publish(gb, ub, tb);
        if (tb + 2 * Q < T) load_rec(gb, ub, tb + 2 * Q);
      }
    }
  }

  // ---- phase 2: every act word of the call into LDS (bounded wait; replica b % DEC2_REPS),
  // then the rows. Polling starts once this workgroup's own records are published (its
  // polls would otherwise compete with the record stream at the memory side). Wave NW-1
  // (one of the streaming waves with the fewest records, so the first to finish) first
  // runs this code once dry (one poll round, no waits, no output): the instruction cache
  // is cold at each launch, and the dry pass brings the code in before the real pass
  // needs it. (Wave 0 is busy with the down-row DMAs until late in the stream: a dry
  // pass there delays the workgroup's first real poll.)
  const int k = k_s;
  const int T = k * G;
  const uint32_t* rbank = bank + (b % DEC2_REPS) * DEC2_RS;
#pragma nounroll
  for (int pass = wv == NW - 1 ? 0 : 1; pass < 2; ++pass) {
    const bool dry = pass == 0;
    if (!dry) __syncthreads();
    // every word of this thread loaded at once (T <= 16 * G <= 16 * NT), then the words
    // still 0 re-polled together: one memory round trip per round
    bool fail = false;
    uint32_t v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = tid + NT * u;
      v[u] = i < T ? ld_rlx(&rbank[i]) : 1u;
    }
    uint32_t n = 0;
    while (!dry && !fail) {
      bool pending = false;
#pragma unroll
      for (int u = 0; u < 16; ++u) pending |= v[u] == 0u;
      if (!pending) break;
      __builtin_amdgcn_s_sleep(4);
      if (++n > DEC_SPIN_LIMIT) {
        fail = true;
        break;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (v[u] == 0u) v[u] = ld_rlx(&rbank[tid + NT * u]);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = tid + NT * u;
      if (i < T) act_s[i] = __uint_as_float(~v[u]);
    }
    bool failed = false;
    if (!dry) {
      if (fail) fail_s = 1;
      vm_wait();  // this wave's down-row DMAs have landed
      __syncthreads();
      failed = fail_s != 0;
      if (failed && tid == 0) {
        __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_rlx(&st->error_call, epoch + 1u);
      }
    }
    for (int r0 = h0; r0 < h1; r0 += rp) {
      const int r1 = min(h1, r0 + rp);
      if (r0 != h0) {  // later passes (grids smaller than H / rp): DMA, then compute
        if (dry) break;
        __syncthreads();
        for (int s = wv; s < k; s += NW) dma_rows(s, L_s[s], r0, r1);
        vm_wait();
        __syncthreads();
      }
      const int r = r0 + wv;  // wave wv: one row of the pass, lane: one 16-byte chunk
      if (r < r1) {
        float acc = 0.0f;
        if (lane < cpr) {
          const unsigned char* dp = dn_s + (size_t)(wv * G + 8 * lane) * 2;
          const float* ap = act_s + 8 * lane;
#pragma unroll 4
          for (int s = 0; s < k; ++s) {
            const uint4 w = *(const uint4*)(dp + (size_t)s * slot_bytes);
            const float4 a0 = *(const float4*)(ap + s * G), a1 = *(const float4*)(ap + s * G + 4);
            const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            acc += dot8(w, av);
          }
        }
        acc = wave_sum_dpp(acc);
        if (lane == 0 && !dry) out[r] = failed ? (bf16_t)0x7fc0 : f32_to_bf16(acc);
      }
    }
  }
}

// ------------------------------------------------------------------ two-phase decode, any E
// decode2p_kernel: the two phases of decode16_kernel for the other shapes with E*G <= 8192
// and G <= 512 (the checkpoint's E = 192, G = 32 among them). Routing as decode_kernel:
// every workgroup routes when the router is small (E <= 16 and 16*H <= 32768); otherwise
// workgroup e < E computes logit e and publishes it as a word (~bits, 0 = not yet written)
// in DEC2_LREPS replicas kept in this call's act bank, and every workgroup gathers the E
// words of replica b % DEC2_LREPS (the bank is cleared by the previous call, so no tags).
// Selection by wave 0 (E <= 16) or by the workgroup selection (one wave up to E = 128).
// No speculation. The down rows of the k selected experts are one flat list of 16-byte
// chunks, DMA'd by wave 0 (idle during the stream) into contiguous LDS (a G = 32 row is
// only 64 bytes); phase 2 sums each output row over (rank, chunk) items spread over the
// lanes, in a fixed order. Act words in one replica (DEC2P_REPS).
template <typename XT, int CPL, bool LOCAL>
__global__ __launch_bounds__(512) void decode2p_kernel(
    const XT* __restrict__ x, int H, const float* __restrict__ router, const float* __restrict__ bias, int E,
    int G, float tau, const bf16_t* __restrict__ gu, const bf16_t* __restrict__ down_t, bf16_t* __restrict__ out,
    pp_decode_state* __restrict__ st, uint32_t* __restrict__ banks, int rp, uint32_t layout) {
  constexpr int NW = 8, NT = 512, NS = NW - 1;
  extern __shared__ __align__(16) unsigned char dn_s[];  // down rows of a pass: [rank][row][G] bf16 + one pad chunk per rank
  __shared__ __align__(16) float act_s[DEC2_RS + 4 * PP_MAX_EXPERTS];  // [rank][G + 4]: padded rows
  __shared__ SelScratch ss;
  __shared__ unsigned long long keys_s[PP_MAX_EXPERTS];
  __shared__ float lg_s[PP_MAX_EXPERTS];
  __shared__ float red_s[NW];
  __shared__ int L_s[PP_MAX_EXPERTS];
  __shared__ float Lg_s[PP_MAX_EXPERTS];
  __shared__ int fail_s;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = gridDim.x, b = blockIdx.x;
  const int HC = H >> 3;
  const uint32_t epoch = ld_rlx(&st->epoch16);
  const uint32_t lay = ld_rlx(&st->layout);  // compared before the first workspace write
  uint32_t* bank = banks + (size_t)(epoch & 1u) * DEC2_BANK_WORDS;
  if (tid == 0) {
    if (lay == layout) st_rlx(&bank[DEC2_ALIVE + b], 1u);  // alive (has read the epoch)
    fail_s = (ld_rlx(&st->error) & 1u) != 0u;  // an earlier wait timed out: NaN until re-initialised
  }
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  uint4 xb[CPL];  // x as packed bf16 for the records
#pragma unroll
  for (int c = 0; c < CPL; ++c) xb[c] = lane + 64 * c < HC ? load_x8_bf16<XT>(x, lane + 64 * c) : zero4;

  // ---- logits
  if (LOCAL) local_logits<XT, CPL>(x, H, router, bias, E, lg_s, tid);
  if (!LOCAL && b < E) {  // logit b: every element loaded before the first FMA, added in k order
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
    sacc = wave_sum_dpp(sacc);  // fixed order: rows by DPP, then the four row totals
    if (lane == 0) red_s[wv] = sacc;
    __syncthreads();
  }
  if (lay != layout) {
    dec_refuse(out, H, st, b, tid, NT);
    return;
  }
  if (!LOCAL) {
    uint32_t* lw = bank + DEC2_LOGITS;  // [DEC2_LREPS][PP_MAX_EXPERTS]
    if (b < E && tid < DEC2_LREPS) {
      float l = red_s[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) l = __fadd_rn(l, red_s[w]);
      if (bias) l = __fadd_rn(l, bias[b]);
      st_rlx(&lw[tid * PP_MAX_EXPERTS + b], dec2_word(l));
    }
    const uint32_t* rl = lw + (b % DEC2_LREPS) * PP_MAX_EXPERTS;
    if (tid < E) {  // E <= 256 < NT: one word per thread, bounded wait
      uint32_t v = ld_rlx(&rl[tid]), n = 0;
      while (v == 0u) {
        __builtin_amdgcn_s_sleep(1);
        if (++n > DEC_SPIN_LIMIT) {
          fail_s = 1;
          v = 0x803fffffu;  // ~NaN
          break;
        }
        v = ld_rlx(&rl[tid]);
      }
      lg_s[tid] = __uint_as_float(~v);
    }
    __syncthreads();
  }

  // ---- selection (rank order, gates)
  if (E <= 16) {
    if (wv == 0) select_one_token([&](int j) { return lg_s[j]; }, E, tau, &ss, lane);
    __syncthreads();
  } else {
    select_one_token_wg([&](int j) { return lg_s[j]; }, E, tau, &ss, keys_s, red_s, tid, NT);
  }
  // a selection that is not a permutation of the experts (a broken sort; never, for a
  // correct one) streams nothing and raises the error flag: the output is NaN
  const bool bad = E > 16 && ss.bad;
  const int k = bad ? 0 : ss.k;
  for (int q = tid; q < k; q += NT) {
    const int e = ss.order[q];
    L_s[q] = e;
    Lg_s[q] = pp_sigmoid(lg_s[e]);
  }
  if (tid == 0 && bad) {
    fail_s = 1;
    __hip_atomic_fetch_or(&st->error, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    st_rlx(&st->error_call, epoch + 1u);
  }
  __syncthreads();
  const int T = k * G;
  if (b == 0) {  // telemetry for the caller: logits and selection of this call
    for (int j = tid; j < E; j += NT) st_rlx(&st->logits[j], lg_s[j]);
    for (int q = tid; q < k; q += NT) {
      st_rlx(&st->sel_ids[q], L_s[q]);
      st_rlx(&st->sel_gates[q], Lg_s[q]);
    }
    if (tid == 0) st_rlx(&st->k, k);
  }
  {  // this workgroup's share of clearing the other bank (the next call's)
    uint32_t* nb = banks + (size_t)((epoch + 1u) & 1u) * DEC2_BANK_WORDS;
    int lo_w, hi_w;
    pp_split((uint32_t)DEC2_BANK_WORDS, (uint32_t)W, (uint32_t)b, lo_w, hi_w);
    for (int i = lo_w + tid; i < hi_w; i += NT) st_rlx(&nb[i], 0u);
  }

  int h0, h1;  // output rows of this workgroup
  pp_split((uint32_t)H, (uint32_t)W, (uint32_t)b, h0, h1);
  const int cpr = G >> 3;  // 16-byte chunks per down row
  // down rows [r0, r1) of ranks 0 .. k-1 -> LDS, one wave: rank s's (row, chunk) c at LDS chunk
  // s * (per + 1) + c; the chunk after each rank is padding (it fetches the rank's last
  // chunk again), so ranks sit an odd number of chunks apart and the row sums' reads of
  // consecutive ranks fall in different LDS banks. Four DMA instructions per round: their
  // (rank, chunk) and expert ids are computed and read from LDS together, so one LDS round
  // trip serves four instructions (the issue loop was otherwise the DMAs' bottleneck:
  // E=192 decode 18.9 -> 17.9 us). rank = floor(c / pp) as umulhi(c, floor((2^32-1)/pp)+1),
  // exact for c * pp < 2^32 (here c < 6208, 5 <= pp <= 513)
  auto dma_rows = [&](int r0, int r1) {
    const int per = (r1 - r0) * cpr, pp = per + 1, nq = k * pp;
    const uint32_t magic = 0xffffffffu / (uint32_t)pp + 1u;
    const bf16_t* base = down_t + (int64_t)r0 * G;
    for (int c0 = 0; c0 < nq; c0 += 256) {
      uint32_t e[4];
      int rq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = min(c0 + 64 * j + lane, nq - 1);
        const int s = (int)__umulhi((uint32_t)c, magic);
        rq[j] = min(c - s * pp, per - 1);
        e[j] = (uint32_t)L_s[s];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c0 + 64 * j < nq)
          __builtin_amdgcn_global_load_lds(base + ((int64_t)e[j] * H * G + 8 * rq[j]),
                                           (__attribute__((address_space(3))) void*)(dn_s + 16 * (c0 + 64 * j)), 16, 0, 2);
    }
  };
  if (wv == 0) {
    // the first pass's down rows, all on this wave (idle during the stream): a streaming
    // wave that also DMAs would wait for its DMAs before its first dot (loads complete in
    // issue order)
    if (h0 < h1 && k > 0) dma_rows(h0, min(h1, h0 + rp));
    if (b == 0) {
      // once every workgroup of the call has marked itself alive (so has read the epoch),
      // advance the epoch: the next call uses the other bank
      bool ok = true;
      for (int i = lane; i < W; i += 64) {
        uint32_t n = 0;
        while (ld_rlx(&bank[DEC2_ALIVE + i]) == 0u) {
          __builtin_amdgcn_s_sleep(8);
          if (++n > DEC_SPIN_LIMIT) {
            ok = false;
            break;
          }
        }
      }
      if (!__all(ok) && lane == 0) {
        __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_rlx(&st->error_call, epoch + 1u);
      }
      if (lane == 0) st_rlx(&st->epoch16, epoch + 1u);
    }
  } else {
    // ---- phase 1 (waves 1 .. NW-1): records t0, t0 + Q, ... of the k*G selected ones
    const int Q = W * NS;
    const int t0 = (wv - 1) * W + b, t1 = t0 + Q;
    uint4 ga[CPL], ua[CPL], gb[CPL], ub[CPL];
    auto load_rec = [&](uint4 (&gq)[CPL], uint4 (&uq)[CPL], int t) {
      const int s = t / G;
      const uint4* rec = (const uint4*)(gu + ((int64_t)L_s[s] * G + (t - s * G)) * 3 * H);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + 64 * c;
        gq[c] = ch < HC ? ld_nt(&rec[ch]) : zero4;
        uq[c] = ch < HC ? ld_nt(&rec[HC + ch]) : zero4;
      }
    };
    auto dots_publish = [&](const uint4 (&gq)[CPL], const uint4 (&uq)[CPL], int t) {
      float gs = 0.0f, us = 0.0f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        gs = dot8_bf16(gq[c], xb[c], gs);
        us = dot8_bf16(uq[c], xb[c], us);
      }
      gs = wave_sum_dpp(gs);
      us = wave_sum_dpp(us);
      if (lane < DEC2P_REPS) st_rlx(&bank[lane * DEC2_RS + t], dec2_word(pp_silu(gs) * us * Lg_s[t / G]));
    };
    if (t0 < T) load_rec(ga, ua, t0);
    if (t1 < T) load_rec(gb, ub, t1);
    for (int t = t0; t < T; t += 2 * Q) {
      dots_publish(ga, ua, t);
      const int ta = t + 2 * Q, tb = t + Q;
      if (ta < T) load_rec(ga, ua, ta);
      if (tb < T) {
        dots_publish(gb, ub, tb);
        if (tb + 2 * Q < T) load_rec(gb, ub, tb + 2 * Q);
      }
    }
  }

  // ---- phase 2: every act word of the call into LDS (replica b % DEC2P_REPS, bounded
  // wait), then the rows. Wave NW-1 (among the streaming waves with the fewest records)
  // first runs the polls and act writes once dry (one poll round, no waits): the
  // instruction cache is cold at each launch. Each lane reads
  // four ranks' operands before adding their products (in rank order), one LDS round trip
  // per four ranks.
  const uint32_t* rbank = bank + (b % DEC2P_REPS) * DEC2_RS;
  // lanes: (sub, chunk) with sub = lane / cpr when cpr divides 64 (spl ranks per wave
  // pass), else one rank at a time; row r0 + wv of the pass on wave wv
  const int spl = (64 % cpr == 0) ? 64 / cpr : 1;
  const int sub = lane / cpr, cc = lane - sub * cpr;
#pragma nounroll
  for (int pass = wv == NW - 1 ? 0 : 1; pass < 2; ++pass) {
    const bool dry = pass == 0;
    if (!dry) __syncthreads();
    bool fail = false;
    uint32_t v[16];  // T <= E*G <= 16 * NT
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int i = tid + NT * u;
      v[u] = i < T ? ld_rlx(&rbank[i]) : 1u;
    }
    uint32_t n = 0;
    while (!dry && !fail) {
      bool pending = false;
#pragma unroll
      for (int u = 0; u < 16; ++u) pending |= v[u] == 0u;
      if (!pending) break;
      __builtin_amdgcn_s_sleep(4);
      if (++n > DEC_SPIN_LIMIT) {
        fail = true;
        break;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (v[u] == 0u) v[u] = ld_rlx(&rbank[tid + NT * u]);
    }
    // act of (rank s, neuron g) to act_s[s * (G + 4) + g]: rows padded so the row sums'
    // reads of consecutive ranks fall in different banks; word tid + NT u walks (s, g)
    // by NT per step
    {
      int sa = tid / G, ga = tid - sa * G;
      const int ds = NT / G, dg = NT - ds * G;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (tid + NT * u < T) act_s[sa * (G + 4) + ga] = __uint_as_float(~v[u]);
        sa += ds;
        ga += dg;
        if (ga >= G) {
          ga -= G;
          ++sa;
        }
      }
    }
    bool failed = false;
    if (!dry) {
      if (fail) fail_s = 1;
      vm_wait();  // wave 0's down-row DMAs have landed
      __syncthreads();
      failed = fail_s != 0;
      if (failed && tid == 0) {
        __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_rlx(&st->error_call, epoch + 1u);
      }
    }
    if (dry) continue;  // on to the real pass: the dry one covers the polls and the act
                        // writes (a dry row sum delayed the real pass: 16.8 -> 16.5 us
                        // without it at E = 192)
    for (int r0 = h0; r0 < h1; r0 += rp) {
      const int r1 = min(h1, r0 + rp), nr = r1 - r0;
      if (r0 != h0) {  // later passes (grids smaller than H / rp): DMA, then compute
        __syncthreads();
        if (wv == 0 && k > 0) dma_rows(r0, r1);
        vm_wait();
        __syncthreads();
      }
      const int wr = wv;
      if (wr < nr) {
        float acc = 0.0f;
        if (sub < spl) {
          // four ranks' operands read before their products are added (in rank order)
          const float4* a4 = (const float4*)act_s;
          const int g4 = (G + 4) >> 2, rs = nr * cpr + 1;
          for (int s0 = sub; s0 < k; s0 += 4 * spl) {
            uint4 w[4];
            float4 a0[4], a1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int s = min(s0 + j * spl, k - 1);
              w[j] = *(const uint4*)(dn_s + 16 * (s * rs + wr * cpr + cc));
              a0[j] = a4[s * g4 + 2 * cc];
              a1[j] = a4[s * g4 + 2 * cc + 1];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float av[8] = {a0[j].x, a0[j].y, a0[j].z, a0[j].w, a1[j].x, a1[j].y, a1[j].z, a1[j].w};
              const float d = dot8(w[j], av);
              if (s0 + j * spl < k) acc += d;
            }
          }
        }
        acc = wave_sum_dpp(acc);
        if (lane == 0 && !dry) out[r0 + wr] = failed ? (bf16_t)0x7fc0 : f32_to_bf16(acc);
      }
    }
  }
}

// ------------------------------------------------------------------ batch decode (E = 16)
// decodeb_kernel: one launch for 1 <= N <= 64 tokens (small-batch decode), every workgroup
// resident at once, exchanging data through the batch workspace:
// A. workgroup b < N routes token b (dec16_logits, sel16_wave on wave 0), writes x as bf16
//    in MFMA-fragment order and then publishes its 16 gates as tagged words (gate bits,
//    exactly -1 for an expert not selected; a selected gate is a sigmoid, or NaN);
// B. every workgroup polls the N x 16 tagged gates; the union of the selected experts,
//    ascending, gives T = nu * G union neurons, union neuron q being neuron q % G of
//    expert U[q / G];
// C. gate/up: workgroup b takes union neurons [q0, q1) of an even split of T in groups of
//    8, in blocks of at most 24 neurons, all N tokens. K = H is split over the eight
//    waves (wave w takes the 64-element K-blocks w, w + 8, ...): a wave DMAs the gate and
//    up rows of each of its K-blocks into its own LDS ring of three stages (whole 128-byte
//    lines per request, chunks XOR-swizzled by row) and loads the x fragments into
//    registers (1 KB contiguous per request); 32x32x16 MFMA, tokens x neurons. The eight
//    partials go through LDS and every thread adds them in wave order; act[t][q] =
//    silu(g) * u * gate(t, e) (0 where token t did not select e) is published as bf16 in
//    MFMA-fragment order. Speculation: the first stages are requested before the routing,
//    assuming every expert is hit (16 of 16 in config 3), and drained if not;
// D. down: workgroup b = 16 r + s takes the rows of row group r (8-row blocks of H split
//    over W / 16 groups) and the union neurons of slice s (16-neuron blocks of T split
//    over 16 slices; with all 16 experts hit, slice s is expert s): its down rows are
//    DMA'd to LDS once its acts are published, and MFMA (rows x tokens) over the slice
//    writes a partial [row][token] sum in fp32;
// E. fold: the 8-row block u of H is summed over the 16 slices in slice order by
//    workgroup u % W, so the bf16 output is the same bits on every call.
// Exchanges: data written with coherent (sc1) stores, then made visible by a tag (the
// call's epochb + 1): the gates carry it in their upper word, the acts and partial sums
// by a per-workgroup flag word set once those stores completed; readers wait for the tags
// they depend on, then load with sc1 (a workgroup whose wait timed out publishes NaN acts
// and partial sums, so every output it feeds is NaN). Tags grow by one per call, so
// nothing needs clearing; workgroup 0 advances epochb once every workgroup has set its
// last flag. Every wait is bounded: a timeout sets error bit 1 and the workgroup writes
// NaN. Workspace reads and writes go through buffer descriptors sized to their region.
#define DECB_MAXN 64                   // tokens per call at most
#define DECB_S 16                      // neuron slices of the down projection
#define DECB_NB 24                     // neurons per gate/up block
#define DECB_STAGE (2 * DECB_NB * 128)  // one K-block of a neuron block: gate rows | up rows, 128 B each
#define DECB_RING_WAVE (3 * DECB_STAGE)  // LDS ring of one wave (three stages)
#define DECB_RED_BYTES (2 * 8 * 2048 * 4)  // LDS of the K partials: two token blocks x eight waves x g|u x 16 x 64
#define DECB_SMEM (8 * DECB_RING_WAVE)  // dynamic LDS: the rings; then the partials and acts; then down rows
#define DECB_DOWN_LDS DECB_SMEM         // LDS of the down rows of one pass
static_assert(DECB_RED_BYTES + 64 * 32 * 2 <= DECB_SMEM, "batch decode LDS plan");
// In the decode workspace (zeroed once, private to its epoch): everything that carries a
// tag -- the tagged gates [64][16] u64, then the act and partial flags (a word per
// workgroup). A tag is only meaningful against the epoch of its own workspace, so tagged
// words never live in the batch workspace, which needs no initialisation and may be
// shared by several decode workspaces (layers) or recycled by an allocator.
#define DECB_SELG_BYTES (DECB_MAXN * 16 * 8)
#define DECB_STATE_BYTES (DECB_SELG_BYTES + 2 * DEC2_WMAX * 4)

struct DecbLayout {
  size_t xf, af, part, total;
};
// batch workspace: x fragments (H / 64 K-blocks x 4 k-steps x 2 token blocks x 64 lanes x
// 16 B) | act fragments (16 G / 16 k-steps x 2 x 64 x 16 B) | partial sums [16][H][64] fp32
__host__ __device__ __forceinline__ DecbLayout decb_layout(int H, int G) {
  DecbLayout L;
  size_t o = 0;
  L.xf = o;
  o += (size_t)DECB_MAXN * H * 2;
  L.af = o;
  o += (size_t)DECB_MAXN * 16 * G * 2;
  L.part = o;
  o += (size_t)DECB_S * H * DECB_MAXN * 4;
  L.total = o;
  return L;
}
// byte offset of the 16-byte MFMA fragment (k-step ks, token block tb, lane L) in the x and
// act fragment arrays: lane L holds row tb * 32 + L % 32, elements 16 ks + 8 (L / 32) ..
__device__ __forceinline__ uint32_t decb_frag(int ks, int tb, int L) {
  return (uint32_t)(((ks * 2 + tb) * 64 + L) * 16);
}

typedef __amdgpu_buffer_rsrc_t decb_rsrc_t;
__device__ __forceinline__ decb_rsrc_t decb_rsrc(const void* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
#define DECB_SC1 16  // cache policy: coherent across the device's L2s
#define DECB_NT 2    // cache policy: non-temporal
template <int AUX>
__device__ __forceinline__ uint4 decb_ld16(decb_rsrc_t r, uint32_t off) {
  const dec_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void decb_st16(decb_rsrc_t r, uint32_t off, uint4 v) {
  const dec_u32x4 u = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(u, r, off, 0, DECB_SC1);
}

// bounded wait for a flag word to hold `tag`; false on timeout
__device__ __forceinline__ bool decb_wait(const uint32_t* f, uint32_t tag) {
  uint32_t n = 0;
  while (ld_rlx(f) != tag) {
    __builtin_amdgcn_s_sleep(2);
    if (++n > DEC_SPIN_LIMIT) return false;
  }
  return true;
}

// the loads feeding `v` have completed (the compiler waits for them here), and no memory
// access below moves above this point
__device__ __forceinline__ void decb_ready(dec_u32x4& v) { asm volatile("" : "+v"(v) : : "memory"); }
__device__ __forceinline__ dec_u32x4 decb_ld16v(decb_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, DECB_SC1);
}
__device__ __forceinline__ f32x16_t mfma32x(dec_u32x4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), as_bf16x8(b), c, 0, 0, 0);
}

template <typename XT, int CPL, int TB>
__global__ __launch_bounds__(512) void decodeb_kernel(
    const XT* __restrict__ x, int N, const float* __restrict__ router, const float* __restrict__ bias, int G,
    float tau, const bf16_t* __restrict__ gu, const bf16_t* __restrict__ down_t, bf16_t* __restrict__ out,
    float* __restrict__ logits_out, uint8_t* __restrict__ mask_out, pp_decode_state* __restrict__ st,
    unsigned char* __restrict__ bstate, unsigned char* __restrict__ bw, int rows_pp, uint32_t layout) {
  constexpr int NW = 8, NT = 512, H = 512 * CPL, HC = H / 8;
  constexpr int DP = CPL < 3 ? CPL : 3;  // gate/up stages in flight per wave (CPL K-blocks per wave)
  extern __shared__ __align__(16) unsigned char smem[];  // rings | later: reduction area, down rows
  float* red_s = (float*)smem;                         // [TB][8 waves][g|u][16][64] K partials
  bf16_t* act_s = (bf16_t*)(smem + DECB_RED_BYTES);    // [64][32] acts of a neuron block
  unsigned char* dn_s = smem;                          // down rows (once the acts are published)
  __shared__ __align__(16) float part_s[16 * NW];
  __shared__ __align__(16) float pg_s[32];
  __shared__ __align__(16) float srt_s[16];
  __shared__ __align__(16) float sg_s[DECB_MAXN * 16];  // gate of (token, expert); -1: not selected
  __shared__ int ul_s[16];                              // the union of the selected experts, ascending
  __shared__ int nu_s;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int W = gridDim.x, b = blockIdx.x;
  const uint32_t tag = ld_rlx(&st->epochb) + 1u;
  const uint32_t lay = ld_rlx(&st->layout);  // compared before the first workspace write
  bool fail = (ld_rlx(&st->error) & 1u) != 0u;  // an earlier wait timed out: NaN until re-initialised
  const DecbLayout Lb = decb_layout(H, G);
  unsigned long long* selg = (unsigned long long*)bstate;
  const decb_rsrc_t r_xf = decb_rsrc(bw + Lb.xf, Lb.af - Lb.xf);
  const decb_rsrc_t r_af = decb_rsrc(bw + Lb.af, Lb.part - Lb.af);
  const decb_rsrc_t r_part = decb_rsrc(bw + Lb.part, Lb.total - Lb.part);
  uint32_t* aflag = (uint32_t*)(bstate + DECB_SELG_BYTES);
  uint32_t* pflag = aflag + DEC2_WMAX;

  const int jn = lane & 31, kh = lane >> 5;
  // gate/up rows of K-block wv + 8 j of the neuron block [nb0, nb0 + nq) -> ring stage j % DP:
  // gate rows 0 .. nq-1, up rows nq .. 2nq-1, chunk c of row r at position c ^ (r & 7) (nq is a
  // multiple of 8: a neuron's gate and up rows share the swizzle); whole 128-byte lines, 1 KB
  // per instruction. expert(u): expert of union position u.
  unsigned char* ring = smem + wv * DECB_RING_WAVE;
  auto issue_w = [&](int nb0, int nq, int j, auto expert) {
    const int kb = wv + NW * j;
    unsigned char* slot = ring + (j % DP) * DECB_STAGE;
    for (int ii = 0; ii < nq / 4; ++ii) {
      const int f = 64 * ii + lane, rr = f >> 3;
      const int which = rr >= nq ? 1 : 0, q = nb0 + rr - which * nq;
      const int eg = q / G;
      const bf16_t* src = gu + (size_t)((expert(eg) * G + q - eg * G) * 3 + which) * H + kb * 64 +
                          8 * ((f & 7) ^ (rr & 7));
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(slot + 1024 * ii), 16, 0,
                                       DECB_NT);
    }
  };
  // x fragments of K-block wv + 8 j (1 KB contiguous per instruction)
  auto issue_x = [&](int j, dec_u32x4 (&xa)[TB][4]) {
    const int kb = wv + NW * j;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) xa[tb][i] = decb_ld16v(r_xf, decb_frag(kb * 4 + i, tb, lane));
  };
  // Speculation: with every expert selected by some token (the usual case for batches of 16
  // and more) the union is 0 .. 15 and this workgroup's first neuron block is known before
  // the routing, so its first DP stages are requested early -- at the start, or, in a
  // routing workgroup, once its gates are out (its x stores must complete first, and loads
  // in flight would hold that wait); a wrong guess only costs the bytes.
  int sp0, sp1;
  pp_split((uint32_t)(16 * G / 8), (uint32_t)W, (uint32_t)b, sp0, sp1);
  const bool spec = sp1 > sp0;
  auto issue_spec = [&]() {
    if (spec)
#pragma unroll
      for (int j = 0; j < DP; ++j) issue_w(8 * sp0, min(DECB_NB, 8 * (sp1 - sp0)), j, [](int e) { return e; });
  };
  if (b >= N) issue_spec();
  // a workspace of another layout: NaN outputs (logits NaN, masks 0), nothing written into it
  auto refuse = [&]() {
    dec_refuse(out, N * H, st, b, tid, NT);
    if (b == 0)
      for (int i = tid; i < N * 16; i += NT) {
        if (logits_out != nullptr) logits_out[i] = __uint_as_float(0x7fc00000u);
        if (mask_out != nullptr) mask_out[i] = 0;
      }
  };
  if (b >= N && lay != layout) {
    refuse();
    return;
  }

  // ---- A: routing of token b
  if (b < N) {
    const XT* xt = x + (size_t)b * H;
    const float xl = dec16_logits<XT, CPL, NW>(xt, router, bias, part_s, lane, wv);
    for (int c = tid; c < HC; c += NT) {  // chunk c: K-block c / 8, k-step c % 4, half (c / 4) % 2
      const int q = c & 7;
      decb_st16(r_xf, decb_frag((c >> 3) * 4 + (q & 3), b >> 5, (b & 31) + 32 * (q >> 2)), load_x8_bf16<XT>(xt, c));
    }
    bool sel = false;
    if (wv == 0) {
      int rank, k;
      sel = sel16_wave(xl, row16_max(xl), tau, pg_s, srt_s, lane, rank, k);
    }
    vm_wait();
    __syncthreads();  // x is stored: the gates may go out
    if (lay != layout) {
      refuse();
      return;
    }
    if (wv == 0 && lane < 16) {
      const uint32_t gb = __float_as_uint(sel ? pg_s[16 + lane] : -1.0f);
      __hip_atomic_store(&selg[b * 16 + lane], ((unsigned long long)tag << 32) | gb, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (logits_out != nullptr) logits_out[b * 16 + lane] = xl;
      if (mask_out != nullptr) mask_out[b * 16 + lane] = sel ? 1 : 0;
    }
    issue_spec();
  }

  // ---- B: every token's gates (tagged words, at most two per thread); the union
  {
    unsigned long long v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = tid + NT * u;
      v[u] = i < N * 16 ? __hip_atomic_load(&selg[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : ((unsigned long long)tag << 32);
    }
    uint32_t n = 0;
    while (!fail && ((uint32_t)(v[0] >> 32) != tag || (uint32_t)(v[1] >> 32) != tag)) {
      __builtin_amdgcn_s_sleep(2);
      if (++n > DEC_SPIN_LIMIT) {
        fail = true;
        break;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
        if ((uint32_t)(v[u] >> 32) != tag)
          v[u] = __hip_atomic_load(&selg[tid + NT * u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (tid + NT * u < N * 16) sg_s[tid + NT * u] = __uint_as_float((uint32_t)v[u]);
  }
  fail = __syncthreads_or(fail);  // from here on a failed workgroup publishes NaN
  if (wv == 0) {
    bool hit = false;
    if (lane < 16)
      for (int t = 0; t < N; ++t) hit |= sg_s[t * 16 + lane] != -1.0f;
    const unsigned long long bal = __ballot(hit);
    if (hit) ul_s[__popcll(bal & ((1ull << lane) - 1ull))] = lane;
    if (lane == 0) nu_s = __popcll(bal);
  }
  __syncthreads();
  const int T = nu_s * G;

  // rows and slice of phase D
  const int R = W / DECB_S, s = b % DECB_S, r = b / DECB_S;
  int rb0, rb1, sb0, sb1;
  pp_split((uint32_t)(H / 8), (uint32_t)R, (uint32_t)r, rb0, rb1);
  pp_split((uint32_t)(T / 16), (uint32_t)DECB_S, (uint32_t)s, sb0, sb1);
  const int hr0 = 8 * rb0, hr1 = 8 * rb1;
  const int a0 = 16 * sb0, nk = 16 * (sb1 - sb0);
  const int cpr = nk / 8, RSB = 16 * (cpr + 1);  // staged row: cpr chunks + one pad chunk
  // down rows [p0, p0 + nr) of the slice -> LDS: row rho at rho * RSB, chunk c (8 union
  // neurons a0 + 8c ..) at + 16 c; the pad chunk fetches the row's last chunk again.
  // Instructions part, part + nparts, ... of the flat list (64 chunks each), four per round
  // (one LDS round trip for their expert ids); the divisions by cpr + 1 and G as
  // multiply-high by floor((2^32-1)/d)+1, exact for n * d < 2^32 (n < 9280 and d <= 65,
  // n < 8192 and d <= 512 here)
  const uint32_t mag_c = 0xffffffffu / (uint32_t)(cpr + 1) + 1u, mag_g = 0xffffffffu / (uint32_t)G + 1u;
  auto dma_rows = [&](int p0, int nr, int part, int nparts) {
    if (cpr == 0) return;
    const int total = nr * (cpr + 1), step = 64 * nparts;
    for (int i00 = 64 * part; i00 < total; i00 += 4 * step) {
      int e[4], off[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = min(i00 + j * step + lane, total - 1);
        const int rho = (int)__umulhi((uint32_t)f, mag_c);
        const int c = min(f - rho * (cpr + 1), cpr - 1);
        const int q = a0 + 8 * c;
        const int ue = (int)__umulhi((uint32_t)q, mag_g);
        e[j] = ul_s[ue];
        off[j] = (p0 + rho) * G + q - ue * G;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i00 + j * step < total)
          __builtin_amdgcn_global_load_lds(down_t + (size_t)e[j] * H * G + off[j],
                                           (__attribute__((address_space(3))) void*)(dn_s + 16 * (i00 + j * step)), 16,
                                           0, DECB_NT);
    }
  };

  // ---- C: gate/up of union neurons [q0, q1), blocks of at most DECB_NB
  int g0, g1;
  pp_split((uint32_t)(T / 8), (uint32_t)W, (uint32_t)b, g0, g1);
  const int q0 = 8 * g0, q1 = 8 * g1;
  const bool spec_hit = spec && nu_s == 16;  // the rows requested at the start are this block's
  if (spec && !spec_hit) vm_wait();          // wrong guess: they land before the rings are reused
  for (int nb0 = q0; nb0 < q1; nb0 += DECB_NB) {
    const int nq = min(DECB_NB, q1 - nb0);  // a multiple of 8
    const int nn = min(jn, nq - 1);         // this lane's neuron (B column; lanes beyond nq repeat the last)
    dec_u32x4 xa[DP][TB][4];
    if (!(spec_hit && nb0 == q0))
#pragma unroll
      for (int j = 0; j < DP; ++j) issue_w(nb0, nq, j, [&](int e) { return ul_s[e]; });
#pragma unroll
    for (int j = 0; j < DP; ++j) issue_x(j, xa[j]);
    f32x16_t ag[TB], au[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int q = 0; q < 16; ++q) ag[tb][q] = au[tb][q] = 0.0f;
    const uint32_t rg = (uint32_t)nn * 128, ru = (uint32_t)(nq + nn) * 128;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      dec_u32x4(&xj)[TB][4] = xa[j % DP];
#pragma unroll
      for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i) decb_ready(xj[tb][i]);  // block j's x and (issued before) its rows
      const unsigned char* slot = ring + (j % DP) * DECB_STAGE;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t pos = 16u * (uint32_t)((i + 4 * kh) ^ (nn & 7));
        const uint4 bg = *(const uint4*)(slot + rg + pos);
        const uint4 bu = *(const uint4*)(slot + ru + pos);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
          ag[tb] = mfma32x(xj[tb][i], bg, ag[tb]);
          au[tb] = mfma32x(xj[tb][i], bu, au[tb]);
        }
      }
      if (j + DP < CPL) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this stage's LDS reads are done
        issue_w(nb0, nq, j + DP, [&](int e) { return ul_s[e]; });
        issue_x(j + DP, xa[j % DP]);
      }
    }
    wg_lds_barrier();  // every wave is done with its ring: the partials may be written
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        red_s[((tb * NW + wv) * 2) * 1024 + q * 64 + lane] = ag[tb][q];
        red_s[((tb * NW + wv) * 2 + 1) * 1024 + q * 64 + lane] = au[tb][q];
      }
    wg_lds_barrier();
    // entry v = (tb, q, l): token tb * 32 + mfma32_row(q, l), neuron nb0 + l % 32; the
    // eight K partials added in wave order, then act = silu(g) * u * gate as bf16
    for (int v = tid; v < TB * 1024; v += NT) {
      const int tb = v >> 10, q = (v >> 6) & 15, l = v & 63;
      const int t = tb * 32 + mfma32_row(q, l), n = l & 31;
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        g += red_s[((tb * NW + w) * 2) * 1024 + q * 64 + l];
        u += red_s[((tb * NW + w) * 2 + 1) * 1024 + q * 64 + l];
      }
      if (t < N && n < nq) {
        const float gt = sg_s[t * 16 + ul_s[(nb0 + n) / G]];
        const float a = fail ? __int_as_float(0x7fc00000) : gt != -1.0f ? pp_silu(g) * u * gt : 0.0f;
        act_s[t * 32 + n] = f32_to_bf16(a);
      }
    }
    wg_lds_barrier();
    // published in fragment order (16 B = 8 neurons of one token) by wave 0 alone, whose
    // store counter then covers every act store of the workgroup
    const int ng = nq / 8;
    if (wv == 0)
      for (int it = lane; it < N * ng; it += 64) {
        const int t = it / ng, gi = it - t * ng;
        const int k = nb0 + 8 * gi;  // union neuron of the group (a multiple of 8)
        decb_st16(r_af, decb_frag(k >> 4, t >> 5, (t & 31) + 32 * ((k >> 3) & 1)),
                  *(const uint4*)(act_s + t * 32 + 8 * gi));
      }
    wg_lds_barrier();  // the acts are read out (and their stores issued): the rings may be refilled
  }
  if (wv == 0) {
    vm_wait();  // the act stores
    if (lane == 0) st_rlx(&aflag[b], tag);
    dma_rows(hr0, min(rows_pp, hr1 - hr0), 7, 8);
  } else {  // the first pass's down rows (LDS is free), behind the act stores
    dma_rows(hr0, min(rows_pp, hr1 - hr0), wv - 1, NW);
  }

  // ---- D: partial sums of rows [hr0, hr1) over slice s
  {
    // the acts of [a0, a0 + nk) come from the workgroups whose [q0, q1) meet it
    for (int p = tid; p < W; p += NT) {
      int lo, hi;
      pp_split((uint32_t)(T / 8), (uint32_t)W, (uint32_t)p, lo, hi);
      if (lo < hi && 8 * lo < a0 + nk && 8 * hi > a0 && !decb_wait(&aflag[p], tag)) fail = true;
    }
    vm_wait();  // the first pass's down rows
    fail = __syncthreads_or(fail);
    const int nks = nk / 16;
    for (int p0 = hr0; p0 < hr1; p0 += rows_pp) {
      const int nr = min(rows_pp, hr1 - p0);
      if (p0 != hr0) {  // later passes (row groups beyond rows_pp rows)
        wg_lds_barrier();
        dma_rows(p0, nr, wv, NW);
        vm_wait();
        __syncthreads();
      }
      const int nrb = (nr + 31) >> 5;
      for (int tile = wv; tile < nrb * TB; tile += NW) {
        const int rbk = tile / TB, tb = tile - rbk * TB;
        const int rho = min(rbk * 32 + jn, nr - 1);  // A row: down row of the pass
        const unsigned char* arow = dn_s + rho * RSB + 16 * kh;
        // every act fragment of the tile requested at once (nk <= G <= DEC2_GMAX)
        uint4 bv[DEC2_GMAX / 16];
#pragma unroll
        for (int ks = 0; ks < DEC2_GMAX / 16; ++ks)
          if (ks < nks) bv[ks] = decb_ld16<DECB_SC1>(r_af, decb_frag(a0 / 16 + ks, tb, lane));
        f32x16_t acc;
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < DEC2_GMAX / 16; ++ks)
          if (ks < nks) acc = mfma32(*(const uint4*)(arow + 32 * ks), bv[ks], acc);
        // D: lane l, element q -> row rbk * 32 + mfma32_row(q, l), token tb * 32 + l % 32
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int rr = rbk * 32 + mfma32_row(q, lane);
          if (rr < nr && tb * 32 + jn < N)  // the padding tokens' sums are never read
            __builtin_amdgcn_raw_buffer_store_b32(fail ? 0x7fc00000u : __float_as_uint(acc[q]), r_part,
                                                  (uint32_t)(((s * H + p0 + rr) * DECB_MAXN + tb * 32 + jn) * 4), 0,
                                                  DECB_SC1);
        }
      }
    }
    vm_wait();
    __syncthreads();
    if (tid == 0) st_rlx(&pflag[b], tag);
  }

  // ---- E: fold of the 8-row blocks u = b, b + W, ... over the 16 slices, in slice order
  for (int u = b; u < H / 8; u += W) {
    int rg = 0;  // the row group holding block u
    for (int i = 0; i < R; ++i) {
      int lo, hi;
      pp_split((uint32_t)(H / 8), (uint32_t)R, (uint32_t)i, lo, hi);
      if (u >= lo && u < hi) rg = i;
    }
    if (tid < DECB_S && !decb_wait(&pflag[rg * DECB_S + tid], tag)) fail = true;
    const bool failed = __syncthreads_or(fail);
    const int t = tid >> 3, hh = tid & 7;
    if (t < N) {
      float acc = 0.0f;
#pragma unroll
      for (int sl = 0; sl < DECB_S; ++sl)
        acc += __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            r_part, (uint32_t)(((sl * H + 8 * u + hh) * DECB_MAXN + t) * 4), 0, DECB_SC1));
      out[(size_t)t * H + 8 * u + hh] = failed ? (bf16_t)0x7fc0 : f32_to_bf16(acc);
    }
  }

  if (b == 0)  // once every workgroup has set its last flag (so has read the tag), advance
    for (int p = tid; p < W; p += NT)
      if (!decb_wait(&pflag[p], tag)) fail = true;
  const bool failed = __syncthreads_or(fail);
  if (tid == 0) {
    if (failed) {
      __hip_atomic_fetch_or(&st->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      st_rlx(&st->error_call, tag);
    }
    if (b == 0) st_rlx(&st->epochb, tag);
  }
}

// Zeroes a workspace of n_words words, then its state header holds `layout` and `error`.
__global__ void decode_ws_clear_kernel(uint32_t* p, size_t n_words, uint32_t layout, uint32_t error) {
  constexpr size_t kLayout = offsetof(pp_decode_state, layout) / 4, kError = offsetof(pp_decode_state, error) / 4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = i == kLayout ? layout : i == kError ? error : 0u;
}

// Workspace: state | decode_kernel: 2 x DEC_NCOPY x hs fixed-point accumulators,
// DEC_SLOT_REPS x PP_MAX_EXPERTS 64-bit logit slots, completion-ticket counters | the
// two-phase kernels: two act banks of DEC2_BANK_WORDS words | the batch kernel: its tagged
// gates and flags. The kernel families keep separate epochs (router_ticket, epoch16,
// epochb), so calls of any kind may follow each other on one workspace.
static constexpr size_t dec_general_bytes(int hs) {
  return (size_t)2 * DEC_NCOPY * hs * sizeof(dec_acc_t) + (size_t)DEC_SLOT_REPS * PP_MAX_EXPERTS * sizeof(unsigned long long) +
         (size_t)DEC_TICKET_WORDS * sizeof(uint32_t);
}
static constexpr size_t dec_banks_offset(int hs) { return (dec_acc_offset() + dec_general_bytes(hs) + 255) / 256 * 256; }
static constexpr size_t dec_banks_bytes() { return (size_t)2 * DEC2_BANK_WORDS * sizeof(uint32_t); }

// the batch kernel's tagged state follows the banks (the allocation-free scratch stops before it)
static constexpr size_t dec_bflags_offset(int hs) { return dec_banks_offset(hs) + dec_banks_bytes(); }

extern "C" size_t pp_decode_workspace_bytes(int H, int E) {
  (void)E;
  return dec_bflags_offset(H) + (size_t)DECB_STATE_BYTES;
}

extern "C" int pp_decode_workspace_init(void* workspace, int H, int E, void* stream) {
  int rc = pp_check_shape(H, E, 32);
  if (rc) return rc;
  PP_REQUIRE(workspace, PP_ERR_INVALID, "pp_decode_workspace_init: null workspace");
  size_t words = pp_decode_workspace_bytes(H, E) / 4;
  decode_ws_clear_kernel<<<64, 256, 0, (hipStream_t)stream>>>((uint32_t*)workspace, words, dec_layout_tag(H), 0u);
  return pp_check_launch("pp_decode_workspace_init");
}

extern "C" uint32_t pp_decode_layout_tag(int H) {
  if (H < 128 || H > 4096 || H % 128 != 0) return 0u;  // the shape limits of every entry point
  return dec_layout_tag(H);
}

extern "C" int pp_decode_state_check(const pp_decode_state* state, int H) {
  PP_REQUIRE(state != nullptr, PP_ERR_INVALID, "pp_decode_state_check: null state");
  const uint32_t want = pp_decode_layout_tag(H);
  PP_REQUIRE(want != 0u, PP_ERR_INVALID, "pp_decode_state_check: H=%d outside the shape limits", H);
  PP_REQUIRE(state->layout == want, PP_ERR_INVALID,
             "pp_decode_state_check: workspace layout tag 0x%08x, this library expects 0x%08x for H=%d (a "
             "workspace initialised by another build or for another H, or never initialised)",
             state->layout, want, H);
  return PP_OK;
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
                         pp_decode_state* st, dec_acc_t* acc, int hs, int hclear, uint32_t layout) {
#define PP_DEC_CASE(C)                                                                                  \
  case C: {                                                                                             \
    const size_t sm = (size_t)DecNW<C>::NW * H * sizeof(float);                                         \
    if (!LOCAL) {                                                                                       \
      const int rc = dec_check_coresident((const void*)decode_kernel<XT, C, LOCAL>, DecNW<C>::NT, sm, E); \
      if (rc) return rc;                                                                                \
    }                                                                                                   \
    decode_kernel<XT, C, LOCAL><<<grid, DecNW<C>::NT, sm, s>>>(x, H, router, bias, E, G, tau, rows, out, st, acc, \
                                                               hs, hclear, layout);                      \
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

// Default grid of the E = 16 two-phase kernel: one workgroup per CU. The record stream
// and the row sums gain from every CU: at H = 1536 on 256 CUs, 256 workgroups of 6 rows
// take 10.65 us against 11.04 us with 192 of 8 rows (224: 10.71; 232-248, rows 6 and 7
// mixed: 10.76-10.87; 176, two row passes: 12.2); at H = 512, 1024, 2048, 3072 and 4096
// 256 workgroups are as fast as any smaller default (within 0.02 us). (With the dry
// phase-2 pass on wave 0, which issues the down-row DMAs, 192 had been faster than 256.)
static int dec2_default_grid(int H) {
  (void)H;
  return std::max(8, pp_device_cus());
}

// The launch shared by both entry points: st / acc = the state and the accumulators of
// the workspace in use, hs = the stride of one accumulator copy, hclear = how much of
// each copy of the previous call's set to clear.
static int decode_dispatch(const void* x, int x_dtype, int H, const float* router_packed, const float* bias,
                           int E, int G, float tau, const void* packed, void* out_bf16, pp_decode_state* st,
                           dec_acc_t* acc, int hs, int hclear, uint32_t* banks, int grid, hipStream_t s) {
  const int grid_in = grid;
  const uint32_t layout = dec_layout_tag(hs);  // the workspace's tag its kernels expect
  if (grid == 0) grid = pp_device_cus();
  if (grid < E) grid = E;  // every expert has its router workgroup
  const int cpl = (H / 8 + 63) / 64;  // 16-byte chunks per lane per row (H <= 4096 -> <= 8)
  if (E == 16 && H % 512 == 0 && G <= DEC2_GMAX) {
    // the two-phase kernel: every workgroup waits for acts from all the others, so the
    // grid is clamped to what the device holds at once (and to DEC2_WMAX); rows of the
    // output per workgroup are handled rp at a time, their down rows staged in LDS
    PP_REQUIRE(banks != nullptr, PP_ERR_INVALID, "pp_moe_decode: workspace without the E = 16 act banks");
    int W = min(grid_in == 0 ? dec2_default_grid(H) : grid_in, DEC2_WMAX);
    const int nh = (H + W - 1) / W;
    const int rp = max(1, min(min(8, nh), DEC2_DOWN_LDS / (16 * G * 2)));
    const int slot_bytes = (rp * G * 2 + 1023) / 1024 * 1024;
    const size_t smem = (size_t)16 * slot_bytes;
    const bf16_t* gu = (const bf16_t*)packed;
    const bf16_t* down_t = gu + (size_t)16 * G * 3 * H;
#define PP_DEC16_CASE(C)                                                                                        \
  case C: {                                                                                                     \
    const void* kf = x_dtype == PP_DTYPE_F32 ? (const void*)decode16_kernel<float, C>                          \
                                             : (const void*)decode16_kernel<bf16_t, C>;                         \
    const int cap = dec_capacity(kf, 512, smem);                                                               \
    PP_REQUIRE(cap >= 1, PP_ERR_UNSUPPORTED, "pp_moe_decode: the E = 16 kernel does not fit the device");     \
    W = min(W, cap);                                                                                            \
    if (x_dtype == PP_DTYPE_F32)                                                                                \
      decode16_kernel<float, C><<<W, 512, smem, s>>>((const float*)x, router_packed, bias, G, tau, gu, 3, down_t,  \
                                                     (bf16_t*)out_bf16, st, banks, rp, slot_bytes, layout);    \
    else                                                                                                        \
      decode16_kernel<bf16_t, C><<<W, 512, smem, s>>>((const bf16_t*)x, router_packed, bias, G, tau, gu, 3, down_t, \
                                                      (bf16_t*)out_bf16, st, banks, rp, slot_bytes, layout);   \
  } break;
    switch (H / 512) {
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
  if (E * G <= DEC2_RS && G <= DEC2_GMAX) {
    // two phases, routing as decode_kernel (every workgroup routes for small routers up to
    // H = 1536, where the router rows fit the registers); every workgroup waits for the
    // others' acts (and, with published logits, for the E router workgroups), so the grid
    // is at least E and at most what the device holds at once
    PP_REQUIRE(banks != nullptr, PP_ERR_INVALID, "pp_moe_decode: workspace without the act banks");
    int W = max(min(grid_in == 0 ? pp_device_cus() : grid_in, DEC2_WMAX), E);
    const int nh = (H + W - 1) / W;
    // rows per pass: the largest rp <= 8 whose LDS (E ranks x (rp rows x G / 8 chunks + one
    // pad chunk), rounded up to whole DMA instructions) fits DEC2_DOWN_LDS
    int rp = min(8, nh);
    while (rp > 1 && (size_t)((E * (rp * (G / 8) + 1) + 63) / 64 * 64) * 16 > DEC2_DOWN_LDS) --rp;
    const size_t smem = (size_t)((E * (rp * (G / 8) + 1) + 63) / 64 * 64) * 16;
    const bf16_t* gu = (const bf16_t*)packed;
    const bf16_t* down_t = gu + (size_t)E * G * 3 * H;
    bf16_t* o = (bf16_t*)out_bf16;
    int rc = PP_OK;
    auto launch = [&](auto kern, auto xp) {
      const int cap = dec_capacity((const void*)kern, 512, smem);
      W = min(W, cap);
      if (W < E || W < 1) {
        pp_set_error("pp_moe_decode: the device holds %d decode workgroups at once, fewer than the %d experts' "
                     "router workgroups", cap, E);
        rc = PP_ERR_UNSUPPORTED;
        return;
      }
      kern<<<W, 512, smem, s>>>(xp, H, router_packed, bias, E, G, tau, gu, down_t, o, st, banks, rp, layout);
    };
#define PP_DEC2P_CASE(C)                                                                                           \
  case C:                                                                                                          \
    if (x_dtype == PP_DTYPE_F32) {                                                                                 \
      if (local && C <= 3) launch(decode2p_kernel<float, (C <= 3 ? C : 3), true>, (const float*)x);                \
      else launch(decode2p_kernel<float, C, false>, (const float*)x);                                              \
    } else {                                                                                                       \
      if (local && C <= 3) launch(decode2p_kernel<bf16_t, (C <= 3 ? C : 3), true>, (const bf16_t*)x);              \
      else launch(decode2p_kernel<bf16_t, C, false>, (const bf16_t*)x);                                            \
    }                                                                                                              \
    break;
    switch (cpl) {
      PP_DEC2P_CASE(1)
      PP_DEC2P_CASE(2)
      PP_DEC2P_CASE(3)
      PP_DEC2P_CASE(4)
      PP_DEC2P_CASE(5)
      PP_DEC2P_CASE(6)
      PP_DEC2P_CASE(7)
      PP_DEC2P_CASE(8)
    }
#undef PP_DEC2P_CASE
    if (rc) return rc;
    return pp_check_launch("pp_moe_decode");
  }
  const bf16_t* rows = (const bf16_t*)packed;
  bf16_t* o = (bf16_t*)out_bf16;
  int rc;
  if (x_dtype == PP_DTYPE_F32) {
    if (local) rc = launch_decode<float, true>(cpl, grid, s, (const float*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear, layout);
    else rc = launch_decode<float, false>(cpl, grid, s, (const float*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear, layout);
  } else {
    if (local) rc = launch_decode<bf16_t, true>(cpl, grid, s, (const bf16_t*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear, layout);
    else rc = launch_decode<bf16_t, false>(cpl, grid, s, (const bf16_t*)x, H, router_packed, bias, E, G, tau, rows, o, st, acc, hs, hclear, layout);
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
  uint32_t* banks = (uint32_t*)((char*)workspace + dec_banks_offset(H));
  return decode_dispatch(x, x_dtype, H, router_packed, bias, E, G, tau, packed, out_bf16, st, acc, H, H, banks, grid,
                         (hipStream_t)stream);
}

// ------------------------------------------------------------------ batch entry
extern "C" size_t pp_decode_batch_workspace_bytes(int H, int E, int G) {
  (void)E;
  return decb_layout(H, G).total;
}

extern "C" int pp_moe_decode_batch(const void* x, int x_dtype, int64_t n_tokens, int H, const float* router_packed,
                                   const float* bias, int E, int G, float tau, const void* packed, void* out_bf16,
                                   float* logits_out, uint8_t* mask_out, void* workspace, void* batch_workspace,
                                   int grid, void* stream) {
  int rc = decode_check_args(x, x_dtype, H, router_packed, E, G, packed, out_bf16, grid);
  if (rc) return rc;
  PP_REQUIRE(workspace && batch_workspace, PP_ERR_INVALID, "pp_moe_decode_batch: null workspace");
  PP_REQUIRE(n_tokens >= 1 && n_tokens <= DECB_MAXN, PP_ERR_UNSUPPORTED,
             "pp_moe_decode_batch: n_tokens %lld unsupported (1..%d)", (long long)n_tokens, DECB_MAXN);
  PP_REQUIRE(E == 16 && H % 512 == 0 && G <= DEC2_GMAX, PP_ERR_UNSUPPORTED,
             "pp_moe_decode_batch: H=%d E=%d G=%d unsupported (E = 16, H %% 512 == 0, G <= %d)", H, E, G, DEC2_GMAX);
  const int N = (int)n_tokens;
  hipStream_t s = (hipStream_t)stream;
  pp_decode_state* st = (pp_decode_state*)workspace;
  unsigned char* bstate = (unsigned char*)workspace + dec_bflags_offset(H);
  const bf16_t* gu = (const bf16_t*)packed;
  const bf16_t* down_t = gu + (size_t)16 * G * 3 * H;
  // W: a multiple of DECB_S, at least N, at most what the device holds at once (every
  // workgroup waits for others); rows per pass: a row group's rows as far as LDS allows
  int W = min(grid == 0 ? pp_device_cus() : grid, DEC2_WMAX) / DECB_S * DECB_S;
  const int R0 = max(W / DECB_S, 1);
  int rp = 8 * ((H / 8 + R0 - 1) / R0);
  auto lds_rows = [&](int rows) { return (size_t)((rows * (G / 8 + 1) + 63) / 64 * 64) * 16; };
  while (rp > 1 && lds_rows(rp) > DECB_DOWN_LDS) --rp;
  const size_t smem = DECB_SMEM;
  auto launch = [&](auto kern, auto xp) {
    const int cap = dec_capacity((const void*)kern, 512, smem);
    W = min(W, cap) / DECB_S * DECB_S;
    if (W < max(N, DECB_S)) {
      pp_set_error("pp_moe_decode_batch: %d workgroups resident at once, the batch kernel needs %d", W,
                   max(N, DECB_S));
      rc = PP_ERR_UNSUPPORTED;
      return;
    }
    kern<<<W, 512, smem, s>>>(xp, N, router_packed, bias, G, tau, gu, down_t, (bf16_t*)out_bf16, logits_out, mask_out,
                              st, bstate, (unsigned char*)batch_workspace, rp, dec_layout_tag(H));
  };
#define PP_DECB_CASE(C)                                                                      \
  case C:                                                                                    \
    if (x_dtype == PP_DTYPE_F32) {                                                           \
      if (N <= 32) launch(decodeb_kernel<float, C, 1>, (const float*)x);                     \
      else launch(decodeb_kernel<float, C, 2>, (const float*)x);                             \
    } else {                                                                                 \
      if (N <= 32) launch(decodeb_kernel<bf16_t, C, 1>, (const bf16_t*)x);                   \
      else launch(decodeb_kernel<bf16_t, C, 2>, (const bf16_t*)x);                           \
    }                                                                                        \
    break;
  switch (H / 512) {
    PP_DECB_CASE(1)
    PP_DECB_CASE(2)
    PP_DECB_CASE(3)
    PP_DECB_CASE(4)
    PP_DECB_CASE(5)
    PP_DECB_CASE(6)
    PP_DECB_CASE(7)
    PP_DECB_CASE(8)
  }
#undef PP_DECB_CASE
  if (rc) return rc;
  return pp_check_launch("pp_moe_decode_batch");
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
static constexpr size_t kDecScratchBytes = dec_banks_offset(PP_DECODE_SCRATCH_HS) + dec_banks_bytes();
static_assert(kDecScratchBytes == 609792, "decode scratch: 596 KB per GPU (state, int64 accumulators at stride 4096, "
                                          "slot replicas, ticket counters, the two-phase kernels' act banks)");
static __device__ __align__(256) unsigned char scratch[kDecScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

// The scratch is zeroed (and tagged) by a fill kernel on the caller's stream, ordered before
// the caller's later work on it: at the first call on a device and at every reset. Never
// while `s` is capturing: a captured fill would re-run at every replay of the graph, and a
// graph replayed between eager calls would clear their error state.
static int decode_scratch_not_capturing(hipStream_t s, const char* who) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(s, &cs);
  PP_REQUIRE(e == hipSuccess, PP_ERR_HIP, "%s: hipStreamIsCapturing: %s", who, hipGetErrorString(e));
  PP_REQUIRE(cs == hipStreamCaptureStatusNone, PP_ERR_INVALID,
             "%s: the stream is capturing; the allocation-free decode scratch is initialised and reset by eager "
             "calls only (make one pp_moe_decode_noalloc or pp_decode_noalloc_reset call before capturing)", who);
  return PP_OK;
}
static int decode_scratch_fill(hipStream_t s, void* ptr, uint32_t error, const char* who) {
  const int rc = decode_scratch_not_capturing(s, who);
  if (rc) return rc;
  decode_ws_clear_kernel<<<64, 256, 0, s>>>((uint32_t*)ptr, kDecScratchBytes / 4,
                                            dec_layout_tag(PP_DECODE_SCRATCH_HS), error);
  return pp_check_launch(who);
}

// Device address of this device's scratch (hipGetSymbolAddress once per device, with
// that device current); `init` is set when this call initialised it.
static int decode_scratch(hipStream_t s, void** out, bool* init) {
  int dev = 0;
  PP_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, PP_ERR_HIP,
             "pp_moe_decode_noalloc: no current device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  *init = false;
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    PP_REQUIRE(e == hipSuccess && ptr != nullptr, PP_ERR_HIP, "pp_moe_decode_noalloc: hipGetSymbolAddress: %s",
               hipGetErrorString(e));
    const int rc = decode_scratch_fill(s, ptr, 0u, "pp_moe_decode_noalloc (scratch init)");
    if (rc) return rc;
    g_scratch_ptr[dev] = ptr;
    *init = true;
  }
  *out = g_scratch_ptr[dev];
  return PP_OK;
}

extern "C" int pp_decode_noalloc_reset(uint32_t* error_out, uint32_t error_in, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  int rc = decode_scratch_not_capturing(s, "pp_decode_noalloc_reset");  // before any copy or launch
  if (rc) return rc;
  void* ptr = nullptr;
  bool init = false;
  rc = decode_scratch(s, &ptr, &init);
  if (rc) return rc;
  if (error_out != nullptr) {  // the state before this reset (zero when this call initialised it)
    uint32_t v = 0u;
    if (!init) {
      hipError_t e = hipMemcpyAsync(&v, (char*)ptr + offsetof(pp_decode_state, error), sizeof(v),
                                    hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
      PP_REQUIRE(e == hipSuccess, PP_ERR_HIP, "pp_decode_noalloc_reset: reading the error bits: %s",
                 hipGetErrorString(e));
    }
    *error_out = v;
  }
  if (init && error_in == 0u) return PP_OK;
  return decode_scratch_fill(s, ptr, error_in, "pp_decode_noalloc_reset");
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
  bool init = false;
  rc = decode_scratch(s, &ptr, &init);
  if (rc) return rc;
  pp_decode_state* st = (pp_decode_state*)ptr;
  dec_acc_t* acc = (dec_acc_t*)((char*)ptr + dec_acc_offset());
  uint32_t* banks = (uint32_t*)((char*)ptr + dec_banks_offset(PP_DECODE_SCRATCH_HS));
  return decode_dispatch(x, x_dtype, H, router_packed, bias, E, G, tau, packed, out_bf16, st, acc,
                         PP_DECODE_SCRATCH_HS, PP_DECODE_SCRATCH_HS, banks, grid, s);
}
