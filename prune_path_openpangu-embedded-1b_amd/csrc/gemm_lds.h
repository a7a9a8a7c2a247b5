// LDS-DMA MFMA helpers and the persistent item schedule shared by the pipelined
// GEMMs (grouped: prefill.hip; dense: dense.hip).
#pragma once
#include "pp_common.h"

typedef __attribute__((address_space(3))) void lds_void_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void gl2lds(const void* src, unsigned char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, 0);
}

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

// 16-byte LDS read at a byte address, invisible to the compiler's memory model: it cannot
// be ordered after (made to wait for) LDS-DMA writes the compiler sees as aliasing stores.
// The caller orders it with its own waits (s_waitcnt vmcnt + s_barrier before, lds_wait_all
// after).
__device__ __forceinline__ u32x4 lds_read16(uint32_t lds_addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_addr));
  return v;
}
template <typename T>
__device__ __forceinline__ void lds_tie(T& v) {
  asm volatile("" : "+v"(v));
}
// Every LDS read of this wave has returned; the values v... are used only after this point.
template <typename... T>
__device__ __forceinline__ void lds_wait_all(T&... v) {
  asm volatile("s_waitcnt lgkmcnt(0)");
  (lds_tie(v), ...);
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


__device__ __forceinline__ void gl2lds4(const void* src, unsigned char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 4, 0, 0);
}

template <int N>
__device__ __forceinline__ void gp_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// ---- split items: the K blocks of an item shared by several workgroups
// Schedule of both pipelined GEMMs (GpSched): rank q = XCD-major workgroup index (an
// XCD's ranks are consecutive); full rounds of whole items first -- item r * grid + q in
// round r, so the workgroups sharing a row tile or an expert's weights walk K in step --
// then, with a split workspace, the tail items (n_items % grid) each cut into nparts K
// ranges, one range per workgroup; the workgroups holding the parts of a tail item join
// their fp32 partial sums (gp_join). Without a workspace: whole items, grid-strided.
// Split workspace: sync words [0] (reserved), [1, 1 + grid) tickets (one per tail item),
// then partial-sum slots of NF floats per thread, one slot per part (at most grid). The
// tickets are zero at launch and every launch leaves them zero.
#define GP_MIN_PART_BLOCKS 4  // a part shorter than this does not repay its join (measured)
__device__ __forceinline__ void gp_st(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GpSched {
  int n_whole;       // whole local items
  int first, step;   // whole local item li is first + li * step
  int part_item;     // the tail item of this workgroup's part (-1: none)
  int kb_lo, kb_hi;  // its K blocks
  int unit, nparts;  // part index = unit % nparts
  int tail0;         // first tail item
  __device__ GpSched(int n_items, int nkb, bool can_split, int max_parts = 1 << 30) {
    const int g = gridDim.x, per = g >> 3;
    const int rank = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    const int rounds = n_items / g, tail = n_items - rounds * g;
    nparts = (can_split && tail > 0) ? max(1, min(min(nkb / GP_MIN_PART_BLOCKS, g / tail), max_parts)) : 1;
    part_item = -1;
    kb_lo = kb_hi = 0;
    unit = rank;
    tail0 = rounds * g;
    if (nparts > 1) {
      n_whole = rounds;
      first = rank;
      step = g;
      if (rank < tail * nparts) {
        const int ti = rank / nparts, pi = rank - ti * nparts;
        part_item = tail0 + ti;
        kb_lo = pi * nkb / nparts;
        kb_hi = (pi + 1) * nkb / nparts;
      }
    } else {
      const GvItems it(n_items);
      n_whole = it.first < it.last ? (it.last - it.first + it.step - 1) / it.step : 0;
      first = it.first;
      step = it.step;
    }
  }
  __device__ int n_local() const { return n_whole + (part_item >= 0 ? 1 : 0); }
  __device__ int item(int li) const { return li < n_whole ? first + li * step : part_item; }
  __device__ int units(int nkb) const { return n_whole * nkb + (kb_hi - kb_lo); }
  // local unit f -> (local item, K block)
  __device__ void locate(int f, int nkb, int& li, int& kb) const {
    if (f < n_whole * nkb) {
      li = f / nkb;
      kb = f - li * nkb;
    } else {
      li = n_whole;
      kb = kb_lo + (f - n_whole * nkb);
    }
  }
};

