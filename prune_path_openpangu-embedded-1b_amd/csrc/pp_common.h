// Shared device helpers for the PrunePath MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/prunepath_moe.h"

#define PP_WAVE 64

typedef uint16_t bf16_t;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

// ---------------------------------------------------------------- errors (host)
void pp_set_error(const char* fmt, ...);
int pp_check_launch(const char* what);

#define PP_REQUIRE(cond, code, ...)          \
  do {                                       \
    if (!(cond)) {                           \
      pp_set_error(__VA_ARGS__);             \
      return (code);                         \
    }                                        \
  } while (0)

// Shape limits shared by every entry point.
static inline int pp_check_shape(int H, int E, int G) {
  PP_REQUIRE(H >= 128 && H <= 4096 && H % 128 == 0, PP_ERR_UNSUPPORTED,
             "hidden size H=%d unsupported (need 128 <= H <= 4096, H %% 128 == 0)", H);
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "num_experts E=%d unsupported (1..256)", E);
  PP_REQUIRE(G >= 32 && G % 32 == 0 && G <= 8192, PP_ERR_UNSUPPORTED,
             "group size G=%d unsupported (need G %% 32 == 0, 32 <= G <= 8192)", G);
  return PP_OK;
}

int pp_device_cus();

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// Round to nearest even, NaN kept quiet (the rounding torch uses for .to(bfloat16)):
// one v_cvt_pk_bf16_f32. The software form (add 0x7fff + lsb, NaN branch) costs ~10
// instructions and a branch per value, which matters in kernels whose executed code
// size is part of their latency.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

// v_mfma_f32_32x32x16_bf16: A lane l holds row l % 32, k = 8 (l / 32) .. + 7; B lane l
// holds column l % 32, the same k; D lane l, element q is row mfma32_row(q, l), column l % 32.
__device__ __forceinline__ f32x16_t mfma32(const uint4 a, const uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
__device__ __forceinline__ int mfma32_row(int q, int lane) { return (q >> 2) * 8 + (lane >> 5) * 4 + (q & 3); }

__host__ __device__ __forceinline__ int pp_ceil_div(int a, int b) { return (a + b - 1) / b; }

// Balanced contiguous split of [0, T) into W parts: part b is [lo, hi). One 32-bit
// division of uniform values (a 64-bit T * b / W costs ~130 instructions per use).
__device__ __forceinline__ void pp_split(uint32_t T, uint32_t W, uint32_t b, int& lo, int& hi) {
  const uint32_t q = T / W, rem = T - q * W;
  lo = (int)(b * q + (b < rem ? b : rem));
  hi = lo + (int)q + (b < rem ? 1 : 0);
}

// Load one input element as fp32 (input dtype: fp32 or bf16).
template <typename XT>
__device__ __forceinline__ float load_as_f32(const XT* p, int64_t i);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_as_f32<bf16_t>(const bf16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}

// DPP lane moves inside 16-lane rows: a VALU operand modifier, no LDS round trip
// (__shfl_xor is a ds_bpermute, about a hundred cycles each).
#define PP_DPP_XOR1 0xB1   // quad_perm [1,0,3,2]: lane i^1
#define PP_DPP_XOR2 0x4E   // quad_perm [2,3,0,1]: lane i^2
#define PP_DPP_ROR4 0x124  // row_ror:4: the row rotated by 4 lanes (used where direction does not matter)
#define PP_DPP_ROR8 0x128  // row_ror:8: the row rotated by 8 lanes = lane i^8
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum over each 16-lane row, pairing i^8, i^4, i^2, i^1: bit-identical to four
// __shfl_xor butterfly steps, and every lane of the row ends with the same bits. After
// the i^8 step the row is 8-periodic (IEEE addition commutes), so lane (i+4) mod 16
// holds the value of lane i^4.
__device__ __forceinline__ float row16_sum(float v) {
  v = __fadd_rn(v, dpp_mov<PP_DPP_ROR8>(v));
  v = __fadd_rn(v, dpp_mov<PP_DPP_ROR4>(v));
  v = __fadd_rn(v, dpp_mov<PP_DPP_XOR2>(v));
  return __fadd_rn(v, dpp_mov<PP_DPP_XOR1>(v));
}
// Sum over each 8-lane half row (quad steps, then the mirrored quad); a fixed order,
// the same in every lane group, not the xor butterfly.
#define PP_DPP_HALF_MIRROR 0x141  // row_half_mirror: lane 7 - i of the half row
__device__ __forceinline__ float row8_sum(float v) {
  v = __fadd_rn(v, dpp_mov<PP_DPP_XOR1>(v));
  v = __fadd_rn(v, dpp_mov<PP_DPP_XOR2>(v));
  return __fadd_rn(v, dpp_mov<PP_DPP_HALF_MIRROR>(v));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<PP_DPP_ROR8>(v));
  v = fmaxf(v, dpp_mov<PP_DPP_ROR4>(v));
  v = fmaxf(v, dpp_mov<PP_DPP_XOR2>(v));
  return fmaxf(v, dpp_mov<PP_DPP_XOR1>(v));
}
// The value of lane l ^ 16 (l ^ 32) without an LDS round trip: v_permlane16_swap
// (v_permlane32_swap) of a register with itself swaps its odd and even 16-lane rows (its
// upper and lower halves) between the two results; a lane takes the result holding its
// partner's row (lane layout checked on the device).
__device__ __forceinline__ uint32_t pl_xor16(uint32_t v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return ((lane >> 4) & 1) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t pl_xor32(uint32_t v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return lane >= 32 ? r[0] : r[1];
}
__device__ __forceinline__ float pl_xor16f(float v, int lane) {
  return __uint_as_float(pl_xor16(__float_as_uint(v), lane));
}
__device__ __forceinline__ float pl_xor32f(float v, int lane) {
  return __uint_as_float(pl_xor32(__float_as_uint(v), lane));
}
__device__ __forceinline__ double pl_xor16d(double v, int lane) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  return __longlong_as_double(
      (long long)(((unsigned long long)pl_xor16((uint32_t)(u >> 32), lane) << 32) | pl_xor16((uint32_t)u, lane)));
}
__device__ __forceinline__ double pl_xor32d(double v, int lane) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  return __longlong_as_double(
      (long long)(((unsigned long long)pl_xor32((uint32_t)(u >> 32), lane) << 32) | pl_xor32((uint32_t)u, lane)));
}

// ---------------------------------------------------------------- wave reductions
// The xor butterfly over 32, 16, 8, 4, 2, 1 (the same pairs and order, so the same bits):
// the two cross-row steps by permlane swaps, the row steps by DPP.
__device__ __forceinline__ float wave_sum(float v) {
  const int lane = (int)__lane_id();
  v += pl_xor32f(v, lane);
  v += pl_xor16f(v, lane);
  return row16_sum(v);
}
__device__ __forceinline__ float wave_max(float v) {
  const int lane = (int)__lane_id();
  v = fmaxf(v, pl_xor32f(v, lane));
  v = fmaxf(v, pl_xor16f(v, lane));
  return row16_max(v);
}
// Whole-wave maximum (rows by DPP, then the four row maxima read as scalars); fmaxf is
// order-free, so the value equals wave_max's. Wave-uniform.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = row16_max(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
// quad_perm [3,2,1,0] (lane 3 - i of the quad) followed by row_half_mirror (lane 7 - i
// of the half row) reads lane i ^ 4: both are fixed involutions, with no rotation
// direction to get wrong.
#define PP_DPP_QREV 0x1B
// Inclusive prefix sum of doubles over the 64 lanes in lane order: row_shr:1, 2, 4, 8
// (lane i reads lane i - n of its row; lanes with no source read the identity 0), then
// row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3 -- the gfx9 wave
// scan of LLVM's AMDGPU atomic optimizer. The order of the additions differs from a
// sequential sum, so callers use it where every partial sum is exact.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long u = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf, false);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
  v += dpp_f64<0x111, 0xf>(v);
  v += dpp_f64<0x112, 0xf>(v);
  v += dpp_f64<0x114, 0xf>(v);
  v += dpp_f64<0x118, 0xf>(v);
  v += dpp_f64<0x142, 0xa>(v);
  v += dpp_f64<0x143, 0xc>(v);
  return v;
}
// Minimum over each 16-lane row (every lane of the row ends with it).
__device__ __forceinline__ int row16_min_i(int v) {
  v = min(v, __float_as_int(dpp_mov<PP_DPP_ROR8>(__int_as_float(v))));
  v = min(v, __float_as_int(dpp_mov<PP_DPP_ROR4>(__int_as_float(v))));
  v = min(v, __float_as_int(dpp_mov<PP_DPP_XOR2>(__int_as_float(v))));
  return min(v, __float_as_int(dpp_mov<PP_DPP_XOR1>(__int_as_float(v))));
}
// Whole-wave sum in a fixed order (rows by DPP, then the four row totals read as
// scalars); the result is wave-uniform. Not the xor-butterfly order of wave_sum.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<PP_DPP_XOR1>(v);
  v += dpp_mov<PP_DPP_XOR2>(v);
  v += dpp_mov<PP_DPP_ROR4>(v);
  v += dpp_mov<PP_DPP_ROR8>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------- torch-CPU exp / sigmoid
// SLEEF expf_u10, FMA form (Shibata & Petrogalli, "SLEEF", IEEE TPDS 2020; the
// routine torch's AVX512 Vectorized<float>::exp() calls). Every step is one IEEE
// fp32 operation, so the result is bit-identical to the CPU.
__device__ __forceinline__ float pp_pow2i(int q) { return __uint_as_float((uint32_t)(q + 0x7f) << 23); }

__device__ __forceinline__ float pp_expf_u10(float d) {
  const float R_LN2f = 1.442695040888963407359924681001892137426645954152985934135449406931f;
  const float L2Uf = 0.693145751953125f;
  const float L2Lf = 1.428606765330187045e-06f;
  float t = __fmul_rn(d, R_LN2f);
  int q = (int)__builtin_rintf(t);
  float s = __builtin_fmaf((float)q, -L2Uf, d);
  s = __builtin_fmaf((float)q, -L2Lf, s);
  float u = 0.000198527617612853646278381f;
  u = __builtin_fmaf(u, s, 0.00139304355252534151077271f);
  u = __builtin_fmaf(u, s, 0.00833336077630519866943359f);
  u = __builtin_fmaf(u, s, 0.0416664853692054748535156f);
  u = __builtin_fmaf(u, s, 0.166666671633720397949219f);
  u = __builtin_fmaf(u, s, 0.5f);
  float ss = __fmul_rn(s, s);
  u = __fadd_rn(1.0f, __builtin_fmaf(ss, u, s));
  int qh = q >> 1;
  u = __fmul_rn(__fmul_rn(u, pp_pow2i(qh)), pp_pow2i(q - qh));
  if (d < -104.0f) u = 0.0f;
  if (d > 104.0f) u = __builtin_huge_valf();
  if (d != d) u = d;
  return u;
}

// torch CPU sigmoid for fp32: reciprocal(exp(0 - x) + 1).
__device__ __forceinline__ float pp_sigmoid(float x) {
  float e = pp_expf_u10(__fsub_rn(0.0f, x));
  return __fdiv_rn(1.0f, __fadd_rn(e, 1.0f));
}

// Fast SiLU for the expert activations (not part of the bit-exact routing).
__device__ __forceinline__ float pp_silu(float g) { return g / (1.0f + __expf(-g)); }

// ---------------------------------------------------------------- selection
// Scratch for one token's selection, in LDS, used by one wave.
struct SelScratch {
  float e[PP_MAX_EXPERTS];     // exp values, then probabilities
  float srt[PP_MAX_EXPERTS];   // probabilities in sorted order
  int order[PP_MAX_EXPERTS];   // expert id at each rank
  uint8_t sel[PP_MAX_EXPERTS]; // per expert: selected flag (filled by callers)
  int stk[3 * 24];             // introsort range stack (tie path only)
  int k;                       // number of selected experts
  int tie;                     // a tie group straddles the selection boundary
  int bad;                     // select_one_token_wg: the ranks are not a permutation (never, for a correct sort)
};

// Descending comparator of torch's CPU sort on (value, index) pairs (NaN first).
__device__ __forceinline__ bool kv_before(float a, float b) {
  return (a != a && b == b) || a > b;
}

// torch CPU sort order for E > 16: libstdc++ std::sort (introsort) of
// (value, index) pairs, restated from the published algorithm (bits/stl_algo.h,
// bits/stl_heap.h): median-of-three pivot moved to the front, unguarded
// partition while a range holds more than 16 elements, heapsort once the depth
// limit 2*floor(log2 n) is used up, then a final insertion sort. Run by one
// lane on the rare tokens whose selection boundary cuts through equal values.
static __device__ void kv_adjust_heap(float* K, int* V, int hole, int len, float vk, int vv) {
  int top = hole, sc = hole;
  while (sc < (len - 1) / 2) {
    sc = 2 * (sc + 1);
    if (kv_before(K[sc], K[sc - 1])) sc--;
    K[hole] = K[sc]; V[hole] = V[sc];
    hole = sc;
  }
  if ((len & 1) == 0 && sc == (len - 2) / 2) {
    sc = 2 * (sc + 1);
    K[hole] = K[sc - 1]; V[hole] = V[sc - 1];
    hole = sc - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && kv_before(K[parent], vk)) {
    K[hole] = K[parent]; V[hole] = V[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  K[hole] = vk; V[hole] = vv;
}

static __device__ void kv_heapsort(float* K, int* V, int len) {
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      kv_adjust_heap(K, V, parent, len, K[parent], V[parent]);
      if (parent == 0) break;
    }
  }
  for (int last = len; last > 1;) {
    --last;
    float vk = K[last]; int vv = V[last];
    K[last] = K[0]; V[last] = V[0];
    kv_adjust_heap(K, V, 0, last, vk, vv);
  }
}

static __device__ void kv_linear_insert(float* K, int* V, int last) {
  float vk = K[last]; int vv = V[last];
  int nxt = last - 1;
  while (kv_before(vk, K[nxt])) {
    K[last] = K[nxt]; V[last] = V[nxt];
    last = nxt; --nxt;
  }
  K[last] = vk; V[last] = vv;
}

static __device__ void kv_introsort(float* K, int* V, int n, int* stk) {
  int lg = 0;
  while ((2 << lg) <= n) ++lg;
  int* stf = stk;
  int* stl = stk + 24;
  int* stdp = stk + 48;
  int sp = 0;
  stf[0] = 0; stl[0] = n; stdp[0] = 2 * lg; sp = 1;
  while (sp > 0) {
    --sp;
    int f = stf[sp], l = stl[sp], depth = stdp[sp];
    while (l - f > 16) {
      if (depth == 0) { kv_heapsort(K + f, V + f, l - f); break; }
      --depth;
      int mid = f + (l - f) / 2, a = f + 1, b = mid, c = l - 1, s;
      if (kv_before(K[a], K[b])) {
        if (kv_before(K[b], K[c])) s = b;
        else if (kv_before(K[a], K[c])) s = c;
        else s = a;
      } else if (kv_before(K[a], K[c])) s = a;
      else if (kv_before(K[b], K[c])) s = c;
      else s = b;
      { float tk = K[f]; K[f] = K[s]; K[s] = tk; int tv = V[f]; V[f] = V[s]; V[s] = tv; }
      int lo = f + 1, hi = l;
      for (;;) {
        while (kv_before(K[lo], K[f])) ++lo;
        --hi;
        while (kv_before(K[f], K[hi])) --hi;
        if (!(lo < hi)) break;
        { float tk = K[lo]; K[lo] = K[hi]; K[hi] = tk; int tv = V[lo]; V[lo] = V[hi]; V[hi] = tv; }
        ++lo;
      }
      // each pass pushes at most one frame and the depth drops by one per frame
      // (2*floor(log2 256) = 16 levels), so 24 entries are never exceeded
      stf[sp] = lo; stl[sp] = l; stdp[sp] = depth; ++sp;
      l = lo;
    }
  }
  // final insertion sort: guarded over the first 16, unguarded after
  int head = n < 16 ? n : 16;
  for (int i = 1; i < head; ++i) {
    if (kv_before(K[i], K[0])) {
      float vk = K[i]; int vv = V[i];
      for (int j = i; j > 0; --j) { K[j] = K[j - 1]; V[j] = V[j - 1]; }
      K[0] = vk; V[0] = vv;
    } else {
      kv_linear_insert(K, V, i);
    }
  }
  for (int i = 16; i < n; ++i) kv_linear_insert(K, V, i);
}

// Selection for one token, executed by all 64 lanes of one wave.
// Input: logits read through `lg(j)` for j < E. Output in `ss`: probabilities in
// ss->e, rank order in ss->order, ss->k selected experts (ranks 0..k-1).
// The caller must provide an LDS SelScratch private to this wave.
// Steps follow torch CPU fp32 (softmax_thresholding, src/MoEBlock_origin.py:70-88):
//   max; e = expf_u10(x - max); sum in vec::reduce_all order; p = e * (1/sum);
//   descending sort (stable for E <= 16, introsort ties otherwise); fp64 running
//   sum rounded to fp32 at each rank; keep ranks with cum < tau; keep rank 0.
// Workgroup barrier for LDS traffic only: this wave's LDS operations are complete,
// then s_barrier. Unlike __syncthreads() it does not wait for global loads in flight.
__device__ __forceinline__ void wg_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// fp64 running sum of the sorted probabilities, rounded to fp32 at each rank;
// returns the number of leading ranks with cum < tau (at least 1). `sv(q)` gives the
// q-th largest probability; evaluated identically by every lane.
template <typename SV>
__device__ __forceinline__ int tau_cut(SV sv, int E, float tau) {
  const float tau32 = tau;
  double a = 0.0;
  int k = 0;
  bool stop = false;
  for (int q0 = 0; q0 < E && !stop; q0 += 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (q0 + i < E) ? sv(q0 + i) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (!stop && q0 + i < E) {
        a += (double)v[i];
        if ((float)a < tau32) k = q0 + i + 1;
        else stop = true;
      }
    }
  }
  return k == 0 ? 1 : k;
}

// Selection for E <= EMAX (16 or 64): every lane keeps all E exp values in registers
// (read back from LDS with 16-byte broadcast reads), so the row sum, the probabilities
// and the fp64 running sum need no cross-lane shuffles; ranks are computed per lane
// and scattered through LDS. Same arithmetic, in the same order, as the general path.
template <int EMAX, typename LG>
static __device__ void select_small(LG lg, int E, float tau, SelScratch* ss, int lane) {
  const bool act = lane < E;
  const float x = act ? lg(lane) : -__builtin_huge_valf();
  const float m = wave_max(x);
  const float e = act ? pp_expf_u10(__fsub_rn(x, m)) : 0.0f;
  if (lane < EMAX) ss->e[lane] = act ? e : 0.0f;
  wave_sync_lds();
  float ev[EMAX];
#pragma unroll
  for (int i = 0; i < EMAX / 4; ++i) {
    const float4 v = *(const float4*)&ss->e[4 * i];
    ev[4 * i] = v.x; ev[4 * i + 1] = v.y; ev[4 * i + 2] = v.z; ev[4 * i + 3] = v.w;
  }
  // row sum in torch vec::reduce_all order (16 float lanes)
  float S;
  if (E < 16) {
    S = ev[0];
#pragma unroll
    for (int j = 1; j < (EMAX < 16 ? EMAX : 16); ++j)
      if (j < E) S = __fadd_rn(S, ev[j]);
  } else {
    float a[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = ev[i];
    const int full_end = E - (E % 16);
#pragma unroll
    for (int d = 16; d < EMAX; d += 16) {
      if (d < full_end) {
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = __fadd_rn(a[i], ev[d + i]);
      } else if (d == full_end && E - d > 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < E - d) a[i] = __fadd_rn(a[i], ev[d + i]);
      }
    }
#pragma unroll
    for (int st = 8; st >= 1; st >>= 1)
#pragma unroll
      for (int i = 0; i < st; ++i) a[i] = __fadd_rn(a[i], a[i + st]);
    S = a[0];
  }
  const float r = __fdiv_rn(1.0f, S);
  const float p = act ? __fmul_rn(e, r) : 0.0f;
  int rank = 0;
#pragma unroll
  for (int q = 0; q < EMAX; ++q) {
    const float pq = __fmul_rn(ev[q], r);
    rank += (q < E && (kv_before(pq, p) || (pq == p && q < lane))) ? 1 : 0;
  }
  wave_sync_lds();
  if (act) {
    ss->e[lane] = p;
    ss->srt[rank] = p;
    ss->order[rank] = lane;
  }
  wave_sync_lds();
  float sv[EMAX];
#pragma unroll
  for (int i = 0; i < EMAX / 4; ++i) {
    const float4 v = *(const float4*)&ss->srt[4 * i];
    sv[4 * i] = v.x; sv[4 * i + 1] = v.y; sv[4 * i + 2] = v.z; sv[4 * i + 3] = v.w;
  }
  const float tau32 = tau;
  double acc = 0.0;
  int k = 0;
  bool stop = false;
#pragma unroll
  for (int q = 0; q < EMAX; ++q) {
    if (!stop && q < E) {
      acc += (double)sv[q];
      if ((float)acc < tau32) k = q + 1;
      else stop = true;
    }
  }
  if (k == 0) k = 1;
  bool tie = false;
#pragma unroll
  for (int q = 1; q < EMAX; ++q)
    if (q == k && E > 16 && k < E) tie = sv[q - 1] == sv[q];
  if (lane == 0) {
    ss->k = k;
    ss->tie = tie ? 1 : 0;
    if (tie) {
      for (int j = 0; j < E; ++j) { ss->srt[j] = ss->e[j]; ss->order[j] = j; }
      kv_introsort(ss->srt, ss->order, E, ss->stk);
    }
  }
  wave_sync_lds();
}

template <typename LG>
static __device__ void select_one_token(LG lg, int E, float tau, SelScratch* ss, int lane) {
  if (E <= 16) {
    select_small<16>(lg, E, tau, ss, lane);
    return;
  }
  if (E <= PP_WAVE) {
    // ---- one expert per lane, exchanges through cross-lane shuffles
    const bool act = lane < E;
    const float x = act ? lg(lane) : -__builtin_huge_valf();
    const float m = wave_max(x);
    const float e = act ? pp_expf_u10(__fsub_rn(x, m)) : 0.0f;
    float S;
    if (E < 16) {
      float acc = __shfl(e, 0, PP_WAVE);
      for (int j = 1; j < E; ++j) acc = __fadd_rn(acc, __shfl(e, j, PP_WAVE));
      S = acc;
    } else {
      const int li = lane & 15;
      float acc = __shfl(e, li, PP_WAVE);
      const int full_end = E - (E % 16);
      int d = 16;
      for (; d < full_end; d += 16) acc = __fadd_rn(acc, __shfl(e, d + li, PP_WAVE));
      if (E - d > 0) {
        const float t = __shfl(e, (d + li) & 63, PP_WAVE);
        if (li < E - d) acc = __fadd_rn(acc, t);
      }
      acc = row16_sum(acc);  // the xor 8, 4, 2, 1 butterfly, by DPP
      S = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
    }
    const float p = act ? __fmul_rn(e, __fdiv_rn(1.0f, S)) : 0.0f;
    int rank = 0;
    for (int q = 0; q < E; ++q) {
      const float pq = __shfl(p, q, PP_WAVE);
      rank += (kv_before(pq, p) || (pq == p && q < lane)) ? 1 : 0;
    }
    if (act) {
      ss->e[lane] = p;
      ss->srt[rank] = p;
      ss->order[rank] = lane;
    }
    wave_sync_lds();
    const float mine = act ? ss->srt[lane] : 0.0f;  // lane q holds the q-th largest
    const int k = tau_cut([&](int q) { return __shfl(mine, q, PP_WAVE); }, E, tau);
    const bool tie = E > 16 && k < E && __shfl(mine, k - 1, PP_WAVE) == __shfl(mine, k & 63, PP_WAVE);
    if (lane == 0) {
      ss->k = k;
      ss->tie = tie ? 1 : 0;
      if (tie) {
        // exact torch order for the tie group: (value, index) pairs in index order,
        // then the introsort restatement
        for (int j = 0; j < E; ++j) { ss->srt[j] = ss->e[j]; ss->order[j] = j; }
        kv_introsort(ss->srt, ss->order, E, ss->stk);
      }
    }
    wave_sync_lds();
    return;
  }
  // ---- general path (E > 64): values in LDS
  float m = -__builtin_huge_valf();
  for (int j = lane; j < E; j += PP_WAVE) m = fmaxf(m, lg(j));
  m = wave_max(m);
  for (int j = lane; j < E; j += PP_WAVE) ss->e[j] = pp_expf_u10(__fsub_rn(lg(j), m));
  wave_sync_lds();
  float acc = 0.0f;
  if (lane < 16) {
    acc = ss->e[lane];
    int full_end = E - (E % 16);
    int d = 16;
    for (; d < full_end; d += 16) acc = __fadd_rn(acc, ss->e[d + lane]);
    if (E - d > 0 && lane < E - d) acc = __fadd_rn(acc, ss->e[d + lane]);
  }
  acc = row16_sum(acc);  // the xor 8, 4, 2, 1 butterfly, by DPP
  const float S = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
  const float r = __fdiv_rn(1.0f, S);
  float pv[PP_MAX_EXPERTS / PP_WAVE];
#pragma unroll
  for (int i = 0; i < PP_MAX_EXPERTS / PP_WAVE; ++i) {
    int j = lane + i * PP_WAVE;
    pv[i] = j < E ? __fmul_rn(ss->e[j], r) : 0.0f;
  }
  wave_sync_lds();
#pragma unroll
  for (int i = 0; i < PP_MAX_EXPERTS / PP_WAVE; ++i) {
    int j = lane + i * PP_WAVE;
    if (j < E) ss->e[j] = pv[i];
  }
  wave_sync_lds();
  // ranks of this lane's experts: one pass over the E values, 16 per step read as
  // float4 (independent LDS reads, shared by the lane's up to four experts)
  int rank[PP_MAX_EXPERTS / PP_WAVE];
#pragma unroll
  for (int i = 0; i < PP_MAX_EXPERTS / PP_WAVE; ++i) rank[i] = 0;
  for (int q0 = 0; q0 < E; q0 += 16) {
    float pq[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float4 v4 = *(const float4*)&ss->e[q0 + 4 * u];
      pq[4 * u] = v4.x; pq[4 * u + 1] = v4.y; pq[4 * u + 2] = v4.z; pq[4 * u + 3] = v4.w;
    }
#pragma unroll
    for (int i = 0; i < PP_MAX_EXPERTS / PP_WAVE; ++i) {
      const int j = lane + i * PP_WAVE;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int q = q0 + u;
        rank[i] += (q < E && (kv_before(pq[u], pv[i]) || (pq[u] == pv[i] && q < j))) ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PP_MAX_EXPERTS / PP_WAVE; ++i) {
    const int j = lane + i * PP_WAVE;
    if (j < E) {
      ss->srt[rank[i]] = pv[i];
      ss->order[rank[i]] = j;
    }
  }
  wave_sync_lds();
  if (lane == 0) {
    const int k = tau_cut([&](int q) { return ss->srt[q]; }, E, tau);
    ss->k = k;
    const int tie = (k < E && ss->srt[k - 1] == ss->srt[k]) ? 1 : 0;
    if (tie) {
      for (int j = 0; j < E; ++j) { ss->srt[j] = ss->e[j]; ss->order[j] = j; }
      kv_introsort(ss->srt, ss->order, E, ss->stk);
    }
    ss->tie = tie;
  }
  wave_sync_lds();
}

// Selection of one token by a whole workgroup of nthreads >= E threads, E > 16, with
// the same result as select_one_token. Thread t owns expert t:
// * max (block reduction), e_t = expf_u10(x_t - max); e is zero-padded up to a
//   multiple of 16, so the torch-order sum (16 lane columns added chunk by chunk, the
//   tail into the low lanes, then the halves tree) needs no guards: adding +0.0 to a
//   non-negative running sum changes nothing;
// * p_t = e_t * (1/S) and its 64-bit rank key (~bits(p) << 32 | t) into LDS: for p >= 0
//   and NaN the unsigned key order is exactly "NaN first, then descending, equal
//   values by index" (kv_before plus the index tie-break); padding keys are all ones;
// * rank_t = number of keys below key_t (guard-free loop over the padded keys);
// * the fp64 running-sum cut by wave 0: when every sorted p is 0 or >= 2^-29, every
//   partial sum (< 2) is an exact multiple of 2^-52 and so exact in double, whatever
//   the order of the additions -- a parallel prefix; otherwise the sequential sum;
// * a tie straddling the cut falls back to the introsort restatement (lane 0).
// keys: LDS scratch of PP_MAX_EXPERTS 64-bit words. Every thread must call it. Its
// barriers order LDS traffic only (global loads of the caller may stay in flight).
__device__ __forceinline__ unsigned long long sel_key(float p, int j) {
  const uint32_t b = (p != p) ? 0xffffffffu : __float_as_uint(p);
  return ((unsigned long long)(~b) << 32) | (uint32_t)j;
}

// Value of lane (lane ^ j) for a 64-bit key: DPP for j = 1, 2 (quad permutes), 4 (quad
// reverse then half-row mirror, two involutions) and 8 (the half-row rotation, i ^ 8
// whichever way it turns), permlane swaps for 16 and 32. j is a constant after
// unrolling. (A rotation-based xor 4 depends on the rotation's direction: taken the
// wrong way round it pairs the wrong lanes and the sort loses keys.)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  // every lane has a source lane for these controls, so no old value is needed
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ unsigned long long key_xor(unsigned long long v, int j) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  uint32_t a, b;
  if (j == 1) {
    a = dpp_u32<PP_DPP_XOR1>(lo);
    b = dpp_u32<PP_DPP_XOR1>(hi);
  } else if (j == 2) {
    a = dpp_u32<PP_DPP_XOR2>(lo);
    b = dpp_u32<PP_DPP_XOR2>(hi);
  } else if (j == 4) {
    a = dpp_u32<PP_DPP_HALF_MIRROR>(dpp_u32<PP_DPP_QREV>(lo));
    b = dpp_u32<PP_DPP_HALF_MIRROR>(dpp_u32<PP_DPP_QREV>(hi));
  } else if (j == 8) {
    a = dpp_u32<PP_DPP_ROR8>(lo);
    b = dpp_u32<PP_DPP_ROR8>(hi);
  } else if (j == 16) {
    const int lane = (int)__lane_id();
    a = pl_xor16(lo, lane);
    b = pl_xor16(hi, lane);
  } else {
    const int lane = (int)__lane_id();
    a = pl_xor32(lo, lane);
    b = pl_xor32(hi, lane);
  }
  return ((unsigned long long)b << 32) | a;
}

// This wave's LDS writes visible to its other lanes (LDS executes a wave's operations in order)
__device__ __forceinline__ void sel_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}
template <int NS, typename LG>
static __device__ void select_one_token_w1(LG lg, int E, float tau, SelScratch* ss, unsigned long long* keys,
                                           int lane) {
  constexpr int N = 64 * NS;
  const int E16 = (E + 15) & ~15;
  float x[NS];
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const int i = lane + 64 * q;
    x[q] = i < E ? lg(i) : -__builtin_huge_valf();
  }
  float m = x[0];
#pragma unroll
  for (int q = 1; q < NS; ++q) m = fmaxf(m, x[q]);
  m = wave_max(m);
  float e[NS];
#pragma unroll
  for (int q = 0; q < NS; ++q) e[q] = lane + 64 * q < E ? pp_expf_u10(__fsub_rn(x[q], m)) : 0.0f;
  // row sum in the fixed order: lane j < 16 adds e[16 c + j], c = 0, 1, ... (chunk c sits in
  // row c % 4 of slot c / 4), then the xor 8, 4, 2, 1 butterfly
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < N / 16; ++c) {
    if (16 * c >= E16) break;
    float v = e[c >> 2];
    if ((c & 3) == 1) v = pl_xor16f(v, lane);
    else if ((c & 3) == 2) v = pl_xor32f(v, lane);
    else if ((c & 3) == 3) v = pl_xor16f(pl_xor32f(v, lane), lane);
    acc = c == 0 ? v : __fadd_rn(acc, v);
  }
  acc = row16_sum(acc);
  const float S = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
  const float r = __fdiv_rn(1.0f, S);
  unsigned long long key[NS];
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const int i = lane + 64 * q;
    const float p = __fmul_rn(e[q], r);
    if (i < E) ss->e[i] = p;
    key[q] = i < E ? sel_key(p, i) : ~0ull;
  }
#pragma unroll
  for (int k2 = 2; k2 <= N; k2 <<= 1)
#pragma unroll
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int js = j >> 6;
#pragma unroll
        for (int q = 0; q < NS; ++q)
          if ((q & js) == 0) {
            const int q2 = q | js;
            const bool up = ((64 * q + lane) & k2) == 0;  // ascending block
            const unsigned long long a = key[q], b = key[q2];
            const bool lt = b < a;
            const unsigned long long lo = lt ? b : a, hi = lt ? a : b;
            key[q] = up ? lo : hi;
            key[q2] = up ? hi : lo;
          }
      } else {
#pragma unroll
        for (int q = 0; q < NS; ++q) {
          const int n = 64 * q + lane;
          const unsigned long long o = key_xor(key[q], j);
          const bool keep_min = ((n & j) == 0) == ((n & k2) == 0);
          key[q] = ((o < key[q]) == keep_min) ? o : key[q];
        }
      }
    }
#pragma unroll
  for (int q = 0; q < NS; ++q) keys[64 * q + lane] = key[q];
  sel_lds_sync();
  // sorted positions: rank n holds expert (uint32)key; keys strictly increase over the E
  // real ones (unique by their index bits), else the network lost or duplicated a key
  bool bad = false;
  float v[NS];
  bool exact = true;
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const int n = 64 * q + lane;
    const int idx = (int)(uint32_t)key[q];
    if (n < E) {
      bad |= idx >= E || (n + 1 < E && !(key[q] < keys[min(n + 1, N - 1)]));
      ss->order[n] = idx;
      v[q] = ss->e[min(idx, E - 1)];
      ss->srt[n] = v[q];
    } else {
      v[q] = 0.0f;
    }
    exact = exact && (v[q] == 0.0f || v[q] >= 0x1p-29f);
  }
  bad = __any(bad);
  int k;
  if (__all(exact)) {
    double carry = 0.0;
    int c = 0;
    const float tau32 = tau;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const double incl = carry + wave_incl_scan_f64((double)v[q]);
      c += __popcll(__ballot(64 * q + lane < E && (float)incl < tau32));
      const unsigned long long u = (unsigned long long)__double_as_longlong(incl);
      const uint32_t clo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
      const uint32_t chi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
      carry = __longlong_as_double((long long)(((unsigned long long)chi << 32) | clo));
    }
    k = c > 0 ? c : 1;
  } else {
    sel_lds_sync();
    k = tau_cut([&](int q) { return ss->srt[q]; }, E, tau);
  }
  if (lane == 0) {
    ss->k = k;
    ss->bad = bad ? 1 : 0;
  }
  sel_lds_sync();
  if (lane == 0) ss->tie = (k < E && ss->srt[k - 1] == ss->srt[k]) ? 1 : 0;
}

template <typename LG>
static __device__ void select_one_token_wg(LG lg, int E, float tau, SelScratch* ss, unsigned long long* keys,
                                           float* red, int tid, int nthreads) {
  if (E <= 128) {  // uniform: the one-wave form, the other waves wait
    if ((tid >> 6) == 0) {
      if (E <= 64) select_one_token_w1<1>(lg, E, tau, ss, keys, tid & 63);
      else select_one_token_w1<2>(lg, E, tau, ss, keys, tid & 63);
    }
    wg_lds_barrier();
    if (ss->tie) {  // uniform
      if (tid == 0) {
        for (int j = 0; j < E; ++j) { ss->srt[j] = ss->e[j]; ss->order[j] = j; }
        kv_introsort(ss->srt, ss->order, E, ss->stk);
      }
      wg_lds_barrier();
    }
    return;
  }
  const int lane = tid & 63, wv = tid >> 6, nw = nthreads >> 6;
  const int E16 = (E + 15) & ~15;
  const float x = tid < E ? lg(tid) : -__builtin_huge_valf();
  float m = wave_max_dpp(x);
  if (lane == 0) red[wv] = m;
  wg_lds_barrier();
  m = red[0];
  for (int w = 1; w < nw; ++w) m = fmaxf(m, red[w]);
  const float e = tid < E ? pp_expf_u10(__fsub_rn(x, m)) : 0.0f;
  if (tid < E16) ss->e[tid] = e;
  wg_lds_barrier();
  if (tid < 16) {
    float col[PP_MAX_EXPERTS / 16];
#pragma unroll
    for (int c = 0; c < PP_MAX_EXPERTS / 16; ++c) col[c] = 16 * c < E16 ? ss->e[16 * c + tid] : 0.0f;
    float acc = col[0];
#pragma unroll
    for (int c = 1; c < PP_MAX_EXPERTS / 16; ++c)
      if (16 * c < E16) acc = __fadd_rn(acc, col[c]);
    acc = row16_sum(acc);  // the xor 8, 4, 2, 1 butterfly, by DPP
    if (tid == 0) red[0] = __fdiv_rn(1.0f, acc);
  }
  wg_lds_barrier();
  const float pt = __fmul_rn(e, red[0]);
  // ranks: every wave holding keys sorts its 64 (unique) keys in registers (bitonic, xor
  // shuffles; padding ~0 sorts last), stores the sorted run, and each key's rank is its
  // place in its run plus the number of smaller keys in the other runs (binary search).
  // The same ranks as counting all smaller keys (E LDS reads per key, 2.4 us at E = 192);
  // the whole E = 192 decode layer 24.7 -> 24.35 us with LDS-permute shuffles; 18 of the
  // sort's 21 exchanges go through DPP. The binary searches over the other runs are
  // interleaved (one LDS round trip per step for all runs, not one per run): runs past
  // nwk and the wave's own run are searched too, in bounds of keys, and not counted.
  const int nwk = (E + 63) >> 6;  // waves holding keys
  unsigned long long key = tid < E ? sel_key(pt, tid) : ~0ull;
  if (tid < E) ss->e[tid] = pt;
  if (tid == 0) ss->bad = 0;
  if (wv < nwk) {
#pragma unroll
    for (int k2 = 2; k2 <= 64; k2 <<= 1)
#pragma unroll
      for (int j = k2 >> 1; j > 0; j >>= 1) {
        const unsigned long long o = key_xor(key, j);
        const bool keep_min = ((lane & j) == 0) == ((lane & k2) == 0);
        // one compare: real keys are unique, and two padding keys are equal, so
        // "o < key" decides both the minimum and the maximum
        key = ((o < key) == keep_min) ? o : key;
      }
    keys[tid] = key;
  }
  wg_lds_barrier();
  const bool holder = wv < nwk && key != ~0ull;
  int rank = lane;
  const int idx = (int)(uint32_t)key;
  if (holder) {
    constexpr int NRUN = PP_MAX_EXPERTS / 64;
    int lo[NRUN];  // keys of run r below key
#pragma unroll
    for (int r = 0; r < NRUN; ++r) lo[r] = 0;
#pragma unroll
    for (int step = 32; step >= 1; step >>= 1)
#pragma unroll
      for (int r = 0; r < NRUN; ++r) lo[r] += keys[64 * r + lo[r] + step - 1] < key ? step : 0;
#pragma unroll
    for (int r = 0; r < NRUN; ++r)
      if (r < nwk && r != wv) rank += lo[r] + ((lo[r] == 63 && keys[64 * r + 63] < key) ? 1 : 0);
    if (rank < E && idx < E) {  // always, for a correct sort (else ss->bad below)
      ss->srt[rank] = ss->e[idx];
      ss->order[rank] = idx;
    }
  }
  wg_lds_barrier();
  // Permutation check: E keys, each written to its rank; a lost or duplicated key makes
  // two writers share a rank, and one of them reads back the other's id. No collision
  // and every rank in [0, E) means ss->order is a permutation. A failed check is
  // reported through ss->bad (the caller turns it into an error), never used silently.
  if (holder && !(rank < E && idx < E && ss->order[rank] == idx)) ss->bad = 1;
  if (tid < PP_WAVE) {
    constexpr int QPL = PP_MAX_EXPERTS / PP_WAVE;  // sorted positions per lane
    float v[QPL];
    bool exact = true;
#pragma unroll
    for (int i = 0; i < QPL; ++i) {
      const int q = lane * QPL + i;
      v[i] = q < E ? ss->srt[q] : 0.0f;
      exact = exact && (v[i] == 0.0f || v[i] >= 0x1p-29f);  // NaN fails both
    }
    int k;
    if (__all(exact)) {
      double sv[QPL], run = 0.0;
#pragma unroll
      for (int i = 0; i < QPL; ++i) {
        run += (double)v[i];
        sv[i] = run;
      }
      const double incl = wave_incl_scan_f64(run);
      const double excl = incl - run;
      const float tau32 = tau;
      int c = 0;  // ranks whose running sum stays below tau, counted by ballots
#pragma unroll
      for (int i = 0; i < QPL; ++i)
        c += __popcll(__ballot(lane * QPL + i < E && (float)(excl + sv[i]) < tau32));
      k = c > 0 ? c : 1;
    } else {
      k = tau_cut([&](int q) { return ss->srt[q]; }, E, tau);
    }
    if (lane == 0) {
      ss->k = k;
      ss->tie = (k < E && ss->srt[k - 1] == ss->srt[k]) ? 1 : 0;
    }
  }
  wg_lds_barrier();
  if (ss->tie) {  // uniform; after the permutation check, which reads ss->order
    if (tid == 0) {
      for (int j = 0; j < E; ++j) { ss->srt[j] = ss->e[j]; ss->order[j] = j; }
      kv_introsort(ss->srt, ss->order, E, ss->stk);
    }
    wg_lds_barrier();
  }
}
