// Masked training path: the expert gating of MoELayer.forward (src/MoEBlock_origin.py:205-212),
//   self_moe_mask = experts_prob @ experts_masks      ([N,E] x [E,I] one-hot)
//   intermediate  = intermediate * self_moe_mask
// and its backward, as two HBM-bound kernels over rows of the [N, I] activations.
//
// experts_masks is one-hot per neuron, so the matmul picks gates[n, eid[d]] exactly
// (one product by 1.0 plus zeros: no rounding), and the forward is one multiply per
// element: out[n,d] = inter[n,d] * gates[n, eid[d]] -- bit-identical to the fp32
// reference ops. With bf16 activations the gate is rounded to bf16 first and the
// product rounded to bf16, as the all-bf16 reference (bf16 experts_prob @ bf16 masks,
// bf16 multiply) computes it.
//
// Backward (the autograd of the two ops):
//   d_inter[n,d] = d_out[n,d] * gates[n, eid[d]]
//   d_gates[n,e] = sum over the neurons d of expert e of d_out[n,d] * inter[n,d]
// accumulated in fp32 in a fixed order, so repeated calls give the same bits: the
// products are staged in LDS and summed through the expert-sorted neuron order (perm,
// seg), TPE interleaved partial sums per expert then an xor tree, whatever the partition.
//
// Workgroups of 256 threads; each thread moves 8 consecutive elements per step (16-byte
// bf16 / 32-byte fp32 vectors).
#include "pp_common.h"

#define MG_THREADS 256
#define MG_MAX_I 16384  // LDS holds one row's fp32 products and the expert-sorted order (uint16)

template <typename T>
struct MgVec;
template <>
struct MgVec<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ float gate(float g) { return g; }
};
template <>
struct MgVec<bf16_t> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8]) {
    const uint4 u = *(const uint4*)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[8]) {
    uint4 u;
    u.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    u.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    u.z = (uint32_t)f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
    u.w = (uint32_t)f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
    *(uint4*)p = u;
  }
  static __device__ __forceinline__ float gate(float g) { return bf16_to_f32(f32_to_bf16(g)); }
};

// The backward is persistent over rows: a workgroup stages the neuron -> expert ids
// (uint8) and the expert-sorted order (uint16) in LDS once and then takes rows
// blockIdx.x, + gridDim.x, ...; the gates of the current row sit in one of two LDS
// buffers (row parity). One workgroup per row re-read the order from L2 in a dependent
// loop: 238 against 148 us for 16384 x 6144 bf16 at E = 16.
__device__ __forceinline__ void mg_ids8(const uint8_t* e_s, int d, int (&e)[8]) {
  const uint2 u = *(const uint2*)(e_s + d);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[i] = (u.x >> (8 * i)) & 0xff;
    e[4 + i] = (u.y >> (8 * i)) & 0xff;
  }
}

__device__ __forceinline__ void mg_stage_ids(const int32_t* __restrict__ eid, int I, int E, uint8_t* e_s) {
  for (int d = threadIdx.x; d < I; d += MG_THREADS)
    e_s[d] = (uint8_t)min((unsigned)eid[d], (unsigned)(E - 1));  // ids come from the caller: clamped
}

#define MG_G_BYTES (2 * PP_MAX_EXPERTS * 4)
static size_t mg_bwd_lds(int I) { return MG_G_BYTES + (size_t)I * 7 + (PP_MAX_EXPERTS + 1) * 4; }

// The forward takes one row per workgroup (no barrier between rows; the ids come
// through L2 as int32 -- measured a little faster than the persistent form with the ids
// in LDS, 80 against 85 us for 16384 x 6144 bf16).
__device__ __forceinline__ void mg_eids(const int32_t* eid, int d, int E, int (&e)[8]) {
  const int4 a = *(const int4*)(eid + d), b = *(const int4*)(eid + d + 4);
  const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (int)min((unsigned)v[i], (unsigned)(E - 1));  // clamped
}

template <typename T>
__global__ __launch_bounds__(MG_THREADS) void masked_gate_fwd_kernel(const T* __restrict__ inter,
                                                                     const float* __restrict__ gates,
                                                                     const int32_t* __restrict__ eid, int I, int E,
                                                                     T* __restrict__ out) {
  __shared__ float g_s[PP_MAX_EXPERTS];
  const int64_t n = blockIdx.x;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += MG_THREADS) g_s[e] = MgVec<T>::gate(gates[n * E + e]);
  __syncthreads();
  for (int d = 8 * tid; d < I; d += 8 * MG_THREADS) {
    float v[8];
    int e[8];
    MgVec<T>::load(inter + n * I + d, v);
    mg_eids(eid, d, E, e);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(v[i], g_s[e[i]]);
    MgVec<T>::store(out + n * I + d, v);
  }
}

// tpe: threads per expert for the sums (a power of two <= 64, E * tpe <= MG_THREADS).
// LDS: gates [2][256], products fp32 [I], expert-sorted order uint16 [I], ids uint8 [I],
// segments [E+1]. Per row: gates -> barrier -> d_inter and products -> barrier -> sums
// (the next row's first barrier keeps its products from overwriting these).
template <typename T>
__global__ __launch_bounds__(MG_THREADS) void masked_gate_bwd_kernel(
    const T* __restrict__ d_out, const T* __restrict__ inter, const float* __restrict__ gates,
    const int32_t* __restrict__ eid, const int32_t* __restrict__ perm, const int32_t* __restrict__ seg,
    int64_t n_rows, int I, int E, int tpe, T* __restrict__ d_inter, float* __restrict__ d_gates) {
  extern __shared__ __align__(16) unsigned char mg_smem[];
  float* g_s = (float*)mg_smem;
  float* prod_s = (float*)(mg_smem + MG_G_BYTES);
  uint16_t* p_s = (uint16_t*)(mg_smem + MG_G_BYTES + (size_t)I * 4);
  uint8_t* e_s = mg_smem + MG_G_BYTES + (size_t)I * 6;
  int* seg_s = (int*)(mg_smem + MG_G_BYTES + (size_t)I * 7);
  const int tid = threadIdx.x;
  mg_stage_ids(eid, I, E, e_s);
  for (int k = tid; k < I; k += MG_THREADS) p_s[k] = (uint16_t)min((unsigned)perm[k], (unsigned)(I - 1));
  for (int e = tid; e <= E; e += MG_THREADS) seg_s[e] = min(max(seg[e], 0), I);  // (clamped: from the caller)
  const int ex = tid / tpe, j = tid - ex * tpe;
  int par = 0;
  for (int64_t n = blockIdx.x; n < n_rows; n += gridDim.x, par ^= 1) {
    float* g = g_s + par * PP_MAX_EXPERTS;
    for (int e = tid; e < E; e += MG_THREADS) g[e] = MgVec<T>::gate(gates[n * E + e]);
    __syncthreads();
    for (int d = 8 * tid; d < I; d += 8 * MG_THREADS) {
      float go[8], x[8], gi[8];
      int e[8];
      MgVec<T>::load(d_out + n * I + d, go);
      MgVec<T>::load(inter + n * I + d, x);
      mg_ids8(e_s, d, e);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        gi[i] = __fmul_rn(go[i], g[e[i]]);
        prod_s[d + i] = __fmul_rn(go[i], x[i]);
      }
      if (d_inter) MgVec<T>::store(d_inter + n * I + d, gi);
    }
    __syncthreads();
    // expert ex, partial j over its neurons k = seg[ex] + j, + tpe, ... (expert-sorted
    // order) in four interleaved sums, ((a0 + a1) + (a2 + a3)), then the xor tree
    // inside the tpe-lane group
    float s = 0.0f;
    if (ex < E) {
      const int k1 = seg_s[ex + 1];
      int k = seg_s[ex] + j;
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      for (; k + 3 * tpe < k1; k += 4 * tpe) {
        a0 = __fadd_rn(a0, prod_s[p_s[k]]);
        a1 = __fadd_rn(a1, prod_s[p_s[k + tpe]]);
        a2 = __fadd_rn(a2, prod_s[p_s[k + 2 * tpe]]);
        a3 = __fadd_rn(a3, prod_s[p_s[k + 3 * tpe]]);
      }
      for (; k < k1; k += tpe) a0 = __fadd_rn(a0, prod_s[p_s[k]]);
      s = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
    }
    for (int o = 1; o < tpe; o <<= 1) s = __fadd_rn(s, __shfl_xor(s, o, PP_WAVE));
    if (ex < E && j == 0) d_gates[n * E + ex] = s;
  }
}

// Workgroups per launch: as many as fit the CUs at the kernel's LDS use (at most 8 of
// 256 threads per CU), no more than there are rows.
static unsigned mg_grid(int64_t n_rows, size_t lds) {
  int per_cu = (int)((160 * 1024) / (lds + 1024));
  per_cu = per_cu < 1 ? 1 : per_cu > 8 ? 8 : per_cu;
  const int64_t g = (int64_t)pp_device_cus() * per_cu;
  return (unsigned)(n_rows < g ? n_rows : g);
}

static int mg_check(const void* a, const void* b, int dtype, int64_t n_rows, int I, int E, const char* what) {
  PP_REQUIRE(dtype == PP_DTYPE_F32 || dtype == PP_DTYPE_BF16, PP_ERR_INVALID, "%s: dtype %d", what, dtype);
  PP_REQUIRE(E >= 1 && E <= PP_MAX_EXPERTS, PP_ERR_UNSUPPORTED, "%s: E=%d unsupported (1..256)", what, E);
  PP_REQUIRE(I >= 8 && I % 8 == 0 && I <= MG_MAX_I, PP_ERR_UNSUPPORTED,
             "%s: I=%d unsupported (need I %% 8 == 0, 8 <= I <= %d)", what, I, MG_MAX_I);
  PP_REQUIRE(n_rows >= 0 && n_rows <= 0x7fffffff, PP_ERR_UNSUPPORTED, "%s: n_rows %lld", what, (long long)n_rows);
  PP_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0, PP_ERR_INVALID,
             "%s: activations must be 16-byte aligned", what);
  return PP_OK;
}

extern "C" int pp_masked_gate_fwd(const void* inter, int dtype, const float* gates, const int32_t* expert_ids,
                                  int64_t n_rows, int I, int E, void* out, void* stream) {
  int rc = mg_check(inter, out, dtype, n_rows, I, E, "pp_masked_gate_fwd");
  if (rc) return rc;
  if (n_rows == 0) return PP_OK;
  PP_REQUIRE(inter && gates && expert_ids && out, PP_ERR_INVALID, "pp_masked_gate_fwd: null pointer");
  PP_REQUIRE(((uintptr_t)expert_ids & 15) == 0, PP_ERR_INVALID, "pp_masked_gate_fwd: expert_ids not 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == PP_DTYPE_F32)
    masked_gate_fwd_kernel<float><<<(unsigned)n_rows, MG_THREADS, 0, st>>>((const float*)inter, gates, expert_ids, I,
                                                                           E, (float*)out);
  else
    masked_gate_fwd_kernel<bf16_t><<<(unsigned)n_rows, MG_THREADS, 0, st>>>((const bf16_t*)inter, gates, expert_ids,
                                                                            I, E, (bf16_t*)out);
  return pp_check_launch("pp_masked_gate_fwd");
}

extern "C" int pp_masked_gate_bwd(const void* d_out, const void* inter, int dtype, const float* gates,
                                  const int32_t* expert_ids, const int32_t* perm, const int32_t* seg, int64_t n_rows,
                                  int I, int E, void* d_inter, float* d_gates, void* stream) {
  int rc = mg_check(d_out, inter, dtype, n_rows, I, E, "pp_masked_gate_bwd");
  if (rc) return rc;
  if (n_rows == 0) return PP_OK;
  PP_REQUIRE(d_out && inter && gates && expert_ids && perm && seg && d_gates, PP_ERR_INVALID,
             "pp_masked_gate_bwd: null pointer");
  PP_REQUIRE(((uintptr_t)d_inter & 15) == 0 && ((uintptr_t)expert_ids & 15) == 0, PP_ERR_INVALID,
             "pp_masked_gate_bwd: d_inter / expert_ids not 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  int tpe = 64;
  while (tpe > 1 && tpe * E > MG_THREADS) tpe >>= 1;
  const size_t lds = mg_bwd_lds(I);
  const unsigned grid = mg_grid(n_rows, lds);
  if (dtype == PP_DTYPE_F32)
    masked_gate_bwd_kernel<float><<<grid, MG_THREADS, lds, st>>>((const float*)d_out, (const float*)inter, gates,
                                                                 expert_ids, perm, seg, n_rows, I, E, tpe,
                                                                 (float*)d_inter, d_gates);
  else
    masked_gate_bwd_kernel<bf16_t><<<grid, MG_THREADS, lds, st>>>((const bf16_t*)d_out, (const bf16_t*)inter, gates,
                                                                  expert_ids, perm, seg, n_rows, I, E, tpe,
                                                                  (bf16_t*)d_inter, d_gates);
  return pp_check_launch("pp_masked_gate_bwd");
}
