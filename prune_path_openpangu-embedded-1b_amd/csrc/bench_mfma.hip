// Measurement support, not part of the product ABI (built as ../libpp_bench.so, loaded by
// bench.py only): the bf16 MFMA rate the chip sustains on register operands, so that the
// prefill GEMMs' utilisation can be read against what the MFMA pipe delivers on data like
// theirs, not only against the nominal 2.5 PFLOP/s.
//
// Every wave of a grid x 512-thread launch runs `iters` rounds of 4 x 2
// v_mfma_f32_32x32x16_bf16 (the dense GEMMs' wave tile: 128 x 64 per 16-wide k-step) on
// operands held in registers. mode 0: all-zero operands; mode 1: random bf16 in
// [2^-7, 2) with random signs (a 32-bit LCG per lane). The MFMA power draw, and so the
// clock the chip holds, depends on the operand bits: the two modes bound the rate.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef __bf16 pb_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pb_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int pb_u32x4 __attribute__((ext_vector_type(4)));

#define PB_MI 4
#define PB_NJ 2

__global__ __launch_bounds__(512, 1) void pb_mfma_kernel(float* __restrict__ out, int iters, int mode,
                                                         uint32_t seed) {
  const uint32_t tid = threadIdx.x + blockIdx.x * 512u;
  uint32_t s = (tid * 2654435761u) ^ seed;
  auto next = [&]() {
    s = s * 1664525u + 1013904223u;
    // two bf16: exponent >= 120 (2^-7), random mantissa and sign
    return mode ? ((((s >> 1) & 0x3fff3fffu) | 0x3c003c00u) ^ (s & 0x80008000u)) : 0u;
  };
  pb_u32x4 a[PB_MI], b[PB_NJ];
  for (int i = 0; i < PB_MI; ++i)
    for (int q = 0; q < 4; ++q) a[i][q] = next();
  for (int j = 0; j < PB_NJ; ++j)
    for (int q = 0; q < 4; ++q) b[j][q] = next();
  pb_f32x16 acc[PB_MI][PB_NJ];
  for (int i = 0; i < PB_MI; ++i)
    for (int j = 0; j < PB_NJ; ++j)
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < PB_MI; ++i)
#pragma unroll
      for (int j = 0; j < PB_NJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(pb_bf16x8, a[i]),
                                                            __builtin_bit_cast(pb_bf16x8, b[j]), acc[i][j], 0, 0, 0);
    a[it & (PB_MI - 1)][0] ^= mode ? 0x00010001u : 0u;  // an operand changes every round: nothing is hoisted
  }
  float t = 0.0f;
  for (int i = 0; i < PB_MI; ++i)
    for (int j = 0; j < PB_NJ; ++j)
      for (int q = 0; q < 16; ++q) t += acc[i][j][q];
  out[tid] = t;
}

// Runs `reps` back-to-back launches of grid workgroups (after one untimed launch) and writes
// each launch's milliseconds to ms_out[0 .. reps). Returns 0, or the HIP error code. flops of
// one launch: grid * 8 waves * iters * 8 MFMAs * 32768.
extern "C" int ppb_mfma_rate(int grid, int iters, int mode, int reps, float* ms_out) {
  if (grid < 1 || grid > 65536 || iters < 1 || reps < 1 || reps > 1024 || !ms_out) return (int)hipErrorInvalidValue;
  float* out = nullptr;
  hipError_t e = hipMalloc(&out, (size_t)grid * 512 * sizeof(float));
  if (e != hipSuccess) return (int)e;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if ((e = hipEventCreate(&e0)) == hipSuccess && (e = hipEventCreate(&e1)) == hipSuccess) {
    pb_mfma_kernel<<<grid, 512>>>(out, iters, mode, 12345u);
    e = hipGetLastError();
    for (int r = 0; r < reps && e == hipSuccess; ++r) {
      if ((e = hipEventRecord(e0, 0)) != hipSuccess) break;
      pb_mfma_kernel<<<grid, 512>>>(out, iters, mode, 12345u + (uint32_t)r);
      if ((e = hipGetLastError()) != hipSuccess) break;
      if ((e = hipEventRecord(e1, 0)) != hipSuccess || (e = hipEventSynchronize(e1)) != hipSuccess) break;
      e = hipEventElapsedTime(&ms_out[r], e0, e1);
    }
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  const hipError_t ef = hipFree(out);
  return (int)(e != hipSuccess ? e : ef);
}
