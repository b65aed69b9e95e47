// sas_probe.hip -- on-box peak probes for the roofline figures of the benchmark
// (libsas_probe.so; measurement only, not part of the operator's C ABI).
//
//   sas_probe_mfma   register-only v_mfma_f32_32x32x16_bf16 throughput: each wave
//                    keeps 8 independent accumulators (or, `dependent`, one chain)
//                    and cycles its A and B operands through 8 fragments each of
//                    pseudo-random bf16 values, so the operands change on every MFMA
//                    (operand toggling sets the power the matrix cores draw, and with
//                    it the clock they sustain).
//   sas_probe_read   streaming 16-byte loads over a buffer (HBM read bandwidth).
//
// Both write one value per thread (out[blockIdx.x * 256 + threadIdx.x]) so that the
// work is not optimised away; out holds at least blocks * 256 entries.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Two bf16 values with random sign and mantissa and exponents 2^-3 .. 2^1.
__device__ __forceinline__ uint32_t rnd_bf16x2(uint32_t h) {
  const uint32_t g = mix32(h);
  const uint32_t lo = (h & 0x807fu) | ((124u + ((h >> 7) % 5u)) << 7);
  const uint32_t hi = (g & 0x807fu) | ((124u + ((g >> 7) % 5u)) << 7);
  return (lo & 0xffffu) | (hi << 16);
}

// NACC independent accumulators per wave (8: throughput; 1: one dependent chain,
// each MFMA accumulating into the previous one's result).
template <int NACC>
__global__ __launch_bounds__(256) void probe_mfma_kernel(float* __restrict__ out,
                                                         uint64_t* __restrict__ ticks, int iters) {
  u32x4_t A[8], B[8];
  const uint32_t seed = mix32(blockIdx.x * 256u + threadIdx.x + 1u);
  for (int i = 0; i < 8; ++i)
    for (int e = 0; e < 4; ++e) {
      A[i][e] = rnd_bf16x2(mix32(seed + 97u * i + e));
      B[i][e] = rnd_bf16x2(mix32(seed * 31u + 89u * i + e + 7u));
    }
  f32x16_t acc[NACC];
  for (int k = 0; k < NACC; ++k) acc[k] = f32x16_t{};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; it += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        acc[k % NACC] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, A[(k + u) & 7]), __builtin_bit_cast(bf16x8_t, B[(3 * k + u) & 7]),
            acc[k % NACC], 0, 0, 0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  for (int k = 0; k < NACC; ++k)
    for (int r = 0; r < 16; ++r) s += acc[k][r];
  const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
  out[gid] = s;
  if ((threadIdx.x & 63) == 0) ticks[gid >> 6] = t1 - t0;
}

__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4_t* __restrict__ src, size_t n,
                                                         uint32_t* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * 256;
  uint32_t acc = 0;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const u32x4_t a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a[0] ^ a[3] ^ b[1] ^ b[2] ^ c[0] ^ c[1] ^ d[2] ^ d[3];
  }
  for (; i < n; i += stride) acc ^= src[i][0];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// iters: rounds of 8 MFMAs per wave (a multiple of 8); ticks: blocks * 4 per-wave
// s_memtime spans (shader clock cycles).  dependent != 0: one accumulator per wave.
int sas_probe_mfma(float* out, uint64_t* ticks, int iters, int blocks, int dependent, void* stream) {
  if (!out || !ticks || iters <= 0 || (iters & 7) || blocks <= 0) return -1;
  if (dependent)
    hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out,
                       ticks, iters);
  else
    hipLaunchKernelGGL(probe_mfma_kernel<8>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out,
                       ticks, iters);
  return hipGetLastError() == hipSuccess ? 0 : -9;
}

// src: bytes (a multiple of 16, 16-B aligned) read once per call.
int sas_probe_read(const void* src, size_t bytes, uint32_t* out, int blocks, void* stream) {
  if (!src || !out || bytes < 16 || (bytes & 15) || ((uintptr_t)src & 15) || blocks <= 0) return -1;
  hipLaunchKernelGGL(probe_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const u32x4_t*>(src), bytes / 16, out);
  return hipGetLastError() == hipSuccess ? 0 : -9;
}

}  // extern "C"
